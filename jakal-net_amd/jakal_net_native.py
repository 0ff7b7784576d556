"""jakal_net_native -- the native-backend module, backed by the gfx950 HIP library.

Stands where the reference's pybind extension ``jakal_net_native``
(``native/jakal_net_native.cpp:7379-7500``) stands: same module name, same
``supported_ops() / supported_devices() / backend_name()`` contract and the
same positional op signatures, so ``jakal_net.native_backend`` (and the
reference's own loader) dispatch to it unchanged.

Each op flattens batch dimensions, casts to fp32 contiguous buffers and calls
the C ABI of ``lib/libjakal_net_hip.so`` (declared in ``include/jakal_net_hip.h``)
through ctypes on the current HIP stream.  bf16 layers keep their value rows
in bf16 on the edge-list ops (the *_bf16 entry points): the gathers move bf16
rows, the top-k scores run on bf16 MFMAs, and the outputs and value gradients
come back in bf16.  Gradients come from
``torch.autograd.Function`` wrappers whose backward calls the library's
backward entry points.  Importing this module fails if the library cannot be
loaded; nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch
from torch import Tensor

LIB_ENV = "JAKAL_NET_HIP_LIB"
_HERE = Path(__file__).resolve().parent


def library_path() -> Path:
    override = os.environ.get(LIB_ENV)
    return Path(override) if override else _HERE / "lib" / "libjakal_net_hip.so"


_LIB = ctypes.CDLL(str(library_path()))

_P, _I64, _I32, _F, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_size_t


def _declare(name: str, argtypes: list, restype=ctypes.c_int) -> None:
    fn = getattr(_LIB, name)
    fn.argtypes = argtypes
    fn.restype = restype


_declare("jn_last_error", [], ctypes.c_char_p)
_declare("jn_abi_version", [])
_declare("jn_profile_enable", [_I32])
_declare("jn_profile_collect", [ctypes.c_char_p, _SZ])
_declare("jn_set_gemm_tile", [_I32])
_declare("jn_set_select_mode", [_I32])
_declare("jn_set_window_kernels", [_I32])
_declare("jn_set_side_streams", [_I32])
_declare(
    "jn_lowrank_topk_select",
    [_P, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _F, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ, _P],
)
_declare("jn_lowrank_topk_select_workspace_bytes", [_I64] * 3, _SZ)
_declare(
    "jn_propagation_topk_forward",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P,
     _P, _SZ, _P, _SZ, _P],
)
_declare("jn_propagation_topk_forward_workspace_bytes", [_I64] * 3, _SZ)
_declare("jn_propagation_topk_layout_bytes", [_I64] * 3, _SZ)
_declare("jn_propagation_topk_workspace_bytes", [_I64, _I64, _I64, _I64, _I64, _I64], _SZ)
_declare(
    "jn_propagation_topk_backward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_propagation_window_forward",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P],
)
_declare("jn_propagation_window_workspace_bytes", [_I64, _I64, _I64, _I64, _I64, _I64], _SZ)
_declare(
    "jn_propagation_window_backward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare("jn_transition_topk_workspace_bytes", [_I64] * 8, _SZ)
_declare(
    "jn_transition_topk_forward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32,
     _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_transition_topk_backward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
     _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare(
    "jn_transition_dense_forward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P,
     _P],
)
_declare("jn_transition_dense_workspace_bytes", [_I64] * 7, _SZ)
_declare(
    "jn_transition_dense_backward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare(
    "jn_propagation_dense_forward",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _P, _P, _P, _P, _P],
)
_declare("jn_propagation_dense_workspace_bytes", [_I64] * 5 + [_I32, _I32], _SZ)
_declare("jn_propagation_dense_chunked_workspace_bytes", [_I64] * 5 + [_I32, _I64, _I32], _SZ)
_declare(
    "jn_propagation_dense_forward_chunked",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I64, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_propagation_dense_backward_chunked",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I64, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_propagation_dense_backward",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare("jn_propagation_dense_multihead_chunk_bytes", [_I64] * 3, _SZ)
_declare("jn_propagation_dense_multihead_workspace_bytes", [_I64] * 6 + [_I32, _I64], _SZ)
_declare(
    "jn_propagation_dense_forward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I64, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_propagation_dense_backward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I64,
     _I32, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_transition_dense_forward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P,
     _P, _P, _P],
)
_declare("jn_transition_dense_multihead_workspace_bytes", [_I64] * 8, _SZ)
_declare(
    "jn_transition_dense_backward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
     _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare("jn_propagation_topk_forward_multihead_workspace_bytes", [_I64] * 4, _SZ)
_declare(
    "jn_propagation_topk_forward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P,
     _P, _SZ, _P, _SZ, _P],
)
_declare("jn_propagation_topk_multihead_workspace_bytes", [_I64] * 7, _SZ)
_declare(
    "jn_propagation_topk_backward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_propagation_window_forward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P],
)
_declare("jn_propagation_window_multihead_workspace_bytes", [_I64] * 7, _SZ)
_declare(
    "jn_propagation_window_backward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare("jn_transition_topk_multihead_workspace_bytes", [_I64] * 9, _SZ)
_declare(
    "jn_transition_topk_forward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32,
     _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)
_declare(
    "jn_transition_topk_backward_multihead",
    [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
     _I64, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
)

_declare("jn_lowrank_topk_select_heads", [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ, _P])
_declare("jn_lowrank_topk_select_heads_workspace_bytes", [_I64] * 4, _SZ)
_declare("jn_softsign_backward", [_P, _P, _I64, _P, _P])
_declare("jn_softmax_backward", [_P, _P, _I64, _I64, _P, _P])
_declare("jn_edge_aggregate", [_P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P])
_declare("jn_edge_reduce_backward",
         [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P])
_declare("jn_edge_reduce_backward_workspace_bytes", [_I64] * 4, _SZ)
_declare("jn_route_topk_aggregate", [_P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P, _P, _P, _P, _P, _SZ, _P])
_declare("jn_route_topk_aggregate_workspace_bytes", [_I64] * 4, _SZ)
_declare("jn_lowrank_pair_backward",
         [_P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
          _P, _P, _P, _P, _P, _P, _P, _SZ, _P])
_declare("jn_lowrank_pair_backward_workspace_bytes", [_I64] * 7, _SZ)

_declare("jn_unit_scale_forward", [_P, _I64, _I64, _F, _P, _P])
_declare("jn_unit_scale_backward", [_P, _P, _I64, _I64, _F, _P, _P])

# bf16 layers: the fp32 entry points' argument lists with bf16 value tensors
for _name in ("jn_propagation_topk_forward", "jn_propagation_topk_backward", "jn_propagation_window_forward",
              "jn_propagation_window_backward", "jn_transition_topk_forward", "jn_transition_topk_backward",
              "jn_propagation_dense_forward", "jn_propagation_dense_backward", "jn_propagation_dense_forward_chunked",
              "jn_propagation_dense_backward_chunked", "jn_transition_dense_forward", "jn_transition_dense_backward"):
    _declare(_name + "_bf16", list(getattr(_LIB, _name).argtypes))

ABI_VERSION = int(_LIB.jn_abi_version())

_COMPRESS_KINDS = {"softsign": 0, "signed_abs_softmax": 1, "signed_entmax15": 2}
# Limits of the library's kernels.  A call beyond one raises NotImplementedError
# (a RuntimeError subclass) before anything is launched, so callers that have
# another path for such shapes (implementation="kernel") can take it.
MAX_TOPK = 64          # edges per row of the register top-k select (larger k: scored rows)
MAX_TOPK_LARGE = 4096  # edges per row of a propagation top-k (scored rows, radix select)
MAX_RANK = 1024        # low-rank score rank of one head
MAX_RANK_HEADS = 128   # ranks over all heads of a multi-head score
MAX_SELECT_KEYS = 65535  # keys the register select ranks per batch element (more: scored rows)
CAUSAL_DENSE_MIN_NODES = 128  # full causal windows from this many nodes run on the dense MFMA path
MAX_HEADS = 8          # heads of a max-aggregated multi-head score

_SUPPORTED_OPS = (
    "propagation_topk",
    "propagation_window",
    "propagation_dense",
    "transition_pairwise_topk",
    "transition_pairwise_dense",
    "low_rank_topk_select",
    # the reference extension's raw edge ops (see the raw-op section below)
    "softsign_backward_cuda",
    "softmax_backward_cuda",
    "query_topk_reduce_cuda",
    "query_topk_reduce_backward_cuda",
    "low_rank_propagation_topk_forward_cuda",
    "low_rank_pairwise_topk_forward_cuda",
    "low_rank_pairwise_topk_backward_cuda",
)
_ROUTE_COMPRESS_KINDS = {"softmax": 0, "signed_abs_softmax": 1, "signed_entmax15": 2}
MAX_ROUTE_TOPK = 64  # routes over every destination (more run dense); the raw pairwise op's k range


def supported_ops() -> list[str]:
    return list(_SUPPORTED_OPS)


def supported_devices() -> list[str]:
    # ROCm PyTorch reports HIP devices with device.type == "cuda".
    return ["cuda"]


def backend_name() -> str:
    return "hip_gfx950"


def loaded_library() -> str:
    return str(library_path())


def profile_enable(on: bool = True) -> None:
    """Start (or stop) per-kernel HIP-event timing inside the library."""
    _check(_LIB.jn_profile_enable(1 if on else 0))


def set_gemm_tile(tile: int = 0) -> None:
    """Force the GEMM workgroup tile (64 or 128; 32 on the projection products)
    for later calls; 0 restores the per-call choice."""
    _check(_LIB.jn_set_gemm_tile(int(tile)))


WINDOW_BAND = 0
WINDOW_EDGES = 1


def set_window_kernels(mode: int = WINDOW_BAND) -> None:
    """Window propagation kernels for later calls (process-wide): WINDOW_BAND
    (default) multiplies each 64-row tile's span of the causal band on MFMAs
    where it fits (band <= 128 wide, 16-byte value rows); WINDOW_EDGES runs the
    per-edge gather kernels for every window."""
    _check(_LIB.jn_set_window_kernels(int(mode)))


def set_side_streams(on: bool = True) -> None:
    """Whether the library may run independent kernels of a call on its side
    stream beside the caller's (True, the default) or runs every kernel on the
    caller's stream (False: each kernel can be timed alone).  Process-wide;
    results are bit-identical either way."""
    _check(_LIB.jn_set_side_streams(1 if on else 0))


SELECT_SPLIT_F16 = 0
SELECT_F32 = 1
SELECT_SPLIT_F16_WAVE = 2
SELECT_SPLIT_F16_COOP4 = 4
SELECT_SPLIT_F16_KEYSPLIT = 5
SELECT_SPLIT_F16_REGISTER = 6


def set_select_mode(mode: int = SELECT_SPLIT_F16) -> None:
    """Score arithmetic of the top-k select for later calls (process-wide).

    SELECT_SPLIT_F16 (default): fp16 MFMAs over two-term fp16 operand splits,
    fp32 accumulation, the kernel chosen per call; SELECT_F32: fp32 MFMAs.
    The split arithmetic on one kernel only: SELECT_SPLIT_F16_WAVE (per-wave
    streaming), SELECT_SPLIT_F16_COOP4 (LDS-staged cooperative, rank <= 64)
    and SELECT_SPLIT_F16_KEYSPLIT (the four waves of a workgroup split the keys
    of 16 query rows, k <= 16).  The default takes rows of at most 1024 keys
    (one head, fp32, k <= 64) on the small-key select instead (fp32 MFMA score
    rows in LDS, a radix select per row); SELECT_SPLIT_F16_REGISTER keeps them
    on the split kernels.  Every mode selects the same entries."""
    _check(_LIB.jn_set_select_mode(int(mode)))


def profile_collect() -> dict[str, tuple[int, float]]:
    """Wait for the recorded kernels; return {kernel: (launches, total_ms)} and clear."""
    buf = ctypes.create_string_buffer(1 << 16)
    _check(_LIB.jn_profile_collect(buf, len(buf)))
    out: dict[str, tuple[int, float]] = {}
    for line in buf.value.decode().splitlines():
        name, count, total = line.rsplit(" ", 2)
        out[name] = (int(count), float(total))
    return out


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"jakal_net HIP library error {rc}: {_LIB.jn_last_error().decode(errors='replace')}")


def _ptr(t: Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*tensors: Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"jakal_net_native ops need GPU tensors, got a tensor on {t.device}.")
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError("jakal_net_native ops need all tensors on one device.")
    assert device is not None
    return device


def _f32(t: Tensor | None) -> Tensor | None:
    return None if t is None else t.float().contiguous()


def _same_storage_view(a: Tensor, b: Tensor) -> bool:
    return a is b or (
        a.data_ptr() == b.data_ptr() and a.shape == b.shape and a.stride() == b.stride() and a.dtype == b.dtype
    )


# ---------------------------------------------------------------------------
# edge-list propagation (top-k and window)
# ---------------------------------------------------------------------------
_EDGE_OPS = {
    # (mode, multi-head): (forward, workspace_bytes, backward)
    ("topk", False): ("jn_propagation_topk_forward", "jn_propagation_topk_workspace_bytes",
                      "jn_propagation_topk_backward"),
    ("window", False): ("jn_propagation_window_forward", "jn_propagation_window_workspace_bytes",
                        "jn_propagation_window_backward"),
    ("topk", True): ("jn_propagation_topk_forward_multihead", "jn_propagation_topk_multihead_workspace_bytes",
                     "jn_propagation_topk_backward_multihead"),
    ("window", True): ("jn_propagation_window_forward_multihead", "jn_propagation_window_multihead_workspace_bytes",
                       "jn_propagation_window_backward_multihead"),
    ("topk", "bf16"): ("jn_propagation_topk_forward_bf16", "jn_propagation_topk_workspace_bytes",
                       "jn_propagation_topk_backward_bf16"),
    ("window", "bf16"): ("jn_propagation_window_forward_bf16", "jn_propagation_window_workspace_bytes",
                         "jn_propagation_window_backward_bf16"),
}


def _edges_per_row(mode: str, param: int, N: int) -> int:
    return param if mode == "topk" else min(param + 1, N)


class _PropagationEdges(torch.autograd.Function):
    """Differentiable low-rank propagation over an edge list on the HIP library.

    mode "topk" (param = k) selects each row's k best sources; mode "window"
    (param = window) takes the causal band j in [i - window, i].  Inputs (all
    fp32, contiguous): layer_val X [B,N,Din], projected_state [B,N],
    projected_val [B,N,Dout] or None when it is X itself, V and U [r,Din],
    w_hat [r], bias [] or None.  With heads > 1 the r ranks are `heads`
    equal head slices (max-aggregated scores) and bias is [heads].  With
    bf16, X and pv are bf16 (one head) and delta_val comes back in bf16."""

    @staticmethod
    def forward(ctx, X, ps, pv, V, U, w_hat, bias, mode: str, param: int, compress: int, heads: int = 1,  # noqa: N803
                bf16: bool = False):
        B, N, Din = X.shape
        pv_is_x = pv is None
        pv_t = X if pv_is_x else pv
        Dout = pv_t.shape[-1]
        r = U.shape[0]
        mh = heads > 1
        rank_arg = [r // heads, heads] if mh else [r]
        k = _edges_per_row(mode, param, N)
        dev = X.device
        variant = "bf16" if bf16 else mh
        fwd = getattr(_LIB, _EDGE_OPS[mode, variant][0])
        with torch.cuda.device(dev):
            ds = torch.empty(B, N, device=dev, dtype=torch.float32)
            dv = torch.empty(B, N, Dout, device=dev, dtype=torch.bfloat16 if bf16 else torch.float32)
            proj = torch.empty(B * N, 2 * r, device=dev, dtype=torch.float32)
            idx = torch.empty(B, N, k, device=dev, dtype=torch.int32)
            score = torch.empty(B, N, k, device=dev, dtype=torch.float32)
            head = torch.empty(B, N, k, device=dev, dtype=torch.uint8) if mh else None
            args = [
                _ptr(X), _ptr(ps), _ptr(pv_t), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias),
                B, N, Din, Dout, *rank_arg, param, compress,
                _ptr(ds), _ptr(dv), _ptr(proj), _ptr(idx), _ptr(score),
            ]
            if mh:
                args.append(_ptr(head))
            layout = None
            if mode == "topk":
                # the edges grouped by key for the backward, built beside the
                # forward's row pass when a backward will follow
                if EDGE_LAYOUT and any(ctx.needs_input_grad[:7]):
                    layout_bytes = int(_LIB.jn_propagation_topk_layout_bytes(B, N, k))
                    layout = torch.empty(layout_bytes, device=dev, dtype=torch.uint8)
                    args += [_ptr(layout), layout_bytes]
                else:
                    args += [None, 0]
                # the select's scratch
                ws_bytes = int(_LIB.jn_propagation_topk_forward_multihead_workspace_bytes(B, N, *rank_arg) if mh
                               else _LIB.jn_propagation_topk_forward_workspace_bytes(B, N, r))
                ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
                args += [_ptr(ws), ws_bytes]
            _check(fwd(*args, _stream(dev)))
        ctx.save_for_backward(X, ps, pv_t, V, U, w_hat, proj, idx, score, head)
        ctx.edge_layout = layout
        ctx.meta = (mode, param, compress, pv_is_x, bias is not None, heads, bf16)
        ctx.mark_non_differentiable(idx, score)
        ctx.set_materialize_grads(False)  # no zero-filled gradients for the edge-list outputs
        return ds, dv, idx, score

    @staticmethod
    def backward(ctx, g_ds, g_dv, _g_idx=None, _g_score=None):
        X, ps, pv, V, U, w_hat, proj, idx, score, head = ctx.saved_tensors
        mode, param, compress, pv_is_x, has_bias, heads, bf16 = ctx.meta
        mh = heads > 1
        _, ws_name, bwd_name = _EDGE_OPS[mode, "bf16" if bf16 else mh]
        B, N, Din = X.shape
        Dout = pv.shape[-1]
        r = U.shape[0]
        rank_arg = [r // heads, heads] if mh else [r]
        dev = X.device
        need = ctx.needs_input_grad
        ds_used = g_ds is not None  # projected_state reaches delta_state only
        with torch.cuda.device(dev):
            vdt = torch.bfloat16 if bf16 else torch.float32
            g_ds = torch.zeros(B, N, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, N, Dout, device=dev, dtype=vdt) if g_dv is None else g_dv.to(vdt).contiguous()
            gX = torch.empty_like(X) if need[0] else None
            gps = torch.empty_like(ps) if need[1] and ds_used else None
            gpv = torch.empty_like(pv) if (not pv_is_x and need[2]) else None
            gV = torch.empty_like(V)
            gU = torch.empty_like(U)
            gw = torch.empty_like(w_hat)
            gb = torch.empty((heads,) if mh else (), device=dev, dtype=torch.float32) if has_bias else None
            ws_bytes = int(getattr(_LIB, ws_name)(B, N, Din, Dout, *rank_arg, param))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            edge_args = [_ptr(idx), _ptr(score)] + ([_ptr(head)] if mh else [])
            layout_arg = [_ptr(ctx.edge_layout)] if mode == "topk" else []
            _check(
                getattr(_LIB, bwd_name)(
                    _ptr(X), _ptr(ps), _ptr(pv), _ptr(U), _ptr(V), _ptr(w_hat),
                    _ptr(proj), *edge_args, _ptr(g_ds), _ptr(g_dv),
                    B, N, Din, Dout, *rank_arg, param, compress, 1 if pv_is_x else 0,
                    _ptr(gX), _ptr(gps), _ptr(gpv), _ptr(gU), _ptr(gV), _ptr(gw), _ptr(gb),
                    *layout_arg, _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (
            gX,
            gps,
            gpv,
            gV if need[3] else None,
            gU if need[4] else None,
            gw if need[5] else None,
            gb if (has_bias and need[6]) else None,
            None,
            None,
            None,
            None,
            None,
        )


UNIT_SCALE_EPS = 1e-6  # LowRankBilinearPairwise.normalized_weight's clamp (modules.py:85-87)


class _UnitScale(torch.autograd.Function):
    """w / max(||w||_2, 1e-6) per row of an fp32 [rows, r] stack, one kernel
    forward and one backward (jn_unit_scale_*)."""

    @staticmethod
    def forward(ctx, w):  # noqa: D401
        out = torch.empty_like(w)
        with torch.cuda.device(w.device):
            _check(_LIB.jn_unit_scale_forward(_ptr(w), w.shape[0], w.shape[1], UNIT_SCALE_EPS, _ptr(out),
                                              _stream(w.device)))
        ctx.save_for_backward(w)
        return out

    @staticmethod
    def backward(ctx, g):
        (w,) = ctx.saved_tensors
        g = g.float().contiguous()
        gw = torch.empty_like(w)
        with torch.cuda.device(w.device):
            _check(_LIB.jn_unit_scale_backward(_ptr(w), _ptr(g), w.shape[0], w.shape[1], UNIT_SCALE_EPS,
                                               _ptr(gw), _stream(w.device)))
        return gw


def unit_scale(weight: Tensor) -> Tensor:
    """The low-rank score scale w / max(||w||_2, 1e-6) of a [r] vector, or of
    each row of an [H, r] stack, on the HIP library (differentiable).  Same
    values as LowRankBilinearPairwise.normalized_weight (modules.py:85-87) up
    to fp32 rounding of the norm."""
    if not weight.is_cuda or weight.dtype != torch.float32 or weight.dim() not in (1, 2):
        raise NotImplementedError("unit_scale takes an fp32 [r] or [H, r] tensor on a HIP device")
    w2 = weight.contiguous().view(1, -1) if weight.dim() == 1 else weight.contiguous()
    out = _UnitScale.apply(w2)
    return out.view(-1) if weight.dim() == 1 else out


def _bf16_rows(*tensors: Tensor | None) -> bool:
    """True when every given tensor (None: skipped) is bf16: the bf16 entry points apply."""
    return all(t is None or t.dtype == torch.bfloat16 for t in tensors)


def _bf16(t: Tensor | None) -> Tensor | None:
    return None if t is None else t.contiguous()


EDGE_LAYOUT = True  # top-k forwards group their edges by key for the backward


def set_edge_layout(on: bool = True) -> None:
    """Whether top-k propagation forwards that a backward will follow build the
    edge layout (the edges grouped by key) beside their row pass and hand it to
    the backward (True, the default), or leave the grouping to the backward.
    Results are identical either way."""
    global EDGE_LAYOUT
    EDGE_LAYOUT = bool(on)


DENSE_EDGE_BYTES = 512 << 20  # edge-matrix bytes above which dense propagation runs in batch chunks


def set_dense_edge_bytes(limit: int = 512 << 20) -> None:
    """Edge-matrix bytes (B * N * N * 4) up to which dense propagation keeps the
    whole edge matrix from forward to backward; above it the forward and
    backward run chunks of batch elements whose edge matrices fit the limit,
    and the backward rebuilds each chunk's edges from the saved projections."""
    global DENSE_EDGE_BYTES
    DENSE_EDGE_BYTES = int(limit)


class _PropagationDense(torch.autograd.Function):
    """Differentiable dense low-rank propagation on the HIP library.  Inputs as
    _PropagationEdges; causal keeps only sources j <= i in row i.  Small
    problems keep the edge matrix for the backward; larger ones run in batch
    chunks of at most DENSE_EDGE_BYTES of edges and rebuild them.  With bf16,
    X and pv are bf16 and delta_val comes back in bf16 (the *_bf16 entry
    points); the edge matrix stays fp32."""

    @staticmethod
    def _entry(name: str, bf16: bool):
        return getattr(_LIB, name + "_bf16" if bf16 else name)

    @staticmethod
    def forward(ctx, X, ps, pv, V, U, w_hat, bias, compress: int, causal: bool = False,  # noqa: N803
                bf16: bool = False):
        B, N, Din = X.shape
        pv_is_x = pv is None
        pv_t = X if pv_is_x else pv
        Dout = pv_t.shape[-1]
        r = U.shape[0]
        dev = X.device
        edge_bytes = N * N * 4
        chunk = B if B * edge_bytes <= DENSE_EDGE_BYTES else max(1, DENSE_EDGE_BYTES // edge_bytes)
        with torch.cuda.device(dev):
            ds = torch.empty(B, N, device=dev, dtype=torch.float32)
            dv = torch.empty(B, N, Dout, device=dev, dtype=torch.bfloat16 if bf16 else torch.float32)
            proj = torch.empty(B * N, 2 * r, device=dev, dtype=torch.float32)
            if chunk >= B:
                edges = torch.empty(B, N, N, device=dev, dtype=torch.float32)
                _check(
                    _PropagationDense._entry("jn_propagation_dense_forward", bf16)(
                        _ptr(X), _ptr(ps), _ptr(pv_t), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias),
                        B, N, Din, Dout, r, compress, 1 if causal else 0, _ptr(ds), _ptr(dv), _ptr(proj),
                        _ptr(edges), _stream(dev),
                    )
                )
            else:
                # the forward's chunk buffer keeps the last chunk's edges for the backward
                ws_bytes = int(_LIB.jn_propagation_dense_chunked_workspace_bytes(B, N, Din, Dout, r, compress,
                                                                                 chunk, 0))
                edges = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
                _check(
                    _PropagationDense._entry("jn_propagation_dense_forward_chunked", bf16)(
                        _ptr(X), _ptr(ps), _ptr(pv_t), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias),
                        B, N, Din, Dout, r, compress, 1 if causal else 0, chunk, _ptr(ds), _ptr(dv), _ptr(proj),
                        _ptr(edges), ws_bytes, _stream(dev),
                    )
                )
        ctx.save_for_backward(X, ps, pv_t, V, U, w_hat, proj, edges, bias)
        ctx.meta = (compress, pv_is_x, bias is not None, bool(causal), chunk, bool(bf16))
        ctx.edges_consumed = False
        ctx.set_materialize_grads(False)  # an unused delta_state arrives as None
        return ds, dv

    @staticmethod
    def backward(ctx, g_ds, g_dv):
        X, ps, pv, V, U, w_hat, proj, edges, bias = ctx.saved_tensors
        compress, pv_is_x, has_bias, causal, chunk, bf16 = ctx.meta
        # a softsign backward writes the score gradient over the saved edge
        # matrix (no [B, N, N] workspace); a later backward (retain_graph)
        # rebuilds the edges there from the saved projections, as the chunked
        # backward does for its chunks
        if chunk < X.shape[0] or ctx.edges_consumed:
            return _PropagationDense._backward_chunked(ctx, X, ps, pv, V, U, w_hat, proj, edges, bias, g_ds, g_dv)
        reuse = 1 if compress == 0 else 0
        ctx.edges_consumed = bool(reuse)
        B, N, Din = X.shape
        Dout = pv.shape[-1]
        r = U.shape[0]
        dev = X.device
        need = ctx.needs_input_grad
        ds_used = g_ds is not None  # projected_state reaches delta_state only
        with torch.cuda.device(dev):
            vdt = torch.bfloat16 if bf16 else torch.float32
            g_ds = torch.zeros(B, N, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, N, Dout, device=dev, dtype=vdt) if g_dv is None else g_dv.to(vdt).contiguous()
            gX = torch.empty_like(X) if need[0] else None
            gps = torch.empty_like(ps) if need[1] and ds_used else None
            gpv = torch.empty_like(pv) if (not pv_is_x and need[2]) else None
            gV, gU, gw = torch.empty_like(V), torch.empty_like(U), torch.empty_like(w_hat)
            gb = torch.empty((), device=dev, dtype=torch.float32) if has_bias else None
            ws_bytes = int(_LIB.jn_propagation_dense_workspace_bytes(B, N, Din, Dout, r, compress, reuse))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            _check(
                _PropagationDense._entry("jn_propagation_dense_backward", bf16)(
                    _ptr(X), _ptr(ps), _ptr(pv), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(proj), _ptr(edges),
                    _ptr(g_ds), _ptr(g_dv), B, N, Din, Dout, r, compress, 1 if causal else 0, 1 if pv_is_x else 0,
                    reuse, _ptr(gX), _ptr(gps), _ptr(gpv), _ptr(gU), _ptr(gV), _ptr(gw), _ptr(gb),
                    _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (gX, gps, gpv, gV if need[3] else None, gU if need[4] else None, gw if need[5] else None,
                gb if (has_bias and need[6]) else None, None, None, None)

    @staticmethod
    def _backward_chunked(ctx, X, ps, pv, V, U, w_hat, proj, edge_chunk, bias, g_ds, g_dv):
        compress, pv_is_x, has_bias, causal, chunk, bf16 = ctx.meta
        chunk = min(chunk, X.shape[0])  # a whole saved edge matrix is one chunk
        # the chunk buffer holds the forward's last chunk until a softsign
        # backward writes its gradient there; a later backward rebuilds it too
        resident = 0 if ctx.edges_consumed else 1
        ctx.edges_consumed = ctx.edges_consumed or compress == 0
        B, N, Din = X.shape
        Dout = pv.shape[-1]
        r = U.shape[0]
        dev = X.device
        need = ctx.needs_input_grad
        ds_used = g_ds is not None  # projected_state reaches delta_state only
        with torch.cuda.device(dev):
            vdt = torch.bfloat16 if bf16 else torch.float32
            g_ds = torch.zeros(B, N, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, N, Dout, device=dev, dtype=vdt) if g_dv is None else g_dv.to(vdt).contiguous()
            gX = torch.empty_like(X) if need[0] else None
            gps = torch.empty_like(ps) if need[1] and ds_used else None
            gpv = torch.empty_like(pv) if (not pv_is_x and need[2]) else None
            gV, gU, gw = torch.empty_like(V), torch.empty_like(U), torch.empty_like(w_hat)
            gb = torch.empty((), device=dev, dtype=torch.float32) if has_bias else None
            ws_bytes = int(_LIB.jn_propagation_dense_chunked_workspace_bytes(B, N, Din, Dout, r, compress, chunk, 1))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            _check(
                _PropagationDense._entry("jn_propagation_dense_backward_chunked", bf16)(
                    _ptr(X), _ptr(ps), _ptr(pv), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias), _ptr(proj),
                    _ptr(edge_chunk), _ptr(g_ds), _ptr(g_dv), B, N, Din, Dout, r, compress, 1 if causal else 0,
                    1 if pv_is_x else 0, chunk, resident, _ptr(gX), _ptr(gps), _ptr(gpv), _ptr(gU), _ptr(gV),
                    _ptr(gw), _ptr(gb), _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (gX, gps, gpv, gV if need[3] else None, gU if need[4] else None, gw if need[5] else None,
                gb if (has_bias and need[6]) else None, None, None, None)


class _PropagationDenseMultihead(torch.autograd.Function):
    """Dense low-rank propagation with max-aggregated multi-head scores on the
    HIP library.  Inputs as _PropagationEdges with heads > 1 (U, V, w_hat the
    heads' ranks stacked flat, bias [heads] or None); causal keeps only
    sources j <= i.  The forward keeps a chunk of batch elements' edge
    matrices and winning heads (the whole batch when it fits DENSE_EDGE_BYTES)
    for the backward, which rebuilds the other chunks from the projections."""

    @staticmethod
    def forward(ctx, X, ps, pv, V, U, w_hat, bias, compress: int, causal: bool, heads: int):  # noqa: N803
        B, N, Din = X.shape
        pv_is_x = pv is None
        pv_t = X if pv_is_x else pv
        Dout = pv_t.shape[-1]
        R = U.shape[0]
        dev = X.device
        per = N * N * 5  # fp32 edge and uint8 head per pair
        chunk = B if B * per <= DENSE_EDGE_BYTES else max(1, DENSE_EDGE_BYTES // per)
        with torch.cuda.device(dev):
            ds = torch.empty(B, N, device=dev, dtype=torch.float32)
            dv = torch.empty(B, N, Dout, device=dev, dtype=torch.float32)
            proj = torch.empty(B * N, 2 * R, device=dev, dtype=torch.float32)
            cbytes = int(_LIB.jn_propagation_dense_multihead_chunk_bytes(B, N, chunk))
            edge_chunk = torch.empty(max(cbytes, 1), device=dev, dtype=torch.uint8)
            _check(
                _LIB.jn_propagation_dense_forward_multihead(
                    _ptr(X), _ptr(ps), _ptr(pv_t), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias),
                    B, N, Din, Dout, R // heads, heads, compress, 1 if causal else 0, chunk,
                    _ptr(ds), _ptr(dv), _ptr(proj), _ptr(edge_chunk), cbytes, _stream(dev),
                )
            )
        ctx.save_for_backward(X, ps, pv_t, V, U, w_hat, proj, edge_chunk, bias)
        ctx.meta = (compress, pv_is_x, bias is not None, bool(causal), chunk, heads)
        ctx.edges_consumed = False
        ctx.set_materialize_grads(False)  # an unused delta_state arrives as None
        return ds, dv

    @staticmethod
    def backward(ctx, g_ds, g_dv):
        X, ps, pv, V, U, w_hat, proj, edge_chunk, bias = ctx.saved_tensors
        compress, pv_is_x, has_bias, causal, chunk, heads = ctx.meta
        # the chunk holds the forward's last edges until a softsign backward
        # writes its gradient there; a later backward rebuilds them
        resident = 0 if ctx.edges_consumed else 1
        ctx.edges_consumed = ctx.edges_consumed or compress == 0
        B, N, Din = X.shape
        Dout = pv.shape[-1]
        R = U.shape[0]
        dev = X.device
        need = ctx.needs_input_grad
        ds_used = g_ds is not None  # projected_state reaches delta_state only
        with torch.cuda.device(dev):
            g_ds = torch.zeros(B, N, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, N, Dout, device=dev) if g_dv is None else g_dv.float().contiguous()
            gX = torch.empty_like(X) if need[0] else None
            gps = torch.empty_like(ps) if need[1] and ds_used else None
            gpv = torch.empty_like(pv) if (not pv_is_x and need[2]) else None
            gV, gU, gw = torch.empty_like(V), torch.empty_like(U), torch.empty_like(w_hat)
            gb = torch.empty(heads, device=dev, dtype=torch.float32) if has_bias else None
            ws_bytes = int(_LIB.jn_propagation_dense_multihead_workspace_bytes(B, N, Din, Dout, R // heads, heads,
                                                                               compress, chunk))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            _check(
                _LIB.jn_propagation_dense_backward_multihead(
                    _ptr(X), _ptr(ps), _ptr(pv), _ptr(U), _ptr(V), _ptr(w_hat), _ptr(bias), _ptr(proj),
                    _ptr(edge_chunk), edge_chunk.numel(), _ptr(g_ds), _ptr(g_dv), B, N, Din, Dout, R // heads,
                    heads, compress, 1 if causal else 0, 1 if pv_is_x else 0, chunk, resident,
                    _ptr(gX), _ptr(gps), _ptr(gpv), _ptr(gU), _ptr(gV), _ptr(gw), _ptr(gb),
                    _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (gX, gps, gpv, gV if need[3] else None, gU if need[4] else None, gw if need[5] else None,
                gb if (has_bias and need[6]) else None, None, None, None)


def dense_bf16_shapes_ok(nodes: int, out_dim: int) -> bool:
    """Whether a bf16 dense layer of these sizes runs on the bf16 entry points
    (their N x N products need 128 x 128 tiles of 8-element rows)."""
    return nodes >= 128 and out_dim >= 128 and nodes % 8 == 0 and out_dim % 8 == 0


def propagation_dense(
    pairwise_kind: str,
    weight: Tensor,
    bias: Tensor | None,
    in_weight: Tensor | None,
    in_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    source_state: Tensor | None,
    target_block_size: int,
    source_block_size: int,
    _causal: bool = False,
) -> tuple[Tensor, Tensor]:
    """Dense propagation over all N x N pairs; signature of jakal_net_native.cpp:5962-5976.

    The trailing ``_causal`` (no counterpart in the reference signature) keeps
    only sources j <= i in row i: propagation_window's full causal window.

    With ``source_state`` the edges are weighted by it per source, which
    equals the unweighted op on (source_state, source_state * projected_val)
    (jakal_net_native.cpp:5991-6015); the fold is done here, differentiably."""
    w_hat, bias, V, U, heads = _lowrank_pairwise_args(pairwise_kind, weight, bias, in_weight, in_bias, out_weight,
                                                      out_bias)
    if edge_compress_name not in _COMPRESS_KINDS:
        raise RuntimeError(f"Unsupported edge_compress_name for the HIP backend: {edge_compress_name!r}.")
    if target_block_size <= 0 or source_block_size <= 0:
        raise RuntimeError("block sizes must be positive.")
    _require_gpu(layer_val, projected_state, projected_val, w_hat, V, U, bias, source_state)
    if source_state is not None and source_state.numel() > 0:
        projected_val = projected_val * source_state.unsqueeze(-1)
        projected_state = source_state
    batch_shape = tuple(layer_val.shape[:-2])
    N, Din = layer_val.shape[-2], layer_val.shape[-1]
    Dout = projected_val.shape[-1]
    pv_is_x = _same_storage_view(projected_val, layer_val)
    # bf16 layers keep bf16 value rows on the bf16 MFMA products when the
    # shapes fit their tiles (one head); anything else computes in fp32
    bf16 = heads == 1 and _bf16_rows(layer_val, projected_val) and dense_bf16_shapes_ok(N, Dout)
    rows = _bf16 if bf16 else _f32
    X = rows(layer_val.reshape(-1, N, Din))
    ps = _f32(projected_state.reshape(-1, N))
    pv = None if pv_is_x else rows(projected_val.reshape(-1, N, Dout))
    if heads > 1:
        ds, dv = _PropagationDenseMultihead.apply(X, ps, pv, _f32(V), _f32(U), _f32(w_hat), _f32(bias),
                                                  _COMPRESS_KINDS[edge_compress_name], _causal, heads)
    else:
        ds, dv = _PropagationDense.apply(X, ps, pv, _f32(V), _f32(U), _f32(w_hat), _f32(bias),
                                         _COMPRESS_KINDS[edge_compress_name], _causal, bf16)
    return (ds.reshape(*batch_shape, N).to(projected_state.dtype),
            dv.reshape(*batch_shape, N, Dout).to(projected_val.dtype))


def _lowrank_pairwise_args(kind, weight, bias, in_weight, in_bias, out_weight, out_bias):
    """(w_hat [R], bias, V [R, D], U [R, D], heads) of a low-rank pairwise spec.

    A ``multihead_max_low_rank_bilinear`` spec stacks H heads on a leading axis
    (weight [H, r], bias [H], projections [H, r, D]); they are passed flat as
    R = H * r ranks, head h owning ranks [h * r, (h + 1) * r)."""
    if kind not in ("low_rank_bilinear", "multihead_max_low_rank_bilinear"):
        raise TypeError(f"jakal_net_native supports pairwise kinds 'low_rank_bilinear' and "
                        f"'multihead_max_low_rank_bilinear', got {kind!r}.")
    if in_weight is None or out_weight is None:
        raise RuntimeError("Low-rank bilinear pairwise kernel is missing projection weights.")
    if in_bias is not None or out_bias is not None:
        raise TypeError("low_rank_bilinear projections carry no bias.")
    if kind == "low_rank_bilinear":
        _check_rank(out_weight.shape[0])
        return weight, bias, in_weight, out_weight, 1
    return _flatten_heads(weight, bias, in_weight, out_weight)


def _flatten_heads(core, bias, first, second):
    """Stacked heads ([H, r] core, [H] bias, [H, r, D] projections) as flat ranks, plus H."""
    if core.dim() != 2 or first.dim() != 3 or second.dim() != 3:
        raise RuntimeError("multi-head weights must be stacked [heads, rank] and [heads, rank, dim].")
    heads, rank = core.shape
    if heads > MAX_HEADS:
        raise NotImplementedError(f"the HIP library takes up to {MAX_HEADS} heads (got {heads}).")
    _check_rank(heads * rank, MAX_RANK_HEADS)
    if bias is not None and bias.numel() != heads:
        raise RuntimeError("multi-head bias must hold one value per head.")
    flat_bias = None if bias is None else bias.reshape(heads)
    if heads == 1:
        return core[0], None if bias is None else bias.reshape(()), first[0], second[0], 1
    return core.reshape(-1), flat_bias, first.reshape(heads * rank, -1), second.reshape(heads * rank, -1), heads


def _check_rank(rank: int, limit: int = MAX_RANK) -> None:
    if rank > limit:
        raise NotImplementedError(f"the HIP library scores ranks up to {limit} here (got {rank}).")


def _check_select(k: int, limit: int = MAX_TOPK_LARGE) -> None:
    """A top-k select of k edges per row of any number of keys: the register
    select takes k <= MAX_TOPK of at most MAX_SELECT_KEYS keys (and multi-head
    scores of at most four 32-rank K-steps), the scored-rows select the rest up
    to MAX_TOPK_LARGE; `limit` is the caller's own bound."""
    if k > limit:
        raise NotImplementedError(f"the HIP top-k select keeps up to {limit} edges per row here (got {k}).")


def _propagation_edges(mode, pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias,
                       edge_compress_name, layer_val, projected_state, projected_val, param, target_block_size,
                       source_block_size):
    w_hat, bias, V, U, heads = _lowrank_pairwise_args(pairwise_kind, weight, bias, in_weight, in_bias, out_weight,
                                                      out_bias)
    if edge_compress_name not in _COMPRESS_KINDS:
        raise RuntimeError(f"Unsupported edge_compress_name for the HIP backend: {edge_compress_name!r}.")
    if target_block_size <= 0 or source_block_size <= 0:
        raise RuntimeError("block sizes must be positive.")
    _require_gpu(layer_val, projected_state, projected_val, w_hat, V, U, bias)
    batch_shape = tuple(layer_val.shape[:-2])
    N, Din = layer_val.shape[-2], layer_val.shape[-1]
    Dout = projected_val.shape[-1]
    pv_is_x = _same_storage_view(projected_val, layer_val)
    # bf16 layers keep bf16 value rows (one head); anything else computes in fp32
    bf16 = heads == 1 and _bf16_rows(layer_val, projected_val)
    rows = _bf16 if bf16 else _f32
    X = rows(layer_val.reshape(-1, N, Din))
    ps = _f32(projected_state.reshape(-1, N))
    pv = None if pv_is_x else rows(projected_val.reshape(-1, N, Dout))
    ds, dv, idx, score = _PropagationEdges.apply(
        X, ps, pv, _f32(V), _f32(U), _f32(w_hat), _f32(bias), mode, int(param), _COMPRESS_KINDS[edge_compress_name],
        heads, bf16,
    )
    k = idx.shape[-1]
    return (
        ds.reshape(*batch_shape, N).to(projected_state.dtype),
        dv.reshape(*batch_shape, N, Dout).to(projected_val.dtype),
        idx.reshape(*batch_shape, N, k),
        score.reshape(*batch_shape, N, k),
    )


def propagation_topk_selection(
    pairwise_kind: str,
    weight: Tensor,
    bias: Tensor | None,
    in_weight: Tensor | None,
    in_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    target_block_size: int,
    source_block_size: int,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Top-k propagation returning (delta_state, delta_val, topk_index, topk_score).

    Same arguments as ``propagation_topk``; the selection (int32 source
    indices and their scores, best first) is what the forward aggregated."""
    if topk <= 0:
        raise RuntimeError("topk must be positive.")
    N = layer_val.shape[-2]
    k = min(int(topk), N)
    if k == N:
        raise NotImplementedError("top-k with k == N keeps every source: that is dense propagation "
                                  "(propagation_dense, or propagation_topk, which routes it there).")
    _check_select(k)
    return _propagation_edges("topk", pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias,
                              edge_compress_name, layer_val, projected_state, projected_val, k, target_block_size,
                              source_block_size)


def propagation_window_edges(
    pairwise_kind: str,
    weight: Tensor,
    bias: Tensor | None,
    in_weight: Tensor | None,
    in_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    window: int,
    target_block_size: int,
    source_block_size: int,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Window propagation returning (delta_state, delta_val, edge_index, edge_score).

    Row i's slots e < min(window + 1, N) hold source i - (width - 1 - e)
    (index -1 where that is negative) and its score."""
    if window < 0:
        raise RuntimeError("window must be non-negative.")
    return _propagation_edges("window", pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias,
                              edge_compress_name, layer_val, projected_state, projected_val, int(window),
                              target_block_size, source_block_size)


def propagation_window(
    pairwise_kind: str,
    weight: Tensor,
    bias: Tensor | None,
    in_weight: Tensor | None,
    in_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    window: int,
    target_block_size: int,
    source_block_size: int,
) -> tuple[Tensor, Tensor]:
    """Causal-window propagation; signature of jakal_net_native.cpp:6190-6204.

    A window covering every earlier source (window >= N - 1, the causal dense
    query propagation of progressive_b_example.py:1990-2003) on at least
    CAUSAL_DENSE_MIN_NODES nodes runs as causal dense propagation on MFMA
    GEMMs instead of an N-wide edge list."""
    N = layer_val.shape[-2]
    full_causal = window >= N - 1
    if full_causal and N >= CAUSAL_DENSE_MIN_NODES:
        if window < 0:
            raise RuntimeError("window must be non-negative.")
        return propagation_dense(pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias,
                                 edge_compress_name, layer_val, projected_state, projected_val, None,
                                 target_block_size, source_block_size, _causal=True)
    ds, dv, _, _ = propagation_window_edges(
        pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias, edge_compress_name, layer_val,
        projected_state, projected_val, window, target_block_size, source_block_size,
    )
    return ds, dv


def propagation_topk(
    pairwise_kind: str,
    weight: Tensor,
    bias: Tensor | None,
    in_weight: Tensor | None,
    in_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    edge_compress_name: str,
    layer_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    target_block_size: int,
    source_block_size: int,
) -> tuple[Tensor, Tensor]:
    """Top-k propagation; signature of jakal_net_native.cpp:6305-6319.

    ``weight`` is the normalised core weight, ``in_weight`` the source and
    ``out_weight`` the target projection (kernel_common.py:185-192).  With
    k >= N every source is kept, which is dense propagation
    (propagation.py:471, kernel_common.py:433-440)."""
    if topk >= layer_val.shape[-2]:
        return propagation_dense(pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias,
                                 edge_compress_name, layer_val, projected_state, projected_val, None,
                                 target_block_size, source_block_size)
    ds, dv, _, _ = propagation_topk_selection(
        pairwise_kind, weight, bias, in_weight, in_bias, out_weight, out_bias, edge_compress_name, layer_val,
        projected_state, projected_val, topk, target_block_size, source_block_size,
    )
    return ds, dv


# ---------------------------------------------------------------------------
# sparse transition (low-rank pairwise route, top-k destinations per source)
# ---------------------------------------------------------------------------
class _TransitionTopK(torch.autograd.Function):
    """Differentiable SparseTransition routing on the HIP library.

    Inputs (fp32, contiguous): sender strength rho [B,Ns], src_val [B,Ns,Dsrc],
    dst_val [B,Nd,Ddst], projected_state [B,Ns], projected_val [B,Ns,Dv],
    Ws [r,Dsrc], Wt [r,Ddst], w [r] (raw), bias [] or None."""

    @staticmethod
    def forward(ctx, rho, src, dst, ps, pv, Ws, Wt, w, bias, temperature: float, topk: int, compress: int,  # noqa: N803
                heads: int = 1, bf16: bool = False):
        B, Ns, Dsrc = src.shape
        Nd, Ddst = dst.shape[1], dst.shape[2]
        Dv = pv.shape[-1]
        r = Ws.shape[0]
        mh = heads > 1
        rank_arg = [r // heads, heads] if mh else [r]
        k = min(int(topk), Nd)
        dev = src.device
        with torch.cuda.device(dev):
            ds = torch.empty(B, Nd, device=dev, dtype=torch.float32)
            dv = torch.empty(B, Nd, Dv, device=dev, dtype=torch.bfloat16 if bf16 else torch.float32)
            sp = torch.empty(B * Ns, r, device=dev, dtype=torch.float32)
            dp = torch.empty(B * Nd, r, device=dev, dtype=torch.float32)
            idx = torch.empty(B, Ns, k, device=dev, dtype=torch.int32)
            logit = torch.empty(B, Ns, k, device=dev, dtype=torch.float32)
            head = torch.empty(B, Ns, k, device=dev, dtype=torch.uint8) if mh else None
            ws_fn = _LIB.jn_transition_topk_multihead_workspace_bytes if mh else _LIB.jn_transition_topk_workspace_bytes
            ws_bytes = int(ws_fn(B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg, topk))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            fwd = (_LIB.jn_transition_topk_forward_multihead if mh else
                   _LIB.jn_transition_topk_forward_bf16 if bf16 else _LIB.jn_transition_topk_forward)
            _check(
                fwd(
                    _ptr(rho), _ptr(src), _ptr(dst), _ptr(ps), _ptr(pv), _ptr(Ws), _ptr(Wt), _ptr(w), _ptr(bias),
                    float(temperature), B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg, topk, compress,
                    _ptr(ds), _ptr(dv), _ptr(sp), _ptr(dp), _ptr(idx), _ptr(logit), *([_ptr(head)] if mh else []),
                    _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        ctx.save_for_backward(rho, src, dst, ps, pv, Ws, Wt, w, sp, dp, idx, logit, head)
        ctx.meta = (float(temperature), int(topk), compress, bias is not None, heads, bf16)
        ctx.mark_non_differentiable(idx, logit)
        ctx.set_materialize_grads(False)  # no zero-filled gradients for the edge-list outputs
        return ds, dv, idx, logit

    @staticmethod
    def backward(ctx, g_ds, g_dv, _g_idx=None, _g_logit=None):
        rho, src, dst, ps, pv, Ws, Wt, w, sp, dp, idx, logit, head = ctx.saved_tensors
        temperature, topk, compress, has_bias, heads, bf16 = ctx.meta
        B, Ns, Dsrc = src.shape
        Nd, Ddst = dst.shape[1], dst.shape[2]
        Dv = pv.shape[-1]
        r = Ws.shape[0]
        mh = heads > 1
        rank_arg = [r // heads, heads] if mh else [r]
        dev = src.device
        need = ctx.needs_input_grad
        # the projected source state reaches delta_state only
        need_in = list(need[:5])
        need_in[3] = need_in[3] and g_ds is not None
        with torch.cuda.device(dev):
            vdt = torch.bfloat16 if bf16 else torch.float32
            g_ds = torch.zeros(B, Nd, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, Nd, Dv, device=dev, dtype=vdt) if g_dv is None else g_dv.to(vdt).contiguous()
            out = [torch.empty_like(t) if n else None for t, n in zip((rho, src, dst, ps, pv), need_in)]
            gWs = torch.empty_like(Ws) if need[5] else None
            gWt = torch.empty_like(Wt) if need[6] else None
            gw = torch.empty_like(w)
            gb = torch.empty((heads,) if mh else (), device=dev, dtype=torch.float32) if has_bias else None
            ws_fn = _LIB.jn_transition_topk_multihead_workspace_bytes if mh else _LIB.jn_transition_topk_workspace_bytes
            ws_bytes = int(ws_fn(B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg, topk))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            bwd = (_LIB.jn_transition_topk_backward_multihead if mh else
                   _LIB.jn_transition_topk_backward_bf16 if bf16 else _LIB.jn_transition_topk_backward)
            _check(
                bwd(
                    _ptr(rho), _ptr(src), _ptr(dst), _ptr(ps), _ptr(pv), _ptr(Ws), _ptr(Wt), _ptr(w),
                    _ptr(sp), _ptr(dp), _ptr(idx), _ptr(logit), *([_ptr(head)] if mh else []), _ptr(g_ds), _ptr(g_dv),
                    float(temperature), B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg, topk, compress,
                    _ptr(out[0]), _ptr(out[1]), _ptr(out[2]), _ptr(out[3]), _ptr(out[4]), _ptr(gWs), _ptr(gWt),
                    _ptr(gw), _ptr(gb), _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (*out, gWs, gWt, gw if need[7] else None, gb if (has_bias and need[8]) else None, None, None, None,
                None, None)


def transition_pairwise_topk_routes(
    route_kind: str,
    source_weight: Tensor | None,
    source_bias: Tensor | None,
    target_weight: Tensor | None,
    target_bias: Tensor | None,
    core_weight: Tensor,
    bias: Tensor | None,
    hidden_weight: Tensor | None,
    hidden_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    temperature: float,
    sender_strength: Tensor,
    src_val: Tensor,
    dst_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    src_block_size: int,
    dst_block_size: int,
    route_compress_name: str = "softmax",
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Sparse transition returning (delta_state, delta_val, route_index, route_logit).

    Same arguments as ``transition_pairwise_topk``; route_index/route_logit
    [..., Ns, k] are each source's selected destinations (best first) and
    their logits."""
    if route_kind not in ("low_rank_bilinear_route", "multihead_max_low_rank_bilinear_route"):
        raise TypeError(f"jakal_net_native supports route kinds 'low_rank_bilinear_route' and "
                        f"'multihead_max_low_rank_bilinear_route', got {route_kind!r}.")
    if source_weight is None or target_weight is None:
        raise RuntimeError("Low-rank bilinear route is missing projection weights.")
    heads = 1
    if route_kind.startswith("multihead_"):
        core_weight, bias, source_weight, target_weight, heads = _flatten_heads(core_weight, bias, source_weight,
                                                                                target_weight)
    if source_bias is not None or target_bias is not None or hidden_weight is not None or out_weight is not None:
        raise TypeError("low_rank_bilinear_route carries no projection biases or hidden layers.")
    if route_compress_name not in _ROUTE_COMPRESS_KINDS:
        raise TypeError(f"Unsupported route_compress_name for the HIP backend: {route_compress_name!r}.")
    if topk <= 0:
        raise RuntimeError("topk must be positive.")
    if src_block_size <= 0 or dst_block_size <= 0:
        raise RuntimeError("block sizes must be positive.")
    if not temperature > 0:
        raise RuntimeError("temperature must be positive.")
    _require_gpu(sender_strength, src_val, dst_val, projected_state, projected_val, source_weight, target_weight,
                 core_weight, bias)
    batch_shape = tuple(src_val.shape[:-2])
    Ns, Dsrc = src_val.shape[-2], src_val.shape[-1]
    Nd, Ddst = dst_val.shape[-2], dst_val.shape[-1]
    Dv = projected_val.shape[-1]
    k = min(int(topk), Nd)
    _check_rank(source_weight.shape[0])
    if k < Nd:
        _check_select(k)
    elif Nd > MAX_ROUTE_TOPK:
        raise NotImplementedError("HIP sparse transition over every destination supports up to 64 destinations "
                                  "(transition_pairwise_topk runs more as the dense transition).")
    # bf16 layers keep bf16 value rows (one head); anything else computes in fp32
    bf16 = heads == 1 and _bf16_rows(src_val, dst_val, projected_val)
    rows = _bf16 if bf16 else _f32
    ds, dv, idx, logit = _TransitionTopK.apply(
        _f32(sender_strength.reshape(-1, Ns)), rows(src_val.reshape(-1, Ns, Dsrc)),
        rows(dst_val.reshape(-1, Nd, Ddst)), _f32(projected_state.reshape(-1, Ns)),
        rows(projected_val.reshape(-1, Ns, Dv)), _f32(source_weight), _f32(target_weight), _f32(core_weight),
        _f32(bias), float(temperature), k, _ROUTE_COMPRESS_KINDS[route_compress_name], heads, bf16,
    )
    return (
        ds.reshape(*batch_shape, Nd).to(projected_state.dtype),
        dv.reshape(*batch_shape, Nd, Dv).to(projected_val.dtype),
        idx.reshape(*batch_shape, Ns, k),
        logit.reshape(*batch_shape, Ns, k),
    )


def transition_pairwise_topk(
    route_kind: str,
    source_weight: Tensor | None,
    source_bias: Tensor | None,
    target_weight: Tensor | None,
    target_bias: Tensor | None,
    core_weight: Tensor,
    bias: Tensor | None,
    hidden_weight: Tensor | None,
    hidden_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    temperature: float,
    sender_strength: Tensor,
    src_val: Tensor,
    dst_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    topk: int,
    src_block_size: int,
    dst_block_size: int,
    route_compress_name: str = "softmax",
) -> tuple[Tensor, Tensor]:
    """Sparse pairwise transition; signature of jakal_net_native.cpp:6916-6936.

    ``core_weight`` is the raw route weight w; ``source_weight`` and
    ``target_weight`` the route projections (kernel_common.py:285-294).  The
    optional trailing ``route_compress_name`` ("softmax", "signed_abs_softmax"
    or "signed_entmax15") has no counterpart in the reference's composite op,
    which is softmax-only."""
    if topk >= dst_val.shape[-2] > 64:
        # every destination kept (transition.py:437-440): the dense transition
        return transition_pairwise_dense(
            route_kind, source_weight, source_bias, target_weight, target_bias, core_weight, bias, hidden_weight,
            hidden_bias, out_weight, out_bias, route_compress_name, temperature, sender_strength, src_val, dst_val,
            projected_state, projected_val, src_block_size, dst_block_size,
        )
    ds, dv, _, _ = transition_pairwise_topk_routes(
        route_kind, source_weight, source_bias, target_weight, target_bias, core_weight, bias, hidden_weight,
        hidden_bias, out_weight, out_bias, temperature, sender_strength, src_val, dst_val, projected_state,
        projected_val, topk, src_block_size, dst_block_size, route_compress_name,
    )
    return ds, dv


class _TransitionDense(torch.autograd.Function):
    """Differentiable dense pairwise Transition on the HIP library.

    Inputs (fp32, contiguous): sender strength rho [B,Ns], src_val [B,Ns,Dsrc],
    dst_val [B,Nd,Ddst], projected_state [B,Ns], projected_val [B,Ns,Dv],
    Ws [r,Dsrc], Wt [r,Ddst], w [r] (raw), bias [] or None.  With bf16,
    src_val, dst_val and projected_val are bf16 and delta_val comes back in
    bf16 (the *_bf16 entry points)."""

    @staticmethod
    def forward(ctx, rho, src, dst, ps, pv, Ws, Wt, w, bias, temperature: float, compress: int,  # noqa: N803
                heads: int = 1, bf16: bool = False):
        B, Ns, Dsrc = src.shape
        Nd, Ddst = dst.shape[1], dst.shape[2]
        Dv = pv.shape[-1]
        r = Ws.shape[0]
        dev = src.device
        mh = heads > 1
        with torch.cuda.device(dev):
            ds = torch.empty(B, Nd, device=dev, dtype=torch.float32)
            dv = torch.empty(B, Nd, Dv, device=dev, dtype=torch.bfloat16 if bf16 else torch.float32)
            sp = torch.empty(B * Ns, r, device=dev, dtype=torch.float32)
            dp = torch.empty(B * Nd, r, device=dev, dtype=torch.float32)
            routes = torch.empty(B, Ns, Nd, device=dev, dtype=torch.float32)
            route_heads = torch.empty(B, Ns, Nd, device=dev, dtype=torch.uint8) if mh else None
            fwd = (_LIB.jn_transition_dense_forward_multihead if mh else
                   _LIB.jn_transition_dense_forward_bf16 if bf16 else _LIB.jn_transition_dense_forward)
            _check(
                fwd(
                    _ptr(rho), _ptr(src), _ptr(dst), _ptr(ps), _ptr(pv), _ptr(Ws), _ptr(Wt), _ptr(w), _ptr(bias),
                    float(temperature), B, Ns, Nd, Dsrc, Ddst, Dv, *([r // heads, heads] if mh else [r]), compress,
                    _ptr(ds), _ptr(dv), _ptr(sp), _ptr(dp), _ptr(routes), *([_ptr(route_heads)] if mh else []),
                    _stream(dev),
                )
            )
        ctx.save_for_backward(rho, src, dst, ps, pv, Ws, Wt, w, sp, dp, routes, route_heads)
        ctx.meta = (float(temperature), compress, bias is not None, heads, bool(bf16))
        ctx.set_materialize_grads(False)  # an unused delta_state arrives as None
        return ds, dv

    @staticmethod
    def backward(ctx, g_ds, g_dv):
        rho, src, dst, ps, pv, Ws, Wt, w, sp, dp, routes, route_heads = ctx.saved_tensors
        temperature, compress, has_bias, heads, bf16 = ctx.meta
        mh = heads > 1
        B, Ns, Dsrc = src.shape
        Nd, Ddst = dst.shape[1], dst.shape[2]
        Dv = pv.shape[-1]
        r = Ws.shape[0]
        dev = src.device
        need = ctx.needs_input_grad
        # the projected source state reaches delta_state only
        need_in = list(need[:5])
        need_in[3] = need_in[3] and g_ds is not None
        with torch.cuda.device(dev):
            vdt = torch.bfloat16 if bf16 else torch.float32
            g_ds = torch.zeros(B, Nd, device=dev) if g_ds is None else g_ds.float().contiguous()
            g_dv = torch.zeros(B, Nd, Dv, device=dev, dtype=vdt) if g_dv is None else g_dv.to(vdt).contiguous()
            out = [torch.empty_like(t) if n else None for t, n in zip((rho, src, dst, ps, pv), need_in)]
            gWs = torch.empty_like(Ws) if need[5] else None
            gWt = torch.empty_like(Wt) if need[6] else None
            gw = torch.empty_like(w)
            gb = torch.empty((heads,) if mh else (), device=dev, dtype=torch.float32) if has_bias else None
            rank_arg = [r // heads, heads] if mh else [r]
            ws_fn = (_LIB.jn_transition_dense_multihead_workspace_bytes if mh else
                     _LIB.jn_transition_dense_workspace_bytes)
            ws_bytes = int(ws_fn(B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg))
            ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
            bwd = (_LIB.jn_transition_dense_backward_multihead if mh else
                   _LIB.jn_transition_dense_backward_bf16 if bf16 else _LIB.jn_transition_dense_backward)
            _check(
                bwd(
                    _ptr(rho), _ptr(src), _ptr(dst), _ptr(ps), _ptr(pv), _ptr(Ws), _ptr(Wt), _ptr(w),
                    _ptr(sp), _ptr(dp), _ptr(routes), *([_ptr(route_heads)] if mh else []), _ptr(g_ds), _ptr(g_dv),
                    float(temperature), B, Ns, Nd, Dsrc, Ddst, Dv, *rank_arg, compress,
                    _ptr(out[0]), _ptr(out[1]), _ptr(out[2]), _ptr(out[3]), _ptr(out[4]), _ptr(gWs), _ptr(gWt),
                    _ptr(gw), _ptr(gb), _ptr(ws), ws_bytes, _stream(dev),
                )
            )
        return (*out, gWs, gWt, gw if need[7] else None, gb if (has_bias and need[8]) else None, None, None, None,
                None)


def _check_route_spec(route_kind, source_weight, source_bias, target_weight, target_bias, hidden_weight, out_weight,
                      route_compress_name, temperature):
    if route_kind not in ("low_rank_bilinear_route", "multihead_max_low_rank_bilinear_route"):
        raise TypeError(f"jakal_net_native supports route kinds 'low_rank_bilinear_route' and "
                        f"'multihead_max_low_rank_bilinear_route', got {route_kind!r}.")
    if source_weight is None or target_weight is None:
        raise RuntimeError("Low-rank bilinear route is missing projection weights.")
    if source_bias is not None or target_bias is not None or hidden_weight is not None or out_weight is not None:
        raise TypeError("low_rank_bilinear_route carries no projection biases or hidden layers.")
    if route_compress_name not in _ROUTE_COMPRESS_KINDS:
        raise TypeError(f"Unsupported route_compress_name for the HIP backend: {route_compress_name!r}.")
    if not temperature > 0:
        raise RuntimeError("temperature must be positive.")


def dense_transition_bf16_shapes_ok(src_nodes: int, dst_nodes: int, val_dim: int) -> bool:
    """Whether a bf16 dense transition of these sizes runs on the bf16 entry
    points (their Ns x Nd products need 128 x 128 tiles of 8-element rows)."""
    return all(n >= 128 and n % 8 == 0 for n in (src_nodes, dst_nodes, val_dim))


def transition_pairwise_dense(
    route_kind: str,
    source_weight: Tensor | None,
    source_bias: Tensor | None,
    target_weight: Tensor | None,
    target_bias: Tensor | None,
    core_weight: Tensor,
    bias: Tensor | None,
    hidden_weight: Tensor | None,
    hidden_bias: Tensor | None,
    out_weight: Tensor | None,
    out_bias: Tensor | None,
    route_compress_name: str,
    temperature: float,
    sender_strength: Tensor,
    src_val: Tensor,
    dst_val: Tensor,
    projected_state: Tensor,
    projected_val: Tensor,
    src_block_size: int,
    dst_block_size: int,
) -> tuple[Tensor, Tensor]:
    """Dense pairwise transition; signature of jakal_net_native.cpp:6705-6725.

    Every source routes to every destination with routes
    compress(((P_s * w) . P_t + b) / T) over destinations ("softmax",
    "signed_abs_softmax" or "signed_entmax15").  The block sizes are validated and otherwise
    ignored: the HIP kernels tile for gfx950 themselves."""
    _check_route_spec(route_kind, source_weight, source_bias, target_weight, target_bias, hidden_weight, out_weight,
                      route_compress_name, temperature)
    heads = 1
    if route_kind.startswith("multihead_"):
        core_weight, bias, source_weight, target_weight, heads = _flatten_heads(core_weight, bias, source_weight,
                                                                                target_weight)
    _check_rank(source_weight.shape[0])
    if src_block_size < 0 or dst_block_size < 0:
        raise RuntimeError("block sizes must be non-negative.")
    _require_gpu(sender_strength, src_val, dst_val, projected_state, projected_val, source_weight, target_weight,
                 core_weight, bias)
    batch_shape = tuple(src_val.shape[:-2])
    Ns, Dsrc = src_val.shape[-2], src_val.shape[-1]
    Nd, Ddst = dst_val.shape[-2], dst_val.shape[-1]
    Dv = projected_val.shape[-1]
    # bf16 layers keep bf16 value rows on the bf16 MFMA products when the
    # shapes fit their tiles (one head); anything else computes in fp32
    bf16 = (heads == 1 and _bf16_rows(src_val, dst_val, projected_val)
            and dense_transition_bf16_shapes_ok(Ns, Nd, Dv))
    rows = _bf16 if bf16 else _f32
    ds, dv = _TransitionDense.apply(
        _f32(sender_strength.reshape(-1, Ns)), rows(src_val.reshape(-1, Ns, Dsrc)),
        rows(dst_val.reshape(-1, Nd, Ddst)), _f32(projected_state.reshape(-1, Ns)),
        rows(projected_val.reshape(-1, Ns, Dv)), _f32(source_weight), _f32(target_weight), _f32(core_weight),
        _f32(bias), float(temperature), _ROUTE_COMPRESS_KINDS[route_compress_name], heads, bf16,
    )
    return ds.reshape(*batch_shape, Nd).to(projected_state.dtype), dv.reshape(*batch_shape, Nd, Dv).to(
        projected_val.dtype)


# ---------------------------------------------------------------------------
# raw score + select (no autograd; used by tests and the benchmark)
# ---------------------------------------------------------------------------
def low_rank_topk_select(
    query: Tensor,
    key: Tensor,
    scale: Tensor | None,
    bias: Tensor | None,
    scale_on_query: bool,
    temperature: float,
    topk: int,
) -> tuple[Tensor, Tensor]:
    """Per-row top-k of ((query*cq) . (key*ck) + bias) / temperature.

    query [B,Nq,r], key [B,Nk,r] fp32; returns (index int32 [B,Nq,k], score fp32 [B,Nq,k])."""
    dev = _require_gpu(query, key, scale, bias)
    q = _f32(query)
    kk = _f32(key)
    B, Nq, r = q.shape
    Nk = kk.shape[1]
    idx = torch.empty(B, Nq, topk, device=dev, dtype=torch.int32)
    score = torch.empty(B, Nq, topk, device=dev, dtype=torch.float32)
    sc = _f32(scale)
    bi = _f32(bias)
    with torch.cuda.device(dev):
        ws_bytes = int(_LIB.jn_lowrank_topk_select_workspace_bytes(B, Nk, r))
        ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
        _check(
            _LIB.jn_lowrank_topk_select(
                _ptr(q), r, Nq * r, _ptr(kk), r, Nk * r, _ptr(sc), 1 if scale_on_query else 0, _ptr(bi),
                float(temperature), B, Nq, Nk, r, topk, _ptr(idx), _ptr(score), _ptr(ws), ws_bytes, _stream(dev),
            )
        )
    return idx, score


# ---------------------------------------------------------------------------
# Raw edge ops: the reference extension's *_cuda ops, which its Python
# dispatcher composes into its own autograd functions
# (src/jakal_net/native_backend.py:4002-4134 _LowRankPropagationQueryTopK,
# 4408-4600 _LowRankTransitionPairwiseTopK; probed at 657-667 and 5962-5975).
# Same names, argument order, shapes and return layouts
# (native/jakal_net_native.cpp:140-189, 398-414, 449-477); index tensors are
# int64 as there.  Outputs are fp32 accumulators except where the reference
# returns the input dtype (query_topk_reduce_cuda, the forward deltas).
# ---------------------------------------------------------------------------
def _raw_f32(name: str, t: Tensor) -> Tensor:
    if not t.is_floating_point():
        raise RuntimeError(f"{name} must be a floating-point tensor.")
    return t.float().contiguous()


def _raw_index(name: str, t: Tensor, limit: int, distinct: bool = False) -> Tensor:
    """int32 copy of an index tensor [..., k] whose entries lie in [-1, limit)
    (-1: no edge) and, with `distinct`, name each node at most once per row
    (the edge grouping of the backward ops keys its records by (row, node), as
    top-k index rows are); anything else is refused here, before a kernel
    could read out of bounds with it (one device-to-host read)."""
    if t.dtype not in (torch.int64, torch.int32):
        raise RuntimeError(f"{name} must use torch.long dtype.")
    if limit >= 2**31:
        raise NotImplementedError(f"{name}: node counts beyond 2^31 are not supported here.")
    if t.numel():
        lo, hi = torch.aminmax(t)
        flags = [lo, hi]
        if distinct and t.shape[-1] > 1:
            srt = torch.sort(t, dim=-1).values
            flags.append(((srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)).any())
        vals = torch.stack([f.to(torch.int64) for f in flags]).tolist()
        if vals[0] < -1 or vals[1] >= limit:
            raise RuntimeError(f"{name} must lie in [0, {limit}) (-1 for no edge); got [{vals[0]}, {vals[1]}].")
        if len(vals) > 2 and vals[2]:
            raise RuntimeError(f"{name} names a node twice in one row; rows of distinct nodes (top-k index rows) "
                               "are supported.")
    return t.to(torch.int32).contiguous()


def _raw_dims(name: str, t: Tensor, dims: int) -> None:
    if t.dim() != dims:
        raise RuntimeError(f"{name} must have {dims} dimensions (got shape {tuple(t.shape)}).")


def softsign_backward_cuda(scores: Tensor, grad_edges: Tensor) -> Tensor:
    """grad_scores = grad_edges / (1 + |scores|)^2 (native/jakal_net_native_cuda.cu:3426-3453)."""
    dev = _require_gpu(scores, grad_edges)
    if scores.shape != grad_edges.shape:
        raise RuntimeError("scores and grad_edges must share shape.")
    s = _raw_f32("scores", scores)
    g = _raw_f32("grad_edges", grad_edges)
    out = torch.empty(s.shape, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _check(_LIB.jn_softsign_backward(_ptr(s), _ptr(g), s.numel(), _ptr(out), _stream(dev)))
    return out


def softmax_backward_cuda(routes: Tensor, grad_routes: Tensor) -> Tensor:
    """Softmax backward over the last axis of [batch, query_nodes, topk]:
    grad = p (g - sum p g) (native/jakal_net_native_cuda.cu:3455-3483)."""
    dev = _require_gpu(routes, grad_routes)
    if routes.shape != grad_routes.shape or routes.dim() != 3:
        raise RuntimeError("routes and grad_routes must be shaped [batch, query_nodes, topk].")
    p = _raw_f32("routes", routes)
    g = _raw_f32("grad_routes", grad_routes)
    out = torch.empty(p.shape, device=dev, dtype=torch.float32)
    rows, k = p.shape[0] * p.shape[1], p.shape[2]
    if rows and k:
        with torch.cuda.device(dev):
            _check(_LIB.jn_softmax_backward(_ptr(p), _ptr(g), rows, k, _ptr(out), _stream(dev)))
    return out


def _edge_aggregate(index: Tensor, score: Tensor, compress: int, ps: Tensor, pv: Tensor):
    B, Nq, k = score.shape
    Ns, D = ps.shape[1], pv.shape[2]
    dev = score.device
    ds = torch.empty(B, Nq, device=dev, dtype=torch.float32)
    dv = torch.empty(B, Nq, D, device=dev, dtype=torch.float32)
    if B * Nq * k == 0 or Ns == 0:
        return ds.zero_(), dv.zero_()
    with torch.cuda.device(dev):
        _check(_LIB.jn_edge_aggregate(_ptr(index), _ptr(score), B, Nq, Ns, k, D, compress, _ptr(ps), _ptr(pv),
                                      _ptr(ds), _ptr(dv), _stream(dev)))
    return ds, dv


def _check_reduce_shapes(edges, indices, projected_state, projected_val):
    _raw_dims("edges", edges, 3)
    if indices.shape != edges.shape:
        raise RuntimeError("indices must have the same shape as edges.")
    _raw_dims("projected_state", projected_state, 2)
    _raw_dims("projected_val", projected_val, 3)
    if projected_state.shape[0] != edges.shape[0] or projected_val.shape[0] != edges.shape[0]:
        raise RuntimeError("projected tensors must share the edge batch dimension.")
    if projected_state.shape[1] != projected_val.shape[1]:
        raise RuntimeError("projected_state and projected_val must share source_nodes.")


def query_topk_reduce_cuda(edges: Tensor, indices: Tensor, projected_state: Tensor,
                           projected_val: Tensor) -> tuple[Tensor, Tensor]:
    """delta_state[b,i] = sum_e edges[b,i,e] ps[b,j], delta_val likewise over pv,
    j = indices[b,i,e] (native/jakal_net_native_cuda.cu:2335-2418); outputs in
    the projected tensors' dtype."""
    dev = _require_gpu(edges, indices, projected_state, projected_val)
    _check_reduce_shapes(edges, indices, projected_state, projected_val)
    idx = _raw_index("indices", indices, projected_state.shape[1])
    ds, dv = _edge_aggregate(idx, _raw_f32("edges", edges), 3, _raw_f32("projected_state", projected_state),
                             _raw_f32("projected_val", projected_val))
    return ds.to(projected_state.dtype), dv.to(projected_val.dtype)


def query_topk_reduce_backward_cuda(edges: Tensor, indices: Tensor, projected_state: Tensor, projected_val: Tensor,
                                    grad_delta_state: Tensor,
                                    grad_delta_val: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """(grad_edges, grad_projected_state, grad_projected_val) of query_topk_reduce_cuda
    (native/jakal_net_native_cuda.cu:2112-2175, 3352-3424), fp32."""
    dev = _require_gpu(edges, indices, projected_state, projected_val, grad_delta_state, grad_delta_val)
    _check_reduce_shapes(edges, indices, projected_state, projected_val)
    dtypes = {t.dtype for t in (edges, projected_state, projected_val, grad_delta_state, grad_delta_val)}
    if len(dtypes) != 1:
        raise RuntimeError("query_topk_reduce_backward_cuda inputs must share dtype.")
    B, Nq, k = edges.shape
    Ns, D = projected_state.shape[1], projected_val.shape[2]
    if tuple(grad_delta_state.shape) != (B, Nq) or tuple(grad_delta_val.shape) != (B, Nq, D):
        raise RuntimeError("grad_delta_state / grad_delta_val must be shaped [batch, query_nodes(, out_dim)].")
    idx = _raw_index("indices", indices, Ns, distinct=True)
    e, ps, pv = (_raw_f32(n, t) for n, t in (("edges", edges), ("projected_state", projected_state),
                                              ("projected_val", projected_val)))
    gs, gv = _raw_f32("grad_delta_state", grad_delta_state), _raw_f32("grad_delta_val", grad_delta_val)
    g_edges = torch.empty(B, Nq, k, device=dev, dtype=torch.float32)
    g_ps = torch.empty(B, Ns, device=dev, dtype=torch.float32)
    g_pv = torch.empty(B, Ns, D, device=dev, dtype=torch.float32)
    if B * Nq * k == 0:
        return g_edges, g_ps.zero_(), g_pv.zero_()
    with torch.cuda.device(dev):
        ws_bytes = int(_LIB.jn_edge_reduce_backward_workspace_bytes(B, Nq, Ns, k))
        if ws_bytes == 0:
            raise NotImplementedError("query_topk_reduce_backward_cuda: edge list too large for the edge grouping.")
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        _check(_LIB.jn_edge_reduce_backward(_ptr(e), _ptr(idx), _ptr(ps), _ptr(pv), _ptr(gs), _ptr(gv), B, Nq, Ns, k,
                                            D, _ptr(g_edges), _ptr(g_ps), _ptr(g_pv), _ptr(ws), ws_bytes,
                                            _stream(dev)))
    return g_edges, g_ps, g_pv


def _raw_select(wps: Tensor, pt: Tensor, topk: int, score_bias: float, limit: int):
    """Top-k of (wps[b,i] . pt[b,j] + bias) per row i, max over heads for
    [batch, heads, nodes, rank] operands (cu:740-813, 881-930)."""
    multihead = wps.dim() == 4 and pt.dim() == 4
    if not multihead and (wps.dim() != 3 or pt.dim() != 3):
        raise RuntimeError("weighted_projected_source and projected_target must be shaped [batch, nodes, rank] or "
                           "[batch, heads, nodes, rank].")
    if wps.shape[0] != pt.shape[0] or wps.shape[-1] != pt.shape[-1] or (multihead and wps.shape[1] != pt.shape[1]):
        raise RuntimeError("weighted_projected_source and projected_target must share batch, heads and rank_dim.")
    H = wps.shape[1] if multihead else 1
    if multihead:  # heads innermost: [B, N, H * r]
        q = wps.float().permute(0, 2, 1, 3).reshape(wps.shape[0], wps.shape[2], -1).contiguous()
        kk = pt.float().permute(0, 2, 1, 3).reshape(pt.shape[0], pt.shape[2], -1).contiguous()
    else:
        q, kk = wps.float().contiguous(), pt.float().contiguous()
    B, Nq, R = q.shape
    Nk = kk.shape[1]
    rh = R // H
    if R > (MAX_RANK if H == 1 else MAX_RANK_HEADS) or H > MAX_HEADS:
        raise NotImplementedError(f"the HIP select takes {MAX_RANK} ranks of one head, or up to {MAX_HEADS} heads "
                                  f"of {MAX_RANK_HEADS} ranks in all.")
    if topk <= 0 or topk > limit:
        raise RuntimeError(f"topk must be in the supported fused range [1, {limit}].")
    k = min(int(topk), Nk)
    dev = q.device
    bias = torch.full((H,), float(score_bias), device=dev, dtype=torch.float32)
    idx = torch.empty(B, Nq, k, device=dev, dtype=torch.int32)
    score = torch.empty(B, Nq, k, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        ws_bytes = int(_LIB.jn_lowrank_topk_select_heads_workspace_bytes(B, Nk, rh, H))
        ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
        _check(_LIB.jn_lowrank_topk_select_heads(_ptr(q), _ptr(kk), _ptr(bias), B, Nq, Nk, rh, H, k, _ptr(idx),
                                                 _ptr(score), _ptr(ws), ws_bytes, _stream(dev)))
    return idx, score


def low_rank_propagation_topk_forward_cuda(weighted_projected_source: Tensor, projected_target: Tensor,
                                           projected_state: Tensor, projected_val: Tensor, topk: int,
                                           score_bias: float, compress_kind: int) -> tuple[Tensor, Tensor]:
    """Each target row keeps its top-k sources by pt . wps, compresses
    (score + bias) (0 softsign, 1 signed |s| softmax, 2 signed entmax-1.5) and
    sums the chosen sources' projected state and values
    (native/jakal_net_native_cuda.cu:1029-1175, 2545-2630); fp32 outputs."""
    dev = _require_gpu(weighted_projected_source, projected_target, projected_state, projected_val)
    if compress_kind not in (0, 1, 2):
        raise RuntimeError("compress_kind must be 0 (softsign), 1 (signed_abs_softmax), or 2 (signed_entmax15).")
    _raw_dims("projected_state", projected_state, 2)
    _raw_dims("projected_val", projected_val, 3)
    if projected_state.dtype != torch.float32 or projected_val.dtype != torch.float32:
        raise RuntimeError("projected_state and projected_val must be float32 accumulators.")
    Ns = weighted_projected_source.shape[-2]
    if projected_state.shape[1] != Ns or projected_val.shape[1] != Ns:
        raise RuntimeError("projected_state/projected_val must share source_nodes.")
    # rows are the targets, keys the sources
    idx, score = _raw_select(projected_target, weighted_projected_source, topk, score_bias, MAX_TOPK_LARGE)
    return _edge_aggregate(idx, score, int(compress_kind), projected_state.contiguous(), projected_val.contiguous())


def low_rank_pairwise_topk_forward_cuda(weighted_projected_source: Tensor, projected_target: Tensor,
                                        weighted_projected_state: Tensor, weighted_projected_val: Tensor, topk: int,
                                        score_bias: float,
                                        compress_kind: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Each source row keeps its top-k destinations by wps . pt + bias, routes
    them (0 softmax, 1 signed |s| softmax, 2 signed entmax-1.5) and sums the
    weighted state and values per destination.  Returns (delta_state
    [B, Nd], delta_val [B, Nd, D], scores [B, Ns, k], indices int64
    [B, Ns, k]) (native/jakal_net_native_cuda.cu:740-878, 2420-2543)."""
    dev = _require_gpu(weighted_projected_source, projected_target, weighted_projected_state,
                       weighted_projected_val)
    if compress_kind not in (0, 1, 2):
        raise RuntimeError("compress_kind must be 0 (softmax), 1 (signed_abs_softmax), or 2 (signed_entmax15).")
    if weighted_projected_state.dim() != 2 or weighted_projected_val.dim() != 3:
        raise RuntimeError("weighted projected tensors must be shaped [batch, src_nodes] and "
                           "[batch, src_nodes, out_dim].")
    if weighted_projected_state.dtype != torch.float32 or weighted_projected_val.dtype != torch.float32:
        raise RuntimeError("weighted projected state/val must be float32 accumulators.")
    Ns = weighted_projected_source.shape[-2]
    if weighted_projected_state.shape[1] != Ns or weighted_projected_val.shape[1] != Ns:
        raise RuntimeError("weighted projected tensors must share src_nodes.")
    idx, score = _raw_select(weighted_projected_source, projected_target, topk, score_bias, MAX_ROUTE_TOPK)
    B, _, k = score.shape
    Nd = projected_target.shape[-2]
    D = weighted_projected_val.shape[2]
    ws_state = weighted_projected_state.contiguous()
    ws_val = weighted_projected_val.contiguous()
    ds = torch.empty(B, Nd, device=dev, dtype=torch.float32)
    dv = torch.empty(B, Nd, D, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        ws_bytes = int(_LIB.jn_route_topk_aggregate_workspace_bytes(B, Ns, Nd, k))
        if ws_bytes == 0:
            raise NotImplementedError("low_rank_pairwise_topk_forward_cuda: route list too large for the grouping.")
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        _check(_LIB.jn_route_topk_aggregate(_ptr(idx), _ptr(score), B, Ns, Nd, k, D, int(compress_kind),
                                            _ptr(ws_state), _ptr(ws_val), _ptr(ds), _ptr(dv), _ptr(ws), ws_bytes,
                                            _stream(dev)))
    return ds, dv, score, idx.to(torch.int64)


def low_rank_pairwise_topk_backward_cuda(query_val: Tensor, source_val: Tensor, source_weight: Tensor,
                                         target_weight: Tensor, core_weight: Tensor, projected_query: Tensor,
                                         projected_source: Tensor, indices: Tensor, grad_scores: Tensor,
                                         temperature: float) -> tuple[Tensor, ...]:
    """Gradients of the pair scores (Pq[i] * core) . Ps[j] / T + bias on the
    edges (i, indices[b,i,e]): (grad_query, grad_source, grad_source_weight,
    grad_target_weight, grad_core_weight, grad_bias), fp32, with grad_bias =
    sum grad_scores / T as the reference computes it
    (native/jakal_net_native_cuda.cu:2259-2322, 3792-3866).  query_val is
    projected by target_weight, source_val by source_weight."""
    dev = _require_gpu(query_val, source_val, source_weight, target_weight, core_weight, projected_query,
                       projected_source, indices, grad_scores)
    if temperature <= 0.0:
        raise RuntimeError("temperature must be positive.")
    for n, t, d in (("query_val", query_val, 3), ("source_val", source_val, 3), ("source_weight", source_weight, 2),
                    ("target_weight", target_weight, 2), ("core_weight", core_weight, 1),
                    ("projected_query", projected_query, 3), ("projected_source", projected_source, 3),
                    ("indices", indices, 3), ("grad_scores", grad_scores, 3)):
        _raw_dims(n, t, d)
    B, Nq, Dq = query_val.shape
    Ns, Ds = source_val.shape[1], source_val.shape[2]
    r = core_weight.shape[0]
    k = indices.shape[2]
    if (tuple(target_weight.shape) != (r, Dq) or tuple(source_weight.shape) != (r, Ds)
            or tuple(projected_query.shape) != (B, Nq, r) or tuple(projected_source.shape) != (B, Ns, r)
            or tuple(indices.shape[:2]) != (B, Nq) or grad_scores.shape != indices.shape
            or source_val.shape[0] != B):
        raise RuntimeError("low_rank_pairwise_topk_backward_cuda: inconsistent shapes.")
    _check_rank(r, MAX_RANK_HEADS)  # the raw backward's rank slots
    f32 = dict(device=dev, dtype=torch.float32)
    if B * Nq * k == 0 or Ns == 0:
        return (torch.zeros(B, Nq, Dq, **f32), torch.zeros(B, Ns, Ds, **f32), torch.zeros(r, Ds, **f32),
                torch.zeros(r, Dq, **f32), torch.zeros(r, **f32), torch.zeros((), **f32))
    idx = _raw_index("indices", indices, Ns, distinct=True)
    xq, xs, ws_, wt, w, pq, ps, g = (_raw_f32(n, t) for n, t in (
        ("query_val", query_val), ("source_val", source_val), ("source_weight", source_weight),
        ("target_weight", target_weight), ("core_weight", core_weight), ("projected_query", projected_query),
        ("projected_source", projected_source), ("grad_scores", grad_scores)))
    g_q, g_s = torch.empty(B, Nq, Dq, **f32), torch.empty(B, Ns, Ds, **f32)
    g_ws, g_wt = torch.empty(r, Ds, **f32), torch.empty(r, Dq, **f32)
    g_w, g_b = torch.empty(r, **f32), torch.empty((), **f32)
    with torch.cuda.device(dev):
        ws_bytes = int(_LIB.jn_lowrank_pair_backward_workspace_bytes(B, Nq, Ns, Dq, Ds, r, k))
        if ws_bytes == 0:
            raise NotImplementedError("low_rank_pairwise_topk_backward_cuda: edge list too large for the grouping.")
        ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
        _check(_LIB.jn_lowrank_pair_backward(_ptr(xq), _ptr(xs), _ptr(ws_), _ptr(wt), _ptr(w), _ptr(pq), _ptr(ps),
                                             _ptr(idx), _ptr(g), float(temperature), B, Nq, Ns, Dq, Ds, r, k,
                                             _ptr(g_q), _ptr(g_s), _ptr(g_ws), _ptr(g_wt), _ptr(g_w), _ptr(g_b),
                                             _ptr(ws), ws_bytes, _stream(dev)))
    return g_q, g_s, g_ws, g_wt, g_w, g_b
