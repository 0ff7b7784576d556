"""The raw edge ops on the CPU (no device calls): the module offers every op the
reference dispatcher probes before it takes its decomposed CUDA autograd path
for a low-rank top-k transition, under the reference's names and argument
lists, and the C ABI rejects what it cannot take before touching a GPU.

The dispatch condition is restated from src/jakal_net/native_backend.py:
5962-5975 (use_cuda_autograd), 657-667 (_query_backward_ops_available) and
650-655 (_cuda_float_tensor); the argument names from the reference's
bindings, native/jakal_net_native.cpp:140-189, 398-414 and 449-477.
"""

import ctypes
import inspect
from types import SimpleNamespace

import pytest
import torch

from jakal_net import LowRankBilinearRoute, MultiHeadRoute
from jakal_net import native_backend as NB

REFERENCE_ARGS = {
    "softsign_backward_cuda": ("scores", "grad_edges"),
    "softmax_backward_cuda": ("routes", "grad_routes"),
    "query_topk_reduce_cuda": ("edges", "indices", "projected_state", "projected_val"),
    "query_topk_reduce_backward_cuda": ("edges", "indices", "projected_state", "projected_val", "grad_delta_state",
                                        "grad_delta_val"),
    "low_rank_propagation_topk_forward_cuda": ("weighted_projected_source", "projected_target", "projected_state",
                                               "projected_val", "topk", "score_bias", "compress_kind"),
    "low_rank_pairwise_topk_forward_cuda": ("weighted_projected_source", "projected_target",
                                            "weighted_projected_state", "weighted_projected_val", "topk",
                                            "score_bias", "compress_kind"),
    "low_rank_pairwise_topk_backward_cuda": ("query_val", "source_val", "source_weight", "target_weight",
                                             "core_weight", "projected_query", "projected_source", "indices",
                                             "grad_scores", "temperature"),
}


@pytest.fixture
def real_module(monkeypatch):
    import jakal_net_native as JN  # loads the library; no device call

    monkeypatch.setattr(NB._LOADER, "module", JN)
    monkeypatch.setattr(NB._LOADER, "status", NB._LOADER._describe(JN, "jakal_net_native"))
    monkeypatch.delenv(NB.DISABLE_NATIVE_ENV, raising=False)
    return JN


def _cuda_float_tensor(t) -> bool:
    return t is not None and t.device.type == "cuda" and t.dtype in {torch.float16, torch.bfloat16, torch.float32}


def _use_cuda_autograd(inner, compress_kind, topk, tensors, entmax_ops_available=False) -> bool:
    """The reference's condition for _LowRankTransitionPairwiseTopK, restated."""
    query_backward_ops = all(NB.native_supports(n) for n in ("query_topk_reduce_backward_cuda",
                                                            "softsign_backward_cuda", "softmax_backward_cuda"))
    return (query_backward_ops
            and NB.native_supports("low_rank_pairwise_topk_forward_cuda")
            and NB.native_supports("low_rank_pairwise_topk_backward_cuda")
            and isinstance(inner, LowRankBilinearRoute)
            and compress_kind is not None
            and (compress_kind != 2 or entmax_ops_available)
            and topk <= 64
            and all(_cuda_float_tensor(t) for t in tensors))


def _spy_tensor(dtype=torch.float32):
    """Stands in for a HIP tensor (ROCm torch reports device.type == "cuda")."""
    return SimpleNamespace(device=SimpleNamespace(type="cuda"), dtype=dtype)


@pytest.mark.parametrize("compress_kind", [0, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_takes_its_cuda_autograd_path_with_this_module(real_module, compress_kind, dtype):
    inner = LowRankBilinearRoute(8, 8, rank=4)
    tensors = [_spy_tensor(dtype) for _ in range(5)]
    assert _use_cuda_autograd(inner, compress_kind, 16, tensors)
    assert _use_cuda_autograd(inner, compress_kind, 64, tensors)


def test_reference_condition_still_declines_what_it_declines(real_module):
    inner = LowRankBilinearRoute(8, 8, rank=4)
    tensors = [_spy_tensor() for _ in range(5)]
    assert not _use_cuda_autograd(inner, 0, 65, tensors)             # beyond the fused k range
    assert not _use_cuda_autograd(inner, 2, 16, tensors)             # needs torch.ops.jakal_net.signed_entmax15
    heads = MultiHeadRoute([LowRankBilinearRoute(8, 8, rank=4) for _ in range(2)])
    assert not _use_cuda_autograd(heads, 0, 16, tensors)
    cpu = [SimpleNamespace(device=SimpleNamespace(type="cpu"), dtype=torch.float32)] + tensors[1:]
    assert not _use_cuda_autograd(inner, 0, 16, cpu)


def test_raw_ops_carry_the_reference_argument_lists(real_module):
    for name, args in REFERENCE_ARGS.items():
        assert name in real_module.supported_ops(), name
        params = tuple(inspect.signature(getattr(real_module, name)).parameters)
        assert params == args, f"{name}: {params}"


def test_raw_ops_refuse_host_tensors(real_module):
    s = torch.randn(2, 3, 4)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        real_module.softsign_backward_cuda(s, s)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        real_module.softmax_backward_cuda(s, s)


def test_raw_op_entry_points_validate_before_any_device_call():
    import jakal_net_native as JN

    lib = JN._LIB
    # rank beyond the library's 128: rejected with a message, nothing launched
    rc = lib.jn_lowrank_pair_backward(None, None, None, None, None, None, None, None, None, 1.0, 1, 8, 8, 4, 4, 200,
                                      2, None, None, None, None, None, None, None, 0, None)
    assert rc != 0 and b"rank" in lib.jn_last_error()
    rc = lib.jn_lowrank_pair_backward(None, None, None, None, None, None, None, None, None, 0.0, 1, 8, 8, 4, 4, 8,
                                      2, None, None, None, None, None, None, None, 0, None)
    assert rc != 0 and b"temperature" in lib.jn_last_error()
    # routes keep at most 4096 destinations per source
    rc = lib.jn_route_topk_aggregate(None, None, 1, 8, 10000, 5000, 4, 0, None, None, None, None, None, 0, None)
    assert rc != 0 and b"4096" in lib.jn_last_error()
    rc = lib.jn_edge_aggregate(None, None, 1, 8, 8, 2, 4, 5, None, None, None, None, None)
    assert rc != 0 and b"compress" in lib.jn_last_error()
    # empty inputs need no launch
    assert lib.jn_softmax_backward(None, None, 0, 4, None, None) == 0
    assert lib.jn_softsign_backward(None, None, 0, None, None) == 0
    # too many heads for the select
    rc = lib.jn_lowrank_topk_select_heads(None, None, None, 1, 4, 8, 8, 9, 2, None, None, None, 0, None)
    assert rc != 0


def test_raw_op_workspace_queries_without_gpu():
    import jakal_net_native as JN

    lib = JN._LIB
    assert lib.jn_edge_reduce_backward_workspace_bytes(2, 100, 50, 8) > 0
    assert lib.jn_route_topk_aggregate_workspace_bytes(2, 100, 50, 8) > lib.jn_edge_reduce_backward_workspace_bytes(
        2, 100, 50, 8)  # plus the route weights
    small = lib.jn_lowrank_pair_backward_workspace_bytes(2, 100, 50, 16, 16, 8, 8)
    assert small > 0
    assert lib.jn_lowrank_pair_backward_workspace_bytes(2, 100, 50, 16, 64, 8, 8) >= small
    # the edge grouping's table beyond its size limit: no workspace, the op refuses
    assert lib.jn_edge_reduce_backward_workspace_bytes(1, 2_000_000, 2_000_000, 8) == 0
    assert lib.jn_lowrank_topk_select_heads_workspace_bytes(2, 100, 16, 1) == lib.jn_lowrank_topk_select_workspace_bytes(
        2, 100, 16)
    assert lib.jn_lowrank_topk_select_heads_workspace_bytes(2, 100, 64, 3) == 0
    assert ctypes.sizeof(ctypes.c_size_t) == 8
