"""The allocation-free top-k forward (jn_propagation_topk_forward_static)
against jn_propagation_topk_forward, through the C ABI.

Both run the same kernels; only where the select's scratch lives differs (a
static device array against a caller workspace), so every output must be
bit-identical.  Two calls in a row, the second on a smaller input, check that
the shared array carries nothing from one call into the next.  A shape whose
scratch exceeds the array is rejected before any launch.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

_P, _I64, _I32, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
_FWD_ARGS = [_P] * 7 + [_I64] * 6 + [_I32] + [_P] * 5


def _lib():
    import jakal_net_native as jn

    lib = ctypes.CDLL(str(jn.library_path()))
    lib.jn_propagation_topk_forward.argtypes = _FWD_ARGS + [_P, _SZ, _P, _SZ, _P]  # layout, workspace, stream
    lib.jn_propagation_topk_forward_static.argtypes = _FWD_ARGS + [_P]
    lib.jn_propagation_topk_forward_workspace_bytes.argtypes = [_I64] * 3
    lib.jn_propagation_topk_forward_workspace_bytes.restype = _SZ
    lib.jn_static_scratch_bytes.restype = _SZ
    lib.jn_last_error.restype = ctypes.c_char_p
    return lib


def _run(lib, static, X, ps, U, V, w_hat, bias, k, compress):
    B, N, D = X.shape
    r = U.shape[0]
    dev = X.device
    ds = torch.full((B, N), float("nan"), device=dev)
    dv = torch.full((B, N, D), float("nan"), device=dev)
    proj = torch.full((B * N, 2 * r), float("nan"), device=dev)
    idx = torch.full((B, N, k), -7, device=dev, dtype=torch.int32)
    score = torch.full((B, N, k), float("nan"), device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    args = [p(X), p(ps), p(X), p(U), p(V), p(w_hat), p(bias), B, N, D, D, r, k, compress,
            p(ds), p(dv), p(proj), p(idx), p(score)]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if static:
        rc = lib.jn_propagation_topk_forward_static(*args, stream)
    else:
        ws_bytes = int(lib.jn_propagation_topk_forward_workspace_bytes(B, N, r))
        ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
        rc = lib.jn_propagation_topk_forward(*args, None, 0, p(ws), ws_bytes, stream)  # no edge layout
    assert rc == 0, lib.jn_last_error().decode()
    torch.cuda.synchronize()
    return ds, dv, proj, idx, score


def _inputs(seed, B, N, D, r, dev):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, N, D, generator=g).to(dev)
    ps = torch.randn(B, N, generator=g).to(dev)
    U = (torch.randn(r, D, generator=g) / D ** 0.5).to(dev)
    V = (torch.randn(r, D, generator=g) / D ** 0.5).to(dev)
    w = torch.rand(r, generator=g) + 0.5
    return X, ps, U, V, (w / w.norm()).to(dev), torch.tensor([0.1], device=dev)


@pytest.mark.parametrize("compress", [0, 2])
@pytest.mark.parametrize("shapes", [
    ((16, 4096, 128, 64, 32), (3, 700, 72, 24, 9)),   # register select
    ((4, 1500, 64, 32, 100), (2, 600, 40, 16, 70)),   # k > 64: score blocks of the scored-rows select in the array
])
def test_static_scratch_forward_matches_workspace_forward(compress, shapes):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    lib = _lib()
    dev = torch.device("cuda:0")
    # the second call is smaller: nothing of the first may leak into it
    for seed, (B, N, D, r, k) in zip((31, 32), shapes):
        X, ps, U, V, w_hat, bias = _inputs(seed, B, N, D, r, dev)
        want = _run(lib, False, X, ps, U, V, w_hat, bias, k, compress)
        got = _run(lib, True, X, ps, U, V, w_hat, bias, k, compress)
        for a, b, name in zip(got, want, ("delta_state", "delta_val", "projections", "index", "score")):
            assert torch.equal(a, b), f"{name} differs (B={B}, N={N}, r={r}, k={k})"
        print(f"static forward bit-identical at B={B} N={N} D={D} r={r} k={k} compress={compress}", flush=True)


def test_static_scratch_rejects_oversize():
    lib = _lib()
    cap = int(lib.jn_static_scratch_bytes())
    B, N, r = 64, 65535, 64
    assert int(lib.jn_propagation_topk_forward_workspace_bytes(B, N, r)) > cap
    nul = [None] * 7 + [B, N, 64, 64, r, 8, 0] + [None] * 5 + [None]
    rc = lib.jn_propagation_topk_forward_static(*nul)
    assert rc != 0
    assert b"static scratch holds" in lib.jn_last_error()


@pytest.mark.parametrize("k", [32, 100])
def test_static_scratch_forward_captures_without_allocating(k):
    """Captured in a global-mode stream capture (where any device allocation
    fails the capture) the static forward records kernels only; three replays,
    with eager GPU work between them, equal the eager call bit for bit."""
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    lib = _lib()
    dev = torch.device("cuda:0")
    B, N, D, r = 2, 1200, 48, 32
    X, ps, U, V, w_hat, bias = _inputs(40 + k, B, N, D, r, dev)
    want = _run(lib, True, X, ps, U, V, w_hat, bias, k, 0)  # eager (also the per-device set-up)
    outs = [torch.empty_like(t) for t in want]
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    args = [p(X), p(ps), p(X), p(U), p(V), p(w_hat), p(bias), B, N, D, D, r, k, 0] + [p(t) for t in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side, capture_error_mode="global"):
            rc = lib.jn_propagation_topk_forward_static(*args, ctypes.c_void_p(side.cuda_stream))
    assert rc == 0, lib.jn_last_error().decode()
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(3):
        for t in outs:
            t.fill_(float("nan")) if t.is_floating_point() else t.fill_(-7)
        torch.randn(1 << 20, device=dev).sum()  # other GPU work between replays
        graph.replay()
        torch.cuda.synchronize()
        for a, b, name in zip(outs, want, ("delta_state", "delta_val", "projections", "index", "score")):
            assert torch.equal(a, b), f"replay {rep}: {name} differs (k={k})"
