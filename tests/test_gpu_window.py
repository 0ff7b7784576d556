"""GPU parity of causal-window propagation (HIP library) against the numpy oracle.

The window edge list is fixed by the shape (no selection), so the edge
indices must match exactly and values/gradients agree within the fp32
tolerance of the hot path, rtol 1e-4 / atol 1e-5 (parameter gradients, which
sum over every edge, with atol scaled by the size of their terms).
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import check, torch32_propagation

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _np(t):
    return t.detach().double().cpu().numpy()


def _close(got, want, rtol=RTOL, atol=ATOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert err.max() <= 0, f"{what}: max excess {err.max():.3e} (max abs diff {np.abs(got - want).max():.3e})"


def _inputs(seed, B, N, D, r, init="xavier"):
    g = torch.Generator().manual_seed(seed)
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    bound = math.sqrt(6.0 / (D + r)) if init == "xavier" else 1.0 / math.sqrt(D)
    U = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    V = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    b = torch.tensor(0.1)
    return g, state, val, U, V, w, b


def _expected_window_index(N, window):
    width = min(window + 1, N)
    i = np.arange(N)[:, None]
    e = np.arange(width)[None, :]
    j = i - (width - 1 - e)
    return np.where(j >= 0, j, -1)


def _run(dev, seed, B, N, D, r, window, compress, separate_pv, init="xavier"):
    import jakal_net_native as jn

    g, state, val, U, V, w, b = _inputs(seed, B, N, D, r, init)
    pv_cpu = torch.randn(B, N, D, generator=g) if separate_pv else val
    w_hat = w / w.norm()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True) if separate_pv else X
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd, bd = w_hat.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    ds, dv, idx, score = jn.propagation_window_edges("low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X,
                                                     ps, pv, window, N, N)
    gds = torch.randn(B, N, generator=g)
    gdv = torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    want_idx = _expected_window_index(N, window)
    got_idx = idx.cpu().numpy()
    assert (got_idx == want_idx[None]).all(), "window edge indices differ"
    scores = O.lowrank_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), float(b))
    valid = want_idx >= 0
    picked = np.take_along_axis(scores, np.broadcast_to(np.maximum(want_idx, 0), scores.shape[:-1] + want_idx.shape[-1:]),
                                axis=-1)
    got_score = score.cpu().numpy()
    _close(got_score[:, valid], picked[:, valid], rtol=1e-5, atol=1e-5, what="edge scores")

    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="window", window=window, kind=compress)
    mask = np.broadcast_to(O.causal_window_mask(N, window), (B, N, N))
    t32 = torch32_propagation(dev, val, state, pv_cpu if separate_pv else None, U, V, w_hat, float(b), mask,
                              compress, gds, gdv)
    _compare(gr, t32, ds, dv, X, ps, pv if separate_pv else None, Ud, Vd, wd, bd)


def _compare(gr, t32, ds, dv, X, ps, pv, Ud, Vd, wd, bd):
    """Every output and gradient against the oracle (parity.check, calibrated by the fp32 torch run)."""
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    check("grad layer_val", X.grad, gr["val"] + (0.0 if pv is not None else gr["pv"]), t32["val"])
    check("grad projected_state", ps.grad, gr["ps"], t32["ps"])
    if pv is not None:
        check("grad projected_val", pv.grad, gr["pv"], t32["pv"])
    for t, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("separate_pv", [False, True])
def test_window_forward_backward_matches_oracle(dev, compress, separate_pv):
    _run(dev, 2001, B=2, N=64, D=32, r=8, window=8, compress=compress, separate_pv=separate_pv)


@pytest.mark.parametrize("window,N", [(0, 40), (63, 50), (100, 70), (130, 300)])
def test_window_edge_cases(dev, window, N):
    # window 0 (self only), window >= N (full causal), width above one wavefront pass
    compress = "signed_abs_softmax" if min(window + 1, N) <= 64 else "softsign"
    _run(dev, 2002 + window, B=2, N=N, D=20, r=5, window=window, compress=compress, separate_pv=True)


@pytest.mark.parametrize("window,compress", [(100, "softsign"), (40, "signed_abs_softmax")])
def test_window_split_row_backward(dev, window, compress):
    """Value rows of a batch element above 2 MiB with 256 < D <= 1024 (two column
    slabs for the row backward's dot products); width 101 takes two edge blocks."""
    _run(dev, 2100 + window, B=1, N=1100, D=520, r=16, window=window, compress=compress, separate_pv=True)


def test_window_c2_shape(dev):
    """B=8, T=1024, D=384, r=32, window=64, softsign, default init."""
    _run(dev, 1002, B=8, N=1024, D=384, r=32, window=64, compress="softsign", separate_pv=False, init="default")


def test_sparse_propagation_window_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

    torch.manual_seed(41)
    layer = Layer(dim=6, num_nodes=11, state=torch.randn(2, 11, device=dev), val=torch.randn(2, 11, 6, device=dev))
    kw = dict(sparse_type="window", window=3, state_proj_fn=lambda s: s * 1.5 + 0.25, val_proj_fn=lambda v: v - 0.5)
    ref = SparsePropagation(LowRankBilinearPairwise(6, 4).to(dev), implementation="reference", **kw)
    nat = SparsePropagation(LowRankBilinearPairwise(6, 4).to(dev), implementation="native", **kw)
    nat.pairwise_fn.load_state_dict(ref.pairwise_fn.state_dict())
    a, b = ref(layer), nat(layer)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-5)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("separate_pv,window_extra", [(False, 0), (True, 7)])
def test_full_causal_window_runs_dense(dev, compress, separate_pv, window_extra):
    """window >= N - 1 on N >= 128 nodes: every earlier source, computed as
    causal dense propagation (MFMA GEMMs); forward and every gradient against
    the oracle's window mode."""
    import jakal_net_native as jn

    B, N, D, r = 2, 200, 48, 12
    window = N - 1 + window_extra
    assert N >= jn.CAUSAL_DENSE_MIN_NODES
    g, state, val, U, V, w, b = _inputs(2101, B, N, D, r)
    pv_cpu = torch.randn(B, N, D, generator=g) if separate_pv else val
    w_hat = w / w.norm()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True) if separate_pv else X
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd, bd = w_hat.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    ds, dv = jn.propagation_window("low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X, ps, pv, window, N, N)
    gds = torch.randn(B, N, generator=g)
    gdv = torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="window", window=window, kind=compress)
    mask = np.broadcast_to(O.causal_window_mask(N, window), (B, N, N))
    t32 = torch32_propagation(dev, val, state, pv_cpu if separate_pv else None, U, V, w_hat, float(b), mask,
                              compress, gds, gdv)
    _compare(gr, t32, ds, dv, X, ps, pv if separate_pv else None, Ud, Vd, wd, bd)


@pytest.mark.parametrize("compress", ["softsign", "signed_entmax15"])
def test_window_edge_kernels_forced(dev, compress):
    """The per-edge gather kernels (jn_set_window_kernels(1)) against the oracle;
    by default windows up to 128 wide with whole 16-byte value rows run on the
    band's MFMA tiles, and the other tests here cover that path."""
    import jakal_net_native as jn

    jn.set_window_kernels(jn.WINDOW_EDGES)
    try:
        _run(dev, 2001, B=2, N=64, D=32, r=8, window=8, compress=compress, separate_pv=True)
        _run(dev, 2003, B=1, N=200, D=384, r=32, window=63, compress=compress, separate_pv=False)
    finally:
        jn.set_window_kernels(jn.WINDOW_BAND)


@pytest.mark.parametrize("window,N,compress,kernels", [
    (90, 200, "signed_abs_softmax", "band"),      # 91 slots: band tiles, rows of two 64-slot blocks
    (90, 200, "signed_entmax15", "band"),
    (90, 200, "signed_entmax15", "edges"),
    (150, 300, "signed_abs_softmax", "edges"),    # wider than the band: the edge kernels
    (150, 300, "signed_entmax15", "edges"),
    (99, 100, "signed_entmax15", "band"),         # full causal window below 128 nodes: an edge list
])
def test_window_signed_rows_beyond_one_block(dev, window, N, compress, kernels):
    """The row-normalising compressions on windows of more than 64 slots."""
    import jakal_net_native as jn

    jn.set_window_kernels(jn.WINDOW_EDGES if kernels == "edges" else jn.WINDOW_BAND)
    try:
        _run(dev, 2200 + window, B=2, N=N, D=32, r=8, window=window, compress=compress, separate_pv=True)
    finally:
        jn.set_window_kernels(jn.WINDOW_BAND)


def test_window_unaligned_rows_take_the_edge_kernels(dev):
    """D = 30 is not a whole number of 16-byte packs: the edge kernels run."""
    _run(dev, 2004, B=2, N=90, D=30, r=6, window=20, compress="signed_entmax15", separate_pv=True)
