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


def _run(dev, seed, B, N, D, r, window, compress, separate_pv, init="xavier", normwise=False):
    """normwise: the absolute tolerance of the outputs and node gradients
    scales with the tensor's largest entry (long sums at larger D and widths)."""
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

    ref = O.propagation_forward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), mode="window",
                                window=window, kind=compress)

    def node_atol(want):
        return ATOL * max(1.0, float(np.abs(want).max())) if normwise else ATOL

    _close(_np(ds), ref["delta_state"], atol=node_atol(ref["delta_state"]), what="delta_state")
    _close(_np(dv), ref["delta_val"], atol=node_atol(ref["delta_val"]), what="delta_val")
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="window", window=window, kind=compress)
    g_val = gr["val"] + (0.0 if separate_pv else gr["pv"])
    _close(_np(X.grad), g_val, atol=node_atol(g_val), what="grad layer_val")
    _close(_np(ps.grad), gr["ps"], atol=node_atol(gr["ps"]), what="grad projected_state")
    if separate_pv:
        _close(_np(pv.grad), gr["pv"], atol=node_atol(gr["pv"]), what="grad projected_val")
    gs = gr["g_scores"][ref["mask"]]
    scale = max(1.0, float(np.abs(gs).sum() / math.sqrt(gs.size)))
    for got, want, what in ((Ud.grad, gr["U"], "grad target_proj"), (Vd.grad, gr["V"], "grad source_proj"),
                            (wd.grad, gr["w_hat"], "grad w_hat"), (bd.grad, gr["b"], "grad bias")):
        _close(_np(got), want, atol=ATOL * max(scale, float(np.abs(want).max())), what=what)


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
    _run(dev, 2100 + window, B=1, N=1100, D=520, r=16, window=window, compress=compress, separate_pv=True,
         normwise=True)


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
    ref = O.propagation_forward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), mode="window",
                                window=window, kind=compress)
    _close(_np(ds), ref["delta_state"], atol=ATOL * max(1.0, float(np.abs(ref["delta_state"]).max())),
           what="delta_state")
    _close(_np(dv), ref["delta_val"], atol=ATOL * max(1.0, float(np.abs(ref["delta_val"]).max())), what="delta_val")
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="window", window=window, kind=compress)
    g_val = gr["val"] + (0.0 if separate_pv else gr["pv"])
    for got, want, what in ((X.grad, g_val, "grad layer_val"), (ps.grad, gr["ps"], "grad projected_state")) + (
            ((pv.grad, gr["pv"], "grad projected_val"),) if separate_pv else ()):
        _close(_np(got), want, atol=ATOL * max(1.0, float(np.abs(want).max())), what=what)
    gs = gr["g_scores"][ref["mask"]]
    scale = max(1.0, float(np.abs(gs).sum() / math.sqrt(gs.size)))
    for got, want, what in ((Ud.grad, gr["U"], "grad target_proj"), (Vd.grad, gr["V"], "grad source_proj"),
                            (wd.grad, gr["w_hat"], "grad w_hat"), (bd.grad, gr["b"], "grad bias")):
        _close(_np(got), want, atol=ATOL * max(scale, float(np.abs(want).max())), what=what)
