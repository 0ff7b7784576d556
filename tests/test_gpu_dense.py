"""GPU parity of dense low-rank propagation (HIP library) against the numpy oracle.

Dense propagation keeps every (target, source) pair (propagation.py:207-220);
values and gradients are compared with the float64 oracle within rtol 1e-4 /
atol 1e-5 (fp32), or, for long sums (over N sources and D dims) that miss it,
within twice the error of an fp32 torch evaluation of the same op
(tests/parity.py).  The full C4-dense shape is in test_gpu_full_shape.py.
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


def _inputs(seed, B, N, D, r):
    g = torch.Generator().manual_seed(seed)
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    bound = math.sqrt(6.0 / (D + r))
    U = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    V = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    return g, state, val, U, V, w


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("separate_pv", [False, True])
@pytest.mark.parametrize("N,with_bias", [(64, True), (37, False)])
def test_dense_forward_backward_matches_oracle(dev, compress, separate_pv, N, with_bias):
    _check_dense(dev, compress, separate_pv, N, with_bias, B=2, D=24, r=6)


@pytest.mark.parametrize("separate_pv", [False, True])
def test_dense_softsign_more_blocks_than_value_columns(dev, separate_pv):
    # 300 sources = 10 blocks of 32 columns per row > D = 8 value columns: the
    # forward computes softsign in its own pass, the backward keeps the fused epilogue
    _check_dense(dev, "softsign", separate_pv, 300, True, B=2, D=8, r=5)


def _check_dense(dev, compress, separate_pv, N, with_bias, B, D, r):
    import jakal_net_native as jn

    g, state, val, U, V, w = _inputs(4001 + N, B, N, D, r)
    b = torch.tensor(0.15) if with_bias else None
    pv_cpu = torch.randn(B, N, D, generator=g) if separate_pv else val
    w_hat = w / w.norm()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True) if separate_pv else X
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd = w_hat.to(dev).requires_grad_(True)
    bd = b.to(dev).requires_grad_(True) if with_bias else None
    ds, dv = jn.propagation_dense("low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X, ps, pv, None, N, N)
    gds = torch.randn(B, N, generator=g)
    gdv = torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    bval = float(b) if with_bias else 0.0
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), bval, _np(gds),
                                _np(gdv), mode="dense", kind=compress)
    mask = np.ones((B, N, N), dtype=bool)
    t32 = torch32_propagation(dev, val, state, pv_cpu if separate_pv else None, U, V, w_hat,
                              float(b) if with_bias else None, mask, compress, gds, gdv)
    compare_propagation(gr, t32, ds, dv, X, ps, pv if separate_pv else None, Ud, Vd, wd, bd)


def compare_propagation(gr, t32, ds, dv, X, ps, pv, Ud, Vd, wd, bd):
    """Every output and gradient against the oracle (parity.check, calibrated by the fp32 torch run);
    pv None: the projected values are the layer values."""
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    check("grad layer_val", X.grad, gr["val"] + (0.0 if pv is not None else gr["pv"]), t32["val"])
    check("grad projected_state", ps.grad, gr["ps"], t32["ps"])
    if pv is not None:
        check("grad projected_val", pv.grad, gr["pv"], t32["pv"])
    for t, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        if t is not None:
            check(f"grad {name}", t.grad, gr[name], t32[name])


def test_topk_with_k_at_least_n_is_dense(dev):
    import jakal_net_native as jn

    B, N, D, r = 2, 40, 16, 4
    _, state, val, U, V, w = _inputs(4101, B, N, D, r)
    w_hat = (w / w.norm()).to(dev)
    args = ("low_rank_bilinear", w_hat, None, V.to(dev), None, U.to(dev), None, "softsign", val.to(dev),
            state.to(dev), val.to(dev))
    a = jn.propagation_topk(*args, N + 5, N, N)
    b = jn.propagation_dense(*args, None, N, N)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    ref = O.propagation_forward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, mode="dense",
                                kind="softsign")
    _close(_np(a[1]), ref["delta_val"], what="delta_val")


def test_dense_source_state_weighting(dev):
    # edges weighted by the source state == unweighted op on (w, w * pv) (jakal_net_native.cpp:5991-6015)
    import jakal_net_native as jn

    B, N, D, r = 2, 32, 8, 4
    g, state, val, U, V, w = _inputs(4201, B, N, D, r)
    sw = torch.rand(B, N, generator=g) + 0.1
    w_hat = w / w.norm()
    ds, dv = jn.propagation_dense("low_rank_bilinear", w_hat.to(dev), None, V.to(dev), None, U.to(dev), None,
                                  "softsign", val.to(dev), state.to(dev), val.to(dev), sw.to(dev), N, N)
    s = O.lowrank_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), 0.0)
    e = (s / (1 + np.abs(s))) * _np(sw)[:, None, :]
    _close(_np(ds), e.sum(-1), what="state-weighted delta_state")
    _close(_np(dv), e @ _np(val), what="state-weighted delta_val")


def test_dense_propagation_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearPairwise, Propagation

    torch.manual_seed(61)
    layer = Layer(dim=6, num_nodes=13, state=torch.randn(2, 13, device=dev), val=torch.randn(2, 13, 6, device=dev))
    kw = dict(state_proj_fn=lambda s: s * 0.75 + 0.5, val_proj_fn=lambda v: v * 2.0 - 1.0)
    ref = Propagation(LowRankBilinearPairwise(6, 3).to(dev), implementation="reference", **kw)
    nat = Propagation(LowRankBilinearPairwise(6, 3).to(dev), implementation="native", **kw)
    nat.pairwise_fn.load_state_dict(ref.pairwise_fn.state_dict())
    a, b = ref.compute_delta(layer), nat.compute_delta(layer)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-5)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-5)


def test_dense_medium_shape_backward(dev):
    """B=2, N=512, D=64, r=16: full oracle forward and backward."""
    import jakal_net_native as jn

    B, N, D, r = 2, 512, 64, 16
    g, state, val, U, V, w = _inputs(4301, B, N, D, r)
    w_hat = w / w.norm()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    Ud, Vd, wd = (t.to(dev).requires_grad_(True) for t in (U, V, w_hat))
    ds, dv = jn.propagation_dense("low_rank_bilinear", wd, None, Vd, None, Ud, None, "signed_abs_softmax", X, ps, X,
                                  None, N, N)
    gds, gdv = torch.randn(B, N, generator=g), torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    gr = O.propagation_backward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, _np(gds), _np(gdv),
                                mode="dense", kind="signed_abs_softmax")
    t32 = torch32_propagation(dev, val, state, None, U, V, w_hat, None, np.ones((B, N, N), dtype=bool),
                              "signed_abs_softmax", gds, gdv)
    compare_propagation(gr, t32, ds, dv, X, ps, None, Ud, Vd, wd, None)


@pytest.fixture
def chunk_batches():
    """Dense propagation in batch chunks: set the edge budget so that each chunk
    holds `n` batch elements (the default budget keeps small problems whole)."""
    import jakal_net_native as jn

    def use(n, N):
        jn.set_dense_edge_bytes(n * N * N * 4)

    yield use
    jn.set_dense_edge_bytes()


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("separate_pv", [False, True])
def test_dense_batch_chunks(dev, chunk_batches, compress, separate_pv):
    """Chunks of 2 of 3 batch elements (a ragged last chunk): no edge matrix is
    kept; the backward rebuilds each chunk's edges from the projections."""
    chunk_batches(2, 64)
    _check_dense(dev, compress, separate_pv, 64, True, B=3, D=24, r=6)


@pytest.mark.parametrize("compress", ["softsign", "signed_entmax15"])
def test_dense_batch_chunks_causal(dev, chunk_batches, compress):
    import test_gpu_window as TW

    chunk_batches(1, 200)
    TW.test_full_causal_window_runs_dense(dev, compress, True, 0)
