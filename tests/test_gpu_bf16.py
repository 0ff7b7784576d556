"""bf16 layers through the native ops (HIP library) against the float64 oracle.

Layer states and values arrive in bfloat16 (as under autocast).  The edge-list
ops keep the value rows in bf16 (the *_bf16 entry points): gathers read and
write bf16, sums accumulate in fp32, the top-k select ranks
bf16(q * w) . bf16(key) on bf16 MFMAs.  Outputs and the gradients that reach
the bf16 leaves differ from the oracle -- evaluated on the same bf16 inputs --
by bf16 rounding: rtol 2e-2, the bf16 tolerance of the hot path.  Index
parity is exact on rows whose k-th/(k+1)-th gap exceeds twice the bound of
the operand rounding (tests/parity.py, bf16_select_scores).  Dense layers of
at least 128 nodes and value columns (multiples of 8) run their N x N
products on bf16 MFMA with the fp32 edge matrix rounded to bf16 where it
multiplies values; smaller ones compute in fp32 from the bf16 inputs.
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import (bf16_linear64, bf16_select_scores, check_bf16_calibrated, check_selection, torch32_propagation,
                    torch32_transition)

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _np(t):
    return t.detach().double().cpu().numpy()


def _pairwise_params(seed, D, r):
    g = torch.Generator().manual_seed(seed)
    bound = math.sqrt(6.0 / (D + r))
    U = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    V = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    return g, U, V, w


@pytest.mark.parametrize("mode", ["topk", "window", "dense"])
def test_bf16_propagation(dev, mode):
    run_bf16_propagation(dev, mode, B=2, N=128, D=32, r=8)


@pytest.mark.parametrize("mode", ["topk", "window"])
def test_bf16_projection_gemms_on_ragged_tiles(dev, mode):
    """Projection and gradient GEMMs of a bf16 layer on the bf16 MFMA kernel
    (128 x 128 tiles) with every extent ragged: 2,100 rows, D = 200 (K of the
    projection: three whole 64-wide slices and a partial one; N of the input
    gradient), and the weight gradient's K of 2,100 rows in split-K chunks of
    320 (the last chunk empty)."""
    run_bf16_propagation(dev, mode, B=3, N=700, D=200, r=64, k=12, seed=5011)


def run_bf16_propagation(dev, mode, B, N, D, r, k=8, seed=5001):
    import jakal_net_native as jn

    g, U, V, w = _pairwise_params(seed, D, r)
    val = torch.randn(B, N, D, generator=g).bfloat16()
    state = torch.randn(B, N, generator=g).bfloat16()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    w_hat = (w / w.norm()).to(dev)
    args = ("low_rank_bilinear", w_hat, None, V.to(dev), None, U.to(dev), None, "softsign", X, ps, X)
    if mode == "topk":
        ds, dv, idx, score = jn.propagation_topk_selection(*args, k, N, N)
        scores, tol = bf16_select_scores(bf16_linear64(_np(val), _np(U)), bf16_linear64(_np(val), _np(V)),
                                         _np(w_hat))
        assert check_selection(idx.cpu().numpy(), score.cpu().numpy(), scores, k, gap=2 * tol, score_tol=tol) > 0.5
        mask = O.mask_from_indices(idx.cpu().numpy(), N)
        kw = dict(mode="topk", topk=k, mask=mask)
    elif mode == "window":
        ds, dv = jn.propagation_window(*args, 16, N, N)
        kw = dict(mode="window", window=16)
    else:
        ds, dv = jn.propagation_dense(*args, None, N, N)
        kw = dict(mode="dense")
    assert ds.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    gds = torch.randn(B, N, generator=g).bfloat16()
    gdv = torch.randn(B, N, D, generator=g).bfloat16()
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    assert X.grad.dtype == torch.bfloat16
    gr = O.propagation_backward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, _np(gds), _np(gdv),
                                kind="softsign", **kw)
    mask = O.propagation_forward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, kind="softsign",
                                 **kw)["mask"]
    # the top-k scores come from bf16 operands; window and dense scores are fp32;
    # the projections are bf16 GEMMs, except for dense layers off the bf16
    # dense path (upcast to fp32), whose edges multiply the values in bf16
    dense_bf16 = mode == "dense" and jn.dense_bf16_shapes_ok(N, D)
    t = torch32_propagation(dev, val, state, None, U, V, w / w.norm(), None, np.ascontiguousarray(mask), "softsign",
                            gds, gdv, bf16_operands=mode == "topk", bf16_linear=mode != "dense" or dense_bf16,
                            bf16_edges=dense_bf16)
    check_bf16_calibrated("delta_state", ds, gr["delta_state"], t["delta_state"])
    check_bf16_calibrated("delta_val", dv, gr["delta_val"], t["delta_val"])
    check_bf16_calibrated("grad layer_val", X.grad, gr["val"] + gr["pv"], t["val"])
    check_bf16_calibrated("grad projected_state", ps.grad, gr["ps"], t["ps"])


def test_bf16_dense_layer_runs_bf16_products(dev):
    """A bf16 dense layer at the bf16 dense entry points' sizes (softsign, pv
    the layer values): the three N x N products on bf16 MFMA, the edge matrix
    rounded to bf16 where it multiplies values."""
    import jakal_net_native as jn

    assert jn.dense_bf16_shapes_ok(256, 128) and not jn.dense_bf16_shapes_ok(256, 120)
    run_bf16_propagation(dev, "dense", B=2, N=256, D=128, r=16, seed=5021)


@pytest.fixture
def chunk_batches():
    import jakal_net_native as jn

    def use(n, N):
        jn.set_dense_edge_bytes(n * N * N * 4)

    yield use
    jn.set_dense_edge_bytes()


# (compress, causal, separate_pv, chunk): the signed kinds' separate score
# gradient pass, the causal K ranges and epilogue tiles, batch chunks
@pytest.mark.parametrize("compress,causal,separate_pv,chunk", [
    ("softsign", True, True, None),
    ("signed_abs_softmax", False, True, None),
    ("signed_entmax15", True, False, 1),
    ("softsign", False, True, 2),
])
def test_bf16_dense_variants(dev, chunk_batches, compress, causal, separate_pv, chunk):
    import jakal_net_native as jn

    B, N, D, r = 3, 264, 136, 24
    if chunk:
        chunk_batches(chunk, N)
    g, U, V, w = _pairwise_params(5031, D, r)
    val = torch.randn(B, N, D, generator=g).bfloat16()
    state = torch.randn(B, N, generator=g).bfloat16()
    pv_cpu = torch.randn(B, N, D, generator=g).bfloat16() if separate_pv else val
    b = 0.15
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True) if separate_pv else X
    w_hat = w / w.norm()
    Ud, Vd, wd = (t.to(dev).requires_grad_(True) for t in (U, V, w_hat))
    bd = torch.tensor(b, device=dev, requires_grad=True)
    args = ("low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X, ps, pv)
    if causal:
        ds, dv = jn.propagation_window(*args, N - 1, N, N)
        kw = dict(mode="window", window=N - 1)
        mask = np.broadcast_to(O.causal_window_mask(N, N - 1), (B, N, N))
    else:
        ds, dv = jn.propagation_dense(*args, None, N, N)
        kw = dict(mode="dense")
        mask = np.ones((B, N, N), dtype=bool)
    assert ds.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    gds = torch.randn(B, N, generator=g).bfloat16()
    gdv = torch.randn(B, N, D, generator=g).bfloat16()
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), b, _np(gds), _np(gdv),
                                kind=compress, **kw)
    t = torch32_propagation(dev, val, state, pv_cpu if separate_pv else None, U, V, w_hat, b,
                            np.ascontiguousarray(mask), compress, gds, gdv, bf16_linear=True, bf16_edges=True)
    check_bf16_calibrated("delta_state", ds, gr["delta_state"], t["delta_state"])
    check_bf16_calibrated("delta_val", dv, gr["delta_val"], t["delta_val"])
    if separate_pv:
        check_bf16_calibrated("grad layer_val", X.grad, gr["val"], t["val"])
        check_bf16_calibrated("grad projected_val", pv.grad, gr["pv"], t["pv"])
    else:
        check_bf16_calibrated("grad layer_val", X.grad, gr["val"] + gr["pv"], t["val"])
    check_bf16_calibrated("grad projected_state", ps.grad, gr["ps"], t["ps"])
    for p, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        check_bf16_calibrated(f"grad {name}", p.grad, gr[name], t[name])


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
def test_bf16_dense_transition(dev, kind):
    """A bf16 dense transition (every source to every destination) at the bf16
    entry points' sizes: the three Ns x Nd products on bf16 MFMA, the routes
    rounded to bf16 where they multiply values; every gradient checked."""
    import jakal_net_native as jn

    B, Ns, Nd, D, r = 2, 256, 136, 128, 16
    assert jn.dense_transition_bf16_shapes_ok(Ns, Nd, D) and not jn.dense_transition_bf16_shapes_ok(Ns, 120, D)
    g = torch.Generator().manual_seed(5041)
    src = torch.randn(B, Ns, D, generator=g).bfloat16()
    dst = torch.randn(B, Nd, D, generator=g).bfloat16()
    state = torch.randn(B, Ns, generator=g).bfloat16()
    pv_cpu = torch.randn(B, Ns, D, generator=g).bfloat16()
    bound = math.sqrt(6.0 / (D + r))
    Ws = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    Wt = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    b, temperature = 0.2, 1.3
    srcd, dstd, pvd = (t.to(dev).requires_grad_(True) for t in (src, dst, pv_cpu))
    psd = state.to(dev).requires_grad_(True)
    Wsd, Wtd, wd = (t.to(dev).requires_grad_(True) for t in (Ws, Wt, w))
    bd = torch.tensor(b, device=dev, requires_grad=True)
    rho = torch.nn.functional.softplus(psd.float())
    ds, dv = jn.transition_pairwise_dense("low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None, None, None,
                                          None, kind, temperature, rho, srcd, dstd, psd, pvd, Ns, Nd)
    assert dv.dtype == torch.bfloat16
    gds = torch.randn(B, Nd, generator=g).bfloat16()
    gdv = torch.randn(B, Nd, D, generator=g).bfloat16()
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    rho_np = _np(rho)
    mask = np.ones((B, Ns, Nd), dtype=bool)
    gr = O.transition_backward(_np(src), _np(dst), rho_np, _np(state), _np(pv_cpu), _np(Ws), _np(Wt), _np(w), b,
                               _np(gds), _np(gdv), topk=Nd, temperature=temperature, mask=mask, kind=kind)
    t = torch32_transition(dev, src, dst, rho.detach().float().cpu(), state, pv_cpu, Ws, Wt, w, b, temperature, None,
                           kind, gds, gdv, bf16_linear=True, bf16_routes=True)
    check_bf16_calibrated("delta_state", ds, gr["delta_state"], t["delta_state"])
    check_bf16_calibrated("delta_val", dv, gr["delta_val"], t["delta_val"])
    check_bf16_calibrated("grad src_val", srcd.grad, gr["src_val"], t["src_val"])
    check_bf16_calibrated("grad dst_val", dstd.grad, gr["dst_val"], t["dst_val"])
    check_bf16_calibrated("grad projected_val", pvd.grad, gr["pv"], t["pv"])
    # state reaches both the projected state and (through softplus) the sender strength
    sig = 1.0 / (1.0 + np.exp(-_np(state)))
    check_bf16_calibrated("grad state", psd.grad, gr["ps"] + gr["sender"] * sig, t["ps"] + t["sender"] * sig)
    for p, name in ((Wsd, "Ws"), (Wtd, "Wt"), (wd, "w"), (bd, "b")):
        check_bf16_calibrated(f"grad {name}", p.grad, gr[name], t[name])


# min_ok: the fraction of rows whose k-th / (k+1)-th gap exceeds twice the bf16
# score tolerance; at k = 80 of 200 destinations few do (the fp32 tests pin
# those selections), so that case asserts only that some rows are checked.
@pytest.mark.parametrize("Nd,k,min_ok", [(24, 4, 0.5), (200, 80, 0.03)])
def test_bf16_transition(dev, Nd, k, min_ok):
    import jakal_net_native as jn

    B, Ns, D, r = 2, 96, 32, 8
    g = torch.Generator().manual_seed(5002)
    src = torch.randn(B, Ns, D, generator=g).bfloat16()
    dst = torch.randn(B, Nd, D, generator=g).bfloat16()
    state = torch.randn(B, Ns, generator=g).bfloat16()
    bound = math.sqrt(6.0 / (D + r))
    Ws = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    Wt = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    srcd = src.to(dev).requires_grad_(True)
    psd = state.to(dev).requires_grad_(True)
    rho = torch.nn.functional.softplus(psd)
    ds, dv, idx, logit = jn.transition_pairwise_topk_routes(
        "low_rank_bilinear_route", Ws.to(dev), None, Wt.to(dev), None, w.to(dev), None, None, None, None, None, 1.0,
        rho, srcd, dst.to(dev), psd, srcd, k, Ns, Nd)
    assert ds.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    gds = torch.randn(B, Nd, generator=g).bfloat16()
    gdv = torch.randn(B, Nd, D, generator=g).bfloat16()
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    logits, tol = bf16_select_scores(bf16_linear64(_np(src), _np(Ws)), bf16_linear64(_np(dst), _np(Wt)), _np(w))
    assert check_selection(idx.cpu().numpy(), logit.cpu().numpy(), logits, k, gap=2 * tol, score_tol=tol) > min_ok
    mask = O.mask_from_indices(idx.cpu().numpy(), Nd)
    rho_np = _np(rho)
    gr = O.transition_backward(_np(src), _np(dst), rho_np, _np(state), _np(src), _np(Ws), _np(Wt), _np(w), 0.0,
                               _np(gds), _np(gdv), topk=k, mask=mask)
    t = torch32_transition(dev, src, dst, rho.detach().float().cpu(), state, src, Ws, Wt, w, None, 1.0, mask,
                           "softmax", gds, gdv, bf16_operands=True)
    check_bf16_calibrated("delta_state", ds, gr["delta_state"], t["delta_state"])
    check_bf16_calibrated("delta_val", dv, gr["delta_val"], t["delta_val"])
    check_bf16_calibrated("grad src_val", srcd.grad, gr["src_val"] + gr["pv"], t["src_val"] + t["pv"])
    # state reaches both the projected state and (through softplus) the sender strength
    sig = 1.0 / (1.0 + np.exp(-_np(state)))
    check_bf16_calibrated("grad state", psd.grad, gr["ps"] + gr["sender"] * sig, t["ps"] + t["sender"] * sig)
