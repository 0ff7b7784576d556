"""bf16 layers through the native ops (HIP library) against the float64 oracle.

Layer states and values arrive in bfloat16 (as under autocast); the ops score
and aggregate in fp32 and return the layer dtype, so the outputs and the
gradients that reach the bf16 leaves differ from the oracle -- evaluated on
the same bf16-rounded inputs -- by bf16 rounding: rtol 2e-2, the bf16
tolerance of the hot path.  Index parity is exact on rows whose k-th/(k+1)-th
gap exceeds 1e-5 (the scores are fp32 sums of bf16-exact products).
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O

pytestmark = pytest.mark.gpu

RTOL = 2e-2


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _np(t):
    return t.detach().double().cpu().numpy()


def _close_bf16(got, want, what, terms=None):
    """|got - want| <= rtol * |want| (+ a small norm-wise atol).  A leaf reached
    by several paths sums its bf16-rounded path gradients in bf16, so its
    error scales with the summed magnitude of the terms (``terms``)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    mag = np.abs(want) if terms is None else sum(np.abs(np.asarray(t, np.float64)) for t in terms)
    atol = RTOL * 1e-2 * max(1.0, float(np.abs(want).max()))
    err = np.abs(got - want) - (atol + RTOL * mag)
    assert err.max() <= 0, f"{what}: max excess {err.max():.3e} (max abs diff {np.abs(got - want).max():.3e})"


def _pairwise_params(seed, D, r):
    g = torch.Generator().manual_seed(seed)
    bound = math.sqrt(6.0 / (D + r))
    U = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    V = torch.empty(r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    return g, U, V, w


@pytest.mark.parametrize("mode", ["topk", "window", "dense"])
def test_bf16_propagation(dev, mode):
    import jakal_net_native as jn

    B, N, D, r = 2, 128, 32, 8
    g, U, V, w = _pairwise_params(5001, D, r)
    val = torch.randn(B, N, D, generator=g).bfloat16()
    state = torch.randn(B, N, generator=g).bfloat16()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    w_hat = (w / w.norm()).to(dev)
    args = ("low_rank_bilinear", w_hat, None, V.to(dev), None, U.to(dev), None, "softsign", X, ps, X)
    if mode == "topk":
        ds, dv, idx, _ = jn.propagation_topk_selection(*args, 8, N, N)
        scores = O.lowrank_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), 0.0)
        ok = O.checkable_rows(scores, 8)
        same = (np.sort(idx.cpu().numpy(), -1) == np.sort(O.topk_indices(scores, 8), -1)).all(-1)
        assert same[ok].all() and ok.mean() > 0.9
        mask = O.mask_from_indices(idx.cpu().numpy(), N)
        kw = dict(mode="topk", topk=8, mask=mask)
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
    ref = O.propagation_forward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, kind="softsign", **kw)
    _close_bf16(_np(ds), ref["delta_state"], "delta_state")
    _close_bf16(_np(dv), ref["delta_val"], "delta_val")
    gr = O.propagation_backward(_np(val), _np(state), _np(val), _np(U), _np(V), _np(w), 0.0, _np(gds), _np(gdv),
                                kind="softsign", **kw)
    _close_bf16(_np(X.grad), gr["val"] + gr["pv"], "grad layer_val", terms=(gr["val"], gr["pv"]))
    _close_bf16(_np(ps.grad), gr["ps"], "grad projected_state")


def test_bf16_transition(dev):
    import jakal_net_native as jn

    B, Ns, Nd, D, r, k = 2, 96, 24, 32, 8, 4
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
    ds, dv, idx, _ = jn.transition_pairwise_topk_routes(
        "low_rank_bilinear_route", Ws.to(dev), None, Wt.to(dev), None, w.to(dev), None, None, None, None, None, 1.0,
        rho, srcd, dst.to(dev), psd, srcd, k, Ns, Nd)
    assert ds.dtype == torch.bfloat16 and dv.dtype == torch.bfloat16
    gds = torch.randn(B, Nd, generator=g).bfloat16()
    gdv = torch.randn(B, Nd, D, generator=g).bfloat16()
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    logits = O.lowrank_route_logits(_np(src), _np(dst), _np(Ws), _np(Wt), _np(w), 0.0)
    ok = O.checkable_rows(logits, k)
    same = (np.sort(idx.cpu().numpy(), -1) == np.sort(O.topk_indices(logits, k), -1)).all(-1)
    assert same[ok].all() and ok.mean() > 0.9
    mask = O.mask_from_indices(idx.cpu().numpy(), Nd)
    rho_np = _np(rho)
    ref = O.transition_forward(_np(src), _np(dst), rho_np, _np(state), _np(src), _np(Ws), _np(Wt), _np(w), 0.0,
                               topk=k, mask=mask)
    _close_bf16(_np(ds), ref["delta_state"], "delta_state")
    _close_bf16(_np(dv), ref["delta_val"], "delta_val")
    gr = O.transition_backward(_np(src), _np(dst), rho_np, _np(state), _np(src), _np(Ws), _np(Wt), _np(w), 0.0,
                               _np(gds), _np(gdv), topk=k, mask=mask)
    _close_bf16(_np(srcd.grad), gr["src_val"] + gr["pv"], "grad src_val", terms=(gr["src_val"], gr["pv"]))
    # state reaches both the projected state and (through softplus) the sender strength
    sig = 1.0 / (1.0 + np.exp(-_np(state)))
    _close_bf16(_np(psd.grad), gr["ps"] + gr["sender"] * sig, "grad state", terms=(gr["ps"], gr["sender"] * sig))
