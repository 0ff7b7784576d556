"""GPU parity of SparseTransition routing (HIP library) against the numpy oracle.

Each source row selects its top-k destinations (transition.py:437-444).  Index
parity is exact on rows whose k-th/(k+1)-th logit gap exceeds 1e-5; values
and gradients are compared with the oracle evaluated on the selection the GPU
made, within rtol 1e-4 / atol 1e-5 (fp32).  The outputs (sums over a
destination's incoming routes) and the gradients (sums over edges and over D-
or r-long dot products) have terms that can cancel; a tensor that misses the
literal tolerance must stay within twice the error of an fp32 torch
evaluation of the same op on the same selection (tests/parity.py).
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import check, torch32_transition

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


def _run(dev, seed, B, Ns, Nd, Dsrc, Ddst, r, topk, temperature, kind, init="xavier", with_bias=True):
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(seed)
    src = torch.randn(B, Ns, Dsrc, generator=g)
    dst = torch.randn(B, Nd, Ddst, generator=g)
    state = torch.randn(B, Ns, generator=g)
    pv_cpu = torch.randn(B, Ns, Ddst, generator=g)
    rho_cpu = torch.nn.functional.softplus(state)
    if init == "xavier":
        bs, bt = math.sqrt(6.0 / (Dsrc + r)), math.sqrt(6.0 / (Ddst + r))
    else:  # nn.Linear default
        bs, bt = 1.0 / math.sqrt(Dsrc), 1.0 / math.sqrt(Ddst)
    Ws = torch.empty(r, Dsrc).uniform_(-bs, bs, generator=g)
    Wt = torch.empty(r, Ddst).uniform_(-bt, bt, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    b = torch.tensor(0.2) if with_bias else None

    leaves = [t.to(dev).requires_grad_(True) for t in (rho_cpu, src, dst, state, pv_cpu, Ws, Wt, w)]
    rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd = leaves
    bd = b.to(dev).requires_grad_(True) if with_bias else None
    ds, dv, idx, logit = jn.transition_pairwise_topk_routes(
        "low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None, None, None, None, temperature, rho, srcd,
        dstd, psd, pvd, topk, Ns, Nd, kind)
    gds = torch.randn(B, Nd, generator=g)
    gdv = torch.randn(B, Nd, Ddst, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    bval = float(b) if with_bias else 0.0
    logits = O.lowrank_route_logits(_np(src), _np(dst), _np(Ws), _np(Wt), _np(w), bval, temperature)
    k = min(topk, Nd)
    got_idx = idx.cpu().numpy()
    assert got_idx.shape == (B, Ns, k)
    assert (got_idx >= 0).all() and (got_idx < Nd).all()
    srt = np.sort(got_idx, axis=-1)
    if k < Nd:
        assert (np.diff(srt, axis=-1) > 0).all()
        ok = O.checkable_rows(logits, k)
        ref_idx = np.sort(O.topk_indices(logits, k), axis=-1)
        assert (srt == ref_idx).all(-1)[ok].all(), "checkable rows select different destinations"
        assert ok.mean() > 0.5
    else:
        assert (srt == np.arange(Nd)).all()
    _close(logit.cpu().numpy(), np.take_along_axis(logits, got_idx, axis=-1), rtol=1e-5, atol=1e-5,
           what="route logits")

    mask = O.mask_from_indices(got_idx, Nd)
    gr = O.transition_backward(_np(src), _np(dst), _np(rho_cpu), _np(state), _np(pv_cpu), _np(Ws), _np(Wt), _np(w),
                               bval, _np(gds), _np(gdv), topk=k, temperature=temperature, mask=mask, kind=kind)
    t32 = torch32_transition(
        dev, src, dst, rho_cpu, state, pv_cpu, Ws, Wt, w, float(b) if with_bias else None, temperature, mask, kind,
        gds, gdv)
    compare_transition(gr, t32, ds, dv, rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd, bd)


def compare_transition(gr, t32, ds, dv, rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd, bd):
    """Every output and gradient against the oracle (parity.check, calibrated by the fp32 torch run)."""
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    for t, name in ((rho, "sender"), (srcd, "src_val"), (dstd, "dst_val"), (psd, "ps"), (pvd, "pv"), (Wsd, "Ws"),
                    (Wtd, "Wt"), (wd, "w"), (bd, "b")):
        if t is not None:
            check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("temperature", [1.0, 1.7])
def test_transition_forward_backward_matches_oracle(dev, kind, temperature):
    _run(dev, 3001, B=2, Ns=64, Nd=16, Dsrc=32, Ddst=24, r=8, topk=4, temperature=temperature, kind=kind)


@pytest.mark.parametrize("kind", ["signed_abs_softmax", "signed_entmax15"])
def test_transition_topk_above_32(dev, kind):
    _run(dev, 3004, B=2, Ns=80, Nd=100, Dsrc=16, Ddst=12, r=4, topk=48, temperature=1.1, kind=kind)


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
def test_transition_topk_above_64(dev, kind):
    """More than 64 destinations per source: the scored-rows select and the
    route kernels' 64-edge blocks."""
    _run(dev, 3006, B=2, Ns=40, Nd=300, Dsrc=16, Ddst=12, r=6, topk=100, temperature=1.2, kind=kind)


def test_transition_topk_above_64_odd_rows(dev):
    # value rows of 10 elements (no 16-byte packs), no bias
    _run(dev, 3007, B=2, Ns=33, Nd=150, Dsrc=9, Ddst=10, r=3, topk=70, temperature=0.9, kind="signed_abs_softmax",
         with_bias=False)


@pytest.mark.parametrize("topk", [16, 40])
def test_transition_every_destination(dev, topk):
    # k >= Nd keeps every destination (transition.py:437-440)
    _run(dev, 3002, B=2, Ns=48, Nd=16, Dsrc=20, Ddst=12, r=5, topk=topk, temperature=1.3, kind="softmax")


def test_transition_odd_shapes_without_bias(dev):
    _run(dev, 3003, B=3, Ns=37, Nd=29, Dsrc=13, Ddst=7, r=3, topk=5, temperature=0.9, kind="signed_abs_softmax",
         with_bias=False)


@pytest.mark.parametrize("Ns,Nd", [(1024, 256), (256, 1024)])
def test_transition_c3_shape(dev, Ns, Nd):
    """B=8, D=512, r=64, top-16 (S->B and B->S), default init, T=1."""
    _run(dev, 1003, B=8, Ns=Ns, Nd=Nd, Dsrc=512, Ddst=512, r=64, topk=16, temperature=1.0, kind="softmax",
         init="default")


def test_sparse_transition_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearRoute, SparseTransition

    torch.manual_seed(51)
    src = Layer(dim=6, num_nodes=12, state=torch.randn(2, 12, device=dev), val=torch.randn(2, 12, 6, device=dev))
    dst = Layer(dim=5, num_nodes=9, state=torch.randn(2, 9, device=dev), val=torch.randn(2, 9, 5, device=dev))
    kw = dict(topk=3, val_proj_fn=torch.nn.Linear(6, 5).to(dev), state_proj_fn=lambda s: s * 0.5 + 1.0)
    ref = SparseTransition(LowRankBilinearRoute(6, 5, rank=4).to(dev), implementation="reference", **kw)
    nat = SparseTransition(LowRankBilinearRoute(6, 5, rank=4).to(dev), implementation="native", **kw)
    nat.route_fn.load_state_dict(ref.route_fn.state_dict())
    a, b = ref.compute_delta(src, dst), nat.compute_delta(src, dst)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-5)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-5)
