"""GPU parity of the dense pairwise Transition (HIP library) against the numpy oracle.

Every source routes to every destination (transition.py:238-255,
jakal_net_native.cpp:6705-6914).  Outputs and gradients of every input are
compared with the float64 oracle (``transition_forward/backward`` with an
all-true mask): fp32 tolerance rtol 1e-4 / atol 1e-5, or, for long sums that
miss it (the bias gradient of softmax routes cancels to 0 exactly), within
twice the error of an fp32 torch evaluation of the same op (tests/parity.py).
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
import test_gpu_transition as TR
from parity import torch32_transition

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


def _run(dev, seed, B, Ns, Nd, Dsrc, Ddst, r, temperature, kind, init="xavier", with_bias=True, via_topk=False):
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
    if via_topk:  # a top-k transition keeping every destination runs the dense op
        ds, dv = jn.transition_pairwise_topk("low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None, None, None,
                                             None, temperature, rho, srcd, dstd, psd, pvd, Nd + 3, Ns, Nd, kind)
    else:
        ds, dv = jn.transition_pairwise_dense("low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None, None, None,
                                              None, kind, temperature, rho, srcd, dstd, psd, pvd, Ns, Nd)
    gds = torch.randn(B, Nd, generator=g)
    gdv = torch.randn(B, Nd, Ddst, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    bval = float(b) if with_bias else 0.0
    mask = np.ones((B, Ns, Nd), dtype=bool)
    gr = O.transition_backward(_np(src), _np(dst), _np(rho_cpu), _np(state), _np(pv_cpu), _np(Ws), _np(Wt), _np(w),
                               bval, _np(gds), _np(gdv), topk=Nd, temperature=temperature, mask=mask, kind=kind)
    t32 = torch32_transition(dev, src, dst, rho_cpu, state, pv_cpu, Ws, Wt, w, float(b) if with_bias else None,
                             temperature, None, kind, gds, gdv)
    TR.compare_transition(gr, t32, ds, dv, rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd, bd)


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("temperature", [1.0, 1.7])
def test_dense_transition_matches_oracle(dev, kind, temperature):
    _run(dev, 3101, B=2, Ns=64, Nd=16, Dsrc=32, Ddst=24, r=8, temperature=temperature, kind=kind)


def test_dense_transition_odd_shapes_without_bias(dev):
    _run(dev, 3102, B=3, Ns=37, Nd=29, Dsrc=13, Ddst=7, r=3, temperature=0.9, kind="signed_abs_softmax",
         with_bias=False)


@pytest.mark.parametrize("kind", ["softmax", "signed_entmax15"])
def test_dense_transition_medium(dev, kind):
    _run(dev, 3103, B=2, Ns=300, Nd=140, Dsrc=136, Ddst=72, r=48, temperature=1.2, kind=kind)


def test_topk_over_every_destination_runs_dense(dev):
    _run(dev, 3104, B=2, Ns=90, Nd=80, Dsrc=24, Ddst=16, r=8, temperature=1.0, kind="softmax", via_topk=True)


@pytest.mark.parametrize("Ns,Nd", [(1024, 256), (256, 1024)])
def test_dense_transition_c3_shape(dev, Ns, Nd):
    """BASELINE config 3 sizes with every destination kept: B=8, D=512, r=64, default init, T=1."""
    _run(dev, 1003, B=8, Ns=Ns, Nd=Nd, Dsrc=512, Ddst=512, r=64, temperature=1.0, kind="softmax", init="default")


def test_dense_transition_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearRoute, Transition

    torch.manual_seed(52)
    src = Layer(dim=6, num_nodes=12, state=torch.randn(2, 12, device=dev), val=torch.randn(2, 12, 6, device=dev))
    dst = Layer(dim=5, num_nodes=9, state=torch.randn(2, 9, device=dev), val=torch.randn(2, 9, 5, device=dev))
    kw = dict(val_proj_fn=torch.nn.Linear(6, 5).to(dev), state_proj_fn=lambda s: s * 0.5 + 1.0)
    for compress in ("softmax", "signed_abs_softmax", "signed_entmax15"):
        ref = Transition(LowRankBilinearRoute(6, 5, rank=4).to(dev), implementation="reference",
                         route_compress_name=compress, **kw)
        nat = Transition(LowRankBilinearRoute(6, 5, rank=4).to(dev), implementation="native",
                         route_compress_name=compress, **kw)
        nat.route_fn.load_state_dict(ref.route_fn.state_dict())
        a, b = ref.compute_delta(src, dst), nat.compute_delta(src, dst)
        assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-5)
        assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-5)
