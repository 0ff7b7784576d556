"""The fused score-scale op jn_unit_scale_{forward,backward} (w / max(||w||, 1e-6)
per row, LowRankBilinearPairwise.normalized_weight, reference modules.py:85-87)
against the float64 oracle (forward) and float64 autograd of the same formula
(gradient), including rows below the clamp and a zero row."""

import numpy as np
import pytest
import torch

import jakal_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401

    return torch.device("cuda:0")


@pytest.mark.parametrize("rows,r", [(1, 1), (1, 64), (3, 16), (8, 200)])
def test_unit_scale_matches_the_formula(dev, rows, r):
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(7200 + rows * 7 + r)
    w = torch.randn(rows, r, generator=g)
    if rows >= 3:
        w[1] *= 1e-8  # below the clamp: w / 1e-6
        w[2] = 0.0
    gout = torch.randn(rows, r, generator=g)
    wd = w.to(dev).requires_grad_(True)
    out = jn.unit_scale(wd if rows > 1 else wd.view(r))
    out.backward(gout.to(dev) if rows > 1 else gout.view(r).to(dev))
    want = np.stack([O.normalized_weight(x) for x in w.double().numpy()])
    got = out.detach().double().cpu().numpy().reshape(rows, r)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7), np.abs(got - want).max()

    w64 = w.double().requires_grad_(True)
    ref = w64 / w64.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    ref.backward(gout.double())
    # the gradient is g / d minus its projection on w: two terms of size |g| / d
    # that can cancel (r = 1: exactly), so the tolerance scales with them
    gw = wd.grad.double().cpu()
    d = w64.detach().norm(dim=-1, keepdim=True).clamp_min(1e-6)
    term = gout.double().abs().max(dim=-1, keepdim=True).values / d
    err = (gw - w64.grad).abs()
    assert bool((err <= 1e-5 * w64.grad.abs() + 1e-6 * term).all()), float((err / term).max())
