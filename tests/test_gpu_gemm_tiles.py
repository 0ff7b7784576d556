"""Every GEMM workgroup tile (32 x 32, 64 x 64 and 128 x 128) and the automatic
choice (0: the fp32 projection GEMMs of 128+ extents on bf16 thirds) against
the oracle.

The library picks the tile per call from the output extents; these tests force
each tile in turn (jn_set_gemm_tile; 32 applies to the projection products and
their gradients, 64 to the others) on ops whose extents are ragged against
every tile, so every GEMM of the forward and backward passes (projections,
their input and weight gradients, dense scores, aggregation and its
gradients) runs partial tiles, unaligned rows and split-K under every tiling.
The 128 x 128 kernel has preconditions (extents and strides in float4 units,
B split at a multiple of 16); shapes that miss them run the 64 x 64 kernel
even when 128 is forced, and are included too.
Tolerances are those of the per-op tests (fp32: rtol 1e-4, atol 1e-5, or
for long sums within twice the error of an fp32 torch evaluation).
"""

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import torch32_propagation
import test_gpu_bf16 as TB
import test_gpu_dense as TD
import test_gpu_topk as TT
import test_gpu_transition as TR
import test_gpu_window as TW

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[0, 32, 64, 128])
def tile(request):
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native as jn

    jn.set_gemm_tile(request.param)
    yield request.param
    jn.set_gemm_tile(0)


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def test_dense_ragged(dev, tile):
    import jakal_net_native as jn

    B, N, D, r = 2, 200, 72, 12
    g, state, val, U, V, w = TD._inputs(4401, B, N, D, r)
    pv_cpu = torch.randn(B, N, D, generator=g)
    w_hat = w / w.norm()
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True)
    Ud, Vd, wd = (t.to(dev).requires_grad_(True) for t in (U, V, w_hat))
    bd = torch.tensor(0.1, device=dev, requires_grad=True)
    ds, dv = jn.propagation_dense("low_rank_bilinear", wd, bd, Vd, None, Ud, None, "softsign", X, ps, pv, None, N, N)
    gds, gdv = torch.randn(B, N, generator=g), torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    gr = O.propagation_backward(TD._np(val), TD._np(state), TD._np(pv_cpu), TD._np(U), TD._np(V), TD._np(w), 0.1,
                                TD._np(gds), TD._np(gdv), mode="dense", kind="softsign")
    t32 = torch32_propagation(dev, val, state, pv_cpu, U, V, w_hat, 0.1, np.ones((B, N, N), dtype=bool), "softsign",
                              gds, gdv)
    TD.compare_propagation(gr, t32, ds, dv, X, ps, pv, Ud, Vd, wd, bd)


def test_dense_small(dev, tile):
    TD.test_dense_forward_backward_matches_oracle(dev, "signed_abs_softmax", True, 37, False)


def test_dense_softsign_odd_columns(dev, tile):
    # 150 columns (not a multiple of 4): the softsign epilogue stores element-wise from the accumulators
    TD._check_dense(dev, "softsign", True, 150, True, B=2, D=24, r=6)


def test_topk_propagation(dev, tile):
    TT.test_propagation_topk_forward_backward_matches_oracle(dev, "softsign", True, 8)


def test_transition_odd(dev, tile):
    TR._run(dev, 3003, B=3, Ns=37, Nd=29, Dsrc=13, Ddst=7, r=3, topk=5, temperature=0.9, kind="signed_abs_softmax",
            with_bias=False)


@pytest.mark.parametrize("r", [40, 48])  # route weights split at r: 48 keeps the 128 x 128 kernel, 40 does not
def test_transition_medium(dev, tile, r):
    TR._run(dev, 3005, B=2, Ns=300, Nd=140, Dsrc=136, Ddst=72, r=r, topk=8, temperature=1.2, kind="softmax")


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax"])
def test_causal_dense(dev, tile, compress):
    # full causal windows run the dense products with causal K ranges and skip
    # the score tiles above the diagonal (softsign epilogue), under both tiles
    TW.test_full_causal_window_runs_dense(dev, compress, True, 0)


@pytest.mark.parametrize("mode", ["topk", "window"])
def test_bf16_layers(dev, tile, mode):
    # bf16 X in the projection (A), weight-gradient (B) and input-gradient (C)
    # GEMMs; rank 16 splits the weight operands at a multiple of 16, so the
    # 128 x 128 kernel takes all three uses when forced
    TB.run_bf16_propagation(dev, mode, B=2, N=160, D=40, r=16, k=8, seed=5003)


@pytest.mark.parametrize("D,r,separate_pv", [(136, 64, True), (512, 64, False), (200, 96, True)])
def test_fp32_projection_gemms_in_bf16_thirds(dev, D, r, separate_pv):
    """The automatic choice (tile 0) runs the fp32 projection, input-gradient
    and weight-gradient GEMMs with extents of 128 and more on gemm_x3_kernel
    (each fp32 operand split exactly into three bf16 terms, six bf16 MFMA
    products): ragged K (D = 136, 200) and N tails, the addend of grad X when
    pv is X, split-K over the rows; the fp32 tolerance of the per-op tests."""
    TT._run_topk(dev, TT._c1_inputs(seed=4500 + D, B=2, N=640, D=D, r=r), "softsign", separate_pv, 16,
                 min_checkable=0.5)
