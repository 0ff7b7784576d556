"""GPU parity for one head of more than 128 ranks.

The reference composites take any rank (native/jakal_net_native.cpp:714-832,
5962-6076, 6705-6914); its own query-block benchmark leaves the rank at
dim // 2 (scripts/progressive_b_example.py:435-440, 1470-1474), 256 at
d = 512.  Past the register kernels' 128 rank slots the library runs the
scored-rows select, the window scores with the whole query row in LDS, and
the rank-chunked gradient kernels (rank_rows_grad_kernel for dQ of the row
and route passes, rank_cols_grad_kernel for dK and the scale-vector
partials).  Every output and gradient is checked against the float64 oracle
as in the other parity tests (tests/parity.py), on the same runners, at ranks
in 16-byte chunks (160, 192, 256) and off them (131).
"""

import pytest
import torch

from test_gpu_dense import _check_dense
from test_gpu_topk import _c1_inputs, _run_topk
from test_gpu_transition import _run as _run_transition
from test_gpu_transition_dense import _run as _run_transition_dense
from test_gpu_window import _run as _run_window

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


@pytest.mark.parametrize("r,D,compress,separate_pv,k", [
    (256, 64, "softsign", False, 8),           # fused column pass (16-byte value rows)
    (160, 64, "signed_entmax15", True, 70),    # k past the register select
    (131, 62, "signed_abs_softmax", True, 8),  # unaligned ranks and value rows: scalar paths
])
def test_topk_wide_rank_matches_oracle(dev, r, D, compress, separate_pv, k):
    _run_topk(dev, _c1_inputs(seed=2200 + r, B=2, N=300, D=D, r=r), compress, separate_pv, k, min_checkable=0.5)


@pytest.mark.parametrize("r,window,compress,separate_pv", [
    (192, 40, "softsign", False),          # band kernels
    (131, 150, "signed_entmax15", True),   # wider than a band: edge kernels, scalar ranks
])
def test_window_wide_rank_matches_oracle(dev, r, window, compress, separate_pv):
    _run_window(dev, 2300 + r, 2, 260, 48, r, window, compress, separate_pv)


@pytest.mark.parametrize("r,topk,Nd,kind", [
    (256, 8, 96, "softmax"),
    (131, 70, 96, "signed_entmax15"),      # more than 64 routes per source
    (200, 300, 64, "signed_abs_softmax"),  # topk >= Nd: every destination (all-keys scores)
])
def test_transition_wide_rank_matches_oracle(dev, r, topk, Nd, kind):
    _run_transition(dev, 2400 + r, 2, 200, Nd, 40, 48, r, topk, 1.0, kind)


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax"])
def test_dense_wide_rank_matches_oracle(dev, compress):
    _check_dense(dev, compress, True, 96, True, B=2, D=24, r=256)


def test_dense_transition_wide_rank_matches_oracle(dev):
    _run_transition_dense(dev, 2500, 2, 96, 64, 40, 48, 192, 1.0, "softmax")


def test_sparse_propagation_api_native_runs_rank_256(dev):
    """The mirror's SparsePropagation with a rank-256 pairwise module (the
    reference benchmark's default at d = 512) runs on the HIP library and
    agrees with its reference implementation."""
    from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

    torch.manual_seed(41)
    layer = Layer(dim=64, num_nodes=200, state=torch.randn(2, 200, device=dev),
                  val=torch.randn(2, 200, 64, device=dev))
    pair = LowRankBilinearPairwise(64, 256).to(dev)
    ref = SparsePropagation(pair, sparse_type="topk", topk=6, implementation="reference")
    nat = SparsePropagation(pair, sparse_type="topk", topk=6, implementation="native")
    a, b = ref.compute_delta(layer), nat.compute_delta(layer)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-4)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-4)
