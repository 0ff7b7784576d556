"""GPU parity of the top-k hot path (HIP library) against the numpy oracle.

Index parity is exact on rows whose k-th/(k+1)-th score gap exceeds 1e-5;
values and gradients are compared to the oracle evaluated on the selection the
GPU made (identical to the oracle's on every checkable row), fp32 tolerance
rtol 1e-4 / atol 1e-5 as stated for the hot path, or, for long sums that miss
it, at most twice the error of an fp32 torch evaluation (tests/parity.py).
The full C4 shape, forward and backward, is in test_gpu_full_shape.py.
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import check, check_selection, torch32_propagation

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
    if want.size == 0:
        return
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert err.max() <= 0, f"{what}: max excess {err.max():.3e} (max abs diff {np.abs(got - want).max():.3e})"


@pytest.mark.parametrize("r,k,Nq,Nk", [(3, 2, 9, 9), (16, 8, 256, 256), (64, 32, 200, 333), (64, 1, 70, 50),
                                       (32, 16, 130, 1024), (100, 5, 64, 97), (64, 33, 100, 300),
                                       (16, 48, 150, 49), (64, 64, 257, 2000), (8, 64, 64, 65),
                                       (64, 32, 130, 4096), (16, 8, 70, 2048), (64, 64, 100, 3001),
                                       (5, 3, 64, 2500)])
def test_select_matches_oracle(dev, r, k, Nq, Nk):
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(100 + r + k)
    B = 2
    q = torch.randn(B, Nq, r, generator=g)
    key = torch.randn(B, Nk, r, generator=g)
    scale = torch.rand(r, generator=g) + 0.5
    bias = torch.tensor(0.25)
    for scale_on_query, temp in ((False, 1.0), (True, 1.7)):
        idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), scale.to(dev), bias.to(dev),
                                             scale_on_query, temp, k)
        sq = q.double().numpy() * (scale.double().numpy() if scale_on_query else 1.0)
        sk = key.double().numpy() * (1.0 if scale_on_query else scale.double().numpy())
        ref = (sq @ np.swapaxes(sk, 1, 2) + 0.25) / temp
        check_selection(idx.cpu().numpy(), score.cpu().numpy(), ref, k)


@pytest.mark.parametrize("Nk", [200, 2100])
def test_select_exact_ties_go_to_lower_index(dev, Nk):
    import jakal_net_native as jn

    # all keys identical -> all scores tie; the k lowest indices must win
    B, Nq, r, k = 1, 64, 8, 5
    q = torch.randn(B, Nq, r)
    key = torch.ones(B, Nk, r)
    idx, _ = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, k)
    assert (idx.cpu() == torch.arange(k, dtype=torch.int32)).all()


@pytest.mark.parametrize("k,groups", [(8, (4, 2)), (40, (4, 4))])
def test_select_few_dominant_keys(dev, k, groups):
    """Even rows score a few keys near the start (one in each 4-key group of
    several 16-key tiles) far above everything else, so fewer than k keys stand
    out and the rest of the selection comes from the ordinary keys.  Odd rows
    see ordinary random scores."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(77 + k)
    B, Nq, Nk, r = 1, 128, 2048, 4
    ng, nh = groups
    span = 256 // nh
    special = [4 * gi + span * h for h in range(nh) for gi in range(ng)]
    key = torch.zeros(B, Nk, r)
    key[..., 0] = torch.randn(B, Nk, generator=g)
    key[..., 1] = torch.randn(B, Nk, generator=g)
    key[0, special, 0] = 100.0 + 0.5 * torch.arange(len(special), dtype=torch.float32)
    q = torch.zeros(B, Nq, r)
    q[0, 0::2, 0] = 1.0
    q[0, 1::2, 1] = 1.0
    idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, k)
    ref = q.double().numpy() @ np.swapaxes(key.double().numpy(), 1, 2)
    check_selection(idx.cpu().numpy(), score.cpu().numpy(), ref, k)
    top = np.sort(idx.cpu().numpy()[0, 0::2], axis=-1)
    assert set(special) <= set(top[0].tolist())


def _c1_inputs(seed=1001, B=2, N=256, D=64, r=16):
    g = torch.Generator().manual_seed(seed)
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    V = torch.empty(r, D)
    U = torch.empty(r, D)
    bound = math.sqrt(6.0 / (D + r))
    V.uniform_(-bound, bound, generator=g)
    U.uniform_(-bound, bound, generator=g)
    w = torch.rand(r, generator=g) + 0.5
    b = torch.tensor(0.1)
    return state, val, U, V, w, b


@pytest.mark.parametrize("compress", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("separate_pv,k", [(False, 8), (True, 8), (True, 64)])
def test_propagation_topk_forward_backward_matches_oracle(dev, compress, separate_pv, k):
    _run_topk(dev, _c1_inputs(), compress, separate_pv, k, min_checkable=0.9 if k <= 8 else 0.5)


@pytest.mark.parametrize("N,D,k,compress", [(1100, 520, 32, "softsign"), (1500, 388, 64, "signed_entmax15"),
                                            (1300, 512, 5, "signed_abs_softmax")])
def test_propagation_topk_split_row_backward(dev, N, D, k, compress):
    """Value rows of a batch element above 2 MiB with 256 < D <= 1024: the row
    backward computes its dot products in two column slabs first (ragged second
    slab for D = 520 and 388)."""
    _run_topk(dev, _c1_inputs(seed=1100 + k, B=1, N=N, D=D, r=24), compress, True, k, min_checkable=0.3)


def _run_topk(dev, inputs, compress, separate_pv, k, min_checkable):
    """Outputs and gradients against the float64 oracle on the GPU's selection;
    tensors that miss the literal tolerance (long fp32 sums at larger D, r and
    k) must stay within twice the error of an fp32 torch evaluation of the
    same op on the same selection (parity.check)."""
    import jakal_net_native as jn

    state, val, U, V, w, b = inputs
    B, N, D = val.shape
    g = torch.Generator().manual_seed(7)
    pv_cpu = torch.randn(B, N, D, generator=g) if separate_pv else val
    w_hat = w / w.norm()

    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True) if separate_pv else X
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd, bd = w_hat.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    ds, dv, idx, score = jn.propagation_topk_selection("low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X,
                                                       ps, pv, k, 128, 128)
    gds = torch.randn(B, N, generator=g)
    gdv = torch.randn(B, N, D, generator=g)
    (ds * gds.to(dev)).sum().backward(retain_graph=True)
    (dv * gdv.to(dev)).sum().backward()

    # the selection the forward aggregated, against float64 scores
    scores = O.lowrank_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), float(b))
    frac = check_selection(idx.cpu().numpy(), score.cpu().numpy(), scores, k)
    assert frac > min_checkable  # deeper cuts sit in denser parts of the score distribution
    mask = O.mask_from_indices(idx.cpu().numpy(), N)
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="topk", topk=k, kind=compress, mask=mask)
    t32 = torch32_propagation(dev, val, state, pv_cpu if separate_pv else None, U, V, w_hat, float(b), mask,
                              compress, gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    check("grad layer_val", X.grad, gr["val"] + (0.0 if separate_pv else gr["pv"]), t32["val"])
    check("grad projected_state", ps.grad, gr["ps"], t32["ps"])
    if separate_pv:
        check("grad projected_val", pv.grad, gr["pv"], t32["pv"])
    for t, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


def test_sparse_propagation_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearPairwise, SparsePropagation

    torch.manual_seed(31)
    layer = Layer(dim=5, num_nodes=9, state=torch.randn(2, 9, device=dev), val=torch.randn(2, 9, 5, device=dev))
    ref = SparsePropagation(LowRankBilinearPairwise(5, 3).to(dev), sparse_type="topk", topk=3,
                            state_proj_fn=lambda s: s * 1.25 - 0.5, val_proj_fn=lambda v: v * 0.5 + 0.25,
                            implementation="reference")
    nat = SparsePropagation(LowRankBilinearPairwise(5, 3).to(dev), sparse_type="topk", topk=3,
                            state_proj_fn=lambda s: s * 1.25 - 0.5, val_proj_fn=lambda v: v * 0.5 + 0.25,
                            implementation="native")
    nat.pairwise_fn.load_state_dict(ref.pairwise_fn.state_dict())
    a, b = ref(layer), nat(layer)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-5)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-5)


def test_c4_shape_select_every_row(dev):
    """The select at the full C4 shape (B=16, N=4096, r=64, k=32, unit-norm value
    rows, default init) on every one of the 65,536 rows, against fp32 scores of
    all 2.7e8 pairs from torch (scored one batch element at a time): each row's
    k indices are distinct and in range, its scores are sorted descending and
    within 1e-6 of the torch scores of those indices, and no index left out
    scores more than 1e-5 above the row's k-th score (the gap rule).  A
    dropped key, a wrong index, a misplaced merge or a lost candidate fails one
    of these on some row."""
    import jakal_net_native as jn

    B, N, D, r, k = 16, 4096, 512, 64, 32
    g = torch.Generator().manual_seed(1004)
    val = torch.randn(B, N, D, generator=g)
    val = val / val.norm(dim=-1, keepdim=True)
    bound = 1.0 / D ** 0.5
    U = (torch.rand(r, D, generator=g) * 2 - 1) * bound
    V = (torch.rand(r, D, generator=g) * 2 - 1) * bound
    w_hat = torch.ones(r) / r ** 0.5
    P = val.to(dev) @ torch.cat([U, V]).to(dev).T
    q = P[..., :r].contiguous()
    key = P[..., r:].contiguous()
    idx, score = jn.low_rank_topk_select(q, key, w_hat.to(dev), None, False, 1.0, k)
    idx = idx.long()
    assert int(idx.min()) >= 0 and int(idx.max()) < N
    srt = idx.sort(dim=-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all()), "repeated index in a row"
    assert bool((score[..., :-1] >= score[..., 1:]).all()), "scores not sorted"
    worst_val, worst_gap = 0.0, -1.0
    for b in range(B):
        S = q[b] @ (key[b] * w_hat.to(dev)).T  # fp32 [N, N]
        picked = S.gather(1, idx[b])
        worst_val = max(worst_val, float((picked - score[b]).abs().max()))
        kth = score[b, :, -1:]
        S.scatter_(1, idx[b], -float("inf"))  # leave out the selected keys
        worst_gap = max(worst_gap, float((S.max(dim=1, keepdim=True).values - kth).max()))
    print(f"C4 select, all rows: max |score - torch score| {worst_val:.2e}, max excluded-over-kth {worst_gap:.2e}")
    assert worst_val <= 1e-6
    assert worst_gap <= 1e-5


@pytest.mark.parametrize("r,k,Nq,Nk", [(16, 100, 70, 500), (8, 1024, 20, 1500), (64, 65, 130, 4096), (8, 3000, 10, 3500),
                                       (5, 700, 33, 701), (8, 16, 40, 70000)])
def test_select_beyond_register_limits(dev, r, k, Nq, Nk):
    """k above 64 or more than 65,535 keys: scored rows (fp32 MFMA GEMM) and a
    radix select per row, with the register select's ordering and tie rule;
    reported scores within fp32 accumulation error of the exact ones."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(300 + r + k)
    B = 2
    q = torch.randn(B, Nq, r, generator=g)
    key = torch.randn(B, Nk, r, generator=g)
    scale = torch.rand(r, generator=g) + 0.5
    bias = torch.tensor(-0.5)
    for scale_on_query, temp in ((False, 1.0), (True, 0.8)):
        idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), scale.to(dev), bias.to(dev),
                                             scale_on_query, temp, k)
        sq = q.double().numpy() * (scale.double().numpy() if scale_on_query else 1.0)
        sk = key.double().numpy() * (1.0 if scale_on_query else scale.double().numpy())
        ref = (sq @ np.swapaxes(sk, 1, 2) - 0.5) / temp
        tol = r * 2.0 ** -24 * (np.abs(sq) @ np.swapaxes(np.abs(sk), 1, 2)).max(-1) / temp
        frac = check_selection(idx.cpu().numpy(), score.cpu().numpy(), ref, k, gap=2 * tol + 1e-5, score_tol=tol)
        print(f"scored-rows select r={r} k={k} Nq={Nq} Nk={Nk}: rows with an unambiguous set {frac:.4f}", flush=True)
        assert frac > 0.9  # 0.98 at k = 65 of 4096 keys, 1.0 at the other shapes


@pytest.mark.parametrize("Nk,k", [(300, 100), (70000, 7)])
def test_large_select_ties_go_to_lower_index(dev, Nk, k):
    import jakal_net_native as jn

    B, Nq, r = 1, 16, 8
    q = torch.randn(B, Nq, r)
    key = torch.ones(B, Nk, r)
    idx, _ = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, k)
    assert (idx.cpu() == torch.arange(k, dtype=torch.int32)).all()


@pytest.mark.parametrize("k", [65, 200])
def test_propagation_topk_large_k(dev, k):
    """Top-k propagation beyond 64 edges per row (softsign), forward and
    backward against the oracle on the GPU's selection."""
    _run_topk(dev, _c1_inputs(seed=1200 + k, B=2, N=400, D=48, r=16), "softsign", True, k, min_checkable=0.3)


def test_propagation_topk_very_large_k(dev):
    """2000 of 2600 sources per row (the scored-rows select's LDS sort over
    2048 slots), forward and backward against the oracle."""
    _run_topk(dev, _c1_inputs(seed=1250, B=1, N=2600, D=24, r=8), "signed_entmax15", True, 2000, min_checkable=0.3)


@pytest.mark.parametrize("N,D,k,compress,separate_pv", [
    (400, 48, 65, "signed_abs_softmax", True),    # fused column pass, one slab
    (400, 48, 200, "signed_entmax15", False),
    (300, 30, 100, "signed_entmax15", True),      # unaligned rows: the row pass gathers its value rows
    (300, 30, 130, "signed_abs_softmax", False),
    (600, 388, 96, "signed_entmax15", True),      # fused column pass, two slabs
])
def test_propagation_topk_signed_rows_beyond_one_block(dev, N, D, k, compress, separate_pv):
    """The row-normalising compressions on rows of more than 64 edges: the row
    statistics and, in the backward, the row sums of the compress backward
    span several 64-edge blocks (two passes over the row)."""
    _run_topk(dev, _c1_inputs(seed=1300 + k + D, B=2, N=N, D=D, r=16), compress, separate_pv, k, min_checkable=0.3)


def test_propagation_topk_beyond_select_key_limit(dev):
    """Top-k propagation forward and backward over 70,000 nodes (more keys than
    the register select ranks: the scored-rows select, and the edge grouping's
    per-tile key counts at that size).  The N x N oracle is out of reach here,
    so the check is a float64 restatement of the same op on the GPU's
    selection (propagation.py:453-480 over the selected edges, differentiated
    by autograd), plus the selection itself on sampled rows against float64
    scores of every key."""
    import jakal_net_native as jn

    B, N, D, r, k = 1, 70000, 16, 8, 8
    g = torch.Generator().manual_seed(1400)
    val = torch.randn(B, N, D, generator=g)
    state = torch.randn(B, N, generator=g)
    bound = (6.0 / (D + r)) ** 0.5
    U = (torch.rand(r, D, generator=g) * 2 - 1) * bound
    V = (torch.rand(r, D, generator=g) * 2 - 1) * bound
    w = torch.rand(r, generator=g) + 0.5
    w_hat = w / w.norm()
    leaves = [t.to(dev).requires_grad_(True) for t in (val, state, U, V, w_hat)]
    X, ps, Ud, Vd, wd = leaves
    ds, dv, idx, score = jn.propagation_topk_selection("low_rank_bilinear", wd, None, Vd, None, Ud, None, "softsign",
                                                       X, ps, X, k, 128, 128)
    gds = torch.randn(B, N, generator=g).to(dev)
    gdv = torch.randn(B, N, D, generator=g).to(dev)
    torch.autograd.backward([ds, dv], [gds, gdv])

    # selection on sampled rows against float64 scores of every key
    Xd = val.double().to(dev)
    Pt = Xd @ U.double().to(dev).T * w_hat.double().to(dev)
    Ps = Xd @ V.double().to(dev).T
    rows = torch.arange(0, N, N // 64, device=dev)[:64]
    full = (Pt[0, rows] @ Ps[0].T).cpu().numpy()
    frac = check_selection(idx[0, rows].cpu().numpy()[None], score[0, rows].cpu().numpy()[None], full[None], k)
    assert frac > 0.5

    # float64 reference of the op on the selected edges
    ref = [t.double().detach().to(dev).requires_grad_(True) for t in (val, state, U, V, w_hat)]
    xv, sv, u64, v64, w64 = ref
    e = idx.long()[0]                                         # [N, k]
    pt = (xv[0] @ u64.T) * w64                               # [N, r]
    pk = xv[0] @ v64.T                                       # [N, r]
    s = (pt[:, None, :] * pk[e]).sum(-1)                     # [N, k]
    c = s / (1 + s.abs())
    ref_ds = (c * sv[0][e]).sum(-1)
    ref_dv = (c[..., None] * xv[0][e]).sum(1)
    torch.autograd.backward([ref_ds, ref_dv], [gds[0].double(), gdv[0].double()])
    check("delta_state", ds[0], ref_ds)
    check("delta_val", dv[0], ref_dv)
    # absolute tolerance scaled to the tensor: 1e-5 of its largest entry for
    # the per-node gradients, 1e-4 for the weight gradients, which are fp32
    # sums over all 560,000 edges
    for got, want, name, rel in ((X.grad, xv.grad, "grad val", 1e-5), (ps.grad, sv.grad, "grad state", 1e-5),
                                 (Ud.grad, u64.grad, "U", 1e-4), (Vd.grad, v64.grad, "V", 1e-4),
                                 (wd.grad, w64.grad, "w_hat", 1e-4)):
        check(name, got, want, atol=rel * max(1.0, float(want.abs().max())))
