"""GPU parity of the top-k hot path (HIP library) against the numpy oracle.

Index parity is exact on rows whose k-th/(k+1)-th score gap exceeds 1e-5;
values and gradients are compared to the oracle evaluated on the selection the
GPU made (identical to the oracle's on every checkable row), fp32 tolerance
rtol 1e-4 / atol 1e-5 as stated for the hot path.
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
    if want.size == 0:
        return
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert err.max() <= 0, f"{what}: max excess {err.max():.3e} (max abs diff {np.abs(got - want).max():.3e})"


def _check_select(idx, score, ref_scores, k):
    """idx/score from the GPU vs dense oracle scores [B, Nq, Nk]."""
    B, Nq, Nk = ref_scores.shape
    assert idx.shape == (B, Nq, k)
    assert (idx >= 0).all() and (idx < Nk).all()
    # unique per row
    srt = np.sort(idx, axis=-1)
    assert (np.diff(srt, axis=-1) > 0).all()
    # reported scores are the scores of the reported indices
    picked = np.take_along_axis(ref_scores, idx, axis=-1)
    _close(score, picked, rtol=1e-5, atol=1e-5, what="selected scores")
    # descending order
    assert (np.diff(score, axis=-1) <= 1e-6).all()
    # exact index-set parity on checkable rows
    ok = O.checkable_rows(ref_scores, k)
    ref_idx = np.sort(O.topk_indices(ref_scores, k), axis=-1)
    same = (srt == ref_idx).all(-1)
    assert same[ok].all(), f"{(~same[ok]).sum()} checkable rows differ"
    # on ambiguous rows the k-th best score still agrees
    kth = np.sort(ref_scores, axis=-1)[..., ::-1][..., k - 1]
    assert np.abs(score[..., -1] - kth).max() <= 1e-5
    return ok.mean()


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
        _check_select(idx.cpu().numpy(), score.cpu().numpy(), ref, k)


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
    _check_select(idx.cpu().numpy(), score.cpu().numpy(), ref, k)
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
    _run_topk(dev, _c1_inputs(seed=1100 + k, B=1, N=N, D=D, r=24), compress, True, k, min_checkable=0.3,
              normwise=True)


def _run_topk(dev, inputs, compress, separate_pv, k, min_checkable, normwise=False):
    """normwise: the absolute tolerance of the outputs and node gradients
    scales with the tensor's largest entry (at larger D, r and k they are long
    sums of terms far larger than the entries that cancel to near 0)."""
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
    frac = _check_select(idx.cpu().numpy(), score.cpu().numpy(), scores, k)
    assert frac > min_checkable  # deeper cuts sit in denser parts of the score distribution
    mask = O.mask_from_indices(idx.cpu().numpy(), N)
    ref = O.propagation_forward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b),
                                mode="topk", topk=k, kind=compress, mask=mask)

    def node_atol(want):
        return ATOL * max(1.0, float(np.abs(want).max())) if normwise else ATOL

    _close(_np(ds), ref["delta_state"], atol=node_atol(ref["delta_state"]), what="delta_state")
    _close(_np(dv), ref["delta_val"], atol=node_atol(ref["delta_val"]), what="delta_val")

    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), float(b), _np(gds),
                                _np(gdv), mode="topk", topk=k, kind=compress, mask=mask)
    g_val = gr["val"] + (0.0 if separate_pv else gr["pv"])
    _close(_np(X.grad), g_val, atol=node_atol(g_val), what="grad layer_val")
    _close(_np(ps.grad), gr["ps"], atol=node_atol(gr["ps"]), what="grad projected_state")
    if separate_pv:
        _close(_np(pv.grad), gr["pv"], atol=node_atol(gr["pv"]), what="grad projected_val")
    # Parameter gradients are sums over all B*N*k edges.  fp32 error of such a
    # sum grows with the size of its terms, not of the result (which can
    # cancel to ~0), so atol scales with max|want| and with the root-mean L1
    # size of the per-edge score gradients sum|g_s| / sqrt(#edges).
    gs = gr["g_scores"][mask]
    scale = max(1.0, float(np.abs(gs).sum() / math.sqrt(gs.size)))
    for got, want, what in ((Ud.grad, gr["U"], "grad target_proj"), (Vd.grad, gr["V"], "grad source_proj"),
                            (wd.grad, gr["w_hat"], "grad w_hat"), (bd.grad, gr["b"], "grad bias")):
        _close(_np(got), want, atol=ATOL * max(scale, float(np.abs(want).max())), what=what)


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


def test_c4_shape_forward_sampled_rows(dev):
    """Full C4 shape (B=16, N=4096, D=512, r=64, k=32): index parity on sampled
    rows against float64 scores, and delta rows recomputed from the selection."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(1004)
    B, N, D, r, k = 16, 4096, 512, 64, 32
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    val = val / val.norm(dim=-1, keepdim=True)
    lin_t = torch.nn.Linear(D, r, bias=False)
    lin_s = torch.nn.Linear(D, r, bias=False)
    U, V = lin_t.weight.detach(), lin_s.weight.detach()
    w_hat = torch.ones(r) / math.sqrt(r)
    Xd = val.to(dev)
    ds, dv, idx, score = jn.propagation_topk_selection("low_rank_bilinear", w_hat.to(dev), None, V.to(dev), None,
                                                       U.to(dev), None, "softsign", Xd, state.to(dev), Xd, k,
                                                       128, 128)
    pt = (val.double() @ U.double().T)
    psh = (val.double() @ V.double().T) * w_hat.double()
    rows = torch.randint(0, N, (8,), generator=g)
    checked = 0
    for bb in (0, 7, 15):
        s = (pt[bb, rows] @ psh[bb].T).numpy()[None]  # [1, 8, N]
        ii = idx[bb, rows].cpu().numpy()[None]
        ok = O.checkable_rows(s, k)
        ref_idx = np.sort(O.topk_indices(s, k), -1)
        assert (np.sort(ii, -1) == ref_idx).all(-1)[ok].all()
        checked += ok.sum()
        # delta rows from the GPU selection
        e = torch.from_numpy(np.take_along_axis(s, ii.astype(np.int64), -1)[0])
        e = e / (1 + e.abs())
        sel = torch.from_numpy(ii[0].astype(np.int64))
        want_v = (e[:, :, None] * val.double()[bb][sel]).sum(1)
        want_s = (e * state.double()[bb][sel]).sum(1)
        _close(_np(dv[bb, rows]), want_v.numpy(), what="C4 delta_val rows")
        _close(_np(ds[bb, rows]), want_s.numpy(), what="C4 delta_state rows")
    print(f"C4 sampled rows with unambiguous top-k: {checked}/24")


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
