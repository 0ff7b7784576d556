"""GPU parity of the raw edge ops (the reference extension's *_cuda ops that its
Python dispatcher composes into its own autograd functions).

Each op is checked against a float64 evaluation of what it computes: torch
autograd for the elementwise and row backward ops (a library derivative),
the numpy oracle for the selections and the edge sums, and -- for the
composed sequence -- the oracle's transition gradients.  The sequence test
restates the reference's _LowRankTransitionPairwiseTopK
(src/jakal_net/native_backend.py:4408-4600) step by step: these raw ops for
the forward, the route backward and the pair-score backward, and the
reference's own torch steps (_pairwise_routes_from_scores 2232-2237,
_signed_abs_softmax_backward 2190-2196, _pairwise_transition_reduce_backward
3059-3075) in between.  That path scales the pair product, not the bias, by
1/T in its forward (4440-4471) while its backward returns sum(G)/T for the
bias; the module semantics (oracle) divide the whole logit by T, so the
sequence is compared at T = 1, where the two agree, and the op alone at
T != 1.

Tolerances: rtol 1e-5 / atol 1e-6 for the elementwise ops; the sums use the
calibrated check of tests/parity.py (2x the error of an fp32 torch run).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import jakal_oracle as O
from parity import check, torch32_transition

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def jn():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return jakal_net_native


DEV = torch.device("cuda:0")


def _np(t):
    return t.detach().double().cpu().numpy()


def _close(got, want, rtol, atol, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want) - (atol + rtol * np.abs(want))
    assert err.max() <= 0, f"{what}: max excess {err.max():.3e} (max abs diff {np.abs(got - want).max():.3e})"


# ---------------------------------------------------------------------------
# elementwise / row backward ops against torch autograd in float64
# ---------------------------------------------------------------------------
def test_softsign_backward_matches_autograd(jn):
    g = torch.Generator().manual_seed(71)
    s = torch.randn(3, 50, 7, generator=g) * 3.0
    ge = torch.randn(3, 50, 7, generator=g)
    got = jn.softsign_backward_cuda(s.to(DEV), ge.to(DEV))
    s64 = s.double().requires_grad_(True)
    (want,) = torch.autograd.grad(F.softsign(s64), s64, ge.double())
    assert got.dtype == torch.float32 and got.shape == s.shape
    _close(_np(got), want.numpy(), 1e-5, 1e-6, "softsign backward")


@pytest.mark.parametrize("k", [1, 5, 64, 100])
def test_softmax_backward_matches_autograd(jn, k):
    g = torch.Generator().manual_seed(72 + k)
    s = torch.randn(2, 37, k, generator=g) * 2.0
    gr = torch.randn(2, 37, k, generator=g)
    routes = torch.softmax(s, dim=-1)
    got = jn.softmax_backward_cuda(routes.to(DEV), gr.to(DEV))
    s64 = s.double().requires_grad_(True)
    (want,) = torch.autograd.grad(torch.softmax(s64, dim=-1), s64, gr.double())
    _close(_np(got), want.numpy(), 1e-5, 2e-6, f"softmax backward k={k}")


# ---------------------------------------------------------------------------
# edge sums: query_topk_reduce_cuda and its backward
# ---------------------------------------------------------------------------
def _gather_sums64(e, idx, ps, pv):
    """delta_state = sum_e e ps[idx], delta_val = sum_e e pv[idx] in float64 torch."""
    B, Nq, k = e.shape
    D = pv.shape[-1]
    ps_sel = torch.gather(ps[:, None, :].expand(B, Nq, ps.shape[1]), 2, idx)
    pv_sel = torch.gather(pv[:, None].expand(B, Nq, *pv.shape[1:]), 2, idx[..., None].expand(B, Nq, k, D))
    return (e * ps_sel).sum(-1), (e[..., None] * pv_sel).sum(-2)


@pytest.mark.parametrize("B,Nq,Ns,k,D", [(2, 40, 30, 6, 24), (1, 300, 17, 16, 7), (3, 9, 500, 33, 64)])
def test_query_topk_reduce_and_backward(jn, B, Nq, Ns, k, D):
    g = torch.Generator().manual_seed(B * 1000 + Nq + k)
    e = torch.randn(B, Nq, k, generator=g)
    # distinct nodes within a row (top-k index rows), repeated across rows
    idx = torch.stack([torch.stack([torch.randperm(Ns, generator=g)[:k] for _ in range(Nq)]) for _ in range(B)])
    ps = torch.randn(B, Ns, generator=g)
    pv = torch.randn(B, Ns, D, generator=g)
    gds = torch.randn(B, Nq, generator=g)
    gdv = torch.randn(B, Nq, D, generator=g)
    ds, dv = jn.query_topk_reduce_cuda(e.to(DEV), idx.to(DEV), ps.to(DEV), pv.to(DEV))
    leaves = [t.double().requires_grad_(True) for t in (e, ps, pv)]
    ds64, dv64 = _gather_sums64(leaves[0], idx, leaves[1], leaves[2])
    _close(_np(ds), ds64.detach().numpy(), 1e-5, 1e-5, "delta_state")
    _close(_np(dv), dv64.detach().numpy(), 1e-5, 1e-5, "delta_val")
    want = torch.autograd.grad([ds64, dv64], leaves, [gds.double(), gdv.double()])
    got = jn.query_topk_reduce_backward_cuda(e.to(DEV), idx.to(DEV), ps.to(DEV), pv.to(DEV), gds.to(DEV),
                                             gdv.to(DEV))
    for name, a, b in zip(("grad_edges", "grad_projected_state", "grad_projected_val"), got, want):
        assert a.dtype == torch.float32 and a.shape == b.shape
        _close(_np(a), b.numpy(), 1e-5, 1e-5, name)
    # sums over a source's incoming edges walk a fixed order: repeat bit for bit
    again = jn.query_topk_reduce_backward_cuda(e.to(DEV), idx.to(DEV), ps.to(DEV), pv.to(DEV), gds.to(DEV),
                                               gdv.to(DEV))
    for a, b in zip(got, again):
        assert torch.equal(a, b)


def test_query_topk_reduce_backward_refuses_repeated_or_stray_nodes(jn):
    e = torch.randn(1, 4, 3, device=DEV)
    ps, pv = torch.randn(1, 10, device=DEV), torch.randn(1, 10, 5, device=DEV)
    gds, gdv = torch.randn(1, 4, device=DEV), torch.randn(1, 4, 5, device=DEV)
    rep = torch.tensor([[[1, 2, 3], [4, 4, 5], [0, 1, 2], [7, 8, 9]]], device=DEV)
    with pytest.raises(RuntimeError, match="twice"):
        jn.query_topk_reduce_backward_cuda(e, rep, ps, pv, gds, gdv)
    stray = torch.tensor([[[1, 2, 3], [4, 10, 5], [0, 1, 2], [7, 8, 9]]], device=DEV)
    with pytest.raises(RuntimeError, match="must lie in"):
        jn.query_topk_reduce_backward_cuda(e, stray, ps, pv, gds, gdv)
    # repeats are fine where no edge grouping is built (the forward sums)
    ds, _ = jn.query_topk_reduce_cuda(e, rep, ps, pv)
    want = (e * ps[0][rep]).sum(-1)
    assert torch.allclose(ds, want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# fused forwards: select + compress + sums
# ---------------------------------------------------------------------------
def _selection_ok(idx, score, ref, k):
    """Indices in range and distinct, scores the oracle's at those indices and
    descending; the set equals the oracle's on rows with a clear k-th gap."""
    from parity import check_selection

    return check_selection(idx, score, ref, k)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("heads", [1, 3])
def test_low_rank_propagation_topk_forward(jn, kind, heads):
    g = torch.Generator().manual_seed(81 + kind + 10 * heads)
    B, N, D, r, k, bias = 2, 70, 12, 6, 9, 0.25
    shape = (B, heads, N, r) if heads > 1 else (B, N, r)
    wps = torch.randn(*shape, generator=g)
    pt = torch.randn(*shape, generator=g)
    ps = torch.randn(B, N, generator=g)
    pv = torch.randn(B, N, D, generator=g)
    ds, dv = jn.low_rank_propagation_topk_forward_cuda(wps.to(DEV), pt.to(DEV), ps.to(DEV), pv.to(DEV), k, bias,
                                                       kind)
    # float64 scores: targets are rows, sources keys; max over the heads
    s = (pt.double() @ wps.double().transpose(-1, -2).contiguous()) + bias
    if heads > 1:
        s = s.max(dim=1).values
    s = s.numpy()
    mask = O.topk_mask(s, k)
    names = ["softsign", "signed_abs_softmax", "signed_entmax15"]
    want_ds, want_dv, _ = O.propagation_from_scores(s, mask, names[kind], ps.double().numpy(), pv.double().numpy())
    ok = O.checkable_rows(s, k)
    assert ok.mean() > 0.9
    _close(_np(ds)[ok], want_ds[ok], 1e-4, 1e-5, "delta_state")
    _close(_np(dv)[ok], want_dv[ok], 1e-4, 1e-5, "delta_val")


def test_low_rank_pairwise_topk_forward_every_destination(jn):
    """k equal to the destination count keeps every destination in score order."""
    g = torch.Generator().manual_seed(91)
    B, Ns, Nd, r, D = 2, 33, 16, 5, 8
    wps = torch.randn(B, Ns, r, generator=g)
    pt = torch.randn(B, Nd, r, generator=g)
    wst = torch.randn(B, Ns, generator=g)
    wvl = torch.randn(B, Ns, D, generator=g)
    ds, dv, score, idx = jn.low_rank_pairwise_topk_forward_cuda(wps.to(DEV), pt.to(DEV), wst.to(DEV), wvl.to(DEV),
                                                                40, 0.0, 0)
    assert idx.dtype == torch.int64 and idx.shape == (B, Ns, Nd)
    s = (wps.double() @ pt.double().transpose(-1, -2).contiguous()).numpy()
    _selection_ok(idx.cpu().numpy(), score.cpu().numpy(), s, Nd)
    p = torch.softmax(torch.as_tensor(s), dim=-1).numpy()
    _close(_np(ds), np.einsum("bij,bi->bj", p, wst.double().numpy()), 1e-4, 1e-5, "delta_state")
    _close(_np(dv), np.einsum("bij,bid->bjd", p, wvl.double().numpy()), 1e-4, 1e-5, "delta_val")


# ---------------------------------------------------------------------------
# the pair-score backward against autograd of its score formula
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("Dq,Ds,T", [(24, 24, 1.0), (20, 12, 1.7)])
def test_low_rank_pairwise_topk_backward_matches_autograd(jn, Dq, Ds, T):
    g = torch.Generator().manual_seed(101 + Dq + Ds)
    B, Nq, Ns, r, k = 2, 45, 60, 7, 8
    xq = torch.randn(B, Nq, Dq, generator=g)
    xs = torch.randn(B, Ns, Ds, generator=g)
    wt = torch.randn(r, Dq, generator=g) / math.sqrt(Dq)  # projects the query rows
    ws = torch.randn(r, Ds, generator=g) / math.sqrt(Ds)  # projects the source rows
    w = torch.rand(r, generator=g) + 0.5
    idx = torch.stack([torch.stack([torch.randperm(Ns, generator=g)[:k] for _ in range(Nq)]) for _ in range(B)])
    G = torch.randn(B, Nq, k, generator=g)
    pq, psrc = xq @ wt.t(), xs @ ws.t()
    got = jn.low_rank_pairwise_topk_backward_cuda(xq.to(DEV), xs.to(DEV), ws.to(DEV), wt.to(DEV), w.to(DEV),
                                                  pq.to(DEV), psrc.to(DEV), idx.to(DEV), G.to(DEV), T)
    leaves = [t.double().requires_grad_(True) for t in (xq, xs, ws, wt, w)]
    Xq, Xs, Ws, Wt, W = leaves
    b = torch.zeros((), dtype=torch.float64, requires_grad=True)
    Pq, Ps = Xq @ Wt.t(), Xs @ Ws.t()
    full = ((Pq * W) @ Ps.transpose(-1, -2).contiguous() + b) / T  # [B, Nq, Ns]
    score = torch.gather(full, 2, idx)
    want = torch.autograd.grad(score, leaves + [b], G.double())
    names = ("grad_query", "grad_source", "grad_source_weight", "grad_target_weight", "grad_core_weight",
             "grad_bias")
    for name, a, e in zip(names, got, want):
        assert a.dtype == torch.float32 and tuple(a.shape) == tuple(e.shape), name
        _close(_np(a), e.numpy(), 1e-4, 1e-5, name)
    again = jn.low_rank_pairwise_topk_backward_cuda(xq.to(DEV), xs.to(DEV), ws.to(DEV), wt.to(DEV), w.to(DEV),
                                                    pq.to(DEV), psrc.to(DEV), idx.to(DEV), G.to(DEV), T)
    for a, c in zip(got, again):
        assert torch.equal(a, c)


# ---------------------------------------------------------------------------
# the reference's decomposed transition autograd, restated over these ops
# ---------------------------------------------------------------------------
def _signed_abs_softmax_from_scores(scores):
    clean = torch.nan_to_num(scores)
    return torch.sign(clean) * torch.softmax(clean.abs(), dim=-1)


def _signed_abs_softmax_backward(scores, grad_routes):
    clean = torch.nan_to_num(scores)
    signs = torch.sign(clean)
    probs = torch.softmax(clean.abs(), dim=-1)
    dot = (grad_routes * signs * probs).sum(dim=-1, keepdim=True)
    return signs * probs * (signs * grad_routes - dot)


def _gather_rows(x, idx):
    """x [B, Nd(, D)] rows at idx [B, Ns, k] -> [B, Ns, k(, D)]."""
    B, Ns, k = idx.shape
    flat = idx.reshape(B, Ns * k)
    if x.dim() == 2:
        return torch.gather(x, 1, flat).reshape(B, Ns, k)
    return torch.gather(x, 1, flat[..., None].expand(B, Ns * k, x.shape[-1])).reshape(B, Ns, k, x.shape[-1])


class _RestatedPairwiseTopK(torch.autograd.Function):
    """The reference's _LowRankTransitionPairwiseTopK (native_backend.py:
    4408-4600) with this module as `_native_module()`; flat [B, N, ...] inputs."""

    @staticmethod
    def forward(ctx, jn, sender, src, dst, ps, pv, Ws, Wt, w, bias, T, topk, kind):
        Ps = torch.matmul(src, Ws.t()).contiguous()
        wps = Ps * w.view(1, 1, -1)
        if T != 1.0:
            wps = wps / float(T)
        Pt = torch.matmul(dst, Wt.t()).contiguous()
        wstate = (sender * ps).contiguous()
        wval = (sender.unsqueeze(-1) * pv).contiguous()
        ds, dv, scores, idx = jn.low_rank_pairwise_topk_forward_cuda(wps, Pt, wstate, wval, min(topk, dst.shape[1]),
                                                                     float(bias.item()), kind)
        ctx.jn, ctx.T, ctx.kind = jn, T, kind
        ctx.save_for_backward(sender, src, dst, ps, pv, Ws, Wt, w, scores, idx)
        return ds, dv

    @staticmethod
    def backward(ctx, gds, gdv):
        jn = ctx.jn
        sender, src, dst, ps, pv, Ws, Wt, w, scores, idx = ctx.saved_tensors
        routes = (_signed_abs_softmax_from_scores(scores) if ctx.kind == 1 else torch.softmax(scores, dim=-1))
        wstate = sender * ps
        wval = sender.unsqueeze(-1) * pv
        # _pairwise_transition_reduce_backward
        sel_s = _gather_rows(gds.contiguous(), idx)
        sel_v = _gather_rows(gdv.contiguous(), idx)
        grad_routes = sel_s * wstate.unsqueeze(-1) + (sel_v * wval.unsqueeze(-2)).sum(dim=-1)
        g_wstate = (routes * sel_s).sum(dim=-1)
        g_wval = (routes.unsqueeze(-1) * sel_v).sum(dim=-2)
        if ctx.kind == 1:
            grad_scores = _signed_abs_softmax_backward(scores, grad_routes)
        else:
            grad_scores = jn.softmax_backward_cuda(routes.contiguous(), grad_routes.contiguous())
        Pt = torch.matmul(dst, Wt.t()).contiguous()
        Ps = torch.matmul(src, Ws.t()).contiguous()
        g_src, g_dst, g_Wt, g_Ws, g_w, g_b = jn.low_rank_pairwise_topk_backward_cuda(
            src, dst, Wt.contiguous(), Ws.contiguous(), w.contiguous(), Ps, Pt, idx, grad_scores.contiguous(),
            ctx.T)
        g_sender = g_wstate * ps + (g_wval * pv).sum(dim=-1)
        return (None, g_sender, g_src, g_dst, g_wstate * sender, g_wval * sender.unsqueeze(-1), g_Ws, g_Wt, g_w,
                g_b, None, None, None)


@pytest.mark.parametrize("kind", [0, 1])
@pytest.mark.parametrize("Dsrc,Ddst", [(24, 24), (32, 16)])
def test_reference_transition_sequence_matches_oracle(jn, kind, Dsrc, Ddst):
    """_LowRankTransitionPairwiseTopK restated over these ops (softmax and
    signed |l| softmax routes) against the oracle's transition gradients."""
    g = torch.Generator().manual_seed(111 + kind + Dsrc)
    B, Ns, Nd, r, topk, T = 2, 64, 40, 8, 6, 1.0
    src = torch.randn(B, Ns, Dsrc, generator=g)
    dst = torch.randn(B, Nd, Ddst, generator=g)
    state = torch.randn(B, Ns, generator=g)
    pv = torch.randn(B, Ns, Ddst, generator=g)
    rho = F.softplus(state)
    Ws = torch.empty(r, Dsrc).uniform_(-math.sqrt(6.0 / (Dsrc + r)), math.sqrt(6.0 / (Dsrc + r)), generator=g)
    Wt = torch.empty(r, Ddst).uniform_(-math.sqrt(6.0 / (Ddst + r)), math.sqrt(6.0 / (Ddst + r)), generator=g)
    w = torch.rand(r, generator=g) + 0.5
    b = torch.tensor(0.2)
    gds = torch.randn(B, Nd, generator=g)
    gdv = torch.randn(B, Nd, Ddst, generator=g)

    leaves = [t.to(DEV).requires_grad_(True) for t in (rho, src, dst, state, pv, Ws, Wt, w, b)]
    rho_d, src_d, dst_d, ps_d, pv_d, Ws_d, Wt_d, w_d, b_d = leaves
    ds, dv = _RestatedPairwiseTopK.apply(jn, rho_d, src_d, dst_d, ps_d, pv_d, Ws_d, Wt_d, w_d, b_d, T, topk, kind)
    torch.autograd.backward([ds, dv], [gds.to(DEV), gdv.to(DEV)])

    # the selection the forward made (indices of the saved scores)
    logits = O.lowrank_route_logits(_np(src), _np(dst), _np(Ws), _np(Wt), _np(w), float(b), T)
    wps = (src @ Ws.t()) * w
    _, _, _, idx = jn.low_rank_pairwise_topk_forward_cuda(wps.to(DEV), (dst @ Wt.t()).to(DEV),
                                                          (rho * state).to(DEV),
                                                          (rho.unsqueeze(-1) * pv).to(DEV), topk, float(b), kind)
    got_idx = idx.cpu().numpy()
    ok = O.checkable_rows(logits, topk)
    ref_idx = np.sort(O.topk_indices(logits, topk), axis=-1)
    assert (np.sort(got_idx, axis=-1) == ref_idx).all(-1)[ok].all()
    mask = O.mask_from_indices(got_idx, Nd)
    name = ["softmax", "signed_abs_softmax"][kind]
    gr = O.transition_backward(_np(src), _np(dst), _np(rho), _np(state), _np(pv), _np(Ws), _np(Wt), _np(w), float(b),
                               _np(gds), _np(gdv), topk=topk, temperature=T, mask=mask, kind=name)
    t32 = torch32_transition(DEV, src, dst, rho, state, pv, Ws, Wt, w, float(b), T, mask, name, gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    for t, key in ((rho_d, "sender"), (src_d, "src_val"), (dst_d, "dst_val"), (ps_d, "ps"), (pv_d, "pv"),
                   (Ws_d, "Ws"), (Wt_d, "Wt"), (w_d, "w"), (b_d, "b")):
        check(f"grad {key}", t.grad, gr[key], t32[key])
