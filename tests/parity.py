"""Shared checks of the GPU parity tests (imported by tests/test_gpu_*.py).

``check`` compares a HIP result with the float64 oracle.  It passes when the
hot path's literal fp32 tolerance holds elementwise (rtol 1e-4 / atol 1e-5).
Long fp32 sums whose terms cancel (destination sums, gradients over every
edge, D- and N-long dot products) can miss that literal bound in any fp32
implementation; for those the check is calibrated instead: the HIP error,
max |hip - f64| over the tensor, must be at most twice the error of a plain
fp32 PyTorch evaluation of the same op on the same inputs and the same
selection (``torch32_propagation`` / ``torch32_transition``), measured the
same way.  Every check prints both errors and the largest excess under the
literal tolerance, so the logs show how far each tensor is from it.

The fp32 evaluations are the dense masked formulation of the reference
backend (src/jakal_net/propagation.py:453-480, transition.py:431-452) in
torch fp32 on the GPU, differentiated by autograd, one chunk of batch
elements at a time.
"""

from __future__ import annotations

import numpy as np
import torch
from torch.nn import functional as F

RTOL, ATOL = 1e-4, 1e-5
FACTOR = 2.0
BF16_RTOL = 2e-2


def np64(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        return t.detach().double().cpu().numpy()
    return np.asarray(t, dtype=np.float64)


def check(what, got, want, ref32=None, rtol=RTOL, atol=ATOL, factor=FACTOR) -> None:
    """Literal rtol/atol elementwise, else HIP error <= factor x the fp32 torch error."""
    got, want = np64(got), np64(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if want.size == 0:
        return
    err = np.abs(got - want)
    excess = float((err - (atol + rtol * np.abs(want))).max())
    line = f"{what}: max|hip-f64| {err.max():.3e}"
    e32 = None
    if ref32 is not None:
        e32 = float(np.abs(np64(ref32) - want).max())
        line += f", max|torch32-f64| {e32:.3e}"
    line += f", excess under rtol {rtol:g}/atol {atol:g}: {excess:.3e} (max|f64| {np.abs(want).max():.3e})"
    print(line, flush=True)
    if excess <= 0:
        return
    assert e32 is not None, line + " -- literal tolerance missed and no fp32 reference given"
    assert err.max() <= factor * e32, line + f" -- HIP error above {factor:g}x the fp32 reference error"


def _bool_mask(mask, dev, b0, b1):
    m = torch.from_numpy(np.array(mask[b0:b1], dtype=bool, copy=True)).to(dev)
    return m


def _compress32(s, m, kind):
    """Edge compression on the masked entries (propagation.py:67-88); masked entries 0."""
    if kind == "softsign":
        return torch.where(m, F.softsign(s), torch.zeros_like(s))
    if kind == "signed_abs_softmax":
        p = torch.softmax(s.abs().masked_fill(~m, -torch.inf), dim=-1)
        return torch.where(m, torch.sign(s) * p, torch.zeros_like(s))
    if kind == "signed_entmax15":
        from jakal_net.compress import signed_entmax15

        return signed_entmax15(s, mask=m)
    raise ValueError(kind)


def _route32(l, m, kind):
    """Route weights over each source row's masked destinations (transition.py:187-194, 439-446)."""
    if kind == "softmax":
        if m is None:
            return torch.softmax(l, dim=-1)
        p = torch.softmax(l.masked_fill(~m, torch.finfo(l.dtype).min), dim=-1)
        return torch.where(m, p, torch.zeros_like(p))
    if m is None:
        m = torch.ones_like(l, dtype=torch.bool)
    return _compress32(l, m, kind)


def _bf16_st(t):
    """t rounded to bf16 in the forward, the identity in the backward (autocast's casts)."""
    return t + (t.bfloat16().float() - t).detach()


class _Bf16Grad(torch.autograd.Function):
    """The identity, whose incoming gradient is rounded to bf16: the bf16
    grad_output that autocast's nn.Linear backward multiplies."""

    @staticmethod
    def forward(ctx, t):
        return t.clone()

    @staticmethod
    def backward(ctx, g):
        return g.bfloat16().float()


def _linear32(x, W, bf16_linear):
    """x . W^T; bf16_linear: as autocast's nn.Linear on bf16 x -- the weight
    rounded to bf16 (straight-through), fp32 accumulation, the gradient into
    the product rounded to bf16 before it reaches x and W (the library's bf16
    projection GEMMs)."""
    if not bf16_linear:
        return x @ W.T
    return _Bf16Grad.apply(x @ _bf16_st(W).T)


def torch32_propagation(dev, val, ps, pv, U, V, w_hat, b, mask, kind, gds, gdv, chunk=4,
                        bf16_operands=False, bf16_linear=None, bf16_edges=False) -> dict:
    """fp32 torch forward + autograd backward of low-rank propagation on a given mask.

    val [B,N,D], ps [B,N], pv [B,N,Dv] or None (pv is val itself), U/V [r,D],
    w_hat [r] (the normalised core weight), b float or None -- or, for
    max-aggregated heads, U/V [H,r,D], w_hat [H,r], b [H] -- mask [B,N,N]
    bool (numpy), gds [B,N] / gdv [B,N,Dv] the upstream gradients.  Returns
    the oracle's keys: delta_state, delta_val, val (whole gradient of val),
    ps, pv, U, V, w_hat, b.  bf16_operands: the score is
    bf16(P_t * w_hat) . bf16(P_s), the operands of the bf16 top-k select.
    bf16_linear (default: bf16_operands): the projections as the bf16 entry
    points compute them (_linear32).  bf16_edges: the edge matrix rounded to
    bf16 (straight-through) where it multiplies the values, as the bf16 dense
    entry points' E . pv and E^T . gdv take it."""
    if bf16_linear is None:
        bf16_linear = bf16_operands
    f32 = dict(device=dev, dtype=torch.float32)
    Ud = torch.as_tensor(U).to(**f32).requires_grad_(True)
    Vd = torch.as_tensor(V).to(**f32).requires_grad_(True)
    wd = torch.as_tensor(w_hat).to(**f32).requires_grad_(True)
    bd = None if b is None else torch.as_tensor(np.asarray(b, dtype=np.float64)).to(**f32).requires_grad_(True)
    params = [Ud, Vd, wd] + ([bd] if bd is not None else [])
    out = {k: [] for k in ("delta_state", "delta_val", "val", "ps", "pv")}
    acc = [torch.zeros_like(p) for p in params]
    B = val.shape[0]
    for b0 in range(0, B, chunk):
        b1 = min(B, b0 + chunk)
        x = torch.as_tensor(val[b0:b1]).to(**f32).requires_grad_(True)
        p_s = torch.as_tensor(ps[b0:b1]).to(**f32).requires_grad_(True)
        p_v = x if pv is None else torch.as_tensor(pv[b0:b1]).to(**f32).requires_grad_(True)
        m = _bool_mask(mask, dev, b0, b1)
        if Ud.dim() == 3:  # stacked heads [H, r, D]: the max over the heads' scores
            key = ((x[:, None] @ Vd.transpose(-1, -2)) * wd[:, None, :]).transpose(-1, -2).contiguous()
            s = (x[:, None] @ Ud.transpose(-1, -2)) @ key
            if bd is not None:
                s = s + bd[:, None, None]
            s = s.max(dim=1).values
        else:
            pt, pk = _linear32(x, Ud, bf16_linear), _linear32(x, Vd, bf16_linear)
            if bf16_operands:
                s = _bf16_st(pt * wd) @ _bf16_st(pk).transpose(-1, -2).contiguous()
            else:
                s = pt @ (pk * wd).transpose(-1, -2).contiguous()
            if bd is not None:
                s = s + bd
        e = _compress32(s, m, kind)
        ds = (e * p_s[:, None, :]).sum(-1)
        dv = (_bf16_st(e) if bf16_edges else e) @ p_v
        loss = (ds * torch.as_tensor(gds[b0:b1]).to(**f32)).sum() + (dv * torch.as_tensor(gdv[b0:b1]).to(**f32)).sum()
        leaves = [x, p_s] + ([p_v] if pv is not None else []) + params
        grads = torch.autograd.grad(loss, leaves)
        out["delta_state"].append(ds.detach().cpu())
        out["delta_val"].append(dv.detach().cpu())
        out["val"].append(grads[0].cpu())
        out["ps"].append(grads[1].cpu())
        if pv is not None:
            out["pv"].append(grads[2].cpu())
        for a, g in zip(acc, grads[-len(params):]):
            a += g
    res = {k: torch.cat(v).double().numpy() for k, v in out.items() if v}
    names = ["U", "V", "w_hat"] + (["b"] if bd is not None else [])
    for n, a in zip(names, acc):
        res[n] = a.double().cpu().numpy()
    return res


def torch32_transition(dev, src, dst, rho, ps, pv, Ws, Wt, w, b, temperature, mask, kind, gds, gdv,
                       chunk=4, bf16_operands=False, bf16_linear=None, bf16_routes=False) -> dict:
    """fp32 torch forward + autograd backward of low-rank routing on a given mask.

    src [B,Ns,Ds], dst [B,Nd,Dd], rho [B,Ns] (sender strength, a leaf), ps
    [B,Ns], pv [B,Ns,Dv], Ws [r,Ds], Wt [r,Dd], w [r] (raw), b float or None
    (stacked heads: [H,r,Ds], [H,r,Dd], [H,r], [H]), mask [B,Ns,Nd] bool
    (numpy) or None (every destination).  Returns the
    oracle's keys: delta_state, delta_val, sender, src_val, dst_val, ps, pv,
    Ws, Wt, w, b.  bf16_operands: the logit is bf16(P_s * w) . bf16(P_t),
    the operands of the bf16 top-k select; bf16_linear (default:
    bf16_operands): the projections as the bf16 entry points compute them;
    bf16_routes: the sender-weighted routes rounded to bf16 (straight-through)
    where they multiply the values, as the bf16 dense transitions take them."""
    if bf16_linear is None:
        bf16_linear = bf16_operands
    f32 = dict(device=dev, dtype=torch.float32)
    Wsd = torch.as_tensor(Ws).to(**f32).requires_grad_(True)
    Wtd = torch.as_tensor(Wt).to(**f32).requires_grad_(True)
    wd = torch.as_tensor(w).to(**f32).requires_grad_(True)
    bd = None if b is None else torch.as_tensor(np.asarray(b, dtype=np.float64)).to(**f32).requires_grad_(True)
    params = [Wsd, Wtd, wd] + ([bd] if bd is not None else [])
    keys = ("delta_state", "delta_val", "sender", "src_val", "dst_val", "ps", "pv")
    out = {k: [] for k in keys}
    acc = [torch.zeros_like(p) for p in params]
    B = src.shape[0]
    for b0 in range(0, B, chunk):
        b1 = min(B, b0 + chunk)
        leaves = [torch.as_tensor(t[b0:b1]).to(**f32).requires_grad_(True) for t in (rho, src, dst, ps, pv)]
        r_, s_, d_, p_s, p_v = leaves
        m = None if mask is None else _bool_mask(mask, dev, b0, b1)
        if Wsd.dim() == 3:  # stacked heads [H, r, D]: the max over the heads' logits
            tgt = (d_[:, None] @ Wtd.transpose(-1, -2)).transpose(-1, -2).contiguous()
            l = ((s_[:, None] @ Wsd.transpose(-1, -2)) * wd[:, None, :]) @ tgt
            if bd is not None:
                l = l + bd[:, None, None]
            l = l.max(dim=1).values
        else:
            p_src, p_dst = _linear32(s_, Wsd, bf16_linear), _linear32(d_, Wtd, bf16_linear)
            if bf16_operands:
                l = _bf16_st(p_src * wd) @ _bf16_st(p_dst).transpose(-1, -2).contiguous()
            else:
                l = (p_src * wd) @ p_dst.transpose(-1, -2).contiguous()
            if bd is not None:
                l = l + bd
        l = l / float(temperature)
        wr = _route32(l, m, kind) * r_[..., :, None]
        ds = (wr * p_s[..., :, None]).sum(-2)
        dv = (_bf16_st(wr) if bf16_routes else wr).transpose(-1, -2).contiguous() @ p_v
        loss = (ds * torch.as_tensor(gds[b0:b1]).to(**f32)).sum() + (dv * torch.as_tensor(gdv[b0:b1]).to(**f32)).sum()
        grads = torch.autograd.grad(loss, leaves + params)
        out["delta_state"].append(ds.detach().cpu())
        out["delta_val"].append(dv.detach().cpu())
        for k, g in zip(keys[2:], grads[:5]):
            out[k].append(g.cpu())
        for a, g in zip(acc, grads[5:]):
            a += g
    res = {k: torch.cat(v).double().numpy() for k, v in out.items()}
    names = ["Ws", "Wt", "w"] + (["b"] if bd is not None else [])
    for n, a in zip(names, acc):
        res[n] = a.double().cpu().numpy()
    return res


def check_selection(idx, score, ref_scores, k, gap=1e-5, score_tol=0.0) -> float:
    """A GPU top-k selection [B, Nq, k] against float64 scores [B, Nq, Nk].

    Indices in range and distinct per row; the reported scores are the
    oracle scores of the reported indices (1e-5, plus ``score_tol``, a scalar
    or one value per row) and sorted descending; the index set equals the
    oracle's on every row whose k-th/(k+1)-th gap exceeds ``gap`` (scalar or
    per row); on the other rows the k-th reported score equals the oracle's
    k-th best within the same tolerance.  Returns the fraction of rows with an
    unambiguous set."""
    idx = np.asarray(idx)
    score = np.asarray(score, np.float64)
    B, Nq, Nk = ref_scores.shape
    assert idx.shape == (B, Nq, k)
    assert (idx >= 0).all() and (idx < Nk).all()
    srt = np.sort(idx, axis=-1)
    assert (np.diff(srt, axis=-1) > 0).all(), "repeated index in a row"
    stol = np.broadcast_to(np.asarray(score_tol, np.float64), (B, Nq))
    picked = np.take_along_axis(ref_scores, idx.astype(np.int64), axis=-1)
    err = np.abs(score - picked) - (1e-5 + 1e-5 * np.abs(picked) + stol[..., None])
    assert err.max() <= 0, f"selected scores: max excess {err.max():.3e}"
    assert (np.diff(score, axis=-1) <= 1e-6).all(), "scores not sorted descending"
    if k < Nk:
        # the k+1 best scores of each row (a partition, not a full sort: rows of 4096 keys)
        part = np.partition(-ref_scores, k, axis=-1)[..., :k + 1]
        top = -np.sort(part, axis=-1)
        kth, nxt = top[..., k - 1], top[..., k]
        ok = (kth - nxt) > gap
        ref_idx = np.sort(np.argpartition(-ref_scores, k - 1, axis=-1)[..., :k], axis=-1)
    else:
        kth = ref_scores.min(axis=-1)
        ok = np.ones((B, Nq), dtype=bool)
        ref_idx = np.broadcast_to(np.arange(Nk), (B, Nq, Nk))
    same = (srt == ref_idx).all(-1)
    assert same[ok].all(), f"{(~same[ok]).sum()} unambiguous rows select a different set"
    assert (np.abs(score[..., -1] - kth) <= 1e-5 + stol).all()
    return float(ok.mean())


def bf16_round(x) -> np.ndarray:
    """x rounded to fp32 and then to bf16 (nearest even), as float64."""
    t = torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32)))
    return t.bfloat16().double().numpy()


def bf16_linear64(x, W):
    """x . bf16(W)^T in float64: the projection of a bf16 layer, whose GEMM
    rounds the fp32 weight to bf16 (as autocast's nn.Linear) and accumulates
    exact products."""
    return np.asarray(x, np.float64) @ bf16_round(W).T


def bf16_select_scores(q, key, scale, bias=None, temperature=1.0):
    """What the bf16 top-k select ranks, in float64: bf16(q * scale) . bf16(key),
    plus bias, over T, with q [.., Nq, r] and key [.., Nk, r] the score
    projections (given here in float64 and rounded through fp32, as the GEMM
    stores them).  The GPU rounds its own fp32 projections, whose last bit
    can differ from these; that moves a bf16 rounding by one bf16 ulp in
    roughly one element in 10^5, so a score sees at most one such operand on
    each side.  Returns (scores, tol): tol [.., Nq] bounds, per query row, two
    one-ulp operand moves (2^-8 relative each) plus the fp32 accumulation of
    the r products."""
    q = np.asarray(q, np.float64) * np.asarray(scale, np.float64)
    key = np.asarray(key, np.float64)
    qb, kb = bf16_round(q), bf16_round(key)
    s = qb @ np.swapaxes(kb, -1, -2)
    if bias is not None:
        s = s + float(bias)
    s = s / float(temperature)
    r = q.shape[-1]
    kmax = np.abs(kb).max(axis=-2, keepdims=True)                   # [.., 1, r] largest key element per rank
    one_move = 2.0 ** -8 * (np.abs(qb) * kmax).max(axis=-1)          # [.., Nq]
    accumulate = r * 2.0 ** -24 * (np.abs(qb) @ np.swapaxes(np.abs(kb), -1, -2)).max(axis=-1)
    tol = (2.0 * one_move + accumulate) / float(temperature)
    return s, tol


def check_bf16_calibrated(what, got, want, ref_bf16, stored_bf16=None) -> None:
    """bf16 results: elementwise rtol 2e-2 (atol 2e-4 max|f64|), else the HIP
    error at most twice that of the fp32 torch evaluation with bf16 score
    operands (torch32_* with bf16_operands=True), its result rounded to bf16
    where the HIP tensor is stored in bf16 -- the error the bf16 arithmetic and
    storage themselves cause where a sum or a softmax gradient cancels."""
    want64 = np64(want)
    if stored_bf16 is None:
        stored_bf16 = isinstance(got, torch.Tensor) and got.dtype == torch.bfloat16
    if stored_bf16:
        ref_bf16 = bf16_round(ref_bf16)
    check(what + " (bf16)", got, want64, ref_bf16, rtol=BF16_RTOL,
          atol=BF16_RTOL * 1e-2 * max(1.0, float(np.abs(want64).max())))
