"""CPU oracle (numpy) for the Jakal-Net native hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker: it is imported by
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``, never by the product (``jakal-net_amd/``).

It restates the reference's ``implementation="reference"`` backend -- the
dense masked formulation -- in numpy, float64 by default, together with a
hand-derived backward.  Every function cites the reference lines it follows.

Pinning (see tests/test_oracle.py):
  * the reference's known-answer tests: tests/test_kernel_common.py:124-140,175-184;
    tests/test_jakal_net.py:438-458, 810-831, 833-862;
  * closed forms (low-rank score = P_t diag(w_hat) P_s^T + b, softsign, window mask);
  * brute-force top-k by full sort on tiny inputs;
  * every backward against float64 central finite differences of the forward;
  * multi-head max aggregation: one head reduces to the single-head form, the
    score is the largest head's and its gradient reaches only that head.
Tie order: the oracle breaks exact score ties toward the lower index (stable
sort).  CPU torch.topk does not (it is implementation-defined), so exact ties
at the k-th place are excluded from index parity by the 1e-5 gap rule.
"""

from __future__ import annotations

import contextlib

import numpy as np

# Arithmetic type of the oracle.  float64 for parity checks; the benchmark's
# CPU baseline switches to float32 (the reference backend's own precision).
F64 = np.float64


@contextlib.contextmanager
def compute_dtype(dtype):
    """Temporarily run the oracle in ``dtype`` (e.g. np.float32)."""
    global F64
    saved = F64
    F64 = dtype
    try:
        yield
    finally:
        F64 = saved


# ---------------------------------------------------------------------------
# score functions
# ---------------------------------------------------------------------------
def normalized_weight(w):
    """w / max(||w||_2, 1e-6)  (modules.py:85-87)."""
    w = np.asarray(w, dtype=F64)
    return w / max(float(np.sqrt(np.sum(w * w))), 1e-6)


def lowrank_projections(val, U, V):
    """P_t = val U^T, P_s = val V^T  (modules.py:95-97; U = target_proj, V = source_proj)."""
    val = np.asarray(val, dtype=F64)
    return val @ np.asarray(U, F64).T, val @ np.asarray(V, F64).T


def lowrank_pairwise_scores(target_val, source_val, U, V, w, b):
    """s[..., i, j] = (U x_i) . (w_hat * (V x_j)) + b  (modules.py:95-100)."""
    pt = np.asarray(target_val, F64) @ np.asarray(U, F64).T
    ps = (np.asarray(source_val, F64) @ np.asarray(V, F64).T) * normalized_weight(w)
    s = pt @ np.swapaxes(ps, -1, -2)
    return s + (0.0 if b is None else float(b))


def lowrank_route_logits(src_val, dst_val, Ws, Wt, w, b, temperature=1.0):
    """l[..., j, k] = ((w * (Ws s_j)) . (Wt d_k) + b) / T  (modules.py:435-441,
    scripts/progressive_b_example.py:67-68)."""
    ps = (np.asarray(src_val, F64) @ np.asarray(Ws, F64).T) * np.asarray(w, F64)
    pt = np.asarray(dst_val, F64) @ np.asarray(Wt, F64).T
    l = ps @ np.swapaxes(pt, -1, -2)
    if b is not None:
        l = l + float(b)
    return l / float(temperature)


def multihead_pairwise_scores(target_val, source_val, U, V, w, b):
    """Max-aggregated multi-head low-rank scores: s = max_h s_h with s_h the
    low-rank score of head h (its own projections, normalised core weight and
    bias).  MultiHeadPairwise(aggregate="max") (modules.py:259-301, :284-291)
    over LowRankBilinearPairwise heads; the native composite stacks the heads'
    parameters and takes the max over the head axis
    (jakal_net_native.cpp:724-752, kernel_common.py:152-178).

    U, V [H, r, D]; w [H, r] (raw, normalised per head); b [H] or None.
    Returns (scores, head, per_head): head is the first head attaining the max."""
    H = np.shape(U)[0]
    per = np.stack([lowrank_pairwise_scores(target_val, source_val, U[h], V[h], w[h], None if b is None else b[h])
                    for h in range(H)])
    head = np.argmax(per, axis=0)
    return np.take_along_axis(per, head[None], 0)[0], head, per


def multihead_route_logits(src_val, dst_val, Ws, Wt, w, b, temperature=1.0):
    """Max-aggregated multi-head low-rank route logits, max_h l_h
    (MultiHeadRoute(aggregate="max"), modules.py:470-529, :497-514;
    jakal_net_native.cpp:889-917).  Ws [H, r, Ds], Wt [H, r, Dd], w [H, r]
    (raw), b [H] or None; the heads share one temperature.  Returns
    (logits, head, per_head) as multihead_pairwise_scores."""
    H = np.shape(Ws)[0]
    per = np.stack([lowrank_route_logits(src_val, dst_val, Ws[h], Wt[h], w[h], None if b is None else b[h],
                                         temperature) for h in range(H)])
    head = np.argmax(per, axis=0)
    return np.take_along_axis(per, head[None], 0)[0], head, per


def is_multihead(weights):
    """Projection weights of H heads come stacked [H, r, D]; one head is [r, D]."""
    return np.ndim(weights) == 3


# ---------------------------------------------------------------------------
# selection and masks
# ---------------------------------------------------------------------------
def topk_indices(scores, k):
    """Indices of the k largest entries along the last axis, best first, exact
    ties toward the lower index (select_topk, kernel_common.py:426-430)."""
    s = np.asarray(scores)
    order = np.argsort(-s, axis=-1, kind="stable")
    return order[..., :k]


def topk_mask(scores, k):
    """build_topk_mask (kernel_common.py:433-440); k >= n selects everything."""
    s = np.asarray(scores)
    if k >= s.shape[-1]:
        return np.ones(s.shape, dtype=bool)
    mask = np.zeros(s.shape, dtype=bool)
    np.put_along_axis(mask, topk_indices(s, k), True, axis=-1)
    return mask


def causal_window_mask(n, window):
    """mask[i, j] = j <= i and j >= i - window  (kernel_common.py:443-456)."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    return (j <= i) & (j >= i - window)


def masked_softmax(logits, mask):
    """softmax over unmasked entries; masked entries exactly 0 (kernel_common.py:420-423)."""
    x = np.where(mask, np.asarray(logits, F64), -np.inf)
    m = np.max(x, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.where(mask, np.exp(x - m), 0.0)
    return e / np.sum(e, axis=-1, keepdims=True)


def softplus(x):
    x = np.asarray(x, F64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def entmax15(z, mask):
    """1.5-entmax over the unmasked entries of each row, sort-based as the
    reference computes it (native/jakal_net_native.cpp:1133-1169,
    src/jakal_net/kernels.py:155-202): masked entries -> -1e4, shift by the row
    max, halve, sort descending; tau_rho = mean_rho - sqrt(max(0, (1 -
    rho (meansq_rho - mean_rho^2)) / rho)) over the top rho entries; support =
    #{rho : tau_rho <= sorted_rho} (at least 1); p = max(x - tau*, 0)^2, then
    normalised by its sum and zeroed where masked."""
    z = np.where(mask, np.asarray(z, F64), -1e4)
    x = (z - np.max(z, axis=-1, keepdims=True)) / 2.0
    srt = -np.sort(-x, axis=-1)
    rho = np.arange(1, x.shape[-1] + 1, dtype=F64)
    mean = np.cumsum(srt, axis=-1) / rho
    mean_sq = np.cumsum(srt * srt, axis=-1) / rho
    ss = rho * (mean_sq - mean * mean)
    delta = np.maximum((1.0 - ss) / rho, 0.0)
    tau = mean - np.sqrt(delta)
    support = np.maximum(np.sum(tau <= srt, axis=-1, keepdims=True), 1)
    tau_star = np.take_along_axis(tau, support - 1, axis=-1)
    p = np.maximum(x - tau_star, 0.0) ** 2 * mask
    den = np.sum(p, axis=-1, keepdims=True)
    return np.where(den > 0, p / np.where(den > 0, den, 1.0), 0.0)


def signed_entmax15(scores, mask):
    """sign(s) * entmax15(|s|) over the unmasked entries (cpp:1171-1181)."""
    s = np.nan_to_num(np.asarray(scores, F64))
    return np.sign(s) * entmax15(np.abs(s), mask) * mask


def signed_entmax15_backward(scores, mask, grad_routes):
    """cpp:1183-1205: with P = |routes|, u = sqrt(P), gi = sign(s) g u:
    grad s = (gi - u * sum(gi) / sum(u)) * sign(s), masked entries 0."""
    s = np.nan_to_num(np.asarray(scores, F64))
    sg = np.sign(s)
    u = np.sqrt(np.abs(signed_entmax15(s, mask)))
    gi = np.asarray(grad_routes, F64) * sg * u
    us = np.sum(u, axis=-1, keepdims=True)
    corr = np.where(us > 0, np.sum(gi, axis=-1, keepdims=True) / np.where(us > 0, us, 1.0), 0.0)
    return np.where(mask, (gi - corr * u) * sg, 0.0)


# ---------------------------------------------------------------------------
# edge compression (propagation.py:67-88)
# ---------------------------------------------------------------------------
def compress(scores, mask, kind):
    s = np.asarray(scores, F64)
    if kind == "softsign":
        return np.where(mask, s / (1.0 + np.abs(s)), 0.0)
    if kind == "signed_abs_softmax":
        return np.sign(s) * masked_softmax(np.abs(s), mask)
    if kind == "signed_entmax15":
        return signed_entmax15(s, mask)
    raise ValueError(kind)


def compress_backward(scores, mask, kind, grad_edges):
    s = np.asarray(scores, F64)
    g = np.asarray(grad_edges, F64)
    if kind == "softsign":
        return np.where(mask, g / (1.0 + np.abs(s)) ** 2, 0.0)
    if kind == "signed_abs_softmax":
        sg = np.sign(s)
        p = masked_softmax(np.abs(s), mask)
        e = sg * p
        dot = np.sum(g * e, axis=-1, keepdims=True)
        return np.where(mask, sg * p * (sg * g - dot), 0.0)
    if kind == "signed_entmax15":
        return signed_entmax15_backward(s, mask, g)
    raise ValueError(kind)


# ---------------------------------------------------------------------------
# propagation (propagation.py:207-220, 453-480)
# ---------------------------------------------------------------------------
def propagation_mask(scores, mode, *, topk=None, window=None):
    n = scores.shape[-1]
    if mode == "dense":
        return np.ones(scores.shape, dtype=bool)
    if mode == "window":
        return np.broadcast_to(causal_window_mask(n, window), scores.shape)
    if mode == "topk":
        return topk_mask(scores, topk)
    raise ValueError(mode)


def propagation_from_scores(scores, mask, kind, projected_state, projected_val):
    """delta_state = e @ ps, delta_val = e @ pv with e = compress(s) on the mask
    (propagation.py:473-479)."""
    e = compress(scores, mask, kind)
    ds = np.einsum("...ij,...j->...i", e, np.asarray(projected_state, F64))
    dv = np.einsum("...ij,...jd->...id", e, np.asarray(projected_val, F64))
    return ds, dv, e


def propagation_forward(val, ps, pv, U, V, w, b, *, mode="topk", topk=None, window=None, kind="softsign",
                        mask=None):
    """Low-rank propagation forward; returns a dict with deltas and intermediates.

    ``mask`` overrides the selection (used to evaluate the math on a selection
    made elsewhere, e.g. by the GPU, when rows have near-ties).  Stacked
    [H, r, D] projections select the max-aggregated multi-head scores
    (multihead_pairwise_scores); "head" is then each pair's winning head."""
    head = None
    if is_multihead(U):
        s, head, _ = multihead_pairwise_scores(val, val, U, V, w, b)
    else:
        s = lowrank_pairwise_scores(val, val, U, V, w, b)
    if mask is None:
        mask = propagation_mask(s, mode, topk=topk, window=window)
    ds, dv, e = propagation_from_scores(s, mask, kind, ps, pv)
    return {"delta_state": ds, "delta_val": dv, "scores": s, "mask": mask, "edges": e, "head": head}


def _pairwise_score_backward(val, U, V, w, g_s):
    """Gradients of s = (val U^T) diag(w_hat) (val V^T)^T + b given dL/ds."""
    what = normalized_weight(w)
    pt, psrc = lowrank_projections(val, U, V)
    psh = psrc * what
    g_pt = g_s @ psh
    g_psh = np.swapaxes(g_s, -1, -2) @ pt
    g_psrc = g_psh * what
    g_what = np.sum(g_psh * psrc, axis=tuple(range(g_psh.ndim - 1)))
    flat = lambda x: x.reshape(-1, x.shape[-1])  # noqa: E731
    return {"val": g_pt @ U + g_psrc @ V, "U": flat(g_pt).T @ flat(val), "V": flat(g_psrc).T @ flat(val),
            "w": normalized_weight_backward(w, g_what), "w_hat": g_what, "b": float(np.sum(g_s))}


def _per_head_backward(score_backward, head, H, g_s):
    """A max over heads passes each pair's score gradient to its winning head
    only; the heads' gradients are stacked on a leading head axis and the
    input gradients summed."""
    parts = [score_backward(h, np.where(head == h, g_s, 0.0)) for h in range(H)]
    out = {}
    for name in parts[0]:
        vals = [p[name] for p in parts]
        if name in ("val", "src_val", "dst_val"):
            out[name] = np.sum(vals, axis=0)
        else:
            out[name] = np.stack([np.asarray(v, F64) for v in vals])
    return out


def propagation_backward(val, ps, pv, U, V, w, b, g_ds, g_dv, *, mode="topk", topk=None, window=None,
                         kind="softsign", mask=None):
    """Gradients of propagation_forward wrt val (through the scores only), ps,
    pv, U, V, w (raw, through the normalisation) and b; the selection mask is
    treated as constant, as torch.topk's indices are."""
    val = np.asarray(val, F64)
    ps = np.asarray(ps, F64)
    pv = np.asarray(pv, F64)
    U = np.asarray(U, F64)
    V = np.asarray(V, F64)
    w = np.asarray(w, F64)
    g_ds = np.asarray(g_ds, F64)
    g_dv = np.asarray(g_dv, F64)
    fwd = propagation_forward(val, ps, pv, U, V, w, b, mode=mode, topk=topk, window=window, kind=kind, mask=mask)
    s, mask, e = fwd["scores"], fwd["mask"], fwd["edges"]
    g_e = g_ds[..., :, None] * ps[..., None, :] + g_dv @ np.swapaxes(pv, -1, -2)
    g_s = compress_backward(s, mask, kind, g_e)
    g_ps = np.einsum("...ij,...i->...j", e, g_ds)
    g_pv = np.einsum("...ij,...id->...jd", e, g_dv)
    if is_multihead(U):
        g = _per_head_backward(lambda h, gh: _pairwise_score_backward(val, U[h], V[h], w[h], gh), fwd["head"],
                               U.shape[0], g_s)
    else:
        g = _pairwise_score_backward(val, U, V, w, g_s)
    return {**g, "ps": g_ps, "pv": g_pv, "g_scores": g_s, "delta_state": fwd["delta_state"],
            "delta_val": fwd["delta_val"], "head": fwd["head"]}


def normalized_weight_backward(w, g_what):
    """Chain rule through w_hat = w / clamp_min(||w||, 1e-6)."""
    w = np.asarray(w, F64)
    n = float(np.sqrt(np.sum(w * w)))
    if n <= 1e-6:
        return np.asarray(g_what, F64) / 1e-6
    what = w / n
    return (g_what - what * float(np.dot(what, g_what))) / n


# ---------------------------------------------------------------------------
# transition (transition.py:431-452, kernel_common.py:420-423)
# ---------------------------------------------------------------------------
def route_compress(logits, mask, kind="softmax"):
    """Route weights over the masked destinations of each source row:
    softmax (kernel_common.py:420-423) or sign(l) * softmax(|l|)
    (transition.py:53-67, native_backend.py:2184-2188) or sign(l) *
    entmax15(|l|) (transition.py:70-75)."""
    if kind == "softmax":
        return masked_softmax(logits, mask)
    if kind in ("signed_abs_softmax", "signed_entmax15"):
        return compress(logits, mask, kind)
    raise ValueError(kind)


def route_compress_backward(logits, mask, kind, grad_routes):
    if kind == "softmax":
        p = masked_softmax(logits, mask)
        g = np.asarray(grad_routes, F64)
        return np.where(mask, p * (g - np.sum(p * g, axis=-1, keepdims=True)), 0.0)
    if kind in ("signed_abs_softmax", "signed_entmax15"):
        return compress_backward(logits, mask, kind, grad_routes)
    raise ValueError(kind)


def transition_from_logits(logits, mask, sender, ps, pv, kind="softmax"):
    """Per-source route weights over the masked destinations, weighted by the
    sender strength, summed into destinations (transition.py:449-451)."""
    p = route_compress(logits, mask, kind)
    wr = p * np.asarray(sender, F64)[..., :, None]
    ds = np.einsum("...jk,...j->...k", wr, np.asarray(ps, F64))
    dv = np.einsum("...jk,...jd->...kd", wr, np.asarray(pv, F64))
    return ds, dv, p


def transition_forward(src_val, dst_val, sender, ps, pv, Ws, Wt, w, b, *, topk, temperature=1.0, mask=None,
                       kind="softmax"):
    head = None
    if is_multihead(Ws):
        l, head, _ = multihead_route_logits(src_val, dst_val, Ws, Wt, w, b, temperature)
    else:
        l = lowrank_route_logits(src_val, dst_val, Ws, Wt, w, b, temperature)
    if mask is None:
        mask = topk_mask(l, topk)  # per source row, over destinations (transition.py:439-444)
    ds, dv, p = transition_from_logits(l, mask, sender, ps, pv, kind)
    return {"delta_state": ds, "delta_val": dv, "logits": l, "mask": mask, "routes": p, "head": head}


def _route_logit_backward(src_val, dst_val, Ws, Wt, w, g_raw):
    """Gradients of l_raw = ((w * (src Ws^T)) . (dst Wt^T)) + b given dL/dl_raw."""
    psrc = src_val @ Ws.T
    psh = psrc * w
    pt = dst_val @ Wt.T
    g_psh = g_raw @ pt
    g_pt = np.swapaxes(g_raw, -1, -2) @ psh
    g_psrc = g_psh * w
    flat = lambda x: x.reshape(-1, x.shape[-1])  # noqa: E731
    return {"src_val": g_psrc @ Ws, "dst_val": g_pt @ Wt, "Ws": flat(g_psrc).T @ flat(src_val),
            "Wt": flat(g_pt).T @ flat(dst_val), "w": np.sum(g_psh * psrc, axis=tuple(range(g_psh.ndim - 1))),
            "b": float(np.sum(g_raw))}


def transition_backward(src_val, dst_val, sender, ps, pv, Ws, Wt, w, b, g_ds, g_dv, *, topk, temperature=1.0,
                        mask=None, kind="softmax"):
    src_val = np.asarray(src_val, F64)
    dst_val = np.asarray(dst_val, F64)
    sender = np.asarray(sender, F64)
    ps = np.asarray(ps, F64)
    pv = np.asarray(pv, F64)
    Ws = np.asarray(Ws, F64)
    Wt = np.asarray(Wt, F64)
    w = np.asarray(w, F64)
    g_ds = np.asarray(g_ds, F64)
    g_dv = np.asarray(g_dv, F64)
    fwd = transition_forward(src_val, dst_val, sender, ps, pv, Ws, Wt, w, b, topk=topk, temperature=temperature,
                             mask=mask, kind=kind)
    p, mask, logits = fwd["routes"], fwd["mask"], fwd["logits"]
    g_wr = ps[..., :, None] * g_ds[..., None, :] + pv @ np.swapaxes(g_dv, -1, -2)  # [.., Ns, Nd]
    wr = p * sender[..., :, None]
    g_ps = np.sum(wr * g_ds[..., None, :], axis=-1)
    g_pv = wr @ g_dv
    g_sender = np.sum(p * g_wr, axis=-1)
    g_p = g_wr * sender[..., :, None]
    g_l = route_compress_backward(logits, mask, kind, g_p)
    g_raw = g_l / float(temperature)
    if is_multihead(Ws):
        g = _per_head_backward(lambda h, gh: _route_logit_backward(src_val, dst_val, Ws[h], Wt[h], w[h], gh),
                               fwd["head"], Ws.shape[0], g_raw)
    else:
        g = _route_logit_backward(src_val, dst_val, Ws, Wt, w, g_raw)
    return {**g, "sender": g_sender, "ps": g_ps, "pv": g_pv, "g_logits": g_raw,
            "delta_state": fwd["delta_state"], "delta_val": fwd["delta_val"], "head": fwd["head"]}


# ---------------------------------------------------------------------------
# index parity under the gap rule
# ---------------------------------------------------------------------------
def mask_from_indices(idx, n):
    """Boolean [..., Nq, n] mask from a [..., Nq, k] index array (negative = absent)."""
    idx = np.asarray(idx)
    mask = np.zeros(idx.shape[:-1] + (n,), dtype=bool)
    pos = np.nonzero(idx >= 0)
    mask[pos[:-1] + (idx[pos],)] = True
    return mask


def checkable_rows(scores, k, gap=1e-5):
    """Rows whose k-th and (k+1)-th best scores differ by more than ``gap``:
    on these the selected index set is unambiguous."""
    s = np.sort(np.asarray(scores, F64), axis=-1)[..., ::-1]
    if k >= s.shape[-1]:
        return np.ones(s.shape[:-1], dtype=bool)
    return (s[..., k - 1] - s[..., k]) > gap
