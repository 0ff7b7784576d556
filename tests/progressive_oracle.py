"""The Progressive-B query-block step (jakal_net.progressive) as a composition
of oracle calls, float64 numpy, forward only.

Each hot-path operator is the oracle's (propagation_forward in window / top-k
mode, transition_forward with per-source top-k); the glue (embedding rows,
learned positions, LayerNorm, tanh merges, the MLP head with exact GELU, cross
entropy) is restated here from its definition.  Test infrastructure: used by
tests/test_api_cpu.py and tests/test_gpu_progressive.py only.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf

import jakal_oracle as O


def layer_norm(x, w, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _merge(state, val, ds, dv, a, ln):
    return np.tanh(state + a * ds), layer_norm(val + a * dv, *ln)


def _ln(params, prefix):
    return params[prefix + ".weight"], params[prefix + ".bias"]


def _pairwise(params, prefix):
    return (params[prefix + ".target_proj.weight"], params[prefix + ".source_proj.weight"],
            params[prefix + ".weight"], float(params[prefix + ".bias"]))


def _route(params, prefix):
    return (params[prefix + ".source_proj.weight"], params[prefix + ".target_proj.weight"],
            params[prefix + ".weight"], float(params[prefix + ".bias"]))


def _prop(params, prefix, state, val, **mode):
    U, V, w, b = _pairwise(params, prefix)
    f = O.propagation_forward(val, state, val, U, V, w, b, kind="softsign", **mode)
    return f["delta_state"], f["delta_val"]


def _trans(params, prefix, src, dst, topk):
    Ws, Wt, w, b = _route(params, prefix)
    (ss, sv), (_, dv) = src, dst
    f = O.transition_forward(sv, dv, O.softplus(ss), ss, sv, Ws, Wt, w, b, topk=topk)
    return f["delta_state"], f["delta_val"]


def progressive_logits(params, cfg, prefix_ids, target_ids):
    """Logits [B, query, vocab] of ProgressiveBStep for the given float64 parameters."""
    P = params
    B = prefix_ids.shape[0]
    si_w, si_b = P["state_init.weight"], P["state_init.bias"]

    def new_layer(val, ln):
        return np.tanh(val @ si_w.T + si_b)[..., 0], layer_norm(val, *ln)

    s_ln = _ln(P, "s_norm")
    s = new_layer(P["embed.weight"][prefix_ids] + P["positions"][: prefix_ids.shape[1]], s_ln)
    win = dict(mode="window", window=cfg.s_window)
    for i in range(cfg.warmup):
        s = _merge(*s, *_prop(P, f"warmup.{i}.pairwise_fn", *s, **win), cfg.s_scale, s_ln)
    t = np.broadcast_to(P["cmp_slots"], (B,) + P["cmp_slots"].shape)
    cmp = (t[..., 0], t[..., 1:])
    topk = dict(mode="topk", topk=cfg.topk)
    for i in range(cfg.blocks):
        blk = f"blocks.{i}"
        s = _merge(*s, *_prop(P, f"{blk}.s_prop.pairwise_fn", *s, **win), cfg.s_scale, _ln(P, f"{blk}.s_norm"))
        t = np.broadcast_to(P[f"{blk}.exp_slots"], (B,) + P[f"{blk}.exp_slots"].shape)
        exp = (t[..., 0], t[..., 1:])
        e_ln, c_ln, sb_ln = _ln(P, f"{blk}.exp_norm"), _ln(P, f"{blk}.cmp_norm"), _ln(P, f"{blk}.s_norm")
        exp = _merge(*exp, *_trans(P, f"{blk}.expand.route_fn", cmp, exp, cfg.topk), cfg.b_scale, e_ln)
        exp = _merge(*exp, *_prop(P, f"{blk}.exp_prop.pairwise_fn", *exp, **topk), cfg.b_scale, e_ln)
        s = _merge(*s, *_trans(P, f"{blk}.b_to_s.route_fn", exp, s, cfg.topk), cfg.cross_scale, sb_ln)
        cmp = _merge(*cmp, *_trans(P, f"{blk}.compress.route_fn", exp, cmp, cfg.topk), cfg.b_scale, c_ln)
        cmp = _merge(*cmp, *_trans(P, f"{blk}.s_to_b.route_fn", s, cmp, cfg.topk), cfg.cross_scale, c_ln)
        cmp = _merge(*cmp, *_prop(P, f"{blk}.cmp_prop.pairwise_fn", *cmp, **topk), cfg.b_scale, c_ln)
    for i in range(cfg.refine):
        s = _merge(*s, *_prop(P, f"refine.{i}.pairwise_fn", *s, **win), cfg.s_scale, s_ln)

    q_len = target_ids.shape[1]
    shifted = np.concatenate([np.full((B, 1), cfg.vocab - 1), target_ids[:, :-1]], axis=1)
    fb = layer_norm(P["embed.weight"][shifted], *_ln(P, "feedback_norm"))
    fb = fb @ P["feedback_proj.weight"].T + P["feedback_proj.bias"]
    q_ln = _ln(P, "q_norm")
    q = new_layer(fb + P["positions"][prefix_ids.shape[1]:prefix_ids.shape[1] + q_len], q_ln)
    for _ in range(cfg.query_refine):
        q = _merge(*q, *_trans(P, "q_transition.route_fn", s, q, cfg.topk), cfg.cross_scale, q_ln)
        q = _merge(*q, *_prop(P, "q_prop.pairwise_fn", *q, mode="window", window=q_len - 1), cfg.s_scale, q_ln)
    h = layer_norm(q[1], P["head.0.weight"], P["head.0.bias"])
    h = h @ P["head.1.weight"].T + P["head.1.bias"]
    h = 0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))
    return h @ P["head.3.weight"].T + P["head.3.bias"]


def cross_entropy(logits, targets):
    z = logits - logits.max(-1, keepdims=True)
    logp = z - np.log(np.exp(z).sum(-1, keepdims=True))
    return float(-np.take_along_axis(logp, targets[..., None], -1).mean())
