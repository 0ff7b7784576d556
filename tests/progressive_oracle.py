"""The Progressive-B query-block step (jakal_net.progressive) as a composition
of oracle calls, float64 numpy, forward only.

Each hot-path operator is the oracle's (propagation_forward in window / top-k
mode, transition_forward with per-source top-k); the glue is restated here from
the reference's definitions (scripts/progressive_b_example.py): the MLP position
encoding (src/jakal_net/modules.py:706-739), the state head, stabilisation
(tanh state, LayerNorm values: :282-292), scaled replacement by each delta
(:85-98, :1011-1024) with the stage's path scales (:1108-1323), the
teacher-forced query feedback (:2034-2047, :2059-2152) and the head with exact
GELU.  Test infrastructure: used by tests/test_api_cpu.py and
tests/test_gpu_progressive.py only.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf

import jakal_oracle as O


def layer_norm(x, w, b, eps=1e-5):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _ln(params, prefix):
    return params[prefix + ".weight"], params[prefix + ".bias"]


def _linear(params, prefix, x):
    return x @ params[prefix + ".weight"].T + params[prefix + ".bias"]


def _pairwise(params, prefix):
    return (params[prefix + ".target_proj.weight"], params[prefix + ".source_proj.weight"],
            params[prefix + ".weight"], float(params[prefix + ".bias"]))


def _route(params, prefix):
    return (params[prefix + ".source_proj.weight"], params[prefix + ".target_proj.weight"],
            params[prefix + ".weight"], float(params[prefix + ".bias"]))


def _prop(params, prefix, layer, **mode):
    U, V, w, b = _pairwise(params, prefix)
    state, val = layer
    f = O.propagation_forward(val, state, val, U, V, w, b, kind="softsign", **mode)
    return f["delta_state"], f["delta_val"]


def _trans(params, prefix, src, dst, topk):
    Ws, Wt, w, b = _route(params, prefix)
    (ss, sv), (_, dv) = src, dst
    f = O.transition_forward(sv, dv, O.softplus(ss), ss, sv, Ws, Wt, w, b, topk=topk)
    return f["delta_state"], f["delta_val"]


def _replace(layer, delta, scale):
    """merge "replace" of the delta scaled by `scale`; a zero scale keeps the layer."""
    if scale == 0.0:
        return layer
    return delta[0] * scale, delta[1] * scale


def _stab(layer, ln):
    return np.tanh(layer[0]), layer_norm(layer[1], *ln)


def _positions(params, n):
    pos = np.zeros((1, 1)) if n == 1 else np.linspace(0.0, 1.0, n)[:, None]
    h = _linear(params, "positions.net.0", pos)
    h = h / (1.0 + np.exp(-h))  # SiLU
    return _linear(params, "positions.net.2", h)


def _slots(params, prefix, B):
    st, v = params[prefix + "_state"], params[prefix + "_val"]
    return np.broadcast_to(st, (B,) + st.shape), np.broadcast_to(v, (B,) + v.shape)


def progressive_logits(params, cfg, prefix_ids, target_ids):
    """Logits [B, query, vocab] of ProgressiveBStep for the given float64 parameters."""
    P = params
    B = prefix_ids.shape[0]

    def state_head(val):
        return _linear(P, "state_init", val)[..., 0]

    s_ln = _ln(P, "s_norm")
    val = P["embed.weight"][prefix_ids] + _positions(P, prefix_ids.shape[1])[None]
    s = _stab((state_head(val), val), s_ln)
    win = dict(mode="window", window=cfg.s_window)
    for i in range(cfg.warmup):
        s = _stab(_replace(s, _prop(P, f"warmup.{i}.pairwise_fn", s, **win), cfg.warmup_scale), s_ln)
    cmp = None
    for i in range(cfg.blocks):
        blk = f"blocks.{i}"
        a, beta_s_to_b, beta_b_to_s = cfg.stage(i)
        bs_ln, e_ln, c_ln = _ln(P, f"{blk}.s_norm"), _ln(P, f"{blk}.exp_norm"), _ln(P, f"{blk}.cmp_norm")
        s = _stab(_replace(s, _prop(P, f"{blk}.s_prop.pairwise_fn", s, **win), cfg.s_scale), bs_ln)
        if cmp is None:
            cmp = _slots(P, f"{blk}.cmp_slot", B)
        cmp = _stab(cmp, c_ln)
        exp = _slots(P, f"{blk}.exp_slot", B)
        exp = _replace(exp, _trans(P, f"{blk}.expand.route_fn", cmp, exp, cfg.topk), a * cfg.b_scale)
        exp = _replace(exp, _prop(P, f"{blk}.exp_prop.pairwise_fn", exp, mode="topk",
                                  topk=min(cfg.topk, cfg.expanded)), a * cfg.b_scale)
        exp = _stab(exp, e_ln)
        s = _replace(s, _trans(P, f"{blk}.b_to_s.route_fn", exp, s, cfg.topk), a * beta_b_to_s * cfg.cross_scale)
        s = _stab(s, bs_ln)
        nxt = _replace(cmp, _trans(P, f"{blk}.compress.route_fn", exp, cmp, cfg.topk), a * cfg.b_scale)
        nxt = _replace(nxt, _trans(P, f"{blk}.s_to_b.route_fn", s, nxt, cfg.topk),
                       a * beta_s_to_b * cfg.cross_scale)
        nxt = _replace(nxt, _prop(P, f"{blk}.cmp_prop.pairwise_fn", nxt, mode="topk",
                                  topk=min(cfg.topk, cfg.compressed)), a * cfg.b_scale)
        cmp = _stab(nxt, c_ln)
    for i in range(cfg.refine):
        s = _stab(_replace(s, _prop(P, f"refine.{i}.pairwise_fn", s, **win), cfg.refine_scale), s_ln)

    q_len = target_ids.shape[1]
    shifted = np.concatenate([np.full((B, 1), cfg.vocab - 1), target_ids[:, :-1]], axis=1)
    fb = _linear(P, "feedback_proj", layer_norm(P["embed.weight"][shifted], *_ln(P, "feedback_norm")))
    q_ln = _ln(P, "q_norm")
    q = _stab((state_head(fb), fb), q_ln)
    for _ in range(cfg.query_refine):
        q = _stab(_replace(q, _trans(P, "q_transition.route_fn", s, q, cfg.topk), cfg.cross_scale), q_ln)
        q = _stab(_replace(q, _prop(P, "q_prop.pairwise_fn", q, mode="window", window=q_len - 1), cfg.s_scale),
                  q_ln)
    h = _linear(P, "head.0", layer_norm(q[1], *_ln(P, "head_norm")))
    h = 0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))
    return _linear(P, "head.2", h)


def cross_entropy(logits, targets):
    z = logits - logits.max(-1, keepdims=True)
    logp = z - np.log(np.exp(z).sum(-1, keepdims=True))
    return float(-np.take_along_axis(logp, targets[..., None], -1).mean())
