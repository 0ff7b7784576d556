"""Pins the numpy oracle (oracle/jakal_oracle.py) before it is trusted.

Every oracle function is checked against something that does not restate it:
the reference's own known-answer tests, closed forms that reduce to textbook
routines, brute force on tiny inputs, and float64 central finite differences
of the forward for every backward.
"""

import itertools

import numpy as np
import pytest

import jakal_oracle as O


def _rng(seed):
    return np.random.default_rng(seed)


# ---- reference known-answer tests -------------------------------------------

def test_kat_topk_selection_and_mask():
    # tests/test_kernel_common.py:133-140
    s = np.array([[1.0, 5.0, 3.0, -2.0]])
    assert sorted(O.topk_indices(s, 2)[0].tolist()) == [1, 2]
    assert O.topk_mask(s, 2).tolist() == [[False, True, True, False]]


def test_kat_masked_softmax_uses_active_entries():
    # tests/test_kernel_common.py:124-131
    r = O.masked_softmax(np.array([[3.0, 1.0, -4.0]]), np.array([[True, False, True]]))
    assert r[0, 1] == 0.0
    assert abs(r.sum() - 1.0) < 1e-12
    assert np.allclose(r[0, [0, 2]], np.exp([3.0, -4.0]) / np.exp([3.0, -4.0]).sum())


def test_kat_propagation_all_ones_scores():
    # tests/test_jakal_net.py:438-458: scores == 1, softsign(1) == 0.5
    state = np.array([[-1.0, 2.0]])
    val = np.array([[[1.0], [3.0]]])
    mask = np.ones((1, 2, 2), dtype=bool)
    ds, dv, _ = O.propagation_from_scores(np.ones((1, 2, 2)), mask, "softsign", state, val)
    assert np.allclose(ds, [[0.5, 0.5]])
    assert np.allclose(dv, [[[2.0], [2.0]]])


def test_state_weighted_propagation_uses_softplus_strength():
    # Closed form for the configuration of tests/test_jakal_net.py:460-494 under
    # the code's softplus source strength (propagation.py:157-174).  That KAT's
    # literal numbers ([[0.5, 0.5]], [[[3.5], [3.5]]]) assume an identity
    # strength and do not match the code; the "state not squared" property
    # (state_proj_fn is not applied) is what carries over.
    state = np.array([[-1.0, 2.0]])
    val = np.array([[[3.0], [5.0]]])
    strength = O.softplus(state)
    mask = np.ones((1, 2, 2), dtype=bool)
    ds, dv, _ = O.propagation_from_scores(np.ones((1, 2, 2)), mask, "softsign", strength, val * strength[..., None])
    sp = np.log1p(np.exp([-1.0, 2.0]))
    assert np.allclose(ds, 0.5 * sp.sum())
    assert np.allclose(dv[..., 0], 0.5 * (sp[0] * 3.0 + sp[1] * 5.0))


def test_kat_transition_dense_equal_logits():
    # tests/test_jakal_net.py:810-831: zero logits over 2 destinations, rho = state + 1
    state = np.array([[1.0, 2.0]])
    val = np.array([[[1.0, 0.0], [0.0, 2.0]]])
    mask = np.ones((1, 2, 2), dtype=bool)
    ds, dv, _ = O.transition_from_logits(np.zeros((1, 2, 2)), mask, state + 1.0, state, val)
    assert np.allclose(ds, [[4.0, 4.0]])
    assert np.allclose(dv, [[[1.0, 3.0], [1.0, 3.0]]])


def test_kat_sparse_transition_topk_before_softmax():
    # tests/test_jakal_net.py:833-862: per-source top-1, then dst + delta
    logits = np.array([[[3.0, 1.0, 0.0], [0.0, 2.0, 4.0]]])
    state = np.array([[1.0, 2.0]])
    val = np.array([[[10.0], [20.0]]])
    mask = O.topk_mask(logits, 1)
    ds, dv, _ = O.transition_from_logits(logits, mask, state + 1.0, state, val)
    assert np.allclose(ds + 5.0, [[7.0, 5.0, 11.0]])
    assert np.allclose(dv + 1.0, [[[21.0], [1.0], [61.0]]])


def test_kat_gather_helpers_match_manual_selection():
    # tests/test_kernel_common.py:175-184 restated through the oracle's edge form:
    # picking row 3 then row 1 for target 0 is a 0/1 edge matrix times the table
    ps = np.array([[10.0, 20.0, 30.0, 40.0]])
    pv = np.array([[[1.0], [2.0], [3.0], [4.0]]])
    idx = np.array([[[3, 1], [2, 0]]])
    assert np.take_along_axis(ps[:, None, :], idx, axis=-1).tolist() == [[[40.0, 20.0], [30.0, 10.0]]]
    assert pv[0][idx[0]].tolist() == [[[4.0], [2.0]], [[3.0], [1.0]]]


# ---- closed forms and brute force ---------------------------------------------

def test_lowrank_score_equals_effective_bilinear_form():
    r = _rng(1)
    x = r.normal(size=(2, 5, 6))
    U, V = r.normal(size=(3, 6)), r.normal(size=(3, 6))
    w = r.normal(size=3)
    b = 0.3
    what = w / np.linalg.norm(w)
    M = U.T @ np.diag(what) @ V  # x_i^T M x_j
    expect = np.einsum("bid,de,bje->bij", x, M, x) + b
    assert np.allclose(O.lowrank_pairwise_scores(x, x, U, V, w, b), expect)


def test_normalized_weight_small_norm_clamp():
    w = np.array([1e-9, 0.0])
    assert np.allclose(O.normalized_weight(w), w / 1e-6)


def test_route_logits_closed_form():
    r = _rng(2)
    s, d = r.normal(size=(2, 4, 5)), r.normal(size=(2, 3, 6))
    Ws, Wt, w = r.normal(size=(2, 5)), r.normal(size=(2, 6)), r.normal(size=2)
    expect = (np.einsum("bjd,rd->bjr", s, Ws) * w) @ np.swapaxes(np.einsum("bkd,rd->bkr", d, Wt), 1, 2)
    assert np.allclose(O.lowrank_route_logits(s, d, Ws, Wt, w, 0.5, 2.0), (expect + 0.5) / 2.0)


def test_topk_brute_force_with_ties():
    r = _rng(3)
    for _ in range(50):
        s = r.integers(-3, 4, size=(7,)).astype(float)  # many exact ties
        k = int(r.integers(1, 7))
        got = O.topk_indices(s, k).tolist()
        brute = sorted(range(7), key=lambda j: (-s[j], j))[:k]
        assert got == brute


def test_window_mask_closed_form():
    m = O.causal_window_mask(6, 2)
    for i, j in itertools.product(range(6), range(6)):
        assert m[i, j] == (i - 2 <= j <= i)


def test_softsign_and_signed_abs_softmax_closed_forms():
    s = np.array([[-2.0, 0.0, 0.5, 3.0]])
    mask = np.array([[True, True, False, True]])
    assert np.allclose(O.compress(s, mask, "softsign"), [[-2 / 3, 0.0, 0.0, 0.75]])
    e = O.compress(s, mask, "signed_abs_softmax")
    z = np.exp([2.0, 0.0, 3.0])
    assert np.allclose(e, [[-z[0] / z.sum(), 0.0, 0.0, z[2] / z.sum()]])  # sign(0) == 0


def test_entmax15_closed_forms():
    m2 = np.ones((1, 2), dtype=bool)
    assert np.allclose(O.entmax15(np.array([[0.0, 0.0]]), m2), [[0.5, 0.5]])
    # [1, 0]: x = [0, -1/2], both in the support: tau = -1/4 - sqrt(7/16)
    tau = -0.25 - np.sqrt(7.0 / 16.0)
    want = np.array([(0 - tau) ** 2, (-0.5 - tau) ** 2])
    assert np.allclose(O.entmax15(np.array([[1.0, 0.0]]), m2), [want / want.sum()])
    assert np.isclose(want.sum(), 1.0)
    # a dominant entry takes all the mass; masked entries stay 0
    m3 = np.array([[True, True, True, False]])
    assert np.allclose(O.entmax15(np.array([[3.0, 0.0, 0.0, 9.0]]), m3), [[1.0, 0.0, 0.0, 0.0]])
    # sign(0) == 0 drops an entry after the distribution is formed
    e = O.signed_entmax15(np.array([[-1.0, 0.0]]), m2)
    assert e[0, 1] == 0.0 and e[0, 0] < 0


def _entmax_tau_bisection(x, iters=200):
    lo, hi = np.max(x) - 1.0, np.max(x)
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if np.sum(np.maximum(x - mid, 0.0) ** 2) >= 1.0:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


def _entmax_tau_support_iteration(x):
    """Support refinement the HIP kernels use: start from every entry, take the
    closed-form threshold of the current support, keep the entries at or above
    it, repeat until the support no longer changes."""
    tau, n_prev = -np.inf, -1
    for _ in range(x.size + 1):
        s = x[x >= tau]
        if s.size == n_prev:
            break
        n_prev = s.size
        mean, mean_sq = s.mean(), (s * s).mean()
        tau = mean - np.sqrt(max(0.0, (1.0 - s.size * (mean_sq - mean * mean)) / s.size))
    return tau


@pytest.mark.parametrize("n", [1, 2, 5, 17, 64, 300])
def test_entmax15_threshold_solves_its_defining_equation(n):
    """p = max(x - tau, 0)^2 with sum p = 1 (x = z/2 shifted): the sort-based
    restatement, bisection on the defining equation and the support iteration
    of the kernels agree."""
    r = _rng(40 + n)
    for scale in (0.1, 1.0, 10.0):
        z = r.normal(size=(8, n)) * scale
        mask = r.random(size=(8, n)) < 0.8
        mask[:, 0] = True
        p = O.entmax15(z, mask)
        assert np.allclose(p.sum(-1), 1.0)
        for row in range(8):
            zz = z[row][mask[row]]
            x = (zz - zz.max()) / 2.0
            tau_b = _entmax_tau_bisection(x)
            tau_i = _entmax_tau_support_iteration(x)
            assert abs(tau_i - tau_b) < 1e-9
            assert np.allclose(p[row][mask[row]], np.maximum(x - tau_b, 0.0) ** 2, atol=1e-9)
            assert (p[row][~mask[row]] == 0).all()


def test_signed_entmax15_backward_matches_finite_differences():
    r = _rng(41)
    s = r.normal(size=(3, 7)) * 1.5
    mask = r.random(size=(3, 7)) < 0.8
    mask[:, 0] = True
    g = r.normal(size=(3, 7))
    got = O.signed_entmax15_backward(s, mask, g)
    want = _fd(lambda: float(np.sum(O.signed_entmax15(s, mask) * g)), s)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_transition_rows_are_distributions_over_k_destinations():
    r = _rng(4)
    l = r.normal(size=(2, 6, 5))
    mask = O.topk_mask(l, 2)
    p = O.masked_softmax(l, mask)
    assert np.allclose(p.sum(-1), 1.0)
    assert ((p > 0).sum(-1) == 2).all()


# ---- finite-difference pins of every backward -----------------------------------

def _fd(f, x, eps=1e-6):
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = x[i]
        x[i] = old + eps
        fp = f()
        x[i] = old - eps
        fm = f()
        x[i] = old
        g[i] = (fp - fm) / (2 * eps)
    return g


@pytest.mark.parametrize("mode,kind", [("topk", "softsign"), ("window", "softsign"), ("dense", "softsign"),
                                       ("topk", "signed_abs_softmax"), ("window", "signed_abs_softmax"),
                                       ("topk", "signed_entmax15"), ("window", "signed_entmax15"),
                                       ("dense", "signed_entmax15")])
def test_propagation_backward_matches_finite_differences(mode, kind):
    r = _rng(5)
    B, N, D, R = 2, 6, 3, 2
    val = r.normal(size=(B, N, D))
    ps = r.normal(size=(B, N))
    pv = r.normal(size=(B, N, D))
    U, V = r.normal(size=(R, D)), r.normal(size=(R, D))
    w = r.normal(size=R)
    b = np.array(0.2)
    g_ds, g_dv = r.normal(size=(B, N)), r.normal(size=(B, N, D))
    kw = dict(mode=mode, topk=2, window=2, kind=kind)
    mask0 = O.propagation_forward(val, ps, pv, U, V, w, float(b), **kw)["mask"]

    def loss():
        out = O.propagation_forward(val, ps, pv, U, V, w, float(b), **kw)
        assert (out["mask"] == mask0).all(), "selection changed under the FD step"
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    g = O.propagation_backward(val, ps, pv, U, V, w, float(b), g_ds, g_dv, **kw)
    for name, arr in (("val", val), ("ps", ps), ("pv", pv), ("U", U), ("V", V), ("w", w)):
        assert np.allclose(g[name], _fd(loss, arr), rtol=1e-5, atol=1e-6), name
    assert np.allclose(g["b"], _fd(loss, b), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
def test_transition_backward_matches_finite_differences(kind):
    r = _rng(6)
    B, Ns, Nd, D, Dd, R = 2, 5, 4, 3, 2, 2
    src, dst = r.normal(size=(B, Ns, D)), r.normal(size=(B, Nd, D))
    sender = r.normal(size=(B, Ns)) ** 2 + 0.1
    ps, pv = r.normal(size=(B, Ns)), r.normal(size=(B, Ns, Dd))
    Ws, Wt, w = r.normal(size=(R, D)), r.normal(size=(R, D)), r.normal(size=R)
    b = np.array(-0.1)
    g_ds, g_dv = r.normal(size=(B, Nd)), r.normal(size=(B, Nd, Dd))
    kw = dict(topk=2, temperature=1.7, kind=kind)
    mask0 = O.transition_forward(src, dst, sender, ps, pv, Ws, Wt, w, float(b), **kw)["mask"]

    def loss():
        out = O.transition_forward(src, dst, sender, ps, pv, Ws, Wt, w, float(b), **kw)
        assert (out["mask"] == mask0).all()
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    g = O.transition_backward(src, dst, sender, ps, pv, Ws, Wt, w, float(b), g_ds, g_dv, **kw)
    for name, arr in (("src_val", src), ("dst_val", dst), ("sender", sender), ("ps", ps), ("pv", pv),
                      ("Ws", Ws), ("Wt", Wt), ("w", w)):
        assert np.allclose(g[name], _fd(loss, arr), rtol=1e-5, atol=1e-6), name
    assert np.allclose(g["b"], _fd(loss, b), rtol=1e-5, atol=1e-6)


def test_planted_mistake_is_caught_by_finite_differences():
    # A dropped softsign derivative factor must fail the FD check above.
    r = _rng(7)
    B, N, D, R = 1, 5, 2, 2
    val, ps, pv = r.normal(size=(B, N, D)), r.normal(size=(B, N)), r.normal(size=(B, N, D))
    U, V, w = r.normal(size=(R, D)), r.normal(size=(R, D)), r.normal(size=R)
    g_ds, g_dv = r.normal(size=(B, N)), r.normal(size=(B, N, D))
    kw = dict(mode="topk", topk=2, kind="softsign")

    def loss():
        out = O.propagation_forward(val, ps, pv, U, V, w, 0.0, **kw)
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    orig = O.compress_backward
    try:
        O.compress_backward = lambda s, m, k, g: np.where(m, g, 0.0)  # planted: no 1/(1+|s|)^2
        bad = O.propagation_backward(val, ps, pv, U, V, w, 0.0, g_ds, g_dv, **kw)
    finally:
        O.compress_backward = orig
    assert not np.allclose(bad["U"], _fd(loss, U), rtol=1e-4, atol=1e-6)


def test_checkable_rows_gap_rule():
    s = np.array([[3.0, 2.0, 2.0 - 1e-7, 0.0], [3.0, 2.0, 1.0, 0.0]])
    assert O.checkable_rows(s, 2).tolist() == [False, True]


# ---- multi-head max aggregation ---------------------------------------------------

def _heads(r, H, R, D):
    return r.normal(size=(H, R, D)), r.normal(size=(H, R, D)), r.normal(size=(H, R)), r.normal(size=H)


def test_multihead_single_head_reduces_to_the_single_head_form():
    r = _rng(11)
    B, N, D, R = 2, 7, 3, 2
    val, ps, pv = r.normal(size=(B, N, D)), r.normal(size=(B, N)), r.normal(size=(B, N, D))
    U, V, w, b = _heads(r, 1, R, D)
    g_ds, g_dv = r.normal(size=(B, N)), r.normal(size=(B, N, D))
    kw = dict(mode="topk", topk=3, kind="signed_abs_softmax")
    one = O.propagation_backward(val, ps, pv, U[0], V[0], w[0], float(b[0]), g_ds, g_dv, **kw)
    many = O.propagation_backward(val, ps, pv, U, V, w, b, g_ds, g_dv, **kw)
    for name in ("delta_state", "delta_val", "val", "ps", "pv"):
        assert np.allclose(one[name], many[name], rtol=1e-12, atol=1e-12), name
    for name in ("U", "V", "w", "b"):
        assert np.allclose(np.asarray(one[name])[None], many[name], rtol=1e-12, atol=1e-12), name


def test_kat_multihead_scores_are_the_largest_head_score():
    # reference known-answer form (tests/test_jakal_net.py:138-152): the multi-head
    # score is the elementwise maximum of the heads' scores.  Two rank-1 heads
    # with hand-set weights: head 0 scores x_i0 * x_j0 + 1, head 1 scores
    # 2 x_i1 * x_j1 (w_hat = +-1 after normalisation).
    U = np.array([[[1.0, 0.0]], [[0.0, 2.0]]])
    V = np.array([[[1.0, 0.0]], [[0.0, 1.0]]])
    w = np.array([[3.0], [0.5]])
    b = np.array([1.0, 0.0])
    x = np.array([[[1.0, 2.0], [0.5, -1.0], [-2.0, 1.0]]])
    s, head, _ = O.multihead_pairwise_scores(x, x, U, V, w, b)
    h0 = np.outer(x[0, :, 0], x[0, :, 0]) + 1.0
    h1 = 2.0 * np.outer(x[0, :, 1], x[0, :, 1])
    assert np.allclose(s[0], np.maximum(h0, h1))
    assert (head[0] == np.where(h1 > h0, 1, 0)).all()
    l, lhead, _ = O.multihead_route_logits(x, x[:, :2], U, V, w, b, temperature=2.0)
    r0 = 3.0 * np.outer(x[0, :, 0], x[0, :2, 0]) + 1.0
    r1 = 0.5 * 2.0 * np.outer(x[0, :, 1], x[0, :2, 1])
    assert np.allclose(l[0], np.maximum(r0, r1) / 2.0)
    assert (lhead[0] == np.where(r1 > r0, 1, 0)).all()


@pytest.mark.parametrize("mode,kind", [("topk", "softsign"), ("window", "signed_abs_softmax"),
                                       ("dense", "signed_entmax15"), ("topk", "signed_entmax15")])
def test_multihead_propagation_backward_matches_finite_differences(mode, kind):
    r = _rng(12)
    B, N, D, R, H = 2, 6, 3, 2, 3
    val, ps, pv = r.normal(size=(B, N, D)), r.normal(size=(B, N)), r.normal(size=(B, N, D))
    U, V, w, b = _heads(r, H, R, D)
    g_ds, g_dv = r.normal(size=(B, N)), r.normal(size=(B, N, D))
    kw = dict(mode=mode, topk=2, window=2, kind=kind)
    f0 = O.propagation_forward(val, ps, pv, U, V, w, b, **kw)
    assert len(np.unique(f0["head"])) == H, "every head should win some pairs"

    def loss():
        out = O.propagation_forward(val, ps, pv, U, V, w, b, **kw)
        assert (out["mask"] == f0["mask"]).all() and (out["head"] == f0["head"]).all()
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    g = O.propagation_backward(val, ps, pv, U, V, w, b, g_ds, g_dv, **kw)
    for name, arr in (("val", val), ("ps", ps), ("pv", pv), ("U", U), ("V", V), ("w", w), ("b", b)):
        assert np.allclose(g[name], _fd(loss, arr), rtol=1e-5, atol=1e-6), name


@pytest.mark.parametrize("kind", ["softmax", "signed_entmax15"])
def test_multihead_transition_backward_matches_finite_differences(kind):
    r = _rng(13)
    B, Ns, Nd, D, Dd, R, H = 2, 5, 4, 3, 2, 2, 2
    src, dst = r.normal(size=(B, Ns, D)), r.normal(size=(B, Nd, D))
    sender = r.normal(size=(B, Ns)) ** 2 + 0.1
    ps, pv = r.normal(size=(B, Ns)), r.normal(size=(B, Ns, Dd))
    Ws, Wt, w, b = _heads(r, H, R, D)
    g_ds, g_dv = r.normal(size=(B, Nd)), r.normal(size=(B, Nd, Dd))
    kw = dict(topk=2, temperature=1.3, kind=kind)
    f0 = O.transition_forward(src, dst, sender, ps, pv, Ws, Wt, w, b, **kw)

    def loss():
        out = O.transition_forward(src, dst, sender, ps, pv, Ws, Wt, w, b, **kw)
        assert (out["mask"] == f0["mask"]).all() and (out["head"] == f0["head"]).all()
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    g = O.transition_backward(src, dst, sender, ps, pv, Ws, Wt, w, b, g_ds, g_dv, **kw)
    for name, arr in (("src_val", src), ("dst_val", dst), ("sender", sender), ("ps", ps), ("pv", pv),
                      ("Ws", Ws), ("Wt", Wt), ("w", w), ("b", b)):
        assert np.allclose(g[name], _fd(loss, arr), rtol=1e-5, atol=1e-6), name


def test_planted_multihead_mistake_is_caught():
    # Passing every pair's score gradient to all heads (not just the winner) must fail the FD check.
    r = _rng(14)
    B, N, D, R, H = 1, 5, 2, 2, 2
    val, ps, pv = r.normal(size=(B, N, D)), r.normal(size=(B, N)), r.normal(size=(B, N, D))
    U, V, w, b = _heads(r, H, R, D)
    g_ds, g_dv = r.normal(size=(B, N)), r.normal(size=(B, N, D))
    kw = dict(mode="dense", kind="softsign")

    def loss():
        out = O.propagation_forward(val, ps, pv, U, V, w, b, **kw)
        return float(np.sum(out["delta_state"] * g_ds) + np.sum(out["delta_val"] * g_dv))

    def unmasked(score_backward, head, n_heads, g_s):  # planted: no per-head mask
        parts = [score_backward(h, g_s) for h in range(n_heads)]
        return {k: np.stack([np.asarray(p[k]) for p in parts]) for k in parts[0] if k != "val"}

    orig = O._per_head_backward
    try:
        O._per_head_backward = unmasked
        bad = O.propagation_backward(val, ps, pv, U, V, w, b, g_ds, g_dv, **kw)
    finally:
        O._per_head_backward = orig
    assert not np.allclose(bad["U"], _fd(loss, U), rtol=1e-4, atol=1e-6)
