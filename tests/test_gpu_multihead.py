"""GPU parity of max-aggregated multi-head scores (MultiHeadPairwise /
MultiHeadRoute over low-rank heads, reference modules.py:259-301, 470-529;
native composites jakal_net_native.cpp:724-752, 889-917) on the HIP library,
against the float64 oracle (oracle/jakal_oracle.py, multihead_* forms).

Top-k selections are checked on rows whose k-th/(k+1)-th max-aggregated
score gap exceeds 1e-5; outputs and every gradient are compared with the
oracle on the GPU's selection, within rtol 1e-4 / atol 1e-5 or twice the
error of an fp32 torch evaluation of the same max-aggregated op
(tests/parity.py).  Each pair's gradient reaches only its winning head, so a
wrong head per edge shows up in the per-head projection, core-weight and
bias gradients.  Head ranks that are not multiples of 4 run the scalar
(non-float4) paths of the edge kernels.
"""

import math

import numpy as np
import pytest
import torch

import jakal_oracle as O
from parity import check, check_selection, torch32_propagation, torch32_transition

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _np(t):
    return t.detach().double().cpu().numpy()


def _heads(g, H, r, D):
    bound = math.sqrt(6.0 / (D + r))
    U = torch.empty(H, r, D).uniform_(-bound, bound, generator=g)
    V = torch.empty(H, r, D).uniform_(-bound, bound, generator=g)
    w = torch.rand(H, r, generator=g) + 0.5
    b = 0.1 * torch.arange(H, dtype=torch.float32) - 0.05
    return U, V, w, b


def _run_propagation(dev, mode, H, r, param, compress, N, D, B=2, seed=5100, min_checkable=0.5):
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(seed + H * 31 + r)
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    pv_cpu = torch.randn(B, N, D, generator=g)
    U, V, w, b = _heads(g, H, r, D)
    w_hat = w / w.norm(dim=-1, keepdim=True)

    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True)
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd, bd = w_hat.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    op = jn.propagation_topk_selection if mode == "topk" else jn.propagation_window_edges
    ds, dv, idx, score = op("multihead_max_low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X, ps, pv,
                            param, 128, 128)
    gds = torch.randn(B, N, generator=g)
    gdv = torch.randn(B, N, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    scores, head, _ = O.multihead_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), _np(b))
    got_idx = idx.cpu().numpy()
    if mode == "topk":
        frac = check_selection(got_idx, score.cpu().numpy(), scores, param)
        assert frac > min_checkable
        mask = O.mask_from_indices(got_idx, N)
    else:
        width = min(param + 1, N)
        want_idx = np.arange(N)[:, None] - (width - 1 - np.arange(width))[None, :]
        assert (got_idx == np.where(want_idx >= 0, want_idx, -1)[None]).all()
        mask = np.broadcast_to(O.causal_window_mask(N, param), (B, N, N))
        valid = got_idx >= 0
        want_score = np.take_along_axis(scores, np.maximum(got_idx, 0), axis=-1)
        check("window scores", np.where(valid, score.cpu().numpy(), 0.0), np.where(valid, want_score, 0.0))
    print(f"heads winning the kept edges: {np.bincount(head[mask], minlength=H).tolist()}", flush=True)
    assert (np.bincount(head[mask], minlength=H) > 0).all(), "every head should win some kept edges"
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), _np(b), _np(gds),
                                _np(gdv), mode="topk", topk=1, kind=compress, mask=mask)
    t32 = torch32_propagation(dev, val, state, pv_cpu, U, V, w_hat, _np(b), mask, compress, gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    check("grad layer_val", X.grad, gr["val"], t32["val"])
    check("grad projected_state", ps.grad, gr["ps"], t32["ps"])
    check("grad projected_val", pv.grad, gr["pv"], t32["pv"])
    for t, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("H,r,k,compress,N,D", [
    (2, 32, 8, "softsign", 256, 64),
    (4, 16, 16, "signed_abs_softmax", 300, 48),
    (3, 10, 5, "signed_entmax15", 200, 40),      # head rank 10: scalar paths, 3 K-steps
    (2, 64, 32, "softsign", 1100, 96),           # 4 K-steps, k > 16
    (2, 20, 40, "signed_abs_softmax", 500, 32),  # k > 32 (the 80-entry kept region)
    (2, 16, 100, "softsign", 400, 32),           # k > 64: the scored-rows select, one GEMM per head
    (3, 40, 24, "signed_abs_softmax", 300, 48),  # 3 x 64 split ranks > 4 K-steps: scored rows
    (5, 20, 80, "signed_entmax15", 300, 24),     # both
])
def test_multihead_topk_propagation_matches_oracle(dev, H, r, k, compress, N, D):
    _run_propagation(dev, "topk", H, r, k, compress, N, D)


@pytest.mark.parametrize("H,r,window,compress,N,D", [
    (2, 16, 6, "softsign", 120, 32),
    (3, 10, 20, "signed_abs_softmax", 90, 24),
    (4, 8, 63, "signed_entmax15", 64, 16),       # full causal window, every source
    (2, 40, 99, "softsign", 100, 32),            # full causal softsign window of 100: stays an edge list
])
def test_multihead_window_propagation_matches_oracle(dev, H, r, window, compress, N, D):
    _run_propagation(dev, "window", H, r, window, compress, N, D)


def _run_transition(dev, H, r, topk, kind, Ns, Nd, D, temperature, B=2, seed=5200):
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(seed + H * 7 + topk)
    src = torch.randn(B, Ns, D, generator=g)
    dst = torch.randn(B, Nd, D, generator=g)
    state = torch.randn(B, Ns, generator=g)
    pv_cpu = torch.randn(B, Ns, D, generator=g)
    rho_cpu = torch.nn.functional.softplus(state)
    Ws, Wt, w, b = _heads(g, H, r, D)
    leaves = [t.to(dev).requires_grad_(True) for t in (rho_cpu, src, dst, state, pv_cpu, Ws, Wt, w, b)]
    rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd, bd = leaves
    ds, dv, idx, logit = jn.transition_pairwise_topk_routes(
        "multihead_max_low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None, None, None, None, temperature,
        rho, srcd, dstd, psd, pvd, topk, Ns, Nd, kind)
    gds = torch.randn(B, Nd, generator=g)
    gdv = torch.randn(B, Nd, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    logits, head, _ = O.multihead_route_logits(_np(src), _np(dst), _np(Ws), _np(Wt), _np(w), _np(b), temperature)
    k = min(topk, Nd)
    got_idx = idx.cpu().numpy()
    if k < Nd:
        assert check_selection(got_idx, logit.cpu().numpy(), logits, k) > 0.5
    else:
        assert (np.sort(got_idx, axis=-1) == np.arange(Nd)).all()
        check("route logits", logit, np.take_along_axis(logits, got_idx, axis=-1))
    mask = O.mask_from_indices(got_idx, Nd)
    assert (np.bincount(head[mask], minlength=H) > 0).all(), "every head should win some kept routes"
    gr = O.transition_backward(_np(src), _np(dst), _np(rho_cpu), _np(state), _np(pv_cpu), _np(Ws), _np(Wt), _np(w),
                               _np(b), _np(gds), _np(gdv), topk=k, temperature=temperature, mask=mask, kind=kind)
    t32 = torch32_transition(dev, src, dst, rho_cpu, state, pv_cpu, Ws, Wt, w, _np(b), temperature, mask, kind,
                             gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    for t, name in ((rho, "sender"), (srcd, "src_val"), (dstd, "dst_val"), (psd, "ps"), (pvd, "pv"), (Wsd, "Ws"),
                    (Wtd, "Wt"), (wd, "w"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("H,r,topk,kind,Ns,Nd,T", [
    (2, 16, 4, "softmax", 64, 48, 1.0),
    (3, 10, 6, "signed_entmax15", 70, 60, 1.3),
    (4, 8, 12, "signed_abs_softmax", 50, 200, 0.8),
    (2, 8, 40, "softmax", 48, 40, 1.0),   # every destination (no select): heads from the all-keys scores
    (3, 40, 8, "signed_abs_softmax", 64, 90, 1.0),  # beyond the register select's K-steps: scored rows
    (3, 8, 100, "signed_entmax15", 40, 250, 1.1),   # more than 64 routes per source
])
def test_multihead_transition_matches_oracle(dev, H, r, topk, kind, Ns, Nd, T):
    _run_transition(dev, H, r, topk, kind, Ns, Nd, 24, T)


def test_multihead_api_native_matches_reference(dev):
    from jakal_net import (Layer, LowRankBilinearPairwise, LowRankBilinearRoute, MultiHeadPairwise, MultiHeadRoute,
                           SparsePropagation, SparseTransition)

    torch.manual_seed(61)
    layer = Layer(dim=16, num_nodes=40, state=torch.randn(2, 40, device=dev), val=torch.randn(2, 40, 16, device=dev))
    heads = [LowRankBilinearPairwise(16, 8).to(dev) for _ in range(3)]
    with torch.no_grad():
        for i, h in enumerate(heads):
            h.weight.uniform_(0.5, 1.5)
            h.bias.fill_(0.05 * i)
    for sparse in (dict(sparse_type="topk", topk=5), dict(sparse_type="window", window=7)):
        ref = SparsePropagation(MultiHeadPairwise(heads), implementation="reference", **sparse)
        nat = SparsePropagation(MultiHeadPairwise(heads), implementation="native", **sparse)
        a, b = ref(layer), nat(layer)
        assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-4)
        assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-4)
    dst = Layer(dim=16, num_nodes=24, state=torch.randn(2, 24, device=dev), val=torch.randn(2, 24, 16, device=dev))
    rheads = [LowRankBilinearRoute(16, 16, rank=8).to(dev) for _ in range(2)]
    ref = SparseTransition(MultiHeadRoute(rheads), topk=4, implementation="reference")
    nat = SparseTransition(MultiHeadRoute(rheads), topk=4, implementation="native")
    a, b = ref.compute_delta(layer, dst), nat.compute_delta(layer, dst)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-4)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-4)


def _run_dense_propagation(dev, H, r, compress, N, D, causal=False, B=2, seed=5300, edge_bytes=None):
    """Dense (or full causal window) propagation with max-aggregated heads:
    one score GEMM per head folded into a running max, the winning heads
    recorded for the backward (jakal_net_native.cpp:5962-6076 over
    pairwise_scores 724-752)."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(seed + H * 13 + r + (7 if causal else 0))
    state = torch.randn(B, N, generator=g)
    val = torch.randn(B, N, D, generator=g)
    pv_cpu = torch.randn(B, N, D, generator=g)
    U, V, w, b = _heads(g, H, r, D)
    w_hat = w / w.norm(dim=-1, keepdim=True)
    X = val.to(dev).requires_grad_(True)
    ps = state.to(dev).requires_grad_(True)
    pv = pv_cpu.to(dev).requires_grad_(True)
    Ud, Vd = U.to(dev).requires_grad_(True), V.to(dev).requires_grad_(True)
    wd, bd = w_hat.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    saved = jn.DENSE_EDGE_BYTES
    if edge_bytes is not None:
        jn.set_dense_edge_bytes(edge_bytes)
    try:
        args = ("multihead_max_low_rank_bilinear", wd, bd, Vd, None, Ud, None, compress, X, ps, pv)
        if causal:
            ds, dv = jn.propagation_window(*args, N - 1, 128, 128)
        else:
            ds, dv = jn.propagation_dense(*args, None, 128, 128)
        gds = torch.randn(B, N, generator=g)
        gdv = torch.randn(B, N, D, generator=g)
        torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])
    finally:
        jn.set_dense_edge_bytes(saved)

    scores, head, _ = O.multihead_pairwise_scores(_np(val), _np(val), _np(U), _np(V), _np(w), _np(b))
    full = np.tril(np.ones((N, N), bool)) if causal else np.ones((N, N), bool)
    mask = np.broadcast_to(full, (B, N, N))
    wins = np.bincount(head[mask], minlength=H)
    print(f"heads winning the pairs: {wins.tolist()}", flush=True)
    assert (wins > 0).all(), "every head should win some pairs"
    gr = O.propagation_backward(_np(val), _np(state), _np(pv_cpu), _np(U), _np(V), _np(w), _np(b), _np(gds),
                                _np(gdv), mode="topk", topk=1, kind=compress, mask=mask)
    t32 = torch32_propagation(dev, val, state, pv_cpu, U, V, w_hat, _np(b), mask, compress, gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    check("grad layer_val", X.grad, gr["val"], t32["val"])
    check("grad projected_state", ps.grad, gr["ps"], t32["ps"])
    check("grad projected_val", pv.grad, gr["pv"], t32["pv"])
    for t, name in ((Ud, "U"), (Vd, "V"), (wd, "w_hat"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("H,r,compress,N,D", [
    (2, 16, "softsign", 96, 32),
    (3, 8, "signed_abs_softmax", 80, 24),
    (4, 10, "signed_entmax15", 72, 16),   # head rank 10: the 64 x 64 GEMM kernel (unaligned head slices)
    (2, 32, "softsign", 256, 64),         # 128 x 128 GEMM tiles
])
def test_multihead_dense_propagation_matches_oracle(dev, H, r, compress, N, D):
    _run_dense_propagation(dev, H, r, compress, N, D)


@pytest.mark.parametrize("H,r,compress", [(2, 16, "softsign"), (3, 8, "signed_abs_softmax"),
                                          (2, 12, "signed_entmax15")])
def test_multihead_causal_dense_propagation_matches_oracle(dev, H, r, compress):
    # a full causal window of at least 128 nodes runs as causal dense propagation
    _run_dense_propagation(dev, H, r, compress, 160, 32, causal=True)


@pytest.mark.parametrize("compress", ["softsign", "signed_entmax15"])
def test_multihead_dense_propagation_in_ragged_chunks(dev, compress):
    # chunks of two batch elements over three: the backward rebuilds the first
    # chunk's edges and winning heads from the projections
    _run_dense_propagation(dev, 2, 16, compress, 64, 16, B=3, edge_bytes=2 * 64 * 64 * 5)


def _run_transition_dense(dev, H, r, kind, Ns, Nd, D, temperature, B=2, seed=5400):
    """Dense Transition (every source to every destination) with max-aggregated
    multi-head routes (jakal_net_native.cpp:6705-6914 over route_scores 889-917)."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(seed + H * 7 + Nd)
    src = torch.randn(B, Ns, D, generator=g)
    dst = torch.randn(B, Nd, D, generator=g)
    state = torch.randn(B, Ns, generator=g)
    pv_cpu = torch.randn(B, Ns, D, generator=g)
    rho_cpu = torch.nn.functional.softplus(state)
    Ws, Wt, w, b = _heads(g, H, r, D)
    leaves = [t.to(dev).requires_grad_(True) for t in (rho_cpu, src, dst, state, pv_cpu, Ws, Wt, w, b)]
    rho, srcd, dstd, psd, pvd, Wsd, Wtd, wd, bd = leaves
    ds, dv = jn.transition_pairwise_dense("multihead_max_low_rank_bilinear_route", Wsd, None, Wtd, None, wd, bd, None,
                                          None, None, None, kind, temperature, rho, srcd, dstd, psd, pvd, Ns, Nd)
    gds = torch.randn(B, Nd, generator=g)
    gdv = torch.randn(B, Nd, D, generator=g)
    torch.autograd.backward([ds, dv], [gds.to(dev), gdv.to(dev)])

    _, head, _ = O.multihead_route_logits(_np(src), _np(dst), _np(Ws), _np(Wt), _np(w), _np(b), temperature)
    mask = np.ones((B, Ns, Nd), bool)
    wins = np.bincount(head[mask], minlength=H)
    print(f"heads winning the routes: {wins.tolist()}", flush=True)
    assert (wins > 0).all(), "every head should win some routes"
    gr = O.transition_backward(_np(src), _np(dst), _np(rho_cpu), _np(state), _np(pv_cpu), _np(Ws), _np(Wt), _np(w),
                               _np(b), _np(gds), _np(gdv), topk=Nd, temperature=temperature, mask=mask, kind=kind)
    t32 = torch32_transition(dev, src, dst, rho_cpu, state, pv_cpu, Ws, Wt, w, _np(b), temperature, mask, kind,
                             gds, gdv)
    check("delta_state", ds, gr["delta_state"], t32["delta_state"])
    check("delta_val", dv, gr["delta_val"], t32["delta_val"])
    for t, name in ((rho, "sender"), (srcd, "src_val"), (dstd, "dst_val"), (psd, "ps"), (pvd, "pv"), (Wsd, "Ws"),
                    (Wtd, "Wt"), (wd, "w"), (bd, "b")):
        check(f"grad {name}", t.grad, gr[name], t32[name])


@pytest.mark.parametrize("H,r,kind,Ns,Nd,T", [
    (2, 16, "softmax", 96, 80, 1.0),
    (3, 8, "signed_abs_softmax", 72, 100, 0.7),
    (4, 10, "signed_entmax15", 64, 90, 1.3),
    (2, 32, "softmax", 256, 160, 1.0),    # 128 x 128 GEMM tiles on the logits
])
def test_multihead_dense_transition_matches_oracle(dev, H, r, kind, Ns, Nd, T):
    _run_transition_dense(dev, H, r, kind, Ns, Nd, 24, T)


def test_multihead_dense_api_native_matches_reference(dev):
    from jakal_net import Layer, LowRankBilinearPairwise, LowRankBilinearRoute, MultiHeadPairwise, MultiHeadRoute
    from jakal_net import Propagation, SparseTransition

    torch.manual_seed(62)
    layer = Layer(dim=16, num_nodes=70, state=torch.randn(2, 70, device=dev), val=torch.randn(2, 70, 16, device=dev))
    heads = [LowRankBilinearPairwise(16, 8).to(dev) for _ in range(3)]
    with torch.no_grad():
        for i, h in enumerate(heads):
            h.weight.uniform_(0.5, 1.5)
            h.bias.fill_(0.05 * i)
    ref = Propagation(MultiHeadPairwise(heads), implementation="reference")
    nat = Propagation(MultiHeadPairwise(heads), implementation="native")
    a, b = ref(layer), nat(layer)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-4)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-4)
    # top-k over every destination (more than 64): the dense transition
    dst = Layer(dim=16, num_nodes=80, state=torch.randn(2, 80, device=dev), val=torch.randn(2, 80, 16, device=dev))
    rheads = [LowRankBilinearRoute(16, 16, rank=8).to(dev) for _ in range(2)]
    ref = SparseTransition(MultiHeadRoute(rheads), topk=80, implementation="reference")
    nat = SparseTransition(MultiHeadRoute(rheads), topk=80, implementation="native")
    a, b = ref.compute_delta(layer, dst), nat.compute_delta(layer, dst)
    assert torch.allclose(a.delta_state, b.delta_state, atol=1e-5, rtol=1e-4)
    assert torch.allclose(a.delta_val, b.delta_val, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("heads", [1, 2])
@pytest.mark.parametrize("chunked", [False, True])
def test_dense_softsign_backward_twice_repeats(dev, heads, chunked):
    """A softsign dense backward writes its score gradient over the saved edges;
    a second backward through the same graph (retain_graph) rebuilds them from
    the projections and must repeat the first bit for bit."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(5500 + heads)
    B, N, D, r = 3, 64, 16, 8
    X = torch.randn(B, N, D, generator=g).to(dev).requires_grad_(True)
    ps = torch.randn(B, N, generator=g).to(dev).requires_grad_(True)
    U = (0.3 * torch.randn(heads, r, D, generator=g)).to(dev).requires_grad_(True)
    V = (0.3 * torch.randn(heads, r, D, generator=g)).to(dev).requires_grad_(True)
    w = (torch.rand(heads, r, generator=g) + 0.5).to(dev).requires_grad_(True)
    kind = "multihead_max_low_rank_bilinear"
    saved = jn.DENSE_EDGE_BYTES
    if chunked:
        jn.set_dense_edge_bytes(N * N * 5)
    try:
        ds, dv = jn.propagation_dense(kind, w, None, V, None, U, None, "softsign", X, ps, X, None, 128, 128)
        loss = ds.sum() + (dv * dv).sum()
        grads = []
        for _ in range(2):
            for t in (X, ps, U, V, w):
                t.grad = None
            loss.backward(retain_graph=True)
            grads.append([t.grad.clone() for t in (X, ps, U, V, w)])
    finally:
        jn.set_dense_edge_bytes(saved)
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_multihead_limits_raise_before_launch(dev):
    import jakal_net_native as jn

    X = torch.randn(1, 64, 16, device=dev)
    ps = torch.randn(1, 64, device=dev)
    # more than 8 heads, or more than 128 ranks over all heads
    U = torch.randn(9, 4, 16, device=dev)
    with pytest.raises(NotImplementedError):
        jn.propagation_dense("multihead_max_low_rank_bilinear", torch.ones(9, 4, device=dev), None, U, None, U,
                             None, "softsign", X, ps, X, None, 128, 128)
    U2 = torch.randn(3, 48, 16, device=dev)
    with pytest.raises(NotImplementedError):
        jn.propagation_dense("multihead_max_low_rank_bilinear", torch.ones(3, 48, device=dev), None, U2, None, U2,
                             None, "softsign", X, ps, X, None, 128, 128)
