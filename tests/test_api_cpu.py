"""The operator API (jakal_net) on the CPU: containers, the PyTorch forms
against the float64 oracle and the reference's known answers, and the native
dispatch rules (with a stand-in native module, so no GPU is needed).

Reference semantics: src/jakal_net/core.py:30-131, propagation.py:207-220,
453-480, transition.py:431-452; known answers tests/test_jakal_net.py:438-458,
810-831, 833-862 and tests/test_kernel_common.py:124-140.
"""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

import jakal_oracle as O
from jakal_net import (Layer, LayerDelta, LowRankBilinearPairwise, LowRankBilinearRoute, MultiHeadPairwise,
                       MultiHeadRoute, Propagation, SparsePropagation, SparseTransition, TemperatureScaledRoute,
                       Transition)
from jakal_net import kernel_common as KC
from jakal_net import native_backend as NB
from jakal_net.compress import signed_abs_softmax, signed_entmax15



@pytest.fixture(autouse=True)
def _float64_default():
    """float64 tensors and modules in these tests only (restored afterwards)."""
    saved = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(saved)


# ---------------------------------------------------------------------------
# containers
# ---------------------------------------------------------------------------
def test_layer_shapes_and_delta_merge():
    layer = Layer(dim=3, num_nodes=4, state=torch.zeros(2, 4), val=torch.zeros(2, 4, 3))
    assert layer.batch_shape == (2,)
    delta = LayerDelta(delta_state=torch.ones(2, 4), delta_val=torch.full((2, 4, 3), 2.0))
    added = layer.apply_delta(delta)
    assert torch.equal(added.state, torch.ones(2, 4)) and torch.equal(added.val, torch.full((2, 4, 3), 2.0))
    replaced = added.apply_delta(delta, "replace")
    assert replaced.state is delta.delta_state and replaced.val is delta.delta_val
    twice = added.apply_delta(delta, "add")
    assert torch.equal(twice.val, torch.full((2, 4, 3), 4.0))
    z = Layer.zeros(dim=5, num_nodes=7, batch_shape=(3,))
    assert z.state.shape == (3, 7) and z.val.shape == (3, 7, 5)
    assert torch.equal(LayerDelta.zeros_like(z).delta_val, torch.zeros(3, 7, 5))
    c = layer.clone()
    assert c.state is not layer.state and torch.equal(c.val, layer.val)


@pytest.mark.parametrize("state,val,dim,nodes", [
    ((4,), (4, 2), 3, 4),        # wrong dim
    ((4,), (5, 3), 3, 4),        # node axes disagree
    ((2, 4), (3, 4, 3), 3, 4),   # batch shapes disagree
    ((), (4, 3), 3, 4),          # no node axis
    ((4,), (4, 3), 0, 4),        # empty dim
])
def test_layer_rejects_malformed_tensors(state, val, dim, nodes):
    with pytest.raises(ValueError):
        Layer(dim=dim, num_nodes=nodes, state=torch.zeros(state), val=torch.zeros(val))


def test_delta_and_merge_mode_errors():
    layer = Layer.zeros(dim=2, num_nodes=3)
    with pytest.raises(ValueError):
        LayerDelta(delta_state=torch.zeros(3), delta_val=torch.zeros(4, 2))
    with pytest.raises(ValueError):
        layer.apply_delta(LayerDelta(torch.zeros(4), torch.zeros(4, 2)))
    with pytest.raises(ValueError):
        layer.apply_delta(LayerDelta.zeros_like(layer), "multiply")
    with pytest.raises(ValueError):
        Propagation(lambda a, b: a @ b.transpose(-1, -2), implementation="fast")


# ---------------------------------------------------------------------------
# the reference's known answers, through the API
# ---------------------------------------------------------------------------
def _ones_scores(target, source):
    return torch.ones((*target.shape[:-2], target.shape[-2], source.shape[-2]))


@pytest.mark.parametrize("impl", ["reference", "streaming"])
def test_kat_propagation_has_no_state_activation(impl):
    # tests/test_jakal_net.py:438-458: all-ones scores, softsign -> 0.5 per edge
    layer = Layer(dim=1, num_nodes=2, state=torch.tensor([[-1.0, 2.0]]), val=torch.tensor([[[1.0], [3.0]]]))
    delta = Propagation(_ones_scores, implementation=impl, target_block_size=1, source_block_size=1)(layer)
    assert torch.allclose(delta.delta_state, torch.tensor([[0.5, 0.5]]))
    assert torch.allclose(delta.delta_val, torch.tensor([[[2.0], [2.0]]]))


@pytest.mark.parametrize("impl", ["reference", "streaming"])
def test_kat_transition_routes_with_state_activation(impl):
    # tests/test_jakal_net.py:810-831
    src = Layer(dim=2, num_nodes=2, state=torch.tensor([[1.0, 2.0]]), val=torch.tensor([[[1.0, 0.0], [0.0, 2.0]]]))
    dst = Layer.zeros(dim=2, num_nodes=2, batch_shape=(1,))
    op = Transition(lambda v: torch.zeros((*v.shape[:-1], 2)), state_activation_fn=lambda x: x + 1.0,
                    implementation=impl, src_block_size=1)
    out = op(src, dst)
    assert torch.allclose(out.state, torch.tensor([[4.0, 4.0]]))
    assert torch.allclose(out.val, torch.tensor([[[1.0, 3.0], [1.0, 3.0]]]))


@pytest.mark.parametrize("impl", ["reference", "streaming"])
def test_kat_sparse_transition_top1_per_source(impl):
    # tests/test_jakal_net.py:833-862: per-source top-1 before the softmax
    src = Layer(dim=1, num_nodes=2, state=torch.tensor([[1.0, 2.0]]), val=torch.tensor([[[10.0], [20.0]]]))
    dst = Layer(dim=1, num_nodes=3, state=torch.tensor([[5.0, 5.0, 5.0]]), val=torch.ones(1, 3, 1))
    logits = torch.tensor([[[3.0, 1.0, 0.0], [0.0, 2.0, 4.0]]])
    op = SparseTransition(lambda v: logits.expand(v.shape[0], -1, -1), topk=1,
                          state_activation_fn=lambda x: x + 1.0, implementation=impl, src_block_size=2)
    out = op(src, dst)
    assert torch.allclose(out.state, torch.tensor([[7.0, 5.0, 11.0]]))
    assert torch.allclose(out.val, torch.tensor([[[21.0], [1.0], [61.0]]]))


# ---------------------------------------------------------------------------
# the PyTorch forms against the oracle
# ---------------------------------------------------------------------------
def _np(t):
    return t.detach().cpu().numpy()


def _fn(kind):
    return {"softsign": F.softsign, "signed_abs_softmax": signed_abs_softmax,
            "signed_entmax15": signed_entmax15}[kind]


@pytest.mark.parametrize("kind", ["softsign", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("mode", ["dense", "topk", "window"])
def test_propagation_forms_match_oracle(kind, mode):
    torch.manual_seed(11)
    B, N, D, r = 2, 23, 6, 4
    layer = Layer(dim=D, num_nodes=N, state=torch.randn(B, N), val=torch.randn(B, N, D))
    mod = LowRankBilinearPairwise(D, r)
    with torch.no_grad():
        mod.weight.copy_(torch.rand(r) + 0.5)
        mod.bias.fill_(0.1)
    ps_fn, pv_fn = (lambda s: 0.5 * s + 0.25), (lambda v: v * 1.5 - 0.5)
    if mode == "dense":
        ops = [Propagation(mod, edge_compress_fn=_fn(kind), state_proj_fn=ps_fn, val_proj_fn=pv_fn,
                           implementation=impl, target_block_size=5) for impl in ("reference", "streaming")]
        kw = dict(mode="dense")
    else:
        extra = dict(topk=5) if mode == "topk" else dict(window=4)
        ops = [SparsePropagation(mod, sparse_type=mode, edge_compress_fn=_fn(kind), state_proj_fn=ps_fn,
                                 val_proj_fn=pv_fn, implementation=impl, target_block_size=5, **extra)
               for impl in ("reference", "streaming")]
        kw = dict(mode=mode, **extra)
    want = O.propagation_forward(_np(layer.val), _np(ps_fn(layer.state)), _np(pv_fn(layer.val)),
                                 _np(mod.target_proj.weight), _np(mod.source_proj.weight), _np(mod.weight), 0.1,
                                 kind=kind, **kw)
    for op in ops:
        d = op(layer)
        np.testing.assert_allclose(_np(d.delta_state), want["delta_state"], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(_np(d.delta_val), want["delta_val"], rtol=1e-10, atol=1e-12)


def test_state_weighted_edges_scale_by_softplus():
    # state_weight_edges: each edge scaled by softplus(state_j), delta_state = sum_j e_ij (propagation.py:474-478)
    torch.manual_seed(12)
    B, N, D, r = 1, 9, 4, 3
    layer = Layer(dim=D, num_nodes=N, state=torch.randn(B, N), val=torch.randn(B, N, D))
    mod = LowRankBilinearPairwise(D, r)
    s = O.lowrank_pairwise_scores(_np(layer.val), _np(layer.val), _np(mod.target_proj.weight),
                                  _np(mod.source_proj.weight), _np(mod.weight), 0.0)
    e = O.compress(s, O.topk_mask(s, 3), "softsign") * O.softplus(_np(layer.state))[:, None, :]
    for impl in ("reference", "streaming"):
        d = SparsePropagation(mod, sparse_type="topk", topk=3, state_weight_edges=True, implementation=impl)(layer)
        np.testing.assert_allclose(_np(d.delta_state), e.sum(-1), rtol=1e-10)
        np.testing.assert_allclose(_np(d.delta_val), e @ _np(layer.val), rtol=1e-10)


@pytest.mark.parametrize("kind", ["softmax", "signed_abs_softmax", "signed_entmax15"])
@pytest.mark.parametrize("topk", [3, 50])
@pytest.mark.parametrize("direction_only", [False, True])
def test_transition_forms_match_oracle(kind, topk, direction_only):
    torch.manual_seed(13)
    B, Ns, Nd, Ds, Dd, r = 2, 17, 7, 6, 5, 4
    src = Layer(dim=Ds, num_nodes=Ns, state=torch.randn(B, Ns), val=torch.randn(B, Ns, Ds))
    dst = Layer(dim=Dd, num_nodes=Nd, state=torch.randn(B, Nd), val=torch.randn(B, Nd, Dd))
    route = TemperatureScaledRoute(LowRankBilinearRoute(Ds, Dd, rank=r), 1.3)
    with torch.no_grad():
        route.route_fn.weight.copy_(torch.rand(r) + 0.5)
        route.route_fn.bias.fill_(0.2)
    proj = torch.nn.Linear(Ds, Dd)
    ops = [SparseTransition(route, topk=topk, route_compress_name=kind, val_proj_fn=proj, implementation=impl,
                            src_block_size=4, use_direction_only=direction_only)
           for impl in ("reference", "streaming")]
    unit = (lambda v: v / np.maximum(np.linalg.norm(v, axis=-1, keepdims=True), 1e-6)) if direction_only else (
        lambda v: v)
    sv, dv_ = unit(_np(src.val)), unit(_np(dst.val))
    pv = sv @ _np(proj.weight).T + _np(proj.bias)
    rho = O.softplus(_np(src.state))
    want = O.transition_forward(sv, dv_, rho, _np(src.state), pv, _np(route.route_fn.source_proj.weight),
                                _np(route.route_fn.target_proj.weight), _np(route.route_fn.weight), 0.2,
                                topk=min(topk, Nd), temperature=1.3, kind=kind)
    for op in ops:
        d = op.compute_delta(src, dst)
        np.testing.assert_allclose(_np(d.delta_state), want["delta_state"], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(_np(d.delta_val), want["delta_val"], rtol=1e-10, atol=1e-12)


def test_route_statistics_include_topk_overlap():
    torch.manual_seed(14)
    src = Layer(dim=4, num_nodes=6, state=torch.randn(1, 6), val=torch.randn(1, 6, 4))
    dst = Layer(dim=4, num_nodes=5, state=torch.randn(1, 5), val=torch.randn(1, 5, 4))
    op = SparseTransition(LowRankBilinearRoute(4, 4, rank=3), topk=2)
    op.track_stats = True
    op.compute_delta(src, dst)
    stats = op.last_stats
    assert set(stats) == {"entropy", "destination_load_variance", "dead_slot_ratio", "topk_overlap"}
    logits = op.compute_route_logits(src, dst)
    idx = torch.topk(logits, 2, dim=-1).indices[0]
    shared = [(int(j) in set(idx[i - 1].tolist())) for i in range(1, 6) for j in idx[i]]
    assert stats["topk_overlap"] == pytest.approx(np.mean(shared))
    # routes of a top-k transition sum to 1 over each source's kept destinations: no destination beyond k
    assert 0.0 <= stats["dead_slot_ratio"] <= 1.0


# ---------------------------------------------------------------------------
# native dispatch, with a stand-in module reporting the CPU as its device
# ---------------------------------------------------------------------------
class _FakeNative:
    def __init__(self, fail_with=None):
        self.calls = []
        self.fail_with = fail_with

    def _record(self, name, args):
        self.calls.append((name, args))
        if self.fail_with is not None:
            raise self.fail_with

    def propagation_topk(self, *args):
        self._record("propagation_topk", args)
        val, ps, pv = args[8], args[9], args[10]
        return torch.zeros_like(ps), torch.zeros_like(pv)

    def transition_pairwise_topk(self, *args, route_compress_name="softmax"):
        self._record("transition_pairwise_topk", args)
        dst_val, ps, pv = args[14], args[15], args[16]
        return ps.new_zeros(dst_val.shape[:-1]), pv.new_zeros((*dst_val.shape[:-1], pv.shape[-1]))


@pytest.fixture
def fake_native(monkeypatch):
    def install(fail_with=None):
        fake = _FakeNative(fail_with)
        status = NB.NativeStatus(True, "fake", "fake", ("propagation_topk", "transition_pairwise_topk"), ("cpu",),
                                 None)
        monkeypatch.setattr(NB._LOADER, "module", fake)
        monkeypatch.setattr(NB._LOADER, "status", status)
        monkeypatch.delenv(NB.DISABLE_NATIVE_ENV, raising=False)
        return fake
    return install


def _topk_case(impl, topk=3):
    torch.manual_seed(15)
    layer = Layer(dim=4, num_nodes=9, state=torch.randn(2, 9), val=torch.randn(2, 9, 4))
    return SparsePropagation(LowRankBilinearPairwise(4, 3), sparse_type="topk", topk=topk,
                             implementation=impl), layer


def test_native_mode_calls_the_module(fake_native):
    fake = fake_native()
    op, layer = _topk_case("native")
    d = op(layer)
    assert [c[0] for c in fake.calls] == ["propagation_topk"]
    assert torch.equal(d.delta_val, torch.zeros_like(layer.val))


def test_kernel_mode_falls_back_when_the_library_declines(fake_native):
    fake_native(NotImplementedError("beyond the library's limits"))
    op, layer = _topk_case("kernel")
    ref, _ = _topk_case("reference")
    ref.pairwise_fn.load_state_dict(op.pairwise_fn.state_dict())
    got, want = op(layer), ref(layer)
    assert torch.allclose(got.delta_val, want.delta_val) and torch.allclose(got.delta_state, want.delta_state)


def test_native_mode_raises_when_the_library_declines(fake_native):
    fake_native(NotImplementedError("beyond the library's limits"))
    op, layer = _topk_case("native")
    with pytest.raises(NotImplementedError):
        op(layer)


def test_direction_only_transition_reaches_the_module_with_unit_values(fake_native):
    fake = fake_native()
    torch.manual_seed(16)
    src = Layer(dim=4, num_nodes=6, state=torch.randn(1, 6), val=3.0 * torch.randn(1, 6, 4))
    dst = Layer(dim=4, num_nodes=5, state=torch.randn(1, 5), val=2.0 * torch.randn(1, 5, 4))
    op = SparseTransition(LowRankBilinearRoute(4, 4, rank=3), topk=2, implementation="native",
                          use_direction_only=True)
    op.compute_delta(src, dst)
    assert [c[0] for c in fake.calls] == ["transition_pairwise_topk"]
    args = fake.calls[0][1]
    src_val, dst_val, pv = args[13], args[14], args[16]
    assert torch.allclose(src_val.norm(dim=-1), torch.ones(1, 6))
    assert torch.allclose(dst_val.norm(dim=-1), torch.ones(1, 5))
    assert torch.allclose(pv, src_val)  # identity val_proj_fn of the unit directions


def test_cpu_tensors_in_native_mode_run_streaming_without_a_cpu_module():
    # the HIP library reports only "cuda": CPU tensors take the PyTorch form
    if not NB.native_status().available:
        pytest.skip("native module not importable here")
    op, layer = _topk_case("native")
    ref, _ = _topk_case("reference")
    ref.pairwise_fn.load_state_dict(op.pairwise_fn.state_dict())
    assert torch.allclose(op(layer).delta_val, ref(layer).delta_val)


# ---------------------------------------------------------------------------
# the Progressive-B query-block step (a caller of the hot path)
# ---------------------------------------------------------------------------
def _small_progressive():
    from jakal_net.progressive import ProgressiveBConfig

    return ProgressiveBConfig(vocab=97, dim=32, prefix=48, query=8, rank=8, topk=4, s_window=6, warmup=1,
                              blocks=2, expanded=24, compressed=8, refine=1, query_refine=2)


def test_progressive_step_matches_oracle_composition():
    import progressive_oracle as PO
    from jakal_net.progressive import ProgressiveBStep

    cfg = _small_progressive()
    torch.manual_seed(21)
    model = ProgressiveBStep(cfg, implementation="reference")
    g = torch.Generator().manual_seed(22)
    prefix = torch.randint(0, cfg.vocab - 1, (2, cfg.prefix), generator=g)
    target = torch.randint(0, cfg.vocab - 1, (2, cfg.query), generator=g)
    logits = model.query_logits(model.encode_prefix(prefix), target)
    params = {k: v.detach().numpy() for k, v in model.state_dict().items()}
    want = PO.progressive_logits(params, cfg, prefix.numpy(), target.numpy())
    np.testing.assert_allclose(_np(logits), want, rtol=1e-9, atol=1e-10)
    loss = float(model(prefix, target).detach())
    assert loss == pytest.approx(PO.cross_entropy(want, target.numpy()), rel=1e-10)
    # the streaming forms give the same step
    stream = ProgressiveBStep(cfg, implementation="streaming")
    stream.load_state_dict(model.state_dict())
    assert float(stream(prefix, target).detach()) == pytest.approx(loss, rel=1e-10)


# ---------------------------------------------------------------------------
# multi-head scores (reference modules.py:259-301, 470-529)
# ---------------------------------------------------------------------------
def _heads(H, D, r, seed, *, bias=True):
    torch.manual_seed(seed)
    heads = [LowRankBilinearPairwise(D, r, bias=bias) for _ in range(H)]
    with torch.no_grad():
        for i, h in enumerate(heads):
            h.weight.copy_(torch.rand(r) + 0.5)
            if bias:
                h.bias.fill_(0.1 * (i - 1))
    return heads


def _stacked(heads, route=False):
    if route:
        return (np.stack([_np(h.source_proj.weight) for h in heads]), np.stack([_np(h.target_proj.weight) for h in heads]),
                np.stack([_np(h.weight) for h in heads]), np.array([float(h.bias.detach()) for h in heads]))
    return (np.stack([_np(h.target_proj.weight) for h in heads]), np.stack([_np(h.source_proj.weight) for h in heads]),
            np.stack([_np(h.weight) for h in heads]), np.array([float(h.bias.detach()) for h in heads]))


def test_kat_multihead_pairwise_is_the_max_of_its_heads():
    # tests/test_jakal_net.py:138-152 with low-rank heads of hand-set weights
    a, b = LowRankBilinearPairwise(2, 1), LowRankBilinearPairwise(2, 1)
    with torch.no_grad():
        a.target_proj.weight.copy_(torch.tensor([[1.0, 0.0]]))
        a.source_proj.weight.copy_(torch.tensor([[1.0, 0.0]]))
        b.target_proj.weight.copy_(torch.tensor([[0.0, 2.0]]))
        b.source_proj.weight.copy_(torch.tensor([[0.0, 1.0]]))
        a.bias.fill_(1.0)
        b.bias.zero_()
    x = torch.tensor([[[1.0, 2.0], [0.5, -1.0], [-2.0, 1.0]]])
    got = MultiHeadPairwise([a, b])(x, x)
    want = torch.maximum(x[..., :1] @ x[..., :1].transpose(-1, -2) + 1.0, 2.0 * x[..., 1:] @ x[..., 1:].transpose(-1, -2))
    assert torch.allclose(got, want)


@pytest.mark.parametrize("aggregate", ["mean", "sum", "head_mean", "smoothmax", "signed_smoothmax"])
def test_multihead_pairwise_aggregates(aggregate):
    heads = _heads(3, 4, 2, 21)
    x = torch.randn(2, 5, 4)
    per = torch.stack([h(x, x) for h in heads], dim=-1)
    want = {"mean": per.mean(-1), "sum": per.sum(-1), "head_mean": per.sum(-1),
            "smoothmax": torch.logsumexp(per, -1) - np.log(3.0),
            "signed_smoothmax": (per * torch.softmax(per.abs(), -1)).sum(-1)}[aggregate]
    mod = MultiHeadPairwise(heads, aggregate=aggregate)
    assert torch.allclose(mod(x, x), want)
    assert torch.allclose(mod.head_scores(x, x), per)
    assert not KC.supports_pairwise_kernel(mod)  # the library runs the max aggregation only


@pytest.mark.parametrize("mode", ["dense", "topk", "window"])
@pytest.mark.parametrize("kind", ["softsign", "signed_entmax15"])
def test_multihead_propagation_forms_match_oracle(mode, kind):
    heads = _heads(3, 6, 4, 22)
    layer = Layer(dim=6, num_nodes=19, state=torch.randn(2, 19), val=torch.randn(2, 19, 6))
    extra = {} if mode == "dense" else (dict(topk=4) if mode == "topk" else dict(window=3))
    mk = (lambda impl: Propagation(MultiHeadPairwise(heads), edge_compress_fn=_fn(kind), implementation=impl,
                                   target_block_size=5)) if mode == "dense" else (
        lambda impl: SparsePropagation(MultiHeadPairwise(heads), sparse_type=mode, edge_compress_fn=_fn(kind),
                                       implementation=impl, target_block_size=5, **extra))
    U, V, w, b = _stacked(heads)
    want = O.propagation_forward(_np(layer.val), _np(layer.state), _np(layer.val), U, V, w, b, mode=mode, kind=kind,
                                 **extra)
    assert len(np.unique(want["head"])) == 3
    for impl in ("reference", "streaming"):
        d = mk(impl)(layer)
        np.testing.assert_allclose(_np(d.delta_state), want["delta_state"], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(_np(d.delta_val), want["delta_val"], rtol=1e-10, atol=1e-12)


def test_multihead_transition_forms_match_oracle():
    torch.manual_seed(23)
    B, Ns, Nd, D, r = 2, 13, 9, 5, 3
    src = Layer(dim=D, num_nodes=Ns, state=torch.randn(B, Ns), val=torch.randn(B, Ns, D))
    dst = Layer(dim=D, num_nodes=Nd, state=torch.randn(B, Nd), val=torch.randn(B, Nd, D))
    heads = [LowRankBilinearRoute(D, D, rank=r) for _ in range(2)]
    with torch.no_grad():
        for i, h in enumerate(heads):
            h.weight.copy_(torch.rand(r) + 0.5)
            h.bias.fill_(0.3 * i - 0.1)
    route = TemperatureScaledRoute(MultiHeadRoute(heads), 1.4)
    Ws, Wt, w, b = _stacked(heads, route=True)
    want = O.transition_forward(_np(src.val), _np(dst.val), O.softplus(_np(src.state)), _np(src.state), _np(src.val),
                                Ws, Wt, w, b, topk=3, temperature=1.4, kind="signed_abs_softmax")
    for impl in ("reference", "streaming"):
        d = SparseTransition(route, topk=3, route_compress_name="signed_abs_softmax", implementation=impl,
                             src_block_size=4).compute_delta(src, dst)
        np.testing.assert_allclose(_np(d.delta_state), want["delta_state"], rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(_np(d.delta_val), want["delta_val"], rtol=1e-10, atol=1e-12)


def test_multihead_kernel_specs_stack_the_heads():
    heads = _heads(3, 6, 4, 24)
    spec = KC.pairwise_kernel_spec(MultiHeadPairwise(heads))
    assert spec.kind == "multihead_max_low_rank_bilinear"
    assert spec.weight.shape == (3, 4) and spec.bias.shape == (3,)
    assert spec.in_weight.shape == (3, 4, 6) and spec.out_weight.shape == (3, 4, 6)
    assert torch.allclose(spec.weight[1], heads[1].normalized_weight())
    assert KC.pairwise_kernel_spec(MultiHeadPairwise(_heads(2, 6, 4, 25, bias=False))).bias is None
    # heads of different ranks, or a mix of biased and unbiased heads, are not one stacked spec
    assert not KC.supports_pairwise_kernel(MultiHeadPairwise([LowRankBilinearPairwise(6, 4), LowRankBilinearPairwise(6, 3)]))
    assert not KC.supports_pairwise_kernel(MultiHeadPairwise([LowRankBilinearPairwise(6, 4),
                                                              LowRankBilinearPairwise(6, 4, bias=False)]))
    # route heads: one temperature each, times an outer TemperatureScaledRoute's
    rheads = [TemperatureScaledRoute(LowRankBilinearRoute(5, 5, rank=2), 2.0) for _ in range(2)]
    route = TemperatureScaledRoute(MultiHeadRoute(rheads), 1.5)
    rspec = KC.pairwise_route_kernel_spec(route)
    assert rspec.kind == "multihead_max_low_rank_bilinear_route" and rspec.temperature == pytest.approx(3.0)
    assert rspec.source_weight.shape == (2, 2, 5) and rspec.core_weight.shape == (2, 2)
    x, y = torch.randn(1, 4, 5), torch.randn(1, 3, 5)
    raw = torch.maximum(rheads[0].route_fn(x, y), rheads[1].route_fn(x, y))
    assert torch.allclose(route(x, y), raw / 3.0)
    mixed = MultiHeadRoute([TemperatureScaledRoute(LowRankBilinearRoute(5, 5, rank=2), 2.0),
                            LowRankBilinearRoute(5, 5, rank=2)])
    assert not KC.supports_pairwise_route_kernel(mixed)


def test_native_mode_passes_stacked_multihead_specs(fake_native):
    fake = fake_native()
    heads = _heads(2, 4, 3, 26)
    layer = Layer(dim=4, num_nodes=9, state=torch.randn(2, 9), val=torch.randn(2, 9, 4))
    SparsePropagation(MultiHeadPairwise(heads), sparse_type="topk", topk=3, implementation="native")(layer)
    (name, args), = fake.calls
    assert name == "propagation_topk" and args[0] == "multihead_max_low_rank_bilinear"
    assert args[1].shape == (2, 3) and args[2].shape == (2,) and args[3].shape == (2, 3, 4)
    # a smoothmax aggregate is not the library's: native mode runs the streaming form
    fake.calls.clear()
    SparsePropagation(MultiHeadPairwise(heads, aggregate="smoothmax"), sparse_type="topk", topk=3,
                      implementation="native")(layer)
    assert fake.calls == []
