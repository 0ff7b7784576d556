"""HIP-graph capture of whole training steps through the operator API.

The HIP entry points only launch kernels: no device allocation (workspaces
come from the caller), no synchronisation and no memset inside the library.
A forward+backward step through jakal_net's modules with
implementation="native" can therefore be captured into one graph
(torch.cuda.CUDAGraph) -- which the reference cannot do: it sends native
calls made under capture to its PyTorch form (propagation.py:356-357,
775-776; transition.py:332-333, 660-661).

Each case captures one step, then replays it three times with other eager
GPU work and a synchronisation between replays, and requires every replay's
outputs and gradients to equal an eager run of the same step bit for bit
(every kernel on the path has a fixed reduction order).  A spy checks that
the captured step reached the HIP ops and not a PyTorch form.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _layer(g, B, N, D, dev, dtype=torch.float32):
    from jakal_net import Layer

    state = torch.randn(B, N, generator=g).to(dev, dtype).requires_grad_(True)
    val = torch.randn(B, N, D, generator=g).to(dev, dtype).requires_grad_(True)
    return Layer(dim=D, num_nodes=N, state=state, val=val)


def _case(kind, dev):
    """(modules, leaves, loss_terms) of one step."""
    import jakal_net as J

    g = torch.Generator().manual_seed(7100)
    torch.manual_seed(7100)
    B, N, D, r = 2, 256, 64, 16
    if kind == "topk_large":  # 2^20 edges: the backward forks work onto a second stream
        layer = _layer(g, 4, 4096, D, dev)
        op = J.SparsePropagation(J.LowRankBilinearPairwise(D, r), sparse_type="topk", topk=64,
                                 implementation="native").to(dev)

        def loss_terms():
            d = op(layer)
            return [d.delta_state, d.delta_val]

        return [op], [layer.state, layer.val], loss_terms
    if kind == "transition_large":  # 2^20 routes: projections and gradients on two streams
        src, dst = _layer(g, 4, 4096, D, dev), _layer(g, 4, 512, D, dev)
        op = J.SparseTransition(J.LowRankBilinearRoute(D, D, rank=r), topk=64, implementation="native").to(dev)

        def loss_terms():
            d = op.compute_delta(src, dst)
            return [d.delta_state, d.delta_val]

        return [op], [src.state, src.val, dst.state, dst.val], loss_terms
    if kind in ("topk", "window", "dense", "topk_bf16", "topk_multihead"):
        dtype = torch.bfloat16 if kind == "topk_bf16" else torch.float32
        layer = _layer(g, B, N, D, dev, dtype)
        if kind == "topk_multihead":
            pair = J.MultiHeadPairwise([J.LowRankBilinearPairwise(D, r) for _ in range(2)], aggregate="max")
        else:
            pair = J.LowRankBilinearPairwise(D, r)
        if kind == "dense":
            op = J.Propagation(pair, implementation="native")
        elif kind == "window":
            op = J.SparsePropagation(pair, sparse_type="window", window=24, implementation="native")
        else:
            op = J.SparsePropagation(pair, sparse_type="topk", topk=8, implementation="native")
        op = op.to(dev)

        def loss_terms():
            d = op(layer)
            return [d.delta_state, d.delta_val]

        return [op], [layer.state, layer.val], loss_terms
    if kind == "transition":
        src, dst = _layer(g, B, N, D, dev), _layer(g, B, 64, D, dev)
        op = J.SparseTransition(J.LowRankBilinearRoute(D, D, rank=r), topk=8, implementation="native").to(dev)

        def loss_terms():
            d = op.compute_delta(src, dst)
            return [d.delta_state, d.delta_val]

        return [op], [src.state, src.val, dst.state, dst.val], loss_terms
    raise ValueError(kind)


def _step(modules, leaves, loss_terms):
    for m in modules:
        m.zero_grad(set_to_none=True)
    for t in leaves:
        t.grad = None
    outs = loss_terms()
    weights = [torch.linspace(0.5, 1.5, t.numel(), device=t.device).view_as(t).to(t.dtype) for t in outs]
    torch.autograd.backward(outs, weights)
    return outs


def _snapshot(modules, leaves, outs):
    tensors = list(outs) + [t.grad for t in leaves]
    for m in modules:
        tensors += [p.grad for p in m.parameters() if p.requires_grad]
    return [None if t is None else t.detach().clone() for t in tensors]  # leaves the step does not reach: None


@pytest.mark.parametrize("kind", ["topk", "window", "dense", "transition", "topk_bf16", "topk_multihead", "topk_large",
                                  "transition_large"])
def test_captured_step_replays_match_eager(dev, kind, monkeypatch):
    import jakal_net_native as jn

    modules, leaves, loss_terms = _case(kind, dev)
    print(f"[graph capture] case={kind}", flush=True)
    eager = _snapshot(modules, leaves, _step(modules, leaves, loss_terms))
    torch.cuda.synchronize()

    # warm up on a side stream (default priority), then capture one step
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            _step(modules, leaves, loss_terms)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    calls = []
    for name in ("propagation_topk", "propagation_window", "propagation_dense", "transition_pairwise_topk"):
        real = getattr(jn, name)

        def spy(*a, _real=real, _name=name, **k):
            calls.append(_name)
            return _real(*a, **k)

        monkeypatch.setattr(jn, name, spy)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _step(modules, leaves, loss_terms)
    monkeypatch.undo()
    assert calls, "the captured step did not reach a HIP op"
    captured = lambda: _snapshot(modules, leaves, outs)  # noqa: E731

    # other eager GPU work between replays: a second eager step of a fresh case
    other_modules, other_leaves, other_terms = _case("topk" if kind != "topk" else "window", dev)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = captured()
        assert len(got) == len(eager)
        for i, (x, y) in enumerate(zip(got, eager)):
            assert (x is None) == (y is None), f"replay {rep}: tensor {i} reached in one run only"
            if x is None:
                continue
            assert x.shape == y.shape and x.dtype == y.dtype
            assert torch.equal(x, y), f"replay {rep}: tensor {i} differs (max abs {float((x - y).abs().max()):.3e})"
        _step(other_modules, other_leaves, other_terms)
        torch.cuda.synchronize()
