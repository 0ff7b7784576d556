"""The Progressive-B query-block step (jakal_net.progressive) with every
operator on the HIP library, on a reduced configuration.

* the logits and loss of the native step (fp32) against the composition of
  oracle calls (tests/progressive_oracle.py, float64 numpy);
* the gradient of every parameter against the same step run through the
  operators' implementation="reference" backend in float64 on the CPU (the
  reference backend is pinned to the oracle by tests/test_api_cpu.py), each
  within the literal fp32 tolerance or twice the error of that backend run in
  fp32 on the GPU (tests/parity.py);
* the step under bf16 autocast (bf16 activations, fp32 master weights, as
  BASELINE config 5 runs) against the float64 logits at the bf16 tolerance.

Reference composition: scripts/progressive_b_example.py:282-292, 1011-1024,
1108-1323, 1691-1719, 1857-1908, 1957-2021, 2059-2152.
"""

import numpy as np
import pytest
import torch

import progressive_oracle as PO
from parity import check, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _cfg():
    from jakal_net.progressive import ProgressiveBConfig

    return ProgressiveBConfig(vocab=97, dim=32, prefix=48, query=8, rank=8, topk=4, s_window=6, warmup=1,
                              blocks=2, expanded=24, compressed=8, refine=1, query_refine=2)


def _models_and_batch(seed=21):
    from jakal_net.progressive import ProgressiveBStep

    cfg = _cfg()
    torch.manual_seed(seed)
    native = ProgressiveBStep(cfg, implementation="native")
    g = torch.Generator().manual_seed(seed + 1)
    prefix = torch.randint(0, cfg.vocab - 1, (2, cfg.prefix), generator=g)
    target = torch.randint(0, cfg.vocab - 1, (2, cfg.query), generator=g)
    return cfg, native, prefix, target


def _unused(model):
    """Parameters outside the loss, as in the reference's block: every block's
    expanded-slot state (a transition's destination state enters no delta, and
    B_exp is replaced by the expand delta), the compressed-slot templates of the
    blocks after the first (B_cmp is carried from there), and the last block's
    compress and S -> B_cmp routes (that B_cmp feeds only a next block; with one
    block its shared top-k pairwise module too).  The state head is outside the
    loss too: the sequence state it starts is replaced by the B_exp -> S delta
    before any operator reads it, and a query slot's state only enters a
    transition as its destination."""
    n = model.cfg.blocks
    out = {"state_init.weight", "state_init.bias"}
    for name, _ in model.named_parameters():
        parts = name.split(".")
        if parts[0] != "blocks":
            continue
        i, rest = int(parts[1]), ".".join(parts[2:])
        if rest == "exp_slot_state" or (i > 0 and rest.startswith("cmp_slot_")):
            out.add(name)
        elif i == n - 1 and rest.startswith(("compress.", "s_to_b.") + (("cmp_prop.",) if n == 1 else ())):
            out.add(name)
    return out


def _grads(model, prefix, target):
    model.zero_grad(set_to_none=True)
    loss = model(prefix, target)
    loss.backward()
    return float(loss.detach()), {n: p.grad for n, p in model.named_parameters() if p.grad is not None}


def test_progressive_step_native_matches_oracle_and_reference():
    from jakal_net.progressive import ProgressiveBStep

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    dev = torch.device("cuda:0")
    cfg, native, prefix, target = _models_and_batch()
    ref64 = ProgressiveBStep(cfg, implementation="reference").double()
    ref64.load_state_dict(native.state_dict())
    ref32 = ProgressiveBStep(cfg, implementation="reference").to(dev)
    ref32.load_state_dict(native.state_dict())
    native = native.to(dev)

    with torch.no_grad():
        logits = native.query_logits(native.encode_prefix(prefix.to(dev)), target.to(dev))
        logits32 = ref32.query_logits(ref32.encode_prefix(prefix.to(dev)), target.to(dev))
    params = {k: v.detach().double().cpu().numpy() for k, v in native.state_dict().items()}
    want = PO.progressive_logits(params, cfg, prefix.numpy(), target.numpy())
    check("C5 logits vs oracle composition", logits, want, logits32)

    loss_n, g_n = _grads(native, prefix.to(dev), target.to(dev))
    loss_64, g_64 = _grads(ref64, prefix, target)
    loss_32, g_32 = _grads(ref32, prefix.to(dev), target.to(dev))
    check("C5 loss", np.array([loss_n]), np.array([PO.cross_entropy(want, target.numpy())]))
    assert abs(loss_64 - PO.cross_entropy(want, target.numpy())) < 1e-9
    assert set(g_n) == set(g_64), "the native and reference steps differ in which parameters get gradients"
    assert _unused(native) == {n for n, _ in native.named_parameters()} - set(g_n)
    for name in sorted(g_64):
        check(f"C5 grad {name}", g_n[name], g_64[name], g_32[name])


def test_progressive_step_bf16_autocast():
    from jakal_net.progressive import ProgressiveBStep

    dev = torch.device("cuda:0")
    cfg, native, prefix, target = _models_and_batch(seed=31)
    ref64 = ProgressiveBStep(cfg, implementation="reference").double()
    ref64.load_state_dict(native.state_dict())
    native = native.to(dev)
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        loss = native(prefix.to(dev), target.to(dev))
        logits = native.query_logits(native.encode_prefix(prefix.to(dev)), target.to(dev))
    loss.backward()
    got = {n for n, p in native.named_parameters() if p.grad is not None}
    assert got == {n for n, _ in native.named_parameters()} - _unused(native)
    assert all(bool(torch.isfinite(p.grad).all()) for p in native.parameters() if p.grad is not None)
    with torch.no_grad():
        want = ref64.query_logits(ref64.encode_prefix(prefix), target)
    # the logits carry the bf16 rounding of the linear layers' inputs and weights
    # (fp32 accumulation): within the bf16 tolerance 2e-2, norm-wise
    err = float(np.abs(np64(logits) - np64(want)).max())
    scale = float(np.abs(np64(want)).max())
    print(f"C5 bf16 autocast: max|logits - f64| {err:.3e} of max|logit| {scale:.3e}", flush=True)
    assert err <= 2e-2 * scale
    want_loss = float(ref64(prefix, target).detach())
    assert abs(float(loss) - want_loss) <= 2e-2 * abs(want_loss)


@pytest.mark.parametrize("fused", [False, True])
def test_progressive_step_graph_replay_matches_eager(dev, fused):
    """The whole training step (forward, backward, AdamW with capturable state
    -- the multi-tensor or the fused update -- bf16 autocast without its cast
    cache) captured into one HIP graph: from the same parameters and optimizer
    state, every replay gives the eager step's loss and updated parameters bit
    for bit, with other eager GPU work between replays."""
    cfg, model, prefix, target = _models_and_batch(seed=31)
    model = model.to(dev)
    prefix, target = prefix.to(dev), target.to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, capturable=True, fused=fused)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16, cache_enabled=False):
            loss = model(prefix, target)
        loss.backward()
        opt.step()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    tensors = [p.data for p in model.parameters()]
    for st in opt.state.values():
        tensors += [v for v in st.values() if torch.is_tensor(v)]
    snapshot = [t.clone() for t in tensors]

    def restore():
        for t, s in zip(tensors, snapshot):
            t.copy_(s)
        torch.cuda.synchronize()

    want_loss = step().detach().clone()
    want = [p.data.clone() for p in model.parameters()]
    restore()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        loss = step()
    for rep in range(3):
        restore()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(loss, want_loss), f"replay {rep}: loss {float(loss)} != {float(want_loss)}"
        for (name, p), w in zip(model.named_parameters(), want):
            assert torch.equal(p.data, w), f"replay {rep}: {name} differs by {float((p.data - w).abs().max()):.3e}"
        torch.randn(1 << 20, device=dev).sum()  # other eager work between replays
        torch.cuda.synchronize()


def test_progressive_step_at_the_c5_size(dev):
    """BASELINE config 5 at its stated size (vocab 16384, d 512, prefix 512,
    64 query slots, 4 joint blocks, B_exp 256, B_cmp 64, top-k 16, rank 64,
    batch 16) under bf16 autocast with a fused AdamW update: finite loss and
    gradients on every parameter the loss reaches, the update applied to
    every parameter with a non-zero gradient, and the step repeated from the
    same parameters and optimizer state giving the same loss and update bit
    for bit (the library sums in fixed orders).  The graph-capture check runs
    at the reduced size above; bench.py captures this size itself."""
    from jakal_net.progressive import ProgressiveBConfig, ProgressiveBStep

    cfg = ProgressiveBConfig(vocab=16384, dim=512, prefix=512, query=64, rank=64, topk=16, blocks=4, expanded=256,
                             compressed=64, s_window=32)
    torch.manual_seed(1005)
    model = ProgressiveBStep(cfg, implementation="native").to(dev)
    g = torch.Generator().manual_seed(1005)
    prefix = torch.randint(0, cfg.vocab - 1, (16, cfg.prefix), generator=g).to(dev)
    target = torch.randint(0, cfg.vocab - 1, (16, cfg.query), generator=g).to(dev)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, fused=True)

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = model(prefix, target)
        loss.backward()
        opt.step()
        return loss.detach()

    step()  # optimizer state exists from here on
    torch.cuda.synchronize()
    tensors = [p.data for p in model.parameters()]
    for st in opt.state.values():
        tensors += [v for v in st.values() if torch.is_tensor(v)]
    snapshot = [t.clone() for t in tensors]
    before = [p.detach().clone() for p in model.parameters()]
    loss = step()
    torch.cuda.synchronize()
    assert bool(torch.isfinite(loss)), f"loss {float(loss)}"
    # a freshly initialised head over 16384 tokens starts near log(vocab)
    assert abs(float(loss) - float(np.log(cfg.vocab))) < 2.0, float(loss)
    reached = {n for n, p in model.named_parameters() if p.grad is not None}
    assert reached == {n for n, _ in model.named_parameters()} - _unused(model)
    for n, p in model.named_parameters():
        if p.grad is not None:
            assert bool(torch.isfinite(p.grad).all()), f"non-finite gradient in {n}"
    # every parameter with a non-zero gradient moved (zero-initialised ones whose
    # gradient is exactly 0, e.g. the bias of one-sign signed routes, stay put)
    stuck = [n for (n, p), b in zip(model.named_parameters(), before)
             if p.grad is not None and bool((p.grad != 0).any()) and torch.equal(p.detach(), b)]
    assert not stuck, f"parameters with gradients that the update did not change: {stuck}"
    want = [p.data.clone() for p in model.parameters()]
    for t, v in zip(tensors, snapshot):
        t.copy_(v)
    again = step()
    torch.cuda.synchronize()
    assert torch.equal(again, loss), f"repeated step: loss {float(again)} != {float(loss)}"
    for (name, p), w in zip(model.named_parameters(), want):
        assert torch.equal(p.data, w), f"repeated step: {name} differs by {float((p.data - w).abs().max()):.3e}"
