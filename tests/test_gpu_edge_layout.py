"""The edge layout a top-k forward builds for its backward.

With a backward to follow, the top-k forwards group the selected edges by key
(CSR segments, edge records and each edge's record index) beside their row
pass and hand that layout to the backward, which otherwise groups the edges
itself.  The grouping depends only on the edge list and the backward runs the
same kernels on it either way, so every output and gradient must be
bit-identical with and without the forward's layout (jakal_net_native.
set_edge_layout).  Cases cover one and two column slabs, all three compress
kinds, bf16 layers, two max-aggregated heads, and an edge list of 2^20 edges,
where the forward builds the layout on its second stream.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401  (fails loudly when the library is missing)

    return torch.device("cuda:0")


def _run(dev, B, N, D, r, k, compress, dtype, heads, seed):
    import jakal_net as J
    from jakal_net import Layer

    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    state = torch.randn(B, N, generator=g).to(dev, dtype).requires_grad_(True)
    val = torch.randn(B, N, D, generator=g).to(dev, dtype).requires_grad_(True)
    layer = Layer(dim=D, num_nodes=N, state=state, val=val)
    if heads > 1:
        pair = J.MultiHeadPairwise([J.LowRankBilinearPairwise(D, r) for _ in range(heads)], aggregate="max")
    else:
        pair = J.LowRankBilinearPairwise(D, r)
    from jakal_net.compress import signed_abs_softmax, signed_entmax15
    from torch.nn import functional as F

    fn = {"softsign": F.softsign, "signed_abs_softmax": signed_abs_softmax, "signed_entmax15": signed_entmax15}
    op = J.SparsePropagation(pair, sparse_type="topk", topk=k, edge_compress_fn=fn[compress],
                             implementation="native").to(dev)
    d = op(layer)
    gs = torch.randn(d.delta_state.shape, generator=g).to(dev, d.delta_state.dtype)
    gv = torch.randn(d.delta_val.shape, generator=g).to(dev, d.delta_val.dtype)
    torch.autograd.backward([d.delta_state, d.delta_val], [gs, gv])
    out = [d.delta_state, d.delta_val, state.grad, val.grad] + [p.grad for p in op.parameters() if p.grad is not None]
    torch.cuda.synchronize()
    return [t.detach().clone() for t in out]


@pytest.mark.parametrize("B,N,D,r,k,compress,dtype,heads", [
    (2, 600, 64, 16, 12, "softsign", torch.float32, 1),             # one column slab
    (2, 700, 512, 64, 32, "softsign", torch.float32, 1),            # two column slabs
    (2, 300, 128, 32, 24, "signed_abs_softmax", torch.float32, 1),
    (2, 300, 96, 32, 40, "signed_entmax15", torch.float32, 1),
    (2, 500, 256, 32, 16, "softsign", torch.bfloat16, 1),
    (2, 400, 64, 16, 8, "softsign", torch.float32, 2),
    (4, 4096, 64, 16, 64, "softsign", torch.float32, 1),            # 2^20 edges: built on the second stream
])
def test_forward_layout_matches_backward_grouping(dev, B, N, D, r, k, compress, dtype, heads):
    import jakal_net_native as jn

    print(f"edge layout: B={B} N={N} D={D} r={r} k={k} {compress} {dtype} heads={heads}", flush=True)
    try:
        jn.set_edge_layout(True)
        with_layout = _run(dev, B, N, D, r, k, compress, dtype, heads, 9100 + k)
        jn.set_edge_layout(False)
        without = _run(dev, B, N, D, r, k, compress, dtype, heads, 9100 + k)
    finally:
        jn.set_edge_layout(True)
    assert len(with_layout) == len(without) >= 6
    for i, (a, b) in enumerate(zip(with_layout, without)):
        assert torch.equal(a, b), f"output {i} differs: max |diff| {(a.float() - b.float()).abs().max().item():.3e}"
