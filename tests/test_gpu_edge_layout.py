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


def _layout_views(buf, B, N, k):
    """(seg_start [B, N+1], records [B*N*k, 4] as int32 words, pos [B*N*k]) of
    the edge-layout buffer: three 256-byte-aligned regions in that order."""
    def up(n):
        return (n + 255) // 256 * 256
    raw = buf.cpu()
    o_rec = up(B * (N + 1) * 4)
    o_pos = o_rec + up(B * N * k * 16)
    seg = raw[: B * (N + 1) * 4].view(torch.int32).view(B, N + 1)
    rec = raw[o_rec: o_rec + B * N * k * 16].view(torch.int32).view(-1, 4)
    pos = raw[o_pos: o_pos + B * N * k * 4].view(torch.int32)
    return seg.numpy(), rec.numpy(), pos.numpy()


@pytest.mark.parametrize("B,N,k", [
    (3, 1000, 40),    # 64-row tiles, 32-row fill chunks
    (1, 5000, 8),     # two LDS key slices of the fill
    (2, 700, 300),    # 13-row fill chunks
    (4, 4096, 32),    # the C4 tiling (256-row tiles), one batch element's worth of keys per slice
])
def test_edge_layout_is_the_stable_key_sort(dev, B, N, k):
    """The grouping the forward builds is a stable sort of the edges by key:
    segment starts are the exclusive prefix of the key degrees, each segment
    lists its edges in increasing row order, records carry (row, softsign
    coefficient, edge id) and pos maps each edge to its record."""
    import ctypes

    import numpy as np

    import jakal_net_native as jn

    print(f"layout sort: B={B} N={N} k={k}", flush=True)
    g = torch.Generator().manual_seed(9300 + k)
    D, r = 16, 8
    X = torch.randn(B, N, D, generator=g).to(dev)
    ps = torch.randn(B, N, generator=g).to(dev)
    U = (0.5 * torch.randn(r, D, generator=g)).to(dev)
    V = (0.5 * torch.randn(r, D, generator=g)).to(dev)
    w = torch.full((r,), r ** -0.5).to(dev)
    ds = torch.empty(B, N, device=dev)
    dv = torch.empty(B, N, D, device=dev)
    proj = torch.empty(B * N, 2 * r, device=dev)
    idx = torch.empty(B, N, k, device=dev, dtype=torch.int32)
    score = torch.empty(B, N, k, device=dev)
    lb = int(jn._LIB.jn_propagation_topk_layout_bytes(B, N, k))
    layout = torch.empty(lb, device=dev, dtype=torch.uint8)
    wb = int(jn._LIB.jn_propagation_topk_forward_workspace_bytes(B, N, r))
    ws = torch.empty(max(wb, 1), device=dev, dtype=torch.uint8)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rc = jn._LIB.jn_propagation_topk_forward(
        P(X), P(ps), P(X), P(U), P(V), P(w), None, B, N, D, D, r, k, 0, P(ds), P(dv), P(proj), P(idx), P(score),
        P(layout), lb, P(ws), wb, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, jn._LIB.jn_last_error().decode()
    torch.cuda.synchronize()
    seg, rec, pos = _layout_views(layout, B, N, k)
    I = idx.cpu().numpy().reshape(B, N * k)
    S = score.cpu().numpy().reshape(B, N * k)
    for b in range(B):
        keys = I[b]
        rows = np.repeat(np.arange(N), k)
        order = np.lexsort((rows, keys))  # by key, then row
        deg = np.bincount(keys, minlength=N)
        assert (seg[b, :N] == np.concatenate([[0], np.cumsum(deg)[:-1]])).all()
        assert seg[b, N] == N * k
        base = b * N * k
        got = rec[base: base + N * k]
        assert (got[:, 0] == b * N + rows[order]).all(), "records out of key/row order"
        assert (got[:, 2] == base + order).all(), "record edge ids"
        cf = S[b][order] / (1.0 + np.abs(S[b][order]))
        np.testing.assert_allclose(np.ascontiguousarray(got[:, 1]).view(np.float32), cf, rtol=1e-6, atol=0)
        want_pos = np.empty(N * k, np.int64)
        want_pos[order] = base + np.arange(N * k)
        assert (pos[base: base + N * k] == want_pos).all()
