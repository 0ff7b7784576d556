"""Both score arithmetics of the top-k select against the oracle.

The per-op tests run the default split-fp16 select (fp16 MFMAs over two-term
fp16 splits of power-of-two-scaled operands, fp32 accumulation).  These tests
cover the fp32-MFMA select (jn_set_select_mode(1)) and each split-fp16 kernel
on its own (per-wave streaming, mode 2; LDS-staged cooperative, mode 4;
key-split per-wave, mode 5; mode 0 on the register kernels only, mode 6) on
the same select, top-k propagation and transition cases, check that the split
kernels pick identical entries and values up to the C4 shape, and the split path on what its scaling has
to survive: key and query rows whose magnitudes span many octaves, all-zero
rows, ranks that are not a multiple of the 32-rank K-step, and bias and
temperature on the unscaled-domain path.  Tolerances are the hot path's
(index parity where the k-th/(k+1)-th gap exceeds 1e-5, values rtol 1e-4 /
atol 1e-5).
"""

import numpy as np
import pytest
import torch

import test_gpu_topk as TT
import test_gpu_transition as TR
from parity import check_selection

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import jakal_net_native  # noqa: F401

    return torch.device("cuda:0")


def _mode_value(name):
    import jakal_net_native as jn

    return {"split_f16": jn.SELECT_SPLIT_F16, "f32": jn.SELECT_F32, "split_wave": jn.SELECT_SPLIT_F16_WAVE,
            "split_coop4": jn.SELECT_SPLIT_F16_COOP4, "split_keysplit": jn.SELECT_SPLIT_F16_KEYSPLIT,
            "split_register": jn.SELECT_SPLIT_F16_REGISTER}[name]


@pytest.fixture(params=["split_f16", "f32", "split_wave", "split_coop4", "split_keysplit", "split_register"])
def mode(request):
    import jakal_net_native as jn

    jn.set_select_mode(_mode_value(request.param))
    yield request.param
    jn.set_select_mode(jn.SELECT_SPLIT_F16)


@pytest.fixture
def f32_mode():
    import jakal_net_native as jn

    jn.set_select_mode(jn.SELECT_F32)
    yield
    jn.set_select_mode(jn.SELECT_SPLIT_F16)


def _select(dev, q, key, scale, bias, scale_on_query, temp, k):
    import jakal_net_native as jn

    idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), None if scale is None else scale.to(dev),
                                         None if bias is None else bias.to(dev), scale_on_query, temp, k)
    sq = q.double().numpy() * (scale.double().numpy() if (scale is not None and scale_on_query) else 1.0)
    sk = key.double().numpy() * (scale.double().numpy() if (scale is not None and not scale_on_query) else 1.0)
    ref = (sq @ np.swapaxes(sk, 1, 2) + (0.0 if bias is None else float(bias))) / temp
    return idx.cpu().numpy(), score.cpu().numpy(), ref


@pytest.mark.parametrize("r,k,Nq,Nk", [(64, 32, 200, 333), (20, 8, 130, 1024), (100, 5, 64, 97), (64, 64, 257, 2000),
                                       (128, 16, 64, 700), (33, 33, 70, 500)])
@pytest.mark.parametrize("spread", [0.3, 1.0])
def test_select_both_modes(dev, mode, r, k, Nq, Nk, spread):
    """spread 0.3: O(1) scores, the regime of the absolute 1e-5 index and k-th
    score checks.  spread 1.0: N(0,1) operands, scores up to |s| ~ 40, where one
    fp32 ulp of a score is already ~4e-6 and an fp32 rank-r sum is off by up
    to ~r ulps; there the gap rule and the score checks are applied relative
    to each row's largest |score| (1e-5 of it)."""
    g = torch.Generator().manual_seed(300 + r + k)
    q = torch.randn(2, Nq, r, generator=g) * spread
    key = torch.randn(2, Nk, r, generator=g) * spread
    scale = torch.rand(r, generator=g) + 0.5
    for scale_on_query, temp, bias in ((False, 1.0, None), (True, 1.7, torch.tensor(0.25)),
                                       (False, 1.0, torch.tensor(-0.5))):
        idx, score, ref = _select(dev, q, key, scale, bias, scale_on_query, temp, k)
        if spread == 1.0:
            row = np.maximum(np.abs(ref).max(-1, keepdims=True), 1.0)
            check_selection(idx, score / row, ref / row, k)
        else:
            check_selection(idx, score, ref, k)


@pytest.mark.parametrize("r,k,B,Nq,Nk", [(64, 64, 2, 100, 65), (64, 64, 3, 50, 1024), (1, 4, 2, 33, 512),
                                         (3, 16, 2, 40, 513), (127, 20, 1, 17, 300), (128, 64, 2, 64, 700),
                                         (8, 1, 4, 16, 2)])
def test_small_key_select_matches_oracle(dev, r, k, B, Nq, Nk):
    """Rows of at most 1024 keys take the small-key select in the default
    mode: every key's score is kept in LDS (512- and 1024-key tiles, so the
    513-key case is the first of the larger tile) and each row is
    radix-selected.  k = 64 against 65 keys leaves one key out of every row; a
    rank of 1 or 3 runs the rank loop's tail alone; Nq off the 16-row tile
    leaves a partial last tile.  Checked against the oracle on the three
    scale / bias / temperature placements, and against the register kernels
    (mode 6) for identical index sets where the k-th/(k+1)-th gap is clear."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(8100 + r + k + Nk)
    q = torch.randn(B, Nq, r, generator=g) * 0.5
    key = torch.randn(B, Nk, r, generator=g) * 0.5
    scale = torch.rand(r, generator=g) + 0.5
    for scale_on_query, temp, bias in ((False, 1.0, None), (True, 1.7, torch.tensor(0.25)),
                                       (False, 0.6, torch.tensor(-0.5))):
        idx, score, ref = _select(dev, q, key, scale, bias, scale_on_query, temp, k)
        check_selection(idx, score, ref, k)
        try:
            jn.set_select_mode(jn.SELECT_SPLIT_F16_REGISTER)
            idx6, score6, _ = _select(dev, q, key, scale, bias, scale_on_query, temp, k)
        finally:
            jn.set_select_mode(jn.SELECT_SPLIT_F16)
        srt = np.sort(ref, axis=-1)[..., ::-1]
        clear = (srt[..., k - 1] - srt[..., k]) > 1e-4 if k < Nk else np.ones(srt.shape[:-1], bool)
        same = np.sort(idx, -1) == np.sort(idx6, -1)
        assert same[clear].all()
        assert np.abs(score - score6)[clear].max() < 1e-5 * max(1.0, np.abs(ref).max())


def test_small_key_select_ties_keep_lowest_index(dev):
    """Equal scores across the k-th boundary: the radix select's tie rule keeps
    the lowest key indices, like the register kernels, and emits them in key
    order within each run of equal scores."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(8200)
    key = torch.randn(2, 600, 16, generator=g)
    key[:, 7] *= 3.0  # |key 7|^2 ~ 144, far above any other key's score against it
    key[:, 100:400] = key[:, 7:8]  # 300 copies of key 7
    q = key[:, 7:8].repeat(1, 40, 1) + 0.0
    idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, 50)
    idx = idx.cpu()
    ref = (q.double() @ key.double().transpose(1, 2))
    top = ref.max(-1).values
    # every row's winners: key 7 and keys 100..148, all of the tied maximum
    expect = torch.cat([torch.tensor([7]), torch.arange(100, 149)]).to(torch.int32)
    tied = (ref == top[..., None]).sum(-1)
    assert bool((tied >= 50).all())
    assert torch.equal(idx, expect.expand_as(idx))


@pytest.mark.parametrize("Nk", [200, 2100])
def test_select_ties_both_modes(dev, mode, Nk):
    import jakal_net_native as jn

    q = torch.randn(1, 64, 8)
    key = torch.ones(1, Nk, 8)
    idx, _ = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, 5)
    assert (idx.cpu() == torch.arange(5, dtype=torch.int32)).all()


def test_select_wide_row_magnitudes(dev, mode):
    """Key rows spread over 2^-20 .. 2^20 and query rows over 2^-30 .. 2^30
    (each batch element gets its own key exponent, each query row its own);
    some query and key rows are all zero."""
    g = torch.Generator().manual_seed(4242)
    B, Nq, Nk, r, k = 2, 96, 1500, 64, 16
    q = torch.randn(B, Nq, r, generator=g) * torch.pow(2.0, torch.randint(-30, 31, (B, Nq, 1), generator=g).float())
    key = torch.randn(B, Nk, r, generator=g) * torch.pow(2.0, torch.randint(-20, 21, (B, Nk, 1), generator=g).float())
    key[1] *= 2.0 ** 40  # a batch element on another scale altogether
    q[0, 5] = 0.0
    key[0, 100:140] = 0.0
    idx, score, ref = _select(dev, q, key, None, None, False, 1.0, k)
    # relative tolerances per row: scores of a row live on that row's scale
    scale = np.abs(ref).max(-1, keepdims=True)
    scale[scale == 0] = 1.0
    check_selection(idx, score / scale, ref / scale, k)


def test_split_scores_track_f32_scores(dev):
    """The split path's selected scores agree with the fp32-MFMA path's to well
    within the parity tolerance."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(99)
    q = torch.randn(2, 128, 64, generator=g)
    key = torch.randn(2, 4096, 64, generator=g)
    outs = {}
    try:
        for m in (jn.SELECT_SPLIT_F16, jn.SELECT_F32):
            jn.set_select_mode(m)
            outs[m] = jn.low_rank_topk_select(q.to(dev), key.to(dev), None, None, False, 1.0, 32)
    finally:
        jn.set_select_mode(jn.SELECT_SPLIT_F16)
    ref = (q.double().numpy() @ np.swapaxes(key.double().numpy(), 1, 2))
    for m, (idx, score) in outs.items():
        picked = np.take_along_axis(ref, idx.cpu().numpy(), axis=-1)
        rel = np.abs(score.cpu().numpy() - picked).max() / np.abs(ref).max()
        assert rel < 5e-6, f"mode {m}: relative score error {rel:.2e}"


@pytest.mark.parametrize("compress", ["softsign", "signed_entmax15"])
def test_propagation_topk_f32_mode(dev, f32_mode, compress):
    TT.test_propagation_topk_forward_backward_matches_oracle(dev, compress, True, 8)


def test_transition_f32_mode(dev, f32_mode):
    TR.test_transition_forward_backward_matches_oracle(dev, "softmax", 1.7)


@pytest.mark.parametrize("r,k,B,Nq,Nk,dominant", [(64, 32, 16, 4096, 4096, False), (64, 64, 2, 700, 3001, False),
                                                  (32, 7, 3, 300, 5000, False), (17, 16, 1, 129, 48, False),
                                                  (64, 32, 2, 256, 4000, True), (64, 16, 8, 1024, 256, False),
                                                  (64, 16, 8, 256, 1024, False), (100, 12, 2, 77, 1000, False),
                                                  (64, 16, 2, 300, 2000, True)])
def test_split_kernels_agree(dev, r, k, B, Nq, Nk, dominant):
    """The per-wave, the cooperative and (k <= 16) the key-split kernels
    compute every score with the same MFMA sequence and keep the k best by the
    same rule, so their outputs are bit-identical (the C4 and C3 shapes
    included); the others merge at other chunks or over key quarters, which
    must not change the result."""
    import jakal_net_native as jn

    g = torch.Generator().manual_seed(7000 + r + k + Nk)
    q = torch.randn(B, Nq, r, generator=g)
    key = torch.randn(B, Nk, r, generator=g)
    key = key / key.norm(dim=-1, keepdim=True)  # many close scores, as in C4
    if dominant:  # a few keys win every row late in the scan: merges with many ties
        key[:, -40:] = key[:, -40:] * 0 + key[:, -40:-39]
    scale = torch.rand(r, generator=g) + 0.5
    out = {}
    try:
        for m in (jn.SELECT_SPLIT_F16_WAVE, jn.SELECT_SPLIT_F16_COOP4, jn.SELECT_SPLIT_F16_KEYSPLIT):
            jn.set_select_mode(m)
            idx, score = jn.low_rank_topk_select(q.to(dev), key.to(dev), scale.to(dev), None, False, 1.0, k)
            out[m] = (idx.cpu(), score.cpu())
    finally:
        jn.set_select_mode(jn.SELECT_SPLIT_F16)
    wi, ws = out[jn.SELECT_SPLIT_F16_WAVE]
    for m in (jn.SELECT_SPLIT_F16_COOP4, jn.SELECT_SPLIT_F16_KEYSPLIT):
        ci, cs = out[m]
        assert torch.equal(wi, ci)
        assert torch.equal(ws, cs)
    # and the result is a top-k: sorted, in range, no repeats
    assert bool((ws[..., :-1] >= ws[..., 1:]).all())
    assert int(wi.min()) >= 0 and int(wi.max()) < Nk
    srt = wi.sort(dim=-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all())
