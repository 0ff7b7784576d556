// Exact top-k over whole score rows (gfx950), for the selects the register
// and LDS kernels of jn_select.hip do not take: k above 64 (up to
// kSelectLargeMaxK), k equal to the key count, or more than 65,535 keys per
// batch element.  The reference's composite op takes any k
// (native/jakal_net_native.cpp:6399-6424: blockwise scores, then torch.topk).
//
// Rows are scored in blocks: a batched fp32 MFMA GEMM writes the low-rank
// scores q_i . (scale * k_j) of as many query rows as the select workspace
// holds, then one workgroup per row finds its k best:
//   1. a radix select over order-preserving uint32 keys of
//      s = (score + bias) / T (four 8-bit passes, LDS histograms) finds the
//      k-th largest key and how many entries tie with it;
//   2. one pass over the row in index order collects every entry above it and
//      the lowest-index ties, so the choice at the k-th value goes toward the
//      lower index, as in the register select;
//   3. a bitonic sort in LDS orders the k entries by descending score,
//      ascending index, and the row is written.
// Score arithmetic is fp32 MFMA (as select mode 1), whatever the layer dtype.
// Max-aggregated multi-head scores (heads > 1) run one GEMM per head over its
// rank slice, each folding its scores plus its bias into the block's running
// max (ties keep the earlier head), so any number of heads, keys and k <=
// kSelectLargeMaxK is taken.
#include <algorithm>
#include "jn_internal.hpp"

namespace jakal {

namespace {

// Monotone map float -> uint32 with larger floats to smaller keys (ascending
// key order = descending score); -0 and +0 map together.
__device__ __forceinline__ uint32_t desc_key(float s) {
  const uint32_t u = __float_as_uint(s + 0.0f);
  return ~((u & 0x80000000u) ? ~u : (u | 0x80000000u));
}

__device__ __forceinline__ bool before(float as, int ai, float bs, int bi) {
  return as > bs || (as == bs && ai < bi);
}

__global__ __launch_bounds__(256) void topk_rows_kernel(const float* S, int64_t lds, int Nk, int k,
                                                        const float* bias_ptr, float inv_temp, int64_t out_row0,
                                                        int32_t* out_idx, float* out_score) {
  __shared__ int hist[256];
  __shared__ int s_bin, s_below;
  __shared__ int s_less, s_ties;
  __shared__ int wave_ties[4];
  __shared__ float cs[kSelectLargeMaxK];
  __shared__ int ci[kSelectLargeMaxK];
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const float* row = S + (int64_t)blockIdx.x * lds;
  const float bias = bias_ptr ? bias_ptr[0] : 0.0f;
  auto score_at = [&](int j) { return (row[j] + bias) * inv_temp; };

  // 1. radix select: the k-th smallest key (the k-th largest score)
  uint32_t prefix = 0, mask = 0;
  int need = k;  // entries still to take at or below the current prefix
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;
    __syncthreads();
    for (int j = tid; j < Nk; j += 256) {
      const uint32_t u = desc_key(score_at(j));
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1);
    }
    __syncthreads();
    if (wave == 0) {
      // inclusive prefix over the 256 bins: lane l holds bins 4l..4l+3
      const int h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
      const int own = h0 + h1 + h2 + h3;
      int incl = own;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __builtin_amdgcn_ds_bpermute(((lane - o) & 63) << 2, incl);
        if (lane >= o) incl += y;
      }
      const int excl = incl - own;
      // the bin where the cumulative count first reaches `need` (exactly one lane)
      if (excl < need && incl >= need) {
        int c = excl, b = 4 * lane;
        if (c + h0 >= need) b = 4 * lane;
        else if ((c += h0) + h1 >= need) b = 4 * lane + 1;
        else if ((c += h1) + h2 >= need) b = 4 * lane + 2;
        else { c += h2; b = 4 * lane + 3; }
        s_bin = b;
        s_below = c;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)s_bin << shift;
    mask |= 0xFFu << shift;
    need -= s_below;
    __syncthreads();  // s_bin / s_below are rewritten by the next pass
  }
  // `prefix` is the k-th key; `need` of its ties are taken, k - need entries lie below it

  // 2. collect in index order: entries below the key anywhere in [0, k - need),
  //    ties at [k - need, k) by their rank in index order
  if (tid == 0) {
    s_less = 0;
    s_ties = 0;
  }
  __syncthreads();
  const int n_less = k - need;
  for (int base = 0; base < Nk; base += 256) {
    const int j = base + tid;
    const float s = j < Nk ? score_at(j) : 0.0f;
    const uint32_t u = j < Nk ? desc_key(s) : 0xFFFFFFFFu;
    const bool less = j < Nk && u < prefix;
    const bool tie = j < Nk && u == prefix;
    if (less) {
      const int slot = atomicAdd(&s_less, 1);
      cs[slot] = s;
      ci[slot] = j;
    }
    const uint64_t tb = __ballot(tie);
    if (lane == 0) wave_ties[wave] = __popcll(tb);
    __syncthreads();
    int rank = s_ties + __popcll(tb & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) rank += wave_ties[w];
    if (tie && rank < need) {
      cs[n_less + rank] = s;
      ci[n_less + rank] = j;
    }
    __syncthreads();
    if (tid == 0) s_ties += wave_ties[0] + wave_ties[1] + wave_ties[2] + wave_ties[3];
    __syncthreads();
  }

  // 3. bitonic sort of the k entries (padded to a power of two) into
  //    descending score, ascending index
  int n = 1;
  while (n < k) n <<= 1;
  for (int x = k + tid; x < n; x += 256) {
    cs[x] = -INFINITY;
    ci[x] = 0x7fffffff;
  }
  __syncthreads();
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int x = tid; x < n / 2; x += 256) {
        const int lo = 2 * x - (x & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;  // this run sorts "before" first
        const float a = cs[lo], b = cs[hi];
        const int ia = ci[lo], ib = ci[hi];
        if (before(b, ib, a, ia) == desc) {
          cs[lo] = b; ci[lo] = ib;
          cs[hi] = a; ci[hi] = ia;
        }
      }
      __syncthreads();
    }
  }
  const int64_t orow = out_row0 + blockIdx.x;
  for (int e = tid; e < k; e += 256) {
    out_idx[orow * k + e] = ci[e];
    out_score[orow * k + e] = cs[e];
  }
}

}  // namespace

int launch_topk_select_large(const SelectArgs& a, hipStream_t stream) {
  JN_REQUIRE(a.k >= 1 && a.k <= kSelectLargeMaxK, kUnsupported, "top-k select supports 1 <= k <= %d (got %d)",
             kSelectLargeMaxK, a.k);
  JN_REQUIRE(a.k <= a.Nk, kInvalidArgument, "top-k select needs k <= key count (k=%d, Nk=%d)", a.k, a.Nk);
  const bool mh = a.heads > 1;
  JN_REQUIRE(!mh || (a.heads <= kMaxHeads && a.head_rank >= 1 && a.heads * a.head_rank == a.r), kUnsupported,
             "multi-head select: %d heads of rank %d (rank %d)", a.heads, a.head_rank, a.r);
  JN_REQUIRE(a.temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  JN_REQUIRE(a.r >= 1 && a.Nq >= 1 && a.B >= 1, kInvalidArgument, "empty select");
  // score rows per block: as many as the select's own workspace size holds
  // (the register select's split-key scratch for this shape), whatever a
  // larger buffer the caller passes, so the blocks -- and with them the GEMM
  // tiles and every score bit -- depend on the shape only
  const size_t own = mh ? select_workspace_bytes_heads(a.B, a.Nk, a.head_rank, a.heads)
                        : select_workspace_bytes(a.B, a.Nk, a.r);
  const size_t usable = std::min(own, a.ws_bytes);
  const int64_t rows_fit = a.ws ? (int64_t)(usable / sizeof(float)) / a.Nk : 0;
  JN_REQUIRE(rows_fit >= 1, kWorkspaceTooSmall, "select workspace holds no score row (%zu bytes for %d keys)",
             a.ws_bytes, a.Nk);
  float* S = static_cast<float*>(a.ws);
  const float inv_temp = 1.0f / a.temperature;
  auto block = [&](int b0, int nb, int r0, int nr) -> int {
    // scores of rows [r0, r0 + nr) of batch elements [b0, b0 + nb): the scale
    // multiplies the query side (the same product as scaling the keys)
    const int heads = mh ? a.heads : 1, rh = mh ? a.head_rank : a.r;
    for (int h = 0; h < heads; ++h) {
      BatchedGemm m{};
      m.A = a.q + (int64_t)b0 * a.q_batch_stride + (int64_t)r0 * a.ldq + h * rh;
      m.lda = a.ldq; m.a_bs = a.q_batch_stride; m.a_kcontig = true;
      m.B = a.key + (int64_t)b0 * a.k_batch_stride + h * rh;
      m.ldb = a.ldk; m.b_bs = a.k_batch_stride; m.b_kcontig = true;
      m.C = S; m.ldc = a.Nk; m.c_bs = (int64_t)nr * a.Nk;
      m.a_kscale = a.scale ? a.scale + h * rh : nullptr;
      m.M = nr; m.N = a.Nk; m.K = rh; m.batch = nb;
      if (mh) {  // running max over the heads, each with its own bias
        m.fold = h == 0 ? 1 : 2; m.fold_head = h; m.fold_bias = a.bias ? a.bias + h : nullptr;
      }
      const int rc = gemm_batched(m, kGemmSelectScores, stream);
      if (rc) return rc;
    }
    const int64_t rows = (int64_t)nb * nr;
    JN_PROFILE("topk_rows_kernel", stream);
    hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)rows), dim3(256), 0, stream, S, (int64_t)a.Nk, a.Nk, a.k,
                       mh ? nullptr : a.bias, inv_temp, (int64_t)b0 * a.Nq + r0, a.out_idx, a.out_score);
    JN_LAUNCH_CHECK();
    return kOk;
  };
  int rc;
  if (rows_fit >= a.Nq) {  // whole batch elements per block
    const int G = (int)std::min<int64_t>(a.B, rows_fit / a.Nq);
    for (int b0 = 0; b0 < a.B; b0 += G) {
      rc = block(b0, std::min(G, a.B - b0), 0, a.Nq);
      if (rc) return rc;
    }
  } else {  // blocks of rows of one batch element
    const int R = (int)rows_fit;
    for (int b = 0; b < a.B; ++b)
      for (int r0 = 0; r0 < a.Nq; r0 += R) {
        rc = block(b, 1, r0, std::min(R, a.Nq - r0));
        if (rc) return rc;
      }
  }
  return kOk;
}

}  // namespace jakal
