// Fixed edge lists with low-rank scores (gfx950).
//
// Causal band (window propagation): row i of a batch element has
// `width` = min(window + 1, N) edge slots; slot e is the source
// j = i - (width - 1 - e), absent (index -1, score 0) when j < 0: the sources
// j with i - window <= j <= i, oldest first (kernel_common.py:443-456
// causal_window_mask; native_backend.py:3044-3056).
// All keys (a transition whose top-k covers every destination,
// transition.py:437-440): slot e is key e.
// Edge scores follow LowRankBilinearPairwise / LowRankBilinearRoute
// (modules.py:95-100, 435-441) with an optional temperature:
//     s[i, e] = (sum_r q[i, r] * scale[r] * key[j, r] + bias) / T.
// The edge list then feeds the same row/column kernels as top-k selection.
//
// Multi-head max aggregation (MultiHeadPairwise / MultiHeadRoute with
// aggregate="max", modules.py:259-301, 470-529; jakal_net_native.cpp:724-752,
// 889-917): the ranks split into equal head slices and
//     s[i, e] = max_h (sum_{r in h} q[i, r] * scale[r] * key[j, r] + bias[h]) / T,
// with the first winning head recorded per edge for the backward.
//
// One wavefront per query row: the scaled query row sits in LDS, lane e
// scores slot e (64 slots per pass) against its key row.  The keys of a row's
// window are the previous `width` rows, so neighbouring rows re-read the same
// band from L2.
#include "jn_internal.hpp"

namespace jakal {

// Dot product of n ranks of a (LDS) and b (global), 16-byte reads when VEC.
template <bool VEC>
__device__ __forceinline__ float rank_dot(const float* a, const float* b, int n) {
  float acc = 0.0f;
  if constexpr (VEC) {
    for (int rr = 0; rr < n; rr += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(b + rr);
      const float4 qv = *reinterpret_cast<const float4*>(a + rr);
      acc += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
    }
  } else {
    for (int rr = 0; rr < n; ++rr) acc += a[rr] * b[rr];
  }
  return acc;
}

// MH: multi-head max aggregation over a.heads rank slices of a.head_rank
// (VEC then needs head_rank % 4 == 0).  all_keys == 2 reads the edge list and
// writes only the heads (the edges of a top-k select).
template <bool VEC, bool MH>
__global__ __launch_bounds__(256) void window_scores_kernel(WindowScoreArgs a) {
  __shared__ __align__(16) float s_q[4][kMaxRank];
  const int lane = lane_id(), wave = wave_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave;
  if (row >= (int64_t)a.B * a.Nq) return;  // wave-uniform; no workgroup barrier below
  const int64_t b = row / a.Nq;
  const int i = (int)(row % a.Nq);
  float* q = s_q[wave];
  for (int rr = lane; rr < a.r; rr += kWave) q[rr] = a.q[row * a.ldq + rr] * (a.scale ? a.scale[rr] : 1.0f);
  wave_lds_sync();
  const float bias = a.bias ? a.bias[0] : 0.0f;
  const bool given = a.all_keys == 2;
  for (int e0 = 0; e0 < a.width; e0 += kWave) {
    const int e = e0 + lane;
    if (e >= a.width) break;
    const int j = given ? a.idx[row * a.width + e] : a.all_keys ? e : i - (a.width - 1 - e);
    int32_t jo = -1;
    float s = 0.0f;
    int head = 0;
    if (j >= 0) {
      const float* kr = a.key + (b * a.Nk + j) * a.ldk;
      if constexpr (MH) {
        // first head attaining the max (strictly greater replaces)
        float best = -INFINITY;
        for (int h = 0; h < a.heads; ++h) {
          const float acc = rank_dot<VEC>(q + h * a.head_rank, kr + h * a.head_rank, a.head_rank);
          const float sh = (acc + (a.bias ? a.bias[h] : 0.0f)) * a.inv_temperature;
          if (sh > best) {
            best = sh;
            head = h;
          }
        }
        s = best;
      } else {
        s = (rank_dot<VEC>(q, kr, a.r) + bias) * a.inv_temperature;
      }
      jo = j;
    }
    if (!given) {
      a.idx[row * a.width + e] = jo;
      a.score[row * a.width + e] = s;
    }
    if (MH && a.head) a.head[row * a.width + e] = (uint8_t)head;
  }
}

int launch_window_scores(const WindowScoreArgs& a, hipStream_t stream) {
  const bool mh = a.heads > 1;
  JN_REQUIRE(a.r >= 1 && a.r <= (mh ? kRegRank : kMaxRank), kUnsupported, "rank must be in [1, %d] (got %d)",
             mh ? kRegRank : kMaxRank, a.r);
  JN_REQUIRE(a.width >= 1, kInvalidArgument, "window width must be positive");
  JN_REQUIRE(a.all_keys != 1 || a.width == a.Nk, kInvalidArgument, "an all-keys edge list has one slot per key");
  JN_REQUIRE(!mh || (a.heads <= kMaxHeads && a.head_rank >= 1 && a.heads * a.head_rank == a.r), kUnsupported,
             "multi-head scores need 2..%d heads of equal rank (heads=%d, head rank=%d, rank=%d)", kMaxHeads, a.heads,
             a.head_rank, a.r);
  JN_REQUIRE(a.all_keys != 2 || mh, kInvalidArgument, "a given edge list only has heads to find");
  const int64_t rows = (int64_t)a.B * a.Nq;
  if (rows == 0) return kOk;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  const bool vec = (a.r % 4 == 0) && (!mh || a.head_rank % 4 == 0) && (a.ldk % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0);
  JN_PROFILE(mh ? "window_scores_heads_kernel" : "window_scores_kernel", stream);
  if (mh) {
    if (vec) hipLaunchKernelGGL((window_scores_kernel<true, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((window_scores_kernel<false, true>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((window_scores_kernel<true, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((window_scores_kernel<false, false>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
