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
// One wavefront per query row: the scaled query row sits in LDS, lane e
// scores slot e (64 slots per pass) against its key row.  The keys of a row's
// window are the previous `width` rows, so neighbouring rows re-read the same
// band from L2.
#include "jn_internal.hpp"

namespace jakal {

template <bool VEC>
__global__ __launch_bounds__(256) void window_scores_kernel(WindowScoreArgs a) {
  __shared__ __align__(16) float s_q[4][128];
  const int lane = lane_id(), wave = wave_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave;
  if (row >= (int64_t)a.B * a.Nq) return;  // wave-uniform; no workgroup barrier below
  const int64_t b = row / a.Nq;
  const int i = (int)(row % a.Nq);
  float* q = s_q[wave];
  for (int rr = lane; rr < a.r; rr += kWave) q[rr] = a.q[row * a.ldq + rr] * (a.scale ? a.scale[rr] : 1.0f);
  wave_lds_sync();
  const float bias = a.bias ? a.bias[0] : 0.0f;
  for (int e0 = 0; e0 < a.width; e0 += kWave) {
    const int e = e0 + lane;
    if (e >= a.width) break;
    const int j = a.all_keys ? e : i - (a.width - 1 - e);
    int32_t jo = -1;
    float s = 0.0f;
    if (j >= 0) {
      const float* kr = a.key + (b * a.Nk + j) * a.ldk;
      float acc = 0.0f;
      if constexpr (VEC) {
        for (int rr = 0; rr < a.r; rr += 4) {
          const float4 kv = *reinterpret_cast<const float4*>(kr + rr);
          const float4 qv = *reinterpret_cast<const float4*>(q + rr);
          acc += qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
        }
      } else {
        for (int rr = 0; rr < a.r; ++rr) acc += q[rr] * kr[rr];
      }
      jo = j;
      s = (acc + bias) * a.inv_temperature;
    }
    a.idx[row * a.width + e] = jo;
    a.score[row * a.width + e] = s;
  }
}

int launch_window_scores(const WindowScoreArgs& a, hipStream_t stream) {
  JN_REQUIRE(a.r >= 1 && a.r <= 128, kUnsupported, "rank must be in [1, 128]");
  JN_REQUIRE(a.width >= 1, kInvalidArgument, "window width must be positive");
  JN_REQUIRE(!a.all_keys || a.width == a.Nk, kInvalidArgument, "an all-keys edge list has one slot per key");
  const int64_t rows = (int64_t)a.B * a.Nq;
  if (rows == 0) return kOk;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  const bool vec = (a.r % 4 == 0) && (a.ldk % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0);
  JN_PROFILE("window_scores_kernel", stream);
  if (vec) hipLaunchKernelGGL(window_scores_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(window_scores_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
