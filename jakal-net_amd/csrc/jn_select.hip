// Low-rank pairwise scoring fused with per-row top-k selection (gfx950).
//
// For every query row i of a batch element this kernel computes
//     s[i, j] = ((sum_r q[i,r] * c_q[r] * key[j,r] * c_k[r]) + bias) / T
// for all key rows j, and keeps the k best (j, s) pairs, ties toward the lower
// key index.  No score matrix is written anywhere: score tiles live in MFMA
// accumulators, candidates in LDS.
//
// Reference semantics:
//   * propagation: LowRankBilinearPairwise (modules.py:95-100), query = target
//     projection, key = source projection scaled by the normalised weight,
//     top-k over all sources (kernel_common.py:426-440, propagation.py:471).
//   * transition: LowRankBilinearRoute (modules.py:435-441) / pairwise route
//     logits (jakal_net_native.cpp:874-1009): query = source projection scaled
//     by the raw weight, key = destination projection, bias then /temperature,
//     top-k per source over destinations (transition.py:439-444).
//
// Layout of one workgroup (256 threads = 4 waves):
//   * 64 query rows per workgroup, 16 per wave.  A wave keeps the query
//     fragment of its 16 rows in VGPRs for the whole kernel (B operand of
//     v_mfma_f32_16x16x4f32; lane l owns query row l%16, rank slice l/16).
//   * Keys stream through LDS in chunks of 32 rows (two 16-row MFMA tiles,
//     A operand), double buffered, one workgroup barrier per chunk.
//   * After a chunk, lane l holds 8 scores of query row l%16.  Each is compared
//     against the row's current k-th best (theta); survivors are appended to a
//     per-row candidate buffer in LDS.  When a row has >= 32 waiting candidates
//     (or at the end) the wave merges them into the row's sorted top-32 list
//     with a 64-lane bitonic sort (list in lanes 0..31, candidates in 32..63).
//   * The threshold filter rejects almost every score once the list is full,
//     so the select costs a compare per score plus O(k log N) merges per row.
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSelWaves = 4;
constexpr int kSelRowsPerWave = 16;
constexpr int kSelRows = kSelWaves * kSelRowsPerWave;  // 64 query rows / workgroup
constexpr int kSelChunk = 32;                          // key rows per LDS chunk
constexpr int kSelTop = kSelectMaxK;                   // list length per query row
constexpr int kSelCap = 64;                            // candidate slots per query row
constexpr int kSelMergeAt = 32;                        // merge threshold (cap - chunk)
static_assert(kSelMergeAt + kSelChunk <= kSelCap + 0, "candidate buffer can overflow");


// Sort 64 (score, index) pairs held one per lane into descending order,
// ties toward the lower index.  Standard bitonic network over lane ids.
__device__ __forceinline__ void bitonic_sort64_desc(float& vs, int& vi) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      float ps = shfl_xor_f(vs, stride);
      int pi = shfl_xor_i(vi, stride);
      bool desc = (lane & size) == 0;
      bool lower = (lane & stride) == 0;
      bool partner_better = ranks_before(ps, pi, vs, vi);
      bool self_better = ranks_before(vs, vi, ps, pi);
      bool take = (lower == desc) ? partner_better : self_better;
      if (take) {
        vs = ps;
        vi = pi;
      }
    }
  }
}

// Map the hardware workgroup id to a logical tile so that consecutive logical
// tiles (same batch element, same key set) run on the same XCD and share its L2.
__device__ __forceinline__ int xcd_swizzle(int bid, int nblk) {
  constexpr int kXcd = 8;
  if (nblk % kXcd != 0) return bid;
  return (bid % kXcd) * (nblk / kXcd) + bid / kXcd;
}

template <int RQ>  // rank values per lane group: r padded to 4*RQ
__global__ __launch_bounds__(256, 2) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr int RP = 4 * RQ;
  constexpr int KSTRIDE = RP + 4;  // padded LDS row (floats)

  __shared__ __align__(16) float s_key[2][kSelChunk * KSTRIDE];
  __shared__ float s_top_s[kSelRows * kSelTop];
  __shared__ int s_top_i[kSelRows * kSelTop];
  __shared__ float s_cand_s[kSelRows * kSelCap];
  __shared__ int s_cand_i[kSelRows * kSelCap];
  __shared__ int s_cnt[kSelRows];
  __shared__ float s_theta[kSelRows];
  __shared__ float s_scale[RP];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;   // rank slice owned by this lane group
  const int col = lane & 15; // query row within the wave's 16

  const int tiles_per_batch = (a.Nq + kSelRows - 1) / kSelRows;
  const int logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int b = logical / tiles_per_batch;
  const int row0 = (logical % tiles_per_batch) * kSelRows;
  if (b >= a.B) return;

  const float* qb = a.q + (int64_t)b * a.q_batch_stride;
  const float* kb = a.key + (int64_t)b * a.k_batch_stride;

  // ---- set-up: scale vector, zero padding, empty lists ----------------------
  for (int i = tid; i < RP; i += blockDim.x) s_scale[i] = (i < a.r) ? (a.scale ? a.scale[i] : 1.0f) : 0.0f;
  for (int i = tid; i < 2 * kSelChunk * KSTRIDE; i += blockDim.x) (&s_key[0][0])[i] = 0.0f;
  for (int i = tid; i < kSelRows * kSelTop; i += blockDim.x) {
    s_top_s[i] = -INFINITY;
    s_top_i[i] = 0x7fffffff;
  }
  if (tid < kSelRows) {
    s_cnt[tid] = 0;
    s_theta[tid] = -INFINITY;
  }
  __syncthreads();

  // ---- query fragment in registers -----------------------------------------
  const int my_row = row0 + wave * kSelRowsPerWave + col;  // query row of this lane
  const bool row_ok = my_row < a.Nq;
  float qf[RQ];
#pragma unroll
  for (int s = 0; s < RQ; ++s) {
    int rr = g * RQ + s;
    float v = 0.0f;
    if (row_ok && rr < a.r) {
      v = qb[(int64_t)my_row * a.ldq + rr];
      if (a.scale_on_query) v *= s_scale[rr];
    }
    qf[s] = v;
  }
  const float bias = a.bias ? a.bias[0] : 0.0f;
  const bool use_temp = a.temperature != 1.0f;
  const float temp = a.temperature;
  const bool scale_key = !a.scale_on_query;

  // ---- key chunk loader (global -> registers -> LDS) ------------------------
  // A chunk is kSelChunk consecutive key rows; each thread moves up to
  // kLoadPerThread values.
  constexpr int kChunkVals = kSelChunk * RP;
  constexpr int kLoadPerThread = (kChunkVals + 255) / 256;
  float pf[kLoadPerThread];
  auto load_chunk = [&](int c0) {
#pragma unroll
    for (int u = 0; u < kLoadPerThread; ++u) {
      int e = tid + u * 256;
      int rrow = e / RP, rc = e % RP;
      float v = 0.0f;
      int krow = c0 + rrow;
      if (e < kChunkVals && rc < a.r && krow < a.Nk) v = kb[(int64_t)krow * a.ldk + rc];
      pf[u] = v;
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kLoadPerThread; ++u) {
      int e = tid + u * 256;
      if (e < kChunkVals) {
        int rrow = e / RP, rc = e % RP;
        float v = pf[u];
        if (scale_key) v *= s_scale[rc];
        s_key[buf][rrow * KSTRIDE + rc] = v;
      }
    }
  };

  const int nchunks = (a.Nk + kSelChunk - 1) / kSelChunk;
  load_chunk(0);
  store_chunk(0);
  __syncthreads();

  float theta = row_ok ? -INFINITY : INFINITY;
  const int lrow = wave * kSelRowsPerWave + col;  // row slot within the workgroup
  const int k = a.k;

  for (int c = 0; c < nchunks; ++c) {
    const int cur = c & 1;
    const int c0 = c * kSelChunk;
    if (c + 1 < nchunks) load_chunk(c0 + kSelChunk);

    // -- scores for 32 keys x 16 query rows (two MFMA tiles) --
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc1 = {0.f, 0.f, 0.f, 0.f};
    const float* k0 = &s_key[cur][(0 * 16 + col) * KSTRIDE + g * RQ];
    const float* k1 = &s_key[cur][(1 * 16 + col) * KSTRIDE + g * RQ];
    if constexpr (RQ % 4 == 0) {
#pragma unroll
      for (int s4 = 0; s4 < RQ / 4; ++s4) {
        float4 x0 = *reinterpret_cast<const float4*>(k0 + 4 * s4);
        float4 x1 = *reinterpret_cast<const float4*>(k1 + 4 * s4);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.x, qf[4 * s4 + 0], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.x, qf[4 * s4 + 0], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.y, qf[4 * s4 + 1], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.y, qf[4 * s4 + 1], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.z, qf[4 * s4 + 2], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.z, qf[4 * s4 + 2], acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(x0.w, qf[4 * s4 + 3], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(x1.w, qf[4 * s4 + 3], acc1, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int s = 0; s < RQ; ++s) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0[s], qf[s], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1[s], qf[s], acc1, 0, 0, 0);
      }
    }

    // -- threshold filter: lane holds keys c0 + 16t + 4g + v for its row --
    float sc[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sc[v] = acc0[v];
      sc[4 + v] = acc1[v];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float s = sc[u] + bias;
      if (use_temp) s = s / temp;
      int key = c0 + (u >> 2) * 16 + 4 * g + (u & 3);
      bool pass = (key < a.Nk) && (s > theta);
      if (pass) {
        int pos = atomicAdd(&s_cnt[lrow], 1);
        s_cand_s[lrow * kSelCap + pos] = s;
        s_cand_i[lrow * kSelCap + pos] = key;
      }
    }
    wave_lds_sync();

    // -- merge rows whose candidate buffer filled up (or everything at the end) --
    const bool last = (c + 1 == nchunks);
    int need = 0;
    if (lane < kSelRowsPerWave) {
      int cnt = s_cnt[wave * kSelRowsPerWave + lane];
      need = (cnt >= kSelMergeAt) || (last && cnt > 0);
    }
    uint64_t mask = __ballot(need);
    const bool merged_any = mask != 0;
    while (mask) {
      const int t = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int slot = wave * kSelRowsPerWave + t;
      int cnt = __builtin_amdgcn_readfirstlane(s_cnt[slot]);
      float* ts = s_top_s + slot * kSelTop;
      int* ti = s_top_i + slot * kSelTop;
      float vs;
      int vi;
      while (cnt > 0) {
        const int take = cnt < 32 ? cnt : 32;
        if (lane < 32) {
          vs = ts[lane];
          vi = ti[lane];
        } else {
          int qd = lane - 32;
          if (qd < take) {
            vs = s_cand_s[slot * kSelCap + cnt - take + qd];
            vi = s_cand_i[slot * kSelCap + cnt - take + qd];
          } else {
            vs = -INFINITY;
            vi = 0x7fffffff;
          }
        }
        bitonic_sort64_desc(vs, vi);
        if (lane < 32) {
          ts[lane] = vs;
          ti[lane] = vi;
        }
        cnt -= take;
        wave_lds_sync();
      }
      const float th = readlane_f(vs, k - 1);
      if (lane == 0) {
        s_cnt[slot] = 0;
        s_theta[slot] = th;
      }
    }
    if (merged_any) {
      wave_lds_sync();
      if (row_ok) theta = s_theta[lrow];
    }

    // -- next key chunk into the other LDS buffer --
    if (c + 1 < nchunks) store_chunk(cur ^ 1);
    __syncthreads();
  }

  // ---- write the sorted top-k of this wave's 16 rows ------------------------
  for (int e = lane; e < kSelRowsPerWave * k; e += kWave) {
    int t = e / k, slot_e = e % k;
    int row = row0 + wave * kSelRowsPerWave + t;
    if (row < a.Nq) {
      int slot = wave * kSelRowsPerWave + t;
      int64_t o = ((int64_t)b * a.Nq + row) * k + slot_e;
      a.out_idx[o] = s_top_i[slot * kSelTop + slot_e];
      a.out_score[o] = s_top_s[slot * kSelTop + slot_e];
    }
  }
}

int launch_topk_select(const SelectArgs& a, hipStream_t stream) {
  JN_REQUIRE(a.k >= 1 && a.k <= kSelTop, kUnsupported, "top-k select supports 1 <= k <= %d (got %d)", kSelTop, a.k);
  JN_REQUIRE(a.k < a.Nk, kInvalidArgument, "top-k select needs k < key count (k=%d, Nk=%d)", a.k, a.Nk);
  JN_REQUIRE(a.r >= 1 && a.r <= 128, kUnsupported, "rank must be in [1, 128] (got %d)", a.r);
  JN_REQUIRE(a.temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  const int tiles = (a.Nq + kSelRows - 1) / kSelRows;
  const int64_t blocks = (int64_t)tiles * a.B;
  JN_REQUIRE(blocks > 0 && blocks < (1LL << 31), kInvalidArgument, "bad grid size");
  dim3 grid((unsigned)blocks), block(256);
  const int rq = (a.r + 3) / 4;
  if (rq <= 1) hipLaunchKernelGGL(lowrank_topk_select_kernel<1>, grid, block, 0, stream, a);
  else if (rq <= 2) hipLaunchKernelGGL(lowrank_topk_select_kernel<2>, grid, block, 0, stream, a);
  else if (rq <= 4) hipLaunchKernelGGL(lowrank_topk_select_kernel<4>, grid, block, 0, stream, a);
  else if (rq <= 8) hipLaunchKernelGGL(lowrank_topk_select_kernel<8>, grid, block, 0, stream, a);
  else if (rq <= 16) hipLaunchKernelGGL(lowrank_topk_select_kernel<16>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(lowrank_topk_select_kernel<32>, grid, block, 0, stream, a);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
