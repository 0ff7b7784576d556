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
//     A operand), double buffered with a one-chunk register prefetch and one
//     workgroup barrier per chunk.
//   * After a chunk, lane l holds 8 scores of row l%16.  Scores above the
//     row's current k-th best (theta) are appended to the row's slot array in
//     LDS; the 4 lanes of a row find their write offsets with a 4-lane prefix
//     sum (no LDS atomics).  Counts and thresholds live in registers.
//   * A row with >= 32 waiting candidates (or any at the end) is merged: the
//     wave loads the row's k kept entries plus candidates (up to 96 slots, two
//     per lane), finds the k-th largest order key by a 32-step ballot radix
//     select, and compacts the k winners back to the front of the slot array.
//     Ties at the k-th value keep the lower key indices.  The kept set stays
//     unsorted until one bitonic sort per row at the end.
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSelWaves = 4;
constexpr int kSelRowsPerWave = 16;
constexpr int kSelRows = kSelWaves * kSelRowsPerWave;  // 64 query rows / workgroup
constexpr int kSelChunk = 32;                          // key rows per LDS chunk
constexpr int kSelKeep = kSelectMaxK;                  // kept-entry region per row
constexpr int kSelMergeAt = 32;                        // merge once this many candidates wait
constexpr int kSelSlots = kSelKeep + kSelMergeAt - 1 + kSelChunk;  // 95 used
constexpr int kSelSlotStride = 96;
static_assert(kSelSlots <= kSelSlotStride, "slot array too small");
static_assert(kSelSlotStride <= 128, "merge reads at most two slots per lane");

// Monotone map float -> uint32 (larger float -> larger key); -0 and +0 map together.
__device__ __forceinline__ uint32_t order_key(float s) {
  uint32_t u = __float_as_uint(s + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Branchless bitonic sort of 64 (score, index) pairs into descending score,
// ascending index on ties.
__device__ __forceinline__ void bitonic_sort64_desc(float& vs, int& vi) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float ps = shfl_xor_f(vs, stride);
      const int pi = shfl_xor_i(vi, stride);
      const bool partner_better = (ps > vs) | ((ps == vs) & (pi < vi));
      const bool self_better = (vs > ps) | ((vs == ps) & (vi < pi));
      const bool keep_better = ((lane & stride) == 0) == ((lane & size) == 0);
      const bool take = keep_better ? partner_better : self_better;
      vs = take ? ps : vs;
      vi = take ? pi : vi;
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

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// Lanes whose id is below this lane, within mask m.
__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Merge one row: keep the k best of its k kept entries and `cnt` candidates,
// compacted to slots [0, k); returns the new k-th best score (wave-uniform).
__device__ float merge_row(float* row_s, int* row_i, int k, int cnt) {
  const int lane = lane_id();
  const int n_used = kSelKeep + cnt;
  const int sa = lane, sb = 64 + lane;
  const bool va = (sa < k) || (sa >= kSelKeep && sa < n_used);
  const bool vb = sb < n_used;
  float fa = 0.f, fb = 0.f;
  int ia = 0, ib = 0;
  if (va) {
    fa = row_s[sa];
    ia = row_i[sa];
  }
  if (vb) {
    fb = row_s[sb];
    ib = row_i[sb];
  }
  const uint32_t ka = va ? order_key(fa) : 0u;
  const uint32_t kb = vb ? order_key(fb) : 0u;

  // k-th largest key: the largest t with #(key >= t) >= k
  uint32_t t = 0;
#pragma unroll 4
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    const int n = popc64(__ballot(ka >= c)) + popc64(__ballot(kb >= c));
    t = (n >= k) ? c : t;
  }
  bool keep_a = ka > t, keep_b = kb > t;
  const int n_gt = popc64(__ballot(keep_a)) + popc64(__ballot(keep_b));
  bool eq_a = (ka == t) && va, eq_b = (kb == t) && vb;
  int need = k - n_gt;
  const int n_eq = popc64(__ballot(eq_a)) + popc64(__ballot(eq_b));
  if (n_eq == need) {
    keep_a |= eq_a;
    keep_b |= eq_b;
  } else {
    // exact ties at the k-th value: take the lowest key indices, one at a time
    for (; need > 0; --need) {
      int m = 0x7fffffff;
      if (eq_a) m = min(m, ia);
      if (eq_b) m = min(m, ib);
#pragma unroll
      for (int s = 32; s >= 1; s >>= 1) m = min(m, shfl_xor_i(m, s));
      if (eq_a && ia == m) {
        keep_a = true;
        eq_a = false;
      }
      if (eq_b && ib == m) {
        keep_b = true;
        eq_b = false;
      }
    }
  }
  // the k-th best score: any element whose key equals t
  const uint64_t eqm_a = __ballot((ka == t) && va);
  const uint64_t eqm_b = __ballot((kb == t) && vb);
  const float theta = eqm_a ? readlane_f(fa, __builtin_ctzll(eqm_a)) : readlane_f(fb, __builtin_ctzll(eqm_b));

  const uint64_t ma = __ballot(keep_a);
  const uint64_t mb = __ballot(keep_b);
  const int pa = mbcnt64(ma);
  const int pb = popc64(ma) + mbcnt64(mb);
  // the reads above have returned (their values feed these stores)
  if (keep_a) {
    row_s[pa] = fa;
    row_i[pa] = ia;
  }
  if (keep_b) {
    row_s[pb] = fb;
    row_i[pb] = ib;
  }
  wave_lds_sync();
  return theta;
}

// VEC: r == 4*RQ and 16-byte aligned key rows -> unconditional float4 chunk loads.
template <int RQ, bool VEC>
__global__ __launch_bounds__(256, 2) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr int RP = 4 * RQ;
  constexpr int KSTRIDE = RP + 4;  // padded LDS row (floats)

  __shared__ __align__(16) float s_key[2][kSelChunk * KSTRIDE];
  __shared__ float s_slot_s[kSelRows * kSelSlotStride];
  __shared__ int s_slot_i[kSelRows * kSelSlotStride];
  __shared__ __align__(16) float s_scale[RP];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;    // rank slice owned by this lane group
  const int col = lane & 15;  // query row within the wave's 16

  const int tiles_per_batch = (a.Nq + kSelRows - 1) / kSelRows;
  const int logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int b = logical / tiles_per_batch;
  const int row0 = (logical % tiles_per_batch) * kSelRows;
  if (b >= a.B) return;

  const float* qb = a.q + (int64_t)b * a.q_batch_stride;
  const float* kbase = a.key + (int64_t)b * a.k_batch_stride;
  const int k = a.k;

  // ---- set-up -------------------------------------------------------------
  for (int i = tid; i < RP; i += blockDim.x) s_scale[i] = (i < a.r) ? (a.scale ? a.scale[i] : 1.0f) : 0.0f;
  if (!VEC)
    for (int i = tid; i < 2 * kSelChunk * KSTRIDE; i += blockDim.x) (&s_key[0][0])[i] = 0.0f;
  // the kept region starts as k sentinels that lose to every finite score
  for (int i = tid; i < kSelRows * kSelKeep; i += blockDim.x) {
    const int rrow = i / kSelKeep, e = i % kSelKeep;
    s_slot_s[rrow * kSelSlotStride + e] = -INFINITY;
    s_slot_i[rrow * kSelSlotStride + e] = 0x7fffffff;
  }
  __syncthreads();

  // ---- query fragment in registers ------------------------------------------
  const int my_row = row0 + wave * kSelRowsPerWave + col;
  const bool row_ok = my_row < a.Nq;
  float qf[RQ];
#pragma unroll
  for (int s = 0; s < RQ; ++s) {
    const int rr = g * RQ + s;
    float v = 0.0f;
    if (row_ok && rr < a.r) {
      v = qb[(int64_t)my_row * a.ldq + rr];
      if (a.scale_on_query) v *= s_scale[rr];
    }
    qf[s] = v;
  }
  const float bias = a.bias ? a.bias[0] : 0.0f;
  // (dot + bias) / T as a multiply by the reciprocal: exact for T == 1, within
  // 1.5 ulp of the division otherwise
  const float inv_temp = 1.0f / a.temperature;
  const bool scale_key = !a.scale_on_query;

  // ---- key chunk loader ---------------------------------------------------
  constexpr int kChunkVals = kSelChunk * RP;
  constexpr int kChunkF4 = kChunkVals / 4;
  constexpr int kLoads = VEC ? (kChunkF4 + 255) / 256 : (kChunkVals + 255) / 256;
  float4 pf4[VEC ? kLoads : 1];
  float pf1[VEC ? 1 : kLoads];
  auto load_chunk = [&](int c0) {
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int f = tid + u * 256;
        if (kChunkF4 % 256 == 0 || f < kChunkF4) {
          const int rrow = f / RQ, c4 = f % RQ;
          const int krow = min(c0 + rrow, a.Nk - 1);  // tail rows: a valid row, masked at the compare
          pf4[u] = *reinterpret_cast<const float4*>(kbase + (int64_t)krow * a.ldk + 4 * c4);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int e = tid + u * 256;
        const int rrow = e / RP, rc = e % RP;
        const int krow = c0 + rrow;
        float v = 0.0f;
        if (e < kChunkVals && rc < a.r && krow < a.Nk) v = kbase[(int64_t)krow * a.ldk + rc];
        pf1[u] = v;
      }
    }
  };
  auto store_chunk = [&](int buf) {
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int f = tid + u * 256;
        if (kChunkF4 % 256 == 0 || f < kChunkF4) {
          const int rrow = f / RQ, c4 = f % RQ;
          float4 v = pf4[u];
          if (scale_key) {
            const float4 sc = *reinterpret_cast<const float4*>(&s_scale[4 * c4]);
            v.x *= sc.x;
            v.y *= sc.y;
            v.z *= sc.z;
            v.w *= sc.w;
          }
          *reinterpret_cast<float4*>(&s_key[buf][rrow * KSTRIDE + 4 * c4]) = v;
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int e = tid + u * 256;
        if (e < kChunkVals) {
          const int rrow = e / RP, rc = e % RP;
          s_key[buf][rrow * KSTRIDE + rc] = scale_key ? pf1[u] * s_scale[rc] : pf1[u];
        }
      }
    }
  };

  const int nchunks = (a.Nk + kSelChunk - 1) / kSelChunk;
  load_chunk(0);
  store_chunk(0);
  __syncthreads();

  float theta = row_ok ? -INFINITY : INFINITY;  // invalid rows never admit
  int cnt = 0;                                  // candidates waiting for this lane's row
  const int lrow = wave * kSelRowsPerWave + col;
  float* my_slot_s = s_slot_s + lrow * kSelSlotStride;
  int* my_slot_i = s_slot_i + lrow * kSelSlotStride;
  // 4-lane prefix sources: the lanes of the same row in the lower rank slices
  const int src16 = (lane - 16) & 63, src32 = (lane - 32) & 63, src_top = col + 48;

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
        const float4 x0 = *reinterpret_cast<const float4*>(k0 + 4 * s4);
        const float4 x1 = *reinterpret_cast<const float4*>(k1 + 4 * s4);
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

    // -- threshold filter: lane holds keys c0 + 16t + 4g + v of its row --
    float sc[8];
    uint32_t pass_mask = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float s = (((u < 4) ? acc0[u & 3] : acc1[u & 3]) + bias) * inv_temp;
      sc[u] = s;
      const int key = c0 + (u >> 2) * 16 + 4 * g + (u & 3);
      pass_mask |= ((key < a.Nk) & (s > theta)) ? (1u << u) : 0u;
    }
    if (__ballot(pass_mask != 0)) {
      const int np = __builtin_popcount(pass_mask);
      const int up16 = __builtin_amdgcn_ds_bpermute(src16 << 2, np);
      const int incl1 = np + (g >= 1 ? up16 : 0);
      const int up32 = __builtin_amdgcn_ds_bpermute(src32 << 2, incl1);
      const int incl2 = incl1 + (g >= 2 ? up32 : 0);
      const int total = __builtin_amdgcn_ds_bpermute(src_top << 2, incl2);
      int pos = kSelKeep + cnt + incl2 - np;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (pass_mask & (1u << u)) {
          my_slot_s[pos] = sc[u];
          my_slot_i[pos] = c0 + (u >> 2) * 16 + 4 * g + (u & 3);
          ++pos;
        }
      }
      cnt += total;
      wave_lds_sync();
    }

    // -- merge rows whose candidates filled up (or everything at the end) --
    const bool last = (c + 1 == nchunks);
    uint64_t m = __ballot(lane < kSelRowsPerWave && (cnt >= kSelMergeAt || (last && cnt > 0)));
    while (m) {
      const int t = __builtin_ctzll(m);
      m &= m - 1;
      const int row_cnt = readlane_i(cnt, t);
      const int slot = wave * kSelRowsPerWave + t;
      const float th = merge_row(s_slot_s + slot * kSelSlotStride, s_slot_i + slot * kSelSlotStride, k, row_cnt);
      if (col == t) {
        theta = th;
        cnt = 0;
      }
    }

    // -- next key chunk into the other LDS buffer --
    if (c + 1 < nchunks) store_chunk(cur ^ 1);
    __syncthreads();
  }

  // ---- sort each row's k winners and write them -----------------------------
  for (int t = 0; t < kSelRowsPerWave; ++t) {
    const int row = row0 + wave * kSelRowsPerWave + t;
    if (row >= a.Nq) break;
    const int slot = wave * kSelRowsPerWave + t;
    float vs = -INFINITY;
    int vi = 0x7fffffff;
    if (lane < k) {
      vs = s_slot_s[slot * kSelSlotStride + lane];
      vi = s_slot_i[slot * kSelSlotStride + lane];
    }
    bitonic_sort64_desc(vs, vi);
    if (lane < k) {
      const int64_t o = ((int64_t)b * a.Nq + row) * k + lane;
      a.out_idx[o] = vi;
      a.out_score[o] = vs;
    }
  }
}

template <int RQ>
static void launch_rq(const SelectArgs& a, bool vec, dim3 grid, hipStream_t stream) {
  if (vec) hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, true>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, false>), grid, dim3(256), 0, stream, a);
}

int launch_topk_select(const SelectArgs& a, hipStream_t stream) {
  JN_REQUIRE(a.k >= 1 && a.k <= kSelKeep, kUnsupported, "top-k select supports 1 <= k <= %d (got %d)", kSelKeep, a.k);
  JN_REQUIRE(a.k < a.Nk, kInvalidArgument, "top-k select needs k < key count (k=%d, Nk=%d)", a.k, a.Nk);
  JN_REQUIRE(a.r >= 1 && a.r <= 128, kUnsupported, "rank must be in [1, 128] (got %d)", a.r);
  JN_REQUIRE(a.temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  const int tiles = (a.Nq + kSelRows - 1) / kSelRows;
  const int64_t blocks = (int64_t)tiles * a.B;
  JN_REQUIRE(blocks > 0 && blocks < (1LL << 31), kInvalidArgument, "bad grid size");
  dim3 grid((unsigned)blocks);
  int rq = (a.r + 3) / 4;
  rq = rq <= 1 ? 1 : rq <= 2 ? 2 : rq <= 4 ? 4 : rq <= 8 ? 8 : rq <= 16 ? 16 : 32;
  const bool vec = (a.r == 4 * rq) && (a.ldk % 4 == 0) && (a.k_batch_stride % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0);
  JN_PROFILE("lowrank_topk_select_kernel", stream);
  switch (rq) {
    case 1: launch_rq<1>(a, vec, grid, stream); break;
    case 2: launch_rq<2>(a, vec, grid, stream); break;
    case 4: launch_rq<4>(a, vec, grid, stream); break;
    case 8: launch_rq<8>(a, vec, grid, stream); break;
    case 16: launch_rq<16>(a, vec, grid, stream); break;
    default: launch_rq<32>(a, vec, grid, stream); break;
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
