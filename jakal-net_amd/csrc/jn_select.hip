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
// Layout of one workgroup (256 threads = 4 waves, 64 query rows):
//   * 16 query rows per wave.  A wave keeps the query fragment of its rows in
//     VGPRs for the whole kernel (B operand of v_mfma_f32_16x16x4f32; lane l
//     owns row l%16, rank slice l/16).
//   * Keys stream through LDS in chunks of 32 rows (two 16-row MFMA tiles,
//     A operand), double buffered with a one-chunk register prefetch and one
//     workgroup barrier per chunk.
//   * After a chunk, lane l holds 8 scores of row l%16.  Scores above the
//     row's current k-th best (theta) are appended to the row's slot array in
//     LDS; the 4 lanes of a row (l, l^16, l^32, l^48) exchange their counts
//     with the gfx950 permlane swaps to get write offsets (no LDS atomics).
//     Counts and thresholds live in registers.
//   * Once any row of a wave has >= 64 waiting candidates (or any at the end),
//     all 16 rows of the wave merge together: lane (g, row) loads 32 slots of
//     its row into registers and a radix select over order keys finds each
//     row's k-th largest key, counting per lane and summing over the row's 4
//     lanes with permlane swaps; it starts below the bits shared by all of the
//     row's keys and stops once exactly k keys remain.  The k winners are
//     compacted to the front of the slot array.  A row whose k-th value is
//     tied (more equal keys than places) is merged again by the exact per-row
//     path, which keeps the lower key indices.  The kept set stays unsorted
//     until one bitonic sort per row at the end.
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSelWaves = 4;
constexpr int kSelRowsPerWave = 16;
constexpr int kSelRows = kSelWaves * kSelRowsPerWave;  // 64 query rows / workgroup
constexpr int kSelChunk = 32;                          // key rows per LDS chunk
// A row's 128 slots hold a kept region of KEEP entries (the k <= KEEP best so
// far; KEEP = 32 for k <= 32, 64 for k <= 64) followed by the candidates
// appended since the last merge.  A merge runs once a row holds
// merge_at(KEEP) candidates; one more chunk can add 32, so the largest slot
// used is KEEP + merge_at - 1 + 32 - 1 = 126 either way.
__host__ __device__ constexpr int merge_at(int keep) { return keep == 32 ? 64 : 32; }
constexpr int kSelSlots = 32 + merge_at(32) - 1 + kSelChunk;  // 127 used (KEEP = 32)
static_assert(64 + merge_at(64) - 1 + kSelChunk == kSelSlots, "both kept-region sizes use the same slots");
// Row strides are 16-byte multiples (vector reads) that shift successive rows by
// 4 LDS banks, so the 16 rows of a wave read and write on distinct banks.
constexpr int kSelScoreStride = 132;  // floats
constexpr int kSelIndexStride = 136;  // uint16 (68 words)
constexpr int kSelTrash = 127;        // slot that absorbs writes of non-winners
constexpr int kSelMaxKeys = 65535;    // key indices are stored as uint16
static_assert(kSelSlots <= 128, "merge reads at most two slots per lane");

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

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// Lanes whose id is below this lane, within mask m.
__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Merge one row: keep the k best of its `kept` kept entries (slots [0, kept))
// and `cnt` candidates (slots [KEEP, KEEP + cnt)), k < kept + cnt, compacted
// to slots [0, k); returns the new k-th best score (wave-uniform).
template <int KEEP>
__device__ float merge_row(float* row_s, uint16_t* row_i, int k, int kept, int cnt) {
  const int lane = lane_id();
  const int n_used = KEEP + cnt;
  const int sa = lane, sb = 64 + lane;
  const bool va = (sa < kept) || (sa >= KEEP && sa < n_used);
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

  // Radix select of the k-th largest key.  All valid keys lie in [lo, hi]; the
  // bits above the highest bit where lo and hi differ are common to every
  // candidate threshold, so the search starts below them.
  const uint32_t hi = __builtin_amdgcn_readfirstlane(wave_max_u32(max(ka, kb)));
  const uint32_t lo =
      __builtin_amdgcn_readfirstlane(wave_min_u32(min(va ? ka : 0xffffffffu, vb ? kb : 0xffffffffu)));
  const uint32_t diff = hi ^ lo;
  int bit = diff ? 31 - __builtin_clz(diff) : -1;
  uint32_t t = diff ? (hi & ~((2u << bit) - 1u)) : hi;  // common prefix (bit 31 case handled below)
  if (bit == 31) t = 0;
  int n_at_t = k + 1;  // unknown; forces the tie path if the loop never lands on exactly k
  for (; bit >= 0; --bit) {
    const uint32_t c = t | (1u << bit);
    const int n = popc64(__ballot(ka >= c)) + popc64(__ballot(kb >= c));
    if (n >= k) {
      t = c;
      n_at_t = n;
      if (n == k) break;  // exactly k keys >= t: they are the winners
    }
  }
  bool keep_a, keep_b;
  uint32_t theta_key;
  if (n_at_t == k) {
    keep_a = va && ka >= t;
    keep_b = vb && kb >= t;
    uint32_t m = 0xffffffffu;
    if (keep_a) m = ka;
    if (keep_b) m = min(m, kb);
    theta_key = __builtin_amdgcn_readfirstlane(wave_min_u32(m));
  } else {
    // t is the k-th largest key itself; resolve ties at t toward lower indices
    theta_key = t;
    keep_a = ka > t;
    keep_b = kb > t;
    const int n_gt = popc64(__ballot(keep_a)) + popc64(__ballot(keep_b));
    bool eq_a = va && (ka == t), eq_b = vb && (kb == t);
    int need = k - n_gt;
    const int n_eq = popc64(__ballot(eq_a)) + popc64(__ballot(eq_b));
    if (n_eq == need) {
      keep_a |= eq_a;
      keep_b |= eq_b;
    } else {
      for (; need > 0; --need) {
        int m = 0x7fffffff;
        if (eq_a) m = min(m, ia);
        if (eq_b) m = min(m, ib);
        m = wave_min_i32(m);
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
  }
  // the k-th best score: an element whose key equals theta_key
  const uint64_t eqm_a = __ballot(va && ka == theta_key);
  const uint64_t eqm_b = __ballot(vb && kb == theta_key);
  const float theta = eqm_a ? readlane_f(fa, __builtin_ctzll(eqm_a)) : readlane_f(fb, __builtin_ctzll(eqm_b));

  const uint64_t ma = __ballot(keep_a);
  const uint64_t mb = __ballot(keep_b);
  const int pa = mbcnt64(ma);
  const int pb = popc64(ma) + mbcnt64(mb);
  // the reads above have returned (their values feed these stores)
  if (keep_a) {
    row_s[pa] = fa;
    row_i[pa] = (uint16_t)ia;
  }
  if (keep_b) {
    row_s[pb] = fb;
    row_i[pb] = (uint16_t)ib;
  }
  wave_lds_sync();
  return theta;
}


__device__ __forceinline__ float key_to_float(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Merge every row of the wave at once.  Lane (g, col) owns slots
// [32g, 32g+32) of row col: kept entries or candidates.  A row keeps the
// min(k, kept + cnt) best of its `kept` kept entries and `cnt` candidates (a
// row that has not yet seen k keys keeps them all and its threshold stays
// -inf).  The radix select runs per lane over its 32 keys, with row counts
// summed over the row's 4 lanes by permlane swaps.  Rows with exact ties at
// the k-th value return fallback = true and are left untouched for merge_row.
template <int KEEP>
__device__ void merge_rows_batched(float* row_s, uint16_t* row_i, int k, int kept, int cnt_row, float& theta,
                                   bool& fallback) {
  const int lane = lane_id();
  const int g = lane >> 4;
  const int base = 32 * g;
  const int total = kept + cnt_row;
  const int kk = min(k, total);  // entries the row keeps
  // kept entries [0, kept), then cnt_row candidates from KEEP on
  const int n_valid = base < KEEP ? max(0, min(32, kept - base)) : max(0, min(32, KEEP + cnt_row - base));
  uint32_t key[32];
  int id[32];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 v = *reinterpret_cast<const float4*>(row_s + base + 4 * q);
    key[4 * q + 0] = (4 * q + 0 < n_valid) ? order_key(v.x) : 0u;
    key[4 * q + 1] = (4 * q + 1 < n_valid) ? order_key(v.y) : 0u;
    key[4 * q + 2] = (4 * q + 2 < n_valid) ? order_key(v.z) : 0u;
    key[4 * q + 3] = (4 * q + 3 < n_valid) ? order_key(v.w) : 0u;
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 v = *reinterpret_cast<const uint4*>(row_i + base + 8 * q);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      id[8 * q + 2 * h] = (int)(w[h] & 0xffffu);
      id[8 * q + 2 * h + 1] = (int)(w[h] >> 16);
    }
  }
  // row range of valid keys
  uint32_t hi = 0, lo = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    hi = max(hi, key[i]);
    lo = min(lo, (i < n_valid) ? key[i] : 0xffffffffu);
  }
  hi = max(hi, (uint32_t)xor16_i((int)hi));
  hi = max(hi, (uint32_t)xor32_i((int)hi));
  lo = min(lo, (uint32_t)xor16_i((int)lo));
  lo = min(lo, (uint32_t)xor32_i((int)lo));
  const uint32_t diff = hi ^ lo;
  const int start = diff ? 31 - __builtin_clz(diff) : -1;
  uint32_t t = diff ? (hi & ~((2u << start) - 1u)) : hi;  // shared prefix of the row's keys
  if (start == 31) t = 0;
  const int wave_start = (int)wave_max_u32((uint32_t)(start + 1)) - 1;  // uniform loop bound
  // a row whose entries all fit keeps every valid key (valid keys are > 0)
  bool done = total <= k;
  if (done) t = 0;
  for (int bit = wave_start; bit >= 0; --bit) {
    if (!__ballot(!done)) break;
    const uint32_t c = t | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) cnt += (key[i] >= c) ? 1 : 0;
    int n = cnt + xor16_i(cnt);
    n += xor32_i(n);
    if (!done && n >= kk) {
      t = c;
      done = (n == kk);
    }
  }
  // winners: exactly k keys >= t (done), or the k-th largest key is t itself
  uint32_t keep_bits = 0;
  uint32_t theta_key;
  bool tie_row = false;
  if (done) {
    uint32_t m = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const bool kp = (i < n_valid) && key[i] >= t;
      keep_bits |= kp ? (1u << i) : 0u;
      m = kp ? min(m, key[i]) : m;
    }
    m = min(m, (uint32_t)xor16_i((int)m));
    m = min(m, (uint32_t)xor32_i((int)m));
    theta_key = m;
  } else {
    int gt = 0, eq = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      gt += (key[i] > t) ? 1 : 0;
      eq += ((i < n_valid) && key[i] == t) ? 1 : 0;
    }
    gt += xor16_i(gt);
    gt += xor32_i(gt);
    eq += xor16_i(eq);
    eq += xor32_i(eq);
    tie_row = (eq != kk - gt);
#pragma unroll
    for (int i = 0; i < 32; ++i) keep_bits |= ((i < n_valid) && key[i] >= t) ? (1u << i) : 0u;
    theta_key = t;
  }
  fallback = tie_row;
  // compact the winners of non-tie rows to slots [0, k)
  const int w = __builtin_popcount(keep_bits);
  const int w1 = xor16_i(w);
  const int w2 = xor32_i(w);
  const int w3 = xor16_i(w2);
  int pos = (g == 0) ? 0 : (g == 1) ? w1 : (g == 2) ? (w2 + w3) : (w1 + w2 + w3);
  if (!tie_row) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const bool kp = (keep_bits >> i) & 1u;
      const int dst = kp ? pos : kSelTrash;
      row_s[dst] = key_to_float(key[i]);
      row_i[dst] = (uint16_t)id[i];
      pos += kp ? 1 : 0;
    }
    theta = total < k ? -INFINITY : key_to_float(theta_key);
  }
  wave_lds_sync();
}

// VEC: r == 4*RQ and 16-byte aligned key rows -> unconditional float4 chunk loads.
template <int RQ, bool VEC, int KEEP>
__global__ __launch_bounds__(256, 2) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr int kMergeAt = merge_at(KEEP);
  constexpr int RP = 4 * RQ;
  constexpr int KSTRIDE = RP + 4;  // padded key row (floats)

  __shared__ __align__(16) float s_key[2][kSelChunk * KSTRIDE];
  __shared__ __align__(16) float s_slot_s[kSelRows * kSelScoreStride];
  __shared__ __align__(16) uint16_t s_slot_i[kSelRows * kSelIndexStride];
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
  __syncthreads();

  // ---- query fragment in registers ------------------------------------------
  const int lrow = wave * kSelRowsPerWave + col;  // row slot within the workgroup
  const int my_row = row0 + lrow;
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
          const int krow = min(c0 + rrow, a.Nk - 1);  // tail rows: a valid row, masked later
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
  int kept = 0;                                 // valid kept entries of this lane's row (<= k)
  float* my_slot_s = s_slot_s + lrow * kSelScoreStride;
  uint16_t* my_slot_i = s_slot_i + lrow * kSelIndexStride;

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
#pragma unroll
    for (int u = 0; u < 8; ++u) sc[u] = (((u < 4) ? acc0[u & 3] : acc1[u & 3]) + bias) * inv_temp;
    if (c0 + kSelChunk > a.Nk) {  // uniform: only the last chunk holds padding keys
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + (u >> 2) * 16 + 4 * g + (u & 3) >= a.Nk) sc[u] = -INFINITY;
    }
    uint64_t any = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) any |= __ballot(sc[u] > theta);
    if (any) {
      uint32_t pass_mask = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) pass_mask |= (sc[u] > theta) ? (1u << u) : 0u;
      // counts of the row's 4 lanes (lane groups g^1, g^2, g^3) via permlane swaps
      const int np = __builtin_popcount(pass_mask);
      const int n1 = xor16_i(np);
      const int n2 = xor32_i(np);
      const int n3 = xor16_i(n2);
      const int excl = (g == 0) ? 0 : (g == 1) ? n1 : (g == 2) ? (n2 + n3) : (n1 + n2 + n3);
      const int total = np + n1 + n2 + n3;
      int pos = KEEP + cnt + excl;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const bool ok = (pass_mask >> u) & 1u;
        const int dst = ok ? pos : kSelTrash;
        my_slot_s[dst] = sc[u];
        my_slot_i[dst] = (uint16_t)(c0 + (u >> 2) * 16 + 4 * g + (u & 3));
        pos += ok ? 1 : 0;
      }
      cnt += total;
      wave_lds_sync();
    }

    // -- merge rows whose candidates filled up (or everything at the end) --
    const bool last = (c + 1 == nchunks);
    if (__ballot(lane < kSelRowsPerWave && (cnt >= kMergeAt || (last && cnt > 0)))) {
      bool fallback;
      merge_rows_batched<KEEP>(my_slot_s, my_slot_i, k, kept, cnt, theta, fallback);
      // rows with exact ties at the k-th value: exact per-row merge (such a
      // row holds more than k entries, so the merge fills it)
      uint64_t m = __ballot(lane < kSelRowsPerWave && fallback);
      while (m) {
        const int t = __builtin_ctzll(m);
        m &= m - 1;
        const int row_cnt = readlane_i(cnt, t);
        const int row_kept = readlane_i(kept, t);
        const int slot = wave * kSelRowsPerWave + t;
        const float th = merge_row<KEEP>(s_slot_s + slot * kSelScoreStride, s_slot_i + slot * kSelIndexStride, k,
                                         row_kept, row_cnt);
        if (col == t) theta = th;
      }
      if (!row_ok) theta = INFINITY;  // rows past Nq stay closed
      kept = min(k, kept + cnt);
      cnt = 0;
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
      vs = s_slot_s[slot * kSelScoreStride + lane];
      vi = s_slot_i[slot * kSelIndexStride + lane];
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
  if (a.k <= 32) {
    if (vec) hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, true, 32>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, false, 32>), grid, dim3(256), 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, true, 64>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, false, 64>), grid, dim3(256), 0, stream, a);
  }
}

int launch_topk_select(const SelectArgs& a, hipStream_t stream) {
  JN_REQUIRE(a.k >= 1 && a.k <= kSelectMaxK, kUnsupported, "top-k select supports 1 <= k <= %d (got %d)", kSelectMaxK,
             a.k);
  JN_REQUIRE(a.k < a.Nk, kInvalidArgument, "top-k select needs k < key count (k=%d, Nk=%d)", a.k, a.Nk);
  JN_REQUIRE(a.Nk <= kSelMaxKeys, kUnsupported, "top-k select supports at most %d keys (got %d)", kSelMaxKeys, a.Nk);
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
