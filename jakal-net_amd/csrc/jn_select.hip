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
//     row's threshold theta are appended to the lane's own candidate region
//     of the row (the row's 4 lanes never share a region, so appends need no
//     cross-lane offsets).  Counts and thresholds live in registers.
//   * Once any lane of a wave has filled its region to within one chunk of
//     its capacity (or at the end), all 16 rows of the wave merge together:
//     lane (g, row) loads a quarter of the row's kept entries and its own
//     candidates into registers, and a radix select over order keys finds
//     each row's k-th largest key, counting per lane and summing over the
//     row's 4 lanes with permlane swaps; it starts below the bits shared by
//     all of the row's keys and stops once exactly k keys remain.  The k
//     winners are compacted into the row's kept region.  A row whose k-th
//     value is tied (more equal keys than places) is merged again by the
//     exact per-row path, which keeps the lower key indices.  The kept set
//     stays unsorted until one bitonic sort per row at the end.
#include <type_traits>

#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kSelWaves = 4;
constexpr int kSelRowsPerWave = 16;
constexpr int kSelRows = kSelWaves * kSelRowsPerWave;  // 64 query rows / workgroup
constexpr int kSelChunk = 32;                          // key rows per LDS chunk
// A row's slots: a kept region of KEEP entries (the k <= KEEP best so far;
// KEEP = 32 for k <= 32, 64 for k <= 64), then one candidate region of
// sel_lane_cap(KEEP) slots per lane of the row.  A lane takes at most 8
// candidates per chunk, so merging once a lane holds more than cap - 8 keeps
// every region within its capacity.
constexpr int kSelRowSlots = 144;
__host__ __device__ constexpr int sel_lane_cap(int keep) { return (kSelRowSlots - keep) / 4; }
static_assert(sel_lane_cap(32) % 4 == 0 && sel_lane_cap(64) % 4 == 0, "candidate regions hold whole float4s");
static_assert(32 / 4 + sel_lane_cap(32) == 64 / 4 + sel_lane_cap(64), "both kept-region sizes merge as many keys");
constexpr int kSelMergeKeys = 32 / 4 + sel_lane_cap(32);  // keys per lane in a batched merge (36)
// Row strides are 16-byte multiples (vector reads) that shift successive rows by
// 20 (scores) LDS banks, so the 16 rows of a wave read on distinct banks.
constexpr int kSelScoreStride = 148;  // floats
constexpr int kSelIndexStride = 152;  // uint16 (76 words)
constexpr int kSelMaxKeys = 65535;    // key indices are stored as uint16

// Monotone map float -> uint32 (larger float -> larger key); -0 and +0 map together.
__device__ __forceinline__ uint32_t order_key(float s) {
  uint32_t u = __float_as_uint(s + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
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

// Sum over the 4 lanes of a row (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ int row_sum4(int v) {
  v += xor16_i(v);
  return v + xor32_i(v);
}

// Exact merge of one row by the whole wave: keep the k best (ties toward the
// lower key index) of its `kept` kept entries and the c[g] candidates of lane
// region g, compacted to slots [0, k); k < kept + sum(c).  Returns the new
// k-th best score (wave-uniform).  Lane l holds slots l, l + 64, l + 128.
template <int KEEP>
__device__ float merge_row_exact(float* row_s, uint16_t* row_i, int k, int kept, const int (&c)[4]) {
  constexpr int CAP = sel_lane_cap(KEEP);
  const int lane = lane_id();
  float f[3];
  int ix[3];
  uint32_t kk[3];
  bool v[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int s = lane + 64 * j;
    bool ok;
    if (s < KEEP) {
      ok = s < kept;
    } else if (s < kSelRowSlots) {
      const int rg = (s - KEEP) / CAP;
      const int ri = s - KEEP - rg * CAP;
      const int cr = rg == 0 ? c[0] : rg == 1 ? c[1] : rg == 2 ? c[2] : c[3];
      ok = ri < cr;
    } else {
      ok = false;
    }
    v[j] = ok;
    f[j] = ok ? row_s[s] : 0.f;
    ix[j] = ok ? (int)row_i[s] : 0;
    kk[j] = ok ? order_key(f[j]) : 0u;
  }

  // Radix select of the k-th largest key.  All valid keys lie in [lo, hi]; the
  // bits above the highest bit where lo and hi differ are common to every
  // candidate threshold, so the search starts below them.
  uint32_t hmax = 0, lmin = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    hmax = max(hmax, kk[j]);
    lmin = min(lmin, v[j] ? kk[j] : 0xffffffffu);
  }
  const uint32_t hi = __builtin_amdgcn_readfirstlane(wave_max_u32(hmax));
  const uint32_t lo = __builtin_amdgcn_readfirstlane(wave_min_u32(lmin));
  const uint32_t diff = hi ^ lo;
  int bit = diff ? 31 - __builtin_clz(diff) : -1;
  uint32_t t = diff ? (hi & ~((2u << bit) - 1u)) : hi;  // common prefix (bit 31 case handled below)
  if (bit == 31) t = 0;
  int n_at_t = k + 1;  // unknown; forces the tie path if the loop never lands on exactly k
  for (; bit >= 0; --bit) {
    const uint32_t cth = t | (1u << bit);
    int n = 0;
#pragma unroll
    for (int j = 0; j < 3; ++j) n += popc64(__ballot(kk[j] >= cth));
    if (n >= k) {
      t = cth;
      n_at_t = n;
      if (n == k) break;  // exactly k keys >= t: they are the winners
    }
  }
  bool keep[3];
  uint32_t theta_key;
  if (n_at_t == k) {
    uint32_t m = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      keep[j] = v[j] && kk[j] >= t;
      if (keep[j]) m = min(m, kk[j]);
    }
    theta_key = __builtin_amdgcn_readfirstlane(wave_min_u32(m));
  } else {
    // t is the k-th largest key itself; resolve ties at t toward lower indices
    theta_key = t;
    int n_gt = 0, n_eq = 0;
    bool eq[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      keep[j] = kk[j] > t;
      eq[j] = v[j] && kk[j] == t;
      n_gt += popc64(__ballot(keep[j]));
      n_eq += popc64(__ballot(eq[j]));
    }
    int need = k - n_gt;
    if (n_eq == need) {
#pragma unroll
      for (int j = 0; j < 3; ++j) keep[j] |= eq[j];
    } else {
      for (; need > 0; --need) {
        int m = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 3; ++j)
          if (eq[j]) m = min(m, ix[j]);
        m = wave_min_i32(m);
#pragma unroll
        for (int j = 0; j < 3; ++j)
          if (eq[j] && ix[j] == m) {
            keep[j] = true;
            eq[j] = false;
          }
      }
    }
  }
  // the k-th best score: an element whose key equals theta_key
  float theta = 0.f;
#pragma unroll
  for (int j = 2; j >= 0; --j) {
    const uint64_t e = __ballot(v[j] && kk[j] == theta_key);
    if (e) theta = readlane_f(f[j], __builtin_ctzll(e));
  }
  int base = 0;
  int pos[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const uint64_t m = __ballot(keep[j]);
    pos[j] = base + mbcnt64(m);
    base += popc64(m);
  }
  // the reads above have returned (their values feed these stores)
#pragma unroll
  for (int j = 0; j < 3; ++j)
    if (keep[j]) {
      row_s[pos[j]] = f[j];
      row_i[pos[j]] = (uint16_t)ix[j];
    }
  wave_lds_sync();
  return theta;
}

// Merge every row of the wave at once.  Lane (g, col) holds a quarter of row
// col's kept entries (slots [g*KEEP/4, (g+1)*KEEP/4), valid below `kept`) and
// its own `cnt` candidates.  A row keeps the min(k, total) best of its
// `total` = kept + candidates entries (a row that has not yet seen k keys keeps
// them all and its threshold is unchanged).  The radix select runs per lane
// over its keys, with row counts summed over the row's 4 lanes by permlane
// swaps.  Rows with exact ties at the k-th value return fallback = true and
// are left untouched for merge_row_exact.
template <int KEEP>
__device__ void merge_rows_batched(float* row_s, uint16_t* row_i, int k, int kept, int cnt, int total, float& theta,
                                   bool& fallback) {
  constexpr int KQ = KEEP / 4;
  constexpr int CAP = sel_lane_cap(KEEP);
  constexpr int NK = KQ + CAP;
  static_assert(NK == kSelMergeKeys, "merge width");
  const int lane = lane_id();
  const int g = lane >> 4;
  const int kk = min(k, total);  // entries the row keeps
  const int kv = max(0, min(KQ, kept - g * KQ));
  const float* kept_s = row_s + g * KQ;
  const float* cand_s = row_s + KEEP + g * CAP;
  const uint16_t* kept_i = row_i + g * KQ;
  const uint16_t* cand_i = row_i + KEEP + g * CAP;
  uint32_t key[NK];
  int id[NK];
#pragma unroll
  for (int q = 0; q < NK / 4; ++q) {
    const bool kpt = 4 * q < KQ;
    const int o = kpt ? 4 * q : 4 * q - KQ;
    const int lim = kpt ? kv : cnt;
    const float4 s4 = *reinterpret_cast<const float4*>((kpt ? kept_s : cand_s) + o);
    const uint2 i4 = *reinterpret_cast<const uint2*>((kpt ? kept_i : cand_i) + o);
    key[4 * q + 0] = (o + 0 < lim) ? order_key(s4.x) : 0u;
    key[4 * q + 1] = (o + 1 < lim) ? order_key(s4.y) : 0u;
    key[4 * q + 2] = (o + 2 < lim) ? order_key(s4.z) : 0u;
    key[4 * q + 3] = (o + 3 < lim) ? order_key(s4.w) : 0u;
    id[4 * q + 0] = (int)(i4.x & 0xffffu);
    id[4 * q + 1] = (int)(i4.x >> 16);
    id[4 * q + 2] = (int)(i4.y & 0xffffu);
    id[4 * q + 3] = (int)(i4.y >> 16);
  }
  // valid keys are > 0 (order keys of finite or infinite floats are nonzero)
  uint32_t hi = 0, lo = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    hi = max(hi, key[i]);
    lo = min(lo, key[i] ? key[i] : 0xffffffffu);
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
  // a row whose entries all fit keeps every valid key
  bool done = total <= k;
  if (done) t = 1;
  for (int bit = wave_start; bit >= 0; --bit) {
    if (!__ballot(!done)) break;
    const uint32_t c = t | (1u << bit);
    int n = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) n += (key[i] >= c) ? 1 : 0;
    n = row_sum4(n);
    if (!done && n >= kk) {
      t = c;
      done = (n == kk);
    }
  }
  // winners: exactly kk keys >= t (done), or the k-th largest key is t itself
  uint64_t keep_bits = 0;
  uint32_t theta_key;
  bool tie_row = false;
  if (done) {
    uint32_t m = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const bool kp = key[i] >= t;
      keep_bits |= kp ? (1ull << i) : 0ull;
      m = kp ? min(m, key[i]) : m;
    }
    m = min(m, (uint32_t)xor16_i((int)m));
    m = min(m, (uint32_t)xor32_i((int)m));
    theta_key = m;
  } else {
    int gt = 0, eq = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      gt += (key[i] > t) ? 1 : 0;
      eq += (key[i] == t) ? 1 : 0;
    }
    gt = row_sum4(gt);
    eq = row_sum4(eq);
    tie_row = (eq != kk - gt);
#pragma unroll
    for (int i = 0; i < NK; ++i) keep_bits |= (key[i] >= t) ? (1ull << i) : 0ull;
    theta_key = t;
  }
  fallback = tie_row;
  // compact the winners of non-tie rows to kept slots [0, kk): lane g starts
  // after the winners of the row's lanes g' < g
  const int w = popc64(keep_bits);
  const int w1 = xor16_i(w);   // lane g ^ 1
  const int w2 = xor32_i(w);   // lane g ^ 2
  const int w3 = xor16_i(w2);  // lane g ^ 3
  int pos = ((g & 1) ? w1 : 0) + ((g & 2) ? (w2 + w3) : 0);
  if (!tie_row) {
    // the reads above have returned (their values feed these stores)
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      if ((keep_bits >> i) & 1ull) {
        row_s[pos] = key_to_float(key[i]);
        row_i[pos] = (uint16_t)id[i];
        ++pos;
      }
    }
    if (total >= k) theta = key_to_float(theta_key);
  }
  wave_lds_sync();
}

// VEC: r == 4*RQ and 16-byte aligned key rows -> float4 chunk loads.
template <int RQ, bool VEC, int KEEP>
__global__ __launch_bounds__(256, RQ > 16 ? 1 : 2) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr int CAP = sel_lane_cap(KEEP);
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
  const int ldk = (int)a.ldk;

  // ---- set-up -------------------------------------------------------------
  for (int i = tid; i < RP; i += blockDim.x) s_scale[i] = (i < a.r) ? (a.scale ? a.scale[i] : 1.0f) : 0.0f;
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

  // ---- key chunk loader: buffer loads relative to the chunk's first row;
  // rows past Nk (and padding columns) read as zeros and are masked later.
  // Two register sets hold the chunks two and three ahead of the one being
  // scored, so a load has two chunk iterations to return before its store.
  constexpr int kChunkVals = kSelChunk * RP;
  constexpr int kChunkF4 = kChunkVals / 4;
  constexpr int kLoads = VEC ? (kChunkF4 + 255) / 256 : (kChunkVals + 255) / 256;
  float4 pf4[2][VEC ? kLoads : 1];
  float pf1[2][VEC ? 1 : kLoads];
  // SET is a compile-time register set (std::integral_constant), so the
  // prefetch registers stay in VGPRs.
  auto load_chunk = [&](auto SET, int c) {
    constexpr int S = decltype(SET)::value;
    const int c0 = c * kSelChunk;
    const auto rs = make_rsrc(kbase + (int64_t)c0 * ldk, 0x80000000u);
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int f = tid + u * 256;
        if (kChunkF4 % 256 == 0 || f < kChunkF4) {
          const int rrow = f / RQ, c4 = f % RQ;
          pf4[S][u] = buf_load4(rs, c0 + rrow < a.Nk ? (uint32_t)(rrow * ldk + 4 * c4) * 4u : kOobOffset);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int e = tid + u * 256;
        const int rrow = e / RP, rc = e % RP;
        const bool ok = e < kChunkVals && rc < a.r && c0 + rrow < a.Nk;
        pf1[S][u] = buf_load1(rs, ok ? (uint32_t)(rrow * ldk + rc) * 4u : kOobOffset);
      }
    }
  };
  auto store_chunk = [&](auto SET) {
    constexpr int S = decltype(SET)::value;  // register set == LDS buffer
    if constexpr (VEC) {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int f = tid + u * 256;
        if (kChunkF4 % 256 == 0 || f < kChunkF4) {
          const int rrow = f / RQ, c4 = f % RQ;
          float4 v = pf4[S][u];
          if (scale_key) {
            const float4 sc = *reinterpret_cast<const float4*>(&s_scale[4 * c4]);
            v.x *= sc.x;
            v.y *= sc.y;
            v.z *= sc.z;
            v.w *= sc.w;
          }
          *reinterpret_cast<float4*>(&s_key[S][rrow * KSTRIDE + 4 * c4]) = v;
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kLoads; ++u) {
        const int e = tid + u * 256;
        if (e < kChunkVals) {
          const int rrow = e / RP, rc = e % RP;
          s_key[S][rrow * KSTRIDE + rc] = scale_key ? pf1[S][u] * s_scale[rc] : pf1[S][u];
        }
      }
    }
  };
  constexpr std::integral_constant<int, 0> kSet0{};
  constexpr std::integral_constant<int, 1> kSet1{};

  const int nchunks = (a.Nk + kSelChunk - 1) / kSelChunk;

  float theta = row_ok ? -INFINITY : INFINITY;  // invalid rows never admit
  int cnt = 0;   // candidates in this lane's region of its row
  int kept = 0;  // valid kept entries of this lane's row (<= k)
  float* my_slot_s = s_slot_s + lrow * kSelScoreStride;
  uint16_t* my_slot_i = s_slot_i + lrow * kSelIndexStride;
  float* my_cand_s = my_slot_s + KEEP + g * CAP;
  uint16_t* my_cand_i = my_slot_i + KEEP + g * CAP;

  // chunk c lives in register set c & 1 and LDS buffer c & 1
  load_chunk(kSet0, 0);
  store_chunk(kSet0);
  if (nchunks > 1) load_chunk(kSet1, 1);
  if (nchunks > 2) load_chunk(kSet0, 2);
  __syncthreads();

  for (int c = 0; c < nchunks; ++c) {
    const int cur = c & 1;
    const int c0 = c * kSelChunk;
    // chunk c + 1 into the other LDS buffer (read by everyone before the last
    // barrier), then reuse its registers for chunk c + 3
    if (c + 1 < nchunks) {
      if (cur == 0) {
        store_chunk(kSet1);
        if (c + 3 < nchunks) load_chunk(kSet1, c + 3);
      } else {
        store_chunk(kSet0);
        if (c + 3 < nchunks) load_chunk(kSet0, c + 3);
      }
    }

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
      for (int q = 0; q < RQ; ++q) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(k0[q], qf[q], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(k1[q], qf[q], acc1, 0, 0, 0);
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
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (sc[u] > theta) {
          my_cand_s[cnt] = sc[u];
          my_cand_i[cnt] = (uint16_t)(c0 + (u >> 2) * 16 + 4 * g + (u & 3));
          ++cnt;
        }
      }
    }

    // -- merge rows once a lane region is nearly full (or everything at the end) --
    const bool last = (c + 1 == nchunks);
    if (__ballot(cnt > CAP - 8 || (last && cnt > 0))) {
      wave_lds_sync();
      const int total = kept + row_sum4(cnt);
      bool fallback;
      merge_rows_batched<KEEP>(my_slot_s, my_slot_i, k, kept, cnt, total, theta, fallback);
      // rows with exact ties at the k-th value: exact per-row merge (such a
      // row holds more than k entries, so the merge fills it)
      uint64_t m = __ballot(lane < kSelRowsPerWave && fallback);
      while (m) {
        const int t = __builtin_ctzll(m);
        m &= m - 1;
        const int rc[4] = {readlane_i(cnt, t), readlane_i(cnt, t + 16), readlane_i(cnt, t + 32),
                           readlane_i(cnt, t + 48)};
        const int slot = wave * kSelRowsPerWave + t;
        const float th = merge_row_exact<KEEP>(s_slot_s + slot * kSelScoreStride, s_slot_i + slot * kSelIndexStride,
                                               k, readlane_i(kept, t), rc);
        if (col == t) theta = th;
      }
      if (!row_ok) theta = INFINITY;  // rows past Nq stay closed
      kept = min(k, total);
      cnt = 0;
    }
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
  JN_REQUIRE(a.ldk >= a.r && a.ldk < (1 << 22), kUnsupported, "key row stride must be in [r, 2^22) (got %lld)",
             (long long)a.ldk);
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
