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
//   * Each wave streams the keys itself, in chunks of 48 rows (three 16-row MFMA
//     tiles, A operand), loaded straight into VGPRs one chunk ahead.  The waves
//     of a workgroup share nothing but the LDS allocation, so no barrier
//     couples them: a wave that merges does not hold up the others.
//   * After a chunk, lane l holds 12 scores of row l%16.  Scores above the
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
constexpr int kSelTiles = 3;                           // 16-key MFMA tiles per chunk
constexpr int kSelChunk = 16 * kSelTiles;              // key rows per chunk
constexpr int kSelLaneKeys = 4 * kSelTiles;            // scores of one row per lane and chunk
// A row's slots: a kept region of KEEP entries (the k <= KEEP best so far;
// KEEP = 32 for k <= 32, 64 for k <= 64), then one candidate region of
// sel_lane_cap(KEEP) slots per lane of the row.  A lane takes at most
// kSelLaneKeys candidates per chunk, so merging once a lane holds more than
// cap - kSelLaneKeys keeps every region within its capacity.
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

// VEC: r == 4*RQ and 16-byte aligned key rows -> float4 key loads (RQ % 4 == 0).
template <int RQ, bool VEC, int KEEP>
__global__ __launch_bounds__(256, RQ > 16 ? 1 : 2) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr int CAP = sel_lane_cap(KEEP);
  constexpr bool V4 = VEC && RQ % 4 == 0;

  __shared__ __align__(16) float s_slot_s[kSelRows * kSelScoreStride];
  __shared__ __align__(16) uint16_t s_slot_i[kSelRows * kSelIndexStride];

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

  // ---- query fragment in registers, times the scale vector: both score forms
  // (scaled query or scaled key) equal sum_r q[r] * c[r] * key[r] ---------------
  const int lrow = wave * kSelRowsPerWave + col;  // row slot within the workgroup
  const int my_row = row0 + lrow;
  const bool row_ok = my_row < a.Nq;
  // unconditional loads (invalid rows and ranks read row 0 / rank 0 and are
  // zeroed after), so they all issue before one wait
  float qf[RQ];
  {
    const float* qrow = qb + (int64_t)(row_ok ? my_row : 0) * a.ldq;
    float qs[RQ];
#pragma unroll
    for (int s = 0; s < RQ; ++s) {
      const int rr = g * RQ + s;
      qf[s] = qrow[rr < a.r ? rr : 0];
      qs[s] = a.scale ? a.scale[rr < a.r ? rr : 0] : 1.0f;
    }
#pragma unroll
    for (int s = 0; s < RQ; ++s) qf[s] = (row_ok && g * RQ + s < a.r) ? qf[s] * qs[s] : 0.0f;
  }
  const float bias = a.bias ? a.bias[0] : 0.0f;
  // (dot + bias) / T as a multiply by the reciprocal: exact for T == 1, within
  // 1.5 ulp of the division otherwise
  const float inv_temp = 1.0f / a.temperature;

  // ---- key fragments straight from memory: every wave streams the keys on its
  // own (no LDS staging, no workgroup barrier in the loop), so a wave that
  // merges does not hold up the others.  Lane (g, col) reads key rows
  // c0 + col and c0 + 16 + col, ranks [g*RQ, g*RQ + RQ): the A operand of its
  // two MFMA tiles.  Buffer loads are relative to the chunk's first row; rows
  // past Nk read as zeros and are masked later.  Two register sets: the next
  // chunk loads while the current one is scored.
  // The resource of a chunk ends after its last row below Nk, so rows past
  // the end read as zeros with loop-invariant lane offsets.
  float kx[2][kSelTiles][RQ];
  uint32_t kbase_off[kSelTiles];
#pragma unroll
  for (int t = 0; t < kSelTiles; ++t) kbase_off[t] = (uint32_t)((16 * t + col) * ldk + g * RQ) * 4u;
  auto load_keys = [&](auto SET, int c) {
    constexpr int S = decltype(SET)::value;
    const int c0 = c * kSelChunk;
    const int rows = max(0, min(kSelChunk, a.Nk - c0));
    // uniform (readfirstlane keeps the resource in SGPRs)
    const uint32_t nrec = __builtin_amdgcn_readfirstlane((uint32_t)(rows * ldk) * 4u);
    const auto rs = make_rsrc(kbase + (int64_t)c0 * ldk, nrec);
#pragma unroll
    for (int t = 0; t < kSelTiles; ++t) {
      if constexpr (V4) {
#pragma unroll
        for (int q = 0; q < RQ / 4; ++q) {
          const float4 v = buf_load4(rs, kbase_off[t] + 16u * q);
          kx[S][t][4 * q + 0] = v.x;
          kx[S][t][4 * q + 1] = v.y;
          kx[S][t][4 * q + 2] = v.z;
          kx[S][t][4 * q + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < RQ; ++q) kx[S][t][q] = buf_load1(rs, (g * RQ + q < a.r) ? kbase_off[t] + 4u * q : kOobOffset);
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

  auto process = [&](auto SET, int c) {
    constexpr int S = decltype(SET)::value;
    const int c0 = c * kSelChunk;
    // -- scores for 32 keys x 16 query rows (two MFMA tiles) --
    floatx4 acc[kSelTiles];
#pragma unroll
    for (int t = 0; t < kSelTiles; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < RQ; ++q)
#pragma unroll
      for (int t = 0; t < kSelTiles; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kx[S][t][q], qf[q], acc[t], 0, 0, 0);

    // -- threshold filter: lane holds keys c0 + 16t + 4g + v of its row --
    float sc[kSelLaneKeys];
#pragma unroll
    for (int u = 0; u < kSelLaneKeys; ++u) sc[u] = acc[u >> 2][u & 3];
    if (inv_temp != 1.0f) {  // uniform
#pragma unroll
      for (int u = 0; u < kSelLaneKeys; ++u) sc[u] = (sc[u] + bias) * inv_temp;
    } else if (bias != 0.0f) {
#pragma unroll
      for (int u = 0; u < kSelLaneKeys; ++u) sc[u] += bias;
    }
    if (c0 + kSelChunk > a.Nk) {  // uniform: only the last chunk holds padding keys
#pragma unroll
      for (int u = 0; u < kSelLaneKeys; ++u)
        if (c0 + (u >> 2) * 16 + 4 * g + (u & 3) >= a.Nk) sc[u] = -INFINITY;
    }
    uint64_t any = 0;
#pragma unroll
    for (int u = 0; u < kSelLaneKeys; ++u) any |= __ballot(sc[u] > theta);
    if (any) {
      // branchless append: every entry is written at the running count, which
      // advances only past candidates, so the next write overwrites a
      // rejected entry (cnt <= CAP - kSelLaneKeys on entry keeps every write in
      // the region)
#pragma unroll
      for (int u = 0; u < kSelLaneKeys; ++u) {
        my_cand_s[cnt] = sc[u];
        my_cand_i[cnt] = (uint16_t)(c0 + (u >> 2) * 16 + 4 * g + (u & 3));
        cnt += (sc[u] > theta) ? 1 : 0;
      }
    }

    // -- merge rows once a lane region is nearly full (or everything at the end) --
    const bool last = (c + 1 == nchunks);
    if (__ballot(cnt > CAP - kSelLaneKeys || (last && cnt > 0))) {
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
  };

  // chunk c lives in register set c & 1.  The loads are unconditional (chunks
  // past the end read rows >= Nk: zeros, no memory access), so the wait before
  // a chunk's MFMAs covers only its own loads, not the prefetch behind them.
  load_keys(kSet0, 0);
  for (int c = 0; c < nchunks; c += 2) {
    load_keys(kSet1, c + 1);
    process(kSet0, c);
    if (c + 1 < nchunks) {
      load_keys(kSet0, c + 2);
      process(kSet1, c + 1);
    }
  }
  wave_lds_sync();

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
