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
// Three forms share the scoring, filter, merge and sort code below:
//   * per-wave (described next): every wave streams all keys itself;
//   * cooperative (rank <= 64, large grids): the workgroup stages each key
//     chunk once in LDS and every wave reads its fragments from there, with a
//     barrier per chunk and workgroup-wide merges (see the kernel template);
//   * key-split (k <= 16, small grids): the four waves share 16 query rows,
//     each over a quarter of the keys, merged by one sort per row at the end.
//
// Layout of one per-wave workgroup (256 threads = 4 waves, 64 query rows):
//   * 16 query rows per wave.  A wave keeps the query fragment of its rows in
//     VGPRs for the whole kernel (B operand of the MFMAs; lane l owns row
//     l%16, rank slice l/16).
//   * Each wave streams the keys itself, in chunks of 48 rows (three 16-row MFMA
//     tiles, A operand), loaded straight into VGPRs one chunk ahead.  The waves
//     of a workgroup share nothing but the LDS allocation, so no barrier
//     couples them: a wave that merges does not hold up the others.
//   * After a chunk, lane l holds 12 scores of row l%16.  Scores above the
//     row's threshold theta are appended to the lane's own candidate region
//     of the row (the row's 4 lanes never share a region, so appends need no
//     cross-lane offsets; regions are stored slot-major per wave, so the
//     appends are free of bank conflicts).  Counts and thresholds live in
//     registers.
//   * Once any lane of a wave has filled its region to within one chunk of
//     its capacity (or at the end), all 16 rows of the wave merge together:
//     lane (g, row) loads a quarter of the row's kept entries (held as order
//     keys) and its own candidates into registers, and a threshold search
//     over order keys counts per lane and sums over the row's 4 lanes with
//     permlane swaps: probes interpolated in score value between a bracket of
//     keys, bisection in key space after eight probes.  A merge during the
//     scan stops as soon as the entries at or above its probe fit the kept
//     region (between k and 48 of them for k <= 32): any threshold not above
//     the k-th best filters safely, and the probe becomes the row's threshold.
//     The merge after the last chunk keeps exactly k.  Winners are compacted
//     into the row's kept region without branches.  A row whose k-th value is
//     tied (more equal keys than places) is merged again by the exact per-row
//     path, which keeps the lower key indices.  The kept set stays unsorted
//     until one bitonic sort per row at the end (DPP and permlane exchanges).
//   * Score arithmetic: fp16 MFMAs over two-term fp16 splits of the operands
//     (see select_split_keys_kernel), or fp32 MFMAs (select mode 1), or, for
//     bf16 layers, bf16 MFMAs over bf16 operands (select_bf16_keys_kernel).
#include <atomic>
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
// A row's slots: a kept region of KEEP entries, then one candidate region of
// sel_lane_cap(KEEP) slots per lane of the row.  The kept region holds between
// k and KEEP of the best entries so far: a merge during the scan only needs a
// threshold no higher than the k-th best, so it stops as soon as the number of
// entries at or above its threshold fits (KEEP = 48 for k <= 32, 80 for
// k <= 64); the merge after the last chunk keeps exactly k.  A lane takes at
// most kSelLaneKeys candidates per chunk, so merging once a lane holds more
// than cap - kSelLaneKeys keeps every region within its capacity.
// Candidate regions are stored slot-major per wave: slot j of lane l is word
// j * 64 + l of the wave's candidate array, so the 64 appends of a wave (each
// lane at its own count) and a merge's per-slot reads hit 64 distinct banks.
constexpr int kSelRowSlots = 160;
__host__ __device__ constexpr int sel_lane_cap(int keep) { return (kSelRowSlots - keep) / 4; }
__host__ __device__ constexpr int sel_keep_for(int k) { return k <= 32 ? 48 : 80; }
static_assert(sel_lane_cap(48) % 4 == 0 && sel_lane_cap(80) % 4 == 0, "candidate regions hold whole float4s");
static_assert(48 / 4 + sel_lane_cap(48) == 80 / 4 + sel_lane_cap(80), "both kept-region sizes merge as many keys");
static_assert(sel_keep_for(32) - 32 >= 16 && sel_keep_for(64) - 64 >= 16, "kept regions leave room above k");
constexpr int kSelMergeKeys = 48 / 4 + sel_lane_cap(48);  // keys per lane in a batched merge (40)
// Kept rows are KEEP + 4 scores / KEEP + 8 indices apart: 16-byte multiples
// (vector reads) that shift successive rows by 52 or 84 (scores) and 28 or 44
// (indices) banks.
__host__ __device__ constexpr int sel_kept_stride(int keep) { return keep + 4; }
__host__ __device__ constexpr int sel_kept_idx_stride(int keep) { return keep + 8; }
constexpr int kSelMaxKeys = 65535;    // key indices are stored as uint16

// Monotone map float -> uint32 (larger float -> larger key); -0 and +0 map together.
__device__ __forceinline__ uint32_t order_key(float s) {
  uint32_t u = __float_as_uint(s + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Exchange with lane ^ stride (stride a constant once the sort loops below
// unroll), all VALU: DPP quad permutes for 1 and 2, a row shift each way for
// 4 (lanes with bit 2 clear read lane + 4, the others lane - 4, both within
// the 16-lane row), a rotation of the row by 8 for 8, the permlane swaps for
// 16 and 32.
__device__ __forceinline__ int sort_xor_i(int v, int stride) {
  if (stride == 1) return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
  if (stride == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
  if (stride == 4) {
    const int up = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xf, 0xf, false);  // row_shl:4 (lane + 4)
    const int dn = __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false);  // row_shr:4 (lane - 4)
    return (lane_id() & 4) ? dn : up;
  }
  if (stride == 8) return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);  // row_ror:8
  if (stride == 16) return xor16_i(v);
  if (stride == 32) return xor32_i(v);
  return shfl_xor_i(v, stride);
}
__device__ __forceinline__ float sort_xor_f(float v, int stride) {
  return __int_as_float(sort_xor_i(__float_as_int(v), stride));
}

// Branchless bitonic sort of 64 (score, index) pairs into descending score,
// ascending index on ties.
__device__ __forceinline__ void bitonic_sort64_desc(float& vs, int& vi) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float ps = sort_xor_f(vs, stride);
      const int pi = sort_xor_i(vi, stride);
      const bool partner_better = (ps > vs) | ((ps == vs) & (pi < vi));
      const bool self_better = (vs > ps) | ((vs == ps) & (vi < pi));
      const bool keep_better = ((lane & stride) == 0) == ((lane & size) == 0);
      const bool take = keep_better ? partner_better : self_better;
      vs = take ? ps : vs;
      vi = take ? pi : vi;
    }
  }
}

// The same network on each half-wave: two independent 32-entry sorts (the
// final merge stage leaves both halves descending).
__device__ __forceinline__ void bitonic_sort32x2_desc(float& vs, int& vi) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 32; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float ps = sort_xor_f(vs, stride);
      const int pi = sort_xor_i(vi, stride);
      const bool partner_better = (ps > vs) | ((ps == vs) & (pi < vi));
      const bool self_better = (vs > ps) | ((vs == ps) & (vi < pi));
      const bool keep_better = ((lane & stride) == 0) == ((lane & size & 31) == 0);
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

// Exact merge of row `trow` of the wave by the whole wave: keep the k best
// (ties toward the lower key index) of its `kept` kept entries and the c_g
// candidates of lane region g (lane g * 16 + trow of the wave's slot-major
// candidate arrays), compacted to kept slots [0, k); k < kept + sum(c).
// Kept slots hold order keys.  Returns the new k-th best score
// (wave-uniform).  Lane l holds row slots l, l + 64, l + 128 (kept slots
// first, then region 0, 1, 2, 3).
template <int KEEP>
__device__ float merge_row_exact(uint32_t* row_k, uint16_t* row_i, const float* cand_s, const uint16_t* cand_i, int trow,
                                 int k, int kept, int c0, int c1, int c2, int c3) {
  constexpr int CAP = sel_lane_cap(KEEP);
  const int lane = lane_id();
  int ix[3];
  uint32_t kk[3];
  bool v[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int s = lane + 64 * j;
    bool ok;
    int w = 0;  // word of the slot in the candidate arrays
    if (s < KEEP) {
      ok = s < kept;
    } else if (s < kSelRowSlots) {
      const int rg = (s - KEEP) / CAP;
      const int ri = s - KEEP - rg * CAP;
      const int cr = rg == 0 ? c0 : rg == 1 ? c1 : rg == 2 ? c2 : c3;
      ok = ri < cr;
      w = ri * kWave + rg * 16 + trow;
    } else {
      ok = false;
    }
    v[j] = ok;
    ix[j] = ok ? (int)(s < KEEP ? row_i[s] : cand_i[w]) : 0;
    kk[j] = ok ? (s < KEEP ? row_k[s] : order_key(cand_s[w])) : 0u;
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
  // the k-th best score
  const float theta = key_to_float(theta_key);
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
      row_k[pos[j]] = kk[j];
      row_i[pos[j]] = (uint16_t)ix[j];
    }
  wave_lds_sync();
  return theta;
}

// Merge every row of the wave at once.  Lane (g, col) holds a quarter of row
// col's kept entries (slots [g*KEEP/4, (g+1)*KEEP/4), valid below `kept`) and
// its own `cnt` candidates.  Of its `total` = kept + candidates entries a row
// keeps every entry at or above a threshold t with kk <= count(>= t) <= hi,
// kk = min(k, total): hi = kk in the final merge (exactly the kk best), up to
// KEEP during the scan, where any t not above the k-th best serves and the
// search stops as soon as the count fits.  Kept slots hold order keys.  The
// search probes order keys per lane (below), with row counts summed over the
// row's 4 lanes by permlane swaps.  Only the first `cq` quads of each candidate region (the
// wave's largest candidate count, rounded up to 4) are read and searched: a
// wave that merges because another wave of its workgroup had to merges only
// what it holds.  Returns the row's kept count (or -1 for a row with exact
// ties at t that the window cannot separate: its slots are left untouched
// for merge_row_exact).  Once the row has seen k keys its threshold becomes
// the score of t (no higher than its smallest kept entry), else it stays
// `theta`.
struct MergeResult {
  int kept;     // entries now in the kept region, -1 for a tie row
  float theta;  // the row's new threshold
};

template <int KEEP>
__device__ __forceinline__ MergeResult merge_rows_batched(uint32_t* row_k, uint16_t* row_i, float* cand_s, uint16_t* cand_i,
                                                          int k, int kept, int cnt, int total, int hi_target, float theta,
                                                          int cq) {
  constexpr int KQ = KEEP / 4;
  constexpr int CAP = sel_lane_cap(KEEP);
  constexpr int NK = KQ + CAP;
  static_assert(NK == kSelMergeKeys, "merge width");
  const int lane = lane_id();
  const int g = lane >> 4;
  const int kk = min(k, total);  // entries the row keeps at least
  const int hi = max(kk, min(hi_target, KEEP));
  const int kv = max(0, min(KQ, kept - g * KQ));
  const uint32_t* kept_k = row_k + g * KQ;
  const uint16_t* kept_i = row_i + g * KQ;
  uint32_t key[NK];
  int id[NK];
  // quad q of the lane's keys is in use (wave-uniform; q is a constant in
  // every unrolled loop below, so each test is one scalar branch)
  auto act = [&](int q) { return 4 * q < KQ || q - KQ / 4 < cq; };
  // Every load of the active quads is issued first and each value passes an
  // empty asm before its validity select: left alone, the compiler turns
  // "valid ? f(load) : 0" into a branch around the load and waits for each
  // load on its own.
  uint32_t sv[NK];  // order keys (kept slots) or score bits (candidates)
#pragma unroll
  for (int q = 0; q < NK / 4; ++q) {
    if (!act(q)) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sv[4 * q + v] = 0u;
        id[4 * q + v] = 0;
      }
      continue;
    }
    if (4 * q < KQ) {
      const int o = 4 * q;
      const uint4 s4 = *reinterpret_cast<const uint4*>(kept_k + o);
      const uint2 i4 = *reinterpret_cast<const uint2*>(kept_i + o);
      sv[4 * q + 0] = s4.x;
      sv[4 * q + 1] = s4.y;
      sv[4 * q + 2] = s4.z;
      sv[4 * q + 3] = s4.w;
      id[4 * q + 0] = (int)(i4.x & 0xffffu);
      id[4 * q + 1] = (int)(i4.x >> 16);
      id[4 * q + 2] = (int)(i4.y & 0xffffu);
      id[4 * q + 3] = (int)(i4.y >> 16);
    } else {
      const int o = 4 * q - KQ;  // candidate slots o .. o + 3 of this lane
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sv[4 * q + v] = __float_as_uint(cand_s[(o + v) * kWave]);
        id[4 * q + v] = (int)cand_i[(o + v) * kWave];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NK / 4; ++q) {
    const bool kpt = 4 * q < KQ;
    const int o = kpt ? 4 * q : 4 * q - KQ;
    const int lim = kpt ? kv : cnt;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      uint32_t x = sv[4 * q + v];
      if (act(q)) asm volatile("" : "+v"(x));
      key[4 * q + v] = (act(q) && o + v < lim) ? (kpt ? x : order_key(__uint_as_float(x))) : 0u;
    }
  }
  // valid keys are > 0 (order keys of finite or infinite floats are nonzero)
  uint32_t khi = 0, klo = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    if (!act(i / 4)) continue;
    khi = max(khi, key[i]);
    klo = min(klo, key[i] ? key[i] : 0xffffffffu);
  }
  khi = max(khi, (uint32_t)xor16_i((int)khi));
  khi = max(khi, (uint32_t)xor32_i((int)khi));
  klo = min(klo, (uint32_t)xor16_i((int)klo));
  klo = min(klo, (uint32_t)xor32_i((int)klo));
  // A row whose entries all fit keeps every valid key (t = 1: every valid key
  // is >= 1).  Otherwise the search keeps a bracket of order keys a <= b with
  // count(>= a) = ca > hi and count(> b) = cb < kk and probes a key c in
  // (a, b]: interpolated in score value toward a count of (kk + hi) / 2
  // (regula falsi; scores near the threshold are close to linear in rank), or
  // halfway in key space once eight probes have not landed (at most 32 more).
  // A probe whose count lies in [kk, hi] ends the row's search with t = c; a
  // bracket that closes (a == b) leaves the kk-th largest key tied at t = a
  // with more copies than the window holds.
  bool done = total <= hi;
  uint32_t t = done ? 1u : klo;
  int wl = done ? kv + cnt : 0;  // this lane's entries >= t once done
  uint32_t ba = klo, bb = khi;
  float ca = (float)total, cb = 0.0f;
  const float target = 0.5f * (float)(kk + hi);
  for (int it = 0; __ballot(!done && ba != bb); ++it) {
    const uint32_t mid = ba + ((bb - ba) >> 1) + 1u;  // in (ba, bb] when ba < bb
    const float fa = key_to_float(ba), fb = key_to_float(bb);
    const float frac = (ca - target) * __builtin_amdgcn_rcpf(ca - cb);
    const uint32_t ci = order_key(fmaf(fb - fa, frac, fa));
    const uint32_t c = (it < 8 && ci > ba && ci <= bb) ? ci : mid;
    int n = 0;
#pragma unroll
    for (int q = 0; q < NK / 4; ++q) {
      if (!act(q)) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) n += (key[4 * q + v] >= c) ? 1 : 0;
    }
    const int nl = n;
    n = row_sum4(n);
    if (!done && ba != bb) {
      if (n > hi) {
        ba = c;
        ca = (float)n;
      } else if (n < kk) {
        bb = c - 1u;
        cb = (float)n;
      } else {
        t = c;
        done = true;
        wl = nl;
      }
    }
  }
  // Winners: the keys >= t.  A row whose search did not land (its kk-th
  // largest key is tied at ba with more copies than the window holds) is left
  // to merge_row_exact.
  const bool tie_row = !done;
  // compact the winners of non-tie rows to kept slots [0, n): lane g starts
  // after the winners of the row's lanes g' < g.  Branch-free: a lane writes
  // every entry, losers to a slot of its own candidate region (dead after the
  // merge), so no lane writes over another's winners.
  const int w1 = xor16_i(wl);  // lane g ^ 1
  const int w2 = xor32_i(wl);  // lane g ^ 2
  const int w3 = xor16_i(w2);  // lane g ^ 3
  const int n_row = wl + w1 + w2 + w3;
  int pos = ((g & 1) ? w1 : 0) + ((g & 2) ? (w2 + w3) : 0);
  if (!tie_row) {
    uint32_t* trash_k = reinterpret_cast<uint32_t*>(cand_s) + (CAP - 1) * kWave;
    uint16_t* trash_i = cand_i + (CAP - 1) * kWave;
    // the reads above have returned (their values feed these stores)
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      if (!act(i / 4)) continue;
      const bool kp = key[i] >= t;
      *(kp ? row_k + pos : trash_k) = key[i];
      *(kp ? row_i + pos : trash_i) = (uint16_t)id[i];
      pos += kp ? 1 : 0;
    }
    // t = 1 keeps every entry: the threshold is then the smallest of them
    if (total >= k) theta = key_to_float(total <= hi ? klo : t);
  }
  wave_lds_sync();
  return MergeResult{tie_row ? -1 : n_row, theta};
}

// ---- split-fp16 score operands ------------------------------------------------
// A value x, first scaled by a power of two 2^e that puts the largest magnitude
// of its group in [2^14, 2^15), is carried as hi = fp16(x), lo = fp16(x - hi):
// |x - hi - lo| <= 2^-22 |x| with no fp16 overflow.  A score is then
//   q.k = 2^-(eq+ek) * (hi_q.hi_k + hi_q.lo_k + lo_q.hi_k)   (+ lo_q.lo_k, dropped)
// with each product exact in fp32 and an error of about 3 * 2^-22 sum_r |q_r k_r|,
// the size of fp32 accumulation error over a rank-64 dot product.  Keys share
// one exponent per batch element (so a score needs no per-key factor); a query
// row has its own, applied in registers.
// Split key rows: [hi: RP halves][lo: RP halves], RP = r rounded up to 32 (the
// K extent of one v_mfma_f32_16x16x32_f16); ranks past r are zero.
constexpr int kSplitRows = 64;  // key rows per block of the two prep kernels

__device__ __forceinline__ int split_exponent(float maxabs) {
  int e = 0;
  if (!(maxabs > 0.0f) || !(maxabs < INFINITY)) return 0;  // zeros, inf, NaN: unscaled
  (void)frexpf(maxabs, &e);                                // maxabs in [2^(e-1), 2^e)
  return 15 - e;
}

__device__ __forceinline__ float block_max_256(float m) {
  __shared__ float s_max[4];
  m = wave_max_f(m);
  if (lane_id() == 0) s_max[threadIdx.x / kWave] = m;
  __syncthreads();
  return fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
}

// partial[b][blk] = max |key| over rows [64 blk, 64 blk + 64) of batch element b.
__global__ __launch_bounds__(256) void select_split_absmax_kernel(const float* __restrict__ key, int64_t ldk,
                                                                  int64_t kbs, int Nk, int r, int nblk,
                                                                  float* __restrict__ partial) {
  const int blk = blockIdx.x, b = blockIdx.y;
  const int row0 = blk * kSplitRows;
  const int rows = min(kSplitRows, Nk - row0);
  const float* kb = key + (int64_t)b * kbs + (int64_t)row0 * ldk;
  float m = 0.0f;
  // four ranks per thread when rows are whole aligned float4s
  if (r % 4 == 0 && ldk % 4 == 0 && kbs % 4 == 0 && (reinterpret_cast<uintptr_t>(key) & 15) == 0) {
    const int r4 = r / 4;
    for (int e = threadIdx.x; e < rows * r4; e += 256) {
      const int row = e / r4;
      const float4 v = *reinterpret_cast<const float4*>(kb + (int64_t)row * ldk + 4 * (e - row * r4));
      m = fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
    }
  } else {
    for (int e = threadIdx.x; e < rows * r; e += 256) {
      const int row = e / r;
      m = fmaxf(m, fabsf(kb[(int64_t)row * ldk + (e - row * r)]));
    }
  }
  m = block_max_256(m);
  if (threadIdx.x == 0) partial[(int64_t)b * nblk + blk] = m;
}

// Writes the split rows of [64 blk, 64 blk + 64) and, from block 0, the batch
// element's key exponent.  Every block reduces the same partials in the same
// order, so all agree on the exponent.
// Split position c of a row holds rank h * head_rank + (c - h * head_rp) of head
// h = c / head_rp (zero past head_rank): each head starts on a whole K-step.
// One head: head_rank = r, head_rp = RP.
__global__ __launch_bounds__(256) void select_split_keys_kernel(const float* __restrict__ key, int64_t ldk,
                                                                int64_t kbs, int Nk, int head_rank, int head_rp,
                                                                int RP, int nblk, const float* __restrict__ partial,
                                                                _Float16* __restrict__ split, int* __restrict__ kexp) {
  const int blk = blockIdx.x, b = blockIdx.y;
  float m = 0.0f;
  for (int i = threadIdx.x; i < nblk; i += 256) m = fmaxf(m, partial[(int64_t)b * nblk + i]);
  const int ek = split_exponent(block_max_256(m));
  if (blk == 0 && threadIdx.x == 0) kexp[b] = ek;
  const int row0 = blk * kSplitRows;
  const int rows = min(kSplitRows, Nk - row0);
  const float* kb = key + (int64_t)b * kbs + (int64_t)row0 * ldk;
  _Float16* out = split + ((int64_t)b * Nk + row0) * (2 * RP);
  // four split positions per thread (one 16-byte key load, two 8-byte stores)
  // when the head's ranks come in aligned fours; the same arithmetic per element
  if (head_rank % 4 == 0 && ldk % 4 == 0 && kbs % 4 == 0 && (reinterpret_cast<uintptr_t>(key) & 15) == 0) {
    const int RP4 = RP / 4;  // RP and head_rp are multiples of 32
    for (int e = threadIdx.x; e < rows * RP4; e += 256) {
      const int row = e / RP4;
      const int c = 4 * (e - row * RP4);
      const int h = c / head_rp, cc = c - h * head_rp;
      float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
      if (cc < head_rank) {  // then cc + 3 < head_rank too
        x = *reinterpret_cast<const float4*>(kb + (int64_t)row * ldk + h * head_rank + cc);
        x = make_float4(ldexpf(x.x, ek), ldexpf(x.y, ek), ldexpf(x.z, ek), ldexpf(x.w, ek));
      }
      typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));
      halfx4 hi, lo;
      hi[0] = (_Float16)x.x; hi[1] = (_Float16)x.y; hi[2] = (_Float16)x.z; hi[3] = (_Float16)x.w;
      lo[0] = (_Float16)(x.x - (float)hi[0]);
      lo[1] = (_Float16)(x.y - (float)hi[1]);
      lo[2] = (_Float16)(x.z - (float)hi[2]);
      lo[3] = (_Float16)(x.w - (float)hi[3]);
      *reinterpret_cast<halfx4*>(&out[(int64_t)row * 2 * RP + c]) = hi;
      *reinterpret_cast<halfx4*>(&out[(int64_t)row * 2 * RP + RP + c]) = lo;
    }
    return;
  }
  for (int e = threadIdx.x; e < rows * RP; e += 256) {
    const int row = e / RP;
    const int c = e - row * RP;
    const int h = c / head_rp, cc = c - h * head_rp;
    const float x = cc < head_rank ? ldexpf(kb[(int64_t)row * ldk + h * head_rank + cc], ek) : 0.0f;
    const _Float16 hi = (_Float16)x;
    out[(int64_t)row * 2 * RP + c] = hi;
    out[(int64_t)row * 2 * RP + RP + c] = (_Float16)(x - (float)hi);
  }
}

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ---- bf16 score operands (bf16 layers) ---------------------------------------
// Key rows rounded to bf16 (nearest even), [RP] each with ranks past r zero:
// one plane of the split row layout.  The query is scaled by the core weight
// and rounded to bf16 in registers, so a score is the fp32-accumulated dot
// product of two bf16 vectors, (bf16(q * c) . bf16(key)), on
// v_mfma_f32_16x16x32_bf16 -- one MFMA per K-step where the split path
// issues three.
__global__ __launch_bounds__(256) void select_bf16_keys_kernel(const float* __restrict__ key, int64_t ldk,
                                                               int64_t kbs, int Nk, int r, int RP,
                                                               bf16_t* __restrict__ out_rows) {
  const int blk = blockIdx.x, b = blockIdx.y;
  const int row0 = blk * kSplitRows;
  const int rows = min(kSplitRows, Nk - row0);
  const float* kb = key + (int64_t)b * kbs + (int64_t)row0 * ldk;
  bf16_t* out = out_rows + ((int64_t)b * Nk + row0) * RP;
  for (int e = threadIdx.x; e < rows * RP; e += 256) {
    const int row = e / RP;
    const int c = e - row * RP;
    out[(int64_t)row * RP + c] = (bf16_t)(c < r ? kb[(int64_t)row * ldk + c] : 0.0f);
  }
}

__device__ __forceinline__ halfx8 as_halfx8(float a, float b, float c, float d) {
  return __builtin_bit_cast(halfx8, floatx4{a, b, c, d});
}

// VEC: r == 4*RQ and 16-byte aligned key rows -> float4 key loads (RQ % 4 == 0).
// KS > 0: split-fp16 scores over KS K-steps of 32 ranks (RQ and VEC unused);
// the keys are the split rows in a.ws, the queries are split in registers.
// COOP (split keys of rank <= 64 only): 8 waves, 128 query rows, one workgroup
// per CU.  The workgroup stages each key chunk once in LDS (double-buffered,
// one barrier per chunk) and every wave reads its MFMA fragments from there,
// instead of each wave streaming all keys through L1 on its own: per CU that
// is one global read of each key chunk instead of eight.  A wave that needs
// to merge raises a workgroup flag before the barrier and then every wave
// merges after it, so a merge holds up no other wave at the next barrier.
// CW = 4 is the same with 4 waves (64 rows) and one staging buffer (two
// barriers per chunk), two workgroups per CU whose phases drift apart.
// CW = -1 (k <= 16, small grids): the per-wave form with the four waves of a
// workgroup on the same 16 query rows, each over a quarter of the key chunks;
// each keeps the exact top-k of its quarter, and a 64-entry sort per row
// merges the four lists at the end.  Four times the workgroups and a quarter
// of the serial chunk chain per wave.
// MH (split keys, per-wave form only): multi-head max aggregation.  Head h owns
// K-steps [h * head_ks, (h + 1) * head_ks) of the split rows; after a head's
// last K-step its scores, unscaled and with its bias, are folded into a
// running maximum, so the filter and merges see max_h (dot_h + bias[h]) / T.
// BF (split layout, one plane): bf16 key rows and bf16 MFMAs (bf16 layers).
template <int RQ, bool VEC, int KEEP, int KS, int CW, bool MH = false, bool BF = false>
__global__ __launch_bounds__(CW > 0 ? CW * 64 : 256,
                             CW == 8 ? 1 : CW == 4 ? 2 : ((KS > 0 ? KS > 2 : RQ > 16) ? 1 : 2)) void lowrank_topk_select_kernel(SelectArgs a) {
  constexpr bool COOP = CW > 0;
  constexpr bool KSP = CW < 0;
  constexpr int NT = COOP ? CW * kWave : 256;  // threads
  constexpr int NBUF = CW == 8 ? 2 : 1;        // staging buffers
  constexpr int CAP = sel_lane_cap(KEEP);
  constexpr bool SPLIT = KS > 0;
  constexpr bool V4 = VEC && RQ % 4 == 0;
  constexpr int PLANES = BF ? 1 : 2;                  // split rows: fp16 hi + lo planes, or one bf16 plane
  constexpr int FR = SPLIT ? 4 * PLANES * KS : RQ;    // key fragment registers per tile
  constexpr int RP = 32 * KS;                         // split row: ranks per plane
  constexpr int ROWS = COOP ? CW * kSelRowsPerWave : KSP ? kSelRowsPerWave : kSelRows;  // query rows per workgroup
  constexpr int SLOTS = COOP ? CW * kSelRowsPerWave : kSelRows;  // row slots (16 per wave)
  static_assert(!KSP || KEEP == 48, "the key-split form serves k <= 16");
  static_assert(!COOP || (KS >= 1 && KS <= 2), "the cooperative select stages split keys of rank <= 64");
  static_assert(!MH || (SPLIT && CW == 0), "multi-head scores run on the per-wave split kernel");
  static_assert(!BF || (SPLIT && !MH), "bf16 operands use the split layout with one head");
  // staged chunk: kSelChunk split rows of PLANES RP halves plus 8 halves of
  // padding, so the 16 rows one fragment read touches start 4 banks apart
  constexpr int KROW = PLANES * RP + 8;
  constexpr int KBUF = kSelChunk * KROW;
  constexpr int F4 = kSelChunk * PLANES * RP / 8;  // float4s per staged chunk
  constexpr int PER = (F4 + NT - 1) / NT;  // of them per thread

  constexpr int KST = sel_kept_stride(KEEP), KIST = sel_kept_idx_stride(KEEP);
  __shared__ __align__(16) uint32_t s_kept_k[SLOTS * KST];  // order keys
  __shared__ __align__(16) uint16_t s_kept_i[SLOTS * KIST];
  __shared__ __align__(16) float s_cand_s[SLOTS / kSelRowsPerWave * CAP * kWave];
  __shared__ __align__(16) uint16_t s_cand_i[SLOTS / kSelRowsPerWave * CAP * kWave];
  __shared__ __align__(16) _Float16 s_key[COOP ? NBUF * KBUF : 8];
  __shared__ int s_flag[3];

  const int lane = lane_id();
  const int wave = wave_id();
  const int g = lane >> 4;    // rank slice owned by this lane group
  const int col = lane & 15;  // query row within the wave's 16

  const int tiles_per_batch = (a.Nq + ROWS - 1) / ROWS;
  const int logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int b = logical / tiles_per_batch;
  const int row0 = (logical % tiles_per_batch) * ROWS;
  if (b >= a.B) return;

  const float* qb = a.q + (int64_t)b * a.q_batch_stride;
  const float* kbase = a.key + (int64_t)b * a.k_batch_stride;
  const int k = a.k;
  const int ldk = (int)a.ldk;
  // key chunks of this wave: all of them, or a quarter in the key-split form
  const int nchunks_all = (a.Nk + kSelChunk - 1) / kSelChunk;
  int chunk0 = 0, nchunks = nchunks_all, key_end = a.Nk;
  if constexpr (KSP) {
    const int per = (nchunks_all + kSelWaves - 1) / kSelWaves;
    chunk0 = min(nchunks_all, wave * per);
    nchunks = min(nchunks_all, chunk0 + per) - chunk0;
    key_end = min(a.Nk, (chunk0 + nchunks) * kSelChunk);
  }

  // ---- query fragment in registers, times the scale vector: both score forms
  // (scaled query or scaled key) equal sum_r q[r] * c[r] * key[r] ---------------
  const int lrow = wave * kSelRowsPerWave + col;  // row slot within the workgroup
  const int my_row = row0 + (KSP ? col : lrow);
  const bool row_ok = my_row < a.Nq;
  // unconditional loads (invalid rows and ranks read row 0 / rank 0 and are
  // zeroed after), so they all issue before one wait
  // fp32 path: lane (g, col) holds ranks g*RQ + s of row col (K-step s).
  // Split path: ranks 32 s + 8 g + e (K-step s, e < 8), as hi/lo halves, and
  // the row's score exponent E: MFMA results are the scores times 2^E.
  constexpr int QN = SPLIT ? 8 * KS : RQ;
  // MH: K-steps per head (each head's ranks padded to whole K-steps)
  const int head_ks = MH ? (a.head_rank + 31) / 32 : KS;
  // source rank of fragment slot s, or -1 for padding
  auto qrank = [&](int s) {
    if constexpr (MH) {
      const int ks = s / 8, h = ks / head_ks, c = 32 * (ks - h * head_ks) + 8 * g + (s % 8);
      return (h < a.heads && c < a.head_rank) ? h * a.head_rank + c : -1;
    } else {
      const int rr = SPLIT ? 32 * (s / 8) + 8 * g + (s % 8) : g * RQ + s;
      return rr < a.r ? rr : -1;
    }
  };
  float qf[QN];
  {
    const float* qrow = qb + (int64_t)(row_ok ? my_row : 0) * a.ldq;
    float qs[QN];
#pragma unroll
    for (int s = 0; s < QN; ++s) {
      const int rr = qrank(s);
      qf[s] = qrow[rr >= 0 ? rr : 0];
      qs[s] = a.scale ? a.scale[rr >= 0 ? rr : 0] : 1.0f;
    }
#pragma unroll
    for (int s = 0; s < QN; ++s) qf[s] = (row_ok && qrank(s) >= 0) ? qf[s] * qs[s] : 0.0f;
  }
  halfx8 qh[SPLIT ? KS : 1], ql[SPLIT ? KS : 1];
  bf16x8 qbf[BF ? KS : 1];  // bf16 query fragment
  int score_exp = 0;  // E (split path; 0 for bf16 operands)
  if constexpr (BF) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qbf[s][e] = (bf16_t)qf[8 * s + e];
  } else if constexpr (SPLIT) {
    float m = 0.0f;
#pragma unroll
    for (int s = 0; s < QN; ++s) m = fmaxf(m, fabsf(qf[s]));
    m = fmaxf(m, xor16_f(m));
    m = fmaxf(m, xor32_f(m));
    const int eq = split_exponent(m);
    score_exp = eq + a.split_exp[b];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = ldexpf(qf[8 * s + e], eq);
        const _Float16 hi = (_Float16)x;
        qh[s][e] = hi;
        ql[s][e] = (_Float16)(x - (float)hi);
      }
    }
  }
  const float bias = a.bias ? a.bias[0] : 0.0f;
  // (dot + bias) / T as a multiply by the reciprocal: exact for T == 1, within
  // 1.5 ulp of the division otherwise
  const float inv_temp = 1.0f / a.temperature;
  // Split path without bias or temperature: rows are filtered and merged on
  // the scaled scores (scaling a row by 2^E keeps its order and its ties) and
  // only the k winners are scaled back.
  const bool scaled_domain = !MH && SPLIT && inv_temp == 1.0f && bias == 0.0f;
  // MH: K-step s closes head (s + 1) / head_ks - 1 when fold bit s is set;
  // fold_bias[s] is that head's bias
  uint32_t fold_bits = 0;
  float fold_bias[MH ? KS : 1];
  if constexpr (MH) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool closes = (s + 1) % head_ks == 0;
      const int h = (s + 1) / head_ks - 1;
      fold_bits |= closes ? (1u << s) : 0u;
      fold_bias[s] = (closes && a.bias && h < a.heads) ? a.bias[h] : 0.0f;
    }
  }

  // ---- key fragments straight from memory: every wave streams the keys on its
  // own (no LDS staging, no workgroup barrier in the loop), so a wave that
  // merges does not hold up the others.  Lane (g, col) reads key rows
  // c0 + col and c0 + 16 + col, ranks [g*RQ, g*RQ + RQ): the A operand of its
  // two MFMA tiles.  Buffer loads are relative to the chunk's first row; rows
  // past Nk read as zeros and are masked later.  Two register sets: the next
  // chunk loads while the current one is scored.
  // The resource of a chunk ends after its last row below Nk, so rows past
  // the end read as zeros with loop-invariant lane offsets.
  float kx[2][kSelTiles][FR];
  uint32_t kbase_off[kSelTiles];
  // split rows: 2 PLANES RP bytes each; lane group g reads ranks [8g, 8g + 8) of every K-step
#pragma unroll
  for (int t = 0; t < kSelTiles; ++t)
    kbase_off[t] = SPLIT ? (uint32_t)((16 * t + col) * 2 * PLANES * RP + 16 * g)
                         : (uint32_t)((16 * t + col) * ldk + g * RQ) * 4u;
  const _Float16* split_b =
      SPLIT ? reinterpret_cast<const _Float16*>(a.split_key) + (int64_t)b * a.Nk * PLANES * RP : nullptr;
  auto load_keys = [&](auto SET, int c) {
    constexpr int S = decltype(SET)::value;
    const int c0 = (chunk0 + c) * kSelChunk;
    const int rows = max(0, min(kSelChunk, key_end - c0));
    // uniform (readfirstlane keeps the resource in SGPRs)
    const uint32_t nrec = __builtin_amdgcn_readfirstlane(SPLIT ? (uint32_t)(rows * 2 * PLANES * RP)
                                                                : (uint32_t)(rows * ldk) * 4u);
    const auto rs =
        SPLIT ? make_rsrc(split_b + (int64_t)c0 * PLANES * RP, nrec) : make_rsrc(kbase + (int64_t)c0 * ldk, nrec);
#pragma unroll
    for (int t = 0; t < kSelTiles; ++t) {
      if constexpr (BF) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const float4 h = buf_load4(rs, kbase_off[t] + 64u * s);
          kx[S][t][4 * s + 0] = h.x;
          kx[S][t][4 * s + 1] = h.y;
          kx[S][t][4 * s + 2] = h.z;
          kx[S][t][4 * s + 3] = h.w;
        }
      } else if constexpr (SPLIT) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const float4 h = buf_load4(rs, kbase_off[t] + 64u * s);
          const float4 l = buf_load4(rs, kbase_off[t] + 64u * s + 2u * RP);
          kx[S][t][8 * s + 0] = h.x;
          kx[S][t][8 * s + 1] = h.y;
          kx[S][t][8 * s + 2] = h.z;
          kx[S][t][8 * s + 3] = h.w;
          kx[S][t][8 * s + 4] = l.x;
          kx[S][t][8 * s + 5] = l.y;
          kx[S][t][8 * s + 6] = l.z;
          kx[S][t][8 * s + 7] = l.w;
        }
      } else if constexpr (V4) {
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
    // keep every load of the chunk ahead of the MFMAs that follow: left alone,
    // the scheduler sinks most of them below the current chunk's MFMAs, and
    // the prefetch then has only the filter to hide its latency behind
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr std::integral_constant<int, 0> kSet0{};
  constexpr std::integral_constant<int, 1> kSet1{};


  float theta = row_ok ? -INFINITY : INFINITY;  // invalid rows never admit
  int cnt = 0;   // candidates in this lane's region of its row
  int kept = 0;  // valid kept entries of this lane's row (<= k)
  uint32_t* my_kept_k = s_kept_k + lrow * KST;
  uint16_t* my_kept_i = s_kept_i + lrow * KIST;
  float* wave_cand_s = s_cand_s + wave * CAP * kWave;
  uint16_t* wave_cand_i = s_cand_i + wave * CAP * kWave;
  float* my_cand_s = wave_cand_s + lane;
  uint16_t* my_cand_i = wave_cand_i + lane;

  auto process = [&](auto SET, int c) {
    constexpr int S = decltype(SET)::value;
    const int c0 = (chunk0 + c) * kSelChunk;
    if constexpr (COOP) {
      // this wave's fragments of the staged chunk: lane (g, col) reads ranks
      // [32 s + 8 g, +8) of row 16 t + col from each plane
      const _Float16* kb = s_key + (NBUF == 2 ? (c & 1) : 0) * KBUF + col * KROW + 8 * g;
#pragma unroll
      for (int t = 0; t < kSelTiles; ++t)
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const float4 h = *reinterpret_cast<const float4*>(kb + 16 * t * KROW + 32 * s);
          if constexpr (BF) {
            kx[S][t][4 * s + 0] = h.x;
            kx[S][t][4 * s + 1] = h.y;
            kx[S][t][4 * s + 2] = h.z;
            kx[S][t][4 * s + 3] = h.w;
            continue;
          }
          const float4 l = *reinterpret_cast<const float4*>(kb + 16 * t * KROW + 32 * s + RP);
          kx[S][t][8 * s + 0] = h.x;
          kx[S][t][8 * s + 1] = h.y;
          kx[S][t][8 * s + 2] = h.z;
          kx[S][t][8 * s + 3] = h.w;
          kx[S][t][8 * s + 4] = l.x;
          kx[S][t][8 * s + 5] = l.y;
          kx[S][t][8 * s + 6] = l.z;
          kx[S][t][8 * s + 7] = l.w;
        }
    }
    // -- scores for 32 keys x 16 query rows (two MFMA tiles) --
    floatx4 acc[kSelTiles];
#pragma unroll
    for (int t = 0; t < kSelTiles; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (BF) {
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t) {
          const bf16x8 kv = __builtin_bit_cast(
              bf16x8, floatx4{kx[S][t][4 * s], kx[S][t][4 * s + 1], kx[S][t][4 * s + 2], kx[S][t][4 * s + 3]});
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kv, qbf[s], acc[t], 0, 0, 0);
        }
    } else if constexpr (SPLIT) {
      floatx4 best[MH ? kSelTiles : 1];
      if constexpr (MH) {
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t) best[t] = floatx4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
      // small products first: lo.hi + hi.lo, then hi.hi
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t) {
          const halfx8 kh = as_halfx8(kx[S][t][8 * s], kx[S][t][8 * s + 1], kx[S][t][8 * s + 2], kx[S][t][8 * s + 3]);
          const halfx8 kl =
              as_halfx8(kx[S][t][8 * s + 4], kx[S][t][8 * s + 5], kx[S][t][8 * s + 6], kx[S][t][8 * s + 7]);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[s], acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[s], acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t) {
          const halfx8 kh = as_halfx8(kx[S][t][8 * s], kx[S][t][8 * s + 1], kx[S][t][8 * s + 2], kx[S][t][8 * s + 3]);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[s], acc[t], 0, 0, 0);
        }
        if constexpr (MH) {
          if ((fold_bits >> s) & 1u) {  // uniform: the last K-step of a head
#pragma unroll
            for (int t = 0; t < kSelTiles; ++t) {
#pragma unroll
              for (int v = 0; v < 4; ++v)
                best[t][v] = fmaxf(best[t][v], (ldexpf(acc[t][v], -score_exp) + fold_bias[s]) * inv_temp);
              acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
      if constexpr (MH) {
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t) acc[t] = best[t];
      }
    } else {
#pragma unroll
      for (int q = 0; q < RQ; ++q)
#pragma unroll
        for (int t = 0; t < kSelTiles; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kx[S][t][q], qf[q], acc[t], 0, 0, 0);
    }

    // -- threshold filter: lane holds keys c0 + 16t + 4g + v of its row --
    float sc[kSelLaneKeys];
#pragma unroll
    for (int u = 0; u < kSelLaneKeys; ++u) sc[u] = acc[u >> 2][u & 3];
    if constexpr (!MH) {  // multi-head scores are final after the fold
      if (SPLIT && !scaled_domain) {  // uniform
#pragma unroll
        for (int u = 0; u < kSelLaneKeys; ++u) sc[u] = ldexpf(sc[u], -score_exp);
      }
      if (scaled_domain) {
        // compared as they are
      } else if (inv_temp != 1.0f) {  // uniform
#pragma unroll
        for (int u = 0; u < kSelLaneKeys; ++u) sc[u] = (sc[u] + bias) * inv_temp;
      } else if (bias != 0.0f) {
#pragma unroll
        for (int u = 0; u < kSelLaneKeys; ++u) sc[u] += bias;
      }
    }
    if (c0 + kSelChunk > key_end) {  // uniform: only the last chunk holds padding keys
#pragma unroll
      for (int u = 0; u < kSelLaneKeys; ++u)
        if (c0 + (u >> 2) * 16 + 4 * g + (u & 3) >= key_end) sc[u] = -INFINITY;
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
        my_cand_s[cnt * kWave] = sc[u];
        my_cand_i[cnt * kWave] = (uint16_t)(c0 + (u >> 2) * 16 + 4 * g + (u & 3));
        cnt += (sc[u] > theta) ? 1 : 0;
      }
    }

  };

  // -- merge the wave's rows (`go`: wave-uniform).  After the last chunk every
  // row still holding more than k entries merges exactly --
  auto merge = [&](bool go, bool last) {
    if (go) {
      wave_lds_sync();
      const int total = kept + row_sum4(cnt);
      const int cq = (int)(__builtin_amdgcn_readfirstlane(wave_max_u32((uint32_t)cnt)) + 3) / 4;
      const MergeResult mr =
          merge_rows_batched<KEEP>(my_kept_k, my_kept_i, my_cand_s, my_cand_i, k, kept, cnt, total, last ? k : KEEP,
                                   theta, cq);
      const int n_kept = mr.kept;
      theta = mr.theta;
      // rows with exact ties at the k-th value: exact per-row merge (such a
      // row holds more than k entries, so the merge fills it)
      uint64_t m = __ballot(lane < kSelRowsPerWave && n_kept < 0);
      while (m) {
        const int t = __builtin_ctzll(m);
        m &= m - 1;
        const int slot = wave * kSelRowsPerWave + t;
        const float th = merge_row_exact<KEEP>(s_kept_k + slot * KST, s_kept_i + slot * KIST, wave_cand_s, wave_cand_i, t,
                                               k, readlane_i(kept, t), readlane_i(cnt, t), readlane_i(cnt, t + 16),
                                               readlane_i(cnt, t + 32), readlane_i(cnt, t + 48));
        if (col == t) theta = th;
      }
      if (!row_ok) theta = INFINITY;  // rows past Nq stay closed
      kept = n_kept < 0 ? k : n_kept;
      cnt = 0;
    }
  };
  // a wave must merge once any lane region is within one chunk of its capacity
  auto need_merge = [&]() { return __ballot(cnt > CAP - kSelLaneKeys) != 0; };
  auto need_final = [&]() { return __ballot(cnt > 0 || kept > k) != 0; };

  // chunk c lives in register set c & 1.  The loads are unconditional (chunks
  // past the end read rows >= Nk: zeros, no memory access), so the wait before
  // a chunk's MFMAs covers only its own loads, not the prefetch behind them.
  if constexpr (COOP) {
    // cooperative staging: thread x moves float4s x + NT p of the chunk
    float4 pre[PER];
    auto stage_load = [&](int c) {
      const int c0 = c * kSelChunk;
      const int rows = max(0, min(kSelChunk, a.Nk - c0));
      const uint32_t nrec = __builtin_amdgcn_readfirstlane((uint32_t)(rows * 2 * PLANES * RP));
      const auto rs = make_rsrc(split_b + (int64_t)c0 * PLANES * RP, nrec);
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int f = (int)threadIdx.x + NT * p;
        pre[p] = buf_load4(rs, f < F4 ? (uint32_t)f * 16u : kOobOffset);
      }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
      for (int p = 0; p < PER; ++p) {
        const int f = (int)threadIdx.x + NT * p;
        if (f < F4) {
          const int row = f / (PLANES * RP / 8), part = f - row * (PLANES * RP / 8);
          *reinterpret_cast<float4*>(s_key + buf * KBUF + row * KROW + 8 * part) = pre[p];
        }
      }
    };
    if (threadIdx.x < 3) s_flag[threadIdx.x] = 0;
    stage_load(0);
    stage_store(0);
    if (nchunks > 1) stage_load(1);
    __syncthreads();
    // Chunk c: score buffer c & 1, raise flag c % 3 if this wave must merge,
    // stage chunk c + 1 into the other buffer, barrier, issue the loads of
    // chunk c + 2, merge every wave if the flag is up.  Wave 0 clears flag
    // (c + 1) % 3 = (c - 2) % 3, read by all before the previous barrier and
    // raised again only after this one.
    // With one buffer (CW = 4) a second barrier separates the last reads of
    // chunk c from the stores of chunk c + 1.
    int fl = 0;  // c % 3
    for (int c = 0; c < nchunks; ++c) {
      process(kSet0, c);
      const bool last = c + 1 == nchunks;
      if (need_merge() && lane == 0) s_flag[fl] = 1;
      const int fl_next = fl == 2 ? 0 : fl + 1;
      if (wave == 0 && lane == 0) s_flag[fl_next] = 0;
      // With one buffer the flags are final after the first barrier: read
      // there, the flag's LDS latency hides behind the staging store and the
      // second barrier.
      int flag = 0;
      if constexpr (NBUF == 1) {
        __syncthreads();
        flag = s_flag[fl];
      }
      if (!last) stage_store(NBUF == 2 ? (c + 1) & 1 : 0);
      __syncthreads();
      if (c + 2 < nchunks) stage_load(c + 2);
      if constexpr (NBUF == 2) flag = s_flag[fl];
      const bool go = last ? need_final() : __builtin_amdgcn_readfirstlane(flag) != 0;
      merge(go, last);
      fl = fl_next;
    }
  } else {
    load_keys(kSet0, 0);
    for (int c = 0; c < nchunks; c += 2) {
      load_keys(kSet1, c + 1);
      process(kSet0, c);
      const bool last0 = c + 1 == nchunks;
      merge(need_merge() || (last0 && need_final()), last0);
      if (c + 1 < nchunks) {
        load_keys(kSet0, c + 2);
        process(kSet1, c + 1);
        const bool last1 = c + 2 == nchunks;
        merge(need_merge() || (last1 && need_final()), last1);
      }
    }
  }
  wave_lds_sync();

  if constexpr (KSP) {
    // every wave holds the exact top-k of its key quarter for the workgroup's
    // 16 rows, unsorted in its own kept slots; wave w merges rows 4w .. 4w + 3
    // over the four lists (lane (src, e): entry e of wave src's list)
    __shared__ int s_kcnt[kSelRows];
    if (lane < kSelRowsPerWave) s_kcnt[wave * kSelRowsPerWave + lane] = kept;
    __syncthreads();
    const int src = lane >> 4, e = lane & 15;
    for (int t = 0; t < kSelRowsPerWave / kSelWaves; ++t) {
      const int rcol = (kSelRowsPerWave / kSelWaves) * wave + t;
      const int row = row0 + rcol;
      const int slot = src * kSelRowsPerWave + rcol;
      float vs = -INFINITY;
      int vi = 0x7fffffff;
      if (e < s_kcnt[slot]) {
        vs = key_to_float(s_kept_k[slot * KST + e]);
        vi = s_kept_i[slot * KIST + e];
      }
      bitonic_sort64_desc(vs, vi);
      if (scaled_domain) vs = ldexpf(vs, -readlane_i(score_exp, rcol));
      if (lane < k && row < a.Nq) {
        const int64_t o = ((int64_t)b * a.Nq + row) * k + lane;
        a.out_idx[o] = vi;
        a.out_score[o] = vs;
      }
    }
    return;
  }

  // ---- sort each row's k winners and write them -----------------------------
  if constexpr (KEEP == 48) {
    // k <= 32: two rows per pass, row t + h on half-wave h
    const int h = lane >> 5, e = lane & 31;
    for (int t = 0; t < kSelRowsPerWave; t += 2) {
      if (row0 + wave * kSelRowsPerWave + t >= a.Nq) break;
      const int row = row0 + wave * kSelRowsPerWave + t + h;
      const int slot = wave * kSelRowsPerWave + t + h;
      float vs = -INFINITY;
      int vi = 0x7fffffff;
      if (e < k) {
        vs = key_to_float(s_kept_k[slot * KST + e]);
        vi = s_kept_i[slot * KIST + e];
      }
      bitonic_sort32x2_desc(vs, vi);
      if (scaled_domain) {
        const int e0 = readlane_i(score_exp, t), e1 = readlane_i(score_exp, t + 1);
        vs = ldexpf(vs, -(h ? e1 : e0));
      }
      if (e < k && row < a.Nq) {
        const int64_t o = ((int64_t)b * a.Nq + row) * k + e;
        a.out_idx[o] = vi;
        a.out_score[o] = vs;
      }
    }
  } else
  for (int t = 0; t < kSelRowsPerWave; ++t) {
    const int row = row0 + wave * kSelRowsPerWave + t;
    if (row >= a.Nq) break;
    const int slot = wave * kSelRowsPerWave + t;
    float vs = -INFINITY;
    int vi = 0x7fffffff;
    if (lane < k) {
      vs = key_to_float(s_kept_k[slot * KST + lane]);
      vi = s_kept_i[slot * KIST + lane];
    }
    bitonic_sort64_desc(vs, vi);
    if (scaled_domain) vs = ldexpf(vs, -readlane_i(score_exp, t));
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
    if (vec) hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, true, 48, 0, 0>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, false, 48, 0, 0>), grid, dim3(256), 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, true, 80, 0, 0>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((lowrank_topk_select_kernel<RQ, false, 80, 0, 0>), grid, dim3(256), 0, stream, a);
  }
}

template <int KS>
static void launch_split_heads(const SelectArgs& a, dim3 grid, hipStream_t stream) {
  if (a.k <= 32)
    hipLaunchKernelGGL((lowrank_topk_select_kernel<1, false, 48, KS, 0, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((lowrank_topk_select_kernel<1, false, 80, KS, 0, true>), grid, dim3(256), 0, stream, a);
}

template <int KS, int CW, bool BF = false>
static void launch_split(const SelectArgs& a, dim3 grid, hipStream_t stream) {
  const dim3 block(CW > 0 ? CW * kWave : 256);
  if constexpr (CW < 0) {
    hipLaunchKernelGGL((lowrank_topk_select_kernel<1, false, 48, KS, CW, false, BF>), grid, block, 0, stream, a);
  } else {
    if (a.k <= 32)
      hipLaunchKernelGGL((lowrank_topk_select_kernel<1, false, 48, KS, CW, false, BF>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((lowrank_topk_select_kernel<1, false, 80, KS, CW, false, BF>), grid, block, 0, stream, a);
  }
}

// The split-layout kernels of one select: cooperative, key-split or per-wave.
template <bool BF>
static void launch_split_forms(const SelectArgs& a, int RP, bool coop4, bool ksp, dim3 grid, hipStream_t stream) {
  if (coop4) {
    if (RP == 32) launch_split<1, 4, BF>(a, grid, stream);
    else launch_split<2, 4, BF>(a, grid, stream);
  } else if (ksp) {
    const dim3 kgrid((unsigned)((int64_t)((a.Nq + kSelRowsPerWave - 1) / kSelRowsPerWave) * a.B));
    switch (RP / 32) {
      case 1: launch_split<1, -1, BF>(a, kgrid, stream); break;
      case 2: launch_split<2, -1, BF>(a, kgrid, stream); break;
      case 3: launch_split<3, -1, BF>(a, kgrid, stream); break;
      default: launch_split<4, -1, BF>(a, kgrid, stream); break;
    }
  } else {
    switch (RP / 32) {
      case 1: launch_split<1, 0, BF>(a, grid, stream); break;
      case 2: launch_split<2, 0, BF>(a, grid, stream); break;
      case 3: launch_split<3, 0, BF>(a, grid, stream); break;
      default: launch_split<4, 0, BF>(a, grid, stream); break;
    }
  }
}

// The cooperative kernels pay for their barriers with shared key staging,
// which wins once every CU holds two 64-row workgroups (C4: 0.40 ms against
// 0.53 for the per-wave kernel); on smaller grids (C3's 128 and 32
// workgroups) the per-wave kernel is as fast or faster.
constexpr int64_t kSelCoop4MinBlocks = 512;
// Below one 64-row workgroup per CU, with k <= 16 and at least four key chunks,
// the key-split per-wave form runs a quarter of the serial chunk chain.
constexpr int64_t kSelKspMaxBlocks = 256;
constexpr int kSelKspMinKeys = 4 * kSelChunk;

namespace {
std::atomic<int> g_select_mode{kSelectSplitF16};

int split_ranks(int64_t r) { return (int)((r + 31) / 32) * 32; }

struct SelectScratch {
  uint16_t* split;  // [B, Nk, 2 RP] fp16 bits
  int* kexp;        // [B]
  float* partial;   // [B, ceil(Nk / kSplitRows)]
  size_t bytes;
};

SelectScratch carve_select(void* base, size_t size, int64_t B, int64_t Nk, int64_t r) {
  Workspace ws(base, size);
  SelectScratch s{};
  s.split = ws.take<uint16_t>(B * Nk * 2 * split_ranks(r));
  s.kexp = ws.take<int>(B);
  s.partial = ws.take<float>(B * ((Nk + kSplitRows - 1) / kSplitRows));
  s.bytes = ws.used;
  return s;
}
}  // namespace

int select_mode() { return g_select_mode.load(std::memory_order_relaxed); }
void set_select_mode(int mode) { g_select_mode.store(mode, std::memory_order_relaxed); }

// Every mode reports the split workspace (fp32 MFMAs leave it unused).
size_t select_workspace_bytes(int64_t B, int64_t Nk, int64_t r) {
  if (B < 1 || Nk < 1 || r < 1) return 0;
  return carve_select(nullptr, 0, B, Nk, r).bytes;
}

bool select_heads_fit(int64_t head_rank, int64_t heads) {
  return heads >= 2 && heads <= kMaxHeads && head_rank >= 1 && heads * split_ranks(head_rank) <= 128;
}

// Heads beyond the register kernels' K-steps run the scored-rows select,
// whose score blocks take this much workspace too.
size_t select_workspace_bytes_heads(int64_t B, int64_t Nk, int64_t head_rank, int64_t heads) {
  if (heads <= 1) return select_workspace_bytes(B, Nk, head_rank);
  if (heads > kMaxHeads || head_rank < 1 || heads * head_rank > 128) return 0;
  return select_workspace_bytes(B, Nk, heads * split_ranks(head_rank));
}

int launch_topk_select(const SelectArgs& a_in, hipStream_t stream) {
  SelectArgs a = a_in;
  const bool large_heads = a.heads > 1 && !(a.bf16 == 0 && select_heads_fit(a.head_rank, a.heads));
  // k == Nk (every key kept, in score order) runs on the scored rows too
  // so does one head of more ranks than the register kernels hold
  if (a.k > kSelectMaxK || a.Nk > kSelMaxKeys || large_heads || a.k >= a.Nk || (a.heads <= 1 && a.r > kRegRank))
    return launch_topk_select_large(a, stream);
  // rows of few keys: the whole score row in LDS, one radix select per row
  if (select_mode() == kSelectSplitF16 && select_small_fits(a)) return launch_topk_select_small(a, stream);
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
  const bool mh = a.heads > 1;
  JN_REQUIRE(!(mh && a.bf16), kUnsupported, "bf16 score operands take one head");
  JN_REQUIRE(!mh || (select_heads_fit(a.head_rank, a.heads) && a.heads * a.head_rank == a.r), kUnsupported,
             "multi-head top-k select: %d heads of rank %d must fill 4 K-steps of 32 ranks at most (rank %d)",
             a.heads, a.head_rank, a.r);
  // multi-head scores always run on the per-wave split kernel; bf16 operands
  // take the split kernels' forms whatever the mode
  int mode = mh ? kSelectSplitF16Wave : select_mode();
  if (mode == kSelectSplitF16Register) mode = kSelectSplitF16;
  if (a.bf16 && mode == kSelectF32) mode = kSelectSplitF16;

  if (mode != kSelectF32) {
    const int head_rp = mh ? split_ranks(a.head_rank) : split_ranks(a.r);
    const int RP = mh ? a.heads * head_rp : head_rp;
    const SelectScratch s = carve_select(a.ws, a.ws_bytes, a.B, a.Nk, RP);
    JN_REQUIRE(a.ws != nullptr && s.bytes <= a.ws_bytes, kWorkspaceTooSmall,
               "select workspace too small: need %zu bytes, got %zu", s.bytes, a.ws_bytes);
    const int nblk = (a.Nk + kSplitRows - 1) / kSplitRows;
    dim3 pgrid((unsigned)nblk, (unsigned)a.B);
    if (a.bf16) {
      JN_PROFILE("select_bf16_keys_kernel", stream);
      hipLaunchKernelGGL(select_bf16_keys_kernel, pgrid, dim3(256), 0, stream, a.key, a.ldk, a.k_batch_stride, a.Nk,
                         a.r, RP, reinterpret_cast<bf16_t*>(s.split));
      JN_LAUNCH_CHECK();
    } else {
      {
        JN_PROFILE("select_split_absmax_kernel", stream);
        hipLaunchKernelGGL(select_split_absmax_kernel, pgrid, dim3(256), 0, stream, a.key, a.ldk, a.k_batch_stride,
                           a.Nk, a.r, nblk, s.partial);
        JN_LAUNCH_CHECK();
      }
      JN_PROFILE("select_split_keys_kernel", stream);
      hipLaunchKernelGGL(select_split_keys_kernel, pgrid, dim3(256), 0, stream, a.key, a.ldk, a.k_batch_stride, a.Nk,
                         mh ? a.head_rank : a.r, head_rp, RP, nblk, s.partial,
                         reinterpret_cast<_Float16*>(s.split), s.kexp);
      JN_LAUNCH_CHECK();
    }
    a.split_key = s.split;
    a.split_exp = s.kexp;
    const bool coop4 = RP <= 64 && (mode == kSelectSplitF16Coop4 ||
                                    (mode == kSelectSplitF16 && blocks >= kSelCoop4MinBlocks));
    const bool ksp = !coop4 && a.k <= 16 &&
                     (mode == kSelectSplitF16KeySplit ||
                      (mode == kSelectSplitF16 && blocks < kSelKspMaxBlocks && a.Nk >= kSelKspMinKeys));
    JN_PROFILE("lowrank_topk_select_kernel", stream);
    if (mh) {
      switch (RP / 32) {
        case 2: launch_split_heads<2>(a, grid, stream); break;
        case 3: launch_split_heads<3>(a, grid, stream); break;
        default: launch_split_heads<4>(a, grid, stream); break;
      }
    } else if (a.bf16) {
      launch_split_forms<true>(a, RP, coop4, ksp, grid, stream);
    } else {
      launch_split_forms<false>(a, RP, coop4, ksp, grid, stream);
    }
    JN_LAUNCH_CHECK();
    return kOk;
  }

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
