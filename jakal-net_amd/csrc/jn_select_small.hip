// Top-k select for rows of few keys (gfx950): up to 1024 keys, k <= 64, one
// head, fp32 scores.
//
// The register select (jn_select.hip) streams long key rows through a
// threshold filter and batched merges; on rows of a few hundred keys its
// merge and sort machinery sets a fixed cost of tens of microseconds per
// launch (C3's and C5's transitions and slot propagations select over 64 to
// 1024 keys).  Here the whole score row fits LDS instead:
//   1. a workgroup (8 or 16 waves) takes 16 query rows of one batch element;
//      wave w scores key tiles w, w + WV, ... of 16 keys on v_mfma_f32_16x16x4f32
//      (fp32 operands, fp32 accumulation: the arithmetic of select mode 1)
//      and writes each score as an order key into the row's LDS line;
//   2. each wave then selects one or two of the rows: a radix select over the order
//      keys (four 8-bit digits, LDS histograms with integer atomics) finds the
//      exact k-th key T; the keys above T and the lowest-index keys equal to T
//      (index order is lane order within each 64-key block) are the row's k
//      winners, which a 64-lane bitonic network sorts into descending score,
//      ascending index on ties.
// Scores: s[i, j] = ((sum_r q[i, r] c_q[r] key[j, r] c_k[r]) + bias) / T, as
// the register select (modules.py:95-100, 435-441; kernel_common.py:426-440,
// transition.py:439-444).  The rank sum runs in an order that keeps each
// lane's four consecutive ranks in one float4 load: MFMA step (u, c) takes
// rank 16u + 4g + c on lane group g for both operands, which permutes the
// summation but not its terms.
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kSmRows = 16;  // query rows per workgroup

__device__ __forceinline__ uint32_t small_order_key(float s) {
  const uint32_t u = __float_as_uint(s + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float small_key_float(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// Exchange with lane ^ stride on DPP and permlane moves (see jn_select.hip).
__device__ __forceinline__ int sm_xor_i(int v, int stride) {
  if (stride == 1) return __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false);
  if (stride == 2) return __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false);
  if (stride == 4) {
    const int up = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xf, 0xf, false);
    const int dn = __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false);
    return (lane_id() & 4) ? dn : up;
  }
  if (stride == 8) return __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);
  if (stride == 16) return xor16_i(v);
  return xor32_i(v);
}

// Descending score, ascending index on ties, over the 64 lanes.
__device__ __forceinline__ void sm_sort64_desc(float& vs, int& vi) {
  const int lane = lane_id();
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float ps = __int_as_float(sm_xor_i(__float_as_int(vs), stride));
      const int pi = sm_xor_i(vi, stride);
      const bool partner_better = (ps > vs) | ((ps == vs) & (pi < vi));
      const bool self_better = (vs > ps) | ((vs == ps) & (vi < pi));
      const bool keep_better = ((lane & stride) == 0) == ((lane & size) == 0);
      const bool take = keep_better ? partner_better : self_better;
      vs = take ? ps : vs;
      vi = take ? pi : vi;
    }
  }
}

__device__ __forceinline__ int sm_mbcnt(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Inclusive prefix sum over the 64 lanes (lane 0 first).
__device__ __forceinline__ int sm_wave_scan(int v) {
  const int lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __builtin_amdgcn_ds_bpermute((lane - d) << 2, v);
    v += lane >= d ? o : 0;
  }
  return v;
}

// NK: keys per row at most (512 or 1024); RQ: rank quads per lane group
// (ranks up to 16 * RQ); VEC: 16-byte operand rows.
// WV waves per workgroup: they split the key tiles of phase 1 and take
// 16 / WV rows each in phase 2.
template <int NK, int RQ, bool VEC, int WV>
__global__ __launch_bounds__(WV * 64) void select_small_kernel(SelectArgs a) {
  static_assert(kSmRows % WV == 0, "whole rows per wave");
  constexpr int RPW = kSmRows / WV;  // rows per wave in the selection
  constexpr int KSTR = NK + 1;  // LDS row stride of the order keys
  constexpr int PL = NK / kWave;  // keys per lane in the selection
  __shared__ uint32_t s_key[kSmRows * KSTR];
  __shared__ __align__(16) uint32_t s_hist[WV][256];
  __shared__ float s_win_s[WV][kWave];
  __shared__ int s_win_i[WV][kWave];

  const int lane = lane_id(), wave = wave_id();
  const int g = lane >> 4, col = lane & 15;
  const int tiles_per_batch = (a.Nq + kSmRows - 1) / kSmRows;
  const int b = blockIdx.x / tiles_per_batch;
  const int row0 = (blockIdx.x % tiles_per_batch) * kSmRows;
  const float* qb = a.q + (int64_t)b * a.q_batch_stride;
  const float* kb = a.key + (int64_t)b * a.k_batch_stride;
  const float bias = a.bias ? a.bias[0] : 0.0f;
  const float inv_temp = 1.0f / a.temperature;

  // ---- 1. scores of 16 rows x all keys into LDS --------------------------------
  // lane (g, col) holds ranks 16u + 4g + c of query row row0 + col (B operand)
  auto load4 = [&](const float* row, int u) -> float4 {
    const int r0 = 16 * u + 4 * g;
    if constexpr (VEC) {
      return r0 < a.r ? *reinterpret_cast<const float4*>(row + r0) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      return make_float4(r0 < a.r ? row[r0] : 0.f, r0 + 1 < a.r ? row[r0 + 1] : 0.f,
                         r0 + 2 < a.r ? row[r0 + 2] : 0.f, r0 + 3 < a.r ? row[r0 + 3] : 0.f);
    }
  };
  float qf[RQ][4];
  float kscale[RQ][4];
  {
    const int qrow = row0 + col;
    const float* qr = qb + (int64_t)min(qrow, a.Nq - 1) * a.ldq;
#pragma unroll
    for (int u = 0; u < RQ; ++u) {
      const float4 qv = qrow < a.Nq ? load4(qr, u) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 sv = a.scale ? load4(a.scale, u) : make_float4(1.f, 1.f, 1.f, 1.f);
      const bool on_q = a.scale_on_query != 0;
      qf[u][0] = on_q ? qv.x * sv.x : qv.x;
      qf[u][1] = on_q ? qv.y * sv.y : qv.y;
      qf[u][2] = on_q ? qv.z * sv.z : qv.z;
      qf[u][3] = on_q ? qv.w * sv.w : qv.w;
      kscale[u][0] = on_q ? 1.f : sv.x;
      kscale[u][1] = on_q ? 1.f : sv.y;
      kscale[u][2] = on_q ? 1.f : sv.z;
      kscale[u][3] = on_q ? 1.f : sv.w;
    }
  }
  // wave w scores tiles w, w + WV, ...; PD of its tiles' key loads are in
  // flight at a time (slot i of the ring holds tile t0 + WV i), each slot
  // refilled with the tile PD steps ahead as soon as its own is scored
  constexpr int PD = RQ <= 4 ? 4 : 2;
  const int ntiles = (a.Nk + 15) / 16;
  float4 kring[PD][RQ];
  auto load_tile = [&](float4 (&kv)[RQ], int t) {
    const int j = 16 * t + col;  // this lane's key (A operand row)
    const float* kr = kb + (int64_t)min(j, a.Nk - 1) * a.ldk;
#pragma unroll
    for (int u = 0; u < RQ; ++u) kv[u] = (t < ntiles && j < a.Nk) ? load4(kr, u) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
#pragma unroll
  for (int i = 0; i < PD; ++i) load_tile(kring[i], wave + WV * i);
  for (int t0 = wave; t0 < ntiles; t0 += WV * PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      const int t = t0 + WV * i;
      if (t >= ntiles) break;  // wave-uniform
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < RQ; ++u) {
        const float4 kv = kring[i][u];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x * kscale[u][0], qf[u][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y * kscale[u][1], qf[u][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z * kscale[u][2], qf[u][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w * kscale[u][3], qf[u][3], acc, 0, 0, 0);
      }
      load_tile(kring[i], t + WV * PD);
      // lane (g, col) holds keys 16t + 4g + v of row col
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int jj = 16 * t + 4 * g + v;
        if (jj < a.Nk) s_key[col * KSTR + jj] = small_order_key((acc[v] + bias) * inv_temp);
      }
    }
  }
  __syncthreads();

  // ---- 2. wave w selects rows 4w .. 4w + 3 ------------------------------------
  const int k = a.k;
  for (int rr = RPW * wave; rr < RPW * (wave + 1); ++rr) {
    const int row = row0 + rr;
    if (row >= a.Nq) break;  // wave-uniform; no workgroup barrier below
    uint32_t kv[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int j = lane + kWave * i;
      kv[i] = j < a.Nk ? s_key[rr * KSTR + j] : 0u;  // 0: no key (every real score maps above it)
    }
    // radix select of the k-th largest order key, 8 bits at a time
    uint32_t prefix = 0u, pmask = 0u;
    int need = k;
#pragma unroll
    for (int shift = 24; shift >= 0; shift -= 8) {
      *reinterpret_cast<uint4*>(&s_hist[wave][4 * lane]) = make_uint4(0u, 0u, 0u, 0u);
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (kv[i] != 0u && (kv[i] & pmask) == prefix) atomicAdd(&s_hist[wave][(kv[i] >> shift) & 255u], 1u);
      wave_lds_sync();
      // lane l holds digits 255 - 4l - c, c = 0..3 (descending digit order)
      const uint4 h4 = *reinterpret_cast<const uint4*>(&s_hist[wave][252 - 4 * lane]);
      const int h[4] = {(int)h4.w, (int)h4.z, (int)h4.y, (int)h4.x};
      const int incl = sm_wave_scan(h[0] + h[1] + h[2] + h[3]);
      const int src = __builtin_ctzll(__ballot(incl >= need));  // the lane holding the k-th key's digit
      int before = incl - (h[0] + h[1] + h[2] + h[3]);          // keys above this lane's digits
      int c = 0;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        if (c == q && before + h[q] < need) {
          before += h[q];
          c = q + 1;
        }
      }
      const int digit = 255 - 4 * src - readlane_i(c, src);
      need -= readlane_i(before, src);
      prefix |= (uint32_t)digit << shift;
      pmask |= 255u << shift;
      wave_lds_sync();  // every lane has read the histogram before the next pass clears it
    }
    // winners: every key above T = prefix, and the `need` lowest-index keys equal to it
    int taken = 0, ties = 0;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const bool eq = kv[i] == prefix;
      const uint64_t eqm = __ballot(eq);
      const bool take = kv[i] > prefix || (eq && ties + sm_mbcnt(eqm) < need);
      ties += __popcll(eqm);
      const uint64_t tm = __ballot(take);
      if (take) {
        const int pos = taken + sm_mbcnt(tm);
        s_win_s[wave][pos] = small_key_float(kv[i]);
        s_win_i[wave][pos] = lane + kWave * i;
      }
      taken += __popcll(tm);
    }
    wave_lds_sync();
    float vs = lane < k ? s_win_s[wave][lane] : -INFINITY;
    int vi = lane < k ? s_win_i[wave][lane] : 0x7fffffff;
    sm_sort64_desc(vs, vi);
    if (lane < k) {
      const int64_t o = ((int64_t)b * a.Nq + row) * k + lane;
      a.out_idx[o] = vi;
      a.out_score[o] = vs;
    }
    wave_lds_sync();  // the winners are read before the next row writes them
  }
}

// 16 waves (one row each) where the registers allow four waves per SIMD
// (512-key rows of rank <= 64), else 8 waves (two rows each)
template <int NK, bool VEC>
void launch_small_rq(const SelectArgs& a, dim3 grid, hipStream_t stream) {
  const int rq = (a.r + 15) / 16;
  constexpr int W16 = NK == 512 ? 16 : 8;
  switch (rq) {
    case 1: hipLaunchKernelGGL((select_small_kernel<NK, 1, VEC, W16>), grid, dim3(W16 * 64), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((select_small_kernel<NK, 2, VEC, W16>), grid, dim3(W16 * 64), 0, stream, a); break;
    case 3:
    case 4: hipLaunchKernelGGL((select_small_kernel<NK, 4, VEC, W16>), grid, dim3(W16 * 64), 0, stream, a); break;
    default: hipLaunchKernelGGL((select_small_kernel<NK, 8, VEC, 8>), grid, dim3(8 * 64), 0, stream, a); break;
  }
}

}  // namespace

bool select_small_fits(const SelectArgs& a) {
  return a.heads <= 1 && !a.bf16 && a.Nk >= 1 && a.Nk <= kSelectSmallMaxKeys && a.k >= 1 && a.k <= kSelectMaxK &&
         a.k < a.Nk && a.r >= 1 && a.r <= kRegRank && a.Nq >= 1 && a.B >= 1 && a.temperature > 0.0f;
}

int launch_topk_select_small(const SelectArgs& a, hipStream_t stream) {
  JN_REQUIRE(select_small_fits(a), kUnsupported,
             "small select: one head, fp32, 1 <= k < keys <= %d, k <= %d, rank <= %d (got k=%d, keys=%d, rank=%d)",
             kSelectSmallMaxKeys, kSelectMaxK, kRegRank, a.k, a.Nk, a.r);
  JN_REQUIRE(a.q && a.key && a.out_idx && a.out_score, kInvalidArgument, "null tensor pointer");
  const int64_t blocks = (int64_t)a.B * ((a.Nq + kSmRows - 1) / kSmRows);
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "bad grid size");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = a.r % 4 == 0 && a.ldq % 4 == 0 && a.ldk % 4 == 0 && a.q_batch_stride % 4 == 0 &&
                   a.k_batch_stride % 4 == 0 && a16(a.q) && a16(a.key) && (!a.scale || a16(a.scale));
  const dim3 grid((unsigned)blocks);
  JN_PROFILE("select_small_kernel", stream);
  if (a.Nk <= 512) {
    if (vec) launch_small_rq<512, true>(a, grid, stream);
    else launch_small_rq<512, false>(a, grid, stream);
  } else {
    if (vec) launch_small_rq<1024, true>(a, grid, stream);
    else launch_small_rq<1024, false>(a, grid, stream);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
