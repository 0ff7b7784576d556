// Causal-band kernels of window propagation (gfx950).
//
// A window edge list gives query row i the keys j = i - (k - 1 - e) in slots
// e < k, absent below 0 (kernel_common.py:443-456, causal_window_mask;
// propagation.py:459-470).  Cut a batch element's rows into tiles of 64: the
// rows a tile's band touches are a span of 64 + k - 1 neighbouring rows, so
// each sum over the band is a small dense product over that span with the
// band cut out of it, run on v_mfma_f32_16x16x4f32 (fp32 accumulation):
//
//   forward      delta_val[i] = sum_j A(i, j) pv[j],   A(i, j) = c(s[i, j - i + k - 1])
//                delta_state[i] = sum_j A(i, j) ps[j]  (propagation.py:473-479)
//   column pass  grad_pv[j]   = sum_i A(i, j) gdv[i],  i in j .. j + k - 1
//                grad_ps[j]   = sum_i A(i, j) gds[i]
//   dots         G[i, e] = <gdv[i], pv[i - (k - 1) + e]>, the value-row part of
//                the coefficient gradient (the row backward adds the rest)
//
// Each value row is read once per tile instead of once per edge: the band's
// gathers in the edge kernels re-read every row k times through L2.  These
// kernels replace rows_forward, the dot products of rows_backward and the
// value gather of the column pass for window edge lists with k <= 128; the
// coefficients, the compress backward, dQ and dK stay with the edge kernels.
#include <atomic>
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBandRows = 64;                 // rows per tile
constexpr int kBandChunk = 32;                // span rows per aggregate LDS stage
constexpr int kBandKStride = 20;              // LDS row stride of a 16-column dots slice (floats)
// Value columns per aggregate workgroup: 128, or 64 when 128-column slabs
// would leave fewer than two workgroups per CU (more workgroups to hide the
// load latency of each tile's short span, at one more pass over its
// coefficients per slab).
constexpr int kBandColsWide = 128, kBandColsNarrow = 64;
constexpr int64_t kBandNarrowBelow = 512;
// LDS row stride of a staged value chunk (floats): four rows 16 banks apart
__host__ __device__ constexpr int band_vstride(int cols) { return cols + 16; }

// LDS row stride of the 64 x k coefficient tile: the smallest value >= k that
// is 3 mod 32.  A fragment read takes 16 rows at stride - 1 (= 2 mod 32) and 4
// consecutive span offsets, so a half-wave's 32 lanes hit 32 distinct banks.
__host__ __device__ constexpr int band_coef_stride(int k) { return ((k + 28) / 32) * 32 + 3; }

size_t band_aggregate_lds_bytes(int k, int cols) {
  return sizeof(float) * ((size_t)kBandRows * band_coef_stride(k) + (size_t)kBandChunk * band_vstride(cols));
}

// ---------------------------------------------------------------------------
// Aggregation: out[t] = sum_u A(t, u) val[u] over a 64-row tile and a slab of
// COLS columns.  TRANS = false: t are query rows, A from the compressed scores
// (the forward); TRANS = true: t are key rows, A(t, u) = coef[u, t - u + k - 1]
// (the column pass).  In both cases A(t, u) = cs[t - t0][u - t + off] with
// off = k - 1 (forward) or 0, over the span u in [t0 - off, t0 - off + 63 + k).
// ---------------------------------------------------------------------------
template <typename T, bool TRANS, int COLS>
__global__ __launch_bounds__(256) void band_aggregate_kernel(BandAggArgs a) {
  extern __shared__ __align__(16) float lds[];
  constexpr int W = 16 / (int)sizeof(T);                    // elements per 16-byte pack
  constexpr int kPacksPerRow = COLS / W;
  constexpr int kPacks = kBandChunk * kPacksPerRow / 256;   // staged packs per thread
  constexpr int VST = band_vstride(COLS);
  static_assert(kPacks >= 1 && kBandChunk * kPacksPerRow % 256 == 0, "whole packs per thread");
  const int kst = band_coef_stride(a.k);
  float* cs = lds;                                           // [kBandRows][kst]
  float* vs = lds + kBandRows * kst;                         // [kBandChunk][VST]
  const int lane = lane_id(), w = wave_id();
  const int col = lane & 15, grp = lane >> 4;
  const int tiles = (a.N + kBandRows - 1) / kBandRows;
  const int slabs = (a.D + COLS - 1) / COLS;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int t = (int)(logical % tiles);
  const int s = (int)((logical / tiles) % slabs);
  const int64_t b = logical / tiles / slabs;
  const int t0 = t * kBandRows, d0 = s * COLS;
  const int off = TRANS ? 0 : a.k - 1;
  const int64_t base = b * a.N;  // global row of the batch element's first row

  // the span's value rows, in chunks of kBandChunk staged in LDS as fp32, one
  // chunk loaded ahead; the first chunk's loads are issued before the
  // coefficients are formed
  const int u0 = t0 - off;
  const int span = kBandRows - 1 + a.k;
  const T* val = reinterpret_cast<const T*>(a.val);
  const int nchunks = (span + kBandChunk - 1) / kBandChunk;
  Pack<W> pre[kPacks];
  auto load_chunk = [&](Pack<W>(&pk)[kPacks], int uc) {
#pragma unroll
    for (int p = 0; p < kPacks; ++p) {
      const int x = threadIdx.x + p * 256;
      const int u = uc + x / kPacksPerRow, d = d0 + (x % kPacksPerRow) * W;
      // rows outside the batch element and columns past D stage zeros (D % W == 0)
      pk[p] = (u >= 0 && u < a.N && d < a.D) ? load_pack<T, W>(val + (base + u) * a.ld_val + d)
                                              : pack_zero<T, W>();
    }
  };
  auto store_chunk = [&](const Pack<W>(&pk)[kPacks]) {
#pragma unroll
    for (int p = 0; p < kPacks; ++p) {
      const int x = threadIdx.x + p * 256;
      float* dst = vs + (x / kPacksPerRow) * VST + (x % kPacksPerRow) * W;
#pragma unroll
      for (int q = 0; q < W; q += 4)
        *reinterpret_cast<float4*>(dst + q) = make_float4(pk[p].v[q], pk[p].v[q + 1], pk[p].v[q + 2],
                                                          pk[p].v[q + 3]);
    }
  };
  load_chunk(pre, u0);

  // 1. the tile's band coefficients cs[tt][e] and, in slab 0, the state sums.
  //    Span row u = t0 - off + x holds state[u] in sst[x] (0 outside the batch
  //    element); row tt's slot e meets span row x = tt + e.
  float* sst = vs;  // the value staging area is free until the first chunk
  const bool sums = s == 0 && a.out_state && a.state;
  if (sums)
    for (int x = threadIdx.x; x < span; x += 256) {
      const int u = u0 + x;
      sst[x] = (u >= 0 && u < a.N) ? a.state[base + u] : 0.f;
    }
  if (TRANS || a.compress == 0) {
    // elementwise: every (row, slot) independently, all threads at once, in
    // groups of kCoefBatch entries per thread whose loads all issue before
    // the first is used
    // Entry x = tt k + e advances by 256 per step: (tt, e) move by (256 / k,
    // 256 % k) with a carry, so the loop divides only once.
    constexpr int kCoefBatch = 8;
    const int n = kBandRows * a.k;
    const int dt = 256 / a.k, de = 256 - dt * a.k;
    int tt_x = (int)threadIdx.x / a.k, e_x = (int)threadIdx.x - tt_x * a.k;  // entry x0 + threadIdx.x
    for (int x0 = 0; x0 < n; x0 += 256 * kCoefBatch) {
      float c[kCoefBatch];
      int ttj[kCoefBatch], ej[kCoefBatch];
#pragma unroll
      for (int j = 0; j < kCoefBatch; ++j) {
        ttj[j] = tt_x;
        ej[j] = e_x;
        e_x += de;
        tt_x += dt;
        if (e_x >= a.k) {
          e_x -= a.k;
          ++tt_x;
        }
      }
#pragma unroll
      for (int j = 0; j < kCoefBatch; ++j) {
        const int tt = ttj[j], e = ej[j];
        const int i = t0 + tt;
        c[j] = 0.f;
        if constexpr (TRANS) {  // incoming edge from row i + e, which holds this key in slot k - 1 - e
          if (tt < kBandRows && i < a.N && i + e < a.N) c[j] = a.coef[(base + i + e) * a.k + (a.k - 1 - e)];
        } else {  // slot e of row i is key i - (k - 1 - e), absent below 0
          if (tt < kBandRows && i < a.N && i - (a.k - 1 - e) >= 0) c[j] = a.score[(base + i) * a.k + e];
        }
      }
#pragma unroll
      for (int j = 0; j < kCoefBatch; ++j)
        if (ttj[j] < kBandRows) cs[ttj[j] * kst + ej[j]] = TRANS ? c[j] : softsign_f(c[j]);
    }
  } else {
    // row-normalising kinds: one row per wave pass, 64 slots at a time
    for (int tt = w; tt < kBandRows; tt += 4) {
      const int i = t0 + tt;
      const int64_t row = base + i;
      RowStats rst;
      if (i < a.N) rst = row_compress_stats(a.idx, a.score, row, a.k, a.compress);  // wave-uniform
      for (int e0 = 0; e0 < a.k; e0 += kWave) {
        float c = 0.f;
        if (i < a.N) {
          int j;
          float sc;
          row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rst, j, c, sc);  // absent: 0
        }
        if (e0 + lane < a.k) cs[tt * kst + e0 + lane] = c;
      }
    }
  }
  __syncthreads();
  if (sums) {
    // four lanes per row, slots e = part (mod 4), combined in a fixed order
    const int tt = threadIdx.x >> 2, part = threadIdx.x & 3;
    float st = 0.f;
    for (int e = part; e < a.k; e += 4) st += cs[tt * kst + e] * sst[tt + e];
    st += shfl_xor_f(st, 1);
    st += shfl_xor_f(st, 2);
    if (part == 0 && t0 + tt < a.N) a.out_state[base + t0 + tt] = st;
  }

  // 2. the span chunk by chunk
  // this wave's 16 rows touch span rows [wlo, whi)
  const int wlo = u0 + 16 * w, whi = u0 + 16 * w + 15 + a.k;
  floatx4 acc[COLS / 16];
#pragma unroll
  for (int nt = 0; nt < COLS / 16; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // the state sums are done with sst (the value staging area)
  const int tt = 16 * w + col;  // this lane's A row
  auto chunk_mfma = [&](int uc) {
    if (uc + kBandChunk > wlo && uc < whi) {  // wave-uniform
#pragma unroll
      for (int ks = 0; ks < kBandChunk / 4; ++ks) {
        const int e = uc + 4 * ks + grp - (t0 + tt) + off;
        const float av = (e >= 0 && e < a.k) ? cs[tt * kst + e] : 0.f;
#pragma unroll
        for (int nt = 0; nt < COLS / 16; ++nt)
          acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, vs[(4 * ks + grp) * VST + nt * 16 + col], acc[nt], 0,
                                                         0, 0);
      }
    }
  };
  for (int ch = 0; ch < nchunks; ++ch) {
    const int uc = u0 + ch * kBandChunk;
    store_chunk(pre);
    __syncthreads();
    if (ch + 1 < nchunks) load_chunk(pre, uc + kBandChunk);  // in flight during the MFMAs
    chunk_mfma(uc);
    __syncthreads();  // before the next chunk overwrites vs
  }

  // 3. lane holds rows 4 grp + v of each 16 x 16 tile, column col
  T* out = reinterpret_cast<T*>(a.out);
#pragma unroll
  for (int nt = 0; nt < COLS / 16; ++nt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = t0 + 16 * w + 4 * grp + v, d = d0 + nt * 16 + col;
      if (i < a.N && d < a.D) out[(base + i) * a.ld_out + d] = (T)acc[nt][v];
    }
}

// ---------------------------------------------------------------------------
// Dots: G[i, e] = <gdv[i], pv[i - (k - 1) + e]> for a 64-row tile, as the
// 64 x (16 NT) product of the tile's gdv rows with its span of pv rows over
// one half of the D columns (slab 0 writes g_score, slab 1 writes coef; the
// row backward adds the two).  Both operands stage 16-column slices in LDS
// (double buffered, one barrier per slice); a wave owns 16 rows and only
// multiplies the span tiles its band meets.
// ---------------------------------------------------------------------------
template <typename T, int NT, bool SCORES>
__global__ __launch_bounds__(256) void band_dots_kernel(BandDotsArgs a) {
  __shared__ __align__(16) float sA[2][kBandRows * kBandKStride];
  __shared__ __align__(16) float sB[2][NT * 16 * kBandKStride];
  constexpr int W = 16 / (int)sizeof(T);
  constexpr int kPackCols = 16 / W;  // packs per row of a 16-column slice
  const int lane = lane_id(), w = wave_id();
  const int col = lane & 15, grp = lane >> 4;
  const int tiles = (a.N + kBandRows - 1) / kBandRows;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int t = (int)(logical % tiles);
  constexpr bool scores = SCORES;  // score mode: a.score_out is set
  const int halves = scores ? 1 : 2;
  const int half = (int)((logical / tiles) % halves);
  const int64_t b = logical / tiles / halves;
  const int t0 = t * kBandRows, u0 = t0 - (a.k - 1);
  const int64_t base = b * a.N;
  const int dh = ((a.D + halves - 1) / halves + 15) / 16 * 16;
  const int d_begin = half * dh, d_end = min(a.D, d_begin + dh);
  const int nslices = d_end > d_begin ? (d_end - d_begin + 15) / 16 : 0;
  const T* gdv = reinterpret_cast<const T*>(a.gdv);
  const T* pv = reinterpret_cast<const T*>(a.pv);

  // staged packs per thread: A has 64 rows, B 16 NT rows, of kPackCols packs each
  constexpr int kApacks = (kBandRows * kPackCols + 255) / 256;
  constexpr int kBpacks = (NT * 16 * kPackCols + 255) / 256;
  // three slices of loads in flight: register set s % 3 holds slice s from
  // its load (issued three slices ahead) until its store into LDS
  constexpr int kRing = 3;
  Pack<W> pa_ring[kRing][kApacks], pb_ring[kRing][kBpacks];
  auto load_slice = [&](auto SET, int d) {
    constexpr int S = decltype(SET)::value;
    Pack<W>(&pa)[kApacks] = pa_ring[S];
    Pack<W>(&pb)[kBpacks] = pb_ring[S];
#pragma unroll
    for (int p = 0; p < kApacks; ++p) {
      const int x = threadIdx.x + p * 256;
      const int r = x / kPackCols, dd = d + (x % kPackCols) * W;
      const int i = t0 + r;
      const bool ok = r < kBandRows && i < a.N && dd < d_end;
      pa[p] = ok ? load_pack<T, W>(gdv + (base + i) * a.ld_gdv + dd) : pack_zero<T, W>();
      if (a.ascale && ok) {  // score mode (fp32): the scaled query
#pragma unroll
        for (int q = 0; q < W; ++q) pa[p].v[q] = pa[p].v[q] * a.ascale[dd + q];
      }
    }
#pragma unroll
    for (int p = 0; p < kBpacks; ++p) {
      const int x = threadIdx.x + p * 256;
      const int r = x / kPackCols, dd = d + (x % kPackCols) * W;
      const int u = u0 + r;
      pb[p] = (r < NT * 16 && u >= 0 && u < a.N && dd < d_end)
                  ? load_pack<T, W>(pv + (base + u) * a.ld_pv + dd)
                  : pack_zero<T, W>();
    }
  };
  auto store_slice = [&](auto SET, int buf) {
    constexpr int S = decltype(SET)::value;
    const Pack<W>(&pa)[kApacks] = pa_ring[S];
    const Pack<W>(&pb)[kBpacks] = pb_ring[S];
#pragma unroll
    for (int p = 0; p < kApacks; ++p) {
      const int x = threadIdx.x + p * 256;
      if (x / kPackCols < kBandRows) {
        float* dst = &sA[buf][(x / kPackCols) * kBandKStride + (x % kPackCols) * W];
#pragma unroll
        for (int q = 0; q < W; q += 4)
          *reinterpret_cast<float4*>(dst + q) = make_float4(pa[p].v[q], pa[p].v[q + 1], pa[p].v[q + 2],
                                                            pa[p].v[q + 3]);
      }
    }
#pragma unroll
    for (int p = 0; p < kBpacks; ++p) {
      const int x = threadIdx.x + p * 256;
      if (x / kPackCols < NT * 16) {
        float* dst = &sB[buf][(x / kPackCols) * kBandKStride + (x % kPackCols) * W];
#pragma unroll
        for (int q = 0; q < W; q += 4)
          *reinterpret_cast<float4*>(dst + q) = make_float4(pb[p].v[q], pb[p].v[q + 1], pb[p].v[q + 2],
                                                            pb[p].v[q + 3]);
      }
    }
  };

  // span tiles nt this wave's band meets: nt in [w, w + ntb)
  const int ntb = (a.k + 15 + 15) / 16;
  floatx4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
  constexpr std::integral_constant<int, 0> kS0{};
  constexpr std::integral_constant<int, 1> kS1{};
  constexpr std::integral_constant<int, 2> kS2{};
  if (nslices > 0) load_slice(kS0, d_begin);
  if (nslices > 1) load_slice(kS1, d_begin + 16);
  if (nslices > 2) load_slice(kS2, d_begin + 32);
  if (nslices > 0) store_slice(kS0, 0);
  __syncthreads();
  // slice sl: its set (sl % 3) was stored into LDS buffer sl & 1 before the
  // last barrier, so the set takes the loads of slice sl + 3; then the MFMAs
  // over buffer sl & 1 and the store of slice sl + 1 (set (sl + 1) % 3) into
  // the other buffer, which every wave finished reading before that barrier
  auto step = [&](auto SET, auto NEXT, int sl) {
    if (sl >= nslices) return;  // uniform
    const int cur = sl & 1;
    if (sl + kRing < nslices) load_slice(SET, d_begin + (sl + kRing) * 16);
    const float4 av = *reinterpret_cast<const float4*>(&sA[cur][(16 * w + col) * kBandKStride + grp * 4]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt < w || nt >= w + ntb) continue;  // wave-uniform
      const float4 bv = *reinterpret_cast<const float4*>(&sB[cur][(nt * 16 + col) * kBandKStride + grp * 4]);
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc[nt], 0, 0, 0);
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc[nt], 0, 0, 0);
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc[nt], 0, 0, 0);
      acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc[nt], 0, 0, 0);
    }
    if (sl + 1 < nslices) store_slice(NEXT, cur ^ 1);
    __syncthreads();
  };
  for (int sl = 0; sl < nslices; sl += kRing) {
    step(kS0, kS1, sl);
    step(kS1, kS2, sl + 1);
    step(kS2, kS0, sl + 2);
  }

  // lane holds rows 4 grp + v (query i) and column col (span row u) of each tile
  if (scores) {
    const float bias = a.bias ? a.bias[0] : 0.0f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = t0 + 16 * w + 4 * grp + v;
        const int e = u0 + nt * 16 + col - i + (a.k - 1);
        if (i < a.N && e >= 0 && e < a.k) {
          const int j = i - (a.k - 1) + e;
          a.score_out[(base + i) * a.k + e] = j >= 0 ? (acc[nt][v] + bias) * a.inv_temperature : 0.0f;
          a.idx_out[(base + i) * a.k + e] = j >= 0 ? j : -1;
        }
      }
    return;
  }
  float* part = half == 0 ? a.g_score : a.coef;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int i = t0 + 16 * w + 4 * grp + v;
      const int e = u0 + nt * 16 + col - i + (a.k - 1);
      if (i < a.N && e >= 0 && e < a.k) part[(base + i) * a.k + e] = acc[nt][v];
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static std::atomic<int> g_window_kernels{0};
void set_window_kernels(int mode) { g_window_kernels.store(mode, std::memory_order_relaxed); }
int window_kernels() { return g_window_kernels.load(std::memory_order_relaxed); }

bool band_kernels_fit(int k, int D, int64_t ld_a, int64_t ld_b, const void* pa, const void* pb, bool bf16) {
  const int pw = bf16 ? 8 : 4;  // elements per 16-byte pack
  return k >= 1 && k <= kBandMaxK && D >= 1 && D % pw == 0 && ld_a % pw == 0 && ld_b % pw == 0 &&
         (reinterpret_cast<uintptr_t>(pa) & 15) == 0 && (reinterpret_cast<uintptr_t>(pb) & 15) == 0;
}

template <int COLS>
static void launch_band_aggregate_cols(const BandAggArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  if (a.bf16) {
    if (a.trans) hipLaunchKernelGGL((band_aggregate_kernel<bf16_t, true, COLS>), grid, dim3(256), lds, stream, a);
    else hipLaunchKernelGGL((band_aggregate_kernel<bf16_t, false, COLS>), grid, dim3(256), lds, stream, a);
  } else {
    if (a.trans) hipLaunchKernelGGL((band_aggregate_kernel<float, true, COLS>), grid, dim3(256), lds, stream, a);
    else hipLaunchKernelGGL((band_aggregate_kernel<float, false, COLS>), grid, dim3(256), lds, stream, a);
  }
}

int launch_band_aggregate(const BandAggArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.N == 0) return kOk;
  JN_REQUIRE(band_kernels_fit(a.k, a.D, a.ld_val, a.ld_out, a.val, a.out, a.bf16), kInvalidArgument,
             "band aggregate: k in [1, %d], D and row strides in whole 16-byte packs, aligned rows", kBandMaxK);
  JN_REQUIRE(a.trans ? (a.coef != nullptr) : (a.idx && a.score), kInvalidArgument, "null tensor pointer");
  const int64_t tiles = (a.N + kBandRows - 1) / kBandRows;
  const bool narrow = (int64_t)a.B * tiles * ((a.D + kBandColsWide - 1) / kBandColsWide) < kBandNarrowBelow;
  const int cols = narrow ? kBandColsNarrow : kBandColsWide;
  const int64_t blocks = (int64_t)a.B * tiles * ((a.D + cols - 1) / cols);
  JN_REQUIRE(blocks < (1LL << 31) && (int64_t)a.B * a.N * a.k < (1LL << 31), kInvalidArgument, "too many rows");
  const size_t lds = band_aggregate_lds_bytes(a.k, cols);
  const dim3 grid((unsigned)blocks);
  JN_PROFILE(a.trans ? "band_columns_kernel" : "band_forward_kernel", stream);
  if (narrow) launch_band_aggregate_cols<kBandColsNarrow>(a, grid, lds, stream);
  else launch_band_aggregate_cols<kBandColsWide>(a, grid, lds, stream);
  JN_LAUNCH_CHECK();
  return kOk;
}

template <typename T, bool SCORES>
static void launch_band_dots_nt(const BandDotsArgs& a, dim3 grid, hipStream_t stream) {
  const int nt = (kBandRows - 1 + a.k + 15) / 16;  // span tiles of 16 rows
  if (nt <= 6) hipLaunchKernelGGL((band_dots_kernel<T, 6, SCORES>), grid, dim3(256), 0, stream, a);
  else if (nt <= 8) hipLaunchKernelGGL((band_dots_kernel<T, 8, SCORES>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((band_dots_kernel<T, 12, SCORES>), grid, dim3(256), 0, stream, a);
}

int launch_band_dots(const BandDotsArgs& a, hipStream_t stream) {
  if (a.B == 0 || a.N == 0) return kOk;
  JN_REQUIRE(band_kernels_fit(a.k, a.D, a.ld_gdv, a.ld_pv, a.gdv, a.pv, a.bf16), kInvalidArgument,
             "band dots: k in [1, %d], D and row strides in whole 16-byte packs, aligned rows", kBandMaxK);
  const bool scores = a.score_out != nullptr;
  JN_REQUIRE(scores ? (a.idx_out != nullptr && !a.bf16) : (a.g_score && a.coef), kInvalidArgument,
             "null tensor pointer or bf16 scores");
  const int64_t tiles = (a.N + kBandRows - 1) / kBandRows;
  const int64_t blocks = (int64_t)a.B * tiles * (scores ? 1 : 2);
  JN_REQUIRE(blocks < (1LL << 31) && (int64_t)a.B * a.N * a.k < (1LL << 31), kInvalidArgument, "too many rows");
  const dim3 grid((unsigned)blocks);
  JN_PROFILE(scores ? "band_scores_kernel" : "band_dots_kernel", stream);
  if (scores) launch_band_dots_nt<float, true>(a, grid, stream);
  else if (a.bf16) launch_band_dots_nt<bf16_t, false>(a, grid, stream);
  else launch_band_dots_nt<float, false>(a, grid, stream);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
