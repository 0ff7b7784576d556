// Edge-list kernels shared by top-k and window propagation (gfx950).
//
// An edge list is (idx[row, e], score[row, e]) for rows = B*Nq query rows and
// e < k; idx < 0 marks an absent edge (window rows near the start).  Indices
// are local to the batch element of the row.
//
//   rows_forward   : delta_state[i] = sum_e c(s_ie) ps[j],  delta_val[i] = sum_e c(s_ie) pv[j]
//                    (propagation.py:473-479, gather form of jakal_net_native.cpp:6426-6438)
//   rows_backward  : grad wrt coefficients, compress backward, grad wrt the query projection
//   csr_*          : deterministic transpose of the edge list to key-major order
//   cols_backward  : scatter-side grads (grad pv, grad ps, grad key projection) as gathers
//
// Compress kinds: 0 softsign (propagation.py:85-88), 1 signed |s| softmax over the
// row's selected edges (propagation.py:74-82).
#include "jn_internal.hpp"

namespace jakal {

// ---------------------------------------------------------------------------
// Vector helpers: a lane moves W consecutive floats (W = 4 when the row
// stride and base are 16-byte aligned, else 1).
// ---------------------------------------------------------------------------
template <int W>
__device__ __forceinline__ float4 load_w(const float* p) {
  if constexpr (W == 4) return *reinterpret_cast<const float4*>(p);
  else return make_float4(p[0], 0.f, 0.f, 0.f);
}
template <int W>
__device__ __forceinline__ void store_w(float* p, float4 v) {
  if constexpr (W == 4) *reinterpret_cast<float4*>(p) = v;
  else p[0] = v.x;
}
__device__ __forceinline__ void fma4(float4& acc, float c, float4 v) {
  acc.x += c * v.x;
  acc.y += c * v.y;
  acc.z += c * v.z;
  acc.w += c * v.w;
}
__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

__device__ __forceinline__ float sign_f(float s) { return (s > 0.f) ? 1.f : ((s < 0.f) ? -1.f : 0.f); }

// ---------------------------------------------------------------------------
// Row forward: one wavefront per query row.
// ---------------------------------------------------------------------------

// Row statistics for the signed |s| softmax (max |s| and 1/sum exp).
__device__ __forceinline__ void row_abs_softmax_stats(const int32_t* idx, const float* score, int64_t row, int k,
                                                      float& row_max, float& row_inv_sum) {
  const int lane = lane_id();
  float m = -INFINITY;
  for (int e = lane; e < k; e += kWave)
    if (idx[row * k + e] >= 0) m = fmaxf(m, fabsf(score[row * k + e]));
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, shfl_xor_f(m, s));
  float sum = 0.0f;
  for (int e = lane; e < k; e += kWave)
    if (idx[row * k + e] >= 0) sum += __expf(fabsf(score[row * k + e]) - m);
  sum = wave_sum(sum);
  row_max = m;
  row_inv_sum = sum > 0.f ? 1.0f / sum : 0.0f;
}

// Coefficient of edge e0 + lane of a row (0 for absent edges).
__device__ __forceinline__ void row_coefficients(const int32_t* idx, const float* score, int64_t row, int k, int e0,
                                                 int compress, float row_max, float row_inv_sum, int& j, float& c,
                                                 float& s) {
  const int e = e0 + lane_id();
  j = -1;
  c = 0.0f;
  s = 0.0f;
  if (e < k) {
    j = idx[row * k + e];
    if (j >= 0) {
      s = score[row * k + e];
      c = (compress == 0) ? softsign_f(s) : sign_f(s) * __expf(fabsf(s) - row_max) * row_inv_sum;
    }
  }
}

template <int W>
__global__ __launch_bounds__(256) void rows_forward_kernel(RowsFwdArgs a) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Nq;
  const float* pvb = a.pv + b * a.Nk * a.ld_pv;
  const float* psb = a.ps + b * a.Nk;
  float* out = a.out_val + row * a.D;

  float rmax = 0.f, rinv = 0.f;
  if (a.compress == 1) row_abs_softmax_stats(a.idx, a.score, row, a.k, rmax, rinv);

  float st = 0.0f;
  for (int e0 = 0; e0 < a.k; e0 += kWave) {
    int j;
    float c, s;
    row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rmax, rinv, j, c, s);
    if (j >= 0) st += c * psb[j];
    const int ne = min(kWave, a.k - e0);
    for (int d = lane * W; d < a.D; d += kWave * W) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      int q = 0;
      for (; q + 8 <= ne; q += 8) {
        float4 v[8];
        float cc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int jj = readlane_i(j, q + u);
          cc[u] = jj < 0 ? 0.f : readlane_f(c, q + u);
          v[u] = load_w<W>(pvb + (int64_t)(jj < 0 ? 0 : jj) * a.ld_pv + d);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) fma4(acc, cc[u], v[u]);
      }
      for (; q < ne; ++q) {
        const int jj = readlane_i(j, q);
        if (jj < 0) continue;
        fma4(acc, readlane_f(c, q), load_w<W>(pvb + (int64_t)jj * a.ld_pv + d));
      }
      if (e0 > 0) acc = add4(acc, load_w<W>(out + d));
      store_w<W>(out + d, acc);
    }
  }
  st = wave_sum(st);
  if (lane == 0) a.out_state[row] = st;
}

int launch_rows_forward(const RowsFwdArgs& a, hipStream_t stream) {
  if (a.rows == 0) return kOk;
  const int64_t blocks = (a.rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  const bool vec = (a.D % 4 == 0) && (a.ld_pv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.pv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.out_val) & 15) == 0);
  JN_PROFILE("rows_forward_kernel", stream);
  if (vec) hipLaunchKernelGGL(rows_forward_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(rows_forward_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Row backward: one wavefront per query row, edges in groups of KP (<= 64).
//   g_c[e]   = gds[i] * ps[j] + <gdv[i], pv[j]>        (grad wrt edge coefficient)
//   g_s[e]   = compress backward of g_c, times 1/T      (grad wrt score)
//   dQ[i, r] = qscale[r] * sum_e g_s[e] * key[j, r]      (grad wrt query projection)
//   coef[e]  = c(s_e)                                    (kept for the column pass)
//   rowsum_gs[i] = sum_e g_s[e]                          (bias gradient partial)
// Per-edge dot products are accumulated per lane over D and reduced for all KP
// edges at once with a halving butterfly (KP-1 cross-lane ops instead of 6*KP).
// ---------------------------------------------------------------------------

// Reduce p[0..KP) (one partial per edge, per lane) across the wave.  Returns,
// in every lane, the total of edge (lane >> log2(64/KP)).
template <int KP>
__device__ __forceinline__ float multi_reduce(float (&p)[KP]) {
  const int lane = lane_id();
  int m = 32;
#pragma unroll
  for (int h = KP / 2; h >= 1; h >>= 1, m >>= 1) {
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int q = 0; q < h; ++q) {
      float send = upper ? p[q] : p[q + h];
      float keep = upper ? p[q + h] : p[q];
      p[q] = keep + shfl_xor_f(send, m);
    }
  }
  float v = p[0];
  for (; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}

template <int W, int KP>
__global__ __launch_bounds__(256) void rows_backward_kernel(RowsBwdArgs a) {
  constexpr int kShift = (KP == 64) ? 0 : (KP == 32 ? 1 : (KP == 16 ? 2 : 3));
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Nq;
  const float* pvb = a.pv + b * a.Nk * a.ld_pv;
  const float* psb = a.ps + b * a.Nk;
  const float* keyb = a.key + b * a.Nk * a.ldk;
  const float* grow = a.gdv + row * a.D;
  const float gs_row = a.gds[row];

  float rmax = 0.f, rinv = 0.f;
  if (a.compress == 1) row_abs_softmax_stats(a.idx, a.score, row, a.k, rmax, rinv);

  float dq_acc0 = 0.f, dq_acc1 = 0.f;  // rank lanes: lane and lane + 64
  float gsum = 0.f;
  for (int e0 = 0; e0 < a.k; e0 += KP) {
    int j;
    float c, s;
    // lanes < KP hold edges e0 + lane
    row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rmax, rinv, j, c, s);
    if (lane >= KP) j = -1;
    const int ne = min(KP, a.k - e0);
    float p[KP];
#pragma unroll
    for (int q = 0; q < KP; ++q) p[q] = 0.f;
    for (int d = lane * W; d < a.D; d += kWave * W) {
      const float4 gv = load_w<W>(grow + d);
#pragma unroll
      for (int q0 = 0; q0 < KP; q0 += 8) {
        if (q0 < ne) {  // uniform; absent edges (j < 0) read row 0 and are masked
          float4 v[8];
          float msk[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int jj = readlane_i(j, q0 + u);
            msk[u] = jj >= 0 ? 1.f : 0.f;
            v[u] = load_w<W>(pvb + (int64_t)(jj < 0 ? 0 : jj) * a.ld_pv + d);
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) p[q0 + u] += msk[u] * dot4(gv, v[u]);
        }
      }
    }
    const float dot_all = multi_reduce<KP>(p);
    // bring edge `lane` (for lane < KP) to its own lane
    const float dot = __int_as_float(__builtin_amdgcn_ds_bpermute((lane << kShift) << 2, __float_as_int(dot_all)));
    float gc = (j >= 0) ? gs_row * psb[j] + dot : 0.f;
    float gsc = 0.f;
    if (a.compress == 1) {
      const float row_dot = wave_sum(gc * c);  // single group: k <= KP enforced on the host
      if (j >= 0) {
        const float sg = sign_f(s);
        gsc = sg * (sg * c) * (sg * gc - row_dot);
      }
    } else if (j >= 0) {
      gsc = gc * softsign_grad_f(s);
    }
    gsc *= a.inv_temperature;
    if (lane < ne) {
      a.g_score[row * a.k + e0 + lane] = gsc;
      a.coef[row * a.k + e0 + lane] = c;
    }
    gsum += gsc;
    for (int q = 0; q < ne; ++q) {
      const int jj = readlane_i(j, q);
      if (jj < 0) continue;
      const float gg = readlane_f(gsc, q);
      const float* kr = keyb + (int64_t)jj * a.ldk;
      if (lane < a.r) dq_acc0 += gg * kr[lane];
      if (lane + kWave < a.r) dq_acc1 += gg * kr[lane + kWave];
    }
  }
  if (lane < a.r) a.dq[row * a.lddq + lane] = dq_acc0 * (a.qscale ? a.qscale[lane] : 1.f);
  if (lane + kWave < a.r) a.dq[row * a.lddq + lane + kWave] = dq_acc1 * (a.qscale ? a.qscale[lane + kWave] : 1.f);
  gsum = wave_sum(gsum);
  if (lane == 0) a.rowsum_gs[row] = gsum;
}

int launch_rows_backward(const RowsBwdArgs& a, hipStream_t stream) {
  if (a.rows == 0) return kOk;
  JN_REQUIRE(a.r >= 1 && a.r <= 128, kUnsupported, "rank must be in [1, 128]");
  JN_REQUIRE(a.compress == 0 || a.k <= 64, kUnsupported, "signed_abs_softmax backward supports k <= 64");
  const int64_t blocks = (a.rows + 3) / 4;
  const bool vec = (a.D % 4 == 0) && (a.ld_pv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.pv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.gdv) & 15) == 0);
  dim3 grid((unsigned)blocks), block(256);
  JN_PROFILE("rows_backward_kernel", stream);
  if (a.k <= 16) {
    if (vec) hipLaunchKernelGGL((rows_backward_kernel<4, 16>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((rows_backward_kernel<1, 16>), grid, block, 0, stream, a);
  } else if (a.k <= 32) {
    if (vec) hipLaunchKernelGGL((rows_backward_kernel<4, 32>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((rows_backward_kernel<1, 32>), grid, block, 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((rows_backward_kernel<4, 64>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((rows_backward_kernel<1, 64>), grid, block, 0, stream, a);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Deterministic transpose (CSR by key) of the edge list.
//
// Rows are cut into tiles of 64; inside a tile a key column's incoming rows
// form a 64-bit mask in LDS.  The position of edge (row, j) in j's segment is
//   seg_start[j] + rows of earlier tiles hitting j + popcount(mask_j below row).
// Segments therefore list incoming edges in increasing row order and every
// reduction over them is run-to-run reproducible.
// ---------------------------------------------------------------------------
constexpr int kCsrSlice = 8192;  // key columns per LDS pass (64 KiB of masks)


__device__ void csr_build_masks(const CsrArgs& a, int b, int t, int s0, int s1, unsigned long long* masks) {
  for (int x = threadIdx.x; x < s1 - s0; x += blockDim.x) masks[x] = 0ull;
  __syncthreads();
  const int r0 = t * kCsrTile;
  const int nrows = min(kCsrTile, a.Nq - r0);
  for (int x = threadIdx.x; x < nrows * a.k; x += blockDim.x) {
    int rl = x / a.k;
    int j = a.idx[((int64_t)b * a.Nq + r0 + rl) * a.k + (x % a.k)];
    if (j >= s0 && j < s1) atomicOr(&masks[j - s0], 1ull << rl);
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void csr_count_kernel(CsrArgs a) {
  __shared__ unsigned long long masks[kCsrSlice];
  const int t = blockIdx.x, b = blockIdx.y;
  const int T = gridDim.x;
  for (int s0 = 0; s0 < a.Nk; s0 += kCsrSlice) {
    const int s1 = min(a.Nk, s0 + kCsrSlice);
    csr_build_masks(a, b, t, s0, s1, masks);
    for (int x = threadIdx.x; x < s1 - s0; x += blockDim.x)
      a.tile_base[((int64_t)b * T + t) * a.Nk + s0 + x] = __popcll(masks[x]);
    __syncthreads();
  }
}

// Exclusive scan over tiles for every (b, key); the total is the key's in-degree.
__global__ void csr_tile_scan_kernel(CsrArgs a, int T) {
  int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (x >= (int64_t)a.B * a.Nk) return;
  int b = (int)(x / a.Nk), j = (int)(x % a.Nk);
  int run = 0;
  for (int t = 0; t < T; ++t) {
    int32_t* p = a.tile_base + ((int64_t)b * T + t) * a.Nk + j;
    int c = *p;
    *p = run;
    run += c;
  }
  a.seg_start[(int64_t)b * (a.Nk + 1) + j] = run;  // degree, scanned next
}

// In-place exclusive scan of the degrees of one batch element (one workgroup).
__global__ __launch_bounds__(1024) void csr_segment_scan_kernel(CsrArgs a) {
  __shared__ int warp_tot[16];
  __shared__ int carry;
  const int b = blockIdx.x;
  int32_t* seg = a.seg_start + (int64_t)b * (a.Nk + 1);
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const int lane = lane_id(), wave = wave_id();
  for (int base = 0; base < a.Nk; base += 1024) {
    int x = base + threadIdx.x;
    int v = x < a.Nk ? seg[x] : 0;
    // inclusive wave scan
    int s = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      int y = __builtin_amdgcn_ds_bpermute(((lane - o) & 63) << 2, s);
      if (lane >= o) s += y;
    }
    if (lane == 63) warp_tot[wave] = s;
    __syncthreads();
    int woff = 0;
    for (int w = 0; w < wave; ++w) woff += warp_tot[w];
    int excl = carry + woff + s - v;
    __syncthreads();
    if (x < a.Nk) seg[x] = excl;
    if (threadIdx.x == 1023) carry = excl + v;
    __syncthreads();
  }
  if (threadIdx.x == 0) seg[a.Nk] = carry;
}

__global__ __launch_bounds__(256) void csr_fill_kernel(CsrArgs a) {
  __shared__ unsigned long long masks[kCsrSlice];
  const int t = blockIdx.x, b = blockIdx.y;
  const int T = gridDim.x;
  const int r0 = t * kCsrTile;
  const int nrows = min(kCsrTile, a.Nq - r0);
  const int64_t batch_base = (int64_t)b * a.Nq * a.k;
  const int32_t* seg = a.seg_start + (int64_t)b * (a.Nk + 1);
  for (int s0 = 0; s0 < a.Nk; s0 += kCsrSlice) {
    const int s1 = min(a.Nk, s0 + kCsrSlice);
    csr_build_masks(a, b, t, s0, s1, masks);
    for (int x = threadIdx.x; x < nrows * a.k; x += blockDim.x) {
      int rl = x / a.k;
      int64_t eid = ((int64_t)b * a.Nq + r0 + rl) * a.k + (x % a.k);
      int j = a.idx[eid];
      if (j >= s0 && j < s1) {
        unsigned long long below = masks[j - s0] & ((1ull << rl) - 1ull);
        int pos = seg[j] + a.tile_base[((int64_t)b * T + t) * a.Nk + j] + __popcll(below);
        a.edges[batch_base + pos] = (int32_t)eid;
      }
    }
    __syncthreads();
  }
}

size_t csr_workspace_ints(int B, int Nq, int Nk, int k, size_t& tile_ints, size_t& seg_ints, size_t& edge_ints) {
  const int T = (Nq + kCsrTile - 1) / kCsrTile;
  tile_ints = (size_t)B * T * Nk;
  seg_ints = (size_t)B * (Nk + 1);
  edge_ints = (size_t)B * Nq * k;
  return tile_ints + seg_ints + edge_ints;
}

int launch_csr(const CsrArgs& a, hipStream_t stream) {
  const int T = (a.Nq + kCsrTile - 1) / kCsrTile;
  JN_REQUIRE((int64_t)a.B * a.Nq * a.k < (1LL << 31), kUnsupported, "edge count exceeds int32 ids");
  dim3 g2(T, a.B);
  {
    JN_PROFILE("csr_count_kernel", stream);
    hipLaunchKernelGGL(csr_count_kernel, g2, dim3(256), 0, stream, a);
    JN_LAUNCH_CHECK();
  }
  const int64_t n = (int64_t)a.B * a.Nk;
  {
    JN_PROFILE("csr_tile_scan_kernel", stream);
    hipLaunchKernelGGL(csr_tile_scan_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, T);
    JN_LAUNCH_CHECK();
  }
  {
    JN_PROFILE("csr_segment_scan_kernel", stream);
    hipLaunchKernelGGL(csr_segment_scan_kernel, dim3(a.B), dim3(1024), 0, stream, a);
    JN_LAUNCH_CHECK();
  }
  {
    JN_PROFILE("csr_fill_kernel", stream);
    hipLaunchKernelGGL(csr_fill_kernel, g2, dim3(256), 0, stream, a);
    JN_LAUNCH_CHECK();
  }
  return kOk;
}

// ---------------------------------------------------------------------------
// Column backward: one wavefront per key column j, walking its CSR segment.
//   grad_pv[j]  = sum_in coef * gdv[i]
//   grad_ps[j]  = sum_in coef * gds[i]
//   dK[j, r]    = kscale[r] * sum_in g_s * q[i, r]
//   part_c[w,r] += key[j, r] * sum_in g_s * q[i, r]      (scale-vector gradient)
// Each wavefront owns a fixed run of columns so partials are reproducible.
// ---------------------------------------------------------------------------

template <bool VEC>
__global__ __launch_bounds__(256) void cols_backward_kernel(ColsBwdArgs a) {
  const int lane = lane_id();
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave_id();
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  const int64_t nwaves = (total_cols + a.cols_per_wave - 1) / a.cols_per_wave;
  if (gw >= nwaves) return;  // padding waves of the last workgroup own no partial slot
  const int64_t col_begin = gw * a.cols_per_wave;
  float pc0 = 0.f, pc1 = 0.f;
  constexpr int W = VEC ? 4 : 1;
  for (int64_t cc = 0; cc < a.cols_per_wave; ++cc) {
    const int64_t colg = col_begin + cc;
    if (colg >= total_cols) break;
    const int b = (int)(colg / a.Nk), j = (int)(colg % a.Nk);
    const int32_t* seg = a.seg_start + (int64_t)b * (a.Nk + 1);
    const int s_beg = seg[j], s_end = seg[j + 1];
    const int32_t* el = a.edges + (int64_t)b * a.Nq * a.k;

    float dk0 = 0.f, dk1 = 0.f, st = 0.f;
    // value gradient: loop D in passes of 64*W*2 so the accumulators stay in VGPRs
    for (int d0 = 0; d0 < (a.grad_pv ? a.D : 1); d0 += kWave * W * 2) {
      float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      const int dl0 = d0 + lane * W, dl1 = d0 + kWave * W + lane * W;
      const bool first_pass = (d0 == 0);
      for (int p0 = s_beg; p0 < s_end; p0 += kWave) {
        const int n = min(kWave, s_end - p0);
        int eid = 0;
        float cf = 0.f, gsv = 0.f;
        if (lane < n) {
          eid = el[p0 + lane];
          cf = a.coef[eid];
          if (first_pass) gsv = a.g_score[eid];
        }
        const int row_of = eid / a.k;
        if (first_pass && lane < n && a.gds) st += cf * a.gds[row_of];
        const int row0 = readlane_i(row_of, 0);
        for (int q0 = 0; q0 < n; q0 += 4) {
          int64_t rw[4];
          float cu[4], gg[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const bool ok = q0 + u < n;  // uniform
            rw[u] = ok ? readlane_i(row_of, q0 + u) : row0;
            cu[u] = ok ? readlane_f(cf, q0 + u) : 0.f;
            gg[u] = ok ? readlane_f(gsv, q0 + u) : 0.f;
          }
          if (a.grad_pv) {
            float4 v0[4], v1[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float* gr = a.gdv + rw[u] * a.D;
              if (dl0 < a.D) v0[u] = load_w<W>(gr + dl0);
              if (dl1 < a.D) v1[u] = load_w<W>(gr + dl1);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              if (dl0 < a.D) {
                acc[0][0] += cu[u] * v0[u].x;
                acc[0][1] += cu[u] * v0[u].y;
                acc[0][2] += cu[u] * v0[u].z;
                acc[0][3] += cu[u] * v0[u].w;
              }
              if (dl1 < a.D) {
                acc[1][0] += cu[u] * v1[u].x;
                acc[1][1] += cu[u] * v1[u].y;
                acc[1][2] += cu[u] * v1[u].z;
                acc[1][3] += cu[u] * v1[u].w;
              }
            }
          }
          if (first_pass) {
            float qa[4], qb2[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float* qr = a.q + rw[u] * a.ldq;
              qa[u] = lane < a.r ? qr[lane] : 0.f;
              qb2[u] = lane + kWave < a.r ? qr[lane + kWave] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              dk0 += gg[u] * qa[u];
              dk1 += gg[u] * qb2[u];
            }
          }
        }
      }
      if (a.grad_pv) {
        float* out = a.grad_pv + colg * a.ld_gpv;
        if (VEC) {
          if (dl0 < a.D) {
            float4 v = make_float4(acc[0][0], acc[0][1], acc[0][2], acc[0][3]);
            float4* p = reinterpret_cast<float4*>(out + dl0);
            if (a.accumulate_gpv) { float4 o = *p; v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w; }
            *p = v;
          }
          if (dl1 < a.D) {
            float4 v = make_float4(acc[1][0], acc[1][1], acc[1][2], acc[1][3]);
            float4* p = reinterpret_cast<float4*>(out + dl1);
            if (a.accumulate_gpv) { float4 o = *p; v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w; }
            *p = v;
          }
        } else {
          if (dl0 < a.D) out[dl0] = acc[0][0] + (a.accumulate_gpv ? out[dl0] : 0.f);
          if (dl1 < a.D) out[dl1] = acc[1][0] + (a.accumulate_gpv ? out[dl1] : 0.f);
        }
      }
    }
    if (a.grad_ps) {
      st = wave_sum(st);
      if (lane == 0) a.grad_ps[colg] = st;
    }
    const float* kr = a.key + colg * a.ldk;
    if (lane < a.r) {
      a.dk[colg * a.lddk + lane] = dk0 * (a.kscale ? a.kscale[lane] : 1.f);
      pc0 += kr[lane] * dk0;
    }
    if (lane + kWave < a.r) {
      a.dk[colg * a.lddk + lane + kWave] = dk1 * (a.kscale ? a.kscale[lane + kWave] : 1.f);
      pc1 += kr[lane + kWave] * dk1;
    }
  }
  if (lane < a.r) a.part_c[gw * a.r + lane] = pc0;
  if (lane + kWave < a.r) a.part_c[gw * a.r + lane + kWave] = pc1;
}

int cols_backward_waves(int64_t total_cols, int cols_per_wave) {
  return (int)((total_cols + cols_per_wave - 1) / cols_per_wave);
}

int launch_cols_backward(const ColsBwdArgs& a, hipStream_t stream) {
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  if (total_cols == 0) return kOk;
  JN_REQUIRE(a.r >= 1 && a.r <= 128, kUnsupported, "rank must be in [1, 128]");
  const int waves = cols_backward_waves(total_cols, a.cols_per_wave);
  const int blocks = (waves + 3) / 4;
  const bool vec = (a.D % 4 == 0) && (a.ld_gpv % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.gdv) & 15) == 0) &&
                   (a.grad_pv == nullptr || (reinterpret_cast<uintptr_t>(a.grad_pv) & 15) == 0);
  JN_PROFILE("cols_backward_kernel", stream);
  if (vec) hipLaunchKernelGGL(cols_backward_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(cols_backward_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Final reduction of the small gradients (scale vector, bias); one workgroup,
// fixed order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void finalize_small_grads_kernel(const float* part_c, int nparts, int r,
                                                                   float* grad_c, int accumulate_c,
                                                                   const float* rowsum, int64_t nrows,
                                                                   float* grad_bias) {
  // block b < r sums column b of the [nparts, r] partials; block r sums the row sums
  __shared__ float red[256];
  const int b = blockIdx.x;
  float s = 0.f;
  if (b < r) {
    for (int w = threadIdx.x; w < nparts; w += blockDim.x) s += part_c[(int64_t)w * r + b];
  } else {
    for (int64_t i = threadIdx.x; i < nrows; i += blockDim.x) s += rowsum[i];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (b < r) {
      if (grad_c) grad_c[b] = accumulate_c ? grad_c[b] + red[0] : red[0];
    } else if (grad_bias) {
      grad_bias[0] = red[0];
    }
  }
}

int launch_finalize_small_grads(const float* part_c, int nparts, int r, float* grad_c, int accumulate_c,
                                const float* rowsum, int64_t nrows, float* grad_bias, hipStream_t stream) {
  JN_PROFILE("finalize_small_grads_kernel", stream);
  hipLaunchKernelGGL(finalize_small_grads_kernel, dim3(r + 1), dim3(256), 0, stream, part_c, nparts, r, grad_c,
                     accumulate_c, rowsum, nrows, grad_bias);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
