// Dense low-rank propagation over all N x N pairs (gfx950).
//
// Propagation with a LowRankBilinearPairwise score (propagation.py:207-220,
// jakal_net_native.cpp:5962-6076): every target row i aggregates every source
// j with e[i, j] = compress(s[i, j]),
//     s = P_t diag(w_hat) P_s^T + b,
//     compress = softsign (elementwise), sign(s) * softmax(|s|) or sign(s) * entmax15(|s|) over the row,
//     delta_state[i] = sum_j e[i,j] ps[j],   delta_val[i] = sum_j e[i,j] pv[j].
// Like the reference's full-dense branch, the edge matrix E [B, N, N] is
// materialised (in HBM, fp32): the two N x N contractions run as batched MFMA
// GEMMs (jn_gemm.hip) and the kernels here are the row-wise passes between
// them (one wavefront per row, float4 lanes over the row):
//   dense_compress_kernel          : E = compress(S + b) in place (optionally causal:
//                                    row i keeps sources j <= i), delta_state
//   dense_compress_backward_kernel : G_s = compress'(E, G + gds (x) ps) in place,
//                                    and its row sums (bias gradient)
//   dense_part_rowsum_kernel       : delta_state from the per-block partial sums
//                                    of the scores GEMM's softsign epilogue
// Softsign (elementwise) instead runs inside the two score GEMMs' epilogues
// (jn_gemm.hip), which saves the two in-place passes over the N x N matrix.
//   colsum_rows_kernel             : grad ps[j] = sum_i E[i, j] gds[i] (fixed order)
//   scale_grad_partials_kernel     : w_hat partials and scaling of dP_s
#include "jn_internal.hpp"

namespace jakal {

// Row r of a [rows, N] matrix: lane l covers floats 4l + 256t (VEC) or l + 64t.
// causal: row i keeps sources j <= i only (the rest are written as 0 and not
// read; a full causal window, kernel_common.py:443-456 with window >= N - 1).
template <bool VEC>
__global__ __launch_bounds__(256) void dense_compress_kernel(float* S, const float* bias, const float* ps, int N,
                                                             int64_t rows, int compress, int causal,
                                                             float* delta_state) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const int64_t b = row / N;
  const int lim = causal ? (int)(row - b * N) + 1 : N;  // sources [0, lim)
  float* s = S + row * N;
  const float* psb = ps + b * N;
  const float bb = bias ? bias[0] : 0.0f;
  float acc = 0.0f;
  if (compress == 0) {
    if constexpr (VEC) {
      for (int j = 4 * lane; j < N; j += 256) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < lim) {
          const float4 x = *reinterpret_cast<float4*>(s + j);
          const float4 p = *reinterpret_cast<const float4*>(psb + j);
          v.x = softsign_f(x.x + bb);
          v.y = j + 1 < lim ? softsign_f(x.y + bb) : 0.f;
          v.z = j + 2 < lim ? softsign_f(x.z + bb) : 0.f;
          v.w = j + 3 < lim ? softsign_f(x.w + bb) : 0.f;
          acc += v.x * p.x + v.y * p.y + v.z * p.z + v.w * p.w;
        }
        *reinterpret_cast<float4*>(s + j) = v;
      }
    } else {
      for (int j = lane; j < N; j += kWave) {
        const float e = j < lim ? softsign_f(s[j] + bb) : 0.f;
        if (j < lim) acc += e * psb[j];
        s[j] = e;
      }
    }
  } else if (compress == 2) {
    // sign(s) * entmax15(|s|) over the row's sources
    float zmax;
    auto zf = [&](int j) { return fabsf(s[j] + bb); };
    const float tau = entmax15_row_tau(zf, lim, zmax);
    float den = 0.0f;
    for (int j = lane; j < lim; j += kWave) {
      const float d = fmaxf(0.5f * (zf(j) - zmax) - tau, 0.0f);
      den += d * d;
    }
    den = wave_sum(den);
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    for (int j = lane; j < N; j += kWave) {
      float e = 0.f;
      if (j < lim) {
        const float x = s[j] + bb;
        const float d = fmaxf(0.5f * (fabsf(x) - zmax) - tau, 0.0f);
        e = sign_f(x) * (d * d) * inv;
        acc += e * psb[j];
      }
      s[j] = e;
    }
  } else {
    // sign(s) * softmax(|s|) over the row's sources: max, sum of exponentials, then write
    float m = -INFINITY;
    for (int j = lane; j < lim; j += kWave) m = fmaxf(m, fabsf(s[j] + bb));
    m = wave_max_f(m);
    float sum = 0.0f;
    for (int j = lane; j < lim; j += kWave) sum += __expf(fabsf(s[j] + bb) - m);
    const float inv = 1.0f / wave_sum(sum);
    for (int j = lane; j < N; j += kWave) {
      float e = 0.f;
      if (j < lim) {
        const float x = s[j] + bb;
        e = sign_f(x) * __expf(fabsf(x) - m) * inv;
        acc += e * psb[j];
      }
      s[j] = e;
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) delta_state[row] = acc;
}

// G holds gdv . pv^T on entry; on exit the score gradient
//   g_e = G + gds[i] ps[j]; softsign: g_s = g_e (1 - |e|)^2 (= g_e / (1 + |s|)^2);
//   signed |s| softmax: g_s = |e| g_e - e sum_j(g_e e);
//   signed entmax-1.5 (u = sqrt|e|): g_s = sign(e) (sign(e) g_e u - u sum_j(sign(e) g_e u) / sum_j u);
// and 0 for the sources a causal row does not keep (not read).
template <bool VEC>
__global__ __launch_bounds__(256) void dense_compress_backward_kernel(float* G, const float* E, const float* gds,
                                                                      const float* ps, int N, int64_t rows,
                                                                      int compress, int causal, float* rowsum) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const int64_t b = row / N;
  const int lim = causal ? (int)(row - b * N) + 1 : N;
  float* g = G + row * N;
  const float* e = E + row * N;
  const float* psb = ps + b * N;
  const float gs = gds[row];
  float row_dot = 0.0f;
  if (compress == 1) {
    for (int j = lane; j < lim; j += kWave) row_dot += (g[j] + gs * psb[j]) * e[j];
    row_dot = wave_sum(row_dot);
  } else if (compress == 2) {
    // entmax-1.5 backward: u = sqrt(|e|), gi = sign(e) g_e u (sign(e) = sign(s) where u > 0);
    // row_dot = sum(gi) / sum(u)
    float gis = 0.0f, us = 0.0f;
    for (int j = lane; j < lim; j += kWave) {
      const float u = sqrtf(fabsf(e[j]));
      gis += (g[j] + gs * psb[j]) * sign_f(e[j]) * u;
      us += u;
    }
    us = wave_sum(us);
    row_dot = us > 0.0f ? wave_sum(gis) / us : 0.0f;
  }
  float acc = 0.0f;
  if (VEC && compress == 0) {
    for (int j = 4 * lane; j < N; j += 256) {
      float4 gv = make_float4(0.f, 0.f, 0.f, 0.f);
      if (j < lim) {
        gv = *reinterpret_cast<float4*>(g + j);
        const float4 ev = *reinterpret_cast<const float4*>(e + j);
        const float4 pv = *reinterpret_cast<const float4*>(psb + j);
        const float d0 = 1.0f - fabsf(ev.x), d1 = 1.0f - fabsf(ev.y), d2 = 1.0f - fabsf(ev.z),
                    d3 = 1.0f - fabsf(ev.w);
        gv.x = (gv.x + gs * pv.x) * d0 * d0;
        gv.y = j + 1 < lim ? (gv.y + gs * pv.y) * d1 * d1 : 0.f;
        gv.z = j + 2 < lim ? (gv.z + gs * pv.z) * d2 * d2 : 0.f;
        gv.w = j + 3 < lim ? (gv.w + gs * pv.w) * d3 * d3 : 0.f;
        acc += gv.x + gv.y + gv.z + gv.w;
      }
      *reinterpret_cast<float4*>(g + j) = gv;
    }
  } else {
    for (int j = lane; j < N; j += kWave) {
      float gsj = 0.f;
      if (j < lim) {
        const float ge = g[j] + gs * psb[j];
        const float ej = e[j];
        if (compress == 0) {
          const float d = 1.0f - fabsf(ej);
          gsj = ge * d * d;
        } else if (compress == 2) {
          const float sg = sign_f(ej), u = sqrtf(fabsf(ej));
          gsj = (ge * sg * u - row_dot * u) * sg;
        } else {
          gsj = fabsf(ej) * ge - ej * row_dot;
        }
      }
      acc += gsj;
      g[j] = gsj;
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) rowsum[row] = acc;
}

// out[b, j] = sum_i M[b, i, j] * a[b, i] (* c[b, i]) over the Nr rows i in a
// fixed order.  A workgroup of 16 waves owns a tile of 256 columns (VEC: four
// per lane, float4 loads) or 64 (one per lane); wave w sums rows i = w, w + 16,
// ... four at a time, and the 16 partials are added in wave order.
template <bool VEC>
__global__ __launch_bounds__(1024) void colsum_rows_kernel(const float* M, const float* a, const float* c, int B,
                                                           int Nr, int Nc, float* out) {
  constexpr int CT = VEC ? 256 : 64;
  constexpr int W = VEC ? 4 : 1;
  __shared__ float red[16][CT];
  const int lane = lane_id(), wave = wave_id();
  const int tiles = (Nc + CT - 1) / CT;
  const int b = blockIdx.x / tiles;
  const int j = (blockIdx.x % tiles) * CT + W * lane;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (b < B && j < Nc) {
    const float* mb = M + (int64_t)b * Nr * Nc + j;
    const float* ab = a + (int64_t)b * Nr;
    const float* cb = c ? c + (int64_t)b * Nr : nullptr;
    auto wt = [&](int i) { return cb ? ab[i] * cb[i] : ab[i]; };
    int i = wave;
    for (; i + 48 < Nr; i += 64) {
      float4 v[4];
      float f[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u] = load_w<W>(mb + (int64_t)(i + 16 * u) * Nc);
        f[u] = wt(i + 16 * u);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) fma4(s, f[u], v[u]);
    }
    for (; i < Nr; i += 16) fma4(s, wt(i), load_w<W>(mb + (int64_t)i * Nc));
  }
  if constexpr (VEC) {
    *reinterpret_cast<float4*>(&red[wave][4 * lane]) = s;
  } else {
    red[wave][lane] = s.x;
  }
  __syncthreads();
  // wave 0 adds the 16 partials of its columns in wave order
  if (wave == 0 && b < B && j < Nc) {
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      if constexpr (VEC) {
        t = add4(t, *reinterpret_cast<const float4*>(&red[w][4 * lane]));
      } else {
        t.x += red[w][lane];
      }
    }
    store_w<W>(out + (int64_t)b * Nc + j, t);
  }
}

int launch_colsum_rows(const float* M, const float* a, const float* c, int B, int Nr, int Nc, float* out,
                       const char* name, hipStream_t stream) {
  // 256-column tiles with float4 loads when they still give every CU a workgroup
  const bool vec = (Nc % 4 == 0) && ((reinterpret_cast<uintptr_t>(M) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) & 15) == 0) && (int64_t)B * ((Nc + 255) / 256) >= 256;
  const int ct = vec ? 256 : 64;
  const int64_t blocks = (int64_t)B * ((Nc + ct - 1) / ct);
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many columns");
  JN_PROFILE(name, stream);
  if (vec) hipLaunchKernelGGL(colsum_rows_kernel<true>, dim3((unsigned)blocks), dim3(1024), 0, stream, M, a, c, B, Nr,
                              Nc, out);
  else hipLaunchKernelGGL(colsum_rows_kernel<false>, dim3((unsigned)blocks), dim3(1024), 0, stream, M, a, c, B, Nr,
                          Nc, out);
  JN_LAUNCH_CHECK();
  return kOk;
}

// part[m, c] = dps[m, c] * ps[m, c] (w_hat gradient partials), then dps *= w_hat.
__global__ __launch_bounds__(256) void scale_grad_partials_kernel(float* dps, int64_t ld_dps, const float* src,
                                                                  int64_t ld_src, const float* w_hat, int r,
                                                                  int64_t rows, float* part) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * r) return;
  const int64_t m = t / r;
  const int c = (int)(t % r);
  const float g = dps[m * ld_dps + c];
  part[m * r + c] = g * src[m * ld_src + c];
  dps[m * ld_dps + c] = g * w_hat[c];
}

int launch_dense_compress(float* S, const float* bias, const float* ps, int B, int N, int compress, int causal,
                          float* delta_state, hipStream_t stream) {
  const int64_t rows = (int64_t)B * N;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  const bool vec = (N % 4 == 0) && ((reinterpret_cast<uintptr_t>(S) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(ps) & 15) == 0);
  JN_PROFILE("dense_compress_kernel", stream);
  if (vec) hipLaunchKernelGGL(dense_compress_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, S, bias, ps,
                              N, rows, compress, causal, delta_state);
  else hipLaunchKernelGGL(dense_compress_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, S, bias, ps,
                          N, rows, compress, causal, delta_state);
  JN_LAUNCH_CHECK();
  return kOk;
}

int launch_dense_compress_backward(float* G, const float* E, const float* gds, const float* ps, int B, int N,
                                   int compress, int causal, float* rowsum, hipStream_t stream) {
  const int64_t rows = (int64_t)B * N;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  const bool vec = (N % 4 == 0) && ((reinterpret_cast<uintptr_t>(G) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(E) & 15) == 0) && ((reinterpret_cast<uintptr_t>(ps) & 15) == 0);
  JN_PROFILE("dense_compress_backward_kernel", stream);
  if (vec) hipLaunchKernelGGL(dense_compress_backward_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, G,
                              E, gds, ps, N, rows, compress, causal, rowsum);
  else hipLaunchKernelGGL(dense_compress_backward_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, G, E,
                          gds, ps, N, rows, compress, causal, rowsum);
  JN_LAUNCH_CHECK();
  return kOk;
}

// out[row] = sum_t part[row, t], t < P, in a fixed order: one wave per row,
// lane l sums t = l, l + 64, ..., then the wave's butterfly.
__global__ __launch_bounds__(256) void dense_part_rowsum_kernel(const float* part, int P, int64_t rows, float* out) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const float* p = part + row * P;
  float s = 0.0f;
  for (int t = lane; t < P; t += kWave) s += p[t];
  s = wave_sum(s);
  if (lane == 0) out[row] = s;
}

int launch_dense_part_rowsum(const float* part, int P, int64_t rows, float* out, hipStream_t stream) {
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  JN_PROFILE("dense_part_rowsum_kernel", stream);
  hipLaunchKernelGGL(dense_part_rowsum_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, part, P, rows, out);
  JN_LAUNCH_CHECK();
  return kOk;
}

// rowsum[row, h] = sum_j G[row, j] over the columns j whose winning head
// head[row, j] is h (the bias gradients of max-aggregated multi-head scores),
// h < H, in a fixed order: one wave per row, lane l sums columns 4l + 256t
// (VEC) or l + 64t, then a butterfly per head.
template <bool VEC>
__global__ __launch_bounds__(256) void head_rowsum_kernel(const float* G, const uint8_t* head, int N, int64_t ld,
                                                          int64_t rows, int H, float* rowsum) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const float* g = G + row * ld;
  const uint8_t* hd = head + row * ld;
  float acc[kMaxHeads];
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) acc[h] = 0.0f;
  auto add = [&](float v, uint32_t h) {
#pragma unroll
    for (int t = 0; t < kMaxHeads; ++t) acc[t] += (uint32_t)t == h ? v : 0.0f;
  };
  if constexpr (VEC) {
    for (int j = 4 * lane; j < N; j += 256) {
      const float4 v = *reinterpret_cast<const float4*>(g + j);
      const uint32_t hb = *reinterpret_cast<const uint32_t*>(hd + j);
      add(v.x, hb & 0xFFu);
      add(v.y, (hb >> 8) & 0xFFu);
      add(v.z, (hb >> 16) & 0xFFu);
      add(v.w, hb >> 24);
    }
  } else {
    for (int j = lane; j < N; j += kWave) add(g[j], hd[j]);
  }
  for (int h = 0; h < H; ++h) {
    const float t = wave_sum(acc[h]);
    if (lane == 0) rowsum[row * H + h] = t;
  }
}

int launch_head_rowsum(const float* G, const uint8_t* head, int N, int64_t ld, int64_t rows, int H, float* rowsum,
                       hipStream_t stream) {
  JN_REQUIRE(H >= 1 && H <= kMaxHeads, kUnsupported, "1 to %d heads", kMaxHeads);
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  if (rows == 0) return kOk;
  const bool vec = (N % 4 == 0) && (ld % 4 == 0) && ((reinterpret_cast<uintptr_t>(G) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(head) & 3) == 0);
  JN_PROFILE("head_rowsum_kernel", stream);
  if (vec) hipLaunchKernelGGL(head_rowsum_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, G, head, N, ld,
                              rows, H, rowsum);
  else hipLaunchKernelGGL(head_rowsum_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, G, head, N, ld,
                          rows, H, rowsum);
  JN_LAUNCH_CHECK();
  return kOk;
}

int launch_dense_colsum(const float* E, const float* w, int B, int N, float* out, hipStream_t stream) {
  return launch_colsum_rows(E, w, nullptr, B, N, N, out, "dense_colsum_kernel", stream);
}

int launch_scale_grad_partials(float* dps, int64_t ld_dps, const float* src, int64_t ld_src, const float* w_hat,
                               int r, int64_t rows, float* part, hipStream_t stream) {
  const int64_t n = rows * r;
  if (n == 0) return kOk;
  JN_REQUIRE((n + 255) / 256 < (1LL << 31), kUnsupported, "too many rows");
  JN_PROFILE("scale_grad_partials_kernel", stream);
  hipLaunchKernelGGL(scale_grad_partials_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, dps,
                     ld_dps, src, ld_src, w_hat, r, rows, part);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
