// Dense pairwise transitions (gfx950): every source routes to every destination.
//
//   l[j, k]   = ((P_src[j] * w) . P_dst[k] + b) / T         LowRankBilinearRoute
//   R[j, :]   = compress(l[j, :])     softmax, sign(l) * softmax(|l|) or sign(l) * entmax15(|l|)
//                                     over destinations
//   dstate[k] = sum_j R[j, k] rho_j ps_j,   dval[k] = sum_j R[j, k] rho_j pv_j
//
// Reference: transition_pairwise_dense (native/jakal_net_native.cpp:6705-6914;
// full-dense branch 6745-6774 computes routes = compress_scores(logits) and
// bmm(routes^T, rho * projected)), Transition._compute_delta_reference
// (src/jakal_net/transition.py:238-255), signed_abs_softmax
// (src/jakal_net/transition.py:53-67).
//
// The score products are MFMA GEMMs (jn_gemm.hip); this file holds the
// row-wise kernels between them:
//   route_dense_compress_kernel          : R = compress((L + b) / T) in place, one wave per source row
//   (column sums out[k] = sum_j R[j, k] a_j c_j run on colsum_rows_kernel, jn_dense.hip)
//   route_dense_compress_backward_kernel : logit gradient in place, sender / state grads, row sums
#include <cfloat>

#include "jn_internal.hpp"

namespace jakal {

// One wave per row of a [rows, N] matrix; lane l covers floats 4l + 256t (VEC)
// or l + 64t.  Softmax statistics are reduced in a fixed order.
template <bool VEC>
__global__ __launch_bounds__(256) void route_dense_compress_kernel(float* L, const float* bias, float inv_temp, int N,
                                                                   int64_t rows, int kind) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  float* x = L + row * N;
  const float bb = bias ? bias[0] : 0.0f;
  const bool sgn = kind >= 1;
  // logit as the reference forms it, NaN -> 0 and +-inf -> +-FLT_MAX for the
  // signed variants (torch.nan_to_num)
  auto logit = [&](float s) {
    float v = (s + bb) * inv_temp;
    if (sgn) v = (v != v) ? 0.0f : fminf(fmaxf(v, -FLT_MAX), FLT_MAX);
    return v;
  };
  if (kind == 2) {
    // sign(l) * entmax15(|l|) over the row
    float zmax;
    auto zf = [&](int j) { return fabsf(logit(x[j])); };
    const float tau = entmax15_row_tau(zf, N, zmax);
    float den = 0.0f;
    for (int j = lane; j < N; j += kWave) {
      const float d = fmaxf(0.5f * (zf(j) - zmax) - tau, 0.0f);
      den += d * d;
    }
    den = wave_sum(den);
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    for (int j = lane; j < N; j += kWave) {
      const float a = logit(x[j]);
      const float d = fmaxf(0.5f * (fabsf(a) - zmax) - tau, 0.0f);
      x[j] = sign_f(a) * (d * d) * inv;
    }
    return;
  }
  float m = -INFINITY;
  if constexpr (VEC) {
    for (int j = 4 * lane; j < N; j += 256) {
      const float4 s = *reinterpret_cast<const float4*>(x + j);
      const float a0 = logit(s.x), a1 = logit(s.y), a2 = logit(s.z), a3 = logit(s.w);
      m = fmaxf(m, sgn ? fmaxf(fmaxf(fabsf(a0), fabsf(a1)), fmaxf(fabsf(a2), fabsf(a3)))
                       : fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
    }
  } else {
    for (int j = lane; j < N; j += kWave) {
      const float a = logit(x[j]);
      m = fmaxf(m, sgn ? fabsf(a) : a);
    }
  }
  m = wave_max_f(m);
  float sum = 0.0f;
  if constexpr (VEC) {
    for (int j = 4 * lane; j < N; j += 256) {
      const float4 s = *reinterpret_cast<const float4*>(x + j);
      const float a0 = logit(s.x), a1 = logit(s.y), a2 = logit(s.z), a3 = logit(s.w);
      sum += __expf((sgn ? fabsf(a0) : a0) - m) + __expf((sgn ? fabsf(a1) : a1) - m) +
             __expf((sgn ? fabsf(a2) : a2) - m) + __expf((sgn ? fabsf(a3) : a3) - m);
    }
  } else {
    for (int j = lane; j < N; j += kWave) {
      const float a = logit(x[j]);
      sum += __expf((sgn ? fabsf(a) : a) - m);
    }
  }
  sum = wave_sum(sum);
  auto route = [&](float s) {
    const float a = logit(s);
    const float p = __expf((sgn ? fabsf(a) : a) - m) / sum;
    return sgn ? sign_f(a) * p : p;
  };
  if constexpr (VEC) {
    for (int j = 4 * lane; j < N; j += 256) {
      float4 s = *reinterpret_cast<const float4*>(x + j);
      s.x = route(s.x);
      s.y = route(s.y);
      s.z = route(s.z);
      s.w = route(s.w);
      *reinterpret_cast<float4*>(x + j) = s;
    }
  } else {
    for (int j = lane; j < N; j += kWave) x[j] = route(x[j]);
  }
}

// Row j of source rows (batch element b):
//   h_k   = H[j, k] + ps_j gds[b, k]        gradient of the weighted route rho_j R[j, k] / rho_j
//   g_k   = rho_j h_k                       gradient of R[j, k]
//   grad rho_j = sum_k R[j, k] h_k,  grad ps_j = rho_j sum_k R[j, k] gds[b, k]
//   softmax:            g_l = R (g - sum R g)
//   sign * softmax(|l|): g_l = |R| g - R sum R g   (0 where l == 0, as R is)
//   sign * entmax15(|l|): with u = sqrt|R|, g_l = sign(R) (sign(R) g u - u sum(sign(R) g u) / sum u)
//   H[j, k] <- g_l / T (gradient of the raw bilinear logit); rowsum[j] = sum_k H[j, k]
template <bool VEC>
__global__ __launch_bounds__(256) void route_dense_compress_backward_kernel(
    float* H, const float* R, const float* rho, const float* ps, const float* gds, int Ns, int Nd, int64_t rows,
    int kind, float inv_temp, float* grad_rho, float* grad_ps, float* rowsum) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const int64_t b = row / Ns;
  float* h = H + row * Nd;
  const float* rr = R + row * Nd;
  const float* gb = gds + b * Nd;
  const float rj = rho[row], pj = ps[row];
  const bool sgn = kind == 1;
  float dot = 0.0f, srh = 0.0f, srg = 0.0f;
  if constexpr (VEC) {
    for (int k = 4 * lane; k < Nd; k += 256) {
      const float4 hv = *reinterpret_cast<const float4*>(h + k);
      const float4 rv = *reinterpret_cast<const float4*>(rr + k);
      const float4 gv = *reinterpret_cast<const float4*>(gb + k);
      const float h0 = hv.x + pj * gv.x, h1 = hv.y + pj * gv.y, h2 = hv.z + pj * gv.z, h3 = hv.w + pj * gv.w;
      srh += rv.x * h0 + rv.y * h1 + rv.z * h2 + rv.w * h3;
      srg += rv.x * gv.x + rv.y * gv.y + rv.z * gv.z + rv.w * gv.w;
    }
  } else {
    for (int k = lane; k < Nd; k += kWave) {
      const float hk = h[k] + pj * gb[k];
      srh += rr[k] * hk;
      srg += rr[k] * gb[k];
    }
  }
  srh = wave_sum(srh);
  srg = wave_sum(srg);
  dot = rj * srh;  // sum_k R g = rho_j sum_k R h
  if (kind == 2) {
    // entmax-1.5: u = sqrt(|R|), gi = sign(R) g u; dot <- sum(gi) / sum(u)
    float gis = 0.0f, us = 0.0f;
    for (int k = lane; k < Nd; k += kWave) {
      const float u = sqrtf(fabsf(rr[k]));
      gis += rj * (h[k] + pj * gb[k]) * sign_f(rr[k]) * u;
      us += u;
    }
    us = wave_sum(us);
    dot = us > 0.0f ? wave_sum(gis) / us : 0.0f;
  }
  auto grad = [&](float r, float hk) {
    const float g = rj * hk;
    if (kind == 2) {
      const float sg = sign_f(r), u = sqrtf(fabsf(r));
      return (g * sg * u - dot * u) * sg * inv_temp;
    }
    return ((sgn ? fabsf(r) : r) * g - r * dot) * inv_temp;
  };
  float rs = 0.0f;
  if constexpr (VEC) {
    for (int k = 4 * lane; k < Nd; k += 256) {
      float4 hv = *reinterpret_cast<const float4*>(h + k);
      const float4 rv = *reinterpret_cast<const float4*>(rr + k);
      const float4 gv = *reinterpret_cast<const float4*>(gb + k);
      hv.x = grad(rv.x, hv.x + pj * gv.x);
      hv.y = grad(rv.y, hv.y + pj * gv.y);
      hv.z = grad(rv.z, hv.z + pj * gv.z);
      hv.w = grad(rv.w, hv.w + pj * gv.w);
      rs += (hv.x + hv.y) + (hv.z + hv.w);
      *reinterpret_cast<float4*>(h + k) = hv;
    }
  } else {
    for (int k = lane; k < Nd; k += kWave) {
      const float v = grad(rr[k], h[k] + pj * gb[k]);
      rs += v;
      h[k] = v;
    }
  }
  rs = wave_sum(rs);
  if (lane == 0) {
    rowsum[row] = rs;
    if (grad_rho) grad_rho[row] = srh;
    if (grad_ps) grad_ps[row] = rj * srg;
  }
}

static bool rows_vec(int N, const void* p0, const void* p1 = nullptr, const void* p2 = nullptr) {
  auto al = [](const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return N % 4 == 0 && al(p0) && al(p1) && al(p2);
}

int launch_route_dense_compress(float* L, const float* bias, float inv_temp, int B, int Ns, int Nd, int kind,
                                hipStream_t stream) {
  const int64_t rows = (int64_t)B * Ns;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  JN_PROFILE("route_dense_compress_kernel", stream);
  if (rows_vec(Nd, L))
    hipLaunchKernelGGL(route_dense_compress_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, L, bias,
                       inv_temp, Nd, rows, kind);
  else
    hipLaunchKernelGGL(route_dense_compress_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, L, bias,
                       inv_temp, Nd, rows, kind);
  JN_LAUNCH_CHECK();
  return kOk;
}

int launch_route_dense_colsum(const float* R, const float* a, const float* c, int B, int Nr, int Nc, float* out,
                              hipStream_t stream) {
  return launch_colsum_rows(R, a, c, B, Nr, Nc, out, "route_dense_colsum_kernel", stream);
}

int launch_route_dense_compress_backward(float* H, const float* R, const float* rho, const float* ps,
                                         const float* gds, int B, int Ns, int Nd, int kind, float inv_temp,
                                         float* grad_rho, float* grad_ps, float* rowsum, hipStream_t stream) {
  const int64_t rows = (int64_t)B * Ns;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "too many rows");
  JN_PROFILE("route_dense_compress_backward_kernel", stream);
  if (rows_vec(Nd, H, R, gds))
    hipLaunchKernelGGL(route_dense_compress_backward_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, H,
                       R, rho, ps, gds, Ns, Nd, rows, kind, inv_temp, grad_rho, grad_ps, rowsum);
  else
    hipLaunchKernelGGL(route_dense_compress_backward_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       H, R, rho, ps, gds, Ns, Nd, rows, kind, inv_temp, grad_rho, grad_ps, rowsum);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
