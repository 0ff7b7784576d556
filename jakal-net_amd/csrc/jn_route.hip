// Transition routing over an edge list (gfx950).
//
// SparseTransition with a low-rank pairwise route (transition.py:431-452,
// modules.py:415-441): every source row j of a batch element keeps k
// destinations (edge list idx/logit [B*Ns, k], from the top-k select) and
//   p[j, e]    = softmax over the row's edges of the logits (compress 0,
//                kernel_common.py:420-423) or sign(l) * softmax(|l|)
//                (compress 1, native_backend.py:2184-2188) or sign(l) *
//                entmax15(|l|) (compress 2, transition.py:70-75)
//   coef[j, e] = rho[j] * p[j, e]          rho = sender strength (softplus(state))
//   delta_state[k] = sum_{j->k} coef * ps[j],  delta_val[k] = sum_{j->k} coef * pv[j]
// The destination sums run as gathers over the edge list transposed by
// destination (the column kernel of jn_edges.hip), so no atomics are used.
//
//   route_coef_kernel          : coef per edge (one wavefront per source row)
//   route_rows_backward_kernel : per source row, with its edges' destination
//                                gradient rows gathered once:
//       g_c[e]   = gds[k] * ps[j] + <gdv[k], pv[j]>
//       grad pv[j] = sum_e coef[e] * gdv[k],  grad ps[j] = sum_e coef[e] * gds[k]
//       grad rho[j] = sum_e p[e] * g_c[e]
//       g_l[e]   = compress backward of rho * g_c, times 1/T
//       dQ[j, r] = qscale[r] * sum_e g_l[e] * key[k, r]
//       rowsum[j] = sum_e g_l[e]   (bias gradient partial; per head with
//                   multi-head logits, whose dQ reaches each edge's head only)
#include "jn_internal.hpp"

namespace jakal {

// Route probability of edge `lane` of a source row (signed for compress 1) and
// the sign of its logit.  Lanes >= k, and absent edges, get p = 0.
__device__ __forceinline__ float route_probability(int j, float s, int compress) {
  if (compress == 2) return sign_f(s) * entmax15_lane(fabsf(s), j >= 0);
  const float a = compress == 0 ? s : fabsf(s);
  float m = j >= 0 ? a : -INFINITY;
  m = __int_as_float(wave_reduce_i(__float_as_int(m), [](int x, int y) {
    return __float_as_int(fmaxf(__int_as_float(x), __int_as_float(y)));
  }));
  const float ex = j >= 0 ? __expf(a - m) : 0.0f;
  const float sum = wave_sum(ex);
  const float p = sum > 0.0f ? ex / sum : 0.0f;
  return compress == 0 ? p : (s > 0.f ? p : (s < 0.f ? -p : 0.f));
}

__global__ __launch_bounds__(256) void route_coef_kernel(const int32_t* idx, const float* logit, const float* rho,
                                                         int k, int compress, int64_t rows, float* coef) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  int j = -1;
  float s = 0.0f;
  if (lane < k) {
    j = idx[row * k + lane];
    if (j >= 0) s = logit[row * k + lane];
  }
  const float p = route_probability(j, s, compress);
  if (lane < k) coef[row * k + lane] = rho ? rho[row] * p : p;
}

// ---- routes of more than 64 edges per source (up to kSelectLargeMaxK) -----
// The rows run one wavefront each with loops over 64-edge blocks: the row's
// statistics first, then the edges.
// Statistics of a route row of any length: kind 0 a = max l, b = 1 / sum
// exp(l - a); kinds 1 and 2 those of the signed edge compressions
// (row_compress_stats: signed |l| softmax, signed entmax-1.5 of |l|).
__device__ __forceinline__ RowStats route_row_stats(const int32_t* idx, const float* logit, int64_t row, int k,
                                                    int kind) {
  if (kind != 0) return row_compress_stats(idx, logit, row, k, kind);
  const int lane = lane_id();
  float m = -INFINITY;
  // (a route's logit loads beside its index: the slot exists for absent routes too)
  for (int e = lane; e < k; e += kWave) {
    const int32_t j = idx[row * k + e];
    const float l = logit[row * k + e];
    if (j >= 0) m = fmaxf(m, l);
  }
  m = wave_max_f(m);
  float sum = 0.0f;
  for (int e = lane; e < k; e += kWave) {
    const int32_t j = idx[row * k + e];
    const float l = logit[row * k + e];
    if (j >= 0) sum += __expf(l - m);
  }
  sum = wave_sum(sum);
  RowStats st;
  st.a = m;
  st.b = sum > 0.0f ? 1.0f / sum : 0.0f;
  return st;
}

// Route probability of an edge (signed for kinds 1 and 2) from its row's
// statistics; 0 for an absent edge.
__device__ __forceinline__ float route_prob_row(int j, float l, int kind, const RowStats& st) {
  if (j < 0) return 0.0f;
  if (kind == 0) return __expf(l - st.a) * st.b;
  if (kind == 1) return sign_f(l) * __expf(fabsf(l) - st.a) * st.b;
  const float d = fmaxf(0.5f * (fabsf(l) - st.a) - st.b, 0.0f);
  return st.c > 0.0f ? sign_f(l) * (d * d / st.c) : 0.0f;
}

__global__ __launch_bounds__(256) void route_coef_large_kernel(const int32_t* idx, const float* logit,
                                                               const float* rho, int k, int kind, int64_t rows,
                                                               float* coef) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const RowStats st = route_row_stats(idx, logit, row, k, kind);
  const float rh = rho ? rho[row] : 1.0f;
  for (int e = lane; e < k; e += kWave) {
    const int j = idx[row * k + e];
    const float l = logit[row * k + e];
    coef[row * k + e] = rh * route_prob_row(j, j >= 0 ? l : 0.0f, kind, st);
  }
}

int launch_route_coef(const int32_t* idx, const float* logit, const float* rho, int k, int compress, int64_t rows,
                      float* coef, hipStream_t stream) {
  JN_REQUIRE(k >= 1 && k <= kSelectLargeMaxK, kUnsupported, "routes support 1..%d edges per source (got %d)",
             kSelectLargeMaxK, k);
  if (rows == 0) return kOk;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  JN_PROFILE(k > kWave ? "route_coef_large_kernel" : "route_coef_kernel", stream);
  if (k > kWave)
    hipLaunchKernelGGL(route_coef_large_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, idx, logit, rho, k,
                       compress, rows, coef);
  else
    hipLaunchKernelGGL(route_coef_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, idx, logit, rho, k, compress,
                       rows, coef);
  JN_LAUNCH_CHECK();
  return kOk;
}

// One wavefront per source row; its four 16-lane groups take four edges at a
// time (group g takes edges 4i + g) and read whole destination gradient rows
// with 16-byte buffer loads.
// MH: multi-head logits (a.heads > 1): edge e's gradient reaches only the ranks
// of its head a.ehead[e] in dq, and the bias partials are per head.
// T: element type of the value rows (pv, gdv) and of grad_pv.
template <typename T, int W, int NV, int KP, bool MH>
__global__ __launch_bounds__(256) void route_rows_backward_kernel(RouteRowsBwdArgs a) {
  constexpr int NI = KP / 4;
  constexpr int P = 16 * W * NV;
  constexpr uint32_t EB = sizeof(T);
  const int lane = lane_id();
  const int g = lane >> 4, c = lane & 15;
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Ns;
  // 32-bit offsets into buffers of this batch element (sizes checked on the host)
  const auto rs_gdv = make_rsrc(reinterpret_cast<const T*>(a.gdv) + b * a.Nd * a.D, (uint32_t)(a.Nd * a.D * EB));
  const auto rs_key = make_rsrc(a.key + b * a.Nd * a.ldk, (uint32_t)(a.Nd * a.ldk * 4));
  const auto rs_pv = make_rsrc(reinterpret_cast<const T*>(a.pv) + row * a.ld_pv, (uint32_t)(a.D * EB));
  const float* gdsb = a.gds + b * a.Nd;
  const float ps_row = a.ps[row];
  const float rho = a.rho[row];
  const bool kvec = (a.r % 4 == 0) && (a.ldk % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0) &&
                    (!MH || a.head_rank % 4 == 0);

  int j = -1;
  float s = 0.0f;
  int eh = 0;
  if (lane < a.k) {
    j = a.idx[row * a.k + lane];
    if (j >= 0) s = a.logit[row * a.k + lane];
    if (MH && j >= 0) eh = a.ehead[row * a.k + lane];
  }
  const float p = route_probability(j, s, a.compress);
  const float cf = rho * p;
  int jg[NI];
  float cg[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    jg[i] = __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, j);
    cg[i] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * i + g) << 2, __float_as_int(cf)));
  }

  float dots[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) dots[i] = 0.f;
  for (int d0 = 0; d0 < a.D; d0 += P) {
    uint32_t loff[NV];
    Pack<W> pvv[NV], acc[NV];
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      const int off = d0 + (16 * t + c) * W;
      loff[t] = off < a.D ? (uint32_t)off * EB : kOobOffset;
      pvv[t] = buf_load_pack<T, W>(rs_pv, loff[t]);
      acc[t] = pack_zero<T, W>();
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      // absent edges and lanes past D read out of range: zeros, no traffic
      const uint32_t roff = jg[i] >= 0 ? (uint32_t)jg[i] * (uint32_t)a.D * EB : kOobOffset;
      Pack<W> v[NV];
#pragma unroll
      for (int t = 0; t < NV; ++t)
        v[t] = buf_load_pack<T, W>(rs_gdv, (loff[t] == kOobOffset || roff == kOobOffset) ? kOobOffset : roff + loff[t]);
      float pdot = 0.f;
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        pdot += dot_pack(pvv[t], v[t]);
        fma_pack(acc[t], cg[i], v[t]);
      }
      dots[i] += pdot;
      if (((i + 1) * NV) % 16 == 0) __builtin_amdgcn_sched_barrier(0);
    }
    if (a.grad_pv) {
      // sum the four groups' partial rows; group g stores slices t = g, g + 4
      T* out = reinterpret_cast<T*>(a.grad_pv) + row * a.ld_gpv;
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        Pack<W> x = acc[t];
#pragma unroll
        for (int u = 0; u < W; ++u) {
          x.v[u] += xor16_f(x.v[u]);
          x.v[u] += xor32_f(x.v[u]);
        }
        const int off = d0 + (16 * t + c) * W;
        if ((t & 3) == g && off < a.D) store_pack<T, W>(out + off, x);
      }
    }
  }
  float sel = 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float tot = row16_sum(dots[i]);
    sel = (c == i) ? tot : sel;
  }
  const float dot = __int_as_float(__builtin_amdgcn_ds_bpermute(edge_owner_lane(lane) << 2, __float_as_int(sel)));
  const float gd = j >= 0 ? gdsb[j] : 0.f;
  const float gc = j >= 0 ? gd * ps_row + dot : 0.f;
  const float gps = wave_sum(cf * gd);
  const float grho = wave_sum(p * gc);
  const float gp = rho * gc;
  float gl;
  if (a.compress == 0) {
    const float pg = wave_sum(p * gp);
    gl = p * (gp - pg);
  } else if (a.compress == 2) {
    gl = signed_entmax15_backward_lane(s, p, gp);
  } else {
    const float pg = wave_sum(gp * p);
    const float sg = sign_f(s);
    gl = sg * (sg * p) * (sg * gp - pg);
  }
  gl = j >= 0 ? gl * a.inv_temperature : 0.f;
  if (lane < a.k) a.g_logit[row * a.k + lane] = gl;
  if constexpr (MH) {
    // per-head bias partials (a shift of one head's logits is no shift of the row)
    for (int h = 0; h < a.heads; ++h) {  // uniform
      const float t = wave_sum(eh == h ? gl : 0.f);
      if (lane == 0) a.rowsum[row * a.heads + h] = t;
    }
  } else {
    // one-sign rows of the signed compressions: exactly 0 (softmax rows are not summed at all)
    const float gsum = (a.compress != 0 && row_one_sign(j >= 0, s)) ? 0.f : wave_sum(gl);
    if (lane == 0) a.rowsum[row] = gsum;
  }
  if (lane == 0) {
    if (a.grad_ps) a.grad_ps[row] = gps;
    if (a.grad_rho) a.grad_rho[row] = grho;
  }

  // dQ partials: group g sums its edges (absent edges read zeros)
  float4 dqa = make_float4(0.f, 0.f, 0.f, 0.f), dqb = dqa;
  float dqs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // MH: head of each rank slot of this lane (kvec: slots 4c and 64 + 4c; scalar: c + 16m)
  int hslot[8];
  if constexpr (MH) {
#pragma unroll
    for (int m = 0; m < 8; ++m) hslot[m] = (kvec ? (m == 0 ? 4 * c : 64 + 4 * c) : c + 16 * m) / a.head_rank;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const float gg = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * i + g) << 2, __float_as_int(gl)));
    const uint32_t koff = jg[i] >= 0 ? (uint32_t)jg[i] * (uint32_t)a.ldk * 4u : kOobOffset;
    const int hgi = MH ? __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, eh) : 0;
    // MH: slots of other heads read out of range (zeros)
    auto mine = [&](int m) { return !MH || hslot[m] == hgi; };
    if (kvec) {
      fma4(dqa, gg, buf_load4(rs_key, (4 * c < a.r && mine(0)) ? koff + 16u * c : kOobOffset));
      if (a.r > 64)
        fma4(dqb, gg, buf_load4(rs_key, (64 + 4 * c < a.r && mine(1)) ? koff + 256u + 16u * c : kOobOffset));
    } else {
#pragma unroll
      for (int m = 0; m < 8; ++m)
        if (16 * m < a.r)
          dqs[m] += gg * buf_load1(rs_key, (c + 16 * m < a.r && mine(m)) ? koff + 4u * (c + 16 * m) : kOobOffset);
    }
    if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);
  }
  float* dqrow = a.dq + row * a.lddq;
  if (kvec) {
    float v[8] = {dqa.x, dqa.y, dqa.z, dqa.w, dqb.x, dqb.y, dqb.z, dqb.w};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[u] += xor16_f(v[u]);
      v[u] += xor32_f(v[u]);
    }
    float lo = v[0], hi = v[4];
#pragma unroll
    for (int u = 1; u < 4; ++u) {
      lo = (g == u) ? v[u] : lo;
      hi = (g == u) ? v[4 + u] : hi;
    }
    const int r0 = 4 * c + g, r1 = 64 + 4 * c + g;
    if (r0 < a.r) dqrow[r0] = lo * (a.qscale ? a.qscale[r0] : 1.f);
    if (r1 < a.r) dqrow[r1] = hi * (a.qscale ? a.qscale[r1] : 1.f);
  } else {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      dqs[m] += xor16_f(dqs[m]);
      dqs[m] += xor32_f(dqs[m]);
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int rr = c + 16 * m;
      if ((m & 3) == g && rr < a.r) dqrow[rr] = dqs[m] * (a.qscale ? a.qscale[rr] : 1.f);
    }
  }
}

template <typename T, int W, int NV, bool MH>
static void launch_route_bwd_kp(const RouteRowsBwdArgs& a, dim3 grid, hipStream_t stream) {
  if (a.k <= 8) hipLaunchKernelGGL((route_rows_backward_kernel<T, W, NV, 8, MH>), grid, dim3(256), 0, stream, a);
  else if (a.k <= 16)
    hipLaunchKernelGGL((route_rows_backward_kernel<T, W, NV, 16, MH>), grid, dim3(256), 0, stream, a);
  else if (a.k <= 32)
    hipLaunchKernelGGL((route_rows_backward_kernel<T, W, NV, 32, MH>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((route_rows_backward_kernel<T, W, NV, 64, MH>), grid, dim3(256), 0, stream, a);
}

// One 16-byte pack per lane and pass slice (W elements), NV slices per 16-lane group.
// The row backward of route_rows_backward_kernel for rows of more than 64
// edges.  Pass 1 (lane e of each 64-edge block): g_c = gds[j] ps + <gdv[j], pv>
// into g_logit, with the row sums the compress backward needs; the value
// gradient grad_pv = sum_e c_e gdv[j_e] (lanes over the columns); pass 2: the
// compress backward into g_logit, the bias partials and dQ (lanes over the
// ranks, the block's edges in turn).  T: element type of pv, gdv and grad_pv;
// W: elements per load of the dot products (16 bytes, or 1).
template <typename T, int W, bool MH>
__global__ __launch_bounds__(256) void route_rows_backward_large_kernel(RouteRowsBwdArgs a) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Ns;
  const int k = a.k;
  const int32_t* idxr = a.idx + row * k;
  const float* lgr = a.logit + row * k;
  float* glr = a.g_logit + row * k;  // g_c after pass 1, g_l after pass 2 (each lane its own slots)
  const T* gdvb = reinterpret_cast<const T*>(a.gdv) + b * a.Nd * a.D;
  const T* pvr = reinterpret_cast<const T*>(a.pv) + row * a.ld_pv;
  const float* gdsb = a.gds + b * a.Nd;
  const float ps_row = a.ps[row];
  const float rho = a.rho[row];
  const RowStats st = route_row_stats(a.idx, a.logit, row, k, a.compress);

  float gps = 0.f, grho = 0.f, pg = 0.f, us = 0.f, gis = 0.f;
  bool all_pos = true, all_neg = true;
  for (int e0 = 0; e0 < k; e0 += kWave) {
    const int e = e0 + lane;
    const int j = e < k ? idxr[e] : -1;
    const float l = j >= 0 ? lgr[e] : 0.f;
    const float p = route_prob_row(j, l, a.compress, st);
    float gc = 0.f;
    if (j >= 0) {
      const T* gv = gdvb + (int64_t)j * a.D;
      float dot = 0.f;
      for (int d = 0; d < a.D; d += W) {
        const Pack<W> x = load_pack<T, W>(pvr + d), y = load_pack<T, W>(gv + d);
#pragma unroll
        for (int u = 0; u < W; ++u) dot += x.v[u] * y.v[u];
      }
      const float gd = gdsb[j];
      gc = gd * ps_row + dot;
      gps += rho * p * gd;
    }
    if (e < k) glr[e] = gc;
    grho += p * gc;
    const float gp = rho * gc;
    if (a.compress == 2) {
      const float u = sqrtf(fabsf(p));
      us += u;
      gis += gp * sign_f(l) * u;
    } else {
      pg += p * gp;
    }
    const uint64_t live = __ballot(j >= 0);
    all_pos = all_pos && __ballot(j >= 0 && l > 0.f) == live;
    all_neg = all_neg && __ballot(j >= 0 && l < 0.f) == live;
  }
  gps = wave_sum(gps);
  grho = wave_sum(grho);
  pg = wave_sum(pg);
  us = wave_sum(us);
  gis = wave_sum(gis);
  const float corr = us > 0.f ? gis / us : 0.f;

  if (a.grad_pv) {  // lanes over the columns, the row's edges in turn
    T* out = reinterpret_cast<T*>(a.grad_pv) + row * a.ld_gpv;
    for (int d = lane; d < a.D; d += kWave) {
      float acc = 0.f;
      for (int e = 0; e < k; ++e) {
        const int j = idxr[e];
        if (j < 0) continue;
        acc += rho * route_prob_row(j, lgr[e], a.compress, st) * (float)gdvb[(int64_t)j * a.D + d];
      }
      out[d] = (T)acc;
    }
  }

  const float* keyb = a.key + b * a.Nd * a.ldk;
  float dq0 = 0.f, dq1 = 0.f, gsum = 0.f;
  float hs[kMaxHeads];
#pragma unroll
  for (int h = 0; h < kMaxHeads; ++h) hs[h] = 0.f;
  const int h0 = MH ? lane / a.head_rank : 0, h1 = MH ? (lane + kWave) / a.head_rank : 0;
  for (int e0 = 0; e0 < k; e0 += kWave) {
    const int e = e0 + lane;
    const int j = e < k ? idxr[e] : -1;
    const float l = j >= 0 ? lgr[e] : 0.f;
    const float p = route_prob_row(j, l, a.compress, st);
    const float gp = rho * (e < k ? glr[e] : 0.f);
    const float sg = sign_f(l);
    float gl;
    if (a.compress == 0) {
      gl = p * (gp - pg);
    } else if (a.compress == 2) {
      const float u = sqrtf(fabsf(p));
      gl = (gp * sg * u - corr * u) * sg;
    } else {
      gl = sg * (sg * p) * (sg * gp - pg);
    }
    gl = j >= 0 ? gl * a.inv_temperature : 0.f;
    if (e < k) glr[e] = gl;
    const int eh = (MH && j >= 0) ? (int)a.ehead[row * k + e] : 0;
    if constexpr (MH) {
      for (int h = 0; h < a.heads; ++h) hs[h] += eh == h ? gl : 0.f;
    } else {
      gsum += gl;
    }
    const int ne = min(kWave, k - e0);
    for (int q = 0; q < ne; ++q) {
      const int jj = readlane_i(j, q);
      if (jj < 0) continue;
      const float gg = readlane_f(gl, q);
      const int hq = MH ? readlane_i(eh, q) : 0;
      const float* kr = keyb + (int64_t)jj * a.ldk;
      if (lane < a.r && (!MH || h0 == hq)) dq0 += gg * kr[lane];
      if (lane + kWave < a.r && (!MH || h1 == hq)) dq1 += gg * kr[lane + kWave];
    }
  }
  float* dqrow = a.dq + row * a.lddq;
  if (lane < a.r) dqrow[lane] = dq0 * (a.qscale ? a.qscale[lane] : 1.f);
  if (lane + kWave < a.r) dqrow[lane + kWave] = dq1 * (a.qscale ? a.qscale[lane + kWave] : 1.f);
  if constexpr (MH) {
    for (int h = 0; h < a.heads; ++h) {  // uniform
      const float t = wave_sum(hs[h]);
      if (lane == 0) a.rowsum[row * a.heads + h] = t;
    }
  } else {
    // one-sign rows of the signed compressions: exactly 0 (as the 64-edge kernel)
    const float t = (a.compress != 0 && (all_pos || all_neg)) ? 0.f : wave_sum(gsum);
    if (lane == 0) a.rowsum[row] = t;
  }
  if (lane == 0) {
    if (a.grad_ps) a.grad_ps[row] = gps;
    if (a.grad_rho) a.grad_rho[row] = grho;
  }
}

template <typename T, bool MH>
static void launch_route_bwd_large(const RouteRowsBwdArgs& a, bool vec, dim3 grid, hipStream_t stream) {
  constexpr int W = 16 / (int)sizeof(T);
  if (vec) hipLaunchKernelGGL((route_rows_backward_large_kernel<T, W, MH>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((route_rows_backward_large_kernel<T, 1, MH>), grid, dim3(256), 0, stream, a);
}

template <typename T, bool MH>
static void launch_route_bwd(const RouteRowsBwdArgs& a, bool vec, dim3 grid, hipStream_t stream) {
  constexpr int W = 16 / (int)sizeof(T);  // passes of 512, 256, 128 (or 64) elements
  if (!vec) launch_route_bwd_kp<T, 1, 4, MH>(a, grid, stream);
  else if (a.D > 256) launch_route_bwd_kp<T, W, 512 / (16 * W), MH>(a, grid, stream);
  else if (a.D > 128) launch_route_bwd_kp<T, W, 256 / (16 * W), MH>(a, grid, stream);
  else if (a.D > 64 || W == 8) launch_route_bwd_kp<T, W, 128 / (16 * W), MH>(a, grid, stream);
  else launch_route_bwd_kp<T, W, 1, MH>(a, grid, stream);
}

int launch_route_rows_backward(const RouteRowsBwdArgs& a, hipStream_t stream) {
  if (a.rows == 0) return kOk;
  if (a.r > kRegRank) {
    // ranks beyond the kernels' rank slots: the row kernel writes the logit
    // gradients only (rank 0: no dQ loads or stores), then the rank-chunked
    // kernel forms dQ from them
    JN_REQUIRE(a.r <= kMaxRank && a.heads <= 1, kUnsupported,
               "rank must be at most %d (%d over several heads), got %d", kMaxRank, kRegRank, a.r);
    JN_REQUIRE(a.g_logit && a.dq, kInvalidArgument, "wide-rank route backward needs g_logit and dq");
    RouteRowsBwdArgs b = a;
    b.r = 0;
    int rc = launch_route_rows_backward(b, stream);
    if (rc) return rc;
    RankRowsArgs rr{};
    rr.idx = a.idx;
    rr.g = a.g_logit;
    rr.k = a.k;
    rr.key = a.key;
    rr.ldk = a.ldk;
    rr.qscale = a.qscale;
    rr.r = a.r;
    rr.Nq = a.Ns;
    rr.Nk = a.Nd;
    rr.rows = a.rows;
    rr.dq = a.dq;
    rr.lddq = a.lddq;
    return launch_rank_rows_grad(rr, stream);
  }
  JN_REQUIRE(a.r >= 0 && a.r <= kRegRank, kUnsupported, "rank must be in [1, %d]", kRegRank);
  JN_REQUIRE(a.k >= 1 && a.k <= kSelectLargeMaxK, kUnsupported, "routes support 1..%d edges per source (got %d)",
             kSelectLargeMaxK, a.k);
  JN_REQUIRE(a.compress >= 0 && a.compress <= 2, kUnsupported, "route compress kind must be 0, 1 or 2");
  const int64_t blocks = (a.rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  JN_REQUIRE((int64_t)a.Nd * a.D * 4 < (1LL << 31) && (int64_t)a.Nd * a.ldk * 4 < (1LL << 31), kUnsupported,
             "one batch element of the destination rows must stay below 2 GiB");
  const int pw = a.bf16 ? 8 : 4;  // one 16-byte pack: 4 fp32 or 8 bf16 elements
  const bool vec = (a.D % pw == 0) && (a.ld_pv % pw == 0) && ((reinterpret_cast<uintptr_t>(a.pv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.gdv) & 15) == 0) &&
                   (a.grad_pv == nullptr ||
                    ((a.ld_gpv % pw == 0) && (reinterpret_cast<uintptr_t>(a.grad_pv) & 15) == 0));
  dim3 grid((unsigned)blocks);
  const bool mh = a.heads > 1;
  JN_REQUIRE(!mh || (a.ehead && a.heads <= kMaxHeads && a.head_rank >= 1 && a.heads * a.head_rank == a.r),
             kInvalidArgument, "multi-head route backward needs edge heads and 2..%d heads of equal rank", kMaxHeads);
  if (a.k > kWave) {
    JN_PROFILE("route_rows_backward_large_kernel", stream);
    if (a.bf16) {
      if (mh) launch_route_bwd_large<bf16_t, true>(a, vec, grid, stream);
      else launch_route_bwd_large<bf16_t, false>(a, vec, grid, stream);
    } else {
      if (mh) launch_route_bwd_large<float, true>(a, vec, grid, stream);
      else launch_route_bwd_large<float, false>(a, vec, grid, stream);
    }
    JN_LAUNCH_CHECK();
    return kOk;
  }
  JN_PROFILE("route_rows_backward_kernel", stream);
  if (a.bf16) {
    if (mh) launch_route_bwd<bf16_t, true>(a, vec, grid, stream);
    else launch_route_bwd<bf16_t, false>(a, vec, grid, stream);
  } else {
    if (mh) launch_route_bwd<float, true>(a, vec, grid, stream);
    else launch_route_bwd<float, false>(a, vec, grid, stream);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
