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
// row's selected edges (propagation.py:74-82), 2 signed entmax-1.5 over them
// (kernels.py:221-237; native/jakal_net_native.cpp:1171-1205).
#include <algorithm>

#include "jn_internal.hpp"

namespace jakal {

// A 16-byte pack as its raw bits (stored as computed: fp32, or bf16 rounded).
template <typename T, int W>
__device__ __forceinline__ uint4 pack_bits(const Pack<W>& g) {
  static_assert(W * sizeof(T) == 16, "a 16-byte pack");
  if constexpr (sizeof(T) == 4) {
    return make_uint4(__float_as_uint(g.v[0]), __float_as_uint(g.v[1]), __float_as_uint(g.v[2]),
                      __float_as_uint(g.v[3]));
  } else {
    return make_uint4(pack_bf16x2(g.v[0], g.v[1]), pack_bf16x2(g.v[2], g.v[3]), pack_bf16x2(g.v[4], g.v[5]),
                      pack_bf16x2(g.v[6], g.v[7]));
  }
}

// ---------------------------------------------------------------------------
// Row forward: one wavefront per query row.
// ---------------------------------------------------------------------------

// The D columns are processed in slabs of a.slab columns, slab-major over the
// grid: while an XCD works on one slab of a batch element, the value rows it
// gathers (N x slab elements) stay within its L2.  Slab 0 also sums the state.
// T: element type of the value rows and of delta_val (float or bf16).
template <typename T, int W>
__global__ __launch_bounds__(256) void rows_forward_kernel(RowsFwdArgs a) {
  const int lane = lane_id();
  const int64_t row_blocks = (a.rows + 3) / 4;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int slab = (int)(logical / row_blocks);
  const int64_t row = (logical % row_blocks) * 4 + wave_id();
  if (row >= a.rows) return;
  const int d_begin = slab * a.slab, d_end = min(a.D, d_begin + a.slab);
  const int64_t b = row / a.Nq;
  const T* pvb = reinterpret_cast<const T*>(a.pv) + b * a.Nk * a.ld_pv;
  const float* psb = a.ps + b * a.Nk;
  T* out = reinterpret_cast<T*>(a.out_val) + row * a.D;

  const RowStats rst = row_compress_stats(a.idx, a.score, row, a.k, a.compress);

  float st = 0.0f;
  for (int e0 = 0; e0 < a.k; e0 += kWave) {
    int j;
    float c, s;
    row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rst, j, c, s);
    if (slab == 0 && j >= 0) st += c * psb[j];
    const int ne = min(kWave, a.k - e0);
    for (int d = d_begin + lane * W; d < d_end; d += kWave * W) {
      // two accumulation chains (even / odd edges), summed at the end
      Pack<W> acc = pack_zero<T, W>(), acc1 = acc;
      int q = 0;
      for (; q + 8 <= ne; q += 8) {
        Pack<W> v[8];
        float cc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int jj = readlane_i(j, q + u);
          cc[u] = jj < 0 ? 0.f : readlane_f(c, q + u);
          v[u] = load_pack<T, W>(pvb + (int64_t)(jj < 0 ? 0 : jj) * a.ld_pv + d);
        }
#pragma unroll
        for (int u = 0; u < 8; u += 2) {
          fma_pack(acc, cc[u], v[u]);
          fma_pack(acc1, cc[u + 1], v[u + 1]);
        }
      }
      for (; q < ne; ++q) {
        const int jj = readlane_i(j, q);
        if (jj < 0) continue;
        fma_pack((q & 1) ? acc1 : acc, readlane_f(c, q), load_pack<T, W>(pvb + (int64_t)jj * a.ld_pv + d));
      }
      acc = add_pack(acc, acc1);
      if (e0 > 0) acc = add_pack(acc, load_pack<T, W>(out + d));
      if constexpr (W * sizeof(T) == 16) {
        if (a.k <= kWave) store_nt16(out + d, pack_bits<T, W>(acc));  // the row's only pass: written once
        else store_pack<T, W>(out + d, acc);
      } else {
        store_pack<T, W>(out + d, acc);
      }
    }
  }
  if (slab == 0) {
    st = wave_sum(st);
    if (lane == 0) a.out_state[row] = st;
  }
}

int launch_rows_forward(const RowsFwdArgs& args, hipStream_t stream) {
  if (args.rows == 0) return kOk;
  RowsFwdArgs a = args;
  // one 16-byte pack per lane: 4 fp32 or 8 bf16 elements
  const int eb = a.bf16 ? 2 : 4, pw = 16 / eb;
  const bool vec = (a.D % pw == 0) && (a.ld_pv % pw == 0) && ((reinterpret_cast<uintptr_t>(a.pv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.out_val) & 15) == 0);
  // slabs of 64 packs while a batch element's value rows exceed 2 MiB; a
  // slab's rows then fit an XCD's 4 MiB L2
  a.slab = a.D;
  if (vec)
    while (a.slab > 64 * pw && a.slab % (128 * pw) == 0 && (int64_t)a.Nk * a.slab * eb > (2LL << 20)) a.slab /= 2;
  const int64_t slabs = (a.D + a.slab - 1) / a.slab;
  const int64_t blocks = (a.rows + 3) / 4 * slabs;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  JN_PROFILE("rows_forward_kernel", stream);
  const dim3 grid((unsigned)blocks);
  if (a.bf16) {
    if (vec) hipLaunchKernelGGL((rows_forward_kernel<bf16_t, 8>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((rows_forward_kernel<bf16_t, 1>), grid, dim3(256), 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((rows_forward_kernel<float, 4>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((rows_forward_kernel<float, 1>), grid, dim3(256), 0, stream, a);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Row backward: one wavefront per query row.
//   g_c[e]   = gds[i] * ps[j] + <gdv[i], pv[j]>        (grad wrt edge coefficient)
//   g_s[e]   = compress backward of g_c, times 1/T      (grad wrt score)
//   dQ[i, r] = qscale[r] * sum_e g_s[e] * key[j, r]      (grad wrt query projection)
//   coef[e]  = c(s_e)                                    (kept for the column pass)
//   rowsum_gs[i] = sum_e g_s[e]                          (bias gradient partial)
// The four 16-lane groups of the wave take four edges at a time (group g takes
// edges 4i + g): a group reads a whole value row with 16-byte loads, so each
// edge's dot product is reduced inside the group by DPP (4 VALU ops) and the
// key rows of the dQ sum are read 4 edges per instruction.
//
// When a batch element's value rows outgrow an XCD's L2, the dot products run
// first, in two column slabs (rows_backward_dots_kernel: slab 0 into g_score,
// slab 1 into coef), and this kernel (SPLIT) reads their sum back in place.
// ---------------------------------------------------------------------------

// Partial dot products <gdv[i], pv[j]> of every edge over one slab of the D
// columns: slab s of the grid writes into g_score (s = 0) or coef (s = 1).  The
// grid is slab-major, so an XCD gathers value rows of one slab of one batch
// element at a time (Nk x slab floats, sized to its L2).
template <typename T, int NV, int KP>
__global__ __launch_bounds__(256) void rows_backward_dots_kernel(RowsBwdArgs a, int slab) {
  constexpr int NI = KP / 4;
  constexpr int W = 16 / (int)sizeof(T);  // elements per 16-byte pack
  constexpr uint32_t EB = sizeof(T);
  const int lane = lane_id();
  const int g = lane >> 4, c = lane & 15;
  const int64_t row_blocks = (a.rows + 3) / 4;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int s = (int)(logical / row_blocks);
  const int64_t row = (logical % row_blocks) * 4 + wave_id();
  if (row >= a.rows) return;
  const int d_begin = s * slab, d_end = min(a.D, d_begin + slab);
  float* part = (s == 0) ? a.g_score : a.coef;
  const int64_t b = row / a.Nq;
  const auto rs_pv = make_rsrc(reinterpret_cast<const T*>(a.pv) + b * a.Nk * a.ld_pv, (uint32_t)(a.Nk * a.ld_pv * EB));
  const auto rs_g = make_rsrc(reinterpret_cast<const T*>(a.gdv) + row * a.D, (uint32_t)(a.D * EB));
  uint32_t loff[NV];  // byte offsets of this lane's columns; past the slab -> out of range (zeros)
  Pack<W> gv[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    const int off = d_begin + (16 * t + c) * W;
    loff[t] = off < d_end ? (uint32_t)off * EB : kOobOffset;
    gv[t] = buf_load_pack<T, W>(rs_g, loff[t]);
  }
  for (int e0 = 0; e0 < a.k; e0 += KP) {
    const int e = e0 + lane;
    const int j = (lane < KP && e < a.k) ? a.idx[row * a.k + e] : -1;
    const int ne = min(KP, a.k - e0);
    int jg[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) jg[i] = __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, j);
    float sel = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const uint32_t roff = jg[i] >= 0 ? (uint32_t)jg[i] * (uint32_t)a.ld_pv * EB : kOobOffset;
      Pack<W> v[NV];
#pragma unroll
      for (int t = 0; t < NV; ++t)
        v[t] = buf_load_pack<T, W>(rs_pv, (loff[t] == kOobOffset || roff == kOobOffset) ? kOobOffset : roff + loff[t]);
      float pdot = 0.f;
#pragma unroll
      for (int t = 0; t < NV; ++t) pdot += dot_pack(gv[t], v[t]);
      const float tot = row16_sum(pdot);
      sel = (c == i) ? tot : sel;
      if (((i + 1) * NV) % 16 == 0) __builtin_amdgcn_sched_barrier(0);
    }
    const float dot = __int_as_float(__builtin_amdgcn_ds_bpermute(edge_owner_lane(lane) << 2, __float_as_int(sel)));
    if (lane < ne) part[row * a.k + e] = dot;
  }
}

// MH: multi-head scores (a.heads > 1): edge e's gradient reaches only the
// ranks of its head a.ehead[e] in dq, and the bias partials are per head.
template <typename T, int W, int NV, int KP, bool SPLIT, bool MH>
__global__ __launch_bounds__(256) void rows_backward_kernel(RowsBwdArgs a) {
  constexpr int NI = KP / 4;      // iterations per block of KP edges
  constexpr int P = 16 * W * NV;  // D elements per pass of a 16-lane group
  constexpr uint32_t EB = sizeof(T);
  const int lane = lane_id();
  const int g = lane >> 4, c = lane & 15;
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Nq;
  const float* psb = a.ps + b * a.Nk;
  const float gs_row = a.gds[row];
  // 32-bit offsets into buffers of this batch element (sizes checked on the host)
  const auto rs_key = make_rsrc(a.key + b * a.Nk * a.ldk, (uint32_t)(a.Nk * a.ldk * 4));
  // key rows as float4 when 16-byte aligned (rank slots 4c and 64 + 4c; with
  // several heads a float4 must not straddle two of them)
  const bool kvec = (a.r % 4 == 0) && (a.ldk % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0) &&
                    (!MH || a.head_rank % 4 == 0);
  // MH: head of each rank slot of this lane (kvec: slots 4c and 64 + 4c; scalar: c + 16m)
  int hslot[8];
  if constexpr (MH) {
#pragma unroll
    for (int m = 0; m < 8; ++m) hslot[m] = (kvec ? (m == 0 ? 4 * c : 64 + 4 * c) : c + 16 * m) / a.head_rank;
  }

  const RowStats rst = row_compress_stats(a.idx, a.score, row, a.k, a.compress);

  // The coefficient gradient g_c of this lane's edge in the block at e0
  // (lanes < KP hold edges e0 + lane; jg: the block's edges as the 16-lane
  // groups take them).
  auto edge_gc = [&](int e0, int j, const int (&jg)[NI]) -> float {
    const int ne = min(KP, a.k - e0);
    float dot = 0.f;
    if constexpr (SPLIT) {
      // slab partials of this lane's edge, summed in slab order
      if (a.dot_pos) {  // record order: absent edges have no record
        if (lane < ne && j >= 0 && j < a.Nk) {
          const int p = a.dot_pos[row * a.k + e0 + lane];
          dot = a.dots0[p] + (a.dot_parts == 1 ? 0.f : a.coef[p]);
        }
      } else if (lane < ne) {
        dot = a.g_score[row * a.k + e0 + lane] + (a.dot_parts == 1 ? 0.f : a.coef[row * a.k + e0 + lane]);
      }
    } else {
      const auto rs_pv =
          make_rsrc(reinterpret_cast<const T*>(a.pv) + b * a.Nk * a.ld_pv, (uint32_t)(a.Nk * a.ld_pv * EB));
      const auto rs_g = make_rsrc(reinterpret_cast<const T*>(a.gdv) + row * a.D, (uint32_t)(a.D * EB));
      float dots[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) dots[i] = 0.f;
      for (int d0 = 0; d0 < a.D; d0 += P) {
        // byte offsets of this lane's slice of the pass; past D -> out of range (zeros)
        uint32_t loff[NV];
        Pack<W> gv[NV];
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const int off = d0 + (16 * t + c) * W;
          loff[t] = off < a.D ? (uint32_t)off * EB : kOobOffset;
          gv[t] = buf_load_pack<T, W>(rs_g, loff[t]);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          // absent edges, iterations past the block's last edge and lanes past D
          // read out of range: zeros and no memory traffic, without a branch
          const uint32_t roff = jg[i] >= 0 ? (uint32_t)jg[i] * (uint32_t)a.ld_pv * EB : kOobOffset;
          Pack<W> v[NV];
#pragma unroll
          for (int t = 0; t < NV; ++t)
            v[t] = buf_load_pack<T, W>(rs_pv,
                                       (loff[t] == kOobOffset || roff == kOobOffset) ? kOobOffset : roff + loff[t]);
          float pdot = 0.f;
#pragma unroll
          for (int t = 0; t < NV; ++t) pdot += dot_pack(gv[t], v[t]);
          dots[i] += jg[i] >= 0 ? pdot : 0.f;
          // at most 16 row loads in flight per lane: keeps VGPRs (and occupancy) in check
          if (((i + 1) * NV) % 16 == 0) __builtin_amdgcn_sched_barrier(0);
        }
      }
      float sel = 0.f;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float tot = row16_sum(dots[i]);
        sel = (c == i) ? tot : sel;
      }
      dot = __int_as_float(__builtin_amdgcn_ds_bpermute(edge_owner_lane(lane) << 2, __float_as_int(sel)));
    }
    return (j >= 0) ? gs_row * psb[j] + dot : 0.f;
  };

  // Row-normalising kinds over more than one block of edges: a first pass
  // stores every edge's g_c in g_score and forms the row sums their backward
  // needs (kind 1: sum g_c c; kind 2: sum sign(s) g_c u and sum u with
  // u = sqrt(|c|)) and whether all scores share one sign; the main pass reads
  // g_c back.  One block: the same sums come from the block itself.
  const bool two_pass = a.compress != 0 && a.k > KP;
  float row_s1 = 0.f, row_s2 = 0.f;
  bool row_shift_free = false;
  if (two_pass) {
    float npos = 0.f, nneg = 0.f, nall = 0.f;
    for (int e0 = 0; e0 < a.k; e0 += KP) {
      int j;
      float cf, s;
      row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rst, j, cf, s);
      if (lane >= KP) j = -1;
      int jg[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) jg[i] = __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, j);
      const float gc = edge_gc(e0, j, jg);
      if (j >= 0) {  // j >= 0: lane < KP and e0 + lane < k
        a.g_score[row * a.k + e0 + lane] = gc;
        const float sg = sign_f(s);
        if (a.compress == 1) {
          row_s1 += gc * cf;
        } else {
          const float u = sqrtf(fabsf(cf));
          row_s1 += gc * sg * u;
          row_s2 += u;
        }
        npos += s > 0.f ? 1.f : 0.f;
        nneg += s < 0.f ? 1.f : 0.f;
        nall += 1.f;
      }
    }
    row_s1 = wave_sum(row_s1);
    row_s2 = wave_sum(row_s2);
    npos = wave_sum(npos);
    nneg = wave_sum(nneg);
    nall = wave_sum(nall);
    row_shift_free = npos == nall || nneg == nall;
  }

  float4 dqa = make_float4(0.f, 0.f, 0.f, 0.f), dqb = dqa;  // kvec: ranks 4c.., 64+4c..
  float dqs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // scalar: ranks c + 16m
  float gsum = 0.f;
  float hsum[MH ? kMaxHeads : 1] = {};
  for (int e0 = 0; e0 < a.k; e0 += KP) {
    int j;
    float cf, s;
    // lanes < KP hold edges e0 + lane (j = -1 past k)
    row_coefficients(a.idx, a.score, row, a.k, e0, a.compress, rst, j, cf, s);
    if (lane >= KP) j = -1;
    const int ne = min(KP, a.k - e0);
    int jg[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) jg[i] = __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, j);
    int eh = 0, hg[MH ? NI : 1];
    if constexpr (MH) {
      if (j >= 0) eh = a.ehead[row * a.k + e0 + lane];  // j >= 0: lane < KP and e0 + lane < k
#pragma unroll
      for (int i = 0; i < NI; ++i) hg[i] = __builtin_amdgcn_ds_bpermute((4 * i + g) << 2, eh);
    }

    const float gc = two_pass ? (j >= 0 ? a.g_score[row * a.k + e0 + lane] : 0.f) : edge_gc(e0, j, jg);
    float gsc = 0.f;
    if (a.compress == 1) {
      const float row_dot = two_pass ? row_s1 : wave_sum(gc * cf);
      if (j >= 0) {
        const float sg = sign_f(s);
        gsc = sg * (sg * cf) * (sg * gc - row_dot);
      }
    } else if (a.compress == 2) {
      if (two_pass) {  // as signed_entmax15_backward_lane, with the row's sums
        const float sg = sign_f(s);
        const float u = sqrtf(fabsf(cf));
        const float corr = row_s2 > 0.0f ? row_s1 / row_s2 : 0.0f;
        gsc = j >= 0 ? (gc * sg * u - corr * u) * sg : 0.f;
      } else {
        gsc = signed_entmax15_backward_lane(s, cf, gc);  // absent edges: s = cf = gc = 0
      }
    } else if (j >= 0) {
      gsc = gc * softsign_grad_f(s);
    }
    gsc *= a.inv_temperature;
    if (lane < ne) {
      a.g_score[row * a.k + e0 + lane] = gsc;
      if (!(SPLIT && a.dot_pos)) a.coef[row * a.k + e0 + lane] = cf;  // coef holds other rows' partials
    }
    if constexpr (MH) {
      // per-head bias partials (a shift of one head's scores is no shift of the row)
#pragma unroll
      for (int h = 0; h < kMaxHeads; ++h) hsum[h] += (eh == h) ? gsc : 0.f;
    } else {
      // a row of one score sign has no bias gradient under kinds 1 and 2
      const bool shift_free = a.compress != 0 && (two_pass ? row_shift_free : row_one_sign(j >= 0, s));
      gsum += shift_free ? 0.f : gsc;
    }

    // dQ partials: group g sums its edges (absent edges carry gsc = 0)
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const float gg = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * i + g) << 2, __float_as_int(gsc)));
      // absent edges read out of range (zeros, no traffic)
      const uint32_t koff = jg[i] >= 0 ? (uint32_t)jg[i] * (uint32_t)a.ldk * 4u : kOobOffset;
      // MH: slots of other heads read out of range (zeros)
      auto mine = [&](int m) { return !MH || hslot[m] == hg[MH ? i : 0]; };
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
  }
  // sum the four groups; lane (g, c) then stores one rank per slot
  float* dqrow = a.dq + row * a.lddq;
  if (kvec) {
    float v[8] = {dqa.x, dqa.y, dqa.z, dqa.w, dqb.x, dqb.y, dqb.z, dqb.w};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      v[u] += xor16_f(v[u]);
      v[u] += xor32_f(v[u]);
    }
    // lane (g, c) stores component g of both slots: ranks 4c + g and 64 + 4c + g
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
    // lane (g, c) stores slots m = g and m = g + 4: ranks c + 16m
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int rr = c + 16 * m;
      if ((m & 3) == g && rr < a.r) dqrow[rr] = dqs[m] * (a.qscale ? a.qscale[rr] : 1.f);
    }
  }
  if constexpr (MH) {
    for (int h = 0; h < a.heads; ++h) {  // uniform
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < kMaxHeads; ++q) t = (q == h) ? hsum[q] : t;
      t = wave_sum(t);
      if (lane == 0) a.rowsum_gs[row * a.heads + h] = t;
    }
  } else {
    gsum = wave_sum(gsum);
    if (lane == 0) a.rowsum_gs[row] = gsum;
  }
}

template <typename T, int W, int NV, bool SPLIT = false, bool MH = false>
static void launch_rows_bwd_kp(const RowsBwdArgs& a, dim3 grid, hipStream_t stream) {
  if (a.k <= 8) hipLaunchKernelGGL((rows_backward_kernel<T, W, NV, 8, SPLIT, MH>), grid, dim3(256), 0, stream, a);
  else if (a.k <= 16)
    hipLaunchKernelGGL((rows_backward_kernel<T, W, NV, 16, SPLIT, MH>), grid, dim3(256), 0, stream, a);
  else if (a.k <= 32)
    hipLaunchKernelGGL((rows_backward_kernel<T, W, NV, 32, SPLIT, MH>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((rows_backward_kernel<T, W, NV, 64, SPLIT, MH>), grid, dim3(256), 0, stream, a);
}

// Value-row widths of the row backward: one 16-byte pack per lane and pass
// slice, NV slices per 16-lane group (16 * W * NV elements per pass).
template <typename T, bool MH>
static void launch_rows_bwd_width(const RowsBwdArgs& a, bool vec, dim3 grid, hipStream_t stream) {
  constexpr int W = 16 / (int)sizeof(T);  // passes of 512, 256, 128 (or 64) elements
  if (!vec) launch_rows_bwd_kp<T, 1, 4, false, MH>(a, grid, stream);
  else if (a.D > 256) launch_rows_bwd_kp<T, W, 512 / (16 * W), false, MH>(a, grid, stream);
  else if (a.D > 128) launch_rows_bwd_kp<T, W, 256 / (16 * W), false, MH>(a, grid, stream);
  else if (a.D > 64 || W == 8) launch_rows_bwd_kp<T, W, 128 / (16 * W), false, MH>(a, grid, stream);
  else launch_rows_bwd_kp<T, W, 1, false, MH>(a, grid, stream);
}

template <typename T, int NV>
static void launch_rows_bwd_dots(const RowsBwdArgs& a, dim3 grid, int slab, hipStream_t stream) {
  if (a.k <= 8) hipLaunchKernelGGL((rows_backward_dots_kernel<T, NV, 8>), grid, dim3(256), 0, stream, a, slab);
  else if (a.k <= 16) hipLaunchKernelGGL((rows_backward_dots_kernel<T, NV, 16>), grid, dim3(256), 0, stream, a, slab);
  else if (a.k <= 32) hipLaunchKernelGGL((rows_backward_dots_kernel<T, NV, 32>), grid, dim3(256), 0, stream, a, slab);
  else hipLaunchKernelGGL((rows_backward_dots_kernel<T, NV, 64>), grid, dim3(256), 0, stream, a, slab);
}

// Column slab of the split row backward (0: no split).  Two slabs of 256 or
// 512 columns when a batch element's value rows exceed 2 MiB (an XCD's L2 is
// 4 MiB) and 256 < D <= 1024.
int rows_backward_slab(int64_t Nk, int D, bool vec, int elem_bytes) {
  if (!vec || D <= 256 || D > 1024 || Nk * (int64_t)D * elem_bytes <= (2LL << 20)) return 0;
  return D <= 512 ? 256 : 512;
}

int launch_rows_backward(const RowsBwdArgs& a, hipStream_t stream) {
  if (a.rows == 0) return kOk;
  if (a.r > kRegRank) {
    // ranks beyond the kernel's rank slots: the row kernel writes the score
    // gradients only (rank 0: its dQ loads read out of range and store
    // nothing), then the rank-chunked kernel forms dQ from them
    JN_REQUIRE(a.r <= kMaxRank && a.heads <= 1, kUnsupported,
               "rank must be at most %d (%d over several heads), got %d", kMaxRank, kRegRank, a.r);
    JN_REQUIRE(a.g_score && a.dq, kInvalidArgument, "wide-rank row backward needs g_score and dq");
    RowsBwdArgs b = a;
    b.r = 0;
    int rc = launch_rows_backward(b, stream);
    if (rc) return rc;
    RankRowsArgs rr{};
    rr.idx = a.idx;
    rr.g = a.g_score;
    rr.k = a.k;
    rr.key = a.key;
    rr.ldk = a.ldk;
    rr.qscale = a.qscale;
    rr.r = a.r;
    rr.Nq = a.Nq;
    rr.Nk = a.Nk;
    rr.rows = a.rows;
    rr.dq = a.dq;
    rr.lddq = a.lddq;
    return launch_rank_rows_grad(rr, stream);
  }
  JN_REQUIRE(a.r >= 0 && a.r <= kRegRank, kUnsupported, "rank must be in [1, %d]", kRegRank);
  const int64_t blocks = (a.rows + 3) / 4;
  JN_REQUIRE(2 * blocks < (1LL << 31), kInvalidArgument, "too many rows");
  JN_REQUIRE((int64_t)a.Nk * a.ld_pv * 4 < (1LL << 31) && (int64_t)a.Nk * a.ldk * 4 < (1LL << 31) &&
                 (int64_t)a.D * 4 < (1LL << 31),
             kUnsupported, "one batch element of the value or key rows must stay below 2 GiB");
  const int eb = a.bf16 ? 2 : 4, pw = 16 / eb;  // one 16-byte pack: 4 fp32 or 8 bf16 elements
  const bool vec = (a.D % pw == 0) && (a.ld_pv % pw == 0) && ((reinterpret_cast<uintptr_t>(a.pv) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.gdv) & 15) == 0);
  dim3 grid((unsigned)blocks);
  JN_REQUIRE(a.heads <= 1 ||
                 (a.ehead && a.heads <= kMaxHeads && a.head_rank >= 1 && a.heads * a.head_rank == a.r),
             kInvalidArgument, "multi-head row backward needs edge heads and %d..%d heads of equal rank", 2,
             kMaxHeads);
  if (a.heads > 1 && !a.dots_given) {
    JN_PROFILE("rows_backward_kernel", stream);
    if (a.bf16) launch_rows_bwd_width<bf16_t, true>(a, vec, grid, stream);
    else launch_rows_bwd_width<float, true>(a, vec, grid, stream);
    JN_LAUNCH_CHECK();
    return kOk;
  }
  if (a.dots_given) {
    JN_PROFILE("rows_backward_kernel", stream);
    if (a.heads > 1) launch_rows_bwd_kp<float, 4, 1, true, true>(a, grid, stream);
    else launch_rows_bwd_kp<float, 4, 1, true>(a, grid, stream);
    JN_LAUNCH_CHECK();
    return kOk;
  }
  const int slab = rows_backward_slab(a.Nk, a.D, vec, eb);
  if (slab) {
    {
      JN_PROFILE("rows_backward_dots_kernel", stream);
      const dim3 g2((unsigned)(2 * blocks));
      if (a.bf16) {  // 8 bf16 per pack: 16 x 8 x NV columns per group pass
        if (slab == 256) launch_rows_bwd_dots<bf16_t, 2>(a, g2, slab, stream);
        else launch_rows_bwd_dots<bf16_t, 4>(a, g2, slab, stream);
      } else {
        if (slab == 256) launch_rows_bwd_dots<float, 4>(a, g2, slab, stream);
        else launch_rows_bwd_dots<float, 8>(a, g2, slab, stream);
      }
      JN_LAUNCH_CHECK();
    }
    JN_PROFILE("rows_backward_kernel", stream);
    launch_rows_bwd_kp<float, 4, 1, true>(a, grid, stream);  // reads the dot partials, no value rows
    JN_LAUNCH_CHECK();
    return kOk;
  }
  JN_PROFILE("rows_backward_kernel", stream);
  if (a.bf16) launch_rows_bwd_width<bf16_t, false>(a, vec, grid, stream);
  else launch_rows_bwd_width<float, false>(a, vec, grid, stream);
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Rank-chunked gradients for ranks beyond the row and column kernels' rank
// slots (one head, up to kMaxRank ranks).  One wavefront per row (per column
// below); the ranks go in chunks of 64 lanes x 4 (VEC: 16-byte key rows) or
// 64 lanes x 1, each chunk summing the row's edges in index order with eight
// key rows in flight.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void rank_rows_grad_kernel(RankRowsArgs a) {
  constexpr int RC = VEC ? 4 * kWave : kWave;  // ranks per chunk
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= a.rows) return;
  const int64_t b = row / a.Nq;
  const auto rs = make_rsrc(a.key + b * a.Nk * a.ldk, (uint32_t)(a.Nk * a.ldk * 4));
  float* dqrow = a.dq + row * a.lddq;
  for (int r0 = 0; r0 < a.r; r0 += RC) {
    const int rr = r0 + (VEC ? 4 * lane : lane);
    const bool on = rr < a.r;  // VEC: r % 4 == 0, so the lane's four ranks are all in
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e0 = 0; e0 < a.k; e0 += kWave) {
      const int e = e0 + lane;
      const int j = e < a.k ? a.idx[row * a.k + e] : -1;
      const float gv = e < a.k ? a.g[row * a.k + e] : 0.f;
      const int ne = min(kWave, a.k - e0);
      for (int q = 0; q < ne; q += 8) {
        float4 v[8];
        float gq[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int src = min(q + u, kWave - 1);
          const int jj = q + u < ne ? readlane_i(j, src) : -1;
          gq[u] = jj >= 0 ? readlane_f(gv, src) : 0.f;
          const uint32_t off = (jj >= 0 && on) ? (uint32_t)(jj * a.ldk + rr) * 4u : kOobOffset;
          if constexpr (VEC) {
            v[u] = buf_load4(rs, off);
          } else {
            v[u] = make_float4(buf_load1(rs, off), 0.f, 0.f, 0.f);
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) fma4(acc, gq[u], v[u]);
      }
    }
    if (on) {
      if constexpr (VEC) {
        const float4 sc = a.qscale ? *reinterpret_cast<const float4*>(a.qscale + rr) : make_float4(1.f, 1.f, 1.f, 1.f);
        dqrow[rr] = acc.x * sc.x;
        dqrow[rr + 1] = acc.y * sc.y;
        dqrow[rr + 2] = acc.z * sc.z;
        dqrow[rr + 3] = acc.w * sc.w;
      } else {
        dqrow[rr] = acc.x * (a.qscale ? a.qscale[rr] : 1.f);
      }
    }
  }
}

int launch_rank_rows_grad(const RankRowsArgs& a, hipStream_t stream) {
  if (a.rows == 0) return kOk;
  JN_REQUIRE(a.r >= 1 && a.r <= kMaxRank && a.k >= 1, kUnsupported, "rank must be in [1, %d]", kMaxRank);
  JN_REQUIRE(a.idx && a.g && a.key && a.dq, kInvalidArgument, "null tensor pointer");
  JN_REQUIRE((int64_t)a.Nk * a.ldk * 4 < (1LL << 31), kUnsupported,
             "one batch element of the key rows must stay below 2 GiB");
  const int64_t blocks = (a.rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  const bool vec = (a.r % 4 == 0) && (a.ldk % 4 == 0) && (a.lddq % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.key) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(a.qscale) & 15) == 0);
  JN_PROFILE("rank_rows_grad_kernel", stream);
  if (vec) hipLaunchKernelGGL(rank_rows_grad_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(rank_rows_grad_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Deterministic transpose (CSR by key) of the edge list: a stable counting
// sort of the edges, in row order, by key.
//
// Rows are cut into tiles of up to 1024 rows (about one tile per CU).
//   1. csr_count_kernel: per tile, how many of its edges reach each key (LDS
//      counters) -> tile_base[b, t, j].
//   2. csr_tile_prefix_kernel (thread per key): the counts' prefix over the
//      tiles, written over them (edges into j from tiles before t), and per
//      256-key block the degrees' exclusive prefix and their sum (two extra
//      rows of the table).
//   3. csr_fill_kernel: per tile, the segment starts (a scan of the block
//      sums plus the in-block prefix; tile 0 writes them) plus
//      tile_base[b, t, j] become LDS cursors (the tile's first slot in each
//      key's segment); the next chunk's keys load during a chunk; the tile is
//      walked in chunks of at most 32 rows, where a key's incoming rows form a
//      32-bit LDS mask, so edge (row, j) lands at
//        cursor[j] + popcount(mask_j below row).
//      Each chunk costs work per edge only: the edge holding a key's highest
//      mask bit advances its cursor by popcount(mask_j) and clears the mask
//      during the next chunk, whose masks go to the other of two buffers.
// Segments therefore list incoming edges in increasing row order and every
// reduction over them is run-to-run reproducible.  Each slot receives the
// edge's record (row, coef, g_s or edge id, coef * gds[row]), so the column
// pass reads one contiguous 16-byte entry per incoming edge instead of chasing
// edge ids.  Keys are taken in LDS slices of kCsrFillSlice.
// ---------------------------------------------------------------------------
constexpr int kCsrCountSlice = 8192;  // keys per LDS pass of the count (int counters)
constexpr int kCsrFillSlice = 4096;   // keys per LDS pass of the fill (two 32-bit masks + an int cursor)
constexpr int kCsrChunkRows = 32;     // rows per fill chunk (one mask bit per row)
constexpr int kCsrFillEpt = 16;       // edges per thread of a fill chunk at most

// Rows per tile: whole 64-row chunks, about 256 tiles over the batch, at most
// 1024 rows (tile_base then has at most B * ceil(Nq / 64) * Nk entries).
int csr_tile_rows(int64_t B, int64_t Nq) {
  const int64_t want = (B * Nq + 255) / 256;
  return (int)std::min<int64_t>(1024, std::max<int64_t>(kCsrTile, (want + kCsrTile - 1) / kCsrTile * kCsrTile));
}
static int csr_tiles(const CsrArgs& a) { return (int)csr_tiles(a.B, a.Nq); }

bool csr_table_fits(int64_t B, int64_t Nq, int64_t Nk) {
  return B >= 1 && Nq >= 1 && Nk >= 1 && csr_table_entries(B, Nq, Nk) <= kCsrMaxTableEntries;
}

__global__ __launch_bounds__(256) void csr_count_kernel(CsrArgs a, int tile_rows) {
  extern __shared__ int cnt[];  // min(Nk, kCsrCountSlice) counters
  const int t = blockIdx.x, b = blockIdx.y, T = gridDim.x;
  const int r0 = t * tile_rows, nrows = min(tile_rows, a.Nq - r0);
  const int32_t* idx = a.idx + ((int64_t)b * a.Nq + r0) * a.k;
  const int ne = nrows * a.k;
  int32_t* out = a.tile_base + ((int64_t)b * (T + 2) + t) * a.Nk;
  for (int s0 = 0; s0 < a.Nk; s0 += kCsrCountSlice) {
    const int s1 = min(a.Nk, s0 + kCsrCountSlice);
    for (int x = threadIdx.x; x < s1 - s0; x += blockDim.x) cnt[x] = 0;
    __syncthreads();
    for (int x0 = threadIdx.x; x0 < ne; x0 += 256 * 8) {
      int j[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) j[u] = x0 + 256 * u < ne ? idx[x0 + 256 * u] : -1;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (j[u] >= s0 && j[u] < s1) atomicAdd(&cnt[j[u] - s0], 1);
    }
    __syncthreads();
    for (int x = threadIdx.x; x < s1 - s0; x += blockDim.x) out[s0 + x] = cnt[x];
    __syncthreads();
  }
}

// Thread per key j of a batch element (256-key blocks): the prefix of its
// counts over the T tiles is written over them (tile t then holds the edges
// into j from tiles before t); row T of the table receives the exclusive
// prefix of the degrees within the key's block, and row T + 1 the block's
// degree sum at the block's index.
__global__ __launch_bounds__(256) void csr_tile_prefix_kernel(int32_t* tile_base, int T, int Nk) {
  __shared__ int wave_tot[4];
  const int b = blockIdx.y, lane = lane_id(), wave = wave_id();
  const int j = blockIdx.x * 256 + (int)threadIdx.x;
  int32_t* table = tile_base + (int64_t)b * (T + 2) * Nk;
  int run = 0;
  if (j < Nk) {
    int32_t* cnt = table + j;
    int t = 0;
    for (; t + 8 <= T; t += 8) {
      int c[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) c[u] = cnt[(int64_t)(t + u) * Nk];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        cnt[(int64_t)(t + u) * Nk] = run;
        run += c[u];
      }
    }
    for (; t < T; ++t) {
      const int c = cnt[(int64_t)t * Nk];
      cnt[(int64_t)t * Nk] = run;
      run += c;
    }
  }
  int incl = run;  // the block's exclusive scan of the degrees
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __builtin_amdgcn_ds_bpermute(((lane - o) & 63) << 2, incl);
    if (lane >= o) incl += y;
  }
  if (lane == kWave - 1) wave_tot[wave] = incl;
  __syncthreads();
  int excl = incl - run;
  for (int w = 0; w < wave; ++w) excl += wave_tot[w];
  if (j < Nk) table[(int64_t)T * Nk + j] = excl;
  if (threadIdx.x == 0)
    table[(int64_t)(T + 1) * Nk + blockIdx.x] = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
}

// PLAIN: records {row | head, coef, edge id, 0} (no score or state
// gradients): every per-edge load of a chunk is issued before its barrier, so
// the record pass after it waits on nothing but LDS.
template <bool PLAIN>
__global__ __launch_bounds__(256) void csr_fill_kernel(CsrArgs a, int tile_rows, int chunk_rows) {
  extern __shared__ uint32_t lds[];  // masks[2][slice], then slice int cursors
  __shared__ int block_start[kCsrFillSlice / 256];
  __shared__ int slice_total;
  const int slice = min(a.Nk, kCsrFillSlice);
  int* cursor = reinterpret_cast<int*>(lds + 2 * slice);
  const int tid = threadIdx.x, lane = lane_id();
  const int t = blockIdx.x, b = blockIdx.y, T = gridDim.x;
  const int r0 = t * tile_rows, nrows = min(tile_rows, a.Nq - r0);
  const int64_t batch_base = (int64_t)b * a.Nq * a.k;
  const int32_t* table = a.tile_base + (int64_t)b * (T + 2) * a.Nk;
  const int32_t* before = table + (int64_t)t * a.Nk;        // edges into each key from earlier tiles
  const int32_t* in_block = table + (int64_t)T * a.Nk;      // degree prefix within each 256-key block
  const int32_t* block_sum = table + (int64_t)(T + 1) * a.Nk;
  int32_t* seg = a.seg_start + (int64_t)b * (a.Nk + 1);
  const int nchunks = (nrows + chunk_rows - 1) / chunk_rows;
  // the tile's edge index and coefficients (or softsign scores) through
  // buffer resources: loads of a chunk issue together, branch-free
  const int64_t tile_e0 = ((int64_t)b * a.Nq + r0) * a.k;
  const uint32_t tile_bytes = (uint32_t)(nrows * a.k) * 4u;
  const auto rs_idx = make_rsrc(a.idx + tile_e0, tile_bytes);
  const float* cf_src = a.coef ? a.coef : a.score;
  const auto rs_cf = make_rsrc(cf_src ? static_cast<const void*>(cf_src + tile_e0) : static_cast<const void*>(a.idx),
                               cf_src ? tile_bytes : 0u);
  [[maybe_unused]] const auto rs_head =
      make_rsrc(a.ehead ? static_cast<const void*>(a.ehead + tile_e0) : static_cast<const void*>(a.idx),
                a.ehead ? (uint32_t)(nrows * a.k) : 0u);
  int carry = 0;  // edges into the keys of earlier slices
  for (int s0 = 0; s0 < a.Nk; s0 += kCsrFillSlice) {
    const int ns = min(a.Nk, s0 + kCsrFillSlice) - s0;
    // segment starts: the slice's block sums scanned by one wave (every tile
    // forms the same numbers; tile 0 writes them), then this tile's first slot
    if (wave_id() == 0) {
      const int nb = (ns + 255) / 256;
      const int v = lane < nb ? block_sum[s0 / 256 + lane] : 0;
      int incl = v;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __builtin_amdgcn_ds_bpermute(((lane - o) & 63) << 2, incl);
        if (lane >= o) incl += y;
      }
      if (lane < nb) block_start[lane] = carry + incl - v;
      if (lane == kWave - 1) slice_total = incl;
    }
    __syncthreads();
    for (int x = tid; x < ns; x += 256) {
      const int start = block_start[x / 256] + in_block[s0 + x];
      if (t == 0) seg[s0 + x] = start;
      cursor[x] = start + before[s0 + x];
      lds[x] = 0u;
      lds[slice + x] = 0u;
    }
    carry += slice_total;
    __syncthreads();
    // the previous chunk's edges that hold their key's last row there: key
    // (slice-relative, -1 if none) and mask
    int pk[kCsrFillEpt];
    uint32_t pm[kCsrFillEpt];
    int jn[kCsrFillEpt];  // keys of the next chunk (prefetched; slots past it hold 0)
#pragma unroll
    for (int u = 0; u < kCsrFillEpt; ++u) {
      pk[u] = -1;
      const int x = tid + 256 * u;
      const bool in = x < min(chunk_rows, nrows) * a.k;  // (the chunk's test x < ne covers the rest)
      jn[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, in ? (uint32_t)x * 4u : kOobOffset, 0, 0);
    }
    for (int c = 0; c < nchunks; ++c) {
      uint32_t* M = lds + (c & 1) * slice;
      uint32_t* Mp = lds + ((c & 1) ^ 1) * slice;
      const int crow0 = c * chunk_rows;
      const int ne = min(chunk_rows, nrows - crow0) * a.k;
      const int64_t e0 = ((int64_t)b * a.Nq + r0 + crow0) * a.k;  // the chunk's first edge
      // the previous chunk's cursor advances and mask clears, beside this chunk's masks
#pragma unroll
      for (int u = 0; u < kCsrFillEpt; ++u) {
        if (pk[u] >= 0) {
          cursor[pk[u]] += __popc(pm[u]);
          Mp[pk[u]] = 0u;
        }
      }
      int jj[kCsrFillEpt];
      float raw[kCsrFillEpt];                  // coefficient, or the score softsign applies to
      [[maybe_unused]] int eh[kCsrFillEpt];    // head (PLAIN)
#pragma unroll
      for (int u = 0; u < kCsrFillEpt; ++u) {
        const int x = tid + 256 * u;
        const int j = jn[u] - s0;
        const bool in = x < ne && j >= 0 && j < ns;
        raw[u] = buf_load1(rs_cf, in ? (uint32_t)(crow0 * a.k + x) * 4u : kOobOffset);
        if constexpr (PLAIN)
          eh[u] = (int)__builtin_amdgcn_raw_buffer_load_b8(rs_head, in ? (uint32_t)(crow0 * a.k + x) : kOobOffset, 0,
                                                           0);
        if (in) atomicOr(&M[j], 1u << (x / a.k));
        jj[u] = in ? j : -1;
      }
      if (c + 1 < nchunks) {  // the next chunk's keys, in flight during this one
        const int nne = min(chunk_rows, nrows - crow0 - chunk_rows) * a.k;
        const int nx0 = (crow0 + chunk_rows) * a.k;
#pragma unroll
        for (int u = 0; u < kCsrFillEpt; ++u) {
          const int x = tid + 256 * u;
          // read as zeros past the chunk (x < ne rejects those slots); no
          // select here, so the loads stay in flight across the barrier
          jn[u] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_idx, x < nne ? (uint32_t)(nx0 + x) * 4u : kOobOffset,
                                                            0, 0);
        }
      }
      __syncthreads();
#pragma unroll
      for (int u = 0; u < kCsrFillEpt; ++u) {
        pk[u] = -1;
        const int j = jj[u];
        if (j < 0) continue;
        const int x = tid + 256 * u;
        const int rl = x / a.k;
        const uint32_t m = M[j];
        const int pos = cursor[j] + __popc(m & ((1u << rl) - 1u));
        const int64_t eid = e0 + x;
        const int row = b * a.Nq + r0 + crow0 + rl;
        const float cf = a.coef ? raw[u] : (a.score ? softsign_f(raw[u]) : 0.f);
        if constexpr (PLAIN) {
          a.rec[batch_base + pos] =
              make_float4(__int_as_float(row | (eh[u] << kRecHeadShift)), cf, __int_as_float((int)eid), 0.f);
        } else {
          const float gs = a.rec_eid ? __int_as_float((int)eid) : (a.g_score ? a.g_score[eid] : 0.f);
          const float cd = a.gds ? cf * a.gds[row] : 0.f;
          const int hd = a.ehead ? (int)a.ehead[eid] << kRecHeadShift : 0;
          a.rec[batch_base + pos] = make_float4(__int_as_float(row | hd), cf, gs, cd);
        }
        if (a.pos) a.pos[eid] = (int32_t)(batch_base + pos);
        if (31 - __clz(m) == rl) {  // the key's last row in this chunk
          pk[u] = j;
          pm[u] = m;
        }
      }
      __syncthreads();
    }
    __syncthreads();  // the cursors, masks and block starts are reset for the next slice
  }
  if (t == 0 && tid == 0) seg[a.Nk] = carry;
}

int launch_csr(const CsrArgs& a, hipStream_t stream) {
  int rc = launch_csr_layout(a, stream);
  if (rc) return rc;
  return launch_csr_fill(a, stream);
}

int launch_csr_layout(const CsrArgs& a, hipStream_t stream) {
  JN_REQUIRE((int64_t)a.B * a.Nq * a.k < (1LL << 31), kUnsupported, "edge count exceeds int32 ids");
  JN_REQUIRE((int64_t)a.B * a.Nq <= kRecRowMask, kUnsupported,
             "edge records hold rows below 2^%d (B * rows = %lld)", kRecHeadShift, (long long)a.B * a.Nq);
  JN_REQUIRE(csr_table_fits(a.B, a.Nq, a.Nk), kUnsupported,
             "edge grouping table of %lld tiles x %d keys exceeds %lld entries", (long long)a.B * csr_tiles(a),
             a.Nk, (long long)kCsrMaxTableEntries);
  dim3 g2(csr_tiles(a), a.B);
  {
    JN_PROFILE("csr_count_kernel", stream);
    hipLaunchKernelGGL(csr_count_kernel, g2, dim3(256), (size_t)min(a.Nk, kCsrCountSlice) * sizeof(int), stream, a,
                       csr_tile_rows(a.B, a.Nq));
    JN_LAUNCH_CHECK();
  }
  JN_PROFILE("csr_tile_prefix_kernel", stream);
  hipLaunchKernelGGL(csr_tile_prefix_kernel, dim3((a.Nk + 255) / 256, a.B), dim3(256), 0, stream, a.tile_base,
                     csr_tiles(a), a.Nk);
  JN_LAUNCH_CHECK();
  return kOk;
}

int launch_csr_fill(const CsrArgs& a, hipStream_t stream) {
  JN_REQUIRE(!a.score || a.compress == 0, kInvalidArgument, "records take inline coefficients for softsign only");
  JN_REQUIRE(a.k >= 1 && a.k <= 256 * kCsrFillEpt, kUnsupported, "edge grouping takes up to %d edges per row",
             256 * kCsrFillEpt);
  const int chunk_rows = std::max(1, std::min(kCsrChunkRows, 256 * kCsrFillEpt / a.k));
  dim3 g2(csr_tiles(a), a.B);
  const size_t lds = (size_t)min(a.Nk, kCsrFillSlice) * 3 * sizeof(uint32_t);
  JN_PROFILE("csr_fill_kernel", stream);
  if (a.rec_eid && !a.g_score && !a.gds)
    hipLaunchKernelGGL(csr_fill_kernel<true>, g2, dim3(256), lds, stream, a, csr_tile_rows(a.B, a.Nq), chunk_rows);
  else
    hipLaunchKernelGGL(csr_fill_kernel<false>, g2, dim3(256), lds, stream, a, csr_tile_rows(a.B, a.Nq), chunk_rows);
  JN_LAUNCH_CHECK();
  return kOk;
}

// ---------------------------------------------------------------------------
// Column backward: key columns j, walking their CSR segments (edge records in
// increasing row order, so every sum below has a fixed order and the results
// are run-to-run reproducible).
//   grad_pv[j]  = sum_in coef * gdv[i]                   (cols_gather_kernel)
//   grad_ps[j]  = sum_in coef * gds[i]
//   dK[j, r]    = kscale[r] * sum_in g_s * q[i, r]       (cols_keygrad_kernel)
//   part_c[w,r] = sum over the 16 columns of workgroup w of key[j, r] * sum_in g_s * q[i, r]
// ---------------------------------------------------------------------------

// A column's incoming edge records: CSR segment entries, or (BAND) the causal
// band's records built from the edge arrays with the CSR fill's arithmetic.
template <bool BAND>
struct ColRecords {
  const float4* rec;  // CSR: the segment's first record
  int64_t row0;       // BAND: global row of the column's first incoming edge (the key itself)
  int len;

  __device__ __forceinline__ ColRecords(const ColsBwdArgs& a, int64_t col) {
    const int b = (int)(col / a.Nk), j = (int)(col % a.Nk);
    if constexpr (BAND) {
      rec = nullptr;
      row0 = (int64_t)b * a.Nq + j;
      len = min(a.k, a.Nk - j);
    } else {
      const int32_t* seg = a.seg_start + (int64_t)b * (a.Nk + 1);
      const int beg = seg[j];
      len = seg[j + 1] - beg;
      rec = a.rec + (int64_t)b * a.Nq * a.k + beg;
      row0 = 0;
    }
  }
  __device__ __forceinline__ float4 get(const ColsBwdArgs& a, int q) const {
    if constexpr (BAND) {
      const int64_t row = row0 + q;
      const int64_t eid = row * a.k + (a.k - 1 - q);
      const float cf = a.coef ? a.coef[eid] : 0.f;
      const float gs = a.g_score ? a.g_score[eid] : 0.f;
      const float cd = a.gds ? cf * a.gds[row] : 0.f;
      const int hd = a.ehead ? (int)a.ehead[eid] << kRecHeadShift : 0;
      return make_float4(__int_as_float((int)row | hd), cf, gs, cd);
    } else {
      return rec[q];
    }
  }
};

// One wavefront per column and column slab: the gather-accumulate of
// rows_forward_kernel over the column's records.  The grid is slab-major, so an
// XCD gathers rows of one slab of one batch element at a time (Nq x slab floats,
// sized to its L2).  Slab 0 also sums the state.
// T: element type of the gathered rows (gdv) and of grad_pv.
template <typename T, int W, bool BAND>
__global__ __launch_bounds__(256) void cols_gather_kernel(ColsBwdArgs a, int slab_cols) {
  const int lane = lane_id();
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  const int64_t col_blocks = (total_cols + 3) / 4;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int slab = (int)(logical / col_blocks);
  const int64_t col = (logical % col_blocks) * 4 + wave_id();
  if (col >= total_cols) return;
  const ColRecords<BAND> recs(a, col);
  const int len = recs.len;
  const int d_begin = slab * slab_cols, d_end = min(a.D, d_begin + slab_cols);
  const T* gdv = reinterpret_cast<const T*>(a.gdv);
  T* out = a.grad_pv ? reinterpret_cast<T*>(a.grad_pv) + col * a.ld_gpv : nullptr;

  float st = 0.0f;
  const int nblk = max(1, (len + kWave - 1) / kWave);  // a column without edges still writes zeros
  for (int blk = 0; blk < nblk; ++blk) {
    const int q0 = blk * kWave;
    const int n = min(kWave, len - q0);
    int row = 0;
    float cf = 0.f, cd = 0.f;
    if (lane < n) {
      const float4 r = recs.get(a, q0 + lane);
      row = __float_as_int(r.x) & kRecRowMask;
      cf = r.y;
      cd = r.w;
    }
    st += cd;  // lanes past the segment hold 0
    if (!out) continue;
    for (int d = d_begin + lane * W; d < d_end; d += kWave * W) {
      // two accumulation chains (even / odd records), summed at the end
      Pack<W> acc = pack_zero<T, W>(), acc1 = acc;
      int q = 0;
      for (; q + 8 <= n; q += 8) {
        Pack<W> v[8];
        float cc[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          cc[u] = readlane_f(cf, q + u);
          v[u] = load_pack<T, W>(gdv + (int64_t)readlane_i(row, q + u) * a.D + d);
        }
#pragma unroll
        for (int u = 0; u < 8; u += 2) {
          fma_pack(acc, cc[u], v[u]);
          fma_pack(acc1, cc[u + 1], v[u + 1]);
        }
      }
      for (; q < n; ++q)
        fma_pack((q & 1) ? acc1 : acc, readlane_f(cf, q), load_pack<T, W>(gdv + (int64_t)readlane_i(row, q) * a.D + d));
      acc = add_pack(acc, acc1);
      if (blk > 0) acc = add_pack(acc, load_pack<T, W>(out + d));
      store_pack<T, W>(out + d, acc);
    }
  }
  if (slab == 0 && a.grad_ps) {
    st = wave_sum(st);
    if (lane == 0) a.grad_ps[col] = st;
  }
}

// Sums each of v[0..7] over the 64 lanes; lane L receives the total of
// v[L >> 3].  Each exchange halves the values a lane holds: the permlane swaps
// pair lanes L ^ 32 and L ^ 16, a row mirror pairs opposite bit 3, and three
// DPP steps finish the sum inside each 8-lane half-row (10 exchanges for 8
// sums instead of 8 x 6).
__device__ __forceinline__ float transpose_sum8(const float (&v)[8]) {
  float w[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // lanes < 32 keep v[m] (with lane + 32's), lanes >= 32 keep v[m + 4]
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[m]), __float_as_uint(v[m + 4]), false, false);
    w[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  float x[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    // rows 0 and 2 keep w[m] (with the next row's), rows 1 and 3 keep w[m + 2]
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[m]), __float_as_uint(w[m + 2]), false, false);
    x[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  const bool b3 = (lane_id() & 8) != 0;
  float y = (b3 ? x[1] : x[0]) + dpp_f<0x140>(b3 ? x[0] : x[1]);  // row_mirror flips bit 3
  y += dpp_f<0xB1>(y);   // quad_perm [1,0,3,2]
  y += dpp_f<0x4E>(y);   // quad_perm [2,3,0,1]
  y += dpp_f<0x141>(y);  // row_half_mirror
  return y;
}

// Sums each of v[0..3] over the 64 lanes; lane L receives the total of
// v[L >> 4] (two permlane steps, then a sum inside each 16-lane row).
__device__ __forceinline__ float transpose_sum4(const float (&v)[4]) {
  float w[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[m]), __float_as_uint(v[m + 2]), false, false);
    w[m] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[0]), __float_as_uint(w[1]), false, false);
  return row16_sum(__uint_as_float(p[0]) + __uint_as_float(p[1]));
}

template <int G>
__device__ __forceinline__ float transpose_sum(const float (&v)[G]) {
  if constexpr (G == 8) return transpose_sum8(v);
  else return transpose_sum4(v);
}

// Fused column pass: one wavefront per key column and slab of kWave * W
// columns (one 16-byte pack per lane), slab-major over the grid as in
// cols_gather_kernel.  Each incoming edge's gdv row (slab) is read once and
// serves both
//   grad_pv[j] += coef * gdv[i]          (the column sum of cols_gather_kernel)
//   dots_s[x]   = <gdv[i], pv[j]> over slab s, x = the edge's record index
// the second being the edge-coefficient gradient the row backward needs (its
// value-row gather is then not run; it finds x through CsrArgs::pos).
// G records per group: their rows are in flight together, then G dot
// partials are summed over the wave by one transpose-sum.
// BUF (a batch element's gdv rows span less than 2^31 bytes): the rows load
// through a buffer resource over the column's batch element, the record's row
// offset in the scalar offset and the lane's column offset in the vector
// offset; records past the segment and lanes past D read zeros out of range,
// so a group's loads need no per-lane branch, zeroing or 64-bit address.
template <typename T, int W, int G, bool BUF>
__global__ __launch_bounds__(256) void cols_gather_dots_kernel(ColsBwdArgs a) {
  constexpr int SLAB = kWave * W;
  const int lane = lane_id();
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  const int64_t col_blocks = (total_cols + 3) / 4;
  const int64_t logical = xcd_swizzle(blockIdx.x, gridDim.x);
  const int slab = (int)(logical / col_blocks);
  const int64_t col = (logical % col_blocks) * 4 + wave_id();
  if (col >= total_cols) return;
  const ColRecords<false> recs(a, col);
  const int len = recs.len;
  const int d = slab * SLAB + lane * W;
  const bool on = d < a.D;  // a.D % W == 0 (host)
  const T* gdv = reinterpret_cast<const T*>(a.gdv) + (on ? d : 0);
  const Pack<W> pj =
      on ? unpack16<T, W>(load_nt16(reinterpret_cast<const T*>(a.pv) + col * a.ld_pv + d)) : pack_zero<T, W>();
  float* part = slab == 0 ? a.dots0 : a.dots1;
  const int64_t rec_base = recs.rec - a.rec;  // record index of the column's first record
  const int64_t bq = col / a.Nk;              // the column's batch element
  const int row0 = (int)(bq * a.Nq);          // its first global row
  const uint32_t row_bytes = (uint32_t)a.D * (uint32_t)sizeof(T);
  const auto rs_g = make_rsrc(reinterpret_cast<const T*>(a.gdv) + (BUF ? bq * a.Nq * a.D : 0),
                              BUF ? (uint32_t)((int64_t)a.Nq * row_bytes) : 0u);
  const uint32_t voff = on ? (uint32_t)d * (uint32_t)sizeof(T) : kOobOffset;

  Pack<W> acc = pack_zero<T, W>(), acc1 = acc;  // even / odd records
  float st = 0.f;
  for (int q0 = 0; q0 < len; q0 += kWave) {
    const int n = min(kWave, len - q0);
    const int64_t rec0 = rec_base + q0;
    int row = 0;
    float cf = 0.f;
    if (lane < n) {
      const uint4 r = load_nt16(recs.rec + q0 + lane);
      row = (int)r.x & kRecRowMask;
      cf = __uint_as_float(r.y);
      if (a.gds) st += cf * a.gds[row];
    }
    for (int q = 0; q < n; q += G) {  // n and q are wave-uniform
      // the group's rows as raw 16-byte packs (widened where used)
      uint4 raw[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const int src = min(q + u, kWave - 1);
        if constexpr (BUF) {
          const bool live = q + u < n;  // wave-uniform
          const uint32_t so = live ? (uint32_t)(readlane_i(row, src) - row0) * row_bytes : 0u;
          raw[u] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(rs_g, live ? voff : kOobOffset, so, 0));
        } else {
          raw[u] = (q + u < n && on) ? *reinterpret_cast<const uint4*>(gdv + (int64_t)readlane_i(row, src) * a.D)
                                     : make_uint4(0u, 0u, 0u, 0u);
        }
      }
      // lanes (64 / G) u receive record q + u's total
      constexpr int LPR = kWave / G;
      const int ru = q + lane / LPR;
      const bool writer = lane % LPR == 0 && ru < n;
      float pd[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        // records past the segment hold cf = 0 (and zero rows)
        const Pack<W> v = unpack16<T, W>(raw[u]);
        fma_pack((u & 1) ? acc1 : acc, readlane_f(cf, min(q + u, kWave - 1)), v);
        pd[u] = dot_pack(v, pj);
      }
      const float tot = transpose_sum<G>(pd);
      if (writer) part[rec0 + ru] = tot;  // record order: consecutive records, consecutive slots
    }
  }
  if (a.grad_pv && on)
    store_nt16(reinterpret_cast<T*>(a.grad_pv) + col * a.ld_gpv + d, pack_bits<T, W>(add_pack(acc, acc1)));
  if (slab == 0 && a.grad_ps) {
    st = wave_sum(st);
    if (lane == 0) a.grad_ps[col] = st;
  }
}

int cols_gather_dots_slabs(const ColsBwdArgs& a) {
  const int eb = a.bf16 ? 2 : 4, pw = 16 / eb;
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (a.band || !a.rec || !a.pv || !a.dots0 || a.D < 1) return 0;
  if (a.D % pw || a.ld_pv % pw || !a16(a.gdv) || !a16(a.pv)) return 0;
  if (a.grad_pv && (a.ld_gpv % pw || !a16(a.grad_pv))) return 0;
  const int slabs = (a.D + kWave * pw - 1) / (kWave * pw);
  if (slabs > 2 || (slabs == 2 && !a.dots1)) return 0;
  return slabs;
}

int launch_cols_gather_dots(const ColsBwdArgs& a, hipStream_t stream) {
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  if (total_cols == 0) return kOk;
  const int slabs = cols_gather_dots_slabs(a);
  JN_REQUIRE(slabs > 0, kInvalidArgument, "fused column pass needs CSR records with edge ids and aligned rows");
  JN_REQUIRE((int64_t)a.B * a.Nq * a.k < (1LL << 31), kUnsupported, "edge count exceeds int32 ids");
  const int64_t blocks = (total_cols + 3) / 4 * slabs;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many columns");
  JN_PROFILE("cols_gather_dots_kernel", stream);
  const dim3 grid((unsigned)blocks);
  const bool buf = (int64_t)a.Nq * a.D * (a.bf16 ? 2 : 4) < (int64_t)kOobOffset;
  if (a.bf16) {
    if (buf) hipLaunchKernelGGL((cols_gather_dots_kernel<bf16_t, 8, 4, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((cols_gather_dots_kernel<bf16_t, 8, 4, false>), grid, dim3(256), 0, stream, a);
  } else {
    if (buf) hipLaunchKernelGGL((cols_gather_dots_kernel<float, 4, 8, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((cols_gather_dots_kernel<float, 4, 8, false>), grid, dim3(256), 0, stream, a);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

// One wavefront per row: the coefficients row_coefficients gives the row
// kernels, written out for the edge records.
__global__ __launch_bounds__(256) void edge_coefficients_kernel(const int32_t* idx, const float* score, int64_t rows,
                                                                int k, int compress, float* coef) {
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const RowStats rst = row_compress_stats(idx, score, row, k, compress);
  for (int e0 = 0; e0 < k; e0 += kWave) {
    int j;
    float c, s;
    row_coefficients(idx, score, row, k, e0, compress, rst, j, c, s);
    if (e0 + lane_id() < k) coef[row * k + e0 + lane_id()] = c;
  }
}

int launch_edge_coefficients(const int32_t* idx, const float* score, int64_t rows, int k, int compress, float* coef,
                             hipStream_t stream) {
  if (rows == 0) return kOk;
  const int64_t blocks = (rows + 3) / 4;
  JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many rows");
  JN_PROFILE("edge_coefficients_kernel", stream);
  hipLaunchKernelGGL(edge_coefficients_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, idx, score, rows, k,
                     compress, coef);
  JN_LAUNCH_CHECK();
  return kOk;
}

// One 16-lane group per column (16 columns per workgroup).  Lane c of a group
// holds 8 rank slots: ranks 4c..4c+3 and 64+4c..64+4c+3 when the query rows are
// read as float4 (VEC), else ranks c + 16m.  The group walks its column's
// records 16 at a time; each lane loads one record and the group's lanes take
// turns broadcasting theirs (ds_bpermute), so the 4 columns of a wave advance
// together.  The scale-vector partials of the 16 columns are summed in a fixed
// order into one row of part_c per workgroup.
// MH: each record's head (its row word's top bits) selects the ranks it reaches.
template <bool VEC, bool MH, bool BAND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(VEC && !MH ? 5 : 1))) void cols_keygrad_kernel(ColsBwdArgs a) {
  __shared__ float red[4][128];
  const int lane = lane_id(), g = lane >> 4, c = lane & 15, w = wave_id();
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  const int64_t blk = xcd_swizzle(blockIdx.x, gridDim.x);
  const int64_t col = blk * 16 + w * 4 + g;
  const bool valid = col < total_cols;
  const ColRecords<BAND> recs(a, valid ? col : 0);
  const int len = valid ? recs.len : 0;
  int rk[8];  // rank of each slot
#pragma unroll
  for (int m = 0; m < 8; ++m) rk[m] = VEC ? (m < 4 ? 4 * c + m : 64 + 4 * c + (m - 4)) : c + 16 * m;
  int hk[8];  // MH: head of each slot (a float4 never straddles two heads: head_rank % 4 == 0 with VEC)
  if constexpr (MH) {
#pragma unroll
    for (int m = 0; m < 8; ++m) hk[m] = rk[m] / a.head_rank;
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // wave-uniform trip count: the longest of the wave's four columns
  const int wlen = max(max(readlane_i(len, 0), readlane_i(len, 16)), max(readlane_i(len, 32), readlane_i(len, 48)));
  for (int q0 = 0; q0 < wlen; q0 += 16) {
    int row = -1;
    float gs = 0.f;
    if (q0 + c < len) {
      const float4 r = recs.get(a, q0 + c);
      row = __float_as_int(r.x);
      gs = (!BAND && a.rec_eid) ? a.g_score[__float_as_int(r.z)] : r.z;
    }
    const int nu = min(16, wlen - q0);
    for (int u0 = 0; u0 < nu; u0 += 8) {
      float qv[8][8];
      float gg[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int src = (g * 16 + ((u0 + u) & 15)) << 2;
        const int rw_word = __builtin_amdgcn_ds_bpermute(src, row);
        gg[u] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(gs)));
        const bool ok = (u0 + u < nu) && rw_word >= 0;  // past the column's end: row -1, gs 0
        const int rw = MH ? (rw_word & kRecRowMask) : rw_word;
        const int eh = MH ? (rw_word >> kRecHeadShift) : 0;
        auto mine = [&](int m) { return !MH || hk[m] == eh; };
        const float* qr = a.q + (int64_t)(ok ? rw : 0) * a.ldq;
        if (VEC) {
          const float4 lo = (ok && 4 * c < a.r && mine(0)) ? *reinterpret_cast<const float4*>(qr + 4 * c)
                                                           : make_float4(0.f, 0.f, 0.f, 0.f);
          const float4 hi = (ok && 64 + 4 * c < a.r && mine(4)) ? *reinterpret_cast<const float4*>(qr + 64 + 4 * c)
                                                                : make_float4(0.f, 0.f, 0.f, 0.f);
          qv[u][0] = lo.x; qv[u][1] = lo.y; qv[u][2] = lo.z; qv[u][3] = lo.w;
          qv[u][4] = hi.x; qv[u][5] = hi.y; qv[u][6] = hi.z; qv[u][7] = hi.w;
        } else {
#pragma unroll
          for (int m = 0; m < 8; ++m) qv[u][m] = (ok && rk[m] < a.r && mine(m)) ? qr[rk[m]] : 0.f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] += gg[u] * qv[u][m];
    }
  }
  float pc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    pc[m] = 0.f;
    if (valid && rk[m] < a.r) {
      a.dk[col * a.lddk + rk[m]] = acc[m] * (a.kscale ? a.kscale[rk[m]] : 1.f);
      pc[m] = a.key[col * a.ldk + rk[m]] * acc[m];
    }
  }
  if (!a.part_c) return;  // uniform
  // sum the wave's four columns (groups), then the workgroup's four waves
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    pc[m] += xor16_f(pc[m]);
    pc[m] += xor32_f(pc[m]);
  }
  if (g == 0) {
#pragma unroll
    for (int m = 0; m < 8; ++m)
      if (rk[m] < 128) red[w][rk[m]] = pc[m];
  }
  __syncthreads();
  for (int rr = threadIdx.x; rr < a.r; rr += blockDim.x)
    a.part_c[blk * a.r + rr] = (red[0][rr] + red[1][rr]) + (red[2][rr] + red[3][rr]);
}

int cols_backward_parts(int64_t total_cols) { return (int)((total_cols + 15) / 16); }

// ---------------------------------------------------------------------------
// Unit-norm scale vectors (the score scale w_hat = w / max(||w||_2, eps) of
// LowRankBilinearPairwise, modules.py:85-87, one row per head) and the
// gradient of that map,
//   grad_w = g / d - [n >= eps] (g . w) / (d^2 n) w,   n = ||w||, d = max(n, eps)
// (the clamp passes its gradient where n >= eps, as torch's clamp_min does).
// One wavefront per row; both sums in a fixed order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void unit_scale_kernel(const float* w, const float* grad, int r, float eps,
                                                        float* out) {
  const int64_t base = (int64_t)blockIdx.x * r;
  float ss = 0.f, gw = 0.f;
  for (int i = lane_id(); i < r; i += kWave) {
    const float x = w[base + i];
    ss += x * x;
    if (grad) gw += grad[base + i] * x;
  }
  const float n = sqrtf(wave_sum(ss));
  const float d = fmaxf(n, eps);
  if (!grad) {
    for (int i = lane_id(); i < r; i += kWave) out[base + i] = w[base + i] / d;
    return;
  }
  gw = wave_sum(gw);
  const float c = n >= eps ? gw / (d * d * n) : 0.f;
  for (int i = lane_id(); i < r; i += kWave) out[base + i] = grad[base + i] / d - c * w[base + i];
}

int launch_unit_scale(const float* w, const float* grad, int64_t rows, int64_t r, float eps, float* out,
                      hipStream_t stream) {
  JN_REQUIRE(w && out, kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(rows >= 1 && r >= 1 && rows < (1LL << 31) && r < (1LL << 30), kInvalidArgument,
             "unit scale needs 1 <= rows < 2^31 and 1 <= r < 2^30 (rows=%lld, r=%lld)", (long long)rows,
             (long long)r);
  JN_REQUIRE(eps > 0.0f, kInvalidArgument, "eps must be positive");
  JN_PROFILE(grad ? "unit_scale_backward_kernel" : "unit_scale_kernel", stream);
  hipLaunchKernelGGL(unit_scale_kernel, dim3((unsigned)rows), dim3(kWave), 0, stream, w, grad, (int)r, eps, out);
  JN_LAUNCH_CHECK();
  return kOk;
}

// Key-side gradient and scale-vector partials for ranks beyond the column
// kernel's rank slots (one head): dk[j, :] = kscale * sum over j's records
// of g * q[row, :], and partial key[j, :] * (sum g q[row, :]).  Each wave takes
// four of the workgroup's sixteen columns in turn (cols_backward_parts rows of
// part_c, as the column kernel), keeping its columns' partial sums in its own
// LDS row; the four rows are then summed in wave order.
template <bool VEC, bool BAND>
__global__ __launch_bounds__(256) void rank_cols_grad_kernel(ColsBwdArgs a) {
  __shared__ float red[4][kMaxRank];
  constexpr int RC = VEC ? 4 * kWave : kWave;  // ranks per chunk
  const int lane = lane_id(), w = wave_id();
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  const int64_t blk = xcd_swizzle(blockIdx.x, gridDim.x);
  for (int rr = lane; rr < a.r; rr += kWave) red[w][rr] = 0.f;
  wave_lds_sync();
  for (int t = 0; t < 4; ++t) {
    const int64_t col = blk * 16 + w * 4 + t;
    if (col >= total_cols) break;  // wave-uniform; the barrier below is outside the loop
    const ColRecords<BAND> recs(a, col);
    const int len = recs.len;
    for (int r0 = 0; r0 < a.r; r0 += RC) {
      const int rr = r0 + (VEC ? 4 * lane : lane);
      const bool on = rr < a.r;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int q0 = 0; q0 < len; q0 += kWave) {
        int row = -1;
        float gs = 0.f;
        if (q0 + lane < len) {
          const float4 rc = recs.get(a, q0 + lane);
          row = __float_as_int(rc.x) & kRecRowMask;
          gs = (!BAND && a.rec_eid) ? a.g_score[__float_as_int(rc.z)] : rc.z;
        }
        const int n = min(kWave, len - q0);
        for (int q = 0; q < n; q += 8) {
          float4 v[8];
          float gq[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int src = min(q + u, kWave - 1);
            const int rw = q + u < n ? readlane_i(row, src) : -1;
            gq[u] = rw >= 0 ? readlane_f(gs, src) : 0.f;
            const float* qr = a.q + (int64_t)(rw >= 0 ? rw : 0) * a.ldq + (on ? rr : 0);
            if constexpr (VEC) {
              v[u] = (rw >= 0 && on) ? *reinterpret_cast<const float4*>(qr) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
              v[u] = make_float4((rw >= 0 && on) ? *qr : 0.f, 0.f, 0.f, 0.f);
            }
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) fma4(acc, gq[u], v[u]);
        }
      }
      if (on) {
        const float* kr = a.key + col * a.ldk + rr;
        float* dkr = a.dk + col * a.lddk + rr;
        const int nr = VEC ? 4 : 1;
        const float av[4] = {acc.x, acc.y, acc.z, acc.w};
        for (int m = 0; m < nr; ++m) {
          dkr[m] = av[m] * (a.kscale ? a.kscale[rr + m] : 1.f);
          red[w][rr + m] += kr[m] * av[m];
        }
      }
      wave_lds_sync();
    }
  }
  if (!a.part_c) return;  // uniform over the workgroup
  __syncthreads();
  for (int rr = threadIdx.x; rr < a.r; rr += blockDim.x)
    a.part_c[blk * a.r + rr] = (red[0][rr] + red[1][rr]) + (red[2][rr] + red[3][rr]);
}

int launch_cols_backward(const ColsBwdArgs& a, hipStream_t stream) {
  const int64_t total_cols = (int64_t)a.B * a.Nk;
  if (total_cols == 0) return kOk;
  JN_REQUIRE(!a.q || (a.r >= 1 && (a.r <= kRegRank || (a.r <= kMaxRank && a.heads <= 1))), kUnsupported,
             "rank must be in [1, %d] (%d over several heads), got %d", kMaxRank, kRegRank, a.r);
  JN_REQUIRE(!a.q || (a.key && a.dk), kInvalidArgument, "key-side gradient needs key and dk");
  JN_REQUIRE((int64_t)a.B * a.Nq * a.k < (1LL << 31), kUnsupported, "edge count exceeds int32 ids");
  JN_REQUIRE(!a.band || (a.Nq == a.Nk && a.coef && a.g_score && (int64_t)a.B * a.Nq <= kRecRowMask),
             kInvalidArgument, "band records need Nq == Nk, coef and g_score, and rows below 2^%d", kRecHeadShift);
  if (a.grad_pv || a.grad_ps) {
    const int eb = a.bf16 ? 2 : 4, pw = 16 / eb;  // one 16-byte pack: 4 fp32 or 8 bf16 elements
    const bool vec = (a.D % pw == 0) && (a.ld_gpv % pw == 0) && ((reinterpret_cast<uintptr_t>(a.gdv) & 15) == 0) &&
                     (a.grad_pv == nullptr || (reinterpret_cast<uintptr_t>(a.grad_pv) & 15) == 0);
    // slabs of 64 packs while a batch element's gathered rows exceed 2 MiB
    int slab = a.D;
    if (vec)
      while (slab > 64 * pw && slab % (128 * pw) == 0 && (int64_t)a.Nq * slab * eb > (2LL << 20)) slab /= 2;
    const int64_t slabs = a.grad_pv ? (a.D + slab - 1) / slab : 1;
    const int64_t blocks = (total_cols + 3) / 4 * slabs;
    JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many columns");
    JN_PROFILE(a.profile_name ? a.profile_name : "cols_gather_kernel", stream);
    const dim3 grid((unsigned)blocks);
    if (a.band) {
      if (a.bf16) {
        if (vec) hipLaunchKernelGGL((cols_gather_kernel<bf16_t, 8, true>), grid, dim3(256), 0, stream, a, slab);
        else hipLaunchKernelGGL((cols_gather_kernel<bf16_t, 1, true>), grid, dim3(256), 0, stream, a, slab);
      } else {
        if (vec) hipLaunchKernelGGL((cols_gather_kernel<float, 4, true>), grid, dim3(256), 0, stream, a, slab);
        else hipLaunchKernelGGL((cols_gather_kernel<float, 1, true>), grid, dim3(256), 0, stream, a, slab);
      }
    } else if (a.bf16) {
      if (vec) hipLaunchKernelGGL((cols_gather_kernel<bf16_t, 8, false>), grid, dim3(256), 0, stream, a, slab);
      else hipLaunchKernelGGL((cols_gather_kernel<bf16_t, 1, false>), grid, dim3(256), 0, stream, a, slab);
    } else {
      if (vec) hipLaunchKernelGGL((cols_gather_kernel<float, 4, false>), grid, dim3(256), 0, stream, a, slab);
      else hipLaunchKernelGGL((cols_gather_kernel<float, 1, false>), grid, dim3(256), 0, stream, a, slab);
    }
    JN_LAUNCH_CHECK();
  }
  if (a.q && a.r > kRegRank) {  // ranks beyond the column kernel's rank slots
    const bool vec = (a.r % 4 == 0) && (a.ldq % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0);
    const int64_t blocks = cols_backward_parts(total_cols);
    JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many columns");
    JN_PROFILE("rank_cols_grad_kernel", stream);
    const dim3 grid((unsigned)blocks);
    if (a.band) {
      if (vec) hipLaunchKernelGGL((rank_cols_grad_kernel<true, true>), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((rank_cols_grad_kernel<false, true>), grid, dim3(256), 0, stream, a);
    } else {
      if (vec) hipLaunchKernelGGL((rank_cols_grad_kernel<true, false>), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((rank_cols_grad_kernel<false, false>), grid, dim3(256), 0, stream, a);
    }
    JN_LAUNCH_CHECK();
  } else if (a.q) {
    const bool mh = a.heads > 1;
    JN_REQUIRE(!mh || (a.heads <= kMaxHeads && a.head_rank >= 1 && a.heads * a.head_rank == a.r), kInvalidArgument,
               "multi-head column backward needs 2..%d heads of equal rank", kMaxHeads);
    const bool vec = (a.r % 4 == 0) && (a.ldq % 4 == 0) && ((reinterpret_cast<uintptr_t>(a.q) & 15) == 0) &&
                     (!mh || a.head_rank % 4 == 0);
    const int64_t blocks = cols_backward_parts(total_cols);
    JN_REQUIRE(blocks < (1LL << 31), kInvalidArgument, "too many columns");
    JN_PROFILE("cols_keygrad_kernel", stream);
    const dim3 grid((unsigned)blocks);
    if (a.band) {
      if (mh) {
        if (vec) hipLaunchKernelGGL((cols_keygrad_kernel<true, true, true>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((cols_keygrad_kernel<false, true, true>), grid, dim3(256), 0, stream, a);
      } else {
        if (vec) hipLaunchKernelGGL((cols_keygrad_kernel<true, false, true>), grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((cols_keygrad_kernel<false, false, true>), grid, dim3(256), 0, stream, a);
      }
    } else if (mh) {
      if (vec) hipLaunchKernelGGL((cols_keygrad_kernel<true, true, false>), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((cols_keygrad_kernel<false, true, false>), grid, dim3(256), 0, stream, a);
    } else {
      if (vec) hipLaunchKernelGGL((cols_keygrad_kernel<true, false, false>), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((cols_keygrad_kernel<false, false, false>), grid, dim3(256), 0, stream, a);
    }
    JN_LAUNCH_CHECK();
  }
  return kOk;
}

// ---------------------------------------------------------------------------
// Reduction of the small gradients (scale vector, bias) in two fixed-order
// stages: kFinBlocks workgroups each reduce a contiguous share of the [nparts, r]
// partials and of the [nrows, nbias] row sums into stage[blk, 0..r + nbias);
// then workgroup b < r + nbias sums column b of stage over the kFinBlocks rows.
// ---------------------------------------------------------------------------
constexpr int kFinBlocks = 256;

size_t finalize_stage_floats(int r, int nbias) { return (size_t)kFinBlocks * (r + nbias); }

__global__ __launch_bounds__(256) void finalize_partials_kernel(const float* part_c, int nparts, int r,
                                                                const float* rowsum, int64_t nrows, int nbias,
                                                                float* stage) {
  __shared__ float red[256];
  const int t = threadIdx.x, blk = blockIdx.x;
  const int64_t width = r + nbias;
  const int64_t p0 = (int64_t)nparts * blk / kFinBlocks, p1 = (int64_t)nparts * (blk + 1) / kFinBlocks;
  // columns in chunks of at most 256; a chunk of cw columns takes r_pad
  // columns (power of two >= cw) x 256 / r_pad row lanes
  for (int c0 = 0; c0 < r; c0 += 256) {
    const int cw = min(256, r - c0);
    int r_pad = 1;
    while (r_pad < cw) r_pad <<= 1;
    const int col = t & (r_pad - 1), sub = t / r_pad, nsub = 256 / r_pad;
    float s = 0.f;
    if (col < cw)
      for (int64_t p = p0 + sub; p < p1; p += nsub) s += part_c[p * r + c0 + col];
    __syncthreads();  // the previous chunk's reads of red are done
    red[t] = s;
    __syncthreads();
    for (int o = 128; o >= r_pad; o >>= 1) {  // sum the row lanes of each column
      if (t < o) red[t] += red[t + o];
      __syncthreads();
    }
    if (t < cw) stage[blk * width + c0 + t] = red[t];
  }
  const int64_t i0 = nrows * blk / kFinBlocks, i1 = nrows * (blk + 1) / kFinBlocks;
  for (int h = 0; h < nbias; ++h) {
    __syncthreads();
    float q = 0.f;
    for (int64_t i = i0 + t; i < i1; i += 256) q += rowsum[i * nbias + h];
    red[t] = q;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (t < o) red[t] += red[t + o];
      __syncthreads();
    }
    if (t == 0) stage[blk * width + r + h] = red[0];
  }
}

__global__ __launch_bounds__(256) void finalize_small_grads_kernel(const float* stage, int r, int nbias,
                                                                   float* grad_c, int accumulate_c,
                                                                   float* grad_bias) {
  __shared__ float red[256];
  const int b = blockIdx.x, t = threadIdx.x;
  red[t] = stage[(int64_t)t * (r + nbias) + b];  // kFinBlocks == blockDim.x rows
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) red[t] += red[t + o];
    __syncthreads();
  }
  if (t == 0) {
    if (b < r) {
      if (grad_c) grad_c[b] = accumulate_c ? grad_c[b] + red[0] : red[0];
    } else if (grad_bias) {
      grad_bias[b - r] = red[0];
    }
  }
}

// Small problems in one launch: workgroup c sums output column c over every
// partial row (c < r) or row sum (the bias columns), strided by thread, then
// by a fixed tree.  Rows past the end add zeros (no reads).
__global__ __launch_bounds__(256) void finalize_direct_kernel(const float* part_c, int nparts, int r,
                                                              const float* rowsum, int64_t nrows, int nbias,
                                                              float* grad_c, int accumulate_c, float* grad_bias) {
  __shared__ float red[256];
  const int b = blockIdx.x, t = threadIdx.x;
  // eight loads in flight per thread, added in index order
  constexpr int kB = 8;
  const bool bias_col = b >= r;
  const int64_t n = bias_col ? nrows : nparts;
  const float* src = bias_col ? rowsum + (b - r) : part_c + b;
  const int64_t stride = bias_col ? nbias : r;
  float s = 0.f;
  for (int64_t p0 = t; p0 < n; p0 += 256 * kB) {
    float v[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) v[u] = p0 + 256 * u < n ? src[(p0 + 256 * u) * stride] : 0.f;
#pragma unroll
    for (int u = 0; u < kB; ++u) s += v[u];
  }
  red[t] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) red[t] += red[t + o];
    __syncthreads();
  }
  if (t == 0) {
    if (b < r) {
      if (grad_c) grad_c[b] = accumulate_c ? grad_c[b] + red[0] : red[0];
    } else if (grad_bias) {
      grad_bias[b - r] = red[0];
    }
  }
}
constexpr int kFinDirectParts = 4096;   // partial rows summed by one workgroup at most
constexpr int64_t kFinDirectRows = 16384;  // row sums likewise

int launch_finalize_small_grads(const float* part_c, int nparts, int r, float* grad_c, int accumulate_c,
                                const float* rowsum, int64_t nrows, float* grad_bias, float* stage,
                                hipStream_t stream, int nbias) {
  JN_REQUIRE(r >= 1 && r <= kMaxRank, kUnsupported, "rank must be in [1, %d]", kMaxRank);
  JN_REQUIRE(nbias >= 1 && nbias <= kMaxHeads, kUnsupported, "1..%d bias columns", kMaxHeads);
  static_assert(kFinBlocks == 256, "the second stage maps one thread per stage row");
  if (nparts <= kFinDirectParts && nrows <= kFinDirectRows) {
    JN_PROFILE("finalize_direct_kernel", stream);
    hipLaunchKernelGGL(finalize_direct_kernel, dim3(r + nbias), dim3(256), 0, stream, part_c, nparts, r, rowsum,
                       nrows, nbias, grad_c, accumulate_c, grad_bias);
    JN_LAUNCH_CHECK();
    return kOk;
  }
  {
    JN_PROFILE("finalize_partials_kernel", stream);
    hipLaunchKernelGGL(finalize_partials_kernel, dim3(kFinBlocks), dim3(256), 0, stream, part_c, nparts, r, rowsum,
                       nrows, nbias, stage);
    JN_LAUNCH_CHECK();
  }
  JN_PROFILE("finalize_small_grads_kernel", stream);
  hipLaunchKernelGGL(finalize_small_grads_kernel, dim3(r + nbias), dim3(256), 0, stream, stage, r, nbias, grad_c,
                     accumulate_c, grad_bias);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
