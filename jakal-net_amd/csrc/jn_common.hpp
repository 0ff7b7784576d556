// Shared device/host helpers for the Jakal-Net MI355X (gfx950) hot path.
//
// Everything here is written for CDNA4 wave64 execution: one wavefront = 64
// lanes, cross-lane traffic through ds_bpermute / readlane, fp32 MFMA tiles
// from __builtin_amdgcn_mfma_f32_16x16x4f32.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

namespace jakal {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Host-side error channel.  Every C-ABI entry point returns 0 on success and a
// non-zero code on failure; the message is kept per host thread and read back
// through jn_last_error().
// ---------------------------------------------------------------------------
enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kUnsupported = 2,
  kHipError = 3,
  kWorkspaceTooSmall = 4,
};

void set_error(const char* fmt, ...);
const char* last_error();

#define JN_REQUIRE(cond, code, ...)   \
  do {                                \
    if (!(cond)) {                    \
      ::jakal::set_error(__VA_ARGS__);   \
      return (code);                  \
    }                                 \
  } while (0)

#define JN_HIP_TRY(expr)                                                        \
  do {                                                                          \
    hipError_t jn_err__ = (expr);                                               \
    if (jn_err__ != hipSuccess) {                                               \
      ::jakal::set_error("%s failed: %s", #expr, hipGetErrorString(jn_err__));     \
      return ::jakal::kHipError;                                                   \
    }                                                                           \
  } while (0)

#define JN_LAUNCH_CHECK()                                                       \
  do {                                                                          \
    hipError_t jn_err__ = hipGetLastError();                                    \
    if (jn_err__ != hipSuccess) {                                               \
      ::jakal::set_error("kernel launch failed at %s:%d: %s", __FILE__, __LINE__,  \
                      hipGetErrorString(jn_err__));                             \
      return ::jakal::kHipError;                                                   \
    }                                                                           \
  } while (0)

// Optional per-kernel timing with HIP events, off unless jn_profile_enable(1)
// was called.  A scope records an event on `stream` before and after the
// launch it encloses; jn_profile_collect() reads the elapsed times back.
struct ProfileScope {
  ProfileScope(const char* name, hipStream_t stream);
  ~ProfileScope();
  ProfileScope(const ProfileScope&) = delete;
  ProfileScope& operator=(const ProfileScope&) = delete;
  long slot;
  hipStream_t stream;
};
#define JN_PROFILE(name, stream) ::jakal::ProfileScope jn_prof_scope__((name), (stream))

// Bump allocator over a caller-provided workspace.  Offsets are 256-byte
// aligned so every carved buffer is suitable for 16-byte vector access.
struct Workspace {
  char* base;
  size_t size;
  size_t used = 0;
  bool sizing_only;

  Workspace(void* ptr, size_t bytes) : base(static_cast<char*>(ptr)), size(bytes), sizing_only(ptr == nullptr) {}

  template <typename T>
  T* take(size_t count) {
    size_t bytes = (count * sizeof(T) + 255) & ~size_t(255);
    char* p = sizing_only ? nullptr : base + used;
    used += bytes;
    return reinterpret_cast<T*>(p);
  }
  bool overflow() const { return !sizing_only && used > size; }
};

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
// Wave index within the workgroup, as a wave-uniform (scalar) value: values
// derived from it (row ids, base pointers, buffer resources) stay in SGPRs.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  int lane = lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}
__device__ __forceinline__ int shfl_xor_i(int v, int mask) {
  int lane = lane_id();
  return __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, v);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ int readlane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// Exchange with lane ^ 16 / lane ^ 32 through the gfx950 permlane swaps
// (VALU ops, no LDS round trip).
__device__ __forceinline__ int xor16_i(int v) {
  const auto p = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
  return (int)((lane_id() & 16) ? p[0] : p[1]);
}
__device__ __forceinline__ int xor32_i(int v) {
  const auto p = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return (int)((lane_id() & 32) ? p[0] : p[1]);
}

// Wave-wide reductions over DPP quad/mirror patterns plus the two permlane
// swaps; every lane receives the result.
template <typename Op>
__device__ __forceinline__ int wave_reduce_i(int v, Op op) {
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xf, 0xf, false));  // row_mirror
  v = op(v, xor16_i(v));
  v = op(v, xor32_i(v));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return (uint32_t)wave_reduce_i((int)v, [](int a, int b) { return (int)max((uint32_t)a, (uint32_t)b); });
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return (uint32_t)wave_reduce_i((int)v, [](int a, int b) { return (int)min((uint32_t)a, (uint32_t)b); });
}
__device__ __forceinline__ int wave_min_i32(int v) {
  return wave_reduce_i(v, [](int a, int b) { return min(a, b); });
}
__device__ __forceinline__ float wave_max_f(float v) {
  return __int_as_float(wave_reduce_i(__float_as_int(v), [](int a, int b) {
    return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
  }));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float xor16_f(float v) { return __int_as_float(xor16_i(__float_as_int(v))); }
__device__ __forceinline__ float xor32_f(float v) { return __int_as_float(xor32_i(__float_as_int(v))); }

// Sum over the 16 lanes of each DPP row; every lane of the row receives it.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// Sum over the wave (fixed order, identical in every lane).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += xor16_f(v);
  v += xor32_f(v);
  return v;
}

// ---- signed entmax-1.5 ------------------------------------------------------
// entmax15(z) = max(x - tau, 0)^2 with x = (z - max z) / 2 and tau such that
// the result sums to 1 (native/jakal_net_native.cpp:1133-1169).  The
// threshold is found by support refinement: start from every entry, take the
// closed-form threshold of the support S,
//   tau(S) = mean_S x - sqrt(max(0, (1 - |S| var_S x) / |S|)),
// keep the entries at or above it and repeat until the support stops changing.
// This solves the same equation as the reference's sort (whose support is the
// set of the |S| largest entries).
constexpr int kEntmaxMaxIter = 256;

__device__ __forceinline__ float entmax15_tau_of(float s1, float s2, float n) {
  const float mean = s1 / n, msq = s2 / n;
  return mean - sqrtf(fmaxf(0.0f, (1.0f - n * (msq - mean * mean)) / n));
}

// One entry per lane: returns this lane's entmax15 weight (0 where !ok).
__device__ __forceinline__ float entmax15_lane(float z, bool ok) {
  const float zmax = wave_max_f(ok ? z : -INFINITY);
  const float x = ok ? 0.5f * (z - zmax) : -INFINITY;
  float tau = -INFINITY;
  int n_prev = -1;
  for (int it = 0; it < kEntmaxMaxIter; ++it) {
    const bool in = ok && x >= tau;
    const float n = wave_sum(in ? 1.0f : 0.0f);
    if ((int)n == n_prev) break;
    n_prev = (int)n;
    tau = entmax15_tau_of(wave_sum(in ? x : 0.0f), wave_sum(in ? x * x : 0.0f), n);
  }
  const float d = ok ? fmaxf(x - tau, 0.0f) : 0.0f;
  const float p = d * d;
  const float den = wave_sum(p);
  return den > 0.0f ? p / den : 0.0f;
}

// A whole row of n entries per wavefront (lane l reads entries l, l + 64, ...
// through zf(j) >= 0): returns tau and sets zmax; the weights are then
// max(0.5 (z - zmax) - tau, 0)^2 over their sum.
template <class F>
__device__ __forceinline__ float entmax15_row_tau(F zf, int n, float& zmax) {
  const int lane = lane_id();
  float m = -INFINITY;
  for (int j = lane; j < n; j += kWave) m = fmaxf(m, zf(j));
  m = wave_max_f(m);
  zmax = m;
  float tau = -INFINITY;
  int n_prev = -1;
  for (int it = 0; it < kEntmaxMaxIter; ++it) {
    float s1 = 0.0f, s2 = 0.0f, c = 0.0f;
    for (int j = lane; j < n; j += kWave) {
      const float x = 0.5f * (zf(j) - m);
      if (x >= tau) {
        s1 += x;
        s2 += x * x;
        c += 1.0f;
      }
    }
    c = wave_sum(c);
    if ((int)c == n_prev) break;
    n_prev = (int)c;
    tau = entmax15_tau_of(wave_sum(s1), wave_sum(s2), c);
  }
  return tau;
}

// Backward of sign(s) * entmax15(|s|) (native/jakal_net_native.cpp:1183-1205):
// with u = sqrt(|r|) for the lane's output r, gi = sign(s) g u,
//   grad s = (gi - u * sum(gi) / sum(u)) * sign(s).
__device__ __forceinline__ float signed_entmax15_backward_lane(float s, float r, float g) {
  const float sg = (s > 0.f) ? 1.f : ((s < 0.f) ? -1.f : 0.f);
  const float u = sqrtf(fabsf(r));
  const float gi = g * sg * u;
  const float us = wave_sum(u);
  const float corr = us > 0.0f ? wave_sum(gi) / us : 0.0f;
  return (gi - corr * u) * sg;
}

// Workgroups are dispatched round-robin over the 8 XCDs (hardware id % 8).
// Map the hardware id to a logical tile so that each XCD runs a contiguous
// range of logical tiles (same batch element, same gathered rows) and they
// share its L2.
__device__ __forceinline__ int xcd_swizzle(int bid, int nblk) {
  constexpr int kXcd = 8;
  if (nblk % kXcd != 0) return bid;
  return (bid % kXcd) * (nblk / kXcd) + bid / kXcd;
}

// Raw buffer resource over [base, base + bytes): a load at a byte offset past
// `bytes` returns zeros, which masks lanes without a branch.  The base must be
// wave-uniform; offsets are 32-bit (callers keep bytes < 2^31).
constexpr uint32_t kOobOffset = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}
__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}

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

// W consecutive floats at a byte offset of a buffer (zeros when out of range).
template <int W>
__device__ __forceinline__ float4 buf_load_w(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  if constexpr (W == 4) return buf_load4(r, byte_off);
  else return make_float4(buf_load1(r, byte_off), 0.f, 0.f, 0.f);
}

// ---------------------------------------------------------------------------
// Value-row packs: a lane moves W consecutive elements of a value row of
// element type T, held as W floats.  fp32 rows: W = 4 (one 16-byte load) or 1;
// bf16 rows: W = 8 (one 16-byte load) or 1.  bf16 widens exactly; a store
// rounds to nearest even (v_cvt_pk_bf16_f32).
// ---------------------------------------------------------------------------
typedef __bf16 bf16_t;

template <int W>
struct Pack {
  float v[W];
};

__device__ __forceinline__ void unpack_bf16x2(uint32_t x, float& lo, float& hi) {
  lo = __uint_as_float(x << 16);
  hi = __uint_as_float(x & 0xffff0000u);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (bf16_t)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (bf16_t)hi) << 16);
}

template <typename T, int W>
__device__ __forceinline__ Pack<W> unpack16(uint4 x) {
  Pack<W> r;
  if constexpr (sizeof(T) == 4) {
    r.v[0] = __uint_as_float(x.x);
    r.v[1] = __uint_as_float(x.y);
    r.v[2] = __uint_as_float(x.z);
    r.v[3] = __uint_as_float(x.w);
  } else {
    unpack_bf16x2(x.x, r.v[0], r.v[1]);
    unpack_bf16x2(x.y, r.v[2], r.v[3]);
    unpack_bf16x2(x.z, r.v[4], r.v[5]);
    unpack_bf16x2(x.w, r.v[6], r.v[7]);
  }
  return r;
}

template <typename T, int W>
__device__ __forceinline__ Pack<W> pack_zero() {
  Pack<W> r;
#pragma unroll
  for (int i = 0; i < W; ++i) r.v[i] = 0.f;
  return r;
}

template <typename T, int W>
__device__ __forceinline__ Pack<W> load_pack(const T* p) {
  static_assert(W == 1 || W * sizeof(T) == 16, "a pack is one element or 16 bytes");
  if constexpr (W == 1) {
    Pack<1> r;
    r.v[0] = (float)p[0];
    return r;
  } else {
    return unpack16<T, W>(*reinterpret_cast<const uint4*>(p));
  }
}

template <typename T, int W>
__device__ __forceinline__ void store_pack(T* p, const Pack<W>& x) {
  if constexpr (W == 1) {
    p[0] = (T)x.v[0];
  } else if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(x.v[0], x.v[1], x.v[2], x.v[3]);
  } else {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(x.v[0], x.v[1]), pack_bf16x2(x.v[2], x.v[3]),
                                              pack_bf16x2(x.v[4], x.v[5]), pack_bf16x2(x.v[6], x.v[7]));
  }
}

// Streaming accesses (data read or written once): non-temporal, so they do
// not displace data that is reused (gathered rows, GEMM operands) from L2.
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store_nt16(void* p, uint4 x) {
  u32x4_nt v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4_nt*>(p));
}

typedef unsigned int u32x2_nt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 load_nt8(const void* p) {
  const u32x2_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_nt*>(p));
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ void store_nt8(void* p, uint2 x) {
  u32x2_nt v = {x.x, x.y};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2_nt*>(p));
}

// W elements at a byte offset of a buffer (zeros when out of range).
template <typename T, int W>
__device__ __forceinline__ Pack<W> buf_load_pack(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  if constexpr (W == 1) {
    Pack<1> x;
    if constexpr (sizeof(T) == 4) x.v[0] = buf_load1(r, byte_off);
    else x.v[0] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0) << 16);
    return x;
  } else {
    return unpack16<T, W>(__builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0)));
  }
}

template <int W>
__device__ __forceinline__ void fma_pack(Pack<W>& acc, float c, const Pack<W>& v) {
#pragma unroll
  for (int i = 0; i < W; ++i) acc.v[i] += c * v.v[i];
}
template <int W>
__device__ __forceinline__ float dot_pack(const Pack<W>& a, const Pack<W>& b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) s += a.v[i] * b.v[i];
  return s;
}
template <int W>
__device__ __forceinline__ Pack<W> add_pack(const Pack<W>& a, const Pack<W>& b) {
  Pack<W> r;
#pragma unroll
  for (int i = 0; i < W; ++i) r.v[i] = a.v[i] + b.v[i];
  return r;
}

__device__ __forceinline__ float sign_f(float s) { return (s > 0.f) ? 1.f : ((s < 0.f) ? -1.f : 0.f); }

// True when every present edge of the wavefront's row (lanes with `present`)
// has a score of one strict sign.  The row-normalising compressions (signed
// |s| softmax, signed entmax-1.5) then do not change when all of the row's
// scores shift together, so the row's contribution to the bias gradient,
// sum_e g_s[e], is exactly 0 (its fp32 sum would only be rounding noise).
__device__ __forceinline__ bool row_one_sign(bool present, float s) {
  const uint64_t live = __ballot(present);
  return __ballot(present && s > 0.f) == live || __ballot(present && s < 0.f) == live;
}

// Edges of a row processed four at a time by the wave's 16-lane groups (group g
// takes edge 4i + g in iteration i): lane L (< 64) takes the edge held by group
// L % 4 in iteration L / 4.
__device__ __forceinline__ int edge_owner_lane(int lane) { return (lane & 3) * 16 + (lane >> 2); }

// Make LDS writes of this wavefront visible to later LDS reads of the same
// wavefront by other lanes (compiler + hardware ordering, no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Edge compression applied to a selected score (reference: propagation.py:85-88
// softsign; transition softmax is applied per row elsewhere).
__device__ __forceinline__ float softsign_f(float s) { return s / (1.0f + fabsf(s)); }
__device__ __forceinline__ float softsign_grad_f(float s) {
  float d = 1.0f + fabsf(s);
  return 1.0f / (d * d);
}

// "a ranks before b" in a descending top-k with ties toward the lower index.
__device__ __forceinline__ bool ranks_before(float as, int ai, float bs, int bi) {
  return (as > bs) || (as == bs && ai < bi);
}

// ---- edge-list rows ---------------------------------------------------------
// An edge list is (idx[row, e], score[row, e]), e < k, idx < 0 for an absent
// edge; a row's coefficients are its compressed scores.

// Row statistics for the signed |s| softmax (max |s| and 1/sum exp).
__device__ __forceinline__ void row_abs_softmax_stats(const int32_t* idx, const float* score, int64_t row, int k,
                                                      float& row_max, float& row_inv_sum) {
  const int lane = lane_id();
  float m = -INFINITY;
  // (an edge's score loads beside its index: the slot exists for absent edges too)
  for (int e = lane; e < k; e += kWave) {
    const int32_t j = idx[row * k + e];
    const float a = fabsf(score[row * k + e]);
    if (j >= 0) m = fmaxf(m, a);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = fmaxf(m, shfl_xor_f(m, s));
  float sum = 0.0f;
  for (int e = lane; e < k; e += kWave) {
    const int32_t j = idx[row * k + e];
    const float a = fabsf(score[row * k + e]);
    if (j >= 0) sum += __expf(a - m);
  }
  sum = wave_sum(sum);
  row_max = m;
  row_inv_sum = sum > 0.f ? 1.0f / sum : 0.0f;
}

// Statistics of a row's compression, for rows of any length: kind 1:
// a = max |s|, b = 1 / sum exp(|s| - a); kind 2: a = max |s|, b = the entmax
// threshold tau of x = (|s| - a) / 2 (support refinement, as entmax15_lane),
// c = the sum of the weights max(x - tau, 0)^2 (1 up to rounding).  Lane l
// takes the row's edges l, l + 64, ...; absent edges do not count.  For rows
// of at most 64 edges the sums are those of entmax15_lane, term for term.
struct RowStats {
  float a = 0.f, b = 0.f, c = 0.f;
};

__device__ __forceinline__ RowStats row_compress_stats(const int32_t* idx, const float* score, int64_t row, int k,
                                                       int compress) {
  RowStats st;
  if (compress == 1) {
    row_abs_softmax_stats(idx, score, row, k, st.a, st.b);
  } else if (compress == 2) {
    const int lane = lane_id();
    float m = -INFINITY;
    for (int e = lane; e < k; e += kWave) {
      const int32_t j = idx[row * k + e];
      const float a = fabsf(score[row * k + e]);
      if (j >= 0) m = fmaxf(m, a);
    }
    m = wave_max_f(m);
    float tau = -INFINITY;
    int n_prev = -1;
    for (int it = 0; it < kEntmaxMaxIter; ++it) {
      float s1 = 0.f, s2 = 0.f, n = 0.f;
      for (int e = lane; e < k; e += kWave) {
        const int32_t j = idx[row * k + e];
        const float x = 0.5f * (fabsf(score[row * k + e]) - m);
        if (j < 0) continue;
        if (x >= tau) {
          s1 += x;
          s2 += x * x;
          n += 1.0f;
        }
      }
      n = wave_sum(n);
      if ((int)n == n_prev) break;
      n_prev = (int)n;
      tau = entmax15_tau_of(wave_sum(s1), wave_sum(s2), n);
    }
    float den = 0.f;
    for (int e = lane; e < k; e += kWave) {
      const int32_t j = idx[row * k + e];
      const float d = fmaxf(0.5f * (fabsf(score[row * k + e]) - m) - tau, 0.0f);
      if (j < 0) continue;
      den += d * d;
    }
    st.a = m;
    st.b = tau;
    st.c = wave_sum(den);
  }
  return st;
}

// Compress kind whose "scores" are the edge coefficients themselves (edge
// lists that arrive already compressed); it needs no row statistics.
constexpr int kCoefGiven = 3;

// Coefficient of edge e0 + lane of a row (0 for absent edges), given the
// row's statistics (row_compress_stats).
__device__ __forceinline__ void row_coefficients(const int32_t* idx, const float* score, int64_t row, int k, int e0,
                                                 int compress, const RowStats& st, int& j, float& c, float& s) {
  const int e = e0 + lane_id();
  j = -1;
  c = 0.0f;
  s = 0.0f;
  if (e < k) {
    // the score loads beside the index (its slot exists for absent edges too),
    // so the row's gathers wait for one memory round trip, not two
    j = idx[row * k + e];
    const float se = score[row * k + e];
    if (j >= 0) {
      s = se;
      if (compress == 0) {
        c = softsign_f(s);
      } else if (compress == kCoefGiven) {
        c = s;
      } else if (compress == 1) {
        c = sign_f(s) * __expf(fabsf(s) - st.a) * st.b;
      } else {
        const float d = fmaxf(0.5f * (fabsf(s) - st.a) - st.b, 0.0f);
        c = st.c > 0.0f ? sign_f(s) * (d * d / st.c) : 0.0f;
      }
    }
  }
}

}  // namespace jakal
