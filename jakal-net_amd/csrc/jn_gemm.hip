// fp32 MFMA GEMM for the low-rank projections and their gradients (gfx950).
//
//   forward  P  = X  . [U;V]^T     (M = B*N rows, N = 2r, K = in_dim)   "NT"
//   backward dX = dP . [U;V]       (M = B*N, N = in_dim, K = 2r)         "NN"
//   backward dW = dP^T . X         (M = 2r, N = in_dim, K = B*N, split-K) "TN"
//
// The two weight matrices U (target projection) and V (source projection)
// stay separate buffers: the B-operand loader switches pointer at `b_split`
// along N (NT) or K (NN), so no concatenated copy is needed.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, workgroup tile 64x64, K staged
// through LDS in slices of 16 (double buffered, register prefetch).  Each wave
// owns a 32x32 block = 2x2 tiles of v_mfma_f32_16x16x4f32; lane group l/16
// owns a 4-wide k sub-slice so operand fetches are single ds_read_b128s.
#include "jn_internal.hpp"

namespace jakal {

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const float* A;
  int64_t lda;
  const float* B0;
  const float* B1;
  int64_t ldb;
  int b_split;
  float* C;
  int64_t ldc;
  const float* addend;  // optional, same indexing as C
  int64_t ld_add;
  int M, N, K;
  int k_chunk;             // K range per blockIdx.z (split-K)
  int64_t c_split_stride;  // C offset per blockIdx.z
  // batched mode (batch > 1): blockIdx.z is the batch index (no split-K)
  int batch;
  int64_t a_bs, b_bs, c_bs, add_bs;  // per-batch element strides
  const float* a_kscale;   // optional: A(m, k) *= a_kscale[k]
  const float* c_nscale;   // optional: C(m, n) = acc * c_nscale[n] (+ addend)
};

constexpr int kGBM = 64, kGBN = 64, kGBK = 16, kGStride = kGBK + 4;

__device__ __forceinline__ bool aligned16(const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// A(m,k): A_KC -> A[m*lda + k] else A[k*lda + m]
// B(k,n): B_KC -> Bsel(n)[n'*ldb + k] (split along n), else Bsel(k)[k'*ldb + n] (split along k)
// USE tags the call site (GemmUse): the code is the same for a given layout,
// but every use gets its own kernel symbol so profilers attribute time and
// traffic per use.
template <bool A_KC, bool B_KC, int USE>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgs g) {
  __shared__ __align__(16) float sA[2][kGBM * kGStride];
  __shared__ __align__(16) float sB[2][kGBN * kGStride];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, col = lane & 15;

  const int m0 = blockIdx.y * kGBM;
  const int n0 = blockIdx.x * kGBN;
  const bool batched = g.batch > 1;
  const int split = batched ? 0 : blockIdx.z;
  const int64_t bz = batched ? blockIdx.z : 0;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.K, kbeg + g.k_chunk);
  const float* gA = g.A + bz * g.a_bs;
  const float* gB0 = g.B0 + bz * g.b_bs;
  const float* gB1 = g.B1 + bz * g.b_bs;
  const float* gadd = g.addend ? g.addend + bz * g.add_bs : nullptr;
  float* C = g.C + (int64_t)split * g.c_split_stride + bz * g.c_bs;

  // Each thread moves 4 A values and 4 B values per K slice.
  float ra[4], rb[4];

  auto load_slice = [&](int k0) {
    // ---- A ----
    if (A_KC) {
      int m = m0 + tid / 4, kq = k0 + (tid % 4) * 4;
      const float* p = gA + (int64_t)m * g.lda + kq;
      if (m < g.M && kq + 3 < kend && aligned16(p)) {
        float4 v = *reinterpret_cast<const float4*>(p);
        ra[0] = v.x; ra[1] = v.y; ra[2] = v.z; ra[3] = v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[q] = (m < g.M && kq + q < kend) ? p[q] : 0.0f;
      }
    } else {
      int kk = k0 + tid / 16, mq = m0 + (tid % 16) * 4;
      const float* p = gA + (int64_t)kk * g.lda + mq;
      if (kk < kend && mq + 3 < g.M && aligned16(p)) {
        float4 v = *reinterpret_cast<const float4*>(p);
        ra[0] = v.x; ra[1] = v.y; ra[2] = v.z; ra[3] = v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[q] = (kk < kend && mq + q < g.M) ? p[q] : 0.0f;
      }
    }
    if (g.a_kscale) {
      if (A_KC) {
        const int kq = k0 + (tid % 4) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[q] *= (kq + q < kend) ? g.a_kscale[kq + q] : 0.0f;
      } else {
        const int kk = k0 + tid / 16;
        const float sc = kk < kend ? g.a_kscale[kk] : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[q] *= sc;
      }
    }
    // ---- B ----
    if (B_KC) {
      int n = n0 + tid / 4, kq = k0 + (tid % 4) * 4;
      const float* base = (n < g.b_split) ? gB0 + (int64_t)n * g.ldb : gB1 + (int64_t)(n - g.b_split) * g.ldb;
      const float* p = base + kq;
      if (n < g.N && kq + 3 < kend && aligned16(p)) {
        float4 v = *reinterpret_cast<const float4*>(p);
        rb[0] = v.x; rb[1] = v.y; rb[2] = v.z; rb[3] = v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) rb[q] = (n < g.N && kq + q < kend) ? p[q] : 0.0f;
      }
    } else {
      int kk = k0 + tid / 16, nq = n0 + (tid % 16) * 4;
      const float* base = (kk < g.b_split) ? gB0 + (int64_t)kk * g.ldb : gB1 + (int64_t)(kk - g.b_split) * g.ldb;
      const float* p = base + nq;
      if (kk < kend && nq + 3 < g.N && aligned16(p)) {
        float4 v = *reinterpret_cast<const float4*>(p);
        rb[0] = v.x; rb[1] = v.y; rb[2] = v.z; rb[3] = v.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) rb[q] = (kk < kend && nq + q < g.N) ? p[q] : 0.0f;
      }
    }
  };
  auto store_slice = [&](int buf) {
    if (A_KC) {
      float* d = &sA[buf][(tid / 4) * kGStride + (tid % 4) * 4];
      *reinterpret_cast<float4*>(d) = make_float4(ra[0], ra[1], ra[2], ra[3]);
    } else {
      int kk = tid / 16, mq = (tid % 16) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) sA[buf][(mq + q) * kGStride + kk] = ra[q];
    }
    if (B_KC) {
      float* d = &sB[buf][(tid / 4) * kGStride + (tid % 4) * 4];
      *reinterpret_cast<float4*>(d) = make_float4(rb[0], rb[1], rb[2], rb[3]);
    } else {
      int kk = tid / 16, nq = (tid % 16) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) sB[buf][(nq + q) * kGStride + kk] = rb[q];
    }
  };

  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nslices = (kend - kbeg + kGBK - 1) / kGBK;
  if (nslices > 0) {
    load_slice(kbeg);
    store_slice(0);
  }
  __syncthreads();

  for (int s = 0; s < nslices; ++s) {
    const int cur = s & 1;
    if (s + 1 < nslices) load_slice(kbeg + (s + 1) * kGBK);

    float4 av[2], bv[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      av[t] = *reinterpret_cast<const float4*>(&sA[cur][(wm * 32 + t * 16 + col) * kGStride + grp * 4]);
      bv[t] = *reinterpret_cast<const float4*>(&sB[cur][(wn * 32 + t * 16 + col) * kGStride + grp * 4]);
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].x, bv[nt].x, acc[mt][nt], 0, 0, 0);
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].y, bv[nt].y, acc[mt][nt], 0, 0, 0);
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].z, bv[nt].z, acc[mt][nt], 0, 0, 0);
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].w, bv[nt].w, acc[mt][nt], 0, 0, 0);
      }

    if (s + 1 < nslices) store_slice(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 4*grp+v of each 16x16 tile, column col.
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        int m = m0 + wm * 32 + mt * 16 + grp * 4 + v;
        int n = n0 + wn * 32 + nt * 16 + col;
        if (m < g.M && n < g.N) {
          float x = acc[mt][nt][v];
          if (g.c_nscale) x *= g.c_nscale[n];
          if (gadd) x += gadd[(int64_t)m * g.ld_add + n];
          C[(int64_t)m * g.ldc + n] = x;
        }
      }
}

// Sum split-K partials in a fixed order; rows < m_split go to out0, the rest to out1.
// out = sum over splits of part[z] (fixed order).  A workgroup owns 64
// consecutive outputs; wave w sums splits z = w, w + 4, ... for its lane's
// output, then the four partials are added in wave order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int splits, int M, int N,
                                                            int64_t split_stride, float* out0, float* out1,
                                                            int m_split) {
  __shared__ float red[4][64];
  const int lane = lane_id(), wave = wave_id();
  const int64_t total = (int64_t)M * N;
  const int64_t e = (int64_t)blockIdx.x * 64 + lane;
  float s = 0.0f;
  if (e < total)
    for (int z = wave; z < splits; z += 4) s += part[z * split_stride + e];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && e < total) {
    const float t = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    const int m = (int)(e / N), n = (int)(e % N);
    if (m < m_split) out0[(int64_t)m * N + n] = t;
    else out1[(int64_t)(m - m_split) * N + n] = t;
  }
}

// Layout (A k-contiguous, B k-contiguous) and timer label of every GEMM use.
struct GemmUseInfo {
  bool a_kc, b_kc;
  const char* name;
};
constexpr GemmUseInfo kGemmUses[] = {
    {true, true, "gemm_f32_kernel<project>"},
    {true, false, "gemm_f32_kernel<grad_input>"},
    {false, false, "gemm_f32_kernel<grad_weight>"},
    {true, true, "gemm_f32_kernel<dense_scores>"},
    {true, false, "gemm_f32_kernel<dense_aggregate>"},
    {true, true, "gemm_f32_kernel<dense_edge_grad>"},
    {false, false, "gemm_f32_kernel<dense_value_grad>"},
    {true, false, "gemm_f32_kernel<dense_target_grad>"},
    {false, false, "gemm_f32_kernel<dense_source_grad>"},
};

template <int USE>
static void launch_use(const GemmArgs& g, dim3 grid, hipStream_t stream) {
  constexpr GemmUseInfo u = kGemmUses[USE];
  hipLaunchKernelGGL((gemm_f32_kernel<u.a_kc, u.b_kc, USE>), grid, dim3(256), 0, stream, g);
}

int launch_gemm(const GemmArgs& g, GemmUse use, int splits, hipStream_t stream) {
  JN_REQUIRE(g.M >= 0 && g.N >= 0 && g.K >= 0, kInvalidArgument, "negative GEMM extent");
  if (g.M == 0 || g.N == 0) return kOk;
  JN_REQUIRE(g.batch <= 1 || splits == 1, kInvalidArgument, "batched GEMM has no split-K");
  JN_REQUIRE(g.batch < 65536 && splits < 65536, kUnsupported, "GEMM batch or split count too large");
  JN_REQUIRE((g.M + kGBM - 1) / kGBM < 65536, kUnsupported, "GEMM M extent too large");
  dim3 grid((g.N + kGBN - 1) / kGBN, (g.M + kGBM - 1) / kGBM, g.batch > 1 ? g.batch : splits);
  JN_PROFILE(kGemmUses[use].name, stream);
  switch (use) {
    case kGemmProject: launch_use<kGemmProject>(g, grid, stream); break;
    case kGemmGradInput: launch_use<kGemmGradInput>(g, grid, stream); break;
    case kGemmGradWeight: launch_use<kGemmGradWeight>(g, grid, stream); break;
    case kGemmDenseScores: launch_use<kGemmDenseScores>(g, grid, stream); break;
    case kGemmDenseAggregate: launch_use<kGemmDenseAggregate>(g, grid, stream); break;
    case kGemmDenseEdgeGrad: launch_use<kGemmDenseEdgeGrad>(g, grid, stream); break;
    case kGemmDenseValueGrad: launch_use<kGemmDenseValueGrad>(g, grid, stream); break;
    case kGemmDenseTargetGrad: launch_use<kGemmDenseTargetGrad>(g, grid, stream); break;
    case kGemmDenseSourceGrad: launch_use<kGemmDenseSourceGrad>(g, grid, stream); break;
    default: JN_REQUIRE(false, kInvalidArgument, "unknown GEMM use %d", (int)use);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

// Batched C_b = op(A_b) . op(B_b) for b < batch (see BatchedGemm).
int gemm_batched(const BatchedGemm& m, GemmUse use, hipStream_t stream) {
  JN_REQUIRE(use >= kGemmDenseScores && use <= kGemmDenseSourceGrad && m.a_kcontig == kGemmUses[use].a_kc &&
                 m.b_kcontig == kGemmUses[use].b_kc,
             kInvalidArgument, "batched GEMM layout does not match its use");
  GemmArgs g{};
  g.A = m.A; g.lda = m.lda; g.a_bs = m.a_bs;
  g.B0 = m.B; g.B1 = m.B; g.ldb = m.ldb; g.b_bs = m.b_bs; g.b_split = 1 << 30;
  g.C = m.C; g.ldc = m.ldc; g.c_bs = m.c_bs;
  g.addend = m.addend; g.ld_add = m.ld_add; g.add_bs = m.add_bs;
  g.M = m.M; g.N = m.N; g.K = m.K;
  g.k_chunk = m.K; g.c_split_stride = 0;
  g.batch = m.batch;
  g.a_kscale = m.a_kscale;
  g.c_nscale = m.c_nscale;
  return launch_gemm(g, use, 1, stream);
}

// C[M][N] = X[M][K] . [W0;W1]^T with W0 rows [0, split) and W1 rows [split, N).
int gemm_project(const float* X, int64_t ldx, const float* W0, const float* W1, int split, int64_t ldw, float* C,
                 int64_t ldc, int M, int N, int K, hipStream_t stream) {
  GemmArgs g{};
  g.A = X; g.lda = ldx;
  g.B0 = W0; g.B1 = W1; g.ldb = ldw; g.b_split = split;
  g.C = C; g.ldc = ldc;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = K; g.c_split_stride = 0;
  return launch_gemm(g, kGemmProject, 1, stream);
}

// dX[M][N] = dP[M][K] . [W0;W1] (+ addend), W0 rows [0, split) of K.
int gemm_grad_input(const float* dP, int64_t ldp, const float* W0, const float* W1, int split, int64_t ldw,
                    const float* addend, int64_t ld_add, float* dX, int64_t ldx, int M, int N, int K,
                    hipStream_t stream) {
  GemmArgs g{};
  g.A = dP; g.lda = ldp;
  g.B0 = W0; g.B1 = W1; g.ldb = ldw; g.b_split = split;
  g.C = dX; g.ldc = ldx;
  g.addend = addend; g.ld_add = ld_add;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = K; g.c_split_stride = 0;
  return launch_gemm(g, kGemmGradInput, 1, stream);
}

size_t gemm_grad_weight_workspace(int M, int N, int K) {
  int splits = K >= 4096 ? 64 : (K >= 512 ? 8 : 1);
  return (size_t)splits * M * N * sizeof(float);
}

// dW[M][N] = dP^T . X with dP [K][M] (row stride ldp), X [K][N] (row stride ldx).
// Rows [0, m_split) of dW go to out0, the rest to out1.  Deterministic split-K.
int gemm_grad_weight(const float* dP, int64_t ldp, const float* X, int64_t ldx, float* out0, float* out1, int m_split,
                     int M, int N, int K, float* partial, hipStream_t stream) {
  int splits = K >= 4096 ? 64 : (K >= 512 ? 8 : 1);
  int k_chunk = (K + splits - 1) / splits;
  k_chunk = (k_chunk + kGBK - 1) / kGBK * kGBK;
  GemmArgs g{};
  g.A = dP; g.lda = ldp;
  g.B0 = X; g.B1 = X; g.ldb = ldx; g.b_split = 1 << 30;
  g.C = partial; g.ldc = N;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = k_chunk; g.c_split_stride = (int64_t)M * N;
  int rc = launch_gemm(g, kGemmGradWeight, splits, stream);
  if (rc != kOk) return rc;
  const int64_t total = (int64_t)M * N;
  JN_REQUIRE((total + 63) / 64 < (1LL << 31), kUnsupported, "weight gradient too large");
  const int blocks = (int)((total + 63) / 64);
  JN_PROFILE("splitk_reduce_kernel", stream);
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partial, splits, M, N,
                     (int64_t)M * N, out0, out1, m_split);
  JN_LAUNCH_CHECK();
  return kOk;
}

}  // namespace jakal
