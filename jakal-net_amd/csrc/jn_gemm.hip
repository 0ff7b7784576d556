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
// bf16 layers: the *_bf16 uses read X (the projection's A, the weight
// gradient's B) as bf16 and write dX (and read its addend) as bf16.  Operands
// are widened to fp32 on their way into LDS and multiplied on the fp32 MFMA:
// a bf16 x fp32 product is exact in fp32, so the results are those of
// bf16-in/fp32-accumulate arithmetic with half the bytes of X moved.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, workgroup tile 128x128 (64x64
// for small extents), K staged through LDS in slices of 16 (double buffered,
// register prefetch).  Each wave owns a 64x64 (32x32) block of
// v_mfma_f32_16x16x4f32 tiles; lane group l/16 owns a 4-wide k sub-slice so
// operand fetches are single ds_read_b128s.
#include <atomic>
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
  const float* c_mscale;   // optional: C(m, n) *= c_mscale[m] (before the addend)
  int64_t ks_bs, ms_bs;    // per-batch element strides of a_kscale and c_mscale
  // Softsign epilogue of the dense uses (epi != 0; batched over square N x N
  // score matrices, m and n index rows and columns of one batch element):
  //   dense_scores:    C = softsign(acc + bias),                  part += C ps[n]
  //   dense_edge_grad: C = (acc + gds[m] ps[n]) (1 - |E[m, n]|)^2, part += C
  // with C = 0 where a causal row does not keep source n (n > m).  part holds
  // one sum per row and 32-column block: epi_part[(b M + m) P + n / 32], P =
  // ceil(N / 32), each written once, in a fixed order.
  int epi, epi_causal;     // epi_causal: also skips the K loop of tiles wholly above the diagonal
  int causal_k;            // kCausalK*: per-tile K range of a causal square product (BatchedGemm)
  const float* epi_bias;   // scalar or null
  const float* epi_ps;     // [batch, N]
  const float* epi_gds;    // [batch, M]
  const float* epi_E;      // indexed like C
  float* epi_part;
  // Head-max fold of multi-head scores (BatchedGemm::fold, score uses only).
  int fold, fold_head;
  const float* fold_bias;  // this head's bias (scalar) or null
  uint8_t* fold_heads;     // winning head per element (bytes indexed like C) or null
  // Head mask of the A operand (BatchedGemm::a_heads, score-gradient uses only).
  const uint8_t* a_heads;
  int a_head;
};

constexpr int kEpiBlock = 32;  // columns per epilogue partial sum

// Uses whose epilogue may fold a head's scores into a running max, and uses
// whose A operand (a score gradient) may be masked to one head's pairs.
constexpr bool gemm_use_fold(int use) {
  return use == kGemmDenseScores || use == kGemmRouteLogits || use == kGemmSelectScores;
}
constexpr bool gemm_use_amask(int use) {
  return use == kGemmDenseTargetGrad || use == kGemmDenseSourceGrad || use == kGemmRouteSourceGrad ||
         use == kGemmRouteTargetGrad;
}

// One element of the head-max fold: y = acc + this head's bias; the first
// head (fold == 1) stores y, a later head (fold == 2) stores y only where it
// exceeds the stored value (ties keep the earlier head) and records itself as
// the winning head.
__device__ __forceinline__ void fold_store(const GemmArgs& g, float acc, float* c, uint8_t* hd) {
  const float y = acc + (g.fold_bias ? g.fold_bias[0] : 0.0f);
  if (g.fold == 1) {
    *c = y;
    if (hd) *hd = (uint8_t)g.fold_head;
  } else if (y > *c) {
    *c = y;
    if (hd) *hd = (uint8_t)g.fold_head;
  }
}

// Four consecutive elements of the fold (c float4 aligned, hd 4-byte aligned).
__device__ __forceinline__ void fold_store4(const GemmArgs& g, float4 x, float* c, uint8_t* hd) {
  const float b = g.fold_bias ? g.fold_bias[0] : 0.0f;
  x.x += b; x.y += b; x.z += b; x.w += b;
  const uint32_t h = (uint32_t)g.fold_head * 0x01010101u;
  if (g.fold == 1) {
    *reinterpret_cast<float4*>(c) = x;
    if (hd) *reinterpret_cast<uint32_t*>(hd) = h;
    return;
  }
  float4 o = *reinterpret_cast<const float4*>(c);
  uint32_t keep = 0;  // byte q set where the stored value stays
  if (!(x.x > o.x)) { x.x = o.x; keep |= 0xFFu; }
  if (!(x.y > o.y)) { x.y = o.y; keep |= 0xFF00u; }
  if (!(x.z > o.z)) { x.z = o.z; keep |= 0xFF0000u; }
  if (!(x.w > o.w)) { x.w = o.w; keep |= 0xFF000000u; }
  if (keep == 0xFFFFFFFFu) return;
  *reinterpret_cast<float4*>(c) = x;
  if (hd) {
    const uint32_t old = *reinterpret_cast<const uint32_t*>(hd);
    *reinterpret_cast<uint32_t*>(hd) = (old & keep) | (h & ~keep);
  }
}

// bf16 layers multiply as autocast's nn.Linear does: the operands that are
// not bf16 already (the fp32 weights and projection gradients) are rounded to
// bf16 (nearest even), products accumulate in fp32.  The projection's B (W),
// the input gradient's A (dP) and B (W), the weight gradient's A (dP^T).
constexpr bool gemm_use_round_a(int use) { return use == kGemmGradInputBf16 || use == kGemmGradWeightBf16; }
constexpr bool gemm_use_round_b(int use) { return use == kGemmProjectBf16 || use == kGemmGradInputBf16; }
__device__ __forceinline__ float bf16_round(float x) { return (float)(bf16_t)x; }
__device__ __forceinline__ float4 bf16_round4(float4 v) {
  return make_float4(bf16_round(v.x), bf16_round(v.y), bf16_round(v.z), bf16_round(v.w));
}

// The A-operand mask of four consecutive elements: bytes of `heads` equal to
// `head` keep their element.
__device__ __forceinline__ float4 head_mask4(float4 a, uint32_t heads, int head) {
  a.x = (int)(heads & 0xFFu) == head ? a.x : 0.0f;
  a.y = (int)((heads >> 8) & 0xFFu) == head ? a.y : 0.0f;
  a.z = (int)((heads >> 16) & 0xFFu) == head ? a.z : 0.0f;
  a.w = (int)(heads >> 24) == head ? a.w : 0.0f;
  return a;
}

// One element of the softsign epilogue: returns the value to store and adds
// its share of the row's partial sum to `part`.
template <int USE>
__device__ __forceinline__ float dense_epilogue(float x, bool keep, float bias, float ps_n, float gds_m, float e_mn,
                                                float& part) {
  if constexpr (USE == kGemmDenseScores) {
    const float e = keep ? softsign_f(x + bias) : 0.0f;
    part += e * ps_n;
    return e;
  } else {
    const float d = 1.0f - fabsf(e_mn);
    const float gs = keep ? (x + gds_m * ps_n) * d * d : 0.0f;
    part += gs;
    return gs;
  }
}

// Softsign epilogue straight from one wave's accumulators: MT x MT tiles of
// 16 x 16, lane (grp, col) holding rows mb + 16 mt + 4 grp + v and columns
// nb + 16 nt + col (nb a multiple of 32, so tiles 2h and 2h + 1 form block h).
// C (and E) point at the batch element's matrix.
template <int USE, int MT>
__device__ __forceinline__ void dense_epilogue_tiles(const GemmArgs& g, int64_t bz, const floatx4 (&acc)[MT][MT],
                                                     int mb, int nb, float* C, int lane) {
  const int grp = lane >> 4, col = lane & 15;
  const int P = (g.N + kEpiBlock - 1) / kEpiBlock;
  const float* ps = g.epi_ps + bz * g.N;
  [[maybe_unused]] const float* gds = USE == kGemmDenseEdgeGrad ? g.epi_gds + bz * g.M : nullptr;
  [[maybe_unused]] const float* E = USE == kGemmDenseEdgeGrad ? g.epi_E + bz * g.c_bs : nullptr;
  float* part = g.epi_part + bz * (int64_t)g.M * P;
  const float bias = g.epi_bias ? g.epi_bias[0] : 0.0f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = mb + mt * 16 + grp * 4 + v;
      float gm = 0.0f;
      if constexpr (USE == kGemmDenseEdgeGrad) gm = m < g.M ? gds[m] : 0.0f;
#pragma unroll
      for (int h = 0; h < MT / 2; ++h) {
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int n = nb + (2 * h + q) * 16 + col;
          if (m < g.M && n < g.N) {
            float e = 0.0f;
            if constexpr (USE == kGemmDenseEdgeGrad) e = E[(int64_t)m * g.ldc + n];
            C[(int64_t)m * g.ldc + n] =
                dense_epilogue<USE>(acc[mt][2 * h + q][v], !g.epi_causal || n <= m, bias, ps[n], gm, e, s);
          }
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        s += __shfl_xor(s, 4);
        s += __shfl_xor(s, 8);
        const int blk = nb / kEpiBlock + h;
        if (col == 0 && m < g.M && blk < P) part[(int64_t)m * P + blk] = s;
      }
    }
}

constexpr int kGBM = 64, kGBK = 16;

// The K range [kbeg, kend) of the output tile whose rows start at m0 (TILE rows,
// columns from n0): a causal product reads only the k its rows can reach, and a
// causal softsign epilogue tile wholly above the diagonal needs no products at
// all (it stores zeros).  m0 is a multiple of TILE, so the bounds stay float4
// aligned.
template <int TILE>
__device__ __forceinline__ void causal_k_range(const GemmArgs& g, int m0, int n0, int& kbeg, int& kend) {
  if (g.causal_k == kCausalKLower) kend = min(kend, m0 + TILE);
  else if (g.causal_k == kCausalKUpper) kbeg = max(kbeg, m0);
  if (g.epi && g.epi_causal && n0 > m0 + TILE - 1) kend = kbeg;
}

__device__ __forceinline__ bool aligned16(const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// A(m,k): A_KC -> A[m*lda + k] else A[k*lda + m]
// B(k,n): B_KC -> Bsel(n)[n'*ldb + k] (split along n), else Bsel(k)[k'*ldb + n] (split along k)
// TILE x TILE output tile per workgroup (TILE = 64 or 128); wave (wm, wn) owns
// the (TILE/2) x (TILE/2) quadrant as (TILE/32)^2 tiles of 16 x 16.
// USE tags the call site (GemmUse): the code is the same for a given layout,
// but every use gets its own kernel symbol so profilers attribute time and
// traffic per use.
template <bool A_KC, bool B_KC, int USE, int TILE>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(GemmArgs g) {
  // K slice: 32 for the 64 x 64 tile, 128 for the 32 x 32 tile, whose
  // workgroups do too little per 16-wide slice to hide its load latency
  // (16-wide sub-slices, summed in the same order as separate slices)
  constexpr int BK = TILE == 32 ? 128 : 32;
  constexpr int GS = BK + 4;                  // LDS row stride (floats)
  constexpr int KQ = BK / 4;                  // float4s of a k-contiguous row slice
  constexpr int NF4 = TILE * BK / 4;          // float4s per operand and K slice
  constexpr int LPT = (NF4 + 255) / 256;      // of them per thread (TILE 32: threads 0..127 load one)
  constexpr int MT = TILE / 32;               // 16x16 tiles per wave along M (and N)
  static_assert(TILE == 32 || TILE == 64, "generic GEMM tiles are 32 or 64");
  constexpr bool A_BF = USE == kGemmProjectBf16;     // A (k-contiguous) holds bf16
  constexpr bool B_BF = USE == kGemmGradWeightBf16;  // B (k-major) holds bf16
  constexpr bool C_BF = USE == kGemmGradInputBf16;   // C and the addend hold bf16
  static_assert(!A_BF || A_KC, "bf16 A is k-contiguous");
  static_assert(!B_BF || !B_KC, "bf16 B is k-major");
  __shared__ __align__(16) float sA[2][TILE * GS];
  __shared__ __align__(16) float sB[2][TILE * GS];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, col = lane & 15;

  const int m0 = blockIdx.y * TILE;
  const int n0 = blockIdx.x * TILE;
  const bool batched = g.batch > 1;
  const int split = batched ? 0 : blockIdx.z;
  const int64_t bz = batched ? blockIdx.z : 0;
  int kbeg = split * g.k_chunk;
  int kend = min(g.K, kbeg + g.k_chunk);
  causal_k_range<TILE>(g, m0, n0, kbeg, kend);
  const float* gA = g.A + bz * g.a_bs;
  const float* gB0 = g.B0 + bz * g.b_bs;
  const float* gB1 = g.B1 + bz * g.b_bs;
  const float* gadd = g.addend ? g.addend + bz * g.add_bs : nullptr;
  const float* kscale = g.a_kscale ? g.a_kscale + bz * g.ks_bs : nullptr;
  const float* mscale = g.c_mscale ? g.c_mscale + bz * g.ms_bs : nullptr;
  float* C = g.C + (int64_t)split * g.c_split_stride + bz * g.c_bs;

  float ra[LPT][4], rb[LPT][4];

  auto load_slice = [&](int k0) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = tid + 256 * u;
      if (NF4 % 256 != 0 && e >= NF4) continue;
      // ---- A ----
      if constexpr (A_BF) {
        const int m = m0 + e / KQ, kq = k0 + (e % KQ) * 4;
        const bf16_t* p = reinterpret_cast<const bf16_t*>(g.A) + bz * g.a_bs + (int64_t)m * g.lda + kq;
        if (m < g.M && kq + 3 < kend && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
          const uint2 v = *reinterpret_cast<const uint2*>(p);
          unpack_bf16x2(v.x, ra[u][0], ra[u][1]);
          unpack_bf16x2(v.y, ra[u][2], ra[u][3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[u][q] = (m < g.M && kq + q < kend) ? (float)p[q] : 0.0f;
        }
      } else if (A_KC) {
        const int m = m0 + e / KQ, kq = k0 + (e % KQ) * 4;
        const float* p = gA + (int64_t)m * g.lda + kq;
        if (m < g.M && kq + 3 < kend && aligned16(p)) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          ra[u][0] = v.x; ra[u][1] = v.y; ra[u][2] = v.z; ra[u][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[u][q] = (m < g.M && kq + q < kend) ? p[q] : 0.0f;
        }
        if (kscale) {
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[u][q] *= (kq + q < kend) ? kscale[kq + q] : 0.0f;
        }
        if constexpr (gemm_use_amask(USE)) {
          if (g.a_heads) {
            const uint8_t* hp = g.a_heads + bz * g.a_bs + (int64_t)m * g.lda + kq;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (m < g.M && kq + q < kend && (int)hp[q] != g.a_head) ra[u][q] = 0.0f;
          }
        }
      } else {
        const int kk = k0 + e / (TILE / 4), mq = m0 + (e % (TILE / 4)) * 4;
        const float* p = gA + (int64_t)kk * g.lda + mq;
        if (kk < kend && mq + 3 < g.M && aligned16(p)) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          ra[u][0] = v.x; ra[u][1] = v.y; ra[u][2] = v.z; ra[u][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[u][q] = (kk < kend && mq + q < g.M) ? p[q] : 0.0f;
        }
        if (kscale) {
          const float sc = kk < kend ? kscale[kk] : 0.0f;
#pragma unroll
          for (int q = 0; q < 4; ++q) ra[u][q] *= sc;
        }
        if constexpr (gemm_use_amask(USE)) {
          if (g.a_heads) {
            const uint8_t* hp = g.a_heads + bz * g.a_bs + (int64_t)kk * g.lda + mq;
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (kk < kend && mq + q < g.M && (int)hp[q] != g.a_head) ra[u][q] = 0.0f;
          }
        }
      }
      // ---- B ----
      if (B_KC) {
        const int n = n0 + e / KQ, kq = k0 + (e % KQ) * 4;
        const float* base = (n < g.b_split) ? gB0 + (int64_t)n * g.ldb : gB1 + (int64_t)(n - g.b_split) * g.ldb;
        const float* p = base + kq;
        if (n < g.N && kq + 3 < kend && aligned16(p)) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          rb[u][0] = v.x; rb[u][1] = v.y; rb[u][2] = v.z; rb[u][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) rb[u][q] = (n < g.N && kq + q < kend) ? p[q] : 0.0f;
        }
      } else if constexpr (B_BF) {
        const int kk = k0 + e / (TILE / 4), nq = n0 + (e % (TILE / 4)) * 4;
        const bf16_t* base = reinterpret_cast<const bf16_t*>(kk < g.b_split ? g.B0 : g.B1) + bz * g.b_bs +
                             (int64_t)(kk < g.b_split ? kk : kk - g.b_split) * g.ldb;
        const bf16_t* p = base + nq;
        if (kk < kend && nq + 3 < g.N && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
          const uint2 v = *reinterpret_cast<const uint2*>(p);
          unpack_bf16x2(v.x, rb[u][0], rb[u][1]);
          unpack_bf16x2(v.y, rb[u][2], rb[u][3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) rb[u][q] = (kk < kend && nq + q < g.N) ? (float)p[q] : 0.0f;
        }
      } else {
        const int kk = k0 + e / (TILE / 4), nq = n0 + (e % (TILE / 4)) * 4;
        const float* base = (kk < g.b_split) ? gB0 + (int64_t)kk * g.ldb : gB1 + (int64_t)(kk - g.b_split) * g.ldb;
        const float* p = base + nq;
        if (kk < kend && nq + 3 < g.N && aligned16(p)) {
          const float4 v = *reinterpret_cast<const float4*>(p);
          rb[u][0] = v.x; rb[u][1] = v.y; rb[u][2] = v.z; rb[u][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) rb[u][q] = (kk < kend && nq + q < g.N) ? p[q] : 0.0f;
        }
      }
    }
  };
  auto store_slice = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = tid + 256 * u;
      if (NF4 % 256 != 0 && e >= NF4) continue;
      if constexpr (gemm_use_round_a(USE)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) ra[u][q] = bf16_round(ra[u][q]);
      }
      if constexpr (gemm_use_round_b(USE)) {
#pragma unroll
        for (int q = 0; q < 4; ++q) rb[u][q] = bf16_round(rb[u][q]);
      }
      if (A_KC) {
        *reinterpret_cast<float4*>(&sA[buf][(e / KQ) * GS + (e % KQ) * 4]) =
            make_float4(ra[u][0], ra[u][1], ra[u][2], ra[u][3]);
      } else {
        const int kk = e / (TILE / 4), mq = (e % (TILE / 4)) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) sA[buf][(mq + q) * GS + kk] = ra[u][q];
      }
      if (B_KC) {
        *reinterpret_cast<float4*>(&sB[buf][(e / KQ) * GS + (e % KQ) * 4]) =
            make_float4(rb[u][0], rb[u][1], rb[u][2], rb[u][3]);
      } else {
        const int kk = e / (TILE / 4), nq = (e % (TILE / 4)) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) sB[buf][(nq + q) * GS + kk] = rb[u][q];
      }
    }
  };

  // Four accumulation chains per output tile (one per k step of a slice),
  // summed in the epilogue: each chain adds a quarter of the K products, so
  // the fp32 rounding of long reductions (K = node counts in the dense and
  // weight-gradient products) grows half as fast as with one chain.
  floatx4 acc[MT][MT], chain[3][MT][MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 3; ++c) chain[c][i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  const int nslices = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  if (nslices > 0) {
    load_slice(kbeg);
    store_slice(0);
  }
  __syncthreads();

  for (int s = 0; s < nslices; ++s) {
    const int cur = s & 1;
    if (s + 1 < nslices) load_slice(kbeg + (s + 1) * BK);

#pragma unroll
    for (int ss = 0; ss < BK / 16; ++ss) {
      float4 av[MT], bv[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        av[t] = *reinterpret_cast<const float4*>(&sA[cur][(wm * (TILE / 2) + t * 16 + col) * GS + ss * 16 + grp * 4]);
        bv[t] = *reinterpret_cast<const float4*>(&sB[cur][(wn * (TILE / 2) + t * 16 + col) * GS + ss * 16 + grp * 4]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < MT; ++nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].x, bv[nt].x, acc[mt][nt], 0, 0, 0);
          chain[0][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].y, bv[nt].y, chain[0][mt][nt], 0, 0, 0);
          chain[1][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].z, bv[nt].z, chain[1][mt][nt], 0, 0, 0);
          chain[2][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].w, bv[nt].w, chain[2][mt][nt], 0, 0, 0);
        }
    }

    if (s + 1 < nslices) store_slice(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < MT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        acc[mt][nt][v] = (acc[mt][nt][v] + chain[0][mt][nt][v]) + (chain[1][mt][nt][v] + chain[2][mt][nt][v]);

  // Epilogue: lane holds rows 4*grp+v of each 16x16 tile, column col.
  if constexpr (USE == kGemmDenseScores || USE == kGemmDenseEdgeGrad) {
    if (g.epi) {
      dense_epilogue_tiles<USE, MT>(g, bz, acc, m0 + wm * (TILE / 2), n0 + wn * (TILE / 2), C, lane);
      return;
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < MT; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + wm * (TILE / 2) + mt * 16 + grp * 4 + v;
        const int n = n0 + wn * (TILE / 2) + nt * 16 + col;
        if (m < g.M && n < g.N) {
          float x = acc[mt][nt][v];
          if constexpr (gemm_use_fold(USE)) {
            if (g.fold) {
              const int64_t o = (int64_t)m * g.ldc + n;
              fold_store(g, x, C + o, g.fold_heads ? g.fold_heads + bz * g.c_bs + o : nullptr);
              continue;
            }
          }
          if (g.c_nscale) x *= g.c_nscale[n];
          if (mscale) x *= mscale[m];
          if constexpr (C_BF) {
            if (g.addend) x += (float)reinterpret_cast<const bf16_t*>(g.addend)[(int64_t)m * g.ld_add + n];
            reinterpret_cast<bf16_t*>(g.C)[(int64_t)m * g.ldc + n] = (bf16_t)x;
          } else {
            if (gadd) x += gadd[(int64_t)m * g.ld_add + n];
            C[(int64_t)m * g.ldc + n] = x;
          }
        }
      }
}

// Layout (A k-contiguous, B k-contiguous), optional operand features (A
// scaled along k, B rows split over two buffers) and timer label of every use.
struct GemmUseInfo {
  bool a_kc, b_kc, a_kscale, b_split;
  const char* name;
};
constexpr GemmUseInfo kGemmUses[] = {
    {true, true, false, true, "gemm_f32_kernel<project>"},
    {true, false, false, true, "gemm_f32_kernel<grad_input>"},
    {false, false, false, false, "gemm_f32_kernel<grad_weight>"},
    {true, true, true, false, "gemm_f32_kernel<dense_scores>"},
    {true, false, false, false, "gemm_f32_kernel<dense_aggregate>"},
    {true, true, false, false, "gemm_f32_kernel<dense_edge_grad>"},
    {false, false, false, false, "gemm_f32_kernel<dense_value_grad>"},
    {true, false, false, false, "gemm_f32_kernel<dense_target_grad>"},
    {false, false, false, false, "gemm_f32_kernel<dense_source_grad>"},
    {true, true, true, false, "gemm_f32_kernel<route_logits>"},
    {false, false, true, false, "gemm_f32_kernel<route_aggregate>"},
    {true, true, false, false, "gemm_f32_kernel<route_edge_grad>"},
    {true, false, false, false, "gemm_f32_kernel<route_value_grad>"},
    {true, false, false, false, "gemm_f32_kernel<route_source_grad>"},
    {false, false, false, false, "gemm_f32_kernel<route_target_grad>"},
    {true, true, false, true, "gemm_f32_kernel<project_bf16>"},
    {true, false, false, true, "gemm_f32_kernel<grad_input_bf16>"},
    {false, false, false, false, "gemm_f32_kernel<grad_weight_bf16>"},
    {true, true, true, false, "gemm_f32_kernel<select_scores>"},
    {true, false, false, false, "gemm_bf16_kernel<dense_aggregate_bf16>"},
    {false, false, false, false, "gemm_bf16_kernel<dense_value_grad_bf16>"},
    {true, true, false, false, "gemm_bf16_kernel<dense_edge_grad_bf16>"},
    {false, false, true, false, "gemm_bf16_kernel<route_aggregate_bf16>"},
    {true, false, false, false, "gemm_bf16_kernel<route_value_grad_bf16>"},
    {true, true, false, false, "gemm_bf16_kernel<route_edge_grad_bf16>"},
};
static_assert(sizeof(kGemmUses) / sizeof(kGemmUses[0]) == kGemmRouteEdgeGradBf16 + 1, "one entry per GemmUse");
constexpr bool gemm_use_bf16(GemmUse u) {
  return u == kGemmProjectBf16 || u == kGemmGradInputBf16 || u == kGemmGradWeightBf16;
}
// The bf16 dense and dense-route uses run on the bf16 MFMA kernel only (their
// callers check its preconditions first).
constexpr bool gemm_use_dense_bf16(int u) {
  return u == kGemmDenseAggregateBf16 || u == kGemmDenseValueGradBf16 || u == kGemmDenseEdgeGradBf16 ||
         u == kGemmRouteAggregateBf16 || u == kGemmRouteValueGradBf16 || u == kGemmRouteEdgeGradBf16;
}

// ---- 128 x 128 path --------------------------------------------------------
// Workgroup tile 128 x 128, K staged through LDS in slices of BK (double
// buffered, register prefetch of the next slice); each wave owns a 64 x 64
// quadrant as 4 x 4 tiles of v_mfma_f32_16x16x4f32.
//
// Preconditions (checked by the host; otherwise the 64 x 64 kernel runs):
// every float4 the loaders fetch lies wholly inside or wholly outside its
// operand -- K and the split-K chunk are multiples of 4, so is M (N) when A (B)
// is K-major, row strides, batch strides and base pointers are float4
// aligned -- and row strides are below 2^20 floats so that 32-bit buffer
// offsets from a per-slice base reach every row of a slice.  A float4 outside
// the operand is fetched at an offset past the buffer resource and reads as
// zeros, so the loaders have no branches.
//
// LDS layouts: a K-contiguous operand is stored [row][BK + 4] and read as one
// ds_read_b128 per lane (4 consecutive k); a K-major operand is stored
// [k][128 + 4] (float4 stores, no transpose) and read as four ds_read_b32 at
// stride 132 (conflict-free: 4 rows apart = 16 banks).
constexpr int kFT = 128;
constexpr uint32_t kFastRecords = 0x80000000u;

// Four consecutive operand elements at a byte offset of a buffer resource as
// fp32 (zeros when out of range): one 16-byte load of fp32, or one 8-byte load
// of bf16 widened exactly.
template <bool BF>
__device__ __forceinline__ float4 fast_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  if constexpr (BF) {
    const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0));
    float4 f;
    unpack_bf16x2(x.x, f.x, f.y);
    unpack_bf16x2(x.y, f.z, f.w);
    return f;
  } else {
    return buf_load4(r, byte_off);
  }
}

template <bool KC, int BK>
struct FastLds {
  static constexpr int stride = KC ? BK + 4 : kFT + 4;
  static constexpr int floats = KC ? kFT * stride : BK * stride;
};

// Operand fragment of 16x16 tile `t` (of the wave's 4) for k sub-block kb:
// lane (col, grp) gets element (row = base + t*16 + col, k = kb*16 + grp*4 + q)
// in component q.
template <bool KC, int BK>
__device__ __forceinline__ float4 fast_fragment(const float* s, int base, int t, int kb, int col, int grp) {
  constexpr int S = FastLds<KC, BK>::stride;
  if constexpr (KC) {
    return *reinterpret_cast<const float4*>(&s[(base + t * 16 + col) * S + kb * 16 + grp * 4]);
  } else {
    const float* p = &s[(kb * 16 + grp * 4) * S + base + t * 16 + col];
    return make_float4(p[0], p[S], p[2 * S], p[3 * S]);
  }
}

template <bool A_KC, bool B_KC, int USE, int BK>
__global__ __launch_bounds__(256, 4) void gemm_f32_fast_kernel(GemmArgs g, int tiles_m, int tiles_n, int vec_out) {
  constexpr int LPT = kFT * BK / 4 / 256;  // float4 per thread, per operand and slice
  constexpr int KCH = BK / 4;              // float4 per K-contiguous row of a slice
  constexpr int MCH = kFT / 4;             // float4 per K-major row of a slice
  using LA = FastLds<A_KC, BK>;
  using LB = FastLds<B_KC, BK>;
  constexpr int kStageStride = 68;         // epilogue strip: 16 rows x 64 columns per wave
  static_assert(4 * 16 * kStageStride <= 2 * (LA::floats + LB::floats), "epilogue strips must fit in LDS");
  __shared__ __align__(16) float smem[2 * (LA::floats + LB::floats)];
  float(*sA)[LA::floats] = reinterpret_cast<float(*)[LA::floats]>(smem);
  float(*sB)[LB::floats] = reinterpret_cast<float(*)[LB::floats]>(smem + 2 * LA::floats);

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, col = lane & 15;

  // Logical tile: each XCD runs a contiguous range; inside it, bands of 8
  // M-tiles sweep N so that concurrently running tiles share A and B rows.
  const int id = xcd_swizzle(blockIdx.x, gridDim.x);
  const int per = tiles_m * tiles_n;
  const int z = id / per;
  const int t = id - z * per;
  constexpr int kBand = 8;
  const int band = t / (kBand * tiles_n);
  const int bm = min(kBand, tiles_m - band * kBand);
  const int tb = t - band * kBand * tiles_n;
  int mi = band * kBand + tb % bm;
  // A causal product's tiles of rows differ in work: with kCausalKLower (and
  // score tiles above the diagonal skipped) the work grows with the row, so
  // the rows run last to first -- longest first, the short tiles fill the
  // tail.  kCausalKUpper tiles already come longest first.
  if (g.causal_k == kCausalKLower || (g.epi && g.epi_causal)) mi = tiles_m - 1 - mi;
  const int m0 = mi * kFT;
  const int n0 = (tb / bm) * kFT;

  const bool batched = g.batch > 1;
  const int split = batched ? 0 : z;
  const int64_t bz = batched ? z : 0;
  int kbeg = split * g.k_chunk;
  int kend = min(g.K, kbeg + g.k_chunk);
  causal_k_range<kFT>(g, m0, n0, kbeg, kend);
  // bf16 uses: X is the A operand (project), the B operand (weight gradient)
  // or C with its addend (input gradient); offsets below are in elements
  constexpr bool A_BF = USE == kGemmProjectBf16;
  constexpr bool B_BF = USE == kGemmGradWeightBf16;
  constexpr bool C_BF = USE == kGemmGradInputBf16;
  constexpr uint32_t AEB = A_BF ? 2 : 4, BEB = B_BF ? 2 : 4;
  const char* gA = reinterpret_cast<const char*>(g.A) + bz * g.a_bs * AEB;
  const char* gB0 = reinterpret_cast<const char*>(g.B0) + bz * g.b_bs * BEB;
  const char* gB1 = reinterpret_cast<const char*>(g.B1) + bz * g.b_bs * BEB;
  const float* gadd = g.addend ? g.addend + bz * g.add_bs : nullptr;
  const float* kscale = g.a_kscale ? g.a_kscale + bz * g.ks_bs : nullptr;
  const float* mscale = g.c_mscale ? g.c_mscale + bz * g.ms_bs : nullptr;
  float* C = g.C + (int64_t)split * g.c_split_stride + bz * g.c_bs;
  [[maybe_unused]] bf16_t* Cb = reinterpret_cast<bf16_t*>(g.C) + (int64_t)split * g.c_split_stride + bz * g.c_bs;
  [[maybe_unused]] const bf16_t* gaddb =
      g.addend ? reinterpret_cast<const bf16_t*>(g.addend) + bz * g.add_bs : nullptr;
  const int lda = (int)g.lda, ldb = (int)g.ldb;

  // Registers of the prefetched slice.  Everything that combines loaded
  // values (the k scale) waits until the slice is stored to LDS, after the
  // MFMAs, so that the loads stay in flight meanwhile.
  constexpr bool KSCALE = kGemmUses[USE].a_kscale;
  constexpr bool BSPLIT = kGemmUses[USE].b_split;
  constexpr int NSC = KSCALE ? (A_KC ? 4 : 1) : 0;
  float4 ra[LPT], rb[LPT];
  [[maybe_unused]] float rs[LPT][NSC > 0 ? NSC : 1];
  // head bytes of the masked A elements (gemm_use_amask), applied at the LDS store
  constexpr bool AMASK = gemm_use_amask(USE);
  [[maybe_unused]] uint32_t rh[AMASK ? LPT : 1];

  auto load_slice = [&](int k0) {
    // ---- A ----
    const int64_t aoff = A_KC ? (int64_t)m0 * lda + k0 : (int64_t)k0 * lda + m0;
    const char* abase = gA + aoff * AEB;
    const auto ars = make_rsrc(abase, kFastRecords);
    [[maybe_unused]] const auto hrs = make_rsrc(AMASK && g.a_heads ? static_cast<const void*>(g.a_heads + bz * g.a_bs + aoff)
                                                                        : static_cast<const void*>(abase),
                                                kFastRecords);
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = tid + 256 * u;
      const int row = A_KC ? e / KCH : e / MCH;  // m (A_KC) or k offset in the slice
      const int c4 = A_KC ? (e % KCH) * 4 : (e % MCH) * 4;
      const bool ok = A_KC ? (m0 + row < g.M && k0 + c4 < kend) : (k0 + row < kend && m0 + c4 < g.M);
      ra[u] = fast_load4<A_BF>(ars, ok ? (uint32_t)(row * lda + c4) * AEB : kOobOffset);
      if constexpr (AMASK) {
        if (g.a_heads)
          rh[u] = __builtin_amdgcn_raw_buffer_load_b32(hrs, ok ? (uint32_t)(row * lda + c4) : kOobOffset, 0, 0);
      }
      if constexpr (KSCALE) {
        const auto srs = make_rsrc(kscale + k0, kFastRecords);
        if constexpr (A_KC) {
          const float4 sc = buf_load4(srs, k0 + c4 < kend ? (uint32_t)c4 * 4u : kOobOffset);
          rs[u][0] = sc.x; rs[u][NSC > 1 ? 1 : 0] = sc.y; rs[u][NSC > 2 ? 2 : 0] = sc.z; rs[u][NSC - 1] = sc.w;
        } else {
          rs[u][0] = buf_load1(srs, k0 + row < kend ? (uint32_t)row * 4u : kOobOffset);
        }
      }
    }
    // ---- B: rows below b_split come from B0, the rest from B1 ----
    // The rows one wave fetches with one instruction (16 for a K-contiguous B,
    // 2 for a K-major B) never straddle b_split (the host requires b_split to
    // be a multiple of 16), so the buffer is chosen per wave and instruction;
    // both resources address rows relative to the slice's first row.
    const int s0 = B_KC ? n0 : k0;
    const char* base0 = gB0 + (B_KC ? (int64_t)n0 * ldb + k0 : (int64_t)k0 * ldb + n0) * BEB;
    const auto brs0 = make_rsrc(base0, kFastRecords);
    [[maybe_unused]] const auto brs1 =
        make_rsrc(BSPLIT ? gB1 + (B_KC ? (int64_t)(n0 - g.b_split) * ldb + k0 : (int64_t)(k0 - g.b_split) * ldb + n0) *
                               BEB
                         : base0,
                  kFastRecords);
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = tid + 256 * u;
      const int row = B_KC ? e / KCH : e / MCH;  // n (B_KC) or k offset in the slice
      const int c4 = B_KC ? (e % KCH) * 4 : (e % MCH) * 4;
      const bool ok = B_KC ? (n0 + row < g.N && k0 + c4 < kend) : (k0 + row < kend && n0 + c4 < g.N);
      const uint32_t off = ok ? (uint32_t)(row * ldb + c4) * BEB : kOobOffset;
      if constexpr (BSPLIT) {
        const int wrow = B_KC ? (wave * 64 + 256 * u) / KCH : (wave * 64 + 256 * u) / MCH;  // wave-uniform
        rb[u] = fast_load4<B_BF>(s0 + wrow < g.b_split ? brs0 : brs1, off);
      } else {
        rb[u] = fast_load4<B_BF>(brs0, off);
      }
    }
  };
  auto store_slice = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int e = tid + 256 * u;
      const int ia = A_KC ? (e / KCH) * LA::stride + (e % KCH) * 4 : (e / MCH) * LA::stride + (e % MCH) * 4;
      const int ib = B_KC ? (e / KCH) * LB::stride + (e % KCH) * 4 : (e / MCH) * LB::stride + (e % MCH) * 4;
      float4 a = ra[u];
      if constexpr (KSCALE) {
        a.x *= rs[u][0]; a.y *= rs[u][NSC > 1 ? 1 : 0]; a.z *= rs[u][NSC > 2 ? 2 : 0]; a.w *= rs[u][NSC - 1];
      }
      if constexpr (AMASK) {
        if (g.a_heads) a = head_mask4(a, rh[u], g.a_head);
      }
      if constexpr (gemm_use_round_a(USE)) a = bf16_round4(a);
      *reinterpret_cast<float4*>(&sA[buf][ia]) = a;
      *reinterpret_cast<float4*>(&sB[buf][ib]) = gemm_use_round_b(USE) ? bf16_round4(rb[u]) : rb[u];
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nslices = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  if (nslices > 0) {
    load_slice(kbeg);
    store_slice(0);
  }
  __syncthreads();

  for (int s = 0; s < nslices; ++s) {
    const int cur = s & 1;
    if (s + 1 < nslices) load_slice(kbeg + (s + 1) * BK);
#pragma unroll
    for (int kb = 0; kb < BK / 16; ++kb) {
      float4 av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = fast_fragment<A_KC, BK>(sA[cur], wm * 64, i, kb, col, grp);
        bv[i] = fast_fragment<B_KC, BK>(sB[cur], wn * 64, i, kb, col, grp);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].x, bv[nt].x, acc[mt][nt], 0, 0, 0);
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].y, bv[nt].y, acc[mt][nt], 0, 0, 0);
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].z, bv[nt].z, acc[mt][nt], 0, 0, 0);
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[mt].w, bv[nt].w, acc[mt][nt], 0, 0, 0);
        }
    }
    if (s + 1 < nslices) store_slice(cur ^ 1);
    __syncthreads();
  }

  // Epilogue.  With vec_out (N, ldc, ld_add and the batch/split strides
  // multiples of 4, C and the addend float4 aligned) each wave stages a 16 x 64
  // strip of its quadrant in LDS and writes whole float4 rows: 16 lanes cover
  // 256 contiguous bytes of a row.  Otherwise each lane stores its own
  // elements (rows 4*grp+v of each 16x16 tile, column col).
  if (vec_out) {
    float* stage = smem + wave * 16 * kStageStride;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) stage[(grp * 4 + v) * kStageStride + nt * 16 + col] = acc[mt][nt][v];
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = grp + 4 * i, c4 = col * 4;
        const int m = m0 + wm * 64 + mt * 16 + r;
        const int n = n0 + wn * 64 + c4;
        float4 x = *reinterpret_cast<const float4*>(&stage[r * kStageStride + c4]);
        if constexpr (USE == kGemmDenseScores || USE == kGemmDenseEdgeGrad) {
          if (g.epi) {
            // softsign epilogue; lanes col..col+7 of a group hold one row's 32-column block
            const int P = (g.N + kEpiBlock - 1) / kEpiBlock;
            float part = 0.0f;
            if (m < g.M && n < g.N) {
              const float4 p4 = *reinterpret_cast<const float4*>(&g.epi_ps[bz * g.N + n]);
              float4 e4 = make_float4(0.f, 0.f, 0.f, 0.f);
              float gm = 0.0f;
              if constexpr (USE == kGemmDenseEdgeGrad) {
                e4 = *reinterpret_cast<const float4*>(&g.epi_E[bz * g.c_bs + (int64_t)m * g.ldc + n]);
                gm = g.epi_gds[bz * g.M + m];
              }
              const float bias = g.epi_bias ? g.epi_bias[0] : 0.0f;
              const bool all = !g.epi_causal;
              x.x = dense_epilogue<USE>(x.x, all || n <= m, bias, p4.x, gm, e4.x, part);
              x.y = dense_epilogue<USE>(x.y, all || n + 1 <= m, bias, p4.y, gm, e4.y, part);
              x.z = dense_epilogue<USE>(x.z, all || n + 2 <= m, bias, p4.z, gm, e4.z, part);
              x.w = dense_epilogue<USE>(x.w, all || n + 3 <= m, bias, p4.w, gm, e4.w, part);
              *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n]) = x;
            }
            part += __shfl_xor(part, 1);
            part += __shfl_xor(part, 2);
            part += __shfl_xor(part, 4);
            const int blk = (n0 + wn * 64) / kEpiBlock + (col >> 3);
            if ((col & 7) == 0 && m < g.M && blk < P) g.epi_part[(bz * g.M + m) * P + blk] = part;
            continue;
          }
        }
        if constexpr (gemm_use_fold(USE)) {
          if (g.fold) {
            if (m < g.M && n < g.N) {
              const int64_t o = (int64_t)m * g.ldc + n;
              fold_store4(g, x, C + o, g.fold_heads ? g.fold_heads + bz * g.c_bs + o : nullptr);
            }
            continue;
          }
        }
        if (m < g.M && n < g.N) {
          if (g.c_nscale) {
            const float4 sc = *reinterpret_cast<const float4*>(&g.c_nscale[n]);
            x.x *= sc.x; x.y *= sc.y; x.z *= sc.z; x.w *= sc.w;
          }
          if (mscale) {
            const float sm = mscale[m];
            x.x *= sm; x.y *= sm; x.z *= sm; x.w *= sm;
          }
          // the input gradient and its addend are read and written once: non-temporal
          constexpr bool NT = USE == kGemmGradInput || USE == kGemmGradInputBf16;
          if constexpr (C_BF) {
            if (gaddb) {
              const uint2 ab = load_nt8(&gaddb[(int64_t)m * g.ld_add + n]);
              float4 a;
              unpack_bf16x2(ab.x, a.x, a.y);
              unpack_bf16x2(ab.y, a.z, a.w);
              x.x += a.x; x.y += a.y; x.z += a.z; x.w += a.w;
            }
            store_nt8(&Cb[(int64_t)m * g.ldc + n], make_uint2(pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w)));
          } else if constexpr (NT) {
            if (gadd) {
              const uint4 ab = load_nt16(&gadd[(int64_t)m * g.ld_add + n]);
              x.x += __uint_as_float(ab.x); x.y += __uint_as_float(ab.y);
              x.z += __uint_as_float(ab.z); x.w += __uint_as_float(ab.w);
            }
            store_nt16(&C[(int64_t)m * g.ldc + n],
                       make_uint4(__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z), __float_as_uint(x.w)));
          } else {
            if (gadd) {
              const float4 a = *reinterpret_cast<const float4*>(&gadd[(int64_t)m * g.ld_add + n]);
              x.x += a.x; x.y += a.y; x.z += a.z; x.w += a.w;
            }
            *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n]) = x;
          }
        }
      }
      __syncthreads();
    }
  } else {
    if constexpr (USE == kGemmDenseScores || USE == kGemmDenseEdgeGrad) {
      if (g.epi) {
        dense_epilogue_tiles<USE, 4>(g, bz, acc, m0 + wm * 64, n0 + wn * 64, C, lane);
        return;
      }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int m = m0 + wm * 64 + mt * 16 + grp * 4 + v;
          const int n = n0 + wn * 64 + nt * 16 + col;
          if (m < g.M && n < g.N) {
            float x = acc[mt][nt][v];
            if constexpr (gemm_use_fold(USE)) {
              if (g.fold) {
                const int64_t o = (int64_t)m * g.ldc + n;
                fold_store(g, x, C + o, g.fold_heads ? g.fold_heads + bz * g.c_bs + o : nullptr);
                continue;
              }
            }
            if (g.c_nscale) x *= g.c_nscale[n];
            if (mscale) x *= mscale[m];
            if constexpr (C_BF) {
              if (gaddb) x += (float)gaddb[(int64_t)m * g.ld_add + n];
              Cb[(int64_t)m * g.ldc + n] = (bf16_t)x;
            } else {
              if (gadd) x += gadd[(int64_t)m * g.ld_add + n];
              C[(int64_t)m * g.ldc + n] = x;
            }
          }
        }
  }
}

// ---- bf16 MFMA path (bf16 layers) ------------------------------------------
// The projection of bf16 layer values and its two gradients, and a bf16
// dense layer's three N x N products (E . pv, E^T . gdv, gdv . pv^T, causal
// K ranges included), on
// v_mfma_f32_16x16x32_bf16: workgroup tile 128 x 128, 2 x 2 waves of 64 x 64
// (4 x 4 tiles of 16 x 16), K in slices of 64 (two K-steps of 32), LDS double
// buffered with register prefetch.  Both operands sit in LDS as [row][k]
// bf16 (row = m for A, n for B; 8 elements of padding per row), so a lane's
// fragment -- 8 consecutive k of one row -- is one 16-byte LDS read.  fp32
// operands are rounded to bf16 (nearest even) on their way into LDS; K-major
// operands are transposed there in 4 x 4 (fp32) or 4 x 8 (bf16) blocks.
// Accumulation is fp32.  The epilogue stages each wave's 64 x 64 block in LDS
// and writes whole 8-element rows (one 16-byte store of bf16, two of fp32);
// the dense score gradient's softsign epilogue works from the accumulators.
// Preconditions (host-checked, else the fp32 kernels run): M, N >= 128, N and
// the output strides multiples of 8, K and the split-K chunk multiples of 64
// ... of 8 for K-contiguous bf16 rows; row strides and batch strides
// multiples of 8 elements, base pointers 16-byte aligned.  Loads go through
// buffer resources: a vector outside its operand reads as zeros.
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
constexpr int kBfT = 128;           // tile M and N
constexpr int kBfK = 64;            // K per slice
constexpr int kBfS = kBfK + 8;      // LDS row stride in bf16 elements (144 bytes)
constexpr int kBfStage = 64 + 4;    // epilogue row stride in floats

// Operand loader of one slice: R = 128 rows (m or n) x 64 k into LDS [row][k].
//   KC: row-major with k contiguous (row stride ld); else k-major (k rows of stride ld).
//   BF: the source holds bf16; else fp32, rounded to bf16.
//   KS: (k-major fp32 only) each element is first multiplied by a scale per k.
template <bool KC, bool BF, bool KS = false>
struct BfLoader {
  static_assert(!KS || (!KC && !BF), "k scales apply to k-major fp32 operands");
  // 16-byte loads per thread and slice
  static constexpr int kLoads = KC ? (BF ? 4 : 8) : (BF ? 4 : 8);
  uint4 r[kLoads];
  float4 sc[KS ? 2 : 1];  // the scales of a thread's two 4 x 4 blocks (k = 4 kb .. 4 kb + 3)

  // the k scales of the slice's (from k0; ks_rs addresses the scale of k0)
  __device__ __forceinline__ void load_scales(__amdgpu_buffer_rsrc_t ks_rs, int k0, int kend, int tid) {
    if constexpr (KS) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = (tid + 256 * h) >> 5;
        sc[h] = buf_load4(ks_rs, k0 + 4 * kb < kend ? (uint32_t)(16 * kb) : kOobOffset);
      }
    }
  }

  // rs0 addresses the slice's (row 0, k = k0) -- offsets stay within one
  // slice of rows, so 32-bit offsets reach any K; K-contiguous rows from
  // split_row on (tile-relative, a multiple of 8) are read through rs1, which
  // addresses the slice's row 0 as if the second buffer continued the first
  // (the rows a wave loads with one instruction never straddle it: a
  // wave-uniform choice)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs0, __amdgpu_buffer_rsrc_t rs1, int split_row, int ld,
                                       int row0, int rows, int k0, int kend, int tid) {
    constexpr uint32_t EB = BF ? 2 : 4;
    [[maybe_unused]] const int wbase = tid & ~63;
    if constexpr (KC && BF) {  // 128 rows x 8 groups of 8 k
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, row = e >> 3, kq = (e & 7) * 8;
        const bool ok = row0 + row < rows && k0 + kq < kend;
        const auto rs = ((wbase + 256 * u) >> 3) < split_row ? rs0 : rs1;
        r[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, ok ? (uint32_t)(row * ld + kq) * EB : kOobOffset, 0, 0));
      }
    } else if constexpr (KC) {  // 128 rows x 16 groups of 4 k
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = tid + 256 * u, row = e >> 4, kq = (e & 15) * 4;
        const bool ok = row0 + row < rows && k0 + kq < kend;
        const auto rs = ((wbase + 256 * u) >> 4) < split_row ? rs0 : rs1;
        r[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, ok ? (uint32_t)(row * ld + kq) * EB : kOobOffset, 0, 0));
      }
    } else if constexpr (BF) {  // 16 groups of 4 k x 16 groups of 8 rows: one 4 x 8 block per thread
      const int kb = tid >> 4, rb = (tid & 15) * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = 4 * kb + i;
        const bool ok = k0 + kk < kend && row0 + rb < rows;
        r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs0, ok ? (uint32_t)(kk * ld + rb) * EB : kOobOffset, 0, 0));
      }
    } else {  // 16 groups of 4 k x 32 groups of 4 rows: two 4 x 4 blocks per thread
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = tid + 256 * h, kb = blk >> 5, rb = (blk & 31) * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = 4 * kb + i;
          const bool ok = k0 + kk < kend && row0 + rb < rows;
          r[4 * h + i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rs0, ok ? (uint32_t)(kk * ld + rb) * EB : kOobOffset, 0, 0));
        }
      }
    }
  }

  __device__ __forceinline__ static uint32_t pack2(uint32_t lo, uint32_t hi) {  // two fp32 bit patterns -> bf16x2
    return pack_bf16x2(__uint_as_float(lo), __uint_as_float(hi));
  }

  __device__ __forceinline__ void store(bf16_t* s, int tid) const {
    if constexpr (KC && BF) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, row = e >> 3, kq = (e & 7) * 8;
        *reinterpret_cast<uint4*>(&s[row * kBfS + kq]) = r[u];
      }
    } else if constexpr (KC) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = tid + 256 * u, row = e >> 4, kq = (e & 15) * 4;
        *reinterpret_cast<uint2*>(&s[row * kBfS + kq]) = make_uint2(pack2(r[u].x, r[u].y), pack2(r[u].z, r[u].w));
      }
    } else if constexpr (BF) {
      // r[i] holds k = 4 kb + i, rows rb .. rb + 7 (two bf16 per word)
      const int kb = tid >> 4, rb = (tid & 15) * 8;
      const uint32_t w[4][4] = {{r[0].x, r[0].y, r[0].z, r[0].w}, {r[1].x, r[1].y, r[1].z, r[1].w},
                                {r[2].x, r[2].y, r[2].z, r[2].w}, {r[3].x, r[3].y, r[3].z, r[3].w}};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sh = (j & 1) * 16, q = j >> 1;
        const uint32_t e0 = (w[0][q] >> sh) & 0xFFFFu, e1 = (w[1][q] >> sh) & 0xFFFFu;
        const uint32_t e2 = (w[2][q] >> sh) & 0xFFFFu, e3 = (w[3][q] >> sh) & 0xFFFFu;
        *reinterpret_cast<uint2*>(&s[(rb + j) * kBfS + 4 * kb]) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int blk = tid + 256 * h, kb = blk >> 5, rb = (blk & 31) * 4;
        const uint4* v = &r[4 * h];  // v[i]: k = 4 kb + i, rows rb .. rb + 3
        uint32_t c[4][4] = {{v[0].x, v[0].y, v[0].z, v[0].w}, {v[1].x, v[1].y, v[1].z, v[1].w},
                            {v[2].x, v[2].y, v[2].z, v[2].w}, {v[3].x, v[3].y, v[3].z, v[3].w}};
        if constexpr (KS) {
          const float f[4] = {sc[h].x, sc[h].y, sc[h].z, sc[h].w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) c[i][j] = __float_as_uint(__uint_as_float(c[i][j]) * f[i]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint2*>(&s[(rb + j) * kBfS + 4 * kb]) =
              make_uint2(pack2(c[0][j], c[1][j]), pack2(c[2][j], c[3][j]));
      }
    }
  }
};

// C_BF: C and the addend hold bf16 (the input gradient, the dense aggregate
// and value gradient).
template <bool A_KC, bool A_BF, bool B_KC, bool B_BF, bool C_BF, int USE>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  __shared__ __align__(16) bf16_t smem[4 * kBfT * kBfS];  // A[2], B[2]; the epilogue reuses it
  auto sA = [&](int i) { return smem + i * kBfT * kBfS; };
  auto sB = [&](int i) { return smem + (2 + i) * kBfT * kBfS; };
  static_assert(4 * 64 * kBfStage * 4 <= 4 * kBfT * kBfS * 2, "epilogue strips must fit in LDS");

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, col = lane & 15;

  // logical tile: contiguous ranges per XCD, bands of 8 M-tiles sweeping N
  const int id = xcd_swizzle(blockIdx.x, gridDim.x);
  const int per = tiles_m * tiles_n;
  const int z = id / per, t = id - z * per;
  constexpr int kBand = 8;
  const int band = t / (kBand * tiles_n);
  const int bm = min(kBand, tiles_m - band * kBand);
  const int tb = t - band * kBand * tiles_n;
  int mi = band * kBand + tb % bm;
  // causal products: the longest K ranges (or the epilogue's non-empty rows) first
  if (g.causal_k == kCausalKLower || (g.epi && g.epi_causal)) mi = tiles_m - 1 - mi;
  const int m0 = mi * kBfT;
  const int n0 = (tb / bm) * kBfT;
  const bool batched = g.batch > 1;
  const int split = batched ? 0 : z;
  const int64_t bz = batched ? z : 0;
  int kbeg = split * g.k_chunk;
  int kend = min(g.K, kbeg + g.k_chunk);
  causal_k_range<kBfT>(g, m0, n0, kbeg, kend);

  constexpr uint32_t AEB = A_BF ? 2 : 4, BEB = B_BF ? 2 : 4;
  const int lda = (int)g.lda, ldb = (int)g.ldb;
  // operand origins (row0 = m0 / n0 along the row axis, k = 0); each slice's
  // buffer resources start at the slice
  const char* abase = reinterpret_cast<const char*>(g.A) + (bz * g.a_bs + (A_KC ? (int64_t)m0 * lda : m0)) * AEB;
  auto borigin = [&](const float* Bp, int64_t rofs) {
    return reinterpret_cast<const char*>(Bp) + (bz * g.b_bs + (B_KC ? rofs * ldb : rofs)) * BEB;
  };
  // B's rows below b_split come from B0, the rest from B1: along n for a
  // K-contiguous B, along k for a k-major B (whole slices: the host keeps
  // b_split a multiple of 64 there)
  const char* b0base = borigin(g.B0, n0);
  const char* b1base = B_KC ? borigin(g.B1, (int64_t)n0 - g.b_split) : borigin(g.B1, n0);
  const int b_split_row = B_KC ? g.b_split - n0 : 1 << 30;
  auto at_k = [](const char* origin, bool kc, int ld, int64_t k, uint32_t eb) {
    return make_rsrc(origin + (kc ? k : k * ld) * eb, kFastRecords);
  };

  constexpr bool KS = kGemmUses[USE].a_kscale;  // A scaled along k (k-major fp32 A)
  BfLoader<A_KC, A_BF, KS> la;
  BfLoader<B_KC, B_BF> lb;
  [[maybe_unused]] const float* kscale = KS ? g.a_kscale + bz * g.ks_bs : nullptr;
  auto load_slice = [&](int k0) {
    const auto ars = at_k(abase, A_KC, lda, k0, AEB);
    la.load(ars, ars, 1 << 30, lda, m0, g.M, k0, kend, tid);
    if constexpr (KS) la.load_scales(make_rsrc(kscale + k0, kFastRecords), k0, kend, tid);
    if constexpr (!B_KC) {
      if (k0 >= g.b_split) {
        const auto rs = at_k(b1base, false, ldb, (int64_t)k0 - g.b_split, BEB);
        lb.load(rs, rs, 1 << 30, ldb, n0, g.N, k0 - g.b_split, kend - g.b_split, tid);
      } else {
        const auto rs = at_k(b0base, false, ldb, k0, BEB);
        lb.load(rs, rs, 1 << 30, ldb, n0, g.N, k0, min(kend, g.b_split), tid);
      }
    } else {
      lb.load(at_k(b0base, true, ldb, k0, BEB), at_k(b1base, true, ldb, k0, BEB), b_split_row, ldb, n0, g.N, k0,
              kend, tid);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nslices = kend > kbeg ? (kend - kbeg + kBfK - 1) / kBfK : 0;
  if (nslices > 0) {
    load_slice(kbeg);
    la.store(sA(0), tid);
    lb.store(sB(0), tid);
  }
  __syncthreads();
  for (int s = 0; s < nslices; ++s) {
    const int cur = s & 1;
    if (s + 1 < nslices) load_slice(kbeg + (s + 1) * kBfK);
#pragma unroll
    for (int ks = 0; ks < kBfK / 32; ++ks) {
      bf16x8v av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        av[i] = *reinterpret_cast<const bf16x8v*>(&sA(cur)[(wm * 64 + i * 16 + col) * kBfS + ks * 32 + grp * 8]);
        bv[i] = *reinterpret_cast<const bf16x8v*>(&sB(cur)[(wn * 64 + i * 16 + col) * kBfS + ks * 32 + grp * 8]);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
    }
    if (s + 1 < nslices) {
      la.store(sA(cur ^ 1), tid);
      lb.store(sB(cur ^ 1), tid);
    }
    __syncthreads();
  }

  float* C = g.C + (int64_t)split * g.c_split_stride + bz * g.c_bs;
  // the score gradient of a bf16 dense layer: softsign's derivative straight
  // from the accumulators (the 16 x 16 output layout of every MFMA shape)
  if constexpr (USE == kGemmDenseEdgeGradBf16) {
    if (g.epi) {
      dense_epilogue_tiles<kGemmDenseEdgeGrad, 4>(g, bz, acc, m0 + wm * 64, n0 + wn * 64, C, lane);
      return;
    }
  }

  // epilogue: each wave's 64 x 64 block through LDS, then rows of 8 elements
  float* stage = reinterpret_cast<float*>(smem) + wave * 64 * kBfStage;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) stage[(mt * 16 + grp * 4 + v) * kBfStage + nt * 16 + col] = acc[mt][nt][v];
  __syncthreads();
  [[maybe_unused]] bf16_t* Cb = reinterpret_cast<bf16_t*>(g.C) + bz * g.c_bs;
  [[maybe_unused]] const bf16_t* addb =
      g.addend ? reinterpret_cast<const bf16_t*>(g.addend) + bz * g.add_bs : nullptr;
  [[maybe_unused]] const float* mscale = g.c_mscale ? g.c_mscale + bz * g.ms_bs : nullptr;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = it * 8 + (lane >> 3), c0 = (lane & 7) * 8;
    const int m = m0 + wm * 64 + r, n = n0 + wn * 64 + c0;
    if (m >= g.M || n >= g.N) continue;
    const float4 x0 = *reinterpret_cast<const float4*>(&stage[r * kBfStage + c0]);
    const float4 x1 = *reinterpret_cast<const float4*>(&stage[r * kBfStage + c0 + 4]);
    if constexpr (C_BF) {
      float4 y0 = x0, y1 = x1;
      if (mscale) {  // C row m scaled (the route value gradient's diag(rho))
        const float sm = mscale[m];
        y0.x *= sm; y0.y *= sm; y0.z *= sm; y0.w *= sm;
        y1.x *= sm; y1.y *= sm; y1.z *= sm; y1.w *= sm;
      }
      if (addb) {
        const uint4 ab = load_nt16(&addb[(int64_t)m * g.ld_add + n]);
        float a0, a1;
        unpack_bf16x2(ab.x, a0, a1); y0.x += a0; y0.y += a1;
        unpack_bf16x2(ab.y, a0, a1); y0.z += a0; y0.w += a1;
        unpack_bf16x2(ab.z, a0, a1); y1.x += a0; y1.y += a1;
        unpack_bf16x2(ab.w, a0, a1); y1.z += a0; y1.w += a1;
      }
      store_nt16(&Cb[(int64_t)m * g.ldc + n], make_uint4(pack_bf16x2(y0.x, y0.y), pack_bf16x2(y0.z, y0.w),
                                                         pack_bf16x2(y1.x, y1.y), pack_bf16x2(y1.z, y1.w)));
    } else {
      *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n]) = x0;
      *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n + 4]) = x1;
    }
  }
}

// Whether a bf16 use runs on the bf16 MFMA kernel (see its preconditions).
static bool bf16_path_ok(const GemmArgs& g, int use, int splits) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (g.M < kBfT || g.N < kBfT || g.N % 8 != 0 || g.ldc % 8 != 0 || g.lda % 8 != 0 || g.ldb % 8 != 0) return false;
  if (g.a_bs % 8 != 0 || g.b_bs % 8 != 0 || g.c_bs % 8 != 0 || g.c_split_stride % 8 != 0) return false;
  if (g.lda >= (1 << 20) || g.ldb >= (1 << 20)) return false;
  if (!al16(g.A) || !al16(g.B0) || !al16(g.B1) || !al16(g.C)) return false;
  if (g.addend && (g.ld_add % 8 != 0 || g.add_bs % 8 != 0 || !al16(g.addend))) return false;
  if (g.c_nscale || g.fold || g.a_heads) return false;
  if (g.epi && use != kGemmDenseEdgeGradBf16) return false;
  if (g.a_kscale && (use != kGemmRouteAggregateBf16 || !al16(g.a_kscale) || g.ks_bs % 4 != 0)) return false;
  if (g.c_mscale && use != kGemmRouteValueGradBf16) return false;
  if (splits > 1 && g.k_chunk % kBfK != 0) return false;
  if (use == kGemmProjectBf16) return g.K % 8 == 0 && g.b_split % 16 == 0;          // A bf16, B fp32, K-contiguous
  if (use == kGemmGradInputBf16) return g.K % 4 == 0 && g.b_split % kBfK == 0;       // A fp32 K-contig, B fp32 K-major
  if (use == kGemmGradWeightBf16) return g.M % 4 == 0 && g.b_split >= g.K;            // both K-major
  if (use == kGemmDenseAggregateBf16) return g.K % 4 == 0 && g.b_split >= g.K && !g.addend;  // A fp32 K-contig (E)
  if (use == kGemmDenseValueGradBf16) return g.M % 4 == 0 && g.b_split >= g.K && !g.addend;  // A fp32 K-major (E)
  if (use == kGemmDenseEdgeGradBf16) return g.K % 8 == 0 && g.b_split >= g.N && !g.addend;   // both bf16 K-contig
  if (use == kGemmRouteAggregateBf16)  // A fp32 K-major (R^T, k-scaled), B bf16 K-major
    return g.M % 4 == 0 && g.K % 4 == 0 && g.a_kscale && g.b_split >= g.K && !g.addend;
  if (use == kGemmRouteValueGradBf16) return g.K % 4 == 0 && g.b_split >= g.K && !g.addend;  // A fp32 K-contig (R)
  if (use == kGemmRouteEdgeGradBf16) return g.K % 8 == 0 && g.b_split >= g.N && !g.addend;   // both bf16 K-contig
  return false;
}

// ---- fp32 products as three-term bf16 splits --------------------------------
// An fp32 value x splits exactly into three bf16 terms x = h + m + l: h is x
// truncated to bf16 (sign, exponent, 7 fraction bits); r = x - h (exact: the
// 16 low significand bits of x) splits the same way into m and l = r - m, which
// has at most 8 significant bits and so is a bf16 value.  A product a.b is
// taken as the six terms h.h + h.m + m.h + h.l + l.h + m.m, each exact in fp32,
// on v_mfma_f32_16x16x32_bf16 with fp32 accumulation; the three dropped terms
// (m.l, l.m, l.l) stay below 2^-23 |a b| together, about one fp32 rounding of
// the product.  Six 16-cycle bf16 MFMAs per 16 x 16 x 32 block replace eight
// 32-cycle fp32 ones.
//
// gemm_x3_kernel is gemm_bf16_kernel for fp32 operands in this form: the three
// planes of both operands sit in LDS as [row][k] bf16, K in slices of 32, in
// one LDS buffer (61 KB, 70 KB with the epilogue's strips: two workgroups per
// CU) refilled from registers that prefetch the next slice, split on their way
// into LDS; each slice's operand resources start at the slice, so 32-bit
// offsets cover any K.  Used for the projection and its gradients and for the
// dense aggregation E.pv and its value gradient E^T.gdv (causal K ranges
// included) when the 128 x 128 tiles apply (x3_path_ok); jn_set_gemm_tile(128)
// keeps them on fp32 MFMA.  Measured against float64, the bf16 MFMA's
// accumulation leans slightly negative (of order 2^-33 of the accumulator per
// instruction): harmless per element, but summed over the 16.8M score
// gradients of C4's dense bias gradient it left the fp32 tolerance (3.6 of
// 1.6e4), so the score-gradient product gdv.pv^T stays on fp32 MFMA.
constexpr int kX3K = 32;                 // K per slice
constexpr int kX3S = kX3K + 8;           // LDS row stride in bf16 elements (80 bytes: conflict-free fragments)
constexpr int kX3Plane = kBfT * kX3S;    // one plane of one operand

__device__ __forceinline__ void x3_split(uint32_t u, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = u & 0xFFFF0000u;
  const float r = __uint_as_float(u) - __uint_as_float(h);
  m = __float_as_uint(r) & 0xFFFF0000u;
  l = __float_as_uint(r - __uint_as_float(m));
}

// the bf16 values in the high halves of two words as one bf16x2 word (first in the low half)
__device__ __forceinline__ uint32_t x3_pair(uint32_t first, uint32_t second) {
  return __builtin_amdgcn_perm(second, first, 0x07060302u);  // bytes 2, 3 of first, then of second
}

// Operand loader of one slice: 128 rows (m or n) x 32 k of fp32 into the three
// LDS planes [row][k].  KC: rows with k contiguous (row stride ld); else k rows
// of stride ld.  `base` addresses the slice's (row 0, k 0).
template <bool KC>
struct X3Loader {
  uint4 r[4];

  // rs1 serves the rows from split_row on (KC only, a multiple of 8: one wave's
  // load never straddles it)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs0, __amdgpu_buffer_rsrc_t rs1, int split_row, int ld,
                                       int row0, int rows, int k0, int kend, int tid) {
    if constexpr (KC) {  // 128 rows x 8 groups of 4 k
      const int wbase = tid & ~63;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, row = e >> 3, kq = (e & 7) * 4;
        const bool ok = row0 + row < rows && k0 + kq < kend;
        const auto rs = ((wbase + 256 * u) >> 3) < split_row ? rs0 : rs1;
        r[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs, ok ? (uint32_t)(row * ld + kq) * 4u : kOobOffset, 0, 0));
      }
    } else {  // 8 groups of 4 k x 32 groups of 4 rows: one 4 x 4 block per thread
      const int kb = tid >> 5, rb = (tid & 31) * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = 4 * kb + i;
        const bool ok = k0 + kk < kend && row0 + rb < rows;
        r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                             rs0, ok ? (uint32_t)(kk * ld + rb) * 4u : kOobOffset, 0, 0));
      }
    }
  }

  // planes h, m, l at s, s + kX3Plane, s + 2 kX3Plane
  __device__ __forceinline__ void store(bf16_t* s, int tid) const {
    if constexpr (KC) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, row = e >> 3, kq = (e & 7) * 4;
        uint32_t h[4], m[4], l[4];
        x3_split(r[u].x, h[0], m[0], l[0]);
        x3_split(r[u].y, h[1], m[1], l[1]);
        x3_split(r[u].z, h[2], m[2], l[2]);
        x3_split(r[u].w, h[3], m[3], l[3]);
        bf16_t* d = &s[row * kX3S + kq];
        *reinterpret_cast<uint2*>(d) = make_uint2(x3_pair(h[0], h[1]), x3_pair(h[2], h[3]));
        *reinterpret_cast<uint2*>(d + kX3Plane) = make_uint2(x3_pair(m[0], m[1]), x3_pair(m[2], m[3]));
        *reinterpret_cast<uint2*>(d + 2 * kX3Plane) = make_uint2(x3_pair(l[0], l[1]), x3_pair(l[2], l[3]));
      }
    } else {
      // r[i] holds k = 4 kb + i, rows rb .. rb + 3
      const int kb = tid >> 5, rb = (tid & 31) * 4;
      const uint32_t c[4][4] = {{r[0].x, r[0].y, r[0].z, r[0].w}, {r[1].x, r[1].y, r[1].z, r[1].w},
                                {r[2].x, r[2].y, r[2].z, r[2].w}, {r[3].x, r[3].y, r[3].z, r[3].w}};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t h[4], m[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x3_split(c[i][j], h[i], m[i], l[i]);
        bf16_t* d = &s[(rb + j) * kX3S + 4 * kb];
        *reinterpret_cast<uint2*>(d) = make_uint2(x3_pair(h[0], h[1]), x3_pair(h[2], h[3]));
        *reinterpret_cast<uint2*>(d + kX3Plane) = make_uint2(x3_pair(m[0], m[1]), x3_pair(m[2], m[3]));
        *reinterpret_cast<uint2*>(d + 2 * kX3Plane) = make_uint2(x3_pair(l[0], l[1]), x3_pair(l[2], l[3]));
      }
    }
  }
};

template <bool A_KC, bool B_KC, int USE>
__global__ __launch_bounds__(256, 2) void gemm_x3_kernel(GemmArgs g, int tiles_m, int tiles_n) {
  // [A, B][plane] (61 KB), or the epilogue's four 64-row strips (70 KB)
  constexpr int kWords = 4 * 64 * kBfStage > 3 * kX3Plane ? 4 * 64 * kBfStage : 3 * kX3Plane;
  __shared__ __align__(16) uint32_t smem32[kWords];
  bf16_t* smem = reinterpret_cast<bf16_t*>(smem32);
  auto sA = [&](int) { return smem; };
  auto sB = [&](int) { return smem + 3 * kX3Plane; };

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int grp = lane >> 4, col = lane & 15;

  // logical tile: contiguous ranges per XCD, bands of 8 M-tiles sweeping N
  const int id = xcd_swizzle(blockIdx.x, gridDim.x);
  const int per = tiles_m * tiles_n;
  const int z = id / per, t = id - z * per;
  constexpr int kBand = 8;
  const int band = t / (kBand * tiles_n);
  const int bm = min(kBand, tiles_m - band * kBand);
  const int tb = t - band * kBand * tiles_n;
  int mi = band * kBand + tb % bm;
  if (g.causal_k == kCausalKLower) mi = tiles_m - 1 - mi;  // longest K ranges first
  const int m0 = mi * kBfT;
  const int n0 = (tb / bm) * kBfT;
  const bool batched = g.batch > 1;
  const int split = batched ? 0 : z;
  const int64_t bz = batched ? z : 0;
  int kbeg = split * g.k_chunk;
  int kend = min(g.K, kbeg + g.k_chunk);
  causal_k_range<kBfT>(g, m0, n0, kbeg, kend);
  const int lda = (int)g.lda, ldb = (int)g.ldb;
  const float* gA = g.A + bz * g.a_bs;
  const float* gB0 = g.B0 + bz * g.b_bs;
  const float* gB1 = g.B1 + bz * g.b_bs;

  X3Loader<A_KC> la;
  X3Loader<B_KC> lb;
  auto load_slice = [&](int k0) {
    const auto ars = make_rsrc(gA + (A_KC ? (int64_t)m0 * lda + k0 : (int64_t)k0 * lda + m0), kFastRecords);
    la.load(ars, ars, 1 << 30, lda, m0, g.M, k0, kend, tid);
    if constexpr (B_KC) {  // B0 rows below b_split, B1 from there (along n)
      const auto b0 = make_rsrc(gB0 + (int64_t)n0 * ldb + k0, kFastRecords);
      const auto b1 = make_rsrc(gB1 + (int64_t)(n0 - g.b_split) * ldb + k0, kFastRecords);
      lb.load(b0, b1, g.b_split - n0, ldb, n0, g.N, k0, kend, tid);
    } else {  // along k: whole slices (the host keeps b_split a multiple of kX3K)
      const bool second = k0 >= g.b_split;
      const auto b = make_rsrc(second ? gB1 + (int64_t)(k0 - g.b_split) * ldb + n0 : gB0 + (int64_t)k0 * ldb + n0,
                               kFastRecords);
      lb.load(b, b, 1 << 30, ldb, n0, g.N, k0, second ? kend : min(kend, g.b_split), tid);
    }
  };

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nslices = kend > kbeg ? (kend - kbeg + kX3K - 1) / kX3K : 0;
  if (nslices > 0) {
    load_slice(kbeg);
    la.store(sA(0), tid);
    lb.store(sB(0), tid);
  }
  __syncthreads();
  for (int s = 0; s < nslices; ++s) {
    const int cur = s & 1;
    if (s + 1 < nslices) load_slice(kbeg + (s + 1) * kX3K);
    const bf16_t* a = sA(cur) + (wm * 64 + col) * kX3S + grp * 8;
    const bf16_t* b = sB(cur) + (wn * 64 + col) * kX3S + grp * 8;
    bf16x8v ah[4], am[4], al[4], bh[4], bm[4], bl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ah[i] = *reinterpret_cast<const bf16x8v*>(a + i * 16 * kX3S);
      am[i] = *reinterpret_cast<const bf16x8v*>(a + i * 16 * kX3S + kX3Plane);
      al[i] = *reinterpret_cast<const bf16x8v*>(a + i * 16 * kX3S + 2 * kX3Plane);
      bh[i] = *reinterpret_cast<const bf16x8v*>(b + i * 16 * kX3S);
      bm[i] = *reinterpret_cast<const bf16x8v*>(b + i * 16 * kX3S + kX3Plane);
      bl[i] = *reinterpret_cast<const bf16x8v*>(b + i * 16 * kX3S + 2 * kX3Plane);
    }
    // the small terms first
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        floatx4 c = acc[mt][nt];
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[mt], bh[nt], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mt], bl[nt], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am[mt], bm[nt], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am[mt], bh[nt], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mt], bm[nt], c, 0, 0, 0);
        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mt], bh[nt], c, 0, 0, 0);
      }
    __syncthreads();  // the slice is consumed: the next one replaces it
    if (s + 1 < nslices) {
      la.store(sA(cur ^ 1), tid);
      lb.store(sB(cur ^ 1), tid);
      __syncthreads();
    }
  }

  // epilogue: each wave's 64 x 64 block through LDS, then rows of 8 elements
  float* stage = reinterpret_cast<float*>(smem) + wave * 64 * kBfStage;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) stage[(mt * 16 + grp * 4 + v) * kBfStage + nt * 16 + col] = acc[mt][nt][v];
  __syncthreads();
  float* C = g.C + (int64_t)split * g.c_split_stride + bz * g.c_bs;
  const float* add = g.addend ? g.addend + bz * g.add_bs : nullptr;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = it * 8 + (lane >> 3), c0 = (lane & 7) * 8;
    const int m = m0 + wm * 64 + r, n = n0 + wn * 64 + c0;
    if (m >= g.M || n >= g.N) continue;
    float4 x0 = *reinterpret_cast<const float4*>(&stage[r * kBfStage + c0]);
    float4 x1 = *reinterpret_cast<const float4*>(&stage[r * kBfStage + c0 + 4]);
    if (add) {
      const float4 a0 = *reinterpret_cast<const float4*>(&add[(int64_t)m * g.ld_add + n]);
      const float4 a1 = *reinterpret_cast<const float4*>(&add[(int64_t)m * g.ld_add + n + 4]);
      x0.x += a0.x; x0.y += a0.y; x0.z += a0.z; x0.w += a0.w;
      x1.x += a1.x; x1.y += a1.y; x1.z += a1.z; x1.w += a1.w;
    }
    *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n]) = x0;
    *reinterpret_cast<float4*>(&C[(int64_t)m * g.ldc + n + 4]) = x1;
  }
}

// Whether an fp32 projection use runs on gemm_x3_kernel (its preconditions).
static bool x3_path_ok(const GemmArgs& g, int use, int splits) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (g.M < kBfT || g.N < kBfT || g.N % 8 != 0 || g.ldc % 4 != 0 || g.lda % 4 != 0 || g.ldb % 4 != 0) return false;
  if (g.a_bs % 4 != 0 || g.b_bs % 4 != 0 || g.c_bs % 4 != 0 || g.c_split_stride % 4 != 0) return false;
  if (g.lda >= (1 << 20) || g.ldb >= (1 << 20)) return false;
  if (!al16(g.A) || !al16(g.B0) || !al16(g.B1) || !al16(g.C)) return false;
  if (g.addend && (g.ld_add % 4 != 0 || g.add_bs % 4 != 0 || !al16(g.addend))) return false;
  if (g.a_kscale || g.c_nscale || g.c_mscale || g.epi || g.fold || g.a_heads) return false;
  if (splits > 1 && g.k_chunk % kX3K != 0) return false;
  if (use == kGemmProject) return g.K % 4 == 0 && g.b_split % 16 == 0;               // both K-contiguous
  if (use == kGemmGradInput) return g.K % 4 == 0 && g.b_split % kX3K == 0;            // B K-major, split along k
  if (use == kGemmGradWeight) return g.M % 4 == 0 && g.b_split >= g.K;               // both K-major
  if (use == kGemmDenseAggregate) return g.K % 4 == 0 && g.b_split >= g.K;           // E . pv
  if (use == kGemmDenseValueGrad) return g.M % 4 == 0 && g.b_split >= g.K;           // E^T . gdv
  return false;
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


constexpr int kFastBK = 16;

static bool f4_aligned(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15) == 0; }


// The projection uses (and their gradients) on the 32 x 32 tile when a 64 x 64
// grid would leave most CUs idle (small row counts: transitions, C5's slot
// layers); other uses keep 64 x 64 there.
constexpr bool gemm_use_small_tile(int use) {
  return use == kGemmProject || use == kGemmGradInput || use == kGemmGradWeight || use == kGemmProjectBf16 ||
         use == kGemmGradInputBf16 || use == kGemmGradWeightBf16;
}

template <int USE>
static void launch_use(const GemmArgs& g, bool fast, bool small, int zdim, hipStream_t stream) {
  constexpr GemmUseInfo u = kGemmUses[USE];
  if constexpr (gemm_use_small_tile(USE)) {
    if (small) {
      dim3 grid((g.N + 31) / 32, (g.M + 31) / 32, zdim);
      hipLaunchKernelGGL((gemm_f32_kernel<u.a_kc, u.b_kc, USE, 32>), grid, dim3(256), 0, stream, g);
      return;
    }
  }
  if (fast) {
    const int tm = (g.M + kFT - 1) / kFT, tn = (g.N + kFT - 1) / kFT;
    const bool vec = g.N % 4 == 0 && g.ldc % 4 == 0 && g.c_bs % 4 == 0 && g.c_split_stride % 4 == 0 &&
                     f4_aligned(g.C) && f4_aligned(g.c_nscale) && f4_aligned(g.epi_ps) && f4_aligned(g.epi_E) &&
                     (reinterpret_cast<uintptr_t>(g.fold_heads) & 3) == 0 &&
                     (g.addend == nullptr || (g.ld_add % 4 == 0 && g.add_bs % 4 == 0 && f4_aligned(g.addend)));
    hipLaunchKernelGGL((gemm_f32_fast_kernel<u.a_kc, u.b_kc, USE, kFastBK>), dim3(tm * tn * zdim), dim3(256), 0,
                       stream, g, tm, tn, vec ? 1 : 0);
  } else {
    dim3 grid((g.N + kGBM - 1) / kGBM, (g.M + kGBM - 1) / kGBM, zdim);
    hipLaunchKernelGGL((gemm_f32_kernel<u.a_kc, u.b_kc, USE, kGBM>), grid, dim3(256), 0, stream, g);
  }
}

static std::atomic<int> g_gemm_tile{0};

void set_gemm_tile(int tile) { g_gemm_tile.store(tile, std::memory_order_relaxed); }

// Whether the 128 x 128 kernel's preconditions hold (see gemm_f32_fast_kernel).
static bool fast_path_ok(const GemmArgs& g, bool a_kc, bool b_kc) {
  constexpr int64_t kMaxLd = 1 << 20;
  if (g.b_split < (b_kc ? g.N : g.K) && g.b_split % 16 != 0) return false;
  if (g.K % 4 != 0 || g.k_chunk % 4 != 0) return false;
  if ((!a_kc && g.M % 4 != 0) || (!b_kc && g.N % 4 != 0)) return false;
  if (g.lda % 4 != 0 || g.ldb % 4 != 0 || g.a_bs % 4 != 0 || g.b_bs % 4 != 0 || g.ks_bs % 4 != 0) return false;
  if (g.lda >= kMaxLd || g.ldb >= kMaxLd) return false;
  if ((reinterpret_cast<uintptr_t>(g.a_heads) & 3) != 0) return false;
  return f4_aligned(g.A) && f4_aligned(g.B0) && f4_aligned(g.B1) && f4_aligned(g.a_kscale);
}

int launch_gemm(const GemmArgs& g, GemmUse use, int splits, hipStream_t stream) {
  JN_REQUIRE(g.M >= 0 && g.N >= 0 && g.K >= 0, kInvalidArgument, "negative GEMM extent");
  if (g.M == 0 || g.N == 0) return kOk;
  JN_REQUIRE(g.batch <= 1 || splits == 1, kInvalidArgument, "batched GEMM has no split-K");
  JN_REQUIRE(g.batch < 65536 && splits < 65536, kUnsupported, "GEMM batch or split count too large");
  JN_REQUIRE(g.batch > 1 || (int64_t)splits * g.k_chunk >= g.K, kInvalidArgument, "split-K chunks do not cover K");
  const GemmUseInfo& info = kGemmUses[use];
  JN_REQUIRE(g.a_kscale == nullptr || info.a_kscale, kInvalidArgument, "GEMM use %s takes no k scale", info.name);
  JN_REQUIRE(g.b_split >= (info.b_kc ? g.N : g.K) || info.b_split, kInvalidArgument,
             "GEMM use %s takes one B buffer", info.name);
  const int64_t zdim = g.batch > 1 ? g.batch : splits;
  JN_REQUIRE((g.M + kGBM - 1) / kGBM < 65536, kUnsupported, "GEMM M extent too large");
  // 128 x 128 tiles halve the operand traffic per flop; 64 x 64 when an
  // extent is too small to fill them or the grid would be too small
  const int64_t tiles128 = (int64_t)((g.M + kFT - 1) / kFT) * ((g.N + kFT - 1) / kFT) * zdim;
  const int forced = g_gemm_tile.load(std::memory_order_relaxed);
  const bool big = forced ? forced == kFT : (g.M >= kFT && g.N >= kFT && tiles128 >= 256);
  // (the 128 x 128 kernel applies the k scale of a scaled use unconditionally)
  const bool fast = big && tiles128 < (1LL << 31) && fast_path_ok(g, info.a_kc, info.b_kc) &&
                    (!info.a_kscale || g.a_kscale != nullptr);
  // 32 x 32 tiles for the projection uses when a 64 x 64 grid would not reach
  // one workgroup per CU
  const int64_t tiles64 = (int64_t)((g.M + kGBM - 1) / kGBM) * ((g.N + kGBM - 1) / kGBM) * zdim;
  const bool small = !fast && gemm_use_small_tile(use) && (g.M + 31) / 32 < 65536 &&
                     (forced ? forced == 32 : tiles64 < 256);
  if (gemm_use_dense_bf16(use)) {
    JN_REQUIRE(bf16_path_ok(g, use, splits), kUnsupported,
               "%s needs M, N >= 128, N and the strides multiples of 8 and 16-byte aligned operands", info.name);
    const int tm = (g.M + kBfT - 1) / kBfT, tn = (g.N + kBfT - 1) / kBfT;
    const int64_t blocks = (int64_t)tm * tn * zdim;
    JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "GEMM grid too large");
    JN_PROFILE(info.name, stream);
    if (use == kGemmDenseAggregateBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<true, false, false, true, true, kGemmDenseAggregateBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else if (use == kGemmDenseValueGradBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<false, false, false, true, true, kGemmDenseValueGradBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else if (use == kGemmDenseEdgeGradBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<true, true, true, true, false, kGemmDenseEdgeGradBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else if (use == kGemmRouteAggregateBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<false, false, false, true, true, kGemmRouteAggregateBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else if (use == kGemmRouteValueGradBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<true, false, false, true, true, kGemmRouteValueGradBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<true, true, true, true, false, kGemmRouteEdgeGradBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    JN_LAUNCH_CHECK();
    return kOk;
  }
  if (gemm_use_bf16(use) && forced != 32 && forced != 64 && bf16_path_ok(g, use, splits)) {
    const int tm = (g.M + kBfT - 1) / kBfT, tn = (g.N + kBfT - 1) / kBfT;
    const int64_t blocks = (int64_t)tm * tn * zdim;
    JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "GEMM grid too large");
    JN_PROFILE(use == kGemmProjectBf16 ? "gemm_bf16_kernel<project_bf16>"
               : use == kGemmGradInputBf16 ? "gemm_bf16_kernel<grad_input_bf16>"
                                           : "gemm_bf16_kernel<grad_weight_bf16>",
               stream);
    if (use == kGemmProjectBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<true, true, true, false, false, kGemmProjectBf16>), dim3((unsigned)blocks),
                         dim3(256), 0, stream, g, tm, tn);
    else if (use == kGemmGradInputBf16)
      hipLaunchKernelGGL((gemm_bf16_kernel<true, false, false, false, true, kGemmGradInputBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    else
      hipLaunchKernelGGL((gemm_bf16_kernel<false, false, false, true, false, kGemmGradWeightBf16>),
                         dim3((unsigned)blocks), dim3(256), 0, stream, g, tm, tn);
    JN_LAUNCH_CHECK();
    return kOk;
  }
  if ((use == kGemmProject || use == kGemmGradInput || use == kGemmGradWeight || use == kGemmDenseAggregate ||
       use == kGemmDenseValueGrad) &&
      forced == 0 && x3_path_ok(g, use, splits)) {
    const int tm = (g.M + kBfT - 1) / kBfT, tn = (g.N + kBfT - 1) / kBfT;
    const int64_t blocks = (int64_t)tm * tn * zdim;
    JN_REQUIRE(blocks < (1LL << 31), kUnsupported, "GEMM grid too large");
    const dim3 grid((unsigned)blocks);
    switch (use) {
      case kGemmProject: {
        JN_PROFILE("gemm_x3_kernel<project>", stream);
        hipLaunchKernelGGL((gemm_x3_kernel<true, true, kGemmProject>), grid, dim3(256), 0, stream, g, tm, tn);
        break;
      }
      case kGemmGradInput: {
        JN_PROFILE("gemm_x3_kernel<grad_input>", stream);
        hipLaunchKernelGGL((gemm_x3_kernel<true, false, kGemmGradInput>), grid, dim3(256), 0, stream, g, tm, tn);
        break;
      }
      case kGemmGradWeight: {
        JN_PROFILE("gemm_x3_kernel<grad_weight>", stream);
        hipLaunchKernelGGL((gemm_x3_kernel<false, false, kGemmGradWeight>), grid, dim3(256), 0, stream, g, tm, tn);
        break;
      }
      case kGemmDenseAggregate: {
        JN_PROFILE("gemm_x3_kernel<dense_aggregate>", stream);
        hipLaunchKernelGGL((gemm_x3_kernel<true, false, kGemmDenseAggregate>), grid, dim3(256), 0, stream, g, tm,
                           tn);
        break;
      }
      default: {
        JN_PROFILE("gemm_x3_kernel<dense_value_grad>", stream);
        hipLaunchKernelGGL((gemm_x3_kernel<false, false, kGemmDenseValueGrad>), grid, dim3(256), 0, stream, g, tm,
                           tn);
        break;
      }
    }
    JN_LAUNCH_CHECK();
    return kOk;
  }
  JN_PROFILE(info.name, stream);
  switch (use) {
    case kGemmProject: launch_use<kGemmProject>(g, fast, small, (int)zdim, stream); break;
    case kGemmGradInput: launch_use<kGemmGradInput>(g, fast, small, (int)zdim, stream); break;
    case kGemmGradWeight: launch_use<kGemmGradWeight>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseScores: launch_use<kGemmDenseScores>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseAggregate: launch_use<kGemmDenseAggregate>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseEdgeGrad: launch_use<kGemmDenseEdgeGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseValueGrad: launch_use<kGemmDenseValueGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseTargetGrad: launch_use<kGemmDenseTargetGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmDenseSourceGrad: launch_use<kGemmDenseSourceGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteLogits: launch_use<kGemmRouteLogits>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteAggregate: launch_use<kGemmRouteAggregate>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteEdgeGrad: launch_use<kGemmRouteEdgeGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteValueGrad: launch_use<kGemmRouteValueGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteSourceGrad: launch_use<kGemmRouteSourceGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmRouteTargetGrad: launch_use<kGemmRouteTargetGrad>(g, fast, small, (int)zdim, stream); break;
    case kGemmProjectBf16: launch_use<kGemmProjectBf16>(g, fast, small, (int)zdim, stream); break;
    case kGemmGradInputBf16: launch_use<kGemmGradInputBf16>(g, fast, small, (int)zdim, stream); break;
    case kGemmGradWeightBf16: launch_use<kGemmGradWeightBf16>(g, fast, small, (int)zdim, stream); break;
    case kGemmSelectScores: launch_use<kGemmSelectScores>(g, fast, small, (int)zdim, stream); break;
    default: JN_REQUIRE(false, kInvalidArgument, "unknown GEMM use %d", (int)use);
  }
  JN_LAUNCH_CHECK();
  return kOk;
}

// Batched C_b = op(A_b) . op(B_b) for b < batch (see BatchedGemm).
int gemm_batched(const BatchedGemm& m, GemmUse use, hipStream_t stream) {
  JN_REQUIRE(((use >= kGemmDenseScores && use <= kGemmRouteTargetGrad) || use == kGemmSelectScores ||
              gemm_use_dense_bf16(use)) &&
                 m.a_kcontig == kGemmUses[use].a_kc &&
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
  g.a_kscale = m.a_kscale; g.ks_bs = m.ks_bs;
  g.c_nscale = m.c_nscale;
  g.c_mscale = m.c_mscale; g.ms_bs = m.ms_bs;
  JN_REQUIRE(m.causal_k == kCausalKNone || (m.causal_k == kCausalKLower && m.M == m.K) ||
                 (m.causal_k == kCausalKUpper && m.M == m.K),
             kInvalidArgument, "a causal K range needs a square A over one element's nodes");
  g.causal_k = m.causal_k;
  if (m.epi) {
    JN_REQUIRE((use == kGemmDenseScores || use == kGemmDenseEdgeGrad || use == kGemmDenseEdgeGradBf16) &&
                   m.M == m.N && m.epi_ps && m.epi_part &&
                   (use == kGemmDenseScores || (m.epi_gds && m.epi_E)) && m.addend == nullptr &&
                   m.c_nscale == nullptr && m.c_mscale == nullptr,
               kInvalidArgument, "softsign epilogue needs a square dense score use and its operands");
    g.epi = 1; g.epi_causal = m.epi_causal ? 1 : 0;
    g.epi_bias = m.epi_bias; g.epi_ps = m.epi_ps; g.epi_gds = m.epi_gds; g.epi_E = m.epi_E;
    g.epi_part = m.epi_part;
  }
  if (m.fold) {
    JN_REQUIRE(gemm_use_fold(use) && (m.fold == 1 || m.fold == 2) && !m.epi && m.addend == nullptr &&
                   m.c_nscale == nullptr && m.c_mscale == nullptr && m.fold_head >= 0 && m.fold_head < 256,
               kInvalidArgument, "head fold needs a plain score use");
    g.fold = m.fold; g.fold_head = m.fold_head; g.fold_bias = m.fold_bias; g.fold_heads = m.fold_heads;
  }
  if (m.a_heads) {
    JN_REQUIRE(gemm_use_amask(use) && m.a_head >= 0 && m.a_head < 256, kInvalidArgument,
               "head mask needs a score-gradient use");
    g.a_heads = m.a_heads; g.a_head = m.a_head;
  }
  return launch_gemm(g, use, 1, stream);
}

// C[M][N] = X[M][K] . [W0;W1]^T with W0 rows [0, split) and W1 rows [split, N).
// x_bf16: X holds bf16 elements.
int gemm_project(const float* X, int64_t ldx, const float* W0, const float* W1, int split, int64_t ldw, float* C,
                 int64_t ldc, int M, int N, int K, hipStream_t stream, bool x_bf16) {
  GemmArgs g{};
  g.A = X; g.lda = ldx;
  g.B0 = W0; g.B1 = W1; g.ldb = ldw; g.b_split = split;
  g.C = C; g.ldc = ldc;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = K; g.c_split_stride = 0;
  return launch_gemm(g, x_bf16 ? kGemmProjectBf16 : kGemmProject, 1, stream);
}

// dX[M][N] = dP[M][K] . [W0;W1] (+ addend), W0 rows [0, split) of K.
// x_bf16: dX and the addend hold bf16 elements.
int gemm_grad_input(const float* dP, int64_t ldp, const float* W0, const float* W1, int split, int64_t ldw,
                    const float* addend, int64_t ld_add, float* dX, int64_t ldx, int M, int N, int K,
                    hipStream_t stream, bool x_bf16) {
  GemmArgs g{};
  g.A = dP; g.lda = ldp;
  g.B0 = W0; g.B1 = W1; g.ldb = ldw; g.b_split = split;
  g.C = dX; g.ldc = ldx;
  g.addend = addend; g.ld_add = ld_add;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = K; g.c_split_stride = 0;
  return launch_gemm(g, x_bf16 ? kGemmGradInputBf16 : kGemmGradInput, 1, stream);
}

// Split-K of the weight gradients (128 chunks at C4 gained 7 us in the GEMM
// and lost 4 in the reduce, for twice the partial buffer).
static int grad_weight_splits(int K) { return K >= 4096 ? 64 : (K >= 512 ? 8 : 1); }

size_t gemm_grad_weight_workspace(int M, int N, int K) {
  return (size_t)grad_weight_splits(K) * M * N * sizeof(float);
}

// dW[M][N] = dP^T . X with dP [K][M] (row stride ldp), X [K][N] (row stride ldx).
// Rows [0, m_split) of dW go to out0, the rest to out1.  Deterministic split-K.
// x_bf16: X holds bf16 elements.
int gemm_grad_weight(const float* dP, int64_t ldp, const float* X, int64_t ldx, float* out0, float* out1, int m_split,
                     int M, int N, int K, float* partial, hipStream_t stream, bool x_bf16) {
  int splits = grad_weight_splits(K);
  int k_chunk = (K + splits - 1) / splits;
  // chunks of whole K slices: 32 (the fp32 kernels' 16, gemm_x3_kernel's 32), 64 (the bf16 MFMA kernel)
  static_assert(kX3K % kGBK == 0 && kX3K % kFastBK == 0, "fp32 split-K chunks serve every fp32 kernel");
  const int kq = x_bf16 ? kBfK : kX3K;
  k_chunk = (k_chunk + kq - 1) / kq * kq;
  GemmArgs g{};
  g.A = dP; g.lda = ldp;
  g.B0 = X; g.B1 = X; g.ldb = ldx; g.b_split = 1 << 30;
  g.C = partial; g.ldc = N;
  g.M = M; g.N = N; g.K = K;
  g.k_chunk = k_chunk; g.c_split_stride = (int64_t)M * N;
  int rc = launch_gemm(g, x_bf16 ? kGemmGradWeightBf16 : kGemmGradWeight, splits, stream);
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
