// Launch interfaces shared between the kernel translation units and the C ABI.
#pragma once

#include "jn_common.hpp"

namespace jakal {

// ---- score + top-k select (jn_select.hip) ---------------------------------
struct SelectArgs {
  const float* q;       // query rows, row stride ldq, batch stride q_batch_stride
  const float* key;     // key rows, row stride ldk, batch stride k_batch_stride
  int64_t ldq, ldk;
  int64_t q_batch_stride, k_batch_stride;
  const float* scale;   // [r] or null
  const float* bias;    // scalar or null
  int scale_on_query;
  float temperature;
  int B, Nq, Nk, r, k;
  int32_t* out_idx;     // [B, Nq, k]
  float* out_score;     // [B, Nq, k]
  void* ws;             // scratch of select_workspace_bytes(B, Nk, r) bytes (split mode)
  size_t ws_bytes;
  // set by launch_topk_select from ws (split mode): split key rows (fp16 bits)
  // and one key exponent per batch element
  const uint16_t* split_key;
  const int* split_exp;
  // Multi-head max aggregation (heads > 1): r = heads * head_rank ranks, head h
  // owning ranks [h * head_rank, (h + 1) * head_rank) of q, key and scale; bias
  // is [heads] or null.  A pair's score is max_h (dot_h + bias[h]) / T.
  int heads, head_rank;
  // bf16 score operands (bf16 layers): bf16(q * scale) . bf16(key), accumulated
  // in fp32 on bf16 MFMAs, whatever the select mode (one head only).
  int bf16;
};
int launch_topk_select(const SelectArgs& a, hipStream_t stream);
constexpr int kSelectMaxK = 64;
// Selects beyond the register kernels' limits (k > kSelectMaxK or more than
// 65,535 keys) score rows into the workspace with an fp32 MFMA GEMM and pick
// each row's k best by radix select (jn_select_large.hip), up to this k.
constexpr int kSelectLargeMaxK = 4096;
int launch_topk_select_large(const SelectArgs& a, hipStream_t stream);
// Score arithmetic of the select: kSelectSplitF16 (default) runs the score
// tiles on fp16 MFMAs over two-term fp16 splits of the operands (about 22
// significant bits per operand, fp32 accumulation); kSelectF32 runs them on
// fp32 MFMAs.  The split needs select_workspace_bytes() of scratch, which is
// reported for every mode so that a size query and a later launch agree even
// when another thread changes the mode in between.
constexpr int kSelectSplitF16 = 0;
// Split fp16 on one kernel only (tests): the per-wave streaming kernel, or the
// 4-wave cooperative (LDS-staged) kernel whenever the rank is at most 64.
// kSelectSplitF16 picks the cooperative kernel for rank <= 64 on grids of at
// least 512 workgroups, else the per-wave kernel.  (Mode 3 is retired.)
constexpr int kSelectSplitF16Wave = 2;
constexpr int kSelectSplitF16Coop4 = 4;
// Split fp16 on the key-split per-wave kernel whenever k <= 16 (tests); mode 0
// picks it for k <= 16 on grids below 256 workgroups with >= 192 keys.
constexpr int kSelectSplitF16KeySplit = 5;
// Split fp16 on the register kernels only: mode 0 as it was before the
// small-key select (tests and A/B timing).
constexpr int kSelectSplitF16Register = 6;
constexpr int kSelectF32 = 1;
// Rows of at most kSelectSmallMaxKeys keys (one head, fp32 operands, k <= 64):
// mode 0 scores the whole row into LDS on fp32 MFMAs and radix-selects it
// (jn_select_small.hip) instead of running the register select's merges.
constexpr int kSelectSmallMaxKeys = 1024;
bool select_small_fits(const SelectArgs& a);
int launch_topk_select_small(const SelectArgs& a, hipStream_t stream);
// The mode is process-wide and atomic; each launch reads it once.
int select_mode();
void set_select_mode(int mode);
size_t select_workspace_bytes(int64_t B, int64_t Nk, int64_t r);
// Multi-head: each head's ranks padded to whole 32-rank MFMA K-steps.
size_t select_workspace_bytes_heads(int64_t B, int64_t Nk, int64_t head_rank, int64_t heads);
// Heads per pair score (all kernels); the select takes at most 4 K-steps of 32
// ranks over all heads (heads * ceil(head_rank / 32) <= 4).
constexpr int kMaxHeads = 8;
bool select_heads_fit(int64_t head_rank, int64_t heads);
// Ranks.  The register paths (the register select, the row and column kernels'
// rank slots, multi-head scores) hold up to kRegRank ranks over all heads; one
// head takes up to kMaxRank, the ranks beyond kRegRank running the
// scored-rows select and the rank-chunked gradient kernels below.
constexpr int kRegRank = 128;
constexpr int kMaxRank = 1024;

// ---- fp32 MFMA GEMMs (jn_gemm.hip) ----------------------------------------
// x_bf16: the layer operand X (and dX with its addend) holds bf16 elements.
int gemm_project(const float* X, int64_t ldx, const float* W0, const float* W1, int split, int64_t ldw, float* C,
                 int64_t ldc, int M, int N, int K, hipStream_t stream, bool x_bf16 = false);
int gemm_grad_input(const float* dP, int64_t ldp, const float* W0, const float* W1, int split, int64_t ldw,
                    const float* addend, int64_t ld_add, float* dX, int64_t ldx, int M, int N, int K,
                    hipStream_t stream, bool x_bf16 = false);
size_t gemm_grad_weight_workspace(int M, int N, int K);
// Batched fp32 GEMM C_b[M][N] = A_b . B_b (+ addend_b), b < batch.
//   A(m, k) = a_kcontig ? A[m*lda + k] : A[k*lda + m], times a_kscale[k] if given
//   B(k, n) = b_kcontig ? B[n*ldb + k] : B[k*ldb + n]
//   C(m, n) = sum_k A(m,k) B(k,n), times c_nscale[n] if given, plus addend
struct BatchedGemm {
  const float* A; int64_t lda, a_bs; bool a_kcontig;
  const float* B; int64_t ldb, b_bs; bool b_kcontig;
  float* C; int64_t ldc, c_bs;
  const float* addend; int64_t ld_add, add_bs;
  const float* a_kscale; int64_t ks_bs;  // optional, per batch element at stride ks_bs
  const float* c_nscale;
  const float* c_mscale; int64_t ms_bs;  // optional: C(m, n) *= c_mscale[m], per batch element at stride ms_bs
  int M, N, K, batch;
  // Causal structure of a square dense product (M == K or N == K over one
  // batch element's nodes): kCausalKLower when A(m, k) = 0 for k > m (each
  // tile of rows stops its K loop after its last row), kCausalKUpper when
  // A(m, k) = 0 for k < m (it starts at its first row).  Skipped terms are
  // exact zeros of the causal edge matrix, so results do not change.
  int causal_k;
  // softsign epilogue of kGemmDenseScores / kGemmDenseEdgeGrad (M == N): see
  // GemmArgs in jn_gemm.hip; part is [batch, M, dense_epi_parts(N)]
  int epi, epi_causal;
  const float* epi_bias;
  const float* epi_ps;
  const float* epi_gds;
  const float* epi_E;
  float* epi_part;
  // Head-max fold of max-aggregated multi-head scores (uses dense_scores,
  // route_logits, select_scores; no other epilogue): the product is one
  // head's scores, y = C + fold_bias[0] (null: 0).  fold = 1 (the first head)
  // stores y; fold = 2 stores y where it exceeds the stored value (ties keep
  // the earlier head).  fold_heads (bytes indexed like C, or null) records
  // fold_head wherever y is stored.
  int fold, fold_head;
  const float* fold_bias;
  uint8_t* fold_heads;
  // Head mask of A (uses dense_target_grad, dense_source_grad,
  // route_source_grad, route_target_grad): A(m, k) counts only where
  // a_heads (bytes indexed like A: same strides, in elements) equals a_head.
  const uint8_t* a_heads;
  int a_head;
};
constexpr int kCausalKNone = 0, kCausalKLower = 1, kCausalKUpper = 2;
// Partial sums per row that the dense softsign epilogue writes (32 columns each).
inline int dense_epi_parts(int n) { return (n + 31) / 32; }
enum GemmUse {
  kGemmProject, kGemmGradInput, kGemmGradWeight,
  kGemmDenseScores, kGemmDenseAggregate, kGemmDenseEdgeGrad, kGemmDenseValueGrad, kGemmDenseTargetGrad,
  kGemmDenseSourceGrad,
  kGemmRouteLogits, kGemmRouteAggregate, kGemmRouteEdgeGrad, kGemmRouteValueGrad, kGemmRouteSourceGrad,
  kGemmRouteTargetGrad,
  kGemmProjectBf16, kGemmGradInputBf16, kGemmGradWeightBf16,
  kGemmSelectScores,
  // bf16 dense layers: E . pv and E^T . gdv with E rounded to bf16 (bf16 C),
  // gdv . pv^T from bf16 operands (fp32 C, softsign epilogue as dense_edge_grad)
  kGemmDenseAggregateBf16, kGemmDenseValueGradBf16, kGemmDenseEdgeGradBf16,
  // bf16 dense transitions: R^T diag(rho) pv with R rounded to bf16 after
  // its k scale (bf16 C), diag(rho) R gdv (bf16 C), pv . gdv^T (fp32 C)
  kGemmRouteAggregateBf16, kGemmRouteValueGradBf16, kGemmRouteEdgeGradBf16,
};
int gemm_batched(const BatchedGemm& m, GemmUse use, hipStream_t stream);
// Workgroup tile of every later GEMM launch: 0 = chosen per call, 64 or 128 = forced.
void set_gemm_tile(int tile);
int gemm_grad_weight(const float* dP, int64_t ldp, const float* X, int64_t ldx, float* out0, float* out1, int m_split,
                     int M, int N, int K, float* partial, hipStream_t stream, bool x_bf16 = false);

// ---- edge-list kernels (jn_edges.hip) -------------------------------------
struct RowsFwdArgs {
  const int32_t* idx;
  const float* score;
  int k;
  int compress;
  const float* ps;   // [B, Nk]
  const float* pv;   // [B, Nk, D] row stride ld_pv
  int64_t ld_pv;
  int Nq, Nk, D;
  int64_t rows;
  float* out_state;  // [rows]
  float* out_val;    // [rows, D]
  int slab;          // columns per slab (set by the launcher)
  int bf16;          // pv and out_val hold bf16 elements (the pointers are reinterpreted)
};
int launch_rows_forward(const RowsFwdArgs& a, hipStream_t stream);

struct RowsBwdArgs {
  const int32_t* idx;
  const float* score;
  int k;
  int compress;
  float inv_temperature;
  const float* ps;        // [B, Nk]
  const float* pv;        // [B, Nk, D], row stride ld_pv
  int64_t ld_pv;
  const float* gds;       // [rows]
  const float* gdv;       // [rows, D]
  const float* key;       // key projection rows, row stride ldk (batch stride Nk*ldk)
  int64_t ldk;
  const float* qscale;    // [r] scale applied to dQ (null = 1)
  int r;
  int Nq, Nk, D;
  int64_t rows;
  float* g_score;         // [rows, k]
  float* coef;            // [rows, k]
  float* dq;              // [rows, r], row stride lddq
  int64_t lddq;
  float* rowsum_gs;       // [rows] ([rows, heads] with heads > 1)
  // Multi-head (heads > 1): edge e's score is head ehead[e]'s, so its gradient
  // reaches only that head's ranks [h * head_rank, (h + 1) * head_rank) of dq
  // and its bias partial column h.
  const uint8_t* ehead;   // [rows, k]
  int heads, head_rank;
  int bf16;               // pv and gdv hold bf16 elements (the pointers are reinterpreted)
  // The dot products <gdv[i], pv[j]> of every edge are already in g_score + coef
  // (two partial sums, e.g. from launch_band_dots): no value rows are read.
  int dots_given;
  int dot_parts;          // with dots_given: 1 = g_score alone holds the dots (0 or 2: both buffers)
  // With dots_given: the partials are in record order, edge e's at
  // dot_pos[e] of dots0 and coef (coef is then not written).
  const int32_t* dot_pos; // [rows, k] or null
  const float* dots0;     // [rows * k] (with dot_pos)
};
int launch_rows_backward(const RowsBwdArgs& a, hipStream_t stream);

// Rank-chunked query-side gradient for ranks beyond kRegRank (one head):
//   dq[i, :] = qscale * sum_e g[i, e] key[b * Nk + idx[i, e], :]
// over row i's edges in index order (absent edges: idx < 0).
struct RankRowsArgs {
  const int32_t* idx;    // [rows, k]
  const float* g;        // [rows, k] per-edge score gradient
  int k;
  const float* key;      // key rows of batch element b at b * Nk, stride ldk
  int64_t ldk;
  const float* qscale;   // [r] (null = 1)
  int r, Nq, Nk;
  int64_t rows;          // B * Nq
  float* dq;             // [rows, r], stride lddq
  int64_t lddq;
};
int launch_rank_rows_grad(const RankRowsArgs& a, hipStream_t stream);

// ---- causal-band kernels of window edge lists (jn_band.hip) --------------
// Slot e of query row i is key i - (k - 1 - e) (absent below 0); N query rows
// and N keys per batch element.
constexpr int kBandMaxK = 128;
struct BandAggArgs {
  int B, N, k, D;
  int trans;            // 0: forward over query rows; 1: column pass over key rows
  int compress;         // forward: compress kind of the edge scores
  const int32_t* idx;   // forward: [B*N, k] edge index
  const float* score;   // forward: [B*N, k] edge scores
  const float* coef;    // column pass: [B*N, k] edge coefficients
  const float* state;   // forward: ps [B*N]; column pass: gds [B*N] (null: no state sums)
  const float* val;     // forward: pv; column pass: gdv -- [B*N] rows of stride ld_val
  int64_t ld_val;
  float* out_state;     // forward: delta_state; column pass: grad_ps -- [B*N] or null
  float* out;           // forward: delta_val; column pass: grad_pv -- [B*N] rows of stride ld_out
  int64_t ld_out;
  int bf16;             // val and out hold bf16 elements
};
struct BandDotsArgs {
  int B, N, k, D;
  const float* gdv;  // [B*N] rows of stride ld_gdv
  int64_t ld_gdv;
  const float* pv;   // [B*N] rows of stride ld_pv
  int64_t ld_pv;
  float* g_score;    // [B*N, k]: dot partial over the first half of D
  float* coef;       // [B*N, k]: dot partial over the second half
  int bf16;          // gdv and pv hold bf16 elements
  // Score mode (score_out non-null, fp32 rows): the window's pairwise scores.
  // One pass over all D columns of gdv (the query projection, column d times
  // ascale[d] when given) against pv (the key projection); slot e of row i
  // gets score_out = (dot + bias[0]) * inv_temperature and idx_out = its key
  // i - (k - 1) + e, or 0 and -1 before the first row.
  const float* ascale;
  const float* bias;
  float inv_temperature;
  float* score_out;
  int32_t* idx_out;
};
// Whether the band kernels take these operands (k <= kBandMaxK, whole 16-byte
// packs per row, 16-byte aligned rows); otherwise the edge kernels run.
bool band_kernels_fit(int k, int D, int64_t ld_a, int64_t ld_b, const void* pa, const void* pb, bool bf16);
// Window kernels of every later call (process-wide, atomic): 0 = band kernels
// where they fit, 1 = edge kernels only.
void set_window_kernels(int mode);
int window_kernels();
int launch_band_aggregate(const BandAggArgs& a, hipStream_t stream);
int launch_band_dots(const BandDotsArgs& a, hipStream_t stream);

// Fixed edge lists with low-rank scores: the causal band (all_keys = 0: slot e
// of query row i is key i - (width - 1 - e), absent when negative) or every
// key (all_keys = 1: slot e is key e, width = Nk).
struct WindowScoreArgs {
  const float* q;        // query projection rows (global row b*Nq + i), stride ldq
  const float* key;      // key projection rows (global row b*Nk + j), stride ldk
  int64_t ldq, ldk;
  const float* scale;    // [r] applied to the query (null = 1)
  const float* bias;     // scalar or null
  float inv_temperature; // score = (dot + bias) * inv_temperature
  int B, Nq, Nk, r, width;
  int all_keys;          // 2: the edge list idx is given (only the heads are written)
  int32_t* idx;          // [B*Nq, width]
  float* score;          // [B*Nq, width]
  // Multi-head (heads > 1): score = max_h (dot_h + bias[h]) * inv_temperature
  // over head rank slices of head_rank; head[e] = the first head attaining it.
  int heads, head_rank;
  uint8_t* head;         // [B*Nq, width] or null
};
int launch_window_scores(const WindowScoreArgs& a, hipStream_t stream);

// ---- transition routing (jn_route.hip) -------------------------------------
int launch_route_coef(const int32_t* idx, const float* logit, const float* rho, int k, int compress, int64_t rows,
                      float* coef, hipStream_t stream);

struct RouteRowsBwdArgs {
  const int32_t* idx;    // [rows, k] destination per edge (-1 absent)
  const float* logit;    // [rows, k]
  int k;
  int compress;          // 0 softmax, 1 signed |l| softmax
  float inv_temperature;
  const float* rho;      // [rows] sender strength
  const float* ps;       // [rows] projected state of the sources
  const float* pv;       // [rows, ld_pv] projected values of the sources
  int64_t ld_pv;
  const float* gds;      // [B*Nd] grad of delta_state
  const float* gdv;      // [B*Nd, D] grad of delta_val
  const float* key;      // destination projection rows [B*Nd], stride ldk
  int64_t ldk;
  const float* qscale;   // [r] core weight (scales dQ)
  int r, Ns, Nd, D;
  int64_t rows;          // B*Ns
  float* g_logit;        // [rows, k]
  float* grad_rho;       // [rows] (null: skip)
  float* grad_ps;        // [rows] (null: skip)
  float* grad_pv;        // [rows, ld_gpv] (null: skip)
  int64_t ld_gpv;
  float* dq;             // [rows, r], stride lddq
  int64_t lddq;
  float* rowsum;         // [rows] ([rows, heads] with heads > 1)
  const uint8_t* ehead;  // multi-head: [rows, k] head of each edge (see RowsBwdArgs)
  int heads, head_rank;
  int bf16;              // pv, gdv and grad_pv hold bf16 elements (the pointers are reinterpreted)
};
int launch_route_rows_backward(const RouteRowsBwdArgs& a, hipStream_t stream);

// ---- dense propagation (jn_dense.hip) --------------------------------------
int launch_dense_compress(float* S, const float* bias, const float* ps, int B, int N, int compress, int causal,
                          float* delta_state, hipStream_t stream);
int launch_dense_compress_backward(float* G, const float* E, const float* gds, const float* ps, int B, int N,
                                   int compress, int causal, float* rowsum, hipStream_t stream);
int launch_dense_colsum(const float* E, const float* w, int B, int N, float* out, hipStream_t stream);
// out[row] = sum_t part[row * P + t], t < P (fixed order)
int launch_dense_part_rowsum(const float* part, int P, int64_t rows, float* out, hipStream_t stream);
// rowsum[row, h] = sum_j G[row, j] [head[row, j] == h] over the N columns of
// each of `rows` rows (row stride ld), h < H: bias gradients of max-aggregated
// multi-head scores, in a fixed order.
int launch_head_rowsum(const float* G, const uint8_t* head, int N, int64_t ld, int64_t rows, int H, float* rowsum,
                       hipStream_t stream);
// out[b, j] = sum_i M[b, i, j] a[b, i] (c[b, i] if given), i < Nr, j < Nc, fixed order
int launch_colsum_rows(const float* M, const float* a, const float* c, int B, int Nr, int Nc, float* out,
                       const char* name, hipStream_t stream);

// ---- dense transitions (jn_route_dense.hip) --------------------------------
int launch_route_dense_compress(float* L, const float* bias, float inv_temp, int B, int Ns, int Nd, int kind,
                                hipStream_t stream);
int launch_route_dense_colsum(const float* R, const float* a, const float* c, int B, int Nr, int Nc, float* out,
                              hipStream_t stream);
int launch_route_dense_compress_backward(float* H, const float* R, const float* rho, const float* ps,
                                         const float* gds, int B, int Ns, int Nd, int kind, float inv_temp,
                                         float* grad_rho, float* grad_ps, float* rowsum, hipStream_t stream);
int launch_scale_grad_partials(float* dps, int64_t ld_dps, const float* src, int64_t ld_src, const float* w_hat,
                               int r, int64_t rows, float* part, hipStream_t stream);

struct CsrArgs {
  const int32_t* idx;
  int k;
  int B, Nq, Nk;
  int32_t* tile_base;  // [B, T + 1, Nk], T = csr_tiles(B, Nq): build scratch (csr_table_entries)
  int32_t* seg_start;  // [B, Nk + 1]
  // [B * Nq * k] edge records grouped by key: {row | head << kRecHeadShift
  // (int bits), coef[e], g_score[e], coef[e] * gds[row]}; a null source
  // pointer gives 0
  float4* rec;
  const float* coef;     // [B * Nq, k] or null
  const float* g_score;  // [B * Nq, k] or null
  const float* gds;      // [B * Nq] or null
  const uint8_t* ehead;  // [B * Nq, k] head of each edge, or null (head 0)
  int rec_eid;           // 1: record word 2 holds the edge id (int bits) instead of g_score[e]
  int32_t* pos;          // [B * Nq * k] or null: each edge's record index (batch offset included)
  // Without coef: record coefficients softsign(score[e]) (compress kind 0 only)
  const float* score;    // [B * Nq, k] or null
  int compress;
};
constexpr int kCsrTile = 64;
// Rows per tile of the CSR build (whole kCsrTile-row chunks, at most 1024) and
// the tiles of Nq rows: tile_base holds csr_tiles(B, Nq) * Nk counts per batch element.
int csr_tile_rows(int64_t B, int64_t Nq);
inline int64_t csr_tiles(int64_t B, int64_t Nq) {
  const int64_t tr = csr_tile_rows(B, Nq);
  return (Nq + tr - 1) / tr;
}
inline int64_t csr_table_entries(int64_t B, int64_t Nq, int64_t Nk) { return B * (csr_tiles(B, Nq) + 2) * Nk; }
// The build's table of per-tile key counts and key degree prefixes (int32)
// has csr_table_entries(B, Nq, Nk) = B * (csr_tiles + 2) * Nk entries, at most
// kCsrMaxTableEntries (1 GiB); larger groupings are rejected as unsupported.
constexpr int64_t kCsrMaxTableEntries = 1LL << 28;
bool csr_table_fits(int64_t B, int64_t Nq, int64_t Nk);
// An edge record's first word holds its row below bit kRecHeadShift and its
// head above (multi-head scores), so rows stay below 2^27.
constexpr int kRecHeadShift = 27;
constexpr int kRecRowMask = (1 << kRecHeadShift) - 1;
int launch_csr(const CsrArgs& a, hipStream_t stream);
// The two halves of launch_csr: the layout (per-tile edge counts, segment
// starts and per-tile slots; reads only the edge index) and the fill (the
// records; reads the coefficients, score gradients and state gradients as
// well).
int launch_csr_layout(const CsrArgs& a, hipStream_t stream);
int launch_csr_fill(const CsrArgs& a, hipStream_t stream);

// A second stream of the calling thread for the current device, with an event
// pair to fork work onto it from `origin` and join it back: kernels that do not
// depend on each other run side by side (and as parallel branches of a captured
// graph).  Null when none can be made here (first use during a capture).
struct SideStream {
  hipStream_t stream;
  hipEvent_t fork, join;
  // set by fork_to, cleared by join_from: the stream forked from
  mutable bool open;
  mutable hipStream_t origin;
};
SideStream* side_stream(hipStream_t origin);
// side_stream(origin) for problems of at least 2^18 edges, else null
const SideStream* side_stream_for(hipStream_t origin, int64_t edges);
int fork_to(const SideStream* s, hipStream_t origin);   // s->stream waits for origin's work so far
int join_from(const SideStream* s, hipStream_t origin); // origin waits for s->stream's work so far
// Declared at the top of a call that forks: when the call returns (an error
// return between fork_to and join_from included), a side stream of this
// thread still forked is joined back into the stream it was forked from, so
// no return leaves its origin stream -- or a graph under capture -- with an
// unjoined fork.
struct SideForkGuard {
  SideForkGuard() = default;
  SideForkGuard(const SideForkGuard&) = delete;
  SideForkGuard& operator=(const SideForkGuard&) = delete;
  ~SideForkGuard();
};

struct ColsBwdArgs {
  const int32_t* seg_start;  // [B, Nk + 1]
  const float4* rec;         // edge records grouped by key (CsrArgs), batch b at offset b*Nq*k
  int k;
  const float* gdv;          // [rows, D]
  const float* q;            // query projection rows (global row index), stride ldq
  int64_t ldq;
  const float* key;          // key projection rows (global column index), stride ldk
  int64_t ldk;
  const float* kscale;       // [r] (null = 1)
  int r;
  int B, Nq, Nk, D;
  float* grad_pv;            // [B*Nk, D] (null: skip)
  int64_t ld_gpv;
  float* grad_ps;            // [B*Nk] (null: skip)
  float* dk;                 // [B*Nk, r], stride lddk (null q: skip dk and part_c)
  int64_t lddk;
  float* part_c;             // [cols_backward_parts(B*Nk), r] or null
  const char* profile_name;  // label for the gather's kernel timer (null: "cols_gather_kernel")
  // Multi-head (heads > 1): a record's g_score reaches only its head's ranks of dk.
  int heads, head_rank;
  int bf16;                  // gdv and grad_pv hold bf16 elements (the pointers are reinterpreted)
  // Causal band (window edge lists, Nq == Nk): band != 0 builds each record
  // from the edge arrays instead of seg_start / rec.  Key j's incoming edges
  // are rows j + t for 0 <= t < min(k, Nk - j), row j + t holding j in slot
  // k - 1 - t, so the records come in increasing row order as the CSR lists
  // them.
  int band;
  const float* coef;         // [B * Nq, k]
  const float* g_score;      // [B * Nq, k]
  const float* gds;          // [B * Nq] or null (band records: word 3 is then 0; fused pass: grad_ps sums coef * gds[row])
  const uint8_t* ehead;      // [B * Nq, k] or null (head 0)
  // CSR records whose word 2 is the edge id (CsrArgs::rec_eid): the key
  // gradient reads g_score[id].
  int rec_eid;
  // Fused column pass (launch_cols_gather_dots): the value rows pv [B*Nk, D]
  // (stride ld_pv) and the per-edge slab partials of <gdv[i], pv[j]>, slab 0
  // into dots0 and slab 1 into dots1 ([B * Nq * k], by record index).
  const float* pv;
  int64_t ld_pv;
  float* dots0;
  float* dots1;
};
int cols_backward_parts(int64_t total_cols);
// Column slabs of the fused column pass (kWave 16-byte packs each) when it
// applies to these rows (CSR records, 16-byte aligned rows, at most two
// slabs), else 0.
int cols_gather_dots_slabs(const ColsBwdArgs& a);
// grad_pv, grad_ps and the dot-product slab partials in one pass over the
// columns' records (records with edge ids); needs cols_gather_dots_slabs(a) > 0.
int launch_cols_gather_dots(const ColsBwdArgs& a, hipStream_t stream);
// coef[row, e] = the row's compressed score of edge e (0 for absent edges),
// as the row kernels compute it.
int launch_edge_coefficients(const int32_t* idx, const float* score, int64_t rows, int k, int compress, float* coef,
                             hipStream_t stream);

// Unit-norm scale vectors: out = w / max(||w||, eps) per row of [rows, r], or
// with grad (non-null) the gradient of that map at w.
int launch_unit_scale(const float* w, const float* grad, int64_t rows, int64_t r, float eps, float* out,
                      hipStream_t stream);
int launch_cols_backward(const ColsBwdArgs& a, hipStream_t stream);

// Scale-vector and bias gradients: grad_c[r] from the [nparts, r] partials,
// grad_bias[nbias] from the [nrows, nbias] row sums (column h: head h's bias).
size_t finalize_stage_floats(int r, int nbias = 1);
int launch_finalize_small_grads(const float* part_c, int nparts, int r, float* grad_c, int accumulate_c,
                                const float* rowsum, int64_t nrows, float* grad_bias, float* stage,
                                hipStream_t stream, int nbias = 1);

}  // namespace jakal
