// The reference extension's raw edge ops (the *_cuda ops its Python dispatcher
// probes and composes into its own autograd functions), on this library's
// kernels:
//   jn_lowrank_topk_select_heads  the select of low_rank_pairwise_topk_forward_cuda and
//                               low_rank_propagation_topk_forward_cuda, max over heads
//                               (cu:740-813 one head, 881-930 [B, H, N, r] heads)
//   jn_softsign_backward        softsign_backward_cuda       (jakal_net_native_cuda.cu:2177-2190, 3426-3453)
//   jn_softmax_backward         softmax_backward_cuda        (cu:2192-2212, 3455-3483)
//   jn_edge_aggregate           the gather-aggregate of low_rank_propagation_topk_forward_cuda
//   jn_edge_reduce_backward     query_topk_reduce_backward_cuda (cu:2112-2175, 3352-3424)
//   jn_route_topk_aggregate     the route and destination sums of
//                               low_rank_pairwise_topk_forward_cuda (cu:2420-2543)
//   jn_lowrank_pair_backward    low_rank_pairwise_topk_backward_cuda (cu:2259-2322, 3792-3866)
// The reference scatters with float atomics; here every sum over a key's
// incoming edges walks its CSR segment (the same deterministic transpose as
// the propagation backward), so results repeat bit for bit.
//
// Row kernels below: one wavefront per row, lanes over the row's elements,
// sums by the wave's butterfly (fixed order).
#include "../../include/jakal_net_hip.h"
#include "jn_internal.hpp"

namespace jakal {
namespace {

__global__ __launch_bounds__(256) void softsign_backward_kernel(const float* __restrict__ s,
                                                                const float* __restrict__ g, int64_t n,
                                                                float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float d = 1.0f + fabsf(s[i]);
  out[i] = g[i] / (d * d);
}

// grad_s = p (g - sum_e p g) over each row of k
__global__ __launch_bounds__(256) void softmax_rows_backward_kernel(const float* __restrict__ p,
                                                                    const float* __restrict__ g, int64_t rows, int k,
                                                                    float* __restrict__ out) {
  const int lane = lane_id();
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const float* pr = p + row * k;
  const float* gr = g + row * k;
  float dot = 0.0f;
  for (int e = lane; e < k; e += kWave) dot += pr[e] * gr[e];
  dot = wave_sum(dot);
  for (int e = lane; e < k; e += kWave) out[row * k + e] = pr[e] * (gr[e] - dot);
}

// grad_edge[i, e] = gds[i] ps[j] + <gdv[i], pv[j]>, j = idx[i, e] (batch-local;
// absent edges get 0)
__global__ __launch_bounds__(256) void edge_dots_kernel(const int32_t* __restrict__ idx, const float* __restrict__ ps,
                                                        const float* __restrict__ pv, const float* __restrict__ gds,
                                                        const float* __restrict__ gdv, int Nq, int Ns, int k, int D,
                                                        int64_t rows, float* __restrict__ out) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const int64_t b = row / Nq;
  const float* g = gdv + row * D;
  const float gs = gds[row];
  for (int e = 0; e < k; ++e) {
    const int j = idx[row * k + e];
    float dot = 0.0f;
    if (j >= 0) {
      const float* v = pv + (b * Ns + j) * D;
      for (int d = lane; d < D; d += kWave) dot += g[d] * v[d];
    }
    dot = wave_sum(dot);
    if (lane == 0) out[row * k + e] = j >= 0 ? gs * ps[b * Ns + j] + dot : 0.0f;
  }
}

// dPq[i, r] = w[r] sum_e g[i, e] Ps[j, r] and rowsum[i] = sum_e g[i, e], j = idx[i, e]
__global__ __launch_bounds__(256) void pair_rows_grad_kernel(const int32_t* __restrict__ idx,
                                                             const float* __restrict__ g,
                                                             const float* __restrict__ Ps,
                                                             const float* __restrict__ w, int Nq, int Ns, int r,
                                                             int k, int64_t rows, float* __restrict__ dPq,
                                                             float* __restrict__ rowsum) {
  const int lane = lane_id();
  const int64_t row = (int64_t)xcd_swizzle(blockIdx.x, gridDim.x) * 4 + wave_id();
  if (row >= rows) return;
  const int64_t b = row / Nq;
  float acc0 = 0.0f, acc1 = 0.0f, gsum = 0.0f;
  for (int e = 0; e < k; ++e) {
    const int j = idx[row * k + e];
    if (j < 0) continue;
    const float ge = g[row * k + e];
    const float* key = Ps + (b * Ns + j) * r;
    if (lane < r) acc0 += ge * key[lane];
    if (lane + kWave < r) acc1 += ge * key[lane + kWave];
    gsum += ge;
  }
  if (lane < r) dPq[row * r + lane] = w[lane] * acc0;
  if (lane + kWave < r) dPq[row * r + lane + kWave] = w[lane + kWave] * acc1;
  if (lane == 0) rowsum[row] = gsum;
}

__global__ __launch_bounds__(256) void scale_kernel(const float* __restrict__ in, float s, int64_t n,
                                                    float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = in[i] * s;
}

struct CsrScratch {
  int32_t* table;
  int32_t* seg;
  float4* rec;
  size_t bytes;
};

CsrScratch carve_csr(Workspace& ws, int64_t B, int64_t Nq, int64_t Nk, int64_t k) {
  CsrScratch c{};
  c.table = ws.take<int32_t>(csr_table_entries(B, Nq, Nk));
  c.seg = ws.take<int32_t>(B * (Nk + 1));
  c.rec = ws.take<float4>(B * Nq * k);
  return c;
}

int check_raw_edges(int64_t B, int64_t Nq, int64_t Nk, int64_t k, int64_t D) {
  JN_REQUIRE(B >= 1 && Nq >= 1 && Nk >= 1 && k >= 1 && D >= 0, kInvalidArgument,
             "batch, node counts and edges per row must be positive");
  JN_REQUIRE(B * Nq * k < (1LL << 31) && B * Nq <= kRecRowMask && B * Nk * (D > 0 ? D : 1) < (1LL << 31) &&
                 csr_table_fits(B, Nq, Nk),
             kUnsupported, "edge list too large");
  return kOk;
}

int grid_rows(int64_t rows) {
  const int64_t blocks = (rows + 3) / 4;
  return blocks < (1LL << 31) ? (int)blocks : -1;
}

}  // namespace
}  // namespace jakal

using namespace jakal;

extern "C" {

size_t jn_lowrank_topk_select_heads_workspace_bytes(int64_t batch, int64_t nk, int64_t head_rank, int64_t heads) {
  if (heads == 1) return select_workspace_bytes(batch, nk, head_rank);
  return select_workspace_bytes_heads(batch, nk, head_rank, heads);
}

int jn_lowrank_topk_select_heads(const float* query, const float* key, const float* bias, int64_t batch, int64_t nq,
                                 int64_t nk, int64_t head_rank, int64_t heads, int64_t topk, int32_t* out_index,
                                 float* out_score, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  JN_REQUIRE(query && key && out_index && out_score, kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(batch >= 1 && nq >= 1 && nk >= 1, kInvalidArgument, "batch, nq, nk must be positive");
  JN_REQUIRE(heads >= 1 && heads <= kMaxHeads && head_rank >= 1 && heads * head_rank <= 128, kUnsupported,
             "%lld heads of rank %lld: at most %d heads and 128 ranks in all", (long long)heads,
             (long long)head_rank, kMaxHeads);
  JN_REQUIRE(batch * nq * topk < (1LL << 31) && nq < (1LL << 31) && nk < (1LL << 31), kUnsupported,
             "problem too large");
  const int64_t r = heads * head_rank;
  SelectArgs a{};
  a.q = query;
  a.key = key;
  a.ldq = r;
  a.ldk = r;
  a.q_batch_stride = nq * r;
  a.k_batch_stride = nk * r;
  a.bias = bias;
  a.temperature = 1.0f;
  a.B = (int)batch;
  a.Nq = (int)nq;
  a.Nk = (int)nk;
  a.r = (int)r;
  a.k = (int)topk;
  a.heads = (int)heads;
  a.head_rank = (int)head_rank;
  a.out_idx = out_index;
  a.out_score = out_score;
  a.ws = workspace;
  a.ws_bytes = workspace_bytes;
  return launch_topk_select(a, static_cast<hipStream_t>(stream));
}

int jn_softsign_backward(const float* scores, const float* grad_edges, int64_t count, float* grad_scores,
                         jn_stream_t stream) {
  JN_REQUIRE(count >= 0 && (count == 0 || (scores && grad_edges && grad_scores)), kInvalidArgument,
             "null tensor pointer");
  if (count == 0) return kOk;
  JN_REQUIRE((count + 255) / 256 < (1LL << 31), kUnsupported, "too many elements");
  hipStream_t st = static_cast<hipStream_t>(stream);
  JN_PROFILE("softsign_backward_kernel", st);
  hipLaunchKernelGGL(softsign_backward_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st, scores,
                     grad_edges, count, grad_scores);
  JN_LAUNCH_CHECK();
  return kOk;
}

int jn_softmax_backward(const float* routes, const float* grad_routes, int64_t rows, int64_t k, float* grad_scores,
                        jn_stream_t stream) {
  JN_REQUIRE(rows >= 0 && k >= 1 && (rows == 0 || (routes && grad_routes && grad_scores)), kInvalidArgument,
             "bad softmax backward arguments");
  if (rows == 0) return kOk;
  const int blocks = grid_rows(rows);
  JN_REQUIRE(blocks > 0 && k < (1LL << 31), kUnsupported, "too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  JN_PROFILE("softmax_rows_backward_kernel", st);
  hipLaunchKernelGGL(softmax_rows_backward_kernel, dim3(blocks), dim3(256), 0, st, routes, grad_routes, rows, (int)k,
                     grad_scores);
  JN_LAUNCH_CHECK();
  return kOk;
}

int jn_edge_aggregate(const int32_t* edge_index, const float* edge_score, int64_t batch, int64_t query_nodes,
                      int64_t source_nodes, int64_t edges, int64_t dim, int32_t compress_kind,
                      const float* projected_state, const float* projected_val, float* delta_state,
                      float* delta_val, jn_stream_t stream) {
  int rc = check_raw_edges(batch, query_nodes, source_nodes, edges, dim);
  if (rc) return rc;
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= kCoefGiven, kUnsupported, "compress_kind must be 0, 1, 2 or %d",
             kCoefGiven);
  JN_REQUIRE(edge_index && edge_score && projected_state && projected_val && delta_state && delta_val,
             kInvalidArgument, "null tensor pointer");
  RowsFwdArgs f{};
  f.idx = edge_index;
  f.score = edge_score;
  f.k = (int)edges;
  f.compress = compress_kind;
  f.ps = projected_state;
  f.pv = projected_val;
  f.ld_pv = dim;
  f.Nq = (int)query_nodes;
  f.Nk = (int)source_nodes;
  f.D = (int)dim;
  f.rows = batch * query_nodes;
  f.out_state = delta_state;
  f.out_val = delta_val;
  return launch_rows_forward(f, static_cast<hipStream_t>(stream));
}

size_t jn_edge_reduce_backward_workspace_bytes(int64_t batch, int64_t query_nodes, int64_t source_nodes,
                                               int64_t edges) {
  if (batch < 1 || query_nodes < 1 || source_nodes < 1 || edges < 1 ||
      !csr_table_fits(batch, query_nodes, source_nodes))
    return 0;
  Workspace ws(nullptr, 0);
  carve_csr(ws, batch, query_nodes, source_nodes, edges);
  return ws.used;
}

int jn_edge_reduce_backward(const float* edge_weight, const int32_t* edge_index, const float* projected_state,
                            const float* projected_val, const float* grad_delta_state, const float* grad_delta_val,
                            int64_t batch, int64_t query_nodes, int64_t source_nodes, int64_t edges, int64_t dim,
                            float* grad_edge_weight, float* grad_projected_state, float* grad_projected_val,
                            void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_raw_edges(batch, query_nodes, source_nodes, edges, dim);
  if (rc) return rc;
  JN_REQUIRE(edge_weight && edge_index && projected_state && projected_val && grad_delta_state && grad_delta_val,
             kInvalidArgument, "null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = batch * query_nodes;
  if (grad_edge_weight) {
    const int blocks = grid_rows(rows);
    JN_REQUIRE(blocks > 0, kUnsupported, "too many rows");
    JN_PROFILE("edge_dots_kernel", st);
    hipLaunchKernelGGL(edge_dots_kernel, dim3(blocks), dim3(256), 0, st, edge_index, projected_state, projected_val,
                       grad_delta_state, grad_delta_val, (int)query_nodes, (int)source_nodes, (int)edges, (int)dim,
                       rows, grad_edge_weight);
    JN_LAUNCH_CHECK();
  }
  if (!grad_projected_state && !grad_projected_val) return kOk;
  Workspace ws(workspace, workspace_bytes);
  const CsrScratch c = carve_csr(ws, batch, query_nodes, source_nodes, edges);
  JN_REQUIRE(workspace != nullptr && ws.used <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", ws.used, workspace_bytes);
  // the edges grouped by source, with records {row, weight, ., weight * gds[row]}
  CsrArgs ca{};
  ca.idx = edge_index;
  ca.k = (int)edges;
  ca.B = (int)batch;
  ca.Nq = (int)query_nodes;
  ca.Nk = (int)source_nodes;
  ca.tile_base = c.table;
  ca.seg_start = c.seg;
  ca.rec = c.rec;
  ca.coef = edge_weight;
  ca.gds = grad_delta_state;
  rc = launch_csr(ca, st);
  if (rc) return rc;
  ColsBwdArgs cb{};
  cb.seg_start = c.seg;
  cb.rec = c.rec;
  cb.k = (int)edges;
  cb.gdv = grad_delta_val;
  cb.B = (int)batch;
  cb.Nq = (int)query_nodes;
  cb.Nk = (int)source_nodes;
  cb.D = (int)dim;
  cb.grad_pv = grad_projected_val;
  cb.ld_gpv = dim;
  cb.grad_ps = grad_projected_state;
  return launch_cols_backward(cb, st);
}

size_t jn_route_topk_aggregate_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t edges) {
  if (batch < 1 || src_nodes < 1 || dst_nodes < 1 || edges < 1 || !csr_table_fits(batch, src_nodes, dst_nodes))
    return 0;
  Workspace ws(nullptr, 0);
  ws.take<float>(batch * src_nodes * edges);
  carve_csr(ws, batch, src_nodes, dst_nodes, edges);
  return ws.used;
}

int jn_route_topk_aggregate(const int32_t* route_index, const float* route_score, int64_t batch, int64_t src_nodes,
                            int64_t dst_nodes, int64_t edges, int64_t dim, int32_t compress_kind,
                            const float* weighted_state, const float* weighted_val, float* delta_state,
                            float* delta_val, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_raw_edges(batch, src_nodes, dst_nodes, edges, dim);
  if (rc) return rc;
  JN_REQUIRE(edges <= kSelectLargeMaxK, kUnsupported, "routes take up to %d edges per source (got %lld)",
             kSelectLargeMaxK, (long long)edges);
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= 2, kUnsupported, "route compress kind must be 0, 1 or 2");
  JN_REQUIRE(route_index && route_score && weighted_state && weighted_val && delta_state && delta_val,
             kInvalidArgument, "null tensor pointer");
  Workspace ws(workspace, workspace_bytes);
  float* coef = ws.take<float>(batch * src_nodes * edges);
  const CsrScratch c = carve_csr(ws, batch, src_nodes, dst_nodes, edges);
  JN_REQUIRE(workspace != nullptr && ws.used <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", ws.used, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // route weights over each source's edges (no sender strength: the state and
  // values come weighted), then destination sums over the edges grouped by
  // destination
  rc = launch_route_coef(route_index, route_score, nullptr, (int)edges, compress_kind, batch * src_nodes, coef, st);
  if (rc) return rc;
  CsrArgs ca{};
  ca.idx = route_index;
  ca.k = (int)edges;
  ca.B = (int)batch;
  ca.Nq = (int)src_nodes;
  ca.Nk = (int)dst_nodes;
  ca.tile_base = c.table;
  ca.seg_start = c.seg;
  ca.rec = c.rec;
  ca.coef = coef;
  ca.gds = weighted_state;
  rc = launch_csr(ca, st);
  if (rc) return rc;
  ColsBwdArgs cb{};
  cb.seg_start = c.seg;
  cb.rec = c.rec;
  cb.k = (int)edges;
  cb.gdv = weighted_val;
  cb.B = (int)batch;
  cb.Nq = (int)src_nodes;
  cb.Nk = (int)dst_nodes;
  cb.D = (int)dim;
  cb.grad_pv = delta_val;
  cb.ld_gpv = dim;
  cb.grad_ps = delta_state;
  cb.profile_name = "route_gather_kernel";
  return launch_cols_backward(cb, st);
}

namespace {
struct PairScratch {
  float* g;
  float* dPq;
  float* dPs;
  float* rowsum;
  float* part_c;
  float* stage;
  float* splitk;
  CsrScratch csr;
};

PairScratch carve_pair(Workspace& ws, int64_t B, int64_t Nq, int64_t Ns, int64_t Dq, int64_t Ds, int64_t r,
                       int64_t k) {
  PairScratch s{};
  s.g = ws.take<float>(B * Nq * k);
  s.dPq = ws.take<float>(B * Nq * r);
  s.dPs = ws.take<float>(B * Ns * r);
  s.rowsum = ws.take<float>(B * Nq);
  s.part_c = ws.take<float>((size_t)cols_backward_parts(B * Ns) * r);
  s.stage = ws.take<float>(finalize_stage_floats((int)r));
  s.splitk = ws.take<float>(std::max(gemm_grad_weight_workspace((int)r, (int)Dq, (int)(B * Nq)),
                                     gemm_grad_weight_workspace((int)r, (int)Ds, (int)(B * Ns))) /
                            sizeof(float));
  s.csr = carve_csr(ws, B, Nq, Ns, k);
  return s;
}
}  // namespace

size_t jn_lowrank_pair_backward_workspace_bytes(int64_t batch, int64_t query_nodes, int64_t source_nodes,
                                                int64_t query_dim, int64_t source_dim, int64_t rank, int64_t edges) {
  if (batch < 1 || query_nodes < 1 || source_nodes < 1 || query_dim < 1 || source_dim < 1 || rank < 1 ||
      edges < 1 || !csr_table_fits(batch, query_nodes, source_nodes))
    return 0;
  Workspace ws(nullptr, 0);
  carve_pair(ws, batch, query_nodes, source_nodes, query_dim, source_dim, rank, edges);
  return ws.used;
}

int jn_lowrank_pair_backward(const float* query_val, const float* source_val, const float* source_weight,
                             const float* target_weight, const float* core_weight, const float* projected_query,
                             const float* projected_source, const int32_t* edge_index, const float* grad_scores,
                             float temperature, int64_t batch, int64_t query_nodes, int64_t source_nodes,
                             int64_t query_dim, int64_t source_dim, int64_t rank, int64_t edges, float* grad_query,
                             float* grad_source,
                             float* grad_source_weight, float* grad_target_weight, float* grad_core_weight,
                             float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_raw_edges(batch, query_nodes, source_nodes, edges, std::max(query_dim, source_dim));
  if (rc) return rc;
  JN_REQUIRE(query_dim >= 1 && source_dim >= 1, kInvalidArgument, "feature dims must be positive");
  JN_REQUIRE(rank >= 1 && rank <= 128, kUnsupported, "rank must be in [1, 128] (got %lld)", (long long)rank);
  JN_REQUIRE(temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  JN_REQUIRE(query_val && source_val && source_weight && target_weight && core_weight && projected_query &&
                 projected_source && edge_index && grad_scores && grad_query && grad_source && grad_source_weight &&
                 grad_target_weight && grad_core_weight && grad_bias,
             kInvalidArgument, "null tensor pointer");
  Workspace ws(workspace, workspace_bytes);
  const PairScratch s = carve_pair(ws, batch, query_nodes, source_nodes, query_dim, source_dim, rank, edges);
  JN_REQUIRE(workspace != nullptr && ws.used <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", ws.used, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int B = (int)batch, Nq = (int)query_nodes, Ns = (int)source_nodes, r = (int)rank, k = (int)edges;
  const int64_t nedges = batch * query_nodes * edges;
  const int Mq = B * Nq, Ms = B * Ns;
  // g = grad_scores / T: the gradient of each pair score's product term
  {
    JN_PROFILE("scale_kernel", st);
    hipLaunchKernelGGL(scale_kernel, dim3((unsigned)((nedges + 255) / 256)), dim3(256), 0, st, grad_scores,
                       1.0f / temperature, nedges, s.g);
    JN_LAUNCH_CHECK();
  }
  // query side: dPq = w * (g . Ps) per row, and the row sums (bias)
  {
    const int blocks = grid_rows((int64_t)Mq);
    JN_REQUIRE(blocks > 0, kUnsupported, "too many rows");
    JN_PROFILE("pair_rows_grad_kernel", st);
    hipLaunchKernelGGL(pair_rows_grad_kernel, dim3(blocks), dim3(256), 0, st, edge_index, s.g, projected_source,
                       core_weight, Nq, Ns, r, k, (int64_t)Mq, s.dPq, s.rowsum);
    JN_LAUNCH_CHECK();
  }
  // source side: dPs = w * (g^T . Pq) over the edges grouped by source, with
  // the core-weight partials sum g Pq Ps
  CsrArgs ca{};
  ca.idx = edge_index;
  ca.k = k;
  ca.B = B;
  ca.Nq = Nq;
  ca.Nk = Ns;
  ca.tile_base = s.csr.table;
  ca.seg_start = s.csr.seg;
  ca.rec = s.csr.rec;
  ca.g_score = s.g;
  rc = launch_csr(ca, st);
  if (rc) return rc;
  ColsBwdArgs kg{};
  kg.seg_start = s.csr.seg;
  kg.rec = s.csr.rec;
  kg.k = k;
  kg.q = projected_query;
  kg.ldq = r;
  kg.key = projected_source;
  kg.ldk = r;
  kg.kscale = core_weight;
  kg.r = r;
  kg.B = B;
  kg.Nq = Nq;
  kg.Nk = Ns;
  kg.D = 0;
  kg.dk = s.dPs;
  kg.lddk = r;
  kg.part_c = s.part_c;
  rc = launch_cols_backward(kg, st);
  if (rc) return rc;
  // projection weight and input gradients: the query side multiplies
  // target_weight, the source side source_weight
  const int Dq = (int)query_dim, Ds = (int)source_dim;
  rc = gemm_grad_weight(s.dPq, r, query_val, Dq, grad_target_weight, grad_target_weight, r, r, Dq, Mq, s.splitk, st);
  if (rc) return rc;
  rc = gemm_grad_weight(s.dPs, r, source_val, Ds, grad_source_weight, grad_source_weight, r, r, Ds, Ms, s.splitk, st);
  if (rc) return rc;
  rc = gemm_grad_input(s.dPq, r, target_weight, target_weight, r, Dq, nullptr, Dq, grad_query, Dq, Mq, Dq, r, st);
  if (rc) return rc;
  rc = gemm_grad_input(s.dPs, r, source_weight, source_weight, r, Ds, nullptr, Ds, grad_source, Ds, Ms, Ds, r, st);
  if (rc) return rc;
  return launch_finalize_small_grads(s.part_c, cols_backward_parts(Ms), r, grad_core_weight, 0, s.rowsum, Mq,
                                     grad_bias, s.stage, st);
}

}  // extern "C"
