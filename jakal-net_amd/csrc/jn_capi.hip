// C ABI entry points (declared in include/jakal_net_hip.h).  Each entry point
// validates shapes on the host, carves its scratch from the caller's
// workspace and enqueues kernels on the caller's stream.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/jakal_net_hip.h"
#include "jn_internal.hpp"

namespace jakal {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

const char* last_error() { return g_last_error.c_str(); }

namespace {
thread_local std::map<int, SideStream> g_side_per_device;
}

SideForkGuard::~SideForkGuard() {
  for (auto& kv : g_side_per_device)
    if (kv.second.open) join_from(&kv.second, kv.second.origin);
}

SideStream* side_stream(hipStream_t origin) {
  auto& per_device = g_side_per_device;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  auto it = per_device.find(dev);
  if (it != per_device.end()) return &it->second;
  // streams and events are made outside any capture (a first use under
  // capture runs on `origin` alone)
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(origin, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  SideStream s{};
  if (hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) != hipSuccess) return nullptr;
  if (hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&s.join, hipEventDisableTiming) != hipSuccess)
    return nullptr;
  return &per_device.emplace(dev, s).first->second;
}

// Forking pays only when each branch has work enough to hide the extra event
// nodes (on small problems they cost more than the overlap gains).
constexpr int64_t kSideMinEdges = 1 << 18;
static std::atomic<int> g_side_streams{1};
const SideStream* side_stream_for(hipStream_t origin, int64_t edges) {
  if (g_side_streams.load(std::memory_order_relaxed) == 0) return nullptr;
  return edges >= kSideMinEdges ? side_stream(origin) : nullptr;
}

int fork_to(const SideStream* s, hipStream_t origin) {
  JN_HIP_TRY(hipEventRecord(s->fork, origin));
  JN_HIP_TRY(hipStreamWaitEvent(s->stream, s->fork, 0));
  s->open = true;
  s->origin = origin;
  return kOk;
}

int join_from(const SideStream* s, hipStream_t origin) {
  s->open = false;
  JN_HIP_TRY(hipEventRecord(s->join, s->stream));
  JN_HIP_TRY(hipStreamWaitEvent(origin, s->join, 0));
  return kOk;
}

namespace {
struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRecord> g_prof_records;
std::vector<hipEvent_t> g_prof_free;

hipEvent_t prof_event() {
  if (!g_prof_free.empty()) {
    hipEvent_t e = g_prof_free.back();
    g_prof_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

ProfileScope::ProfileScope(const char* name, hipStream_t s) : slot(-1), stream(s) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (!g_prof_on) return;
  ProfRecord r{name, prof_event(), prof_event()};
  if (!r.start || !r.stop) return;
  if (hipEventRecord(r.start, s) != hipSuccess) return;
  g_prof_records.push_back(r);
  slot = (long)g_prof_records.size() - 1;
}

ProfileScope::~ProfileScope() {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (slot < (long)g_prof_records.size()) (void)hipEventRecord(g_prof_records[slot].stop, stream);
}

namespace {

bool fits_int(int64_t v) { return v >= 0 && v < (1LL << 31); }

// Shapes shared by every propagation entry point; `edges` = edge slots per row.
int check_edge_shapes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t edges,
                      int32_t compress_kind) {
  JN_REQUIRE(batch >= 1 && nodes >= 1 && in_dim >= 1 && out_dim >= 1, kInvalidArgument,
             "batch, nodes and dims must be positive (B=%lld N=%lld Din=%lld Dout=%lld)", (long long)batch,
             (long long)nodes, (long long)in_dim, (long long)out_dim);
  JN_REQUIRE(rank >= 1 && rank <= kMaxRank, kUnsupported, "rank must be in [1, %d] (got %lld)", kMaxRank,
             (long long)rank);
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= 2, kUnsupported,
             "compress_kind must be 0 (softsign), 1 (signed_abs_softmax) or 2 (signed_entmax15), got %d",
             compress_kind);
  JN_REQUIRE(edges >= 1 && fits_int(batch * nodes) && fits_int(batch * nodes * edges) &&
                 fits_int(nodes * 2 * rank) && fits_int(nodes * out_dim * 4),
             kUnsupported, "problem too large for 32-bit edge ids and offsets");
  return kOk;
}

int check_propagation_shapes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                             int64_t topk, int32_t compress_kind) {
  JN_REQUIRE(topk >= 1 && topk <= kSelectLargeMaxK, kUnsupported, "topk must be in [1, %d] (got %lld)",
             kSelectLargeMaxK, (long long)topk);
  JN_REQUIRE(topk < nodes, kInvalidArgument, "topk (%lld) must be smaller than nodes (%lld); k == N is dense",
             (long long)topk, (long long)nodes);
  return check_edge_shapes(batch, nodes, in_dim, out_dim, rank, topk, compress_kind);
}

int64_t window_width(int64_t window, int64_t nodes) { return window + 1 < nodes ? window + 1 : nodes; }

// Heads of a multi-head entry point (rank = one head's rank).  A top-k select
// of heads beyond the register kernels' four 32-rank K-steps, of k > 64 or of
// more than 65,535 keys runs as the scored-rows select.
int check_heads(int64_t rank, int64_t heads) {
  JN_REQUIRE(heads >= 2 && heads <= kMaxHeads, kUnsupported,
             "multi-head entry points take 2..%d heads (got %lld); one head is the single-head entry point",
             kMaxHeads, (long long)heads);
  JN_REQUIRE(rank >= 1 && heads * rank <= 128, kUnsupported, "heads x rank must be in [1, 128] (heads=%lld rank=%lld)",
             (long long)heads, (long long)rank);
  return kOk;
}

struct PropBwdScratch {
  float* dP;
  float* g_score;
  float* coef;
  float* rowsum;
  int32_t* tile_base;
  int32_t* seg_start;
  float4* rec;
  int32_t* pos;  // each edge's record index (fused column pass)
  float* dots;   // slab-0 dot partials in record order (fused column pass)
  float* part_c;
  float* stage;
  float* splitk;
  size_t bytes;
};

// r: all ranks (heads * head rank); heads > 1 keeps one bias column per head.
// csr: the edges are grouped by key (top-k lists); a window's causal band has
// a closed-form transpose and takes no grouping space.
PropBwdScratch carve_prop_bwd(void* base, size_t size, int64_t B, int64_t N, int64_t Din, int64_t r, int64_t k,
                              int64_t heads = 1, bool csr = true) {
  Workspace ws(base, size);
  PropBwdScratch s{};
  const int64_t M = B * N;
  s.dP = ws.take<float>(M * 2 * r);
  s.g_score = ws.take<float>(M * k);
  s.coef = ws.take<float>(M * k);
  s.rowsum = ws.take<float>(M * heads);
  s.tile_base = ws.take<int32_t>(csr ? csr_table_entries(B, N, N) : 0);
  s.seg_start = ws.take<int32_t>(csr ? B * (N + 1) : 0);
  s.rec = ws.take<float4>(csr ? M * k : 0);
  s.pos = ws.take<int32_t>(csr ? M * k : 0);
  s.dots = ws.take<float>(M * k);
  s.part_c = ws.take<float>((size_t)cols_backward_parts(M) * r);
  s.stage = ws.take<float>(finalize_stage_floats((int)r, (int)heads));
  s.splitk = ws.take<float>(gemm_grad_weight_workspace((int)(2 * r), (int)Din, (int)M) / sizeof(float));
  s.bytes = ws.used;
  return s;
}

// Edge layout of a top-k edge list, built by the forward for its backward: the
// edges grouped by key (CSR segments and records {row | head << 27, coef,
// edge id, 0}), each edge's record index, and the build's own scratch.  It
// depends only on the edge list, so the forward builds it beside its row pass.
struct EdgeLayout {
  int32_t* seg_start;  // [B, N + 1]
  float4* rec;         // [B * N * k]
  int32_t* pos;        // [B * N * k]
  int32_t* tile_base;  // build scratch
  float* coef;         // build scratch
  size_t bytes;
};

EdgeLayout carve_edge_layout(void* base, size_t size, int64_t B, int64_t N, int64_t k) {
  Workspace ws(base, size);
  EdgeLayout l{};
  l.seg_start = ws.take<int32_t>(B * (N + 1));
  l.rec = ws.take<float4>(B * N * k);
  l.pos = ws.take<int32_t>(B * N * k);
  l.tile_base = ws.take<int32_t>(csr_table_entries(B, N, N));
  l.coef = ws.take<float>(B * N * k);
  l.bytes = ws.used;
  return l;
}

int build_edge_layout(const EdgeLayout& l, const int32_t* idx, const float* score, const uint8_t* ehead, int B,
                      int N, int k, int compress_kind, hipStream_t stream) {
  CsrArgs ca{};
  ca.idx = idx;
  ca.k = k;
  ca.B = B;
  ca.Nq = N;
  ca.Nk = N;
  ca.tile_base = l.tile_base;
  ca.seg_start = l.seg_start;
  ca.rec = l.rec;
  ca.ehead = ehead;
  ca.rec_eid = 1;
  ca.pos = l.pos;
  int rc = launch_csr_layout(ca, stream);
  if (rc) return rc;
  if (compress_kind == 0) {  // softsign: the fill computes each coefficient from its score
    ca.score = score;
  } else {  // row-normalised: the coefficients first
    rc = launch_edge_coefficients(idx, score, (int64_t)B * N, k, compress_kind, l.coef, stream);
    if (rc) return rc;
    ca.coef = l.coef;
  }
  return launch_csr_fill(ca, stream);
}

struct TransitionScratch {
  float* coef;
  int32_t* tile_base;
  int32_t* seg_start;
  float4* rec;
  float* dPs;
  float* dPt;
  float* g_logit;
  float* rowsum;
  float* part_c;
  float* stage;
  float* splitk;    // split-K partials of the destination-side weight gradient
  float* splitk2;   // of the source-side one (the two run side by side)
  void* select_ws;  // split-fp16 key rows of the forward's select
  size_t select_ws_bytes;
  size_t bytes;
};

int64_t route_edges(int64_t topk, int64_t dst_nodes) { return topk < dst_nodes ? topk : dst_nodes; }

// r: all ranks (heads * head rank).
TransitionScratch carve_transition(void* base, size_t size, int64_t B, int64_t Ns, int64_t Nd, int64_t Dsrc,
                                   int64_t Ddst, int64_t r, int64_t k, int64_t heads = 1) {
  Workspace ws(base, size);
  TransitionScratch s{};
  s.coef = ws.take<float>(B * Ns * k);
  s.tile_base = ws.take<int32_t>(csr_table_entries(B, Ns, Nd));
  s.seg_start = ws.take<int32_t>(B * (Nd + 1));
  s.rec = ws.take<float4>(B * Ns * k);
  s.dPs = ws.take<float>(B * Ns * r);
  s.dPt = ws.take<float>(B * Nd * r);
  s.g_logit = ws.take<float>(B * Ns * k);
  s.rowsum = ws.take<float>(B * Ns * heads);
  s.part_c = ws.take<float>((size_t)cols_backward_parts(B * Nd) * r);
  s.stage = ws.take<float>(finalize_stage_floats((int)r, (int)heads));
  s.splitk = ws.take<float>(gemm_grad_weight_workspace((int)r, (int)Ddst, (int)(B * Nd)) / sizeof(float));
  s.splitk2 = ws.take<float>(gemm_grad_weight_workspace((int)r, (int)Dsrc, (int)(B * Ns)) / sizeof(float));
  s.select_ws_bytes = heads > 1 ? select_workspace_bytes_heads(B, Nd, r / heads, heads)
                                : select_workspace_bytes(B, Nd, r);
  s.select_ws = ws.take<char>(s.select_ws_bytes);
  s.bytes = ws.used;
  return s;
}

int check_transition_shapes(int64_t batch, int64_t Ns, int64_t Nd, int64_t Dsrc, int64_t Ddst, int64_t Dv,
                            int64_t rank, int64_t topk, int32_t compress_kind, float temperature) {
  JN_REQUIRE(batch >= 1 && Ns >= 1 && Nd >= 1 && Dsrc >= 1 && Ddst >= 1 && Dv >= 1, kInvalidArgument,
             "batch, node counts and dims must be positive");
  JN_REQUIRE(rank >= 1 && rank <= kMaxRank, kUnsupported, "rank must be in [1, %d] (got %lld)", kMaxRank,
             (long long)rank);
  JN_REQUIRE(topk >= 1, kInvalidArgument, "topk must be positive");
  const int64_t k = route_edges(topk, Nd);
  JN_REQUIRE(k == Nd ? k <= 64 : k <= kSelectLargeMaxK, kUnsupported,
             "routes support topk <= %d below the destination count, or up to 64 destinations in all (topk=%lld, "
             "dst_nodes=%lld)",
             kSelectLargeMaxK, (long long)topk, (long long)Nd);
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= 2, kUnsupported,
             "route compress kind must be 0 (softmax), 1 (signed_abs_softmax) or 2 (signed_entmax15), got %d",
             compress_kind);
  JN_REQUIRE(temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  JN_REQUIRE(fits_int(batch * Ns * k) && fits_int(batch * Nd * rank) && fits_int(batch * Ns * rank) &&
                 fits_int(Nd * Dv * 4) && fits_int(Nd * rank * 4),
             kUnsupported, "problem too large for 32-bit edge ids and offsets");
  return kOk;
}

struct DenseScratch {
  float* E;       // [g_batch... e_batch, N, N] recomputed edge matrix of a chunk (chunked backward)
  float* G;       // [g_batch, N, N] score gradient (absent when it overwrites the edge matrix)
  float* dP;      // [M, 2r]
  float* rowsum;  // [M]
  float* part_c;  // [M, r]
  float* hrowsum; // [M, heads] per-head bias partials (multi-head only)
  float* stage;
  float* splitk;
  size_t bytes;
};

// g_batch / e_batch: batch elements of the score-gradient / edge-matrix buffers
// (0: none); r counts every head's ranks
DenseScratch carve_dense(void* base, size_t size, int64_t B, int64_t N, int64_t Din, int64_t r, int64_t g_batch,
                         int64_t e_batch, int64_t heads = 1) {
  Workspace ws(base, size);
  DenseScratch s{};
  const int64_t M = B * N;
  s.E = e_batch ? ws.take<float>(e_batch * N * N) : nullptr;
  s.G = g_batch ? ws.take<float>(g_batch * N * N) : nullptr;
  s.dP = ws.take<float>(M * 2 * r);
  s.rowsum = ws.take<float>(M * dense_epi_parts((int)N));  // per-row totals, or the epilogue's block partials
  s.part_c = ws.take<float>(M * r);
  s.hrowsum = heads > 1 ? ws.take<float>(M * heads) : nullptr;
  s.stage = ws.take<float>(finalize_stage_floats((int)r, (int)heads));
  s.splitk = ws.take<float>(gemm_grad_weight_workspace((int)(2 * r), (int)Din, (int)M) / sizeof(float));
  s.bytes = ws.used;
  return s;
}

int check_dense_shapes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                       int32_t compress_kind) {
  JN_REQUIRE(batch >= 1 && nodes >= 1 && in_dim >= 1 && out_dim >= 1, kInvalidArgument,
             "batch, nodes and dims must be positive");
  JN_REQUIRE(rank >= 1 && rank <= kMaxRank, kUnsupported, "rank must be in [1, %d] (got %lld)", kMaxRank,
             (long long)rank);
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= 2, kUnsupported,
             "compress_kind must be 0 (softsign), 1 (signed_abs_softmax) or 2 (signed_entmax15), got %d",
             compress_kind);
  JN_REQUIRE(batch < 65536 && fits_int(batch * nodes) && nodes < (1LL << 22) && fits_int(nodes * out_dim),
             kUnsupported, "dense propagation shape too large");
  return kOk;
}

struct TransitionDenseScratch {
  float* G;       // [B, Ns, Nd] route / logit gradient
  float* dPs;     // [B*Ns, r]
  float* dPt;     // [B*Nd, r]
  float* rowsum;  // [B*Ns] ([B*Ns, heads] with heads > 1)
  float* part_c;  // [B*Ns, r]
  float* stage;
  float* splitk;
  size_t bytes;
};

// r counts every head's ranks
TransitionDenseScratch carve_transition_dense(void* base, size_t size, int64_t B, int64_t Ns, int64_t Nd,
                                              int64_t Dsrc, int64_t Ddst, int64_t r, int64_t heads = 1) {
  Workspace ws(base, size);
  TransitionDenseScratch s{};
  s.G = ws.take<float>(B * Ns * Nd);
  s.dPs = ws.take<float>(B * Ns * r);
  s.dPt = ws.take<float>(B * Nd * r);
  s.rowsum = ws.take<float>(B * Ns * heads);
  s.part_c = ws.take<float>(B * Ns * r);
  s.stage = ws.take<float>(finalize_stage_floats((int)r, (int)heads));
  const size_t sk = std::max(gemm_grad_weight_workspace((int)r, (int)Dsrc, (int)(B * Ns)),
                             gemm_grad_weight_workspace((int)r, (int)Ddst, (int)(B * Nd)));
  s.splitk = ws.take<float>(sk / sizeof(float));
  s.bytes = ws.used;
  return s;
}

// Row e of a value tensor (elements, not bytes): bf16 tensors travel as float
// pointers to the GEMMs, which address them in bf16 elements.
inline const float* value_rows(const float* p, int64_t e, bool bf16) {
  return bf16 ? reinterpret_cast<const float*>(reinterpret_cast<const bf16_t*>(p) + e) : p + e;
}

// Max-aggregated multi-head scores of batch elements [b0, b0 + nb)
// (jakal_net_native.cpp:724-752): S = max_h (P_t,h diag(w_h) P_s,h^T + b_h)
// over the heads' rank slices of the [N, 2r] projection rows (r = heads *
// head rank), one fp32 MFMA GEMM per head whose epilogue folds its scores into
// E; head_mat records the first head attaining each pair's max.
int dense_head_scores(const float* core_weight, const float* bias, int b0, int nb, int N, int r, int heads,
                      const float* projections, float* E, uint8_t* head_mat, hipStream_t st) {
  const int64_t pr = (int64_t)b0 * N;
  const int rh = r / heads;
  for (int h = 0; h < heads; ++h) {
    BatchedGemm sg{};
    sg.A = projections + pr * 2 * r + h * rh; sg.lda = 2 * r; sg.a_bs = (int64_t)N * 2 * r; sg.a_kcontig = true;
    sg.B = projections + pr * 2 * r + r + h * rh; sg.ldb = 2 * r; sg.b_bs = (int64_t)N * 2 * r; sg.b_kcontig = true;
    sg.C = E; sg.ldc = N; sg.c_bs = (int64_t)N * N;
    sg.a_kscale = core_weight + h * rh;
    sg.M = N; sg.N = N; sg.K = rh; sg.batch = nb;
    sg.fold = h == 0 ? 1 : 2; sg.fold_head = h; sg.fold_bias = bias ? bias + h : nullptr; sg.fold_heads = head_mat;
    const int rc = gemm_batched(sg, kGemmDenseScores, st);
    if (rc) return rc;
  }
  return kOk;
}

// Dense propagation forward over batch elements [b0, b0 + nb) (propagation.py:
// 207-220): the edge matrix E of those elements (batch stride N*N), then
// delta_state = E ps and delta_val = E pv.  projections holds every batch
// element's [N, 2r] projection rows.  heads > 1: max-aggregated scores over
// the heads' rank slices (r = heads * head rank, bias [heads]), with the
// winning head of every pair in head_mat [nb, N, N].  bf16 (one head):
// projected_val and delta_val hold bf16 elements; E stays fp32 and is rounded
// to bf16 as the aggregate's operand.
int dense_forward_range(const float* projected_state, const float* projected_val, const float* core_weight,
                        const float* bias, int b0, int nb, int N, int D, int r, int compress_kind, bool causal,
                        const float* projections, float* E, float* delta_state, float* delta_val, hipStream_t st,
                        int heads = 1, uint8_t* head_mat = nullptr, bool bf16 = false) {
  const int64_t pr = (int64_t)b0 * N;  // first row of the range
  JN_REQUIRE(!bf16 || heads == 1, kInvalidArgument, "bf16 dense layers have one head");
  if (heads > 1) {
    int rc = dense_head_scores(core_weight, bias, b0, nb, N, r, heads, projections, E, head_mat, st);
    if (rc) return rc;
    // E = compress(S) in place (the heads' biases are in S), delta_state = E ps
    rc = launch_dense_compress(E, nullptr, projected_state + pr, nb, N, compress_kind, causal, delta_state + pr, st);
    if (rc) return rc;
    BatchedGemm ag{};
    ag.A = E; ag.lda = N; ag.a_bs = (int64_t)N * N; ag.a_kcontig = true;
    ag.B = projected_val + pr * D; ag.ldb = D; ag.b_bs = (int64_t)N * D; ag.b_kcontig = false;
    ag.C = delta_val + pr * D; ag.ldc = D; ag.c_bs = (int64_t)N * D;
    ag.M = N; ag.N = D; ag.K = N; ag.batch = nb;
    ag.causal_k = causal ? kCausalKLower : kCausalKNone;
    return gemm_batched(ag, kGemmDenseAggregate, st);
  }
  // S_b = (P_t diag(w_hat)) P_s^T
  BatchedGemm sg{};
  sg.A = projections + pr * 2 * r; sg.lda = 2 * r; sg.a_bs = (int64_t)N * 2 * r; sg.a_kcontig = true;
  sg.B = projections + pr * 2 * r + r; sg.ldb = 2 * r; sg.b_bs = (int64_t)N * 2 * r; sg.b_kcontig = true;
  sg.C = E; sg.ldc = N; sg.c_bs = (int64_t)N * N;
  sg.a_kscale = core_weight;
  sg.M = N; sg.N = N; sg.K = r; sg.batch = nb;
  // Softsign runs in the GEMM's epilogue, whose per-block partials of
  // delta_state are staged in delta_val's storage (the aggregate GEMM below
  // overwrites it); the row-wise compressions run as a pass of their own.
  const int parts = dense_epi_parts(N);
  const bool fused = compress_kind == 0 && parts <= (bf16 ? D / 2 : D);
  float* vstage = bf16 ? reinterpret_cast<float*>(reinterpret_cast<bf16_t*>(delta_val) + pr * D) : delta_val + pr * D;
  if (fused) {
    sg.epi = 1; sg.epi_causal = causal; sg.epi_bias = bias; sg.epi_ps = projected_state + pr;
    sg.epi_part = vstage;
  }
  int rc = gemm_batched(sg, kGemmDenseScores, st);
  if (rc) return rc;
  // E = compress(S + b) (in place when not fused), delta_state = E ps
  rc = fused ? launch_dense_part_rowsum(vstage, parts, (int64_t)nb * N, delta_state + pr, st)
             : launch_dense_compress(E, bias, projected_state + pr, nb, N, compress_kind, causal, delta_state + pr,
                                     st);
  if (rc) return rc;
  // delta_val_b = E_b pv_b
  BatchedGemm ag{};
  ag.A = E; ag.lda = N; ag.a_bs = (int64_t)N * N; ag.a_kcontig = true;
  ag.B = value_rows(projected_val, pr * D, bf16); ag.ldb = D; ag.b_bs = (int64_t)N * D; ag.b_kcontig = false;
  ag.C = const_cast<float*>(value_rows(delta_val, pr * D, bf16)); ag.ldc = D; ag.c_bs = (int64_t)N * D;
  ag.M = N; ag.N = D; ag.K = N; ag.batch = nb;
  ag.causal_k = causal ? kCausalKLower : kCausalKNone;  // row i reads sources j <= i
  return gemm_batched(ag, bf16 ? kGemmDenseAggregateBf16 : kGemmDenseAggregate, st);
}

// Dense propagation backward, chunk_batch batch elements at a time.  E holds
// the chunk's edge matrix (the whole saved matrix when chunk_batch covers
// every batch element and recompute is false; otherwise it is rebuilt from
// the projections for each chunk, exactly as the forward built it), G the
// chunk's score gradient (G == E: written over the edges, softsign only).
// Chunks run last to first; with last_resident E already holds the last
// chunk's edges (the chunked forward leaves them there), which are not rebuilt.
// Each chunk writes its own rows of every per-row output, so the order does
// not change the results.
int dense_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                   const float* target_weight, const float* source_weight, const float* core_weight, const float* bias,
                   const float* projections, float* E, float* G, int chunk_batch, bool recompute, bool last_resident,
                   const float* grad_delta_state, const float* grad_delta_val, int64_t batch, int64_t nodes,
                   int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
                   int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
                   float* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
                   float* grad_core_weight, float* grad_bias, const DenseScratch& s, hipStream_t st, int heads = 1,
                   uint8_t* head_mat = nullptr, bool bf16 = false) {
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 projections && E && G && grad_delta_state && grad_delta_val,
             kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(!projected_val_is_layer_val || in_dim == out_dim, kInvalidArgument,
             "projected_val_is_layer_val requires in_dim == out_dim");
  JN_REQUIRE(G != E || compress_kind == 0, kInvalidArgument, "only the softsign gradient overwrites the edges");
  JN_REQUIRE(!bf16 || heads == 1, kInvalidArgument, "bf16 dense layers have one head");
  const int B = (int)batch, N = (int)nodes, r = (int)rank, D = (int)out_dim;
  const int M = B * N;
  const bool fused = compress_kind == 0;  // softsign's derivative in the score-gradient GEMM's epilogue
  const int parts = dense_epi_parts(N);
  const int lower = causal ? kCausalKLower : kCausalKNone;  // A(i, j) = 0 for j > i
  const int upper = causal ? kCausalKUpper : kCausalKNone;  // A = E^T: A(j, i) = 0 for i < j
  float* gpv = projected_val_is_layer_val ? grad_layer_val : grad_projected_val;
  int rc;
  const int nchunks = (B + chunk_batch - 1) / chunk_batch;
  for (int c = nchunks - 1; c >= 0; --c) {
    const int b0 = c * chunk_batch;
    const int nb = std::min(chunk_batch, B - b0);
    const int64_t pr = (int64_t)b0 * N;
    float* rowsum = s.rowsum + (fused ? pr * parts : pr);
    if (recompute && !(last_resident && c == nchunks - 1) && heads > 1) {
      // the forward's edges and winning heads of this chunk (state sums to scratch)
      rc = dense_head_scores(core_weight, bias, b0, nb, N, r, heads, projections, E, head_mat, st);
      if (rc) return rc;
      rc = launch_dense_compress(E, nullptr, projected_state + pr, nb, N, compress_kind, causal != 0,
                                 s.part_c + pr * r, st);
      if (rc) return rc;
    } else if (recompute && !(last_resident && c == nchunks - 1)) {
      // the forward's edges of this chunk; its state sums go to scratch that
      // later steps overwrite (the row sums, or the scale partials)
      BatchedGemm sg{};
      sg.A = projections + pr * 2 * r; sg.lda = 2 * r; sg.a_bs = (int64_t)N * 2 * r; sg.a_kcontig = true;
      sg.B = projections + pr * 2 * r + r; sg.ldb = 2 * r; sg.b_bs = (int64_t)N * 2 * r; sg.b_kcontig = true;
      sg.C = E; sg.ldc = N; sg.c_bs = (int64_t)N * N;
      sg.a_kscale = core_weight;
      sg.M = N; sg.N = N; sg.K = r; sg.batch = nb;
      if (fused) {
        sg.epi = 1; sg.epi_causal = causal != 0; sg.epi_bias = bias; sg.epi_ps = projected_state + pr;
        sg.epi_part = rowsum;
      }
      rc = gemm_batched(sg, kGemmDenseScores, st);
      if (rc) return rc;
      if (!fused) {
        rc = launch_dense_compress(E, bias, projected_state + pr, nb, N, compress_kind, causal != 0,
                                   s.part_c + pr * r, st);
        if (rc) return rc;
      }
    }

    // 1. value and state grads of the sources: E^T gdv, E^T gds (before E is overwritten)
    if (gpv) {
      BatchedGemm vg{};
      vg.A = E; vg.lda = N; vg.a_bs = (int64_t)N * N; vg.a_kcontig = false;
      vg.B = value_rows(grad_delta_val, pr * D, bf16); vg.ldb = D; vg.b_bs = (int64_t)N * D; vg.b_kcontig = false;
      vg.C = const_cast<float*>(value_rows(gpv, pr * D, bf16)); vg.ldc = D; vg.c_bs = (int64_t)N * D;
      vg.M = N; vg.N = D; vg.K = N; vg.batch = nb;
      vg.causal_k = upper;
      rc = gemm_batched(vg, bf16 ? kGemmDenseValueGradBf16 : kGemmDenseValueGrad, st);
      if (rc) return rc;
    }
    if (grad_projected_state) {
      rc = launch_dense_colsum(E, grad_delta_state + pr, nb, N, grad_projected_state + pr, st);
      if (rc) return rc;
    }

    // 2. G_b = gdv_b pv_b^T, then the score gradient (+ row sums)
    BatchedGemm gg{};
    gg.A = value_rows(grad_delta_val, pr * D, bf16); gg.lda = D; gg.a_bs = (int64_t)N * D; gg.a_kcontig = true;
    gg.B = value_rows(projected_val, pr * D, bf16); gg.ldb = D; gg.b_bs = (int64_t)N * D; gg.b_kcontig = true;
    gg.C = G; gg.ldc = N; gg.c_bs = (int64_t)N * N;
    gg.M = N; gg.N = N; gg.K = D; gg.batch = nb;
    if (fused) {
      gg.epi = 1; gg.epi_causal = causal != 0; gg.epi_ps = projected_state + pr; gg.epi_gds = grad_delta_state + pr;
      gg.epi_E = E; gg.epi_part = rowsum;
    }
    rc = gemm_batched(gg, bf16 ? kGemmDenseEdgeGradBf16 : kGemmDenseEdgeGrad, st);
    if (rc) return rc;
    if (!fused) {
      rc = launch_dense_compress_backward(G, E, grad_delta_state + pr, projected_state + pr, nb, N, compress_kind,
                                          causal != 0, rowsum, st);
      if (rc) return rc;
    }

    // multi-head: each pair's score gradient reaches its winning head only --
    // the per-head bias partials, and the rank-r products below on G masked
    // to that head's pairs
    if (heads > 1) {
      rc = launch_head_rowsum(G, head_mat, N, N, (int64_t)nb * N, heads, s.hrowsum + pr * heads, st);
      if (rc) return rc;
    }

    // 3. projection grads: dP_t = w_hat * (G_s P_s), dP_s = w_hat * (G_s^T P_t) (+ w_hat partials)
    const int rh = r / heads;
    for (int h = 0; h < heads; ++h) {
      BatchedGemm tg{};
      tg.A = G; tg.lda = N; tg.a_bs = (int64_t)N * N; tg.a_kcontig = true;
      tg.B = projections + pr * 2 * r + r + h * rh; tg.ldb = 2 * r; tg.b_bs = (int64_t)N * 2 * r;
      tg.b_kcontig = false;
      tg.C = s.dP + pr * 2 * r + h * rh; tg.ldc = 2 * r; tg.c_bs = (int64_t)N * 2 * r;
      tg.c_nscale = core_weight + h * rh;
      tg.M = N; tg.N = rh; tg.K = N; tg.batch = nb;
      tg.causal_k = lower;
      if (heads > 1) { tg.a_heads = head_mat; tg.a_head = h; }
      rc = gemm_batched(tg, kGemmDenseTargetGrad, st);
      if (rc) return rc;
      BatchedGemm sg2{};
      sg2.A = G; sg2.lda = N; sg2.a_bs = (int64_t)N * N; sg2.a_kcontig = false;
      sg2.B = projections + pr * 2 * r + h * rh; sg2.ldb = 2 * r; sg2.b_bs = (int64_t)N * 2 * r;
      sg2.b_kcontig = false;
      sg2.C = s.dP + pr * 2 * r + r + h * rh; sg2.ldc = 2 * r; sg2.c_bs = (int64_t)N * 2 * r;
      sg2.M = N; sg2.N = rh; sg2.K = N; sg2.batch = nb;
      sg2.causal_k = upper;
      if (heads > 1) { sg2.a_heads = head_mat; sg2.a_head = h; }
      rc = gemm_batched(sg2, kGemmDenseSourceGrad, st);
      if (rc) return rc;
    }
    rc = launch_scale_grad_partials(s.dP + pr * 2 * r + r, 2 * r, projections + pr * 2 * r + r, 2 * r, core_weight, r,
                                    (int64_t)nb * N, s.part_c + pr * r, st);
    if (rc) return rc;
  }
  const int64_t n_rowsum = fused ? (int64_t)M * parts : M;

  // 4. projection weight and input grads
  if (grad_target_weight && grad_source_weight) {
    rc = gemm_grad_weight(s.dP, 2 * r, layer_val, in_dim, grad_target_weight, grad_source_weight, r, 2 * r,
                          (int)in_dim, M, s.splitk, st, bf16);
    if (rc) return rc;
  }
  if (grad_layer_val) {
    const float* addend = (projected_val_is_layer_val && gpv) ? grad_layer_val : nullptr;
    rc = gemm_grad_input(s.dP, 2 * r, target_weight, source_weight, r, in_dim, addend, in_dim, grad_layer_val,
                         in_dim, M, (int)in_dim, 2 * r, st, bf16);
    if (rc) return rc;
  }

  // 5. w_hat and bias grads
  if (heads > 1)
    return launch_finalize_small_grads(s.part_c, M, r, grad_core_weight, 0, s.hrowsum, M, grad_bias, s.stage, st,
                                       heads);
  return launch_finalize_small_grads(s.part_c, M, r, grad_core_weight, 0, s.rowsum, n_rowsum, grad_bias, s.stage,
                                     st);
}

int check_transition_dense_shapes(int64_t batch, int64_t Ns, int64_t Nd, int64_t Dsrc, int64_t Ddst, int64_t Dv,
                                  int64_t rank, int32_t compress_kind, float temperature) {
  JN_REQUIRE(batch >= 1 && Ns >= 1 && Nd >= 1 && Dsrc >= 1 && Ddst >= 1 && Dv >= 1, kInvalidArgument,
             "batch, node counts and dims must be positive");
  JN_REQUIRE(rank >= 1 && rank <= kMaxRank, kUnsupported, "rank must be in [1, %d] (got %lld)", kMaxRank,
             (long long)rank);
  JN_REQUIRE(compress_kind >= 0 && compress_kind <= 2, kUnsupported,
             "route compress kind must be 0 (softmax), 1 (signed_abs_softmax) or 2 (signed_entmax15), got %d",
             compress_kind);
  JN_REQUIRE(temperature > 0.0f, kInvalidArgument, "temperature must be positive");
  JN_REQUIRE(batch < 65536 && fits_int(batch * Ns) && fits_int(batch * Nd) && Ns < (1LL << 22) &&
                 Nd < (1LL << 22) && fits_int(Ns * Dv) && fits_int(Nd * Dv) && fits_int(Ns * Nd),
             kUnsupported, "dense transition shape too large");
  return kOk;
}

// Backward of any edge-list propagation (top-k or window): the edge list
// (edge_index, edge_score) [B*N, k] is what the forward aggregated.
// rank: all ranks (heads * head rank); heads > 1 takes each edge's head.
// band: the list is a window forward's causal band, whose transpose is known
// in closed form (no CSR build; the column pass reads the edge arrays).
int propagation_edges_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                               const float* target_weight, const float* source_weight, const float* core_weight,
                               const float* projections, const int32_t* topk_index, const float* topk_score,
                               const uint8_t* edge_head, const float* grad_delta_state, const float* grad_delta_val,
                               int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                               int64_t heads, int64_t topk, int32_t compress_kind,
                               int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
                               float* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
                               float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
                               hipStream_t stream, bool bf16 = false, bool band = false,
                               const void* edge_layout = nullptr) {
  SideForkGuard join_guard;  // joins a fork left open by an error return
  int rc;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 projections && topk_index && topk_score && grad_delta_state && grad_delta_val &&
                 (heads <= 1 || edge_head),
             kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(!projected_val_is_layer_val || in_dim == out_dim, kInvalidArgument,
             "projected_val_is_layer_val requires in_dim == out_dim");
  const bool mh = heads > 1;
  PropBwdScratch s =
      carve_prop_bwd(workspace, workspace_bytes, batch, nodes, in_dim, rank, topk, mh ? heads : 1, !band);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  hipStream_t st = stream;
  const int B = (int)batch, N = (int)nodes, r = (int)rank, k = (int)topk;
  const int M = B * N;
  const float* src_proj = projections + r;  // unscaled source projection, stride 2r

  // 1. rows: edge-coefficient grads, compress backward, grad of target projection
  RowsBwdArgs rb{};
  rb.idx = topk_index;
  rb.score = topk_score;
  rb.k = k;
  rb.compress = compress_kind;
  rb.inv_temperature = 1.0f;
  rb.ps = projected_state;
  rb.pv = projected_val;
  rb.ld_pv = out_dim;
  rb.gds = grad_delta_state;
  rb.gdv = grad_delta_val;
  rb.key = src_proj;
  rb.ldk = 2 * r;
  rb.qscale = core_weight;
  rb.r = r;
  rb.Nq = N;
  rb.Nk = N;
  rb.D = (int)out_dim;
  rb.rows = M;
  rb.g_score = s.g_score;
  rb.coef = s.coef;
  rb.dq = s.dP;
  rb.lddq = 2 * r;
  rb.rowsum_gs = s.rowsum;
  rb.bf16 = bf16 ? 1 : 0;
  if (mh) {
    rb.ehead = edge_head;
    rb.heads = (int)heads;
    rb.head_rank = (int)(rank / heads);
  }
  // 2a. the CSR layout of the edge list (it reads only the edge index) runs on
  //     a second stream beside the row pass
  CsrArgs ca{};
  ca.idx = topk_index;
  ca.k = k;
  ca.B = B;
  ca.Nq = N;
  ca.Nk = N;
  ca.tile_base = s.tile_base;
  ca.seg_start = s.seg_start;
  ca.rec = s.rec;
  ca.coef = s.coef;
  ca.g_score = s.g_score;
  ca.gds = grad_delta_state;
  ca.ehead = mh ? edge_head : nullptr;
  float* gpv = projected_val_is_layer_val ? grad_layer_val : grad_projected_val;

  // Fused column pass (CSR edge lists whose value rows fit at most two slabs of
  // 16-byte packs): each incoming edge's gdv row is gathered once per column,
  // for the value gradient and for the edge's dot product <gdv[i], pv[j]>, so
  // the row pass reads no value rows.
  ColsBwdArgs fc{};
  fc.seg_start = s.seg_start;
  fc.rec = s.rec;
  fc.k = k;
  fc.gdv = grad_delta_val;
  fc.r = r;
  fc.B = B;
  fc.Nq = N;
  fc.Nk = N;
  fc.D = (int)out_dim;
  fc.grad_pv = gpv;
  fc.ld_gpv = out_dim;
  fc.grad_ps = grad_projected_state;
  fc.bf16 = bf16 ? 1 : 0;
  fc.rec_eid = 1;
  fc.pv = projected_val;
  fc.ld_pv = out_dim;
  fc.dots0 = s.dots;
  fc.dots1 = s.coef;
  const int dot_slabs = band ? 0 : cols_gather_dots_slabs(fc);
  if (dot_slabs) {
    // a. the edges grouped by key: the forward's layout, or built here (the
    //    CSR layout reads the edge index only and runs on the second stream
    //    beside the edge coefficients; then the records {row, coef, edge id, 0})
    const int32_t* seg = s.seg_start;
    const float4* rec = s.rec;
    const int32_t* pos = s.pos;
    if (edge_layout) {
      const EdgeLayout l = carve_edge_layout(const_cast<void*>(edge_layout), SIZE_MAX, B, N, k);
      seg = l.seg_start;
      rec = l.rec;
      pos = l.pos;
    } else {
      ca.g_score = nullptr;
      ca.gds = nullptr;
      ca.rec_eid = 1;
      ca.pos = s.pos;
      const SideStream* side = side_stream_for(st, (int64_t)M * k);
      if (side) {
        rc = fork_to(side, st);
        if (rc) return rc;
      }
      rc = launch_csr_layout(ca, side ? side->stream : st);
      if (rc) return rc;
      if (compress_kind == 0) {  // softsign: the fill computes each coefficient from its score
        ca.coef = nullptr;
        ca.score = topk_score;
      } else {
        rc = launch_edge_coefficients(topk_index, topk_score, M, k, compress_kind, s.coef, st);
        if (rc) return rc;
      }
      if (side) {
        rc = join_from(side, st);
        if (rc) return rc;
      }
      rc = launch_csr_fill(ca, st);
      if (rc) return rc;
    }
    // b. value and state grads of the sources, and the dot partials in record
    //    order (slab 0 into dots, slab 1 into coef)
    fc.seg_start = seg;
    fc.rec = rec;
    fc.gds = grad_delta_state;
    rc = launch_cols_gather_dots(fc, st);
    if (rc) return rc;
    // c. rows: compress backward from the given dots, grad of target projection
    rb.dots_given = 1;
    rb.dot_parts = dot_slabs;
    rb.dot_pos = pos;
    rb.dots0 = s.dots;
    rc = launch_rows_backward(rb, st);
    if (rc) return rc;
    // d. grad of the source projection and the w_hat partials
    ColsBwdArgs kg{};
    kg.seg_start = seg;
    kg.rec = rec;
    kg.k = k;
    kg.q = projections;
    kg.ldq = 2 * r;
    kg.key = src_proj;
    kg.ldk = 2 * r;
    kg.kscale = core_weight;
    kg.r = r;
    kg.B = B;
    kg.Nq = N;
    kg.Nk = N;
    kg.D = (int)out_dim;
    kg.dk = s.dP + r;
    kg.lddk = 2 * r;
    kg.part_c = s.part_c;
    kg.rec_eid = 1;
    kg.g_score = s.g_score;
    if (mh) {
      kg.heads = (int)heads;
      kg.head_rank = (int)(rank / heads);
    }
    rc = launch_cols_backward(kg, st);
    if (rc) return rc;
  }
  if (!dot_slabs) {
    const SideStream* side = side_stream_for(st, (int64_t)M * k);
    if (!band) {
      hipStream_t cs = side ? side->stream : st;
      if (side) {
        rc = fork_to(side, st);
        if (rc) return rc;
      }
      rc = launch_csr_layout(ca, cs);
      if (rc) return rc;
    }

    // a causal band: the value-row dot products as MFMA tiles over each row
    // tile's span, then the row kernel without value rows
    const bool band_mfma = band && window_kernels() == 0 &&
                           band_kernels_fit(k, (int)out_dim, out_dim, out_dim, grad_delta_val, projected_val, bf16);
    if (band_mfma) {
      BandDotsArgs bd{};
      bd.B = B;
      bd.N = N;
      bd.k = k;
      bd.D = (int)out_dim;
      bd.gdv = grad_delta_val;
      bd.ld_gdv = out_dim;
      bd.pv = projected_val;
      bd.ld_pv = out_dim;
      bd.g_score = s.g_score;
      bd.coef = s.coef;
      bd.bf16 = bf16 ? 1 : 0;
      rc = launch_band_dots(bd, st);
      if (rc) return rc;
      rb.dots_given = 1;
    }
    rc = launch_rows_backward(rb, st);
    if (rc) return rc;

    // 2b. the edge records, grouped by key (deterministic transpose; a band's
    //     is closed form and needs none)
    if (!band) {
      if (side) {
        rc = join_from(side, st);
        if (rc) return rc;
      }
      rc = launch_csr_fill(ca, st);
      if (rc) return rc;
    }

    // 3. columns: value/state grads of the sources, grad of source projection, w_hat grad partials
    ColsBwdArgs cb{};
    cb.seg_start = s.seg_start;
    cb.rec = s.rec;
    cb.k = k;
    cb.gdv = grad_delta_val;
    cb.q = projections;
    cb.ldq = 2 * r;
    cb.key = src_proj;
    cb.ldk = 2 * r;
    cb.kscale = core_weight;
    cb.r = r;
    cb.B = B;
    cb.Nq = N;
    cb.Nk = N;
    cb.D = (int)out_dim;
    cb.grad_pv = gpv;
    cb.ld_gpv = out_dim;
    cb.grad_ps = grad_projected_state;
    cb.dk = s.dP + r;
    cb.lddk = 2 * r;
    cb.part_c = s.part_c;
    cb.bf16 = bf16 ? 1 : 0;
    if (mh) {
      cb.heads = (int)heads;
      cb.head_rank = (int)(rank / heads);
    }
    if (band) {
      cb.band = 1;
      cb.coef = s.coef;
      cb.g_score = s.g_score;
      cb.gds = grad_delta_state;
      cb.ehead = mh ? edge_head : nullptr;
    }
    // dK and the scale partials on the second stream, beside the value gather
    if (side) {
      ColsBwdArgs kg = cb;
      kg.grad_pv = nullptr;
      kg.grad_ps = nullptr;
      rc = fork_to(side, st);
      if (rc) return rc;
      rc = launch_cols_backward(kg, side->stream);
      if (rc) return rc;
      cb.q = nullptr;  // the main stream gathers the values only
    }
    if (band_mfma && gpv && band_kernels_fit(k, (int)out_dim, out_dim, out_dim, grad_delta_val, gpv, bf16)) {
      // the value and state gradients of the sources: the transposed band as MFMA tiles
      BandAggArgs cg{};
      cg.B = B;
      cg.N = N;
      cg.k = k;
      cg.D = (int)out_dim;
      cg.trans = 1;
      cg.coef = s.coef;
      cg.state = grad_delta_state;
      cg.val = grad_delta_val;
      cg.ld_val = out_dim;
      cg.out_state = grad_projected_state;
      cg.out = gpv;
      cg.ld_out = out_dim;
      cg.bf16 = bf16 ? 1 : 0;
      rc = launch_band_aggregate(cg, st);
      if (rc) return rc;
      cb.grad_pv = nullptr;  // the column kernels still compute dK and the scale partials
      cb.grad_ps = nullptr;
    }
    rc = launch_cols_backward(cb, st);
    if (rc) return rc;
    if (side) {
      rc = join_from(side, st);
      if (rc) return rc;
    }
  }

  // 4. projection weight grads: [dU; dV] = dP^T . X  (split-K, fixed order).
  //    On large problems on the second stream, beside the input gradient: its
  //    MFMA work fills the other's HBM-bound epilogue.
  const SideStream* gside =
      (grad_target_weight && grad_source_weight && grad_layer_val) ? side_stream_for(st, (int64_t)M * k) : nullptr;
  if (gside) {
    rc = fork_to(gside, st);
    if (rc) return rc;
  }
  if (grad_target_weight && grad_source_weight) {
    rc = gemm_grad_weight(s.dP, 2 * r, layer_val, in_dim, grad_target_weight, grad_source_weight, r, 2 * r,
                          (int)in_dim, M, s.splitk, gside ? gside->stream : st, bf16);
    if (rc) return rc;
  }

  // 5. grad of layer_val through both projections (+ value grad when pv is layer_val)
  if (grad_layer_val) {
    const float* addend = (projected_val_is_layer_val && gpv) ? grad_layer_val : nullptr;
    rc = gemm_grad_input(s.dP, 2 * r, target_weight, source_weight, r, in_dim, addend, in_dim, grad_layer_val,
                         in_dim, M, (int)in_dim, 2 * r, st, bf16);
    if (rc) return rc;
  }

  // 6. w_hat and bias grads (one bias per head)
  const int nparts = cols_backward_parts(M);
  rc = launch_finalize_small_grads(s.part_c, nparts, r, grad_core_weight, 0, s.rowsum, M, grad_bias, s.stage, st,
                                   mh ? (int)heads : 1);
  if (rc) return rc;
  return gside ? join_from(gside, st) : kOk;
}

// Top-k propagation forward over all ranks (heads * head rank); heads > 1
// also writes each edge's winning head.
int propagation_topk_forward_impl(const float* layer_val, const float* projected_state, const float* projected_val,
                                  const float* target_weight, const float* source_weight, const float* core_weight,
                                  const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                  int64_t rank, int64_t heads, int64_t topk, int32_t compress_kind,
                                  float* delta_state, float* delta_val, float* projections, int32_t* topk_index,
                                  float* topk_score, uint8_t* topk_head, void* edge_layout, size_t edge_layout_bytes,
                                  void* workspace, size_t workspace_bytes,
                                  hipStream_t st, bool bf16 = false) {
  SideForkGuard join_guard;  // joins a fork left open by an error return
  int rc = check_propagation_shapes(batch, nodes, in_dim, out_dim, rank, topk, compress_kind);
  if (rc) return rc;
  const bool mh = heads > 1;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 delta_state && delta_val && projections && topk_index && topk_score && (!mh || topk_head),
             kInvalidArgument, "null tensor pointer");
  const int M = (int)(batch * nodes), r = (int)rank, k = (int)topk;

  rc = gemm_project(layer_val, in_dim, target_weight, source_weight, r, in_dim, projections, 2 * r, M, 2 * r,
                    (int)in_dim, st, bf16);
  if (rc) return rc;

  SelectArgs s{};
  s.q = projections;
  s.key = projections + r;
  s.ldq = 2 * r;
  s.ldk = 2 * r;
  s.q_batch_stride = nodes * 2 * r;
  s.k_batch_stride = nodes * 2 * r;
  s.scale = core_weight;
  s.bias = bias;
  s.scale_on_query = 0;
  s.temperature = 1.0f;
  s.B = (int)batch;
  s.Nq = (int)nodes;
  s.Nk = (int)nodes;
  s.r = r;
  s.k = k;
  s.out_idx = topk_index;
  s.out_score = topk_score;
  s.ws = workspace;
  s.ws_bytes = workspace_bytes;
  s.bf16 = bf16 ? 1 : 0;
  if (mh) {
    s.heads = (int)heads;
    s.head_rank = (int)(rank / heads);
  }
  rc = launch_topk_select(s, st);
  if (rc) return rc;

  if (mh) {  // the winning head of every selected edge
    WindowScoreArgs w{};
    w.q = projections;
    w.key = projections + r;
    w.ldq = 2 * r;
    w.ldk = 2 * r;
    w.scale = core_weight;
    w.bias = bias;
    w.inv_temperature = 1.0f;
    w.B = (int)batch;
    w.Nq = (int)nodes;
    w.Nk = (int)nodes;
    w.r = r;
    w.width = k;
    w.all_keys = 2;
    w.idx = topk_index;
    w.score = topk_score;
    w.heads = (int)heads;
    w.head_rank = (int)(rank / heads);
    w.head = topk_head;
    rc = launch_window_scores(w, st);
    if (rc) return rc;
  }

  // the edges grouped by key for the backward, beside the row pass
  const SideStream* side = nullptr;
  if (edge_layout) {
    const EdgeLayout l = carve_edge_layout(edge_layout, edge_layout_bytes, batch, nodes, topk);
    JN_REQUIRE(l.bytes <= edge_layout_bytes, kWorkspaceTooSmall, "edge layout too small: need %zu bytes, got %zu",
               l.bytes, edge_layout_bytes);
    side = side_stream_for(st, (int64_t)M * k);
    if (side) {
      rc = fork_to(side, st);
      if (rc) return rc;
    }
    rc = build_edge_layout(l, topk_index, topk_score, mh ? topk_head : nullptr, (int)batch, (int)nodes, k,
                           compress_kind, side ? side->stream : st);
    if (rc) return rc;
  }

  RowsFwdArgs f{};
  f.idx = topk_index;
  f.score = topk_score;
  f.k = k;
  f.compress = compress_kind;
  f.ps = projected_state;
  f.pv = projected_val;
  f.ld_pv = out_dim;
  f.Nq = (int)nodes;
  f.Nk = (int)nodes;
  f.D = (int)out_dim;
  f.rows = M;
  f.out_state = delta_state;
  f.out_val = delta_val;
  f.bf16 = bf16 ? 1 : 0;
  rc = launch_rows_forward(f, st);
  if (rc) return rc;
  return side ? join_from(side, st) : kOk;
}

// Window propagation forward over all ranks; heads > 1 also writes each edge's head.
int propagation_window_forward_impl(const float* layer_val, const float* projected_state, const float* projected_val,
                                    const float* target_weight, const float* source_weight, const float* core_weight,
                                    const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                    int64_t rank, int64_t heads, int64_t window, int32_t compress_kind,
                                    float* delta_state, float* delta_val, float* projections, int32_t* edge_index,
                                    float* edge_score, uint8_t* edge_head, hipStream_t st, bool bf16 = false) {
  JN_REQUIRE(window >= 0, kInvalidArgument, "window must be non-negative (got %lld)", (long long)window);
  const int64_t width = window_width(window, nodes);
  int rc = check_edge_shapes(batch, nodes, in_dim, out_dim, rank, width, compress_kind);
  if (rc) return rc;
  const bool mh = heads > 1;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 delta_state && delta_val && projections && edge_index && edge_score && (!mh || edge_head),
             kInvalidArgument, "null tensor pointer");
  const int M = (int)(batch * nodes), r = (int)rank;

  rc = gemm_project(layer_val, in_dim, target_weight, source_weight, r, in_dim, projections, 2 * r, M, 2 * r,
                    (int)in_dim, st, bf16);
  if (rc) return rc;

  WindowScoreArgs w{};
  w.q = projections;
  w.key = projections + r;
  w.ldq = 2 * r;
  w.ldk = 2 * r;
  w.scale = core_weight;
  w.bias = bias;
  w.inv_temperature = 1.0f;
  w.B = (int)batch;
  w.Nq = (int)nodes;
  w.Nk = (int)nodes;
  w.r = r;
  w.width = (int)width;
  w.all_keys = 0;
  w.idx = edge_index;
  w.score = edge_score;
  if (mh) {
    w.heads = (int)heads;
    w.head_rank = (int)(rank / heads);
    w.head = edge_head;
  }
  if (!mh && window_kernels() == 0 &&
      band_kernels_fit((int)width, r, 2 * r, 2 * r, projections, projections + r, false)) {
    BandDotsArgs sd{};  // the band's scores as MFMA tiles of queries against their key span
    sd.B = (int)batch;
    sd.N = (int)nodes;
    sd.k = (int)width;
    sd.D = r;
    sd.gdv = projections;
    sd.ld_gdv = 2 * r;
    sd.pv = projections + r;
    sd.ld_pv = 2 * r;
    sd.ascale = core_weight;
    sd.bias = bias;
    sd.inv_temperature = 1.0f;
    sd.score_out = edge_score;
    sd.idx_out = edge_index;
    rc = launch_band_dots(sd, st);
  } else {
    rc = launch_window_scores(w, st);
  }
  if (rc) return rc;

  if (window_kernels() == 0 &&
      band_kernels_fit((int)width, (int)out_dim, out_dim, out_dim, projected_val, delta_val, bf16)) {
    BandAggArgs f{};  // the band's aggregation as MFMA tiles
    f.B = (int)batch;
    f.N = (int)nodes;
    f.k = (int)width;
    f.D = (int)out_dim;
    f.trans = 0;
    f.compress = compress_kind;
    f.idx = edge_index;
    f.score = edge_score;
    f.state = projected_state;
    f.val = projected_val;
    f.ld_val = out_dim;
    f.out_state = delta_state;
    f.out = delta_val;
    f.ld_out = out_dim;
    f.bf16 = bf16 ? 1 : 0;
    return launch_band_aggregate(f, st);
  }
  RowsFwdArgs f{};
  f.idx = edge_index;
  f.score = edge_score;
  f.k = (int)width;
  f.compress = compress_kind;
  f.ps = projected_state;
  f.pv = projected_val;
  f.ld_pv = out_dim;
  f.Nq = (int)nodes;
  f.Nk = (int)nodes;
  f.D = (int)out_dim;
  f.rows = M;
  f.out_state = delta_state;
  f.out_val = delta_val;
  f.bf16 = bf16 ? 1 : 0;
  return launch_rows_forward(f, st);
}

}  // namespace
}  // namespace jakal

using namespace jakal;

extern "C" {

const char* jn_last_error(void) { return jakal::last_error(); }

int jn_abi_version(void) { return 15; }

int jn_unit_scale_forward(const float* weight, int64_t rows, int64_t rank, float eps, float* weight_hat,
                          jn_stream_t stream) {
  return launch_unit_scale(weight, nullptr, rows, rank, eps, weight_hat, static_cast<hipStream_t>(stream));
}

int jn_unit_scale_backward(const float* weight, const float* grad_weight_hat, int64_t rows, int64_t rank, float eps,
                           float* grad_weight, jn_stream_t stream) {
  JN_REQUIRE(grad_weight_hat, kInvalidArgument, "null tensor pointer");
  return launch_unit_scale(weight, grad_weight_hat, rows, rank, eps, grad_weight, static_cast<hipStream_t>(stream));
}

int jn_profile_enable(int32_t on) {
  std::lock_guard<std::mutex> lock(jakal::g_prof_mu);
  for (auto& r : jakal::g_prof_records) {
    jakal::g_prof_free.push_back(r.start);
    jakal::g_prof_free.push_back(r.stop);
  }
  jakal::g_prof_records.clear();
  jakal::g_prof_on = on != 0;
  return kOk;
}

int jn_set_gemm_tile(int32_t tile) {
  JN_REQUIRE(tile == 0 || tile == 32 || tile == 64 || tile == 128, kInvalidArgument,
             "GEMM tile must be 0, 32, 64 or 128, got %d", (int)tile);
  jakal::set_gemm_tile(tile);
  return kOk;
}

int jn_set_window_kernels(int32_t mode) {
  JN_REQUIRE(mode == 0 || mode == 1, kInvalidArgument, "window kernel mode must be 0 (band) or 1 (edge), got %d",
             (int)mode);
  jakal::set_window_kernels(mode);
  return kOk;
}

int jn_set_side_streams(int32_t on) {
  JN_REQUIRE(on == 0 || on == 1, kInvalidArgument, "side streams: 0 (off) or 1 (on), got %d", (int)on);
  jakal::g_side_streams.store(on, std::memory_order_relaxed);
  return kOk;
}

int jn_set_select_mode(int32_t mode) {
  JN_REQUIRE(mode >= jakal::kSelectSplitF16 && mode <= jakal::kSelectSplitF16Register && mode != 3,
             kInvalidArgument,
             "select mode must be 0 (split fp16; the small-key select for rows of up to 1024 keys), 1 (fp32), 2 "
             "(split fp16, per-wave kernel), 4 (split fp16, cooperative kernel), 5 (split fp16, key-split per-wave "
             "kernel) or 6 (split fp16 on the register kernels only), got %d",
             (int)mode);
  jakal::set_select_mode(mode);
  return kOk;
}

size_t jn_lowrank_topk_select_workspace_bytes(int64_t batch, int64_t nk, int64_t rank) {
  return jakal::select_workspace_bytes(batch, nk, rank);
}

int jn_profile_collect(char* buffer, size_t size) {
  std::lock_guard<std::mutex> lock(jakal::g_prof_mu);
  std::map<std::string, std::pair<long, double>> agg;
  for (auto& r : jakal::g_prof_records) {
    float ms = 0.f;
    JN_HIP_TRY(hipEventSynchronize(r.stop));
    JN_HIP_TRY(hipEventElapsedTime(&ms, r.start, r.stop));
    auto& a = agg[r.name];
    a.first += 1;
    a.second += ms;
    jakal::g_prof_free.push_back(r.start);
    jakal::g_prof_free.push_back(r.stop);
  }
  jakal::g_prof_records.clear();
  std::string out;
  char line[256];
  for (auto& kv : agg) {
    snprintf(line, sizeof(line), "%s %ld %.6f\n", kv.first.c_str(), kv.second.first, kv.second.second);
    out += line;
  }
  JN_REQUIRE(buffer != nullptr && size > out.size(), kInvalidArgument, "profile buffer too small (%zu bytes needed)",
             out.size() + 1);
  memcpy(buffer, out.c_str(), out.size() + 1);
  return kOk;
}

int jn_lowrank_topk_select(const float* query, int64_t ldq, int64_t query_batch_stride, const float* key,
                           int64_t ldk, int64_t key_batch_stride, const float* scale, int32_t scale_on_query,
                           const float* bias, float temperature, int64_t batch, int64_t nq, int64_t nk,
                           int64_t rank, int64_t topk, int32_t* out_index, float* out_score, void* workspace,
                           size_t workspace_bytes, jn_stream_t stream) {
  JN_REQUIRE(query && key && out_index && out_score, kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(batch >= 1 && nq >= 1 && nk >= 1, kInvalidArgument, "batch, nq, nk must be positive");
  JN_REQUIRE(fits_int(batch * nq * topk), kUnsupported, "problem too large");
  SelectArgs a{};
  a.q = query;
  a.key = key;
  a.ldq = ldq;
  a.ldk = ldk;
  a.q_batch_stride = query_batch_stride;
  a.k_batch_stride = key_batch_stride;
  a.scale = scale;
  a.bias = bias;
  a.scale_on_query = scale_on_query;
  a.temperature = temperature;
  a.B = (int)batch;
  a.Nq = (int)nq;
  a.Nk = (int)nk;
  a.r = (int)rank;
  a.k = (int)topk;
  a.out_idx = out_index;
  a.out_score = out_score;
  a.ws = workspace;
  a.ws_bytes = workspace_bytes;
  return launch_topk_select(a, static_cast<hipStream_t>(stream));
}

int jn_propagation_topk_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                const float* target_weight, const float* source_weight, const float* core_weight,
                                const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                int64_t rank, int64_t topk, int32_t compress_kind, float* delta_state,
                                float* delta_val, float* projections, int32_t* topk_index, float* topk_score,
                                void* edge_layout, size_t edge_layout_bytes, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return propagation_topk_forward_impl(layer_val, projected_state, projected_val, target_weight, source_weight,
                                       core_weight, bias, batch, nodes, in_dim, out_dim, rank, 1, topk, compress_kind,
                                       delta_state, delta_val, projections, topk_index, topk_score, nullptr,
                                       edge_layout, edge_layout_bytes, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

size_t jn_propagation_topk_forward_workspace_bytes(int64_t batch, int64_t nodes, int64_t rank) {
  return jakal::select_workspace_bytes(batch, nodes, rank);
}

size_t jn_propagation_topk_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                           int64_t rank, int64_t topk) {
  (void)out_dim;
  if (!csr_table_fits(batch, nodes, nodes)) return 0;  // the edge grouping is beyond its size limit
  return carve_prop_bwd(nullptr, 0, batch, nodes, in_dim, rank, topk).bytes;
}

size_t jn_propagation_topk_layout_bytes(int64_t batch, int64_t nodes, int64_t topk) {
  if (batch < 1 || nodes < 1 || topk < 1 || !csr_table_fits(batch, nodes, nodes)) return 0;
  return carve_edge_layout(nullptr, 0, batch, nodes, topk).bytes;
}

int jn_propagation_topk_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                 const float* target_weight, const float* source_weight, const float* core_weight,
                                 const float* projections, const int32_t* topk_index, const float* topk_score,
                                 const float* grad_delta_state, const float* grad_delta_val, int64_t batch,
                                 int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t topk,
                                 int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val,
                                 float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                 float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                 const void* edge_layout, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  const int rc = check_propagation_shapes(batch, nodes, in_dim, out_dim, rank, topk, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(layer_val, projected_state, projected_val, target_weight, source_weight,
                                    core_weight, projections, topk_index, topk_score, nullptr, grad_delta_state,
                                    grad_delta_val, batch, nodes, in_dim, out_dim, rank, 1, topk, compress_kind,
                                    projected_val_is_layer_val, grad_layer_val, grad_projected_state,
                                    grad_projected_val, grad_target_weight, grad_source_weight, grad_core_weight,
                                    grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), false, false, edge_layout);
}

int jn_propagation_window_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                  const float* target_weight, const float* source_weight, const float* core_weight,
                                  const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                  int64_t rank, int64_t window, int32_t compress_kind, float* delta_state,
                                  float* delta_val, float* projections, int32_t* edge_index, float* edge_score,
                                  jn_stream_t stream) {
  return propagation_window_forward_impl(layer_val, projected_state, projected_val, target_weight, source_weight,
                                         core_weight, bias, batch, nodes, in_dim, out_dim, rank, 1, window,
                                         compress_kind, delta_state, delta_val, projections, edge_index, edge_score,
                                         nullptr, static_cast<hipStream_t>(stream));
}

size_t jn_propagation_window_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                             int64_t rank, int64_t window) {
  (void)out_dim;
  if (window < 0 || nodes < 1) return 0;
  return carve_prop_bwd(nullptr, 0, batch, nodes, in_dim, rank, window_width(window, nodes), 1, false).bytes;
}

int jn_propagation_window_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                   const float* target_weight, const float* source_weight, const float* core_weight,
                                   const float* projections, const int32_t* edge_index, const float* edge_score,
                                   const float* grad_delta_state, const float* grad_delta_val, int64_t batch,
                                   int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t window,
                                   int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val,
                                   float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                   float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                   void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  JN_REQUIRE(window >= 0, kInvalidArgument, "window must be non-negative (got %lld)", (long long)window);
  const int64_t width = window_width(window, nodes);
  const int rc = check_edge_shapes(batch, nodes, in_dim, out_dim, rank, width, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(layer_val, projected_state, projected_val, target_weight, source_weight,
                                    core_weight, projections, edge_index, edge_score, nullptr, grad_delta_state,
                                    grad_delta_val, batch, nodes, in_dim, out_dim, rank, 1, width, compress_kind,
                                    projected_val_is_layer_val, grad_layer_val, grad_projected_state,
                                    grad_projected_val, grad_target_weight, grad_source_weight, grad_core_weight,
                                    grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), false,
                                    true);
}

size_t jn_transition_topk_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                          int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t topk) {
  (void)val_dim;
  if (batch < 1 || src_nodes < 1 || dst_nodes < 1 || topk < 1 || !csr_table_fits(batch, src_nodes, dst_nodes))
    return 0;
  return carve_transition(nullptr, 0, batch, src_nodes, dst_nodes, src_dim, dst_dim, rank,
                          route_edges(topk, dst_nodes))
      .bytes;
}

// rank: all ranks (heads * head rank); heads > 1 also writes each route's head.
static int transition_topk_forward_impl(const float* sender_strength, const float* src_val, const float* dst_val,
                                 const float* projected_state, const float* projected_val, const float* source_weight,
                                 const float* target_weight, const float* core_weight, const float* bias,
                                 float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                 int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
                                 int64_t topk, int32_t compress_kind, float* delta_state, float* delta_val,
                                 float* src_proj, float* dst_proj, int32_t* route_index, float* route_logit,
                                 uint8_t* route_head, void* workspace, size_t workspace_bytes, hipStream_t st,
                                 bool bf16 = false) {
  SideForkGuard join_guard;  // joins a fork left open by an error return
  int rc = check_transition_shapes(batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, topk, compress_kind,
                                   temperature);
  if (rc) return rc;
  const bool mh = heads > 1;
  JN_REQUIRE(sender_strength && src_val && dst_val && projected_state && projected_val && source_weight &&
                 target_weight && core_weight && delta_state && delta_val && src_proj && dst_proj && route_index &&
                 route_logit && (!mh || route_head),
             kInvalidArgument, "null tensor pointer");
  const int64_t k = route_edges(topk, dst_nodes);
  TransitionScratch s = carve_transition(workspace, workspace_bytes, batch, src_nodes, dst_nodes, src_dim, dst_dim,
                                         rank, k, mh ? heads : 1);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  const int B = (int)batch, Ns = (int)src_nodes, Nd = (int)dst_nodes, r = (int)rank;

  // 1. projections P_s = src . Ws^T, P_t = dst . Wt^T  (modules.py:435-437), side by side
  const SideStream* side = side_stream_for(st, batch * src_nodes * k);
  if (side) {
    rc = fork_to(side, st);
    if (rc) return rc;
  }
  rc = gemm_project(dst_val, dst_dim, target_weight, target_weight, r, dst_dim, dst_proj, r, B * Nd, r, (int)dst_dim,
                    side ? side->stream : st, bf16);
  if (rc) return rc;
  rc = gemm_project(src_val, src_dim, source_weight, source_weight, r, src_dim, src_proj, r, B * Ns, r, (int)src_dim,
                    st, bf16);
  if (rc) return rc;
  if (side) {
    rc = join_from(side, st);
    if (rc) return rc;
  }

  // 2. per-source edge list: logits ((P_s * w) . P_t + b) / T, top-k over destinations
  if (k < dst_nodes) {
    SelectArgs a{};
    a.q = src_proj;
    a.key = dst_proj;
    a.ldq = r;
    a.ldk = r;
    a.q_batch_stride = src_nodes * r;
    a.k_batch_stride = dst_nodes * r;
    a.scale = core_weight;
    a.bias = bias;
    a.scale_on_query = 1;
    a.temperature = temperature;
    a.B = B;
    a.Nq = Ns;
    a.Nk = Nd;
    a.r = r;
    a.k = (int)k;
    a.out_idx = route_index;
    a.out_score = route_logit;
    a.ws = s.select_ws;
    a.ws_bytes = s.select_ws_bytes;
    a.bf16 = bf16 ? 1 : 0;
    if (mh) {
      a.heads = (int)heads;
      a.head_rank = (int)(rank / heads);
    }
    rc = launch_topk_select(a, st);
  } else {
    WindowScoreArgs w{};
    w.q = src_proj;
    w.key = dst_proj;
    w.ldq = r;
    w.ldk = r;
    w.scale = core_weight;
    w.bias = bias;
    w.inv_temperature = 1.0f / temperature;
    w.B = B;
    w.Nq = Ns;
    w.Nk = Nd;
    w.r = r;
    w.width = Nd;
    w.all_keys = 1;
    w.idx = route_index;
    w.score = route_logit;
    if (mh) {
      w.heads = (int)heads;
      w.head_rank = (int)(rank / heads);
      w.head = route_head;
    }
    rc = launch_window_scores(w, st);
  }
  if (rc) return rc;
  if (mh && k < dst_nodes) {  // the winning head of every selected route
    WindowScoreArgs w{};
    w.q = src_proj;
    w.key = dst_proj;
    w.ldq = r;
    w.ldk = r;
    w.scale = core_weight;
    w.bias = bias;
    w.inv_temperature = 1.0f / temperature;
    w.B = B;
    w.Nq = Ns;
    w.Nk = Nd;
    w.r = r;
    w.width = (int)k;
    w.all_keys = 2;
    w.idx = route_index;
    w.score = route_logit;
    w.heads = (int)heads;
    w.head_rank = (int)(rank / heads);
    w.head = route_head;
    rc = launch_window_scores(w, st);
    if (rc) return rc;
  }

  // 3. coefficients rho * p (beside the CSR layout, which reads only the
  //    edge index), then destination sums as gathers over the edges
  //    transposed by destination
  CsrArgs ca{};
  ca.idx = route_index;
  ca.k = (int)k;
  ca.B = B;
  ca.Nq = Ns;
  ca.Nk = Nd;
  ca.tile_base = s.tile_base;
  ca.seg_start = s.seg_start;
  ca.rec = s.rec;
  ca.coef = s.coef;
  ca.gds = projected_state;
  if (side) {
    rc = fork_to(side, st);
    if (rc) return rc;
  }
  rc = launch_csr_layout(ca, side ? side->stream : st);
  if (rc) return rc;
  rc = launch_route_coef(route_index, route_logit, sender_strength, (int)k, compress_kind, batch * src_nodes, s.coef,
                         st);
  if (rc) return rc;
  if (side) {
    rc = join_from(side, st);
    if (rc) return rc;
  }
  rc = launch_csr_fill(ca, st);
  if (rc) return rc;
  ColsBwdArgs cb{};
  cb.seg_start = s.seg_start;
  cb.rec = s.rec;
  cb.k = (int)k;
  cb.gdv = projected_val;
  cb.B = B;
  cb.Nq = Ns;
  cb.Nk = Nd;
  cb.D = (int)val_dim;
  cb.grad_pv = delta_val;
  cb.ld_gpv = val_dim;
  cb.grad_ps = delta_state;
  cb.profile_name = "route_gather_kernel";
  cb.bf16 = bf16 ? 1 : 0;
  return launch_cols_backward(cb, st);
}

static int transition_topk_backward_impl(const float* sender_strength, const float* src_val, const float* dst_val,
                                  const float* projected_state, const float* projected_val,
                                  const float* source_weight, const float* target_weight, const float* core_weight,
                                  const float* src_proj, const float* dst_proj, const int32_t* route_index,
                                  const float* route_logit, const uint8_t* route_head, const float* grad_delta_state,
                                  const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
                                  int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                  int64_t heads, int64_t topk, int32_t compress_kind, float* grad_sender_strength,
                                  float* grad_src_val, float* grad_dst_val, float* grad_projected_state,
                                  float* grad_projected_val, float* grad_source_weight, float* grad_target_weight,
                                  float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
                                  hipStream_t st, bool bf16 = false) {
  SideForkGuard join_guard;  // joins a fork left open by an error return
  int rc = check_transition_shapes(batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, topk, compress_kind,
                                   temperature);
  if (rc) return rc;
  const bool mh = heads > 1;
  JN_REQUIRE(sender_strength && src_val && dst_val && projected_state && projected_val && source_weight &&
                 target_weight && core_weight && src_proj && dst_proj && route_index && route_logit &&
                 grad_delta_state && grad_delta_val && (!mh || route_head),
             kInvalidArgument, "null tensor pointer");
  const int64_t k = route_edges(topk, dst_nodes);
  TransitionScratch s = carve_transition(workspace, workspace_bytes, batch, src_nodes, dst_nodes, src_dim, dst_dim,
                                         rank, k, mh ? heads : 1);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  const int B = (int)batch, Ns = (int)src_nodes, Nd = (int)dst_nodes, r = (int)rank;

  // 1. source rows: coefficient grads, route compress backward, sender-strength,
  //    projected state/value grads and the grad of the source projection
  RouteRowsBwdArgs rb{};
  rb.idx = route_index;
  rb.logit = route_logit;
  rb.k = (int)k;
  rb.compress = compress_kind;
  rb.inv_temperature = 1.0f / temperature;
  rb.rho = sender_strength;
  rb.ps = projected_state;
  rb.pv = projected_val;
  rb.ld_pv = val_dim;
  rb.gds = grad_delta_state;
  rb.gdv = grad_delta_val;
  rb.key = dst_proj;
  rb.ldk = r;
  rb.qscale = core_weight;
  rb.r = r;
  rb.Ns = Ns;
  rb.Nd = Nd;
  rb.D = (int)val_dim;
  rb.rows = batch * src_nodes;
  rb.g_logit = s.g_logit;
  rb.grad_rho = grad_sender_strength;
  rb.grad_ps = grad_projected_state;
  rb.grad_pv = grad_projected_val;
  rb.ld_gpv = val_dim;
  rb.dq = s.dPs;
  rb.lddq = r;
  rb.rowsum = s.rowsum;
  rb.bf16 = bf16 ? 1 : 0;
  if (mh) {
    rb.ehead = route_head;
    rb.heads = (int)heads;
    rb.head_rank = (int)(rank / heads);
  }
  // the CSR layout of the routes (it reads only the edge index) beside the row pass
  CsrArgs ca{};
  ca.idx = route_index;
  ca.k = (int)k;
  ca.B = B;
  ca.Nq = Ns;
  ca.Nk = Nd;
  ca.tile_base = s.tile_base;
  ca.seg_start = s.seg_start;
  ca.rec = s.rec;
  ca.g_score = s.g_logit;
  ca.ehead = mh ? route_head : nullptr;
  const SideStream* side = side_stream_for(st, (int64_t)B * Ns * k);
  if (side) {
    rc = fork_to(side, st);
    if (rc) return rc;
  }
  rc = launch_csr_layout(ca, side ? side->stream : st);
  if (rc) return rc;
  rc = launch_route_rows_backward(rb, st);
  if (rc) return rc;
  if (side) {
    rc = join_from(side, st);
    if (rc) return rc;
  }

  // 2. destination columns: grad of the destination projection and w partials
  rc = launch_csr_fill(ca, st);
  if (rc) return rc;
  // the source side's projection grads (ready after the row pass) run beside them
  hipStream_t ss = side ? side->stream : st;
  if (side) {
    rc = fork_to(side, st);
    if (rc) return rc;
  }
  if (grad_source_weight) {
    rc = gemm_grad_weight(s.dPs, r, src_val, src_dim, grad_source_weight, grad_source_weight, r, r, (int)src_dim,
                          B * Ns, s.splitk2, ss, bf16);
    if (rc) return rc;
  }
  if (grad_src_val) {
    rc = gemm_grad_input(s.dPs, r, source_weight, source_weight, r, src_dim, nullptr, 0, grad_src_val, src_dim,
                         B * Ns, (int)src_dim, r, ss, bf16);
    if (rc) return rc;
  }
  ColsBwdArgs cb{};
  cb.seg_start = s.seg_start;
  cb.rec = s.rec;
  cb.k = (int)k;
  cb.q = src_proj;
  cb.ldq = r;
  cb.key = dst_proj;
  cb.ldk = r;
  cb.kscale = core_weight;
  cb.r = r;
  cb.B = B;
  cb.Nq = Ns;
  cb.Nk = Nd;
  cb.D = (int)val_dim;
  cb.dk = s.dPt;
  cb.lddk = r;
  cb.part_c = s.part_c;
  if (mh) {
    cb.heads = (int)heads;
    cb.head_rank = (int)(rank / heads);
  }
  rc = launch_cols_backward(cb, st);
  if (rc) return rc;

  // 3. destination-side projection weight and input grads
  if (grad_target_weight) {
    rc = gemm_grad_weight(s.dPt, r, dst_val, dst_dim, grad_target_weight, grad_target_weight, r, r, (int)dst_dim,
                          B * Nd, s.splitk, st, bf16);
    if (rc) return rc;
  }
  if (grad_dst_val) {
    rc = gemm_grad_input(s.dPt, r, target_weight, target_weight, r, dst_dim, nullptr, 0, grad_dst_val, dst_dim,
                         B * Nd, (int)dst_dim, r, st, bf16);
    if (rc) return rc;
  }
  if (side) {
    rc = join_from(side, st);
    if (rc) return rc;
  }

  // 4. core weight and bias grads.  Softmax routes do not change when a row's
  // logits shift together, so their bias gradient is exactly 0 (no rows summed);
  // one head's bias shifts only its own routes, so every head's column is summed.
  return launch_finalize_small_grads(s.part_c, cols_backward_parts((int64_t)B * Nd), r, grad_core_weight, 0,
                                     s.rowsum, (compress_kind == 0 && !mh) ? 0 : batch * src_nodes, grad_bias,
                                     s.stage, st, mh ? (int)heads : 1);
}

int jn_transition_topk_forward(const float* sender_strength, const float* src_val, const float* dst_val,
                               const float* projected_state, const float* projected_val, const float* source_weight,
                               const float* target_weight, const float* core_weight, const float* bias,
                               float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                               int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t topk,
                               int32_t compress_kind, float* delta_state, float* delta_val, float* src_proj,
                               float* dst_proj, int32_t* route_index, float* route_logit, void* workspace,
                               size_t workspace_bytes, jn_stream_t stream) {
  return transition_topk_forward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                      source_weight, target_weight, core_weight, bias, temperature, batch, src_nodes,
                                      dst_nodes, src_dim, dst_dim, val_dim, rank, 1, topk, compress_kind, delta_state,
                                      delta_val, src_proj, dst_proj, route_index, route_logit, nullptr, workspace,
                                      workspace_bytes, static_cast<hipStream_t>(stream));
}

int jn_transition_topk_backward(const float* sender_strength, const float* src_val, const float* dst_val,
                                const float* projected_state, const float* projected_val, const float* source_weight,
                                const float* target_weight, const float* core_weight, const float* src_proj,
                                const float* dst_proj, const int32_t* route_index, const float* route_logit,
                                const float* grad_delta_state, const float* grad_delta_val, float temperature,
                                int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t topk, int32_t compress_kind,
                                float* grad_sender_strength, float* grad_src_val, float* grad_dst_val,
                                float* grad_projected_state, float* grad_projected_val, float* grad_source_weight,
                                float* grad_target_weight, float* grad_core_weight, float* grad_bias,
                                void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return transition_topk_backward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                       source_weight, target_weight, core_weight, src_proj, dst_proj, route_index,
                                       route_logit, nullptr, grad_delta_state, grad_delta_val, temperature, batch,
                                       src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, 1, topk, compress_kind,
                                       grad_sender_strength, grad_src_val, grad_dst_val, grad_projected_state,
                                       grad_projected_val, grad_source_weight, grad_target_weight, grad_core_weight,
                                       grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

// ---- multi-head max-aggregated scores ---------------------------------------
size_t jn_propagation_topk_forward_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t rank,
                                                             int64_t heads) {
  if (batch < 1 || nodes < 1 || heads < 2) return 0;
  return select_workspace_bytes_heads(batch, nodes, rank, heads);
}

size_t jn_propagation_topk_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                     int64_t rank, int64_t heads, int64_t topk) {
  (void)out_dim;
  if (batch < 1 || nodes < 1 || heads < 2 || topk < 1 || !csr_table_fits(batch, nodes, nodes)) return 0;
  return carve_prop_bwd(nullptr, 0, batch, nodes, in_dim, rank * heads, topk, heads).bytes;
}

int jn_propagation_topk_forward_multihead(const float* layer_val, const float* projected_state,
                                          const float* projected_val, const float* target_weight,
                                          const float* source_weight, const float* core_weight, const float* bias,
                                          int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                          int64_t rank, int64_t heads, int64_t topk, int32_t compress_kind,
                                          float* delta_state, float* delta_val, float* projections,
                                          int32_t* topk_index, float* topk_score, uint8_t* topk_head,
                                          void* edge_layout, size_t edge_layout_bytes, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  const int rc = check_heads(rank, heads);
  if (rc) return rc;
  return propagation_topk_forward_impl(layer_val, projected_state, projected_val, target_weight, source_weight,
                                       core_weight, bias, batch, nodes, in_dim, out_dim, rank * heads, heads, topk,
                                       compress_kind, delta_state, delta_val, projections, topk_index, topk_score,
                                       topk_head, edge_layout, edge_layout_bytes, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int jn_propagation_topk_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* projections, const int32_t* topk_index,
    const float* topk_score, const uint8_t* topk_head, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads, int64_t topk,
    int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
    float* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, const void* edge_layout, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  rc = check_propagation_shapes(batch, nodes, in_dim, out_dim, rank * heads, topk, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(layer_val, projected_state, projected_val, target_weight, source_weight,
                                    core_weight, projections, topk_index, topk_score, topk_head, grad_delta_state,
                                    grad_delta_val, batch, nodes, in_dim, out_dim, rank * heads, heads, topk,
                                    compress_kind, projected_val_is_layer_val, grad_layer_val, grad_projected_state,
                                    grad_projected_val, grad_target_weight, grad_source_weight, grad_core_weight,
                                    grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), false, false, edge_layout);
}

size_t jn_propagation_window_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim,
                                                       int64_t out_dim, int64_t rank, int64_t heads, int64_t window) {
  (void)out_dim;
  if (window < 0 || nodes < 1 || batch < 1 || heads < 2) return 0;
  return carve_prop_bwd(nullptr, 0, batch, nodes, in_dim, rank * heads, window_width(window, nodes), heads, false)
      .bytes;
}

int jn_propagation_window_forward_multihead(const float* layer_val, const float* projected_state,
                                            const float* projected_val, const float* target_weight,
                                            const float* source_weight, const float* core_weight, const float* bias,
                                            int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                            int64_t rank, int64_t heads, int64_t window, int32_t compress_kind,
                                            float* delta_state, float* delta_val, float* projections,
                                            int32_t* edge_index, float* edge_score, uint8_t* edge_head,
                                            jn_stream_t stream) {
  const int rc = check_heads(rank, heads);
  if (rc) return rc;
  return propagation_window_forward_impl(layer_val, projected_state, projected_val, target_weight, source_weight,
                                         core_weight, bias, batch, nodes, in_dim, out_dim, rank * heads, heads,
                                         window, compress_kind, delta_state, delta_val, projections, edge_index,
                                         edge_score, edge_head, static_cast<hipStream_t>(stream));
}

int jn_propagation_window_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* projections, const int32_t* edge_index,
    const float* edge_score, const uint8_t* edge_head, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads, int64_t window,
    int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
    float* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  JN_REQUIRE(window >= 0, kInvalidArgument, "window must be non-negative (got %lld)", (long long)window);
  const int64_t width = window_width(window, nodes);
  rc = check_edge_shapes(batch, nodes, in_dim, out_dim, rank * heads, width, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(layer_val, projected_state, projected_val, target_weight, source_weight,
                                    core_weight, projections, edge_index, edge_score, edge_head, grad_delta_state,
                                    grad_delta_val, batch, nodes, in_dim, out_dim, rank * heads, heads, width,
                                    compress_kind, projected_val_is_layer_val, grad_layer_val, grad_projected_state,
                                    grad_projected_val, grad_target_weight, grad_source_weight, grad_core_weight,
                                    grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), false,
                                    true);
}

size_t jn_transition_topk_multihead_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                                    int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                                    int64_t heads, int64_t topk) {
  (void)val_dim;
  if (batch < 1 || src_nodes < 1 || dst_nodes < 1 || topk < 1 || heads < 2 || rank * heads > 128 ||
      !csr_table_fits(batch, src_nodes, dst_nodes))
    return 0;
  return carve_transition(nullptr, 0, batch, src_nodes, dst_nodes, src_dim, dst_dim, rank * heads,
                          route_edges(topk, dst_nodes), heads)
      .bytes;
}

int jn_transition_topk_forward_multihead(const float* sender_strength, const float* src_val, const float* dst_val,
                                         const float* projected_state, const float* projected_val,
                                         const float* source_weight, const float* target_weight,
                                         const float* core_weight, const float* bias, float temperature,
                                         int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                         int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads, int64_t topk,
                                         int32_t compress_kind, float* delta_state, float* delta_val,
                                         float* src_proj, float* dst_proj, int32_t* route_index, float* route_logit,
                                         uint8_t* route_head, void* workspace, size_t workspace_bytes,
                                         jn_stream_t stream) {
  const int rc = check_heads(rank, heads);
  if (rc) return rc;
  return transition_topk_forward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                      source_weight, target_weight, core_weight, bias, temperature, batch, src_nodes,
                                      dst_nodes, src_dim, dst_dim, val_dim, rank * heads, heads, topk, compress_kind,
                                      delta_state, delta_val, src_proj, dst_proj, route_index, route_logit,
                                      route_head, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int jn_transition_topk_backward_multihead(
    const float* sender_strength, const float* src_val, const float* dst_val, const float* projected_state,
    const float* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const int32_t* route_index, const float* route_logit,
    const uint8_t* route_head, const float* grad_delta_state, const float* grad_delta_val, float temperature,
    int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
    int64_t rank, int64_t heads, int64_t topk, int32_t compress_kind, float* grad_sender_strength,
    float* grad_src_val, float* grad_dst_val, float* grad_projected_state, float* grad_projected_val,
    float* grad_source_weight, float* grad_target_weight, float* grad_core_weight, float* grad_bias,
    void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  const int rc = check_heads(rank, heads);
  if (rc) return rc;
  return transition_topk_backward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                       source_weight, target_weight, core_weight, src_proj, dst_proj, route_index,
                                       route_logit, route_head, grad_delta_state, grad_delta_val, temperature, batch,
                                       src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank * heads, heads, topk,
                                       compress_kind, grad_sender_strength, grad_src_val, grad_dst_val,
                                       grad_projected_state, grad_projected_val, grad_source_weight,
                                       grad_target_weight, grad_core_weight, grad_bias, workspace, workspace_bytes,
                                       static_cast<hipStream_t>(stream));
}

// ---- bf16 layers -------------------------------------------------------------------
// The bf16 tensors arrive as bf16 bit patterns; every kernel that touches them
// reads and writes bf16 (the reinterpret_casts only carry the pointers).
int jn_propagation_topk_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                     const uint16_t* projected_val, const float* target_weight,
                                     const float* source_weight, const float* core_weight, const float* bias,
                                     int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                     int64_t topk, int32_t compress_kind, float* delta_state, uint16_t* delta_val,
                                     float* projections, int32_t* topk_index, float* topk_score, void* edge_layout,
                                     size_t edge_layout_bytes, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return propagation_topk_forward_impl(reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val), target_weight,
                                       source_weight, core_weight, bias, batch, nodes, in_dim, out_dim, rank, 1, topk,
                                       compress_kind, delta_state, reinterpret_cast<float*>(delta_val), projections, topk_index,
                                       topk_score, nullptr, edge_layout, edge_layout_bytes, workspace, workspace_bytes,
                                       static_cast<hipStream_t>(stream), true);
}

int jn_propagation_topk_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    const int32_t* topk_index, const float* topk_score, const float* grad_delta_state,
    const uint16_t* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
    int64_t topk, int32_t compress_kind, int32_t projected_val_is_layer_val, uint16_t* grad_layer_val,
    float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, const void* edge_layout, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  const int rc = check_propagation_shapes(batch, nodes, in_dim, out_dim, rank, topk, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val), target_weight,
                                    source_weight, core_weight, projections, topk_index, topk_score, nullptr,
                                    grad_delta_state, reinterpret_cast<const float*>(grad_delta_val), batch, nodes, in_dim, out_dim, rank, 1,
                                    topk, compress_kind, projected_val_is_layer_val, reinterpret_cast<float*>(grad_layer_val),
                                    grad_projected_state, reinterpret_cast<float*>(grad_projected_val), grad_target_weight,
                                    grad_source_weight, grad_core_weight, grad_bias, workspace, workspace_bytes,
                                    static_cast<hipStream_t>(stream), true, false, edge_layout);
}

int jn_propagation_window_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                       const uint16_t* projected_val, const float* target_weight,
                                       const float* source_weight, const float* core_weight, const float* bias,
                                       int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                       int64_t window, int32_t compress_kind, float* delta_state,
                                       uint16_t* delta_val, float* projections, int32_t* edge_index,
                                       float* edge_score, jn_stream_t stream) {
  return propagation_window_forward_impl(reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val), target_weight,
                                         source_weight, core_weight, bias, batch, nodes, in_dim, out_dim, rank, 1,
                                         window, compress_kind, delta_state, reinterpret_cast<float*>(delta_val), projections, edge_index,
                                         edge_score, nullptr, static_cast<hipStream_t>(stream), true);
}

int jn_propagation_window_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    const int32_t* edge_index, const float* edge_score, const float* grad_delta_state,
    const uint16_t* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
    int64_t window, int32_t compress_kind, int32_t projected_val_is_layer_val, uint16_t* grad_layer_val,
    float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  JN_REQUIRE(window >= 0, kInvalidArgument, "window must be non-negative (got %lld)", (long long)window);
  const int64_t width = window_width(window, nodes);
  const int rc = check_edge_shapes(batch, nodes, in_dim, out_dim, rank, width, compress_kind);
  if (rc) return rc;
  return propagation_edges_backward(reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val), target_weight,
                                    source_weight, core_weight, projections, edge_index, edge_score, nullptr,
                                    grad_delta_state, reinterpret_cast<const float*>(grad_delta_val), batch, nodes, in_dim, out_dim, rank, 1,
                                    width, compress_kind, projected_val_is_layer_val, reinterpret_cast<float*>(grad_layer_val),
                                    grad_projected_state, reinterpret_cast<float*>(grad_projected_val), grad_target_weight,
                                    grad_source_weight, grad_core_weight, grad_bias, workspace, workspace_bytes,
                                    static_cast<hipStream_t>(stream), true, true);
}

int jn_transition_topk_forward_bf16(const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val,
                                    const float* projected_state, const uint16_t* projected_val,
                                    const float* source_weight, const float* target_weight, const float* core_weight,
                                    const float* bias, float temperature, int64_t batch, int64_t src_nodes,
                                    int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
                                    int64_t rank, int64_t topk, int32_t compress_kind, float* delta_state,
                                    uint16_t* delta_val, float* src_proj, float* dst_proj, int32_t* route_index,
                                    float* route_logit, void* workspace, size_t workspace_bytes,
                                    jn_stream_t stream) {
  return transition_topk_forward_impl(sender_strength, reinterpret_cast<const float*>(src_val), reinterpret_cast<const float*>(dst_val), projected_state,
                                      reinterpret_cast<const float*>(projected_val), source_weight, target_weight, core_weight, bias,
                                      temperature, batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, 1,
                                      topk, compress_kind, delta_state, reinterpret_cast<float*>(delta_val), src_proj, dst_proj,
                                      route_index, route_logit, nullptr, workspace, workspace_bytes,
                                      static_cast<hipStream_t>(stream), true);
}

int jn_transition_topk_backward_bf16(
    const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val, const float* projected_state,
    const uint16_t* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const int32_t* route_index, const float* route_logit,
    const float* grad_delta_state, const uint16_t* grad_delta_val, float temperature, int64_t batch,
    int64_t src_nodes, int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
    int64_t topk, int32_t compress_kind, float* grad_sender_strength, uint16_t* grad_src_val,
    uint16_t* grad_dst_val, float* grad_projected_state, uint16_t* grad_projected_val, float* grad_source_weight,
    float* grad_target_weight, float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
    jn_stream_t stream) {
  return transition_topk_backward_impl(
      sender_strength, reinterpret_cast<const float*>(src_val), reinterpret_cast<const float*>(dst_val), projected_state, reinterpret_cast<const float*>(projected_val), source_weight,
      target_weight, core_weight, src_proj, dst_proj, route_index, route_logit, nullptr, grad_delta_state,
      reinterpret_cast<const float*>(grad_delta_val), temperature, batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, 1, topk,
      compress_kind, grad_sender_strength, reinterpret_cast<float*>(grad_src_val), reinterpret_cast<float*>(grad_dst_val), grad_projected_state,
      reinterpret_cast<float*>(grad_projected_val), grad_source_weight, grad_target_weight, grad_core_weight, grad_bias, workspace,
      workspace_bytes, static_cast<hipStream_t>(stream), true);
}

// bf16 dense layers (one head): the bf16 MFMA kernel runs the three N x N
// products, so its preconditions hold for every chunk.
static int check_dense_bf16_shapes(int64_t nodes, int64_t out_dim) {
  JN_REQUIRE(nodes >= 128 && out_dim >= 128 && nodes % 8 == 0 && out_dim % 8 == 0, kUnsupported,
             "bf16 dense propagation needs nodes and out_dim >= 128 and multiples of 8 (got %lld, %lld)",
             (long long)nodes, (long long)out_dim);
  return kOk;
}

static int propagation_dense_forward_impl(const float* layer_val, const float* projected_state,
                                          const float* projected_val, const float* target_weight,
                                          const float* source_weight, const float* core_weight, const float* bias,
                                          int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                          int32_t compress_kind, int32_t causal, float* delta_state, float* delta_val,
                                          float* projections, float* edges, hipStream_t st, bool bf16) {
  int rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank, compress_kind);
  if (rc) return rc;
  if (bf16 && (rc = check_dense_bf16_shapes(nodes, out_dim))) return rc;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 delta_state && delta_val && projections && edges,
             kInvalidArgument, "null tensor pointer");
  const int B = (int)batch, N = (int)nodes, r = (int)rank, D = (int)out_dim;
  rc = gemm_project(layer_val, in_dim, target_weight, source_weight, r, in_dim, projections, 2 * r, B * N, 2 * r,
                    (int)in_dim, st, bf16);
  if (rc) return rc;
  return dense_forward_range(projected_state, projected_val, core_weight, bias, 0, B, N, D, r, compress_kind,
                             causal != 0, projections, edges, delta_state, delta_val, st, 1, nullptr, bf16);
}

int jn_propagation_dense_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                 const float* target_weight, const float* source_weight, const float* core_weight,
                                 const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                 int64_t rank, int32_t compress_kind, int32_t causal, float* delta_state,
                                 float* delta_val, float* projections, float* edges, jn_stream_t stream) {
  return propagation_dense_forward_impl(layer_val, projected_state, projected_val, target_weight, source_weight,
                                        core_weight, bias, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
                                        delta_state, delta_val, projections, edges, static_cast<hipStream_t>(stream),
                                        false);
}

int jn_propagation_dense_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                      const uint16_t* projected_val, const float* target_weight,
                                      const float* source_weight, const float* core_weight, const float* bias,
                                      int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                      int32_t compress_kind, int32_t causal, float* delta_state, uint16_t* delta_val,
                                      float* projections, float* edges, jn_stream_t stream) {
  return propagation_dense_forward_impl(reinterpret_cast<const float*>(layer_val), projected_state,
                                        reinterpret_cast<const float*>(projected_val), target_weight, source_weight,
                                        core_weight, bias, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
                                        delta_state, reinterpret_cast<float*>(delta_val), projections, edges,
                                        static_cast<hipStream_t>(stream), true);
}

size_t jn_propagation_dense_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                            int64_t rank, int32_t compress_kind, int32_t reuse_edges) {
  (void)out_dim;
  if (batch < 1 || nodes < 1 || rank < 1) return 0;
  return carve_dense(nullptr, 0, batch, nodes, in_dim, rank, !(compress_kind == 0 && reuse_edges != 0) ? batch : 0,
                     0)
      .bytes;
}

static int propagation_dense_backward_impl(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* projections, float* edges,
    const float* grad_delta_state, const float* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim,
    int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal, int32_t projected_val_is_layer_val,
    int32_t reuse_edges, float* grad_layer_val, float* grad_projected_state, float* grad_projected_val,
    float* grad_target_weight, float* grad_source_weight, float* grad_core_weight, float* grad_bias, void* workspace,
    size_t workspace_bytes, hipStream_t st, bool bf16) {
  int rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank, compress_kind);
  if (rc) return rc;
  if (bf16 && (rc = check_dense_bf16_shapes(nodes, out_dim))) return rc;
  JN_REQUIRE(edges, kInvalidArgument, "null tensor pointer");
  // softsign's derivative runs in the score-gradient GEMM's epilogue, which
  // reads each edge once before writing its gradient: with reuse_edges that
  // gradient overwrites the edge matrix and no [B, N, N] workspace is needed
  const bool in_place = compress_kind == 0 && reuse_edges != 0;
  DenseScratch s = carve_dense(workspace, workspace_bytes, batch, nodes, in_dim, rank, in_place ? 0 : batch, 0);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  return dense_backward(layer_val, projected_state, projected_val, target_weight, source_weight, core_weight, nullptr,
                        projections, edges, in_place ? edges : s.G, (int)batch, false, false, grad_delta_state,
                        grad_delta_val, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
                        projected_val_is_layer_val, grad_layer_val, grad_projected_state, grad_projected_val,
                        grad_target_weight, grad_source_weight, grad_core_weight, grad_bias, s, st, 1, nullptr, bf16);
}

int jn_propagation_dense_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                  const float* target_weight, const float* source_weight, const float* core_weight,
                                  const float* projections, float* edges, const float* grad_delta_state,
                                  const float* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim,
                                  int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
                                  int32_t projected_val_is_layer_val, int32_t reuse_edges, float* grad_layer_val,
                                  float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                  float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                  void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return propagation_dense_backward_impl(
      layer_val, projected_state, projected_val, target_weight, source_weight, core_weight, projections, edges,
      grad_delta_state, grad_delta_val, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
      projected_val_is_layer_val, reuse_edges, grad_layer_val, grad_projected_state, grad_projected_val,
      grad_target_weight, grad_source_weight, grad_core_weight, grad_bias, workspace, workspace_bytes,
      static_cast<hipStream_t>(stream), false);
}

int jn_propagation_dense_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    float* edges, const float* grad_delta_state, const uint16_t* grad_delta_val, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
    int32_t projected_val_is_layer_val, int32_t reuse_edges, uint16_t* grad_layer_val, float* grad_projected_state,
    uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return propagation_dense_backward_impl(
      reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val),
      target_weight, source_weight, core_weight, projections, edges, grad_delta_state,
      reinterpret_cast<const float*>(grad_delta_val), batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
      projected_val_is_layer_val, reuse_edges, reinterpret_cast<float*>(grad_layer_val), grad_projected_state,
      reinterpret_cast<float*>(grad_projected_val), grad_target_weight, grad_source_weight, grad_core_weight,
      grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), true);
}

size_t jn_propagation_dense_chunked_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                    int64_t rank, int32_t compress_kind, int64_t chunk_batch,
                                                    int32_t backward) {
  (void)out_dim;
  if (batch < 1 || nodes < 1 || rank < 1 || chunk_batch < 1) return 0;
  const int64_t cb = chunk_batch < batch ? chunk_batch : batch;
  if (!backward) return (size_t)cb * nodes * nodes * sizeof(float) + 256;
  return carve_dense(nullptr, 0, batch, nodes, in_dim, rank, compress_kind == 0 ? 0 : cb, 0).bytes;
}

static int propagation_dense_forward_chunked_impl(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal, int64_t chunk_batch,
    float* delta_state, float* delta_val, float* projections, void* workspace, size_t workspace_bytes,
    hipStream_t st, bool bf16) {
  int rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank, compress_kind);
  if (rc) return rc;
  if (bf16 && (rc = check_dense_bf16_shapes(nodes, out_dim))) return rc;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 delta_state && delta_val && projections,
             kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(chunk_batch >= 1, kInvalidArgument, "chunk_batch must be positive");
  const int B = (int)batch, N = (int)nodes, r = (int)rank, D = (int)out_dim;
  const int cb = (int)(chunk_batch < batch ? chunk_batch : batch);
  Workspace ws(workspace, workspace_bytes);
  float* E = ws.take<float>((int64_t)cb * N * N);
  JN_REQUIRE(workspace != nullptr && ws.used <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", ws.used, workspace_bytes);
  rc = gemm_project(layer_val, in_dim, target_weight, source_weight, r, in_dim, projections, 2 * r, B * N, 2 * r,
                    (int)in_dim, st, bf16);
  if (rc) return rc;
  for (int b0 = 0; b0 < B; b0 += cb) {
    rc = dense_forward_range(projected_state, projected_val, core_weight, bias, b0, std::min(cb, B - b0), N, D, r,
                             compress_kind, causal != 0, projections, E, delta_state, delta_val, st, 1, nullptr,
                             bf16);
    if (rc) return rc;
  }
  return kOk;
}

int jn_propagation_dense_forward_chunked(const float* layer_val, const float* projected_state,
                                         const float* projected_val, const float* target_weight,
                                         const float* source_weight, const float* core_weight, const float* bias,
                                         int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                         int32_t compress_kind, int32_t causal, int64_t chunk_batch,
                                         float* delta_state, float* delta_val, float* projections, void* workspace,
                                         size_t workspace_bytes, jn_stream_t stream) {
  return propagation_dense_forward_chunked_impl(layer_val, projected_state, projected_val, target_weight,
                                                source_weight, core_weight, bias, batch, nodes, in_dim, out_dim, rank,
                                                compress_kind, causal, chunk_batch, delta_state, delta_val,
                                                projections, workspace, workspace_bytes,
                                                static_cast<hipStream_t>(stream), false);
}

int jn_propagation_dense_forward_chunked_bf16(const uint16_t* layer_val, const float* projected_state,
                                              const uint16_t* projected_val, const float* target_weight,
                                              const float* source_weight, const float* core_weight, const float* bias,
                                              int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                              int64_t rank, int32_t compress_kind, int32_t causal,
                                              int64_t chunk_batch, float* delta_state, uint16_t* delta_val,
                                              float* projections, void* workspace, size_t workspace_bytes,
                                              jn_stream_t stream) {
  return propagation_dense_forward_chunked_impl(
      reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val),
      target_weight, source_weight, core_weight, bias, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
      chunk_batch, delta_state, reinterpret_cast<float*>(delta_val), projections, workspace, workspace_bytes,
      static_cast<hipStream_t>(stream), true);
}

static int propagation_dense_backward_chunked_impl(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, const float* projections,
    float* edge_chunk, const float* grad_delta_state, const float* grad_delta_val, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
    int32_t projected_val_is_layer_val, int64_t chunk_batch, int32_t chunk_resident, float* grad_layer_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, hipStream_t st, bool bf16) {
  int rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank, compress_kind);
  if (rc) return rc;
  if (bf16 && (rc = check_dense_bf16_shapes(nodes, out_dim))) return rc;
  JN_REQUIRE(chunk_batch >= 1, kInvalidArgument, "chunk_batch must be positive");
  JN_REQUIRE(edge_chunk, kInvalidArgument, "null tensor pointer");
  const int cb = (int)(chunk_batch < batch ? chunk_batch : batch);
  DenseScratch s = carve_dense(workspace, workspace_bytes, batch, nodes, in_dim, rank, compress_kind == 0 ? 0 : cb, 0);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  return dense_backward(layer_val, projected_state, projected_val, target_weight, source_weight, core_weight, bias,
                        projections, edge_chunk, compress_kind == 0 ? edge_chunk : s.G, cb, true, chunk_resident != 0,
                        grad_delta_state, grad_delta_val,
                        batch, nodes, in_dim, out_dim, rank, compress_kind, causal, projected_val_is_layer_val,
                        grad_layer_val, grad_projected_state, grad_projected_val, grad_target_weight,
                        grad_source_weight, grad_core_weight, grad_bias, s, st, 1, nullptr, bf16);
}

int jn_propagation_dense_backward_chunked(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, const float* projections,
    float* edge_chunk, const float* grad_delta_state, const float* grad_delta_val, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
    int32_t projected_val_is_layer_val, int64_t chunk_batch, int32_t chunk_resident, float* grad_layer_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return propagation_dense_backward_chunked_impl(
      layer_val, projected_state, projected_val, target_weight, source_weight, core_weight, bias, projections,
      edge_chunk, grad_delta_state, grad_delta_val, batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
      projected_val_is_layer_val, chunk_batch, chunk_resident, grad_layer_val, grad_projected_state,
      grad_projected_val, grad_target_weight, grad_source_weight, grad_core_weight, grad_bias, workspace,
      workspace_bytes, static_cast<hipStream_t>(stream), false);
}

int jn_propagation_dense_backward_chunked_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* bias,
    const float* projections, float* edge_chunk, const float* grad_delta_state, const uint16_t* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind,
    int32_t causal, int32_t projected_val_is_layer_val, int64_t chunk_batch, int32_t chunk_resident,
    uint16_t* grad_layer_val, float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight,
    float* grad_source_weight, float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
    jn_stream_t stream) {
  return propagation_dense_backward_chunked_impl(
      reinterpret_cast<const float*>(layer_val), projected_state, reinterpret_cast<const float*>(projected_val),
      target_weight, source_weight, core_weight, bias, projections, edge_chunk, grad_delta_state,
      reinterpret_cast<const float*>(grad_delta_val), batch, nodes, in_dim, out_dim, rank, compress_kind, causal,
      projected_val_is_layer_val, chunk_batch, chunk_resident, reinterpret_cast<float*>(grad_layer_val),
      grad_projected_state, reinterpret_cast<float*>(grad_projected_val), grad_target_weight, grad_source_weight,
      grad_core_weight, grad_bias, workspace, workspace_bytes, static_cast<hipStream_t>(stream), true);
}

// Dense transition forward; heads > 1: max-aggregated route logits over the
// heads' rank slices (rank = heads * head rank, bias [heads]), the winning
// head of every (source, destination) pair in route_heads [B, Ns, Nd].
// bf16 dense transitions (one head): the bf16 MFMA kernel runs the three
// Ns x Nd products, so its preconditions hold.
static int check_transition_dense_bf16_shapes(int64_t src_nodes, int64_t dst_nodes, int64_t val_dim, int64_t heads) {
  JN_REQUIRE(heads == 1, kUnsupported, "bf16 dense transitions have one head");
  JN_REQUIRE(src_nodes >= 128 && dst_nodes >= 128 && val_dim >= 128 && src_nodes % 8 == 0 && dst_nodes % 8 == 0 &&
                 val_dim % 8 == 0,
             kUnsupported,
             "bf16 dense transitions need src_nodes, dst_nodes and val_dim >= 128 and multiples of 8 (got %lld, %lld, "
             "%lld)",
             (long long)src_nodes, (long long)dst_nodes, (long long)val_dim);
  return kOk;
}

static int transition_dense_forward_impl(const float* sender_strength, const float* src_val, const float* dst_val,
                                         const float* projected_state, const float* projected_val,
                                         const float* source_weight, const float* target_weight,
                                         const float* core_weight, const float* bias, float temperature,
                                         int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                         int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
                                         int32_t compress_kind, float* delta_state, float* delta_val,
                                         float* src_proj, float* dst_proj, float* routes, uint8_t* route_heads,
                                         jn_stream_t stream, bool bf16 = false) {
  int rc = check_transition_dense_shapes(batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, compress_kind,
                                         temperature);
  if (rc) return rc;
  if (bf16 && (rc = check_transition_dense_bf16_shapes(src_nodes, dst_nodes, val_dim, heads))) return rc;
  JN_REQUIRE(heads == 1 || route_heads, kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(sender_strength && src_val && dst_val && projected_state && projected_val && source_weight &&
                 target_weight && core_weight && delta_state && delta_val && src_proj && dst_proj && routes,
             kInvalidArgument, "null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int B = (int)batch, Ns = (int)src_nodes, Nd = (int)dst_nodes, r = (int)rank, Dv = (int)val_dim;

  // 1. projections P_s = src . Ws^T, P_t = dst . Wt^T  (modules.py:435-437)
  rc = gemm_project(src_val, src_dim, source_weight, source_weight, r, src_dim, src_proj, r, B * Ns, r, (int)src_dim,
                    st, bf16);
  if (rc) return rc;
  rc = gemm_project(dst_val, dst_dim, target_weight, target_weight, r, dst_dim, dst_proj, r, B * Nd, r, (int)dst_dim,
                    st, bf16);
  if (rc) return rc;
  // 2. raw logits L_b = (P_s diag(w)) P_t^T; with heads, max_h of each head's
  //    logits plus its bias (one GEMM per head, folded in the epilogue)
  const int H = (int)heads, rh = r / H;
  for (int h = 0; h < H; ++h) {
    BatchedGemm lg{};
    lg.A = src_proj + h * rh; lg.lda = r; lg.a_bs = (int64_t)Ns * r; lg.a_kcontig = true;
    lg.B = dst_proj + h * rh; lg.ldb = r; lg.b_bs = (int64_t)Nd * r; lg.b_kcontig = true;
    lg.C = routes; lg.ldc = Nd; lg.c_bs = (int64_t)Ns * Nd;
    lg.a_kscale = core_weight + h * rh;
    lg.M = Ns; lg.N = Nd; lg.K = rh; lg.batch = B;
    if (H > 1) {
      lg.fold = h == 0 ? 1 : 2; lg.fold_head = h; lg.fold_bias = bias ? bias + h : nullptr;
      lg.fold_heads = route_heads;
    }
    rc = gemm_batched(lg, kGemmRouteLogits, st);
    if (rc) return rc;
  }
  // 3. routes R = compress((L + b) / T) over destinations, in place
  rc = launch_route_dense_compress(routes, H > 1 ? nullptr : bias, 1.0f / temperature, B, Ns, Nd, compress_kind, st);
  if (rc) return rc;
  // 4. delta_state = R^T (rho * ps), delta_val = R^T diag(rho) pv
  rc = launch_route_dense_colsum(routes, sender_strength, projected_state, B, Ns, Nd, delta_state, st);
  if (rc) return rc;
  BatchedGemm ag{};
  ag.A = routes; ag.lda = Nd; ag.a_bs = (int64_t)Ns * Nd; ag.a_kcontig = false;
  ag.B = projected_val; ag.ldb = Dv; ag.b_bs = (int64_t)Ns * Dv; ag.b_kcontig = false;
  ag.C = delta_val; ag.ldc = Dv; ag.c_bs = (int64_t)Nd * Dv;
  ag.a_kscale = sender_strength; ag.ks_bs = Ns;
  ag.M = Nd; ag.N = Dv; ag.K = Ns; ag.batch = B;
  return gemm_batched(ag, bf16 ? kGemmRouteAggregateBf16 : kGemmRouteAggregate, st);
}

int jn_transition_dense_forward(const float* sender_strength, const float* src_val, const float* dst_val,
                                const float* projected_state, const float* projected_val, const float* source_weight,
                                const float* target_weight, const float* core_weight, const float* bias,
                                float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                int32_t compress_kind, float* delta_state, float* delta_val, float* src_proj,
                                float* dst_proj, float* routes, jn_stream_t stream) {
  return transition_dense_forward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                       source_weight, target_weight, core_weight, bias, temperature, batch, src_nodes,
                                       dst_nodes, src_dim, dst_dim, val_dim, rank, 1, compress_kind, delta_state,
                                       delta_val, src_proj, dst_proj, routes, nullptr, stream);
}

size_t jn_transition_dense_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                           int64_t dst_dim, int64_t val_dim, int64_t rank) {
  (void)val_dim;
  if (batch < 1 || src_nodes < 1 || dst_nodes < 1 || rank < 1) return 0;
  return carve_transition_dense(nullptr, 0, batch, src_nodes, dst_nodes, src_dim, dst_dim, rank).bytes;
}

static int transition_dense_backward_impl(
    const float* sender_strength, const float* src_val, const float* dst_val, const float* projected_state,
    const float* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const float* routes, const uint8_t* route_heads,
    const float* grad_delta_state, const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
    int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
    int32_t compress_kind, float* grad_sender_strength, float* grad_src_val, float* grad_dst_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_source_weight, float* grad_target_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream,
    bool bf16 = false) {
  int rc = check_transition_dense_shapes(batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, compress_kind,
                                         temperature);
  if (rc) return rc;
  if (bf16 && (rc = check_transition_dense_bf16_shapes(src_nodes, dst_nodes, val_dim, heads))) return rc;
  JN_REQUIRE(sender_strength && src_val && dst_val && projected_state && projected_val && source_weight &&
                 target_weight && core_weight && src_proj && dst_proj && routes && grad_delta_state &&
                 grad_delta_val && (heads == 1 || route_heads),
             kInvalidArgument, "null tensor pointer");
  TransitionDenseScratch s = carve_transition_dense(workspace, workspace_bytes, batch, src_nodes, dst_nodes, src_dim,
                                                    dst_dim, rank, heads);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int B = (int)batch, Ns = (int)src_nodes, Nd = (int)dst_nodes, r = (int)rank, Dv = (int)val_dim;

  // 1. H_b = pv_b gdv_b^T, then the raw-logit gradient in place (+ sender, state grads, row sums)
  BatchedGemm hg{};
  hg.A = projected_val; hg.lda = Dv; hg.a_bs = (int64_t)Ns * Dv; hg.a_kcontig = true;
  hg.B = grad_delta_val; hg.ldb = Dv; hg.b_bs = (int64_t)Nd * Dv; hg.b_kcontig = true;
  hg.C = s.G; hg.ldc = Nd; hg.c_bs = (int64_t)Ns * Nd;
  hg.M = Ns; hg.N = Nd; hg.K = Dv; hg.batch = B;
  rc = gemm_batched(hg, bf16 ? kGemmRouteEdgeGradBf16 : kGemmRouteEdgeGrad, st);
  if (rc) return rc;
  rc = launch_route_dense_compress_backward(s.G, routes, sender_strength, projected_state, grad_delta_state, B, Ns,
                                            Nd, compress_kind, 1.0f / temperature, grad_sender_strength,
                                            grad_projected_state, s.rowsum, st);
  if (rc) return rc;
  // 2. grad pv = diag(rho) R gdv
  if (grad_projected_val) {
    BatchedGemm vg{};
    vg.A = routes; vg.lda = Nd; vg.a_bs = (int64_t)Ns * Nd; vg.a_kcontig = true;
    vg.B = grad_delta_val; vg.ldb = Dv; vg.b_bs = (int64_t)Nd * Dv; vg.b_kcontig = false;
    vg.C = grad_projected_val; vg.ldc = Dv; vg.c_bs = (int64_t)Ns * Dv;
    vg.c_mscale = sender_strength; vg.ms_bs = Ns;
    vg.M = Ns; vg.N = Dv; vg.K = Nd; vg.batch = B;
    rc = gemm_batched(vg, bf16 ? kGemmRouteValueGradBf16 : kGemmRouteValueGrad, st);
    if (rc) return rc;
  }
  // multi-head: each pair's logit gradient reaches its winning head only (per-head
  // bias partials; the rank-r products below on G masked to that head's pairs)
  const int H = (int)heads, rh = r / H;
  if (H > 1) {
    rc = launch_head_rowsum(s.G, route_heads, Nd, Nd, (int64_t)B * Ns, H, s.rowsum, st);
    if (rc) return rc;
  }
  // 3. projection grads: dP_s = w * (G P_t) (+ w partials), dP_t = w * (G^T P_s)
  for (int h = 0; h < H; ++h) {
    BatchedGemm sg{};
    sg.A = s.G; sg.lda = Nd; sg.a_bs = (int64_t)Ns * Nd; sg.a_kcontig = true;
    sg.B = dst_proj + h * rh; sg.ldb = r; sg.b_bs = (int64_t)Nd * r; sg.b_kcontig = false;
    sg.C = s.dPs + h * rh; sg.ldc = r; sg.c_bs = (int64_t)Ns * r;
    sg.M = Ns; sg.N = rh; sg.K = Nd; sg.batch = B;
    if (H > 1) { sg.a_heads = route_heads; sg.a_head = h; }
    rc = gemm_batched(sg, kGemmRouteSourceGrad, st);
    if (rc) return rc;
  }
  rc = launch_scale_grad_partials(s.dPs, r, src_proj, r, core_weight, r, (int64_t)B * Ns, s.part_c, st);
  if (rc) return rc;
  for (int h = 0; h < H; ++h) {
    BatchedGemm tg{};
    tg.A = s.G; tg.lda = Nd; tg.a_bs = (int64_t)Ns * Nd; tg.a_kcontig = false;
    tg.B = src_proj + h * rh; tg.ldb = r; tg.b_bs = (int64_t)Ns * r; tg.b_kcontig = false;
    tg.C = s.dPt + h * rh; tg.ldc = r; tg.c_bs = (int64_t)Nd * r;
    tg.c_nscale = core_weight + h * rh;
    tg.M = Nd; tg.N = rh; tg.K = Ns; tg.batch = B;
    if (H > 1) { tg.a_heads = route_heads; tg.a_head = h; }
    rc = gemm_batched(tg, kGemmRouteTargetGrad, st);
    if (rc) return rc;
  }
  // 4. projection weight and input grads
  const int Ms = B * Ns, Mt = B * Nd;
  if (grad_source_weight) {
    rc = gemm_grad_weight(s.dPs, r, src_val, src_dim, grad_source_weight, grad_source_weight, r, r, (int)src_dim, Ms,
                          s.splitk, st, bf16);
    if (rc) return rc;
  }
  if (grad_target_weight) {
    rc = gemm_grad_weight(s.dPt, r, dst_val, dst_dim, grad_target_weight, grad_target_weight, r, r, (int)dst_dim, Mt,
                          s.splitk, st, bf16);
    if (rc) return rc;
  }
  if (grad_src_val) {
    rc = gemm_grad_input(s.dPs, r, source_weight, source_weight, r, src_dim, nullptr, src_dim, grad_src_val, src_dim,
                         Ms, (int)src_dim, r, st, bf16);
    if (rc) return rc;
  }
  if (grad_dst_val) {
    rc = gemm_grad_input(s.dPt, r, target_weight, target_weight, r, dst_dim, nullptr, dst_dim, grad_dst_val, dst_dim,
                         Mt, (int)dst_dim, r, st, bf16);
    if (rc) return rc;
  }
  // 5. w and bias grads (one head: exactly 0 for softmax routes, since shifting a
  //    row's logits leaves it unchanged; several: each head's pairs only)
  if (H > 1)
    return launch_finalize_small_grads(s.part_c, Ms, r, grad_core_weight, 0, s.rowsum, Ms, grad_bias, s.stage, st, H);
  return launch_finalize_small_grads(s.part_c, Ms, r, grad_core_weight, 0, s.rowsum, compress_kind == 0 ? 0 : Ms,
                                     grad_bias, s.stage, st);
}

int jn_transition_dense_backward(const float* sender_strength, const float* src_val, const float* dst_val,
                                 const float* projected_state, const float* projected_val, const float* source_weight,
                                 const float* target_weight, const float* core_weight, const float* src_proj,
                                 const float* dst_proj, const float* routes, const float* grad_delta_state,
                                 const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
                                 int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                 int32_t compress_kind, float* grad_sender_strength, float* grad_src_val,
                                 float* grad_dst_val, float* grad_projected_state, float* grad_projected_val,
                                 float* grad_source_weight, float* grad_target_weight, float* grad_core_weight,
                                 float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return transition_dense_backward_impl(
      sender_strength, src_val, dst_val, projected_state, projected_val, source_weight, target_weight, core_weight,
      src_proj, dst_proj, routes, nullptr, grad_delta_state, grad_delta_val, temperature, batch, src_nodes, dst_nodes,
      src_dim, dst_dim, val_dim, rank, 1, compress_kind, grad_sender_strength, grad_src_val, grad_dst_val,
      grad_projected_state, grad_projected_val, grad_source_weight, grad_target_weight, grad_core_weight, grad_bias,
      workspace, workspace_bytes, stream);
}

int jn_transition_dense_forward_bf16(const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val,
                                     const float* projected_state, const uint16_t* projected_val,
                                     const float* source_weight, const float* target_weight, const float* core_weight,
                                     const float* bias, float temperature, int64_t batch, int64_t src_nodes,
                                     int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
                                     int64_t rank, int32_t compress_kind, float* delta_state, uint16_t* delta_val,
                                     float* src_proj, float* dst_proj, float* routes, jn_stream_t stream) {
  return transition_dense_forward_impl(
      sender_strength, reinterpret_cast<const float*>(src_val), reinterpret_cast<const float*>(dst_val),
      projected_state, reinterpret_cast<const float*>(projected_val), source_weight, target_weight, core_weight, bias,
      temperature, batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, 1, compress_kind, delta_state,
      reinterpret_cast<float*>(delta_val), src_proj, dst_proj, routes, nullptr, stream, true);
}

int jn_transition_dense_backward_bf16(
    const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val, const float* projected_state,
    const uint16_t* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const float* routes, const float* grad_delta_state,
    const uint16_t* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
    int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int32_t compress_kind,
    float* grad_sender_strength, uint16_t* grad_src_val, uint16_t* grad_dst_val, float* grad_projected_state,
    uint16_t* grad_projected_val, float* grad_source_weight, float* grad_target_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  return transition_dense_backward_impl(
      sender_strength, reinterpret_cast<const float*>(src_val), reinterpret_cast<const float*>(dst_val),
      projected_state, reinterpret_cast<const float*>(projected_val), source_weight, target_weight, core_weight,
      src_proj, dst_proj, routes, nullptr, grad_delta_state, reinterpret_cast<const float*>(grad_delta_val),
      temperature, batch, src_nodes, dst_nodes, src_dim, dst_dim, val_dim, rank, 1, compress_kind,
      grad_sender_strength, reinterpret_cast<float*>(grad_src_val), reinterpret_cast<float*>(grad_dst_val),
      grad_projected_state, reinterpret_cast<float*>(grad_projected_val), grad_source_weight, grad_target_weight,
      grad_core_weight, grad_bias, workspace, workspace_bytes, stream, true);
}

// ---- max-aggregated multi-head dense forms ---------------------------------

int jn_transition_dense_forward_multihead(const float* sender_strength, const float* src_val, const float* dst_val,
                                          const float* projected_state, const float* projected_val,
                                          const float* source_weight, const float* target_weight,
                                          const float* core_weight, const float* bias, float temperature,
                                          int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                          int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
                                          int32_t compress_kind, float* delta_state, float* delta_val,
                                          float* src_proj, float* dst_proj, float* routes, uint8_t* route_heads,
                                          jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  return transition_dense_forward_impl(sender_strength, src_val, dst_val, projected_state, projected_val,
                                       source_weight, target_weight, core_weight, bias, temperature, batch, src_nodes,
                                       dst_nodes, src_dim, dst_dim, val_dim, rank * heads, heads, compress_kind,
                                       delta_state, delta_val, src_proj, dst_proj, routes, route_heads, stream);
}

size_t jn_transition_dense_multihead_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                                     int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                                     int64_t heads) {
  (void)val_dim;
  if (batch < 1 || src_nodes < 1 || dst_nodes < 1 || rank < 1 || heads < 1) return 0;
  return carve_transition_dense(nullptr, 0, batch, src_nodes, dst_nodes, src_dim, dst_dim, rank * heads, heads).bytes;
}

int jn_transition_dense_backward_multihead(
    const float* sender_strength, const float* src_val, const float* dst_val, const float* projected_state,
    const float* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const float* routes, const uint8_t* route_heads,
    const float* grad_delta_state, const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
    int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
    int32_t compress_kind, float* grad_sender_strength, float* grad_src_val, float* grad_dst_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_source_weight, float* grad_target_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  return transition_dense_backward_impl(
      sender_strength, src_val, dst_val, projected_state, projected_val, source_weight, target_weight, core_weight,
      src_proj, dst_proj, routes, route_heads, grad_delta_state, grad_delta_val, temperature, batch, src_nodes,
      dst_nodes, src_dim, dst_dim, val_dim, rank * heads, heads, compress_kind, grad_sender_strength, grad_src_val,
      grad_dst_val, grad_projected_state, grad_projected_val, grad_source_weight, grad_target_weight,
      grad_core_weight, grad_bias, workspace, workspace_bytes, stream);
}

// The edge chunk of the multi-head dense propagation entry points: E
// [cb, N, N] fp32, then the winning head of every pair [cb, N, N] u8.
struct DenseHeadChunk {
  float* E;
  uint8_t* heads;
  size_t bytes;
};
static DenseHeadChunk carve_dense_head_chunk(void* base, size_t size, int64_t cb, int64_t N) {
  Workspace ws(base, size);
  DenseHeadChunk c{};
  c.E = ws.take<float>(cb * N * N);
  c.heads = ws.take<uint8_t>(cb * N * N);
  c.bytes = ws.used;
  return c;
}

size_t jn_propagation_dense_multihead_chunk_bytes(int64_t batch, int64_t nodes, int64_t chunk_batch) {
  if (batch < 1 || nodes < 1 || chunk_batch < 1) return 0;
  return carve_dense_head_chunk(nullptr, 0, chunk_batch < batch ? chunk_batch : batch, nodes).bytes;
}

size_t jn_propagation_dense_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                      int64_t rank, int64_t heads, int32_t compress_kind,
                                                      int64_t chunk_batch) {
  (void)out_dim;
  if (batch < 1 || nodes < 1 || rank < 1 || heads < 1 || chunk_batch < 1) return 0;
  const int64_t cb = chunk_batch < batch ? chunk_batch : batch;
  return carve_dense(nullptr, 0, batch, nodes, in_dim, rank * heads, compress_kind == 0 ? 0 : cb, 0, heads).bytes;
}

int jn_propagation_dense_forward_multihead(const float* layer_val, const float* projected_state,
                                           const float* projected_val, const float* target_weight,
                                           const float* source_weight, const float* core_weight, const float* bias,
                                           int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                           int64_t rank, int64_t heads, int32_t compress_kind, int32_t causal,
                                           int64_t chunk_batch, float* delta_state, float* delta_val,
                                           float* projections, void* edge_chunk, size_t edge_chunk_bytes,
                                           jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank * heads, compress_kind);
  if (rc) return rc;
  JN_REQUIRE(layer_val && projected_state && projected_val && target_weight && source_weight && core_weight &&
                 delta_state && delta_val && projections && edge_chunk,
             kInvalidArgument, "null tensor pointer");
  JN_REQUIRE(chunk_batch >= 1, kInvalidArgument, "chunk_batch must be positive");
  const int B = (int)batch, N = (int)nodes, R = (int)(rank * heads), D = (int)out_dim;
  const int cb = (int)(chunk_batch < batch ? chunk_batch : batch);
  const DenseHeadChunk ch = carve_dense_head_chunk(edge_chunk, edge_chunk_bytes, cb, N);
  JN_REQUIRE(ch.bytes <= edge_chunk_bytes, kWorkspaceTooSmall, "edge chunk too small: need %zu bytes, got %zu",
             ch.bytes, edge_chunk_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = gemm_project(layer_val, in_dim, target_weight, source_weight, R, in_dim, projections, 2 * R, B * N, 2 * R,
                    (int)in_dim, st);
  if (rc) return rc;
  for (int b0 = 0; b0 < B; b0 += cb) {
    rc = dense_forward_range(projected_state, projected_val, core_weight, bias, b0, std::min(cb, B - b0), N, D, R,
                             compress_kind, causal != 0, projections, ch.E, delta_state, delta_val, st, (int)heads,
                             ch.heads);
    if (rc) return rc;
  }
  return kOk;
}

int jn_propagation_dense_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, const float* projections,
    void* edge_chunk, size_t edge_chunk_bytes, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads,
    int32_t compress_kind, int32_t causal, int32_t projected_val_is_layer_val, int64_t chunk_batch,
    int32_t chunk_resident, float* grad_layer_val, float* grad_projected_state, float* grad_projected_val,
    float* grad_target_weight, float* grad_source_weight, float* grad_core_weight, float* grad_bias,
    void* workspace, size_t workspace_bytes, jn_stream_t stream) {
  int rc = check_heads(rank, heads);
  if (rc) return rc;
  rc = check_dense_shapes(batch, nodes, in_dim, out_dim, rank * heads, compress_kind);
  if (rc) return rc;
  JN_REQUIRE(chunk_batch >= 1, kInvalidArgument, "chunk_batch must be positive");
  JN_REQUIRE(edge_chunk, kInvalidArgument, "null tensor pointer");
  const int cb = (int)(chunk_batch < batch ? chunk_batch : batch);
  const DenseHeadChunk ch = carve_dense_head_chunk(edge_chunk, edge_chunk_bytes, cb, nodes);
  JN_REQUIRE(ch.bytes <= edge_chunk_bytes, kWorkspaceTooSmall, "edge chunk too small: need %zu bytes, got %zu",
             ch.bytes, edge_chunk_bytes);
  const int64_t R = rank * heads;
  DenseScratch s = carve_dense(workspace, workspace_bytes, batch, nodes, in_dim, R, compress_kind == 0 ? 0 : cb, 0,
                               heads);
  JN_REQUIRE(workspace != nullptr && s.bytes <= workspace_bytes, kWorkspaceTooSmall,
             "workspace too small: need %zu bytes, got %zu", s.bytes, workspace_bytes);
  return dense_backward(layer_val, projected_state, projected_val, target_weight, source_weight, core_weight, bias,
                        projections, ch.E, compress_kind == 0 ? ch.E : s.G, cb, true, chunk_resident != 0,
                        grad_delta_state, grad_delta_val, batch, nodes, in_dim, out_dim, R, compress_kind, causal,
                        projected_val_is_layer_val, grad_layer_val, grad_projected_state, grad_projected_val,
                        grad_target_weight, grad_source_weight, grad_core_weight, grad_bias, s,
                        static_cast<hipStream_t>(stream), (int)heads, ch.heads);
}

}  // extern "C"
