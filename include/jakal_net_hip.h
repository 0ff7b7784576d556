/*
 * jakal_net_hip.h -- C ABI of the MI355X (gfx950) Jakal-Net native hot path.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer to
 * a contiguous row-major float32 / int32 buffer on the current HIP device, and
 * `stream` is a hipStream_t (passed as void*).  Calls are asynchronous on
 * `stream`; none allocates device memory (scratch comes in through
 * `workspace`, sized by the matching *_workspace_bytes query).  Edge-list
 * backward passes, top-k forwards that build an edge layout, and top-k
 * transitions on at least 2^18 edges run part of their work on a
 * library-owned side stream (one per host thread and device,
 * created on first use outside graph capture), forked from and joined back to
 * `stream` by events inside the call: work ordered after the call on `stream`
 * sees all of its results.
 *
 * Every entry point returns 0 on success and a non-zero jn status on error;
 * jn_last_error() then holds a message for the calling host thread.
 *
 * Index conventions: B = flattened batch, N = nodes, r = rank, k = top-k.
 * Ranks: single-head entry points take 1 <= r <= 1024 (the reference's
 * composites take any rank, native/jakal_net_native.cpp:714-832); the
 * multi-head ones at most 128 ranks over all heads.
 * "projections" is one [B*N, 2r] buffer: columns [0, r) hold the target
 * projection layer_val . U^T, columns [r, 2r) the unscaled source projection
 * layer_val . V^T (U = target_proj.weight, V = source_proj.weight).
 */
#ifndef JAKAL_NET_HIP_H
#define JAKAL_NET_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* jn_stream_t;

/* Message of the last failing call on this host thread ("" if none). */
const char* jn_last_error(void);

/* ABI revision of this header (bumped on any signature or accepted-range change); this is 15. */
int jn_abi_version(void);

/*
 * Per-kernel timing (no counterpart in the reference; for benchmarks).
 * jn_profile_enable(1) makes every later launch record a HIP event pair on
 * its stream; jn_profile_collect() waits for the recorded events and writes
 * one "kernel_name launches total_ms" line per kernel into `buffer`, then
 * clears the records.  jn_profile_enable(0) stops recording.
 */
int jn_profile_enable(int32_t on);
int jn_profile_collect(char* buffer, size_t size);

/*
 * GEMM tiling control (no counterpart in the reference; for tests and tuning).
 * tile = 64 or 128 forces that square workgroup tile on every later dense
 * product (projections, their gradients, the dense-mode score, aggregation and
 * gradient products); 32 forces the 32 x 32 tile on the projection products
 * and their gradients (64 elsewhere); 0 (the default) picks per call: 128 when
 * both output extents are >= 128 and the grid still has >= 256 workgroups,
 * else 64, or 32 for the projection products when a 64 x 64 grid has fewer
 * than 256 workgroups.  Process-wide; results are the same up to fp32
 * summation order.
 */
int jn_set_gemm_tile(int32_t tile);

/*
 * Window kernels (no counterpart in the reference; for tests and tuning).
 * mode 0 (the default) runs a window edge list's aggregation, value-row dot
 * products and value gradient as MFMA tiles over each 64-row tile's span of
 * the causal band whenever the band is at most 128 wide and the value rows
 * are whole, aligned 16-byte packs; mode 1 runs the per-edge gather kernels
 * for every window.  Process-wide; results agree up to fp32 summation order.
 */
int jn_set_window_kernels(int32_t mode);

/*
 * Side streams (no counterpart in the reference; for measurement and tests).
 * on = 1 (the default) lets the edge-list entry points run independent work on
 * the library's side stream beside the caller's (see the top of this file);
 * on = 0 runs every kernel on the caller's stream in the same order, so each
 * kernel can be timed alone.  Process-wide; results are bit-identical.
 */
int jn_set_side_streams(int32_t on);

/*
 * Score arithmetic of the top-k select (no counterpart in the reference; for
 * tests and tuning).  mode 0 (the default) computes the low-rank score tiles
 * on fp16 MFMAs over two-term fp16 splits of the operands: every operand is
 * scaled by a power of two and written as hi + lo (22 significant bits), and
 * a score is hi.hi + hi.lo + lo.hi accumulated in fp32, within about
 * 3 * 2^-22 * sum_r |q_r k_r| of the exact value (fp32 accumulation itself is
 * within r * 2^-24 of it).  mode 1 computes them on fp32 MFMAs.  Modes 2, 4
 * and 5 are mode 0 on one kernel only: 2 the per-wave streaming kernel, 4 the
 * cooperative kernel (key chunks staged once per 4-wave workgroup in LDS,
 * two workgroups per CU) whenever rank <= 64, 5 a key-split per-wave kernel
 * (the four waves of a workgroup share 16 query rows, each over a quarter of
 * the keys) whenever k <= 16.  Mode 0 picks the cooperative kernel for
 * rank <= 64 when the grid has at least 512 of its 64-row workgroups, the
 * key-split kernel for k <= 16 on grids below 256 of them with >= 192 keys,
 * else the per-wave kernel; rows of at most 1024 keys (one head, fp32
 * operands, k <= 64) it runs on the small-key select instead, which scores
 * each workgroup's 16 rows against every key on fp32 MFMAs into LDS and
 * radix-selects each row (mode 1's arithmetic).  Mode 6 is mode 0 without the
 * small-key select.  All pick the same entries.  Mode 3 is retired
 * (rejected).  The *_workspace_bytes queries report the split workspace in
 * every mode, so a size query and a later launch agree whatever mode another
 * thread sets in between.  Process-wide (atomic); each launch reads it once.
 */
int jn_set_select_mode(int32_t mode);

/*
 * Low-rank score + per-row top-k select, no score matrix materialised.
 *   s[b,i,j] = ((sum_r query[b,i,r]*cq[r] * key[b,j,r]*ck[r]) + bias) / temperature
 * where the scale vector multiplies the query rows when scale_on_query != 0,
 * else the key rows.  Writes the k best (j, s) per row, sorted descending,
 * ties toward the lower j.  1 <= k <= 4096, k <= nk, rank >= 1 (past 128 ranks
 * the select scores rows in its workspace).
 * Replaces the score/select stage of
 *   propagation_topk            (native/jakal_net_native.cpp:6399-6424)
 *   low_rank_propagation_topk_forward_cuda (native/jakal_net_native_cuda.cu:1028-1110)
 *   low_rank_pairwise_topk_forward_cuda    (native/jakal_net_native_cuda.cu:739-813)
 */
int jn_lowrank_topk_select(const float* query, int64_t ldq, int64_t query_batch_stride, const float* key,
                           int64_t ldk, int64_t key_batch_stride, const float* scale, int32_t scale_on_query,
                           const float* bias, float temperature, int64_t batch, int64_t nq, int64_t nk,
                           int64_t rank, int64_t topk, int32_t* out_index, float* out_score, void* workspace,
                           size_t workspace_bytes, jn_stream_t stream);

/* Workspace of jn_lowrank_topk_select (split key rows; unused in select mode 1). */
size_t jn_lowrank_topk_select_workspace_bytes(int64_t batch, int64_t nk, int64_t rank);

/*
 * SparsePropagation(sparse_type="topk", LowRankBilinearPairwise) forward.
 *   layer_val [B,N,Din], projected_state [B,N], projected_val [B,N,Dout],
 *   target_weight U [r,Din], source_weight V [r,Din], core_weight w_hat [r]
 *   (already normalised, kernel_common.py:185-192), bias scalar or NULL.
 * Outputs delta_state [B,N], delta_val [B,N,Dout] and, for the backward,
 * projections [B*N,2r], topk_index [B,N,k] (int32), topk_score [B,N,k].
 * compress_kind: 0 softsign, 1 signed_abs_softmax (sign(s) * softmax(|s|) over the
 * row's k edges), 2 signed_entmax15 (sign(s) * entmax15(|s|) over them,
 * native/jakal_net_native.cpp:1133-1205), for rows of any length.
 * edge_layout (NULL, or jn_propagation_topk_layout_bytes(batch, nodes, topk)
 * bytes): the forward also groups the selected edges by key for the backward,
 * beside its row pass; pass the same buffer, unchanged, to the backward.
 * Replaces propagation_topk (native/jakal_net_native.cpp:6305-6447) and
 * low_rank_propagation_topk_forward_cuda (native/jakal_net_native.cpp:191-213).
 */
int jn_propagation_topk_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                const float* target_weight, const float* source_weight, const float* core_weight,
                                const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                int64_t rank, int64_t topk, int32_t compress_kind, float* delta_state,
                                float* delta_val, float* projections, int32_t* topk_index, float* topk_score,
                                void* edge_layout, size_t edge_layout_bytes, void* workspace,
                                size_t workspace_bytes, jn_stream_t stream);

/*
 * Size of the edge layout the top-k forwards build for their backward (no
 * counterpart in the reference, whose backward regroups the edges itself):
 * the edges grouped by key (segment starts, 16-byte records), each edge's
 * record index, and the build's scratch.
 */
size_t jn_propagation_topk_layout_bytes(int64_t batch, int64_t nodes, int64_t topk);

/* Workspace of jn_propagation_topk_forward (the select's; unused in select mode 1). */
size_t jn_propagation_topk_forward_workspace_bytes(int64_t batch, int64_t nodes, int64_t rank);

/*
 * jn_propagation_topk_forward without workspace and edge-layout arguments
 * (no layout is built): it allocates
 * nothing and takes its scratch from a static device array of
 * jn_static_scratch_bytes() bytes (48 MiB) held by each GPU the library runs
 * on.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * jn_propagation_topk_forward; a shape whose select scratch
 * (jn_propagation_topk_forward_workspace_bytes) exceeds the array is rejected
 * with kUnsupported before anything is launched.  Calls that overlap on one
 * GPU (other streams or host threads) share the array and race on it.
 */
int jn_propagation_topk_forward_static(const float* layer_val, const float* projected_state,
                                       const float* projected_val, const float* target_weight,
                                       const float* source_weight, const float* core_weight, const float* bias,
                                       int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                       int64_t topk, int32_t compress_kind, float* delta_state, float* delta_val,
                                       float* projections, int32_t* topk_index, float* topk_score,
                                       jn_stream_t stream);

/* Size in bytes of the static scratch array of jn_propagation_topk_forward_static. */
size_t jn_static_scratch_bytes(void);

/* Workspace needed by jn_propagation_topk_backward. */
size_t jn_propagation_topk_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                           int64_t rank, int64_t topk);

/*
 * Backward of jn_propagation_topk_forward given grad_delta_state [B,N] and
 * grad_delta_val [B,N,Dout].  Output pointers may be NULL to skip a gradient.
 * When projected_val_is_layer_val != 0 (identity val_proj_fn) the value
 * gradient is folded into grad_layer_val and grad_projected_val is unused.
 * grad_core_weight is the gradient wrt w_hat; grad_bias a single float.
 * edge_layout: the buffer the forward filled for this edge list, or NULL (the
 * backward then groups the edges itself, in its workspace).
 * Deterministic: no floating-point atomics.
 * Replaces _LowRankPropagationTopK.backward (src/jakal_net/native_backend.py:4872-4964):
 * query_topk_reduce_backward_cuda, softsign_backward_cuda and
 * low_rank_pairwise_topk_backward_cuda (native/jakal_net_native.cpp:152-165, 398-416, 449-477).
 */
int jn_propagation_topk_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                 const float* target_weight, const float* source_weight, const float* core_weight,
                                 const float* projections, const int32_t* topk_index, const float* topk_score,
                                 const float* grad_delta_state, const float* grad_delta_val, int64_t batch,
                                 int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t topk,
                                 int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val,
                                 float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                 float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                 const void* edge_layout, void* workspace, size_t workspace_bytes,
                                 jn_stream_t stream);

/*
 * SparsePropagation(sparse_type="window", LowRankBilinearPairwise) forward.
 * Row i aggregates the sources j with i - window <= j <= i: its
 * width = min(window + 1, nodes) edge slots hold j = i - (width - 1 - e) for
 * slot e, index -1 (absent) where j < 0.  Arguments as
 * jn_propagation_topk_forward; edge_index [B,N,width] (int32) and
 * edge_score [B,N,width] receive the edge list for the backward.
 * signed_abs_softmax and signed_entmax15 (compress_kind 1, 2) need width <= 64.
 * Replaces propagation_window (native/jakal_net_native.cpp:6190-6303) and
 * low_rank_propagation_window_forward_cuda (native/jakal_net_native.cpp:268-288).
 */
int jn_propagation_window_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                  const float* target_weight, const float* source_weight, const float* core_weight,
                                  const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                  int64_t rank, int64_t window, int32_t compress_kind, float* delta_state,
                                  float* delta_val, float* projections, int32_t* edge_index, float* edge_score,
                                  jn_stream_t stream);

/* Workspace needed by jn_propagation_window_backward. */
size_t jn_propagation_window_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                             int64_t rank, int64_t window);

/*
 * Backward of jn_propagation_window_forward; arguments as
 * jn_propagation_topk_backward with the window edge list.
 * Replaces _LowRankPropagationWindow.backward (src/jakal_net/native_backend.py:5143-5356).
 */
int jn_propagation_window_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                   const float* target_weight, const float* source_weight, const float* core_weight,
                                   const float* projections, const int32_t* edge_index, const float* edge_score,
                                   const float* grad_delta_state, const float* grad_delta_val, int64_t batch,
                                   int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t window,
                                   int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val,
                                   float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                   float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                   void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Propagation (dense, every target row aggregates every source) with
 * LowRankBilinearPairwise:  s = P_t diag(w_hat) P_s^T + b,  e = softsign(s)
 * (compress_kind 0), sign(s) * softmax(|s|) over the row (1) or
 * sign(s) * entmax15(|s|) over the row (2),
 * delta_state = e . ps, delta_val = e . pv.  Arguments as
 * jn_propagation_topk_forward; `edges` [B,N,N] (fp32, caller-allocated)
 * receives e for the backward.  The two N x N contractions run as batched
 * MFMA GEMMs over the materialised edge matrix.
 * Replaces propagation_dense (native/jakal_net_native.cpp:5962-6076) for
 * source_state = None (the caller folds state weighting into ps and pv,
 * propagation.py:162-170).  causal != 0 keeps only sources j <= i in row i
 * (softmax of the signed variant over those): the full causal window that
 * propagation_window computes for window >= N - 1 (kernel_common.py:443-456;
 * the causal dense query propagation of scripts/progressive_b_example.py:
 * 1990-2003), on the same MFMA path.
 */
int jn_propagation_dense_forward(const float* layer_val, const float* projected_state, const float* projected_val,
                                 const float* target_weight, const float* source_weight, const float* core_weight,
                                 const float* bias, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                 int64_t rank, int32_t compress_kind, int32_t causal, float* delta_state,
                                 float* delta_val, float* projections, float* edges, jn_stream_t stream);

/*
 * Workspace needed by jn_propagation_dense_backward: one [B,N,N] matrix for
 * the score gradient, except for softsign (compress_kind 0) with
 * reuse_edges != 0, where that gradient overwrites the edge matrix (a few MB
 * of row partials and projection gradients remain).
 */
size_t jn_propagation_dense_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                            int64_t rank, int32_t compress_kind, int32_t reuse_edges);

/*
 * Backward of jn_propagation_dense_forward; arguments as
 * jn_propagation_topk_backward with the edge matrix in place of the edge list.
 * reuse_edges != 0 lets a softsign backward write the score gradient over
 * `edges` (the edge matrix is then consumed: a second backward needs the
 * forward again); otherwise `edges` is only read.  In causal mode the
 * products over the edge matrix skip its zero upper triangle.
 * The reference differentiates its composite dense op with autograd
 * (native/jakal_net_native.cpp:5962-6076 has no custom backward).
 */
int jn_propagation_dense_backward(const float* layer_val, const float* projected_state, const float* projected_val,
                                  const float* target_weight, const float* source_weight, const float* core_weight,
                                  const float* projections, float* edges, const float* grad_delta_state,
                                  const float* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim,
                                  int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
                                  int32_t projected_val_is_layer_val, int32_t reuse_edges, float* grad_layer_val,
                                  float* grad_projected_state, float* grad_projected_val, float* grad_target_weight,
                                  float* grad_source_weight, float* grad_core_weight, float* grad_bias,
                                  void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Dense propagation in batch chunks (same reference function and outputs as
 * jn_propagation_dense_forward / _backward): the edge matrices of
 * chunk_batch batch elements at a time live in a chunk buffer at the start of
 * the forward's workspace (chunk_batch * N * N floats), which holds the last
 * chunk's edges when the forward returns.  The backward takes that buffer as
 * edge_chunk; chunk_resident != 0 says it still holds them (so the last
 * chunk is not rebuilt), and every other chunk's edges are rebuilt in it from
 * the saved projections exactly as the forward built them (a rank-r score
 * product).  A softsign backward writes its score gradient over the buffer.
 * The backward workspace (backward != 0 in the query) holds a score-gradient
 * chunk for the signed kinds and the row partials and projection gradients.
 */
size_t jn_propagation_dense_chunked_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                    int64_t rank, int32_t compress_kind, int64_t chunk_batch,
                                                    int32_t backward);
int jn_propagation_dense_forward_chunked(const float* layer_val, const float* projected_state,
                                         const float* projected_val, const float* target_weight,
                                         const float* source_weight, const float* core_weight, const float* bias,
                                         int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                         int32_t compress_kind, int32_t causal, int64_t chunk_batch,
                                         float* delta_state, float* delta_val, float* projections, void* workspace,
                                         size_t workspace_bytes, jn_stream_t stream);
int jn_propagation_dense_backward_chunked(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, const float* projections,
    float* edge_chunk, const float* grad_delta_state, const float* grad_delta_val, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
    int32_t projected_val_is_layer_val, int64_t chunk_batch, int32_t chunk_resident, float* grad_layer_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * SparseTransition with LowRankBilinearRoute (optionally temperature-scaled):
 *   l[j,d]  = ((P_s[j] * w) . P_t[d] + b) / temperature,  P_s = src_val Ws^T,
 *             P_t = dst_val Wt^T, w the raw core weight (modules.py:435-441)
 *   each source row j keeps its k = min(topk, dst_nodes) best destinations
 *   (transition.py:437-444); p = softmax over them (compress_kind 0),
 *   sign(l) * softmax(|l|) (compress_kind 1) or sign(l) * entmax15(|l|) (2)
 *   delta_state[d] = sum_j p[j,d] rho[j] projected_state[j]
 *   delta_val[d]   = sum_j p[j,d] rho[j] projected_val[j]
 * Shapes: sender_strength rho [B,Ns], src_val [B,Ns,Dsrc], dst_val [B,Nd,Ddst],
 * projected_state [B,Ns], projected_val [B,Ns,Dv], Ws [r,Dsrc], Wt [r,Ddst],
 * w [r], bias scalar or NULL.  Outputs delta_state [B,Nd], delta_val [B,Nd,Dv],
 * and for the backward src_proj [B*Ns,r], dst_proj [B*Nd,r], route_index
 * [B,Ns,k] (int32) and route_logit [B,Ns,k].  k <= 4096 when k < dst_nodes;
 * k == dst_nodes <= 64 takes every destination.  Deterministic (the
 * destination sums are gathers over the edges grouped by destination).
 * Replaces transition_pairwise_topk (native/jakal_net_native.cpp:6916-7087) and
 * low_rank_pairwise_topk_forward_cuda (native/jakal_net_native.cpp:167-189).
 */
size_t jn_transition_topk_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                          int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t topk);

int jn_transition_topk_forward(const float* sender_strength, const float* src_val, const float* dst_val,
                               const float* projected_state, const float* projected_val, const float* source_weight,
                               const float* target_weight, const float* core_weight, const float* bias,
                               float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                               int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t topk,
                               int32_t compress_kind, float* delta_state, float* delta_val, float* src_proj,
                               float* dst_proj, int32_t* route_index, float* route_logit, void* workspace,
                               size_t workspace_bytes, jn_stream_t stream);

/*
 * Backward of jn_transition_topk_forward given grad_delta_state [B,Nd] and
 * grad_delta_val [B,Nd,Dv].  Output pointers may be NULL to skip a gradient.
 * Replaces _LowRankTransitionPairwiseTopK.backward
 * (src/jakal_net/native_backend.py:4408-4599): softmax_backward_cuda and
 * low_rank_pairwise_topk_backward_cuda (native/jakal_net_native.cpp:398-416, 449-477).
 */
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
                                void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Dense pairwise transition: every source routes to every destination.
 *   l[b,j,k] = ((P_s[j] * w) . P_t[k] + bias) / temperature,
 *   P_s = src_val . Ws^T [B*Ns, r], P_t = dst_val . Wt^T [B*Nd, r];
 *   R[b,j,:] = compress(l[b,j,:]) over destinations: compress_kind 0 softmax,
 *   1 sign(l) * softmax(|l|), 2 sign(l) * entmax15(|l|);
 *   delta_state[b,k] = sum_j R[b,j,k] rho_j ps_j, delta_val[b,k] = sum_j R[b,j,k] rho_j pv_j.
 * Writes src_proj [B*Ns, r], dst_proj [B*Nd, r] and routes [B,Ns,Nd] (all
 * caller-allocated) for the backward.  Allocates nothing.
 * Replaces transition_pairwise_dense (native/jakal_net_native.cpp:6705-6914),
 * signature at :6705-6725, called from transition_pairwise_dense_native
 * (src/jakal_net/native_backend.py:5755-5822).
 */
int jn_transition_dense_forward(const float* sender_strength, const float* src_val, const float* dst_val,
                                const float* projected_state, const float* projected_val, const float* source_weight,
                                const float* target_weight, const float* core_weight, const float* bias,
                                float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                int32_t compress_kind, float* delta_state, float* delta_val, float* src_proj,
                                float* dst_proj, float* routes, jn_stream_t stream);

/* Workspace bytes jn_transition_dense_backward needs (0 on invalid sizes). */
size_t jn_transition_dense_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                           int64_t dst_dim, int64_t val_dim, int64_t rank);

/*
 * Backward of jn_transition_dense_forward given grad_delta_state [B,Nd] and
 * grad_delta_val [B,Nd,Dv]; src_proj, dst_proj and routes are the forward's.
 * Output pointers may be NULL to skip a gradient (grad_core_weight is always
 * written).  The reference differentiates its composite dense transition with
 * autograd (native/jakal_net_native.cpp:6745-6774 records ATen ops).
 */
int jn_transition_dense_backward(const float* sender_strength, const float* src_val, const float* dst_val,
                                 const float* projected_state, const float* projected_val, const float* source_weight,
                                 const float* target_weight, const float* core_weight, const float* src_proj,
                                 const float* dst_proj, const float* routes, const float* grad_delta_state,
                                 const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
                                 int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                 int32_t compress_kind, float* grad_sender_strength, float* grad_src_val,
                                 float* grad_dst_val, float* grad_projected_state, float* grad_projected_val,
                                 float* grad_source_weight, float* grad_target_weight, float* grad_core_weight,
                                 float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Multi-head max-aggregated scores (MultiHeadPairwise / MultiHeadRoute with
 * aggregate="max" over low-rank heads, src/jakal_net/modules.py:259-301,
 * 470-529).  H = heads (2..8) heads of rank r each score every pair; the pair's
 * score is the largest head score, max_h (dot_h + bias[h]) (/ T for routes),
 * and its gradient reaches only that head (the first winning head on exact
 * ties).  The heads' parameters come stacked as the reference's kernel spec
 * stacks them (kernel_common.py:152-178, 240-270): projection weights
 * [H, r, D] (= [H*r, D] row-major), core weights [H, r] (= [H*r]), bias [H] or
 * NULL.  Projections hold all H*r ranks, head h in columns [h*r, (h+1)*r):
 * projections [B*N, 2*H*r] for propagation, src_proj [B*Ns, H*r] and dst_proj
 * [B*Nd, H*r] for transitions.  The forward also writes each edge's winning
 * head (uint8, shaped like the edge index) for the backward.  Limits:
 * H*r <= 128, and where the edges come from a top-k select
 * H * ceil(r / 32) <= 4 (each head scores on whole 32-rank MFMA K-steps).
 * One head is the single-head entry point.  grad_core_weight is [H, r],
 * grad_bias [H]; other arguments as the single-head entry points.
 *
 * Replace the multi-head branches of pairwise_scores and route_scores
 * (native/jakal_net_native.cpp:724-752, 889-917) under propagation_topk,
 * propagation_window and transition_pairwise_topk, and the multi-head CUDA
 * forwards low_rank_propagation_topk_forward_multihead_kernel and
 * low_rank_pairwise_topk_forward_multihead_kernel
 * (native/jakal_net_native_cuda.cu:1185-1347, 880-1026), whose heads share one
 * bias; here each head keeps its own, as the composite's do.
 */
size_t jn_propagation_topk_forward_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t rank,
                                                             int64_t heads);
int jn_propagation_topk_forward_multihead(const float* layer_val, const float* projected_state,
                                          const float* projected_val, const float* target_weight,
                                          const float* source_weight, const float* core_weight, const float* bias,
                                          int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                          int64_t rank, int64_t heads, int64_t topk, int32_t compress_kind,
                                          float* delta_state, float* delta_val, float* projections,
                                          int32_t* topk_index, float* topk_score, uint8_t* topk_head,
                                          void* edge_layout, size_t edge_layout_bytes, void* workspace,
                                          size_t workspace_bytes, jn_stream_t stream);
size_t jn_propagation_topk_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                     int64_t rank, int64_t heads, int64_t topk);
int jn_propagation_topk_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* projections, const int32_t* topk_index,
    const float* topk_score, const uint8_t* topk_head, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads, int64_t topk,
    int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
    float* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, const void* edge_layout, void* workspace, size_t workspace_bytes, jn_stream_t stream);

int jn_propagation_window_forward_multihead(const float* layer_val, const float* projected_state,
                                            const float* projected_val, const float* target_weight,
                                            const float* source_weight, const float* core_weight, const float* bias,
                                            int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                            int64_t rank, int64_t heads, int64_t window, int32_t compress_kind,
                                            float* delta_state, float* delta_val, float* projections,
                                            int32_t* edge_index, float* edge_score, uint8_t* edge_head,
                                            jn_stream_t stream);
size_t jn_propagation_window_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim,
                                                       int64_t out_dim, int64_t rank, int64_t heads, int64_t window);
int jn_propagation_window_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* projections, const int32_t* edge_index,
    const float* edge_score, const uint8_t* edge_head, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads, int64_t window,
    int32_t compress_kind, int32_t projected_val_is_layer_val, float* grad_layer_val, float* grad_projected_state,
    float* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);

size_t jn_transition_topk_multihead_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                                    int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                                    int64_t heads, int64_t topk);
int jn_transition_topk_forward_multihead(const float* sender_strength, const float* src_val, const float* dst_val,
                                         const float* projected_state, const float* projected_val,
                                         const float* source_weight, const float* target_weight,
                                         const float* core_weight, const float* bias, float temperature,
                                         int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                         int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads, int64_t topk,
                                         int32_t compress_kind, float* delta_state, float* delta_val,
                                         float* src_proj, float* dst_proj, int32_t* route_index, float* route_logit,
                                         uint8_t* route_head, void* workspace, size_t workspace_bytes,
                                         jn_stream_t stream);
int jn_transition_topk_backward_multihead(
    const float* sender_strength, const float* src_val, const float* dst_val, const float* projected_state,
    const float* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const int32_t* route_index, const float* route_logit,
    const uint8_t* route_head, const float* grad_delta_state, const float* grad_delta_val, float temperature,
    int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
    int64_t rank, int64_t heads, int64_t topk, int32_t compress_kind, float* grad_sender_strength,
    float* grad_src_val, float* grad_dst_val, float* grad_projected_state, float* grad_projected_val,
    float* grad_source_weight, float* grad_target_weight, float* grad_core_weight, float* grad_bias,
    void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Max-aggregated multi-head scores on the dense paths: every pair's score is
 * max_h (P_t,h diag(w_h) P_s,h^T + b_h) (H heads of rank r stacked as in the
 * multi-head edge-list entry points; bias [H] or NULL), one fp32 MFMA score
 * GEMM per head folding into a running max whose epilogue records the first
 * head attaining it; the backward passes each pair's score gradient to that
 * head only (rank-r products on the gradient masked per head, per-head bias
 * sums).  H * r <= 128.
 *
 * Dense propagation: arguments as jn_propagation_dense_forward_chunked /
 * _backward_chunked with (rank, heads).  edge_chunk
 * (jn_propagation_dense_multihead_chunk_bytes) holds a chunk of chunk_batch
 * batch elements' edge matrices and winning heads; the forward leaves the
 * last chunk there (chunk_resident = 1 in the backward reuses it), the
 * backward rebuilds the other chunks from the projections.  A softsign
 * backward writes its score gradient over the chunk's edges.
 * Replace propagation_dense's multi-head branch (native/jakal_net_native.cpp:
 * 5962-6076 over pairwise_scores, 724-752).
 */
size_t jn_propagation_dense_multihead_chunk_bytes(int64_t batch, int64_t nodes, int64_t chunk_batch);
size_t jn_propagation_dense_multihead_workspace_bytes(int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                                      int64_t rank, int64_t heads, int32_t compress_kind,
                                                      int64_t chunk_batch);
int jn_propagation_dense_forward_multihead(const float* layer_val, const float* projected_state,
                                           const float* projected_val, const float* target_weight,
                                           const float* source_weight, const float* core_weight, const float* bias,
                                           int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                           int64_t rank, int64_t heads, int32_t compress_kind, int32_t causal,
                                           int64_t chunk_batch, float* delta_state, float* delta_val,
                                           float* projections, void* edge_chunk, size_t edge_chunk_bytes,
                                           jn_stream_t stream);
int jn_propagation_dense_backward_multihead(
    const float* layer_val, const float* projected_state, const float* projected_val, const float* target_weight,
    const float* source_weight, const float* core_weight, const float* bias, const float* projections,
    void* edge_chunk, size_t edge_chunk_bytes, const float* grad_delta_state, const float* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int64_t heads,
    int32_t compress_kind, int32_t causal, int32_t projected_val_is_layer_val, int64_t chunk_batch,
    int32_t chunk_resident, float* grad_layer_val, float* grad_projected_state, float* grad_projected_val,
    float* grad_target_weight, float* grad_source_weight, float* grad_core_weight, float* grad_bias,
    void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Dense transitions with max-aggregated multi-head route logits: arguments
 * as jn_transition_dense_forward / _backward with (rank, heads), plus
 * route_heads [B, Ns, Nd] (uint8), the winning head of every route, which the
 * forward writes and the backward reads.
 * Replace transition_pairwise_dense's multi-head branch
 * (native/jakal_net_native.cpp:6705-6914 over route_scores, 889-917).
 */
int jn_transition_dense_forward_multihead(const float* sender_strength, const float* src_val, const float* dst_val,
                                          const float* projected_state, const float* projected_val,
                                          const float* source_weight, const float* target_weight,
                                          const float* core_weight, const float* bias, float temperature,
                                          int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t src_dim,
                                          int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
                                          int32_t compress_kind, float* delta_state, float* delta_val,
                                          float* src_proj, float* dst_proj, float* routes, uint8_t* route_heads,
                                          jn_stream_t stream);
size_t jn_transition_dense_multihead_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes,
                                                     int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
                                                     int64_t heads);
int jn_transition_dense_backward_multihead(
    const float* sender_strength, const float* src_val, const float* dst_val, const float* projected_state,
    const float* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const float* routes, const uint8_t* route_heads,
    const float* grad_delta_state, const float* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes,
    int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int64_t heads,
    int32_t compress_kind, float* grad_sender_strength, float* grad_src_val, float* grad_dst_val,
    float* grad_projected_state, float* grad_projected_val, float* grad_source_weight, float* grad_target_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * bf16 layers (layer values under autocast, src/jakal_net/modules.py:95-97;
 * bf16/fp16 score operands of native/jakal_net_native_cuda.cu:2492-2497).
 * The uint16_t tensors hold bf16 bit patterns: layer_val, projected_val and
 * delta_val, and in the backward grad_delta_val, grad_layer_val and
 * grad_projected_val (src_val, dst_val and their gradients for transitions).
 * States, weights, projections, edge lists and their gradients stay fp32.
 * Every value row the gathers move is bf16 (half the bytes of the fp32 entry
 * points); projections accumulate bf16 x fp32 products in fp32; top-k scores
 * are bf16(q * core_weight) . bf16(key) accumulated in fp32 on
 * v_mfma_f32_16x16x32_bf16; sums accumulate in fp32 and round to bf16 once
 * per stored element.  Workspaces, limits and the other arguments are those of
 * the fp32 entry point of the same name.
 */
int jn_propagation_topk_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                     const uint16_t* projected_val, const float* target_weight,
                                     const float* source_weight, const float* core_weight, const float* bias,
                                     int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                     int64_t topk, int32_t compress_kind, float* delta_state, uint16_t* delta_val,
                                     float* projections, int32_t* topk_index, float* topk_score, void* edge_layout,
                                     size_t edge_layout_bytes, void* workspace, size_t workspace_bytes,
                                     jn_stream_t stream);
int jn_propagation_topk_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    const int32_t* topk_index, const float* topk_score, const float* grad_delta_state,
    const uint16_t* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
    int64_t topk, int32_t compress_kind, int32_t projected_val_is_layer_val, uint16_t* grad_layer_val,
    float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, const void* edge_layout, void* workspace, size_t workspace_bytes,
    jn_stream_t stream);
int jn_propagation_window_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                       const uint16_t* projected_val, const float* target_weight,
                                       const float* source_weight, const float* core_weight, const float* bias,
                                       int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                       int64_t window, int32_t compress_kind, float* delta_state,
                                       uint16_t* delta_val, float* projections, int32_t* edge_index,
                                       float* edge_score, jn_stream_t stream);
int jn_propagation_window_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    const int32_t* edge_index, const float* edge_score, const float* grad_delta_state,
    const uint16_t* grad_delta_val, int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
    int64_t window, int32_t compress_kind, int32_t projected_val_is_layer_val, uint16_t* grad_layer_val,
    float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight,
    float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);
int jn_transition_topk_forward_bf16(const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val,
                                    const float* projected_state, const uint16_t* projected_val,
                                    const float* source_weight, const float* target_weight, const float* core_weight,
                                    const float* bias, float temperature, int64_t batch, int64_t src_nodes,
                                    int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
                                    int64_t rank, int64_t topk, int32_t compress_kind, float* delta_state,
                                    uint16_t* delta_val, float* src_proj, float* dst_proj, int32_t* route_index,
                                    float* route_logit, void* workspace, size_t workspace_bytes, jn_stream_t stream);
int jn_transition_topk_backward_bf16(
    const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val, const float* projected_state,
    const uint16_t* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const int32_t* route_index, const float* route_logit,
    const float* grad_delta_state, const uint16_t* grad_delta_val, float temperature, int64_t batch,
    int64_t src_nodes, int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank,
    int64_t topk, int32_t compress_kind, float* grad_sender_strength, uint16_t* grad_src_val,
    uint16_t* grad_dst_val, float* grad_projected_state, uint16_t* grad_projected_val, float* grad_source_weight,
    float* grad_target_weight, float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
    jn_stream_t stream);

/*
 * bf16 dense layers (one head): jn_propagation_dense_* with bf16 value
 * tensors, as above.  The edge matrix, the score gradient and the workspaces
 * stay fp32 (the fp32 entry points' workspace queries apply).  E . pv and
 * E^T . gdv take E rounded to bf16 (nearest even), gdv . pv^T multiplies the
 * bf16 rows exactly; all three accumulate in fp32 on
 * v_mfma_f32_16x16x32_bf16, and the score-gradient product keeps softsign's
 * derivative in its epilogue.  nodes and out_dim must be at least 128 and
 * multiples of 8 (kUnsupported otherwise: the fp32 entry points take any
 * shape).
 */
int jn_propagation_dense_forward_bf16(const uint16_t* layer_val, const float* projected_state,
                                      const uint16_t* projected_val, const float* target_weight,
                                      const float* source_weight, const float* core_weight, const float* bias,
                                      int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank,
                                      int32_t compress_kind, int32_t causal, float* delta_state, uint16_t* delta_val,
                                      float* projections, float* edges, jn_stream_t stream);
int jn_propagation_dense_backward_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* projections,
    float* edges, const float* grad_delta_state, const uint16_t* grad_delta_val, int64_t batch, int64_t nodes,
    int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind, int32_t causal,
    int32_t projected_val_is_layer_val, int32_t reuse_edges, uint16_t* grad_layer_val, float* grad_projected_state,
    uint16_t* grad_projected_val, float* grad_target_weight, float* grad_source_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);
int jn_propagation_dense_forward_chunked_bf16(const uint16_t* layer_val, const float* projected_state,
                                              const uint16_t* projected_val, const float* target_weight,
                                              const float* source_weight, const float* core_weight, const float* bias,
                                              int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim,
                                              int64_t rank, int32_t compress_kind, int32_t causal,
                                              int64_t chunk_batch, float* delta_state, uint16_t* delta_val,
                                              float* projections, void* workspace, size_t workspace_bytes,
                                              jn_stream_t stream);
int jn_propagation_dense_backward_chunked_bf16(
    const uint16_t* layer_val, const float* projected_state, const uint16_t* projected_val,
    const float* target_weight, const float* source_weight, const float* core_weight, const float* bias,
    const float* projections, float* edge_chunk, const float* grad_delta_state, const uint16_t* grad_delta_val,
    int64_t batch, int64_t nodes, int64_t in_dim, int64_t out_dim, int64_t rank, int32_t compress_kind,
    int32_t causal, int32_t projected_val_is_layer_val, int64_t chunk_batch, int32_t chunk_resident,
    uint16_t* grad_layer_val, float* grad_projected_state, uint16_t* grad_projected_val, float* grad_target_weight,
    float* grad_source_weight, float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
    jn_stream_t stream);

/*
 * bf16 dense transitions (one head): jn_transition_dense_* with bf16 value
 * tensors (src_val, dst_val, projected_val, delta_val and their gradients),
 * the other arguments and the workspace query as for fp32.  The route matrix
 * stays fp32: R^T diag(rho) pv takes R rho rounded to bf16, diag(rho) R gdv
 * takes R rounded to bf16, pv . gdv^T multiplies the bf16 rows exactly; all
 * accumulate in fp32 on v_mfma_f32_16x16x32_bf16.  src_nodes, dst_nodes and
 * val_dim must be at least 128 and multiples of 8 (kUnsupported otherwise).
 */
int jn_transition_dense_forward_bf16(const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val,
                                     const float* projected_state, const uint16_t* projected_val,
                                     const float* source_weight, const float* target_weight, const float* core_weight,
                                     const float* bias, float temperature, int64_t batch, int64_t src_nodes,
                                     int64_t dst_nodes, int64_t src_dim, int64_t dst_dim, int64_t val_dim,
                                     int64_t rank, int32_t compress_kind, float* delta_state, uint16_t* delta_val,
                                     float* src_proj, float* dst_proj, float* routes, jn_stream_t stream);
int jn_transition_dense_backward_bf16(
    const float* sender_strength, const uint16_t* src_val, const uint16_t* dst_val, const float* projected_state,
    const uint16_t* projected_val, const float* source_weight, const float* target_weight, const float* core_weight,
    const float* src_proj, const float* dst_proj, const float* routes, const float* grad_delta_state,
    const uint16_t* grad_delta_val, float temperature, int64_t batch, int64_t src_nodes, int64_t dst_nodes,
    int64_t src_dim, int64_t dst_dim, int64_t val_dim, int64_t rank, int32_t compress_kind,
    float* grad_sender_strength, uint16_t* grad_src_val, uint16_t* grad_dst_val, float* grad_projected_state,
    uint16_t* grad_projected_val, float* grad_source_weight, float* grad_target_weight, float* grad_core_weight,
    float* grad_bias, void* workspace, size_t workspace_bytes, jn_stream_t stream);

/*
 * Score scale vector of the low-rank pairwise scores: weight_hat[h] =
 * weight[h] / max(||weight[h]||_2, eps) for each of `rows` rows of `rank`
 * (LowRankBilinearPairwise.normalized_weight, modules.py:85-87; one row per
 * head for stacked heads), and the gradient of that map.  No counterpart in
 * the reference's native extension, whose callers compute it with a chain of
 * PyTorch ops (kernel_common.py:182, 188, 196); one kernel each here.
 */
int jn_unit_scale_forward(const float* weight, int64_t rows, int64_t rank, float eps, float* weight_hat,
                          jn_stream_t stream);
int jn_unit_scale_backward(const float* weight, const float* grad_weight_hat, int64_t rows, int64_t rank, float eps,
                           float* grad_weight, jn_stream_t stream);

/* ---------------------------------------------------------------------------
 * Raw edge ops: the reference extension's *_cuda ops that its Python
 * dispatcher composes into its own autograd functions
 * (src/jakal_net/native_backend.py:4408-4600 _LowRankTransitionPairwiseTopK,
 * 4002-4134 _LowRankPropagationQueryTopK; availability probes 657-667 and
 * 5962-5975).  Sums over a node's incoming edges walk the edges grouped by
 * that node (fixed order): results repeat bit for bit, where the reference
 * scatters with float atomics.  Index arrays are int32 ([B, rows, k],
 * batch-local, -1 = absent edge).
 * ------------------------------------------------------------------------- */

/*
 * Per-row top-k of max_h (query_h[b,i] . key_h[b,j] + bias[h]) over `heads`
 * heads of rank head_rank (heads == 1: one dot product), sorted descending,
 * ties toward the lower j; 1 <= k <= nk (k == nk keeps every key in score
 * order).  query [B, nq, heads*head_rank], key [B, nk, heads*head_rank] with
 * head h in ranks [h*head_rank, (h+1)*head_rank); bias [heads] or NULL.
 * Replaces the select of low_rank_pairwise_topk_forward_cuda
 * (native/jakal_net_native_cuda.cu:740-813, multi-head 881-930: [B, H, N, r]
 * operands, which the caller lays out heads-innermost) and of
 * low_rank_propagation_topk_forward_cuda (cu:1029-1065).
 */
int jn_lowrank_topk_select_heads(const float* query, const float* key, const float* bias, int64_t batch, int64_t nq,
                                 int64_t nk, int64_t head_rank, int64_t heads, int64_t topk, int32_t* out_index,
                                 float* out_score, void* workspace, size_t workspace_bytes, jn_stream_t stream);
size_t jn_lowrank_topk_select_heads_workspace_bytes(int64_t batch, int64_t nk, int64_t head_rank, int64_t heads);

/*
 * grad_scores = grad_edges / (1 + |scores|)^2 over `count` elements.
 * Replaces softsign_backward_cuda (native/jakal_net_native.cpp:398-405,
 * native/jakal_net_native_cuda.cu:2177-2190).
 */
int jn_softsign_backward(const float* scores, const float* grad_edges, int64_t count, float* grad_scores,
                         jn_stream_t stream);

/*
 * Softmax backward over rows of k: grad_scores = p * (g - sum_e p g).
 * Replaces softmax_backward_cuda (native/jakal_net_native.cpp:407-414,
 * native/jakal_net_native_cuda.cu:2192-2212).
 */
int jn_softmax_backward(const float* routes, const float* grad_routes, int64_t rows, int64_t k, float* grad_scores,
                        jn_stream_t stream);

/*
 * delta_state[b,i] = sum_e c[b,i,e] ps[b,j]; delta_val[b,i] = sum_e c[b,i,e] pv[b,j],
 * j = edge_index[b,i,e], c = compress(edge_score) per row: 0 softsign,
 * 1 signed |s| softmax, 2 signed entmax-1.5, 3 the scores are the
 * coefficients.  projected_state [B, source_nodes], projected_val
 * [B, source_nodes, dim].
 * Replaces query_topk_reduce_cuda (native/jakal_net_native.cpp:140-150,
 * kind 3) and the edge sums of low_rank_propagation_topk_forward_cuda
 * (native/jakal_net_native_cuda.cu:1084-1175, kinds 0-2).
 */
int jn_edge_aggregate(const int32_t* edge_index, const float* edge_score, int64_t batch, int64_t query_nodes,
                      int64_t source_nodes, int64_t edges, int64_t dim, int32_t compress_kind,
                      const float* projected_state, const float* projected_val, float* delta_state,
                      float* delta_val, jn_stream_t stream);

/*
 * Backward of jn_edge_aggregate with given coefficients (edge_weight):
 *   grad_edge_weight[b,i,e] = gds[b,i] ps[b,j] + <gdv[b,i], pv[b,j]>
 *   grad_projected_state[b,j] = sum over edges into j of edge_weight * gds[b,i]
 *   grad_projected_val[b,j]   = sum over edges into j of edge_weight * gdv[b,i]
 * Any of the three outputs may be NULL (not computed).  The workspace (edges
 * grouped by source) is needed when a projected gradient is asked for; the
 * grouping needs every row's nodes distinct (as in top-k index rows) and in
 * [0, source_nodes) or -1.
 * Replaces query_topk_reduce_backward_cuda (native/jakal_net_native.cpp:
 * 152-165, native/jakal_net_native_cuda.cu:2112-2175).
 */
int jn_edge_reduce_backward(const float* edge_weight, const int32_t* edge_index, const float* projected_state,
                            const float* projected_val, const float* grad_delta_state, const float* grad_delta_val,
                            int64_t batch, int64_t query_nodes, int64_t source_nodes, int64_t edges, int64_t dim,
                            float* grad_edge_weight, float* grad_projected_state, float* grad_projected_val,
                            void* workspace, size_t workspace_bytes, jn_stream_t stream);
size_t jn_edge_reduce_backward_workspace_bytes(int64_t batch, int64_t query_nodes, int64_t source_nodes,
                                               int64_t edges);

/*
 * Routes of a top-k transition and their destination sums:
 *   route[b,i,e] = compress(route_score[b,i,:])[e] (0 softmax, 1 signed |s|
 *   softmax, 2 signed entmax-1.5), k <= 4096 per source;
 *   delta_state[b,j] = sum over routes into j of route * weighted_state[b,i];
 *   delta_val[b,j]   = sum over routes into j of route * weighted_val[b,i].
 * Each source's destinations must be distinct and in [0, dst_nodes) or -1
 * (the routes are grouped by destination), as a top-k select returns them.
 * Replaces the route and destination stage of
 * low_rank_pairwise_topk_forward_cuda (native/jakal_net_native.cpp:167-189,
 * native/jakal_net_native_cuda.cu:2420-2543, kernel 788-878).
 */
int jn_route_topk_aggregate(const int32_t* route_index, const float* route_score, int64_t batch, int64_t src_nodes,
                            int64_t dst_nodes, int64_t edges, int64_t dim, int32_t compress_kind,
                            const float* weighted_state, const float* weighted_val, float* delta_state,
                            float* delta_val, void* workspace, size_t workspace_bytes, jn_stream_t stream);
size_t jn_route_topk_aggregate_workspace_bytes(int64_t batch, int64_t src_nodes, int64_t dst_nodes, int64_t edges);

/*
 * Low-rank pair-score backward.  With g = grad_scores / temperature on the
 * edges (i, j = edge_index[b,i,e]), Pq = projected_query [B, query_nodes, r],
 * Ps = projected_source [B, source_nodes, r], w = core_weight [r]:
 *   dPq[i] = w * sum_e g Ps[j]              dPs[j] = w * sum over edges into j of g Pq[i]
 *   grad_query  = dPq . target_weight       grad_source = dPs . source_weight
 *   grad_target_weight = dPq^T query_val    grad_source_weight = dPs^T source_val
 *   grad_core_weight = sum g Pq * Ps        grad_bias = sum g
 * query_val [B, query_nodes, query_dim] with target_weight [r, query_dim];
 * source_val [B, source_nodes, source_dim] with source_weight [r, source_dim];
 * grad_bias is one float.  Each row's source nodes must be distinct and in
 * [0, source_nodes) or -1 (the edges are grouped by source).  (The reference
 * kernel indexes both sides with
 * query_val's feature dim, so it agrees where the two dims are equal.)
 * Replaces low_rank_pairwise_topk_backward_cuda (native/jakal_net_native.cpp:
 * 449-477, native/jakal_net_native_cuda.cu:2259-2322, 3792-3866).
 */
int jn_lowrank_pair_backward(const float* query_val, const float* source_val, const float* source_weight,
                             const float* target_weight, const float* core_weight, const float* projected_query,
                             const float* projected_source, const int32_t* edge_index, const float* grad_scores,
                             float temperature, int64_t batch, int64_t query_nodes, int64_t source_nodes,
                             int64_t query_dim, int64_t source_dim, int64_t rank, int64_t edges, float* grad_query,
                             float* grad_source, float* grad_source_weight, float* grad_target_weight,
                             float* grad_core_weight, float* grad_bias, void* workspace, size_t workspace_bytes,
                             jn_stream_t stream);
size_t jn_lowrank_pair_backward_workspace_bytes(int64_t batch, int64_t query_nodes, int64_t source_nodes,
                                                int64_t query_dim, int64_t source_dim, int64_t rank, int64_t edges);

#ifdef __cplusplus
}
#endif

#endif /* JAKAL_NET_HIP_H */
