/*
 * cign_amd.h - C ABI of libcign_amd.so, the gfx950 (MI355X) HIP kernels of
 * the CIGN sparse message-passing hot path.
 *
 * Conventions
 *   - Every compute entry point takes the HIP stream (hipStream_t as void*),
 *     enqueues its kernels on it and returns without synchronising.
 *   - Return value: 0 on success; 1 invalid argument; 2 HIP error. The text
 *     of the last error of the calling thread is cign_last_error().
 *   - All tensors are device pointers to contiguous row-major memory owned by
 *     the caller (inputs borrowed, outputs and workspaces preallocated).
 *   - dtype: 0 = float32, 1 = bfloat16 (storage only; math is float32);
 *     the collapsed GAT also takes 2 = bfloat16 features with float32
 *     outputs and gradients (see cign_gat_fwd).
 *   - Row schedules (cign_amd/csrc/schedule.h) are built on the host once per
 *     CSR/CSC row pointer with cign_row_schedule_size / _build and replace the
 *     row pointer in every launch: the caller uploads the buffer and passes it
 *     as (sched = device copy, sched_info = host copy of its first 12 ints)
 *     with an int32 counter array of n_hrow + 1 zeros (n_hrow = sched_info[2])
 *     that the kernels leave zero again. Calls that share a counter array
 *     must be stream-ordered.
 *
 * Each declaration cites the reference interface it replaces (paths relative
 * to the reference repository).
 */
#ifndef CIGN_AMD_H
#define CIGN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ------------------------------------------------------------ */

/* Last error text of the calling thread (C10/TORCH_CHECK messages in the
 * reference extensions, e.g. collapsed_gat_ext/collapsed_gat.cpp:32-43). */
const char* cign_last_error(void);

/* ABI version. */
int cign_version(void);

/* Row schedule sizes for a host row pointer [n_rows + 1] (int64). Replaces
 * the one-time plan preparation of MultiHopCsrPlan::prepare
 * (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:246-262). */
int cign_row_schedule_size(const int64_t* rowptr, int32_t n_rows, int32_t light_max, int32_t seg_edges,
                           int32_t* n_light, int32_t* n_seg, int32_t* n_hrow, int64_t* total_ints);

/* Fills the host schedule buffer (total_ints int32) sized by the call above. */
int cign_row_schedule_build(const int64_t* rowptr, int32_t n_rows, int32_t light_max, int32_t seg_edges,
                            int32_t* out, int64_t total_ints);

/* ---- CSR SpMM / multihop pipeline ---------------------------------------- */

/* Bytes of float scratch `partial` cign_spmm needs for n_seg segments and d
 * dense columns (the cuSPARSE workspace of the reference,
 * multihop_csr_pipeline_cuda.cu:226-262). */
int64_t cign_spmm_partial_bytes(int32_t n_seg, int32_t d);

/* y = P x (+ add). One cusparseSpMM of MultiHopCsrPlan::spmm
 * (multihop_csr_pipeline_cuda.cu:264-285) or one torch.sparse.mm of
 * FixedCSRSpMMFunction (model.py:88-106). col/val are the CSR arrays of P
 * whose row pointer the schedule was built from; add may be NULL. */
int cign_spmm(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
              const int32_t* sched, const int32_t* sched_info, const void* x, const void* add, void* y,
              float* partial, int32_t* counters);

/* y1 = P x, y2 = P y1, y3 = P y2. Replaces MultiHopCsrPlan::forward3
 * (multihop_csr_ext/multihop_csr_pipeline.h:24; .cu:287-297). */
int cign_spmm_fwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
                   const int32_t* sched, const int32_t* sched_info, const void* x, void* y1, void* y2, void* y3,
                   float* partial, int32_t* counters);

/* t2 = g2 + P^T g3, t1 = g1 + P^T t2, gx = P^T t1 (adds fused into the SpMM
 * epilogue; t1/t2 are caller scratch). Replaces MultiHopCsrPlan::backward3
 * (multihop_csr_ext/multihop_csr_pipeline.h:25-28; .cu:299-321). The CSR and
 * schedule passed here are those of P^T. */
int cign_spmm_bwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
                   const int32_t* sched, const int32_t* sched_info, const void* g1, const void* g2, const void* g3,
                   void* t2, void* t1, void* gx, float* partial, int32_t* counters);

/* cign_spmm_fwd3 without caller workspace: the partial sums and merge
 * counters live in a 16 MiB array of the library's own (per GPU, held until
 * the process ends), so the call allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). Limits: the
 * schedule's n_hrow + 1 <= 262144 and cign_spmm_partial_bytes(n_seg, d) <=
 * 15 MiB, else status 1 with the sizes in cign_last_error(). Results are
 * bit-identical to cign_spmm_fwd3. Calls that overlap on one GPU share the
 * scratch and race: keep them stream-ordered. */
int cign_spmm_fwd3_noalloc(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col,
                           const float* val, const int32_t* sched, const int32_t* sched_info, const void* x,
                           void* y1, void* y2, void* y3);

/* ---- collapsed GAT ------------------------------------------------------- */

/* Schedule geometry (light_max, seg_edges) to build the schedules of a GAT
 * pass with: pass 0 = forward (CSR), 1 = backward (CSR and CSC). seg_edges 0
 * means any multiple of 256 (the feature-layout kernels); the host picks it
 * from the graph size like the SpMM's. */
int cign_gat_schedule_params(int32_t pass, int32_t dtype, int32_t heads, int32_t channels, int32_t* light_max,
                             int32_t* seg_edges);

/* Workspace bytes of cign_gat_fwd for a row schedule with n_seg segments. */
int64_t cign_gat_fwd_workspace_bytes(int32_t n_seg, int32_t heads, int32_t channels);

/* Floats of the optional per-row aggregate buffer (row_agg) that
 * cign_gat_fwd fills and cign_gat_bwd reads, n*H*(2C+1) for the shapes of
 * the feature-layout kernels (H <= 8, C a multiple of 16 bytes' worth of
 * elements with C/that a power of two, H*C <= 64 such chunks), 0 otherwise.
 * The buffer holds sum_e s kw x[j], sum_e s kw l' x[j] ([n,H,C] each) and
 * sum_e s l' ([n,H]) per destination row, so the backward need not gather
 * the source rows a second time. No counterpart in the reference: its
 * _CollapsedGATFn saves the same tensors (collapsed_gat.py:106-110) and its
 * backward re-gathers in_feat per edge (collapsed_gat_cuda.cu:176-300). */
int64_t cign_gat_row_agg_floats(int32_t dtype, int32_t n, int32_t heads, int32_t channels);

/* Collapsed GAT forward: edge score, per-destination softmax, edge dropout,
 * weighted aggregation, head mean + bias + SiLU. Replaces the extension
 * `forward` (collapsed_gat_ext/collapsed_gat.cpp:45-72; kernels
 * collapsed_gat_cuda.cu:34-174, host :434-478) with 1<=heads<=32,
 * 1<=channels<=256. Inputs: attn_row/attn_col [n,H] f32, col [nnz] int32
 * (CSR by destination; row_sched built from its row pointer), in_feat
 * [n,H,C] (dtype), bias [C] f32, seed as derived by collapsed_gat.py:204-211.
 * Outputs: out [n,C] (dtype), pre [n,C] f32, edge_max/edge_sum [n,H] f32,
 * edge_mask [nnz,H] u8 (written only when attn_drop > 0). row_agg: null, or
 * cign_gat_row_agg_floats() floats (16-byte aligned) to receive the per-row
 * aggregates of the backward. dtype 2 (shapes with cign_gat_row_agg_floats
 * > 0): in_feat bf16, out (and, in cign_gat_bwd, grad_y and grad_feat)
 * float32: the results of dtype 0 on the same values when in_feat holds the
 * bf16 output of an autocast projection, which _local_amp_linear returns as
 * float32 (model_cign.py:86-103, :546-553), in half the gathered bytes. */
int cign_gat_fwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                 const int32_t* row_sched_info, int32_t* row_counters, float negative_slope, const void* in_feat,
                 const float* bias, float attn_drop, uint64_t seed, void* out, float* pre, float* edge_max,
                 float* edge_sum, uint8_t* edge_mask, void* workspace, int64_t workspace_bytes, float* row_agg);

/* Workspace bytes of cign_gat_bwd; row_blocks = n_seg + ceil(n_light / 4) of
 * the row schedule. */
int64_t cign_gat_bwd_workspace_bytes(int32_t n, int32_t nnz, int32_t heads, int32_t channels, int32_t row_blocks,
                                     int32_t n_seg_rows, int32_t n_seg_cols);

/* Collapsed GAT backward: grad_feat [n,H,C] (dtype), grad_attn_row,
 * grad_attn_col [n,H] f32, grad_bias [C] f32 (deterministic, no atomics).
 * Replaces the extension `backward` (collapsed_gat_ext/collapsed_gat.cpp:
 * 74-102; kernels collapsed_gat_cuda.cu:176-430, host :480-545). rowind /
 * perm are the CSC of the same graph (col_sched built from its column
 * pointer) with perm[k] = CSR id of CSC entry k. grad_y has in_feat's dtype.
 * row_agg: null (the rows pass gathers in_feat per edge) or the buffer the
 * forward filled for the same inputs (the rows pass streams it instead). */
int cign_gat_bwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                 const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                 const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                 const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                 int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                 int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                 float* grad_attn_row, float* grad_attn_col, float* grad_bias, const float* row_agg);

/* cign_gat_fwd over one destination-row shard of a larger graph, the
 * partitioned execution that replaces run_chunked_dgnn_op
 * (chunked_dgnn_gat.py:214-252): n and col are the shard's rows and its
 * in-edges with source ids local to the gathered in_feat / attn_col (its own
 * rows and its source halo); attn_row and the outputs are the shard's rows.
 * edge_base = the CSR id, in the whole graph, of the shard's first edge: the
 * dropout mask is hashed on whole-graph edge ids (and stored at the shard's
 * own). graph_nnz = the whole graph's edges: the kernels run the variant the
 * whole-graph call runs, so with the whole graph's schedule geometry every
 * row's outputs are bit-identical to cign_gat_fwd's. */
int cign_gat_fwd_shard(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                       const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                       const int32_t* row_sched_info, int32_t* row_counters, float negative_slope,
                       const void* in_feat, const float* bias, float attn_drop, uint64_t seed, void* out, float* pre,
                       float* edge_max, float* edge_sum, uint8_t* edge_mask, void* workspace,
                       int64_t workspace_bytes, float* row_agg, int64_t edge_base, int64_t graph_nnz);

/* cign_gat_bwd over one source-column shard: the graph holds the shard's
 * source nodes with all their out-edges and the destination rows those
 * reach (the halo), every per-row input (edge_max, edge_sum, attn_row, pre,
 * grad_y, row_agg) gathered for those rows from the whole-graph forward.
 * row_agg is required: the halo rows have only part of their in-edges here,
 * so their row sums come from the aggregates. grad_feat and grad_attn_col are
 * complete (bit-identical to cign_gat_bwd's) for the shard's sources, and
 * grad_attn_row for every row; grad_bias sums grad_pre rows [bias_row_lo,
 * bias_row_lo + bias_rows) only (the shard's own nodes; the whole graph's is
 * the sum over shards). graph_nnz as in cign_gat_fwd_shard. No counterpart
 * in the reference, whose chunked path leaves the source gradients of
 * overlapping chunks to autograd's scatter-add. */
int cign_gat_bwd_shard(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                       float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                       const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                       const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                       const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                       int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                       int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                       float* grad_attn_row, float* grad_attn_col, float* grad_bias, const float* row_agg,
                       int32_t bias_row_lo, int32_t bias_rows, int64_t graph_nnz);

/* ---- GAT side ops (float32) ---------------------------------------------- */

/* Workspace bytes of a backward entry point below whose parameter gradient
 * sums `quantities` vectors of `width` floats over n rows:
 * cign_attn_logits_bwd (H*C, 2), cign_head_silu_bwd (C, 1),
 * cign_dropout_ln_bwd / cign_add_ln_bwd (D, 2), cign_gamma_residual_bwd (D, 1).
 * Replaces the temporaries of the reference's two-stage reductions
 * (fused_block_ops_cuda.cu PARAM_CHUNK_N partials). */
int64_t cign_colsum_workspace_bytes(int64_t n, int32_t width, int32_t quantities);

/* alpha_src[n,h] = <x[n,h,:], att_src[h,:]>, alpha_dst likewise. x [n,H,C],
 * att_* [1,H,C], alpha_* [n,H]. Replaces ext attention_forward
 * (fused_gat_sideops_ext/fused_gat_sideops.cpp:45-51; kernels
 * fused_gat_sideops_cuda.cu:25-60). C <= 1024. */
int cign_attn_logits_fwd(void* stream, int64_t n, int32_t heads, int32_t channels, const float* x,
                         const float* att_src, const float* att_dst, float* alpha_src, float* alpha_dst);

/* grad_x = gs*att_src + gd*att_dst; grad_att_* [1,H,C] = sum_n g[n,h] x[n,h,:]
 * (deterministic). Replaces ext attention_backward (fused_gat_sideops.cpp:54-66;
 * kernels fused_gat_sideops_cuda.cu:65-167). */
int cign_attn_logits_bwd(void* stream, int64_t n, int32_t heads, int32_t channels, const float* grad_src,
                         const float* grad_dst, const float* x, const float* att_src, const float* att_dst,
                         float* grad_x, float* grad_att_src, float* grad_att_dst, void* workspace,
                         int64_t workspace_bytes);

/* cign_attn_logits_fwd on x stored as bf16 [n,H,C] (the GAT lin's bf16
 * output, see cign_linear_fwd_bf16y). No counterpart in the reference (its x
 * is float32). */
int cign_attn_logits_fwd_bf16(void* stream, int64_t n, int32_t heads, int32_t channels, const void* x,
                              const float* att_src, const float* att_dst, float* alpha_src, float* alpha_dst);

/* cign_attn_logits_bwd that also adds the gradient x receives from its other
 * consumer, the collapsed GAT: grad_x = grad_x_in + gs*att_src + gd*att_dst
 * (grad_x_in may alias grad_x; null for none), the sum autograd forms between
 * ext attention_backward (fused_gat_sideops.cpp:54-66) and the GAT's
 * backward, without a pass of its own. x_dtype: 0 = float32, 1 = bf16
 * storage (as cign_attn_logits_fwd_bf16). grad_x_dtype: 0 = float32, 1 =
 * bf16 (x_dtype 1 with channels a multiple of 8 only; the sum rounded to
 * nearest even, what a bf16-math GEMM reads of it; grad_x_in must not alias
 * it). */
int cign_attn_logits_bwd_acc(void* stream, int64_t n, int32_t heads, int32_t channels, int32_t x_dtype,
                             int32_t grad_x_dtype, const float* grad_src, const float* grad_dst, const void* x,
                             const float* att_src, const float* att_dst, const float* grad_x_in, void* grad_x,
                             float* grad_att_src, float* grad_att_dst, void* workspace, int64_t workspace_bytes);

/* pre = sum_h out[n,h,:] / H + bias, y = SiLU(pre). Replaces ext
 * head_silu_forward (fused_gat_sideops.cpp:68-76; kernel
 * fused_gat_sideops_cuda.cu:171-195). */
int cign_head_silu_fwd(void* stream, int64_t n, int32_t heads, int32_t channels, const float* out,
                       const float* bias, float* y, float* pre);

/* grad_out[n,h,:] = grad_y SiLU'(pre) / H, grad_bias = sum_n grad_y SiLU'(pre).
 * Replaces ext head_silu_backward (fused_gat_sideops.cpp:78-90; kernels
 * fused_gat_sideops_cuda.cu:197-239). */
int cign_head_silu_bwd(void* stream, int64_t n, int32_t heads, int32_t channels, const float* grad_y,
                       const float* pre, float* grad_out, float* grad_bias, void* workspace, int64_t workspace_bytes);

/* ---- block ops (float32, 1 <= D <= 256) ----------------------------------- */

/* q = keep * x / (1-p) (keep: splitmix64 53-bit bits of seed and n*D+c,
 * u >= p; mask [n,D] u8 written), y = LayerNorm(q) * weight + bias; mean,
 * rstd [n]. Replaces ext dropout_layernorm_forward (fused_block_ops.py:15,
 * fused_block_ops_ext/fused_block_ops.cpp:39-45; kernels
 * fused_block_ops_cuda.cu:45-70). */
int cign_dropout_ln_fwd(void* stream, int64_t n, int32_t D, const float* x, const float* weight, const float* bias,
                        float dropout_p, float eps, uint64_t seed, float* y, float* mean, float* rstd, uint8_t* mask);

/* grad_x, grad_weight, grad_bias of the above. Replaces ext
 * dropout_layernorm_backward (fused_block_ops.cpp:46-56; kernels
 * fused_block_ops_cuda.cu:96-118 + param stages). */
int cign_dropout_ln_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* x, const float* weight,
                        const float* mean, const float* rstd, const uint8_t* mask, float dropout_p, float* grad_x,
                        float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes);

/* y = LayerNorm(a + b) * weight + bias. Replaces ext add_layernorm_forward
 * (fused_block_ops.cpp:57-63; kernel fused_block_ops_cuda.cu:72-94). */
int cign_add_ln_fwd(void* stream, int64_t n, int32_t D, const float* a, const float* b, const float* weight,
                    const float* bias, float eps, float* y, float* mean, float* rstd);

/* grad_z (the gradient of both a and b), grad_weight, grad_bias. Replaces ext
 * add_layernorm_backward (fused_block_ops.cpp:64-73; kernels
 * fused_block_ops_cuda.cu:120-139 + param stages). */
int cign_add_ln_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* a, const float* b,
                    const float* weight, const float* mean, const float* rstd, float* grad_z, float* grad_weight,
                    float* grad_bias, void* workspace, int64_t workspace_bytes);

/* y = LayerNorm(a + b) * weight + bias as cign_add_ln_fwd, also written with
 * b into cat [n, 2D] = [b | y]. Replaces the add-LayerNorm and the
 * concatenation of GraphCliffordBlock.forward (C_norm = LN(C_gat + H_norm),
 * HC_norm = cat([H_norm, C_norm]); generic_engine/model_cign.py:781-792). */
int cign_add_ln_cat_fwd(void* stream, int64_t n, int32_t D, const float* a, const float* b, const float* weight,
                        const float* bias, float eps, float* y, float* cat, float* mean, float* rstd);

/* Backward of cign_add_ln_cat_fwd given the gradients of y and cat: the LN
 * backward of grad_y + grad_cat[:, D:] gives grad_a, and grad_b = grad_a +
 * grad_cat[:, :D]; grad_weight, grad_bias; workspace as cign_add_ln_bwd. */
int cign_add_ln_cat_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* grad_cat, const float* a,
                        const float* b, const float* weight, const float* mean, const float* rstd, float* grad_a,
                        float* grad_b, float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes);

/* y = h + gamma * keep * g / (1-p); mask [n,D] u8. Replaces ext
 * dropout_gamma_residual_forward (fused_block_ops.cpp:74-81). */
int cign_gamma_residual_fwd(void* stream, int64_t n, int32_t D, const float* h, const float* g, const float* gamma,
                            float dropout_p, uint64_t seed, float* y, uint8_t* mask);

/* grad_g = grad_y * gamma * m, grad_gamma = sum_n grad_y * g * m (m = keep/(1-p));
 * grad_h = grad_y is the caller's. Replaces ext dropout_gamma_residual_backward
 * (fused_block_ops.cpp:82-90). */
int cign_gamma_residual_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* g,
                            const float* gamma, const uint8_t* mask, float dropout_p, float* grad_g, float* grad_gamma,
                            void* workspace, int64_t workspace_bytes);

/* ---- hop gate (float32) ------------------------------------------------- */

/* Node-mode hop gate: alpha [n,K] = softmax_k(score @ weight^T + bias), score
 * [n,2D] = [H | C] (score_mode 0, old) or [H + C | |H - C|] (1, new); weight
 * [K,2D], bias [K], K <= 16. Replaces GraphCliffordBlock.compute_hop_gate
 * (generic_engine/model_cign.py:721-749: concatenation, Linear, softmax). */
int cign_hop_gate_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t score_mode, const float* H,
                      const float* C, const float* weight, const float* bias, float* alpha);

/* Workspace bytes of cign_hop_gate_bwd. */
int64_t cign_hop_gate_bwd_workspace_bytes(int64_t n, int32_t D, int32_t K);

/* Backward of cign_hop_gate_fwd given alpha and grad_alpha: grad_H, grad_C
 * [n,D], grad_weight [K,2D], grad_bias [K] (deterministic; sign(0) = 0 for the
 * |H - C| term, as torch's abs). Replaces the autograd of the same lines. */
int cign_hop_gate_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t score_mode, const float* H,
                      const float* C, const float* weight, const float* alpha, const float* grad_alpha, float* grad_H,
                      float* grad_C, float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes);

/* Node-mode hop gate fused into the Clifford pack (interaction and weighting
 * codes of cign_pack_fwd): alpha [n,K] from (H, C, gate weight [K,2D], gate
 * bias [K]) as cign_hop_gate_fwd computes it, written to `alpha`, and the
 * pack of cign_pack_fwd with that alpha into `out`, in one pass over H and C.
 * Replaces the compute_hop_gate + fused pack pair of GraphCliffordBlock.forward
 * (generic_engine/model_cign.py:721-749 feeding :803-846, node hop gate). */
int cign_pack_gate_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                       int32_t score_mode, const float* H, const float* C, const float* const* props,
                       int64_t prop_stride, const float* gate_weight, const float* gate_bias, float* alpha,
                       float* out);

/* Backward of cign_pack_gate_fwd given grad_out and its alpha: grad_H and
 * grad_C (the pack's and the gate's terms summed), grad_props, grad_gate_weight
 * [K,2D], grad_gate_bias [K]; workspace of cign_hop_gate_bwd_workspace_bytes.
 * Replaces the autograd of the same lines. */
int cign_pack_gate_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                       int32_t score_mode, const float* grad_out, const float* H, const float* C,
                       const float* const* props, int64_t prop_stride, const float* alpha, const float* gate_weight,
                       float* grad_H, float* grad_C, float* const* grad_props, int64_t grad_prop_stride,
                       float* grad_gate_weight, float* grad_gate_bias, void* workspace, int64_t workspace_bytes);

/* The Clifford pack (weighting old: G = cat_k alpha_k [W_k, D_k], [n, 2KD])
 * built inside the projection's MFMA operand load, with the gamma epilogue
 * of cign_linear_gamma_fwd: g_out = G Wp^T + bias, out = h + gamma *
 * drop(g_out), mask. G is never stored. Replaces the pack feeding `proj`
 * (generic_engine/model_cign.py:803-846 then :927-933). D in {64, 128, 256},
 * 1 <= K <= 4, interaction as cign_pack_fwd, math as cign_linear_fwd; props:
 * HOST array of K device row pointers (row stride prop_stride floats, >= 2D);
 * alpha [n,K] with row stride alpha_stride (K), or one row for every node
 * (stride 0: the global gate, or ones without a gate); w = Wp [D, 2KD];
 * workspace of cign_pack_proj_fwd_workspace_bytes. */
int cign_pack_proj_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t math,
                       const float* H, const float* C, const float* const* props, int64_t prop_stride,
                       const float* alpha, int64_t alpha_stride, const float* w, const float* bias, const float* h,
                       const float* gamma, float dropout_p, uint64_t seed, float* g_out, float* out, uint8_t* mask,
                       void* workspace, int64_t workspace_bytes);

/* Workspace bytes of cign_pack_proj_fwd (with math = 1, the bf16 copy of w
 * the kernel reads; 0 with math = 0 or for shapes it does not take). */
int64_t cign_pack_proj_fwd_workspace_bytes(int32_t D, int32_t K, int32_t math);

/* Workspace bytes of cign_pack_proj_bwd (0 for shapes it does not take). */
int64_t cign_pack_proj_bwd_workspace_bytes(int64_t n, int32_t D, int32_t K);

/* Backward of cign_pack_proj_fwd from grad_g = d out / d g_out (as
 * cign_gamma_residual_bwd gives it): grad_G = grad_g Wp computed per block of
 * 32 channels of every hop and half and consumed in the same kernel by the
 * pack's backward (grad_H, grad_C, grad_props [n,2D] each, grad_alpha [n,K]),
 * grad_w [D,2KD] = grad_g^T G with G rebuilt in the reduction's operand load,
 * grad_b (NULL to skip) = sum_n grad_g. With gate_weight (the node gate of
 * cign_hop_gate_fwd that produced alpha, stride K), the gate's backward is
 * added: its input terms into grad_H / grad_C, grad_gate_weight [K,2D],
 * grad_gate_bias [K]. With math = 1, grad_G, grad_w and grad_b are rounded to
 * bf16 (autocast's backward outputs) and the products read bf16 operands.
 * Replaces the autograd of the same lines. */
int cign_pack_proj_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t math,
                       const float* grad_g, const float* H, const float* C, const float* const* props,
                       int64_t prop_stride, const float* alpha, int64_t alpha_stride, const float* w,
                       int32_t score_mode, const float* gate_weight, float* grad_H, float* grad_C,
                       float* const* grad_props, int64_t grad_prop_stride, float* grad_alpha, float* grad_w,
                       float* grad_b, float* grad_gate_weight, float* grad_gate_bias, void* workspace,
                       int64_t workspace_bytes);

/* ---- Clifford packs (float32) ------------------------------------------- */

/* Fused Clifford interaction + alpha weighting over K <= 16 hops.
 * interaction: 0 old (D = SiLU(bhr), W = bhr - brh), 1 new (D = SiLU((bhr+brh)/2),
 * W = (bhr-brh)/2), 2 new with tanh on W; weighting: 0 old (out [n, K*2D] =
 * cat_k a_k [W_k, D_k]), 1 new (out [n, 2D] = [sum a_k D_k, sum a_k W_k]).
 * props: HOST array of K device row pointers of the propagated hops, rows
 * prop_stride floats apart (2D for separate [n,2D] tensors, 2KD for one
 * stacked [n,K,2D] tensor); alpha [n,K]. Replaces the ext `forward` of
 * fused_clifford_pack_ext/fused_clifford_pack.cpp:50-59 (old, K=3), the generic
 * ext of fused_clifford_pack.py:46-63, generic_engine/fused_clifford_cign_pack_ext/
 * fused_clifford_switch_pack.cpp:69-85 (and its tanh twin in
 * generic_engine/fused_clifford_switch_pack_ext/), and
 * generic_engine/fused_clifford_cign_generic.py:20-41. */
int cign_pack_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                  const float* H, const float* C, const float* const* props, int64_t prop_stride, const float* alpha,
                  float* out);

/* Backward of cign_pack_fwd: grad_H, grad_C [n,D], grad_props (HOST array of
 * K device row pointers, rows grad_prop_stride apart), grad_alpha [n,K].
 * Deterministic, no atomics. Replaces the ext `backward` of the same modules
 * (fused_clifford_pack.cpp:61-80, fused_clifford_switch_pack.cpp:86-121). */
int cign_pack_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                  const float* grad_out, const float* H, const float* C, const float* const* props,
                  int64_t prop_stride, const float* alpha, float* grad_H, float* grad_C, float* const* grad_props,
                  int64_t grad_prop_stride, float* grad_alpha);

/* ---- dense projections on MFMA ------------------------------------------ */

/* math: 0 = float32 (fp32 MFMA, exact fp32 products), 1 = bf16 autocast
 * (x, weight and bias rounded to bf16, bf16 MFMA with fp32 accumulation,
 * output rounded to bf16 and stored as float32). x [M,K] float32 or bfloat16 (x_dtype; bf16
 * needs math 1), weight [N,K] float32 (nn.Linear layout), bias [N] or NULL.
 * Any M, N, K; rows that start 16-byte aligned are read with vector loads. */

/* y [M,N] = x W^T + b. Replaces _local_amp_linear / nn.Linear
 * (generic_engine/model_cign.py:86-103: GAT lin :546-553, proj :927-929,
 * input projections :1165-1171). */
int cign_linear_fwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t math, const void* x,
                    const float* w, const float* bias, float* y);

/* GAT lin + attention logits in one kernel: y [M,H*C] = x W^T (no bias),
 * alpha_src[m,h] = <y[m,h,:], att_src[h,:]>, alpha_dst likewise; C in
 * {16, 32, 64, 128}. Replaces the lin call of CompatibleCollapsedFusedGATConv
 * (model_cign.py:546-553) followed by ext attention_forward
 * (fused_gat_sideops.cpp:45-52). */
int cign_linear_logits_fwd(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K, int32_t x_dtype,
                           int32_t math, const void* x, const float* w, const float* att_src, const float* att_dst,
                           float* y, float* alpha_src, float* alpha_dst);

/* cign_linear_fwd / cign_linear_logits_fwd with math 1 whose y is stored as
 * bf16 [M,N]: the same values (math 1 rounds the output to bf16), half the
 * bytes. For a projection whose only consumers read bf16 (the collapsed GAT
 * with dtype 2, cign_attn_logits_*_bf16): the GAT lin of
 * CompatibleCollapsedFusedGATConv under selective AMP (model_cign.py:546-553),
 * whose float32 result holds bf16 values. */
int cign_linear_fwd_bf16y(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, const void* x,
                          const float* w, const float* bias, void* y);
int cign_linear_logits_fwd_bf16y(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K,
                                 int32_t x_dtype, const void* x, const float* w, const float* att_src,
                                 const float* att_dst, void* y, float* alpha_src, float* alpha_dst);

/* Projection + dropout-gamma-residual: g_out [M,N] = x W^T + b,
 * y = h + gamma * keep * g_out / (1-p), mask [M,N] u8 (keep = 53-bit
 * splitmix64 of seed and m*N+n, keep when u >= p). Replaces proj
 * (model_cign.py:927-929) followed by ext dropout_gamma_residual_forward
 * (fused_block_ops.cpp:72-80). */
int cign_linear_gamma_fwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t math,
                          const void* x, const float* w, const float* bias, const float* h, const float* gamma,
                          float dropout_p, uint64_t seed, float* g_out, float* y, uint8_t* mask);

/* Workspace bytes of cign_linear_bwd. */
int64_t cign_linear_bwd_workspace_bytes(int64_t M, int32_t N, int32_t K, int32_t with_bias);

/* grad_x [M,K] = grad_y W (NULL to skip; the forward MFMA kernel against
 * W^T, which the workspace holds), grad_w [N,K] =
 * grad_y^T x (split-M MFMA partials summed in order) and grad_b [N] =
 * sum_m grad_y (NULL to skip), fp32 accumulation, grad_w and grad_b
 * deterministic; with math = 1 every product reads bf16-rounded operands and
 * grad_x, grad_w, grad_b are rounded to bf16 (grad_b the sum of the rounded
 * grad_y): the outputs of the bf16 Linear's backward under autocast. N <= 16
 * runs two VALU streaming kernels instead, N <= 64 narrow-output MFMA kernels.
 * grad_y,
 * x float32. Replaces the autograd backward of the Linear layers above. */
int cign_linear_bwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t math, const float* grad_y, const float* x,
                    const float* w, float* grad_x, float* grad_w, float* grad_b, void* workspace,
                    int64_t workspace_bytes);

/* cign_linear_bwd with math = 1, no bias and N > 16, whose grad_y is bf16
 * storage [M,N]: the values bf16 math rounds a float32 grad_y to, read in half
 * the bytes; results equal cign_linear_bwd's on the float32 grad_y. Workspace:
 * cign_linear_bwd_workspace_bytes(M, N, K, 0). No counterpart in the
 * reference; the GAT lin's backward under AMP, whose gradient
 * cign_attn_logits_bwd_acc writes as bf16. */
int cign_linear_bwd_bf16gy(void* stream, int64_t M, int32_t N, int32_t K, const void* grad_y, const float* x,
                           const float* w, float* grad_x, float* grad_w, void* workspace, int64_t workspace_bytes);

/* The GAT lin's weight and attention-vector gradients when its input needs
 * none (input features are data): with N = heads*channels,
 * gy = grad_xp + grad_src (x) att_src + grad_dst (x) att_dst per head (the sum
 * cign_attn_logits_bwd_acc forms, never stored), grad_w [N,K] = gy^T x
 * (math 1: gy and x rounded to bf16 before their products and grad_w
 * rounded to bf16, as cign_linear_bwd_bf16gy on the stored sum),
 * grad_att_src [N] = sum_m grad_src[m,h] xp[m,h,c] and grad_att_dst likewise
 * (float32), all deterministic: one fused kernel writes per-row-chunk
 * partials of grad_w and of the two sums and one launch adds them in order.
 * Needs 16 < N <= 64, channels and K multiples of 4, grad_xp and x rows
 * 16-byte aligned, xp (xp_dtype 0 = float32, 1 = bf16 storage) 16-byte
 * (bf16: 8-byte) aligned. Workspace: cign_lin_logits_wgrad_workspace_bytes.
 * No counterpart in the reference: it fuses ext attention_backward
 * (fused_gat_sideops.cpp:54-66) with the weight gradient of the lin's
 * Linear (model_cign.py:546-553) for the narrow projection of config c2. */
int64_t cign_lin_logits_wgrad_workspace_bytes(int64_t M, int32_t N, int32_t K);
int cign_lin_logits_wgrad(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K, int32_t xp_dtype,
                          int32_t math, const float* grad_xp, const float* grad_src, const float* grad_dst,
                          const void* xp, const float* att_src, const float* att_dst, const float* x, float* grad_w,
                          float* grad_att_src, float* grad_att_dst, void* workspace, int64_t workspace_bytes);

#ifdef __cplusplus
}
#endif

#endif /* CIGN_AMD_H */
