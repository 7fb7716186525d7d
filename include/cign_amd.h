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
 *   - dtype: 0 = float32, 1 = bfloat16 (storage only; math is float32).
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

/* ---- collapsed GAT ------------------------------------------------------- */

/* Schedule geometry (light_max, seg_edges) to build the schedules of a GAT
 * pass with: pass 0 = forward (CSR), 1 = backward (CSR and CSC). */
int cign_gat_schedule_params(int32_t pass, int32_t dtype, int32_t heads, int32_t channels, int32_t* light_max,
                             int32_t* seg_edges);

/* Workspace bytes of cign_gat_fwd for a row schedule with n_seg segments. */
int64_t cign_gat_fwd_workspace_bytes(int32_t n_seg, int32_t heads, int32_t channels);

/* Collapsed GAT forward: edge score, per-destination softmax, edge dropout,
 * weighted aggregation, head mean + bias + SiLU. Replaces the extension
 * `forward` (collapsed_gat_ext/collapsed_gat.cpp:45-72; kernels
 * collapsed_gat_cuda.cu:34-174, host :434-478) with 1<=heads<=32,
 * 1<=channels<=256. Inputs: attn_row/attn_col [n,H] f32, col [nnz] int32
 * (CSR by destination; row_sched built from its row pointer), in_feat
 * [n,H,C] (dtype), bias [C] f32, seed as derived by collapsed_gat.py:204-211.
 * Outputs: out [n,C] (dtype), pre [n,C] f32, edge_max/edge_sum [n,H] f32,
 * edge_mask [nnz,H] u8 (written only when attn_drop > 0). */
int cign_gat_fwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 const float* attn_row, const float* attn_col, const int32_t* col, const int32_t* row_sched,
                 const int32_t* row_sched_info, int32_t* row_counters, float negative_slope, const void* in_feat,
                 const float* bias, float attn_drop, uint64_t seed, void* out, float* pre, float* edge_max,
                 float* edge_sum, uint8_t* edge_mask, void* workspace, int64_t workspace_bytes);

/* Workspace bytes of cign_gat_bwd; row_blocks = n_seg + ceil(n_light / 4) of
 * the row schedule. */
int64_t cign_gat_bwd_workspace_bytes(int32_t n, int32_t nnz, int32_t heads, int32_t channels, int32_t row_blocks,
                                     int32_t n_seg_rows, int32_t n_seg_cols);

/* Collapsed GAT backward: grad_feat [n,H,C] (dtype), grad_attn_row,
 * grad_attn_col [n,H] f32, grad_bias [C] f32 (deterministic, no atomics).
 * Replaces the extension `backward` (collapsed_gat_ext/collapsed_gat.cpp:
 * 74-102; kernels collapsed_gat_cuda.cu:176-430, host :480-545). rowind /
 * perm are the CSC of the same graph (col_sched built from its column
 * pointer) with perm[k] = CSR id of CSC entry k. grad_y has in_feat's dtype. */
int cign_gat_bwd(void* stream, int32_t dtype, int32_t n, int32_t nnz, int32_t heads, int32_t channels,
                 float negative_slope, float attn_drop, const int32_t* col, const int32_t* rowind,
                 const int32_t* perm, const float* edge_max, const float* edge_sum, const uint8_t* edge_mask,
                 const void* in_feat, const float* attn_row, const float* attn_col, const float* pre,
                 const void* grad_y, const int32_t* row_sched, const int32_t* row_sched_info,
                 int32_t* row_counters, const int32_t* col_sched, const int32_t* col_sched_info,
                 int32_t* col_counters, void* workspace, int64_t workspace_bytes, void* grad_feat,
                 float* grad_attn_row, float* grad_attn_col, float* grad_bias);

#ifdef __cplusplus
}
#endif

#endif /* CIGN_AMD_H */
