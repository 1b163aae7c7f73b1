/*
 * fuselse_amd C ABI: row-wise log-sum-exp kernels for AMD Instinct MI355X
 * (gfx950).
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers the caller allocated (torch or
 *     hipMalloc); the library allocates nothing.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued asynchronously on it on the current HIP device; the
 *     caller keeps the buffers alive until the stream has run the work.
 *   - Matrices are row-major and contiguous: element (r, i) of a (B, N)
 *     matrix lives at base + r*N + i.  The reduction runs over the last axis.
 *   - Return value: FL_OK (0) on success; FL_EINVAL (1) for a rejected
 *     argument, FL_ELAUNCH (2) when the kernel launch failed, FL_ERANGE (3) for
 *     a size beyond what the kernel indexes.  fl_last_error() then describes
 *     the failure (per calling thread).
 *   - B == 0 (or an empty edge list) returns FL_OK without launching.
 */
#ifndef FUSELSE_AMD_H
#define FUSELSE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FL_ABI_VERSION 1

/* Message for the last failing call on this thread ("" after a success). */
const char* fl_last_error(void);
/* FL_ABI_VERSION the library was built with. */
int fl_abi_version(void);

/* ---------------------------------------------------------------------------
 * fp32 forward: out[r] = log(sum_i exp(x[r, i])), out is fp32 [B].
 * robust != 0 gives torch.logsumexp's special values (all -inf -> -inf, any
 * +inf -> +inf, any NaN -> NaN); robust == 0 assumes finite inputs.
 * Replaces onepass_lse_float / onepass_lse_float_robust
 * (fuselse/gpu/fused_fp32_kernel.cu:154-173, 175-194; kernel :50-133).
 * ------------------------------------------------------------------------- */
int fl_lse_fwd_f32(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream);

/* ---------------------------------------------------------------------------
 * fp32 backward: grad_x[r, i] = grad[r] * exp(x[r, i] - lse[r]).
 * Replaces onepass_lse_float_backward (fused_fp32_kernel.cu:196-252; kernel
 * :135-150).  grad and lse are fp32 [B], x and grad_x fp32 [B, N].
 * ------------------------------------------------------------------------- */
int fl_lse_bwd_f32(const float* grad, const float* x, const float* lse, float* grad_x, int64_t B,
                   int64_t N, void* stream);

/* ---------------------------------------------------------------------------
 * Fused selective log-softmax over fp32 logits [B, N]:
 *   logp[r] = x[r, index[r]] - log(sum_i exp(x[r, i])),
 * with lse[r] (may be NULL) kept for the backward; one pass over x.  It fuses
 * the gather, per-row torch.logsumexp and subtraction of
 * trl.trainer.utils.selective_log_softmax (trl 1.0.0, its fp32 branch), the
 * function the reference's RLHF experiment times with the LSE kernels patched
 * in (experiment_rlhf_logsumexp/run_rlhf.py:28,143-158).  index is int64 [B];
 * an index outside [0, N) gives NaN.  robust as for fl_lse_fwd_f32.
 * workspace: as for fl_lse_fwd_f32_ws, sized by
 * fl_lse_fwd_workspace_bytes(B, N, 4); NULL keeps the one-pass kernels.
 *
 * fl_selective_logsoftmax_bwd_f32:
 *   grad_x[r, i] = grad[r] * ((i == index[r]) - exp(x[r, i] - lse[r])).
 * ------------------------------------------------------------------------- */
int fl_selective_logsoftmax_f32(const float* x, const int64_t* index, float* logp, float* lse, int64_t B,
                                int64_t N, int robust, void* workspace, size_t workspace_bytes, void* stream);
int fl_selective_logsoftmax_bwd_f32(const float* grad, const float* x, const int64_t* index, const float* lse,
                                    float* grad_x, int64_t B, int64_t N, void* stream);

/* ---------------------------------------------------------------------------
 * Half-precision inputs with fp32 accumulation and fp32 output [B].
 * fl_lse_fwd_f16 replaces batched_logsumexp_fp16 (fuselse/gpu/fused_fp16_kernel.cu:
 * 112-132; kernel :25-110).  fl_lse_fwd_bf16 is the bf16 twin, which the
 * reference does not have.  x points to IEEE binary16 / bfloat16 [B, N].
 * ------------------------------------------------------------------------- */
int fl_lse_fwd_f16(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream);
int fl_lse_fwd_bf16(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream);

/* ---------------------------------------------------------------------------
 * Forward for a backward that follows: the arguments, kernels and results of
 * fl_lse_fwd_f32 / _f16 / _bf16 (bit-identical), but the long-row kernels
 * load the first three quarters of x (at most 240 MiB) without the
 * nontemporal hint, so part of x stays in the Infinity Cache (MI355X's 256 MB
 * memory-side cache) for the backward's read of the same rows.  For
 * a backward (fl_lse_bwd_*) that runs right after it on the same x: the
 * pair takes 2-4% less time at (512, 128256) fp32, (256, 128256) fp32 and
 * (2048, 128256) bf16, while this forward alone takes 2-5% more than
 * fl_lse_fwd_*; with a few hundred MB of other traffic between the two the
 * cache holds nothing of x any more and the pair is slower than with
 * fl_lse_fwd_*.  No counterpart in the reference (whose autograd forward
 * calls onepass_lse_float_robust, fused_fp32_kernel.cu:175); the drop-in
 * logsumexp uses it under autograd only when built with keep=True.
 * ------------------------------------------------------------------------- */
int fl_lse_fwd_f32_keep(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream);
int fl_lse_fwd_f16_keep(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream);
int fl_lse_fwd_bf16_keep(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream);

/* ---------------------------------------------------------------------------
 * Half-precision backward: grad_x[r, i] = grad[r] * exp(x[r, i] - lse[r]),
 * computed in fp32 and rounded to nearest even into the input type.  grad
 * and lse are fp32 [B] (lse as the half forward above returns it), x and
 * grad_x binary16 / bfloat16 [B, N].  The reference has no half backward
 * (its drop-in sends fp16 to torch, fuselse/gpu/autograd.py:40); this is the
 * fl_lse_bwd_f32 contract at half storage.
 * ------------------------------------------------------------------------- */
int fl_lse_bwd_f16(const float* grad, const void* x, const float* lse, void* grad_x, int64_t B, int64_t N,
                   void* stream);
int fl_lse_bwd_bf16(const float* grad, const void* x, const float* lse, void* grad_x, int64_t B, int64_t N,
                    void* stream);

/* ---------------------------------------------------------------------------
 * Forward with a caller workspace, for few long rows.  The reference launches
 * one block per row (fused_fp32_kernel.cu:168-170, fused_fp16_kernel.cu:
 * 127-129), which leaves most of the GPU idle when B is small against the
 * CU count; these entries split each such row over several blocks and merge
 * the partial (max, sum) pairs in a fixed order, so results are deterministic.
 * Same results contract as fl_lse_fwd_f32 / _f16 / _bf16 (same tolerance; not
 * bit-identical to the one-pass kernels, whose summation order differs).
 *
 * fl_lse_fwd_workspace_bytes: bytes the _ws entries need for a (B, N) problem
 *   of elem_bytes-sized elements (4 = fp32, 2 = fp16/bf16); 0 when the
 *   one-pass kernels cover the shape (then workspace may be NULL).
 * workspace: device memory of at least that many bytes, 8-byte aligned, any
 *   contents; it holds per-segment partials between the two kernels the call
 *   enqueues, so calls that may run concurrently (other streams) need
 *   separate buffers.
 * ------------------------------------------------------------------------- */
size_t fl_lse_fwd_workspace_bytes(int64_t B, int64_t N, int elem_bytes);
int fl_lse_fwd_f32_ws(const float* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                      size_t workspace_bytes, void* stream);
int fl_lse_fwd_f16_ws(const void* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                      size_t workspace_bytes, void* stream);
int fl_lse_fwd_bf16_ws(const void* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * fl_lse_fwd_f32_noalloc: fl_lse_fwd_f32_ws with the split partials in a
 * static device array instead of a caller workspace, so the call allocates
 * nothing (no hipMalloc, no workspace argument).  No counterpart in the
 * reference: it is for callers that cannot allocate, such as code under HIP
 * graph capture or a serving loop that forbids allocation.  Same kernels,
 * plan and results as fl_lse_fwd_f32_ws (bit-identical).
 * Limit: the array holds 160 KiB per GPU (held until the process ends); every
 * split plan fits (B < 320 rows, at most 64 segments), and a shape needing
 * more is rejected with FL_ERANGE.  The first call on a device whose shape
 * takes the split plan (few long rows; other shapes never touch the array)
 * takes the array's address on that device (hipGetSymbolAddress), so make
 * one such call outside graph capture first.  The address is kept only once
 * it was taken; a call that failed to take it returns FL_ELAUNCH and the next
 * call tries again.  The array's address is per device, so a call whose
 * split plan uses it checks that `stream` belongs to the current device
 * (FL_EINVAL otherwise).  All calls on one GPU share the array: calls that
 * can run concurrently on one GPU (different streams) race and must not
 * overlap.
 * ------------------------------------------------------------------------- */
int fl_lse_fwd_f32_noalloc(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream);

/* ---------------------------------------------------------------------------
 * IntLSE fixed-point row LSE, bit-exact to the reference's GPU reduction tree
 * (256 virtual threads, warp-32 butterflies).  out is fp32 base-e [B];
 * acc_out (may be NULL) receives the final base-2 fixed-point accumulators.
 *
 * fl_intlse_q16_f32: fp32 input, quantised in the kernel as
 *   rne_sat(fl32(x * 94548.4609375)); use_lut == 0 drops the correction table
 *   (the reference's ablation).  Replaces batched_logsumexp /
 *   batched_logsumexp_nolut (intlse/gpu/lse_kernel.cu:164-202; kernel :67-159).
 * fl_intlse_q16_i32: the same tree over pre-quantised Q16.16 int32 input (the
 *   reference has no int32-input entry; its kernel quantises inside the tree).
 * fl_intlse_q10_6: Q10.6 int16 input.  Replaces batched_logsumexp_q10_6
 *   (intlse/gpu/lse_kernel_q10_6.cu:144-165; kernel :55-139).
 * ------------------------------------------------------------------------- */
int fl_intlse_q16_f32(const float* x, float* out, int32_t* acc_out, int64_t B, int64_t N, int use_lut,
                      void* stream);
int fl_intlse_q16_i32(const int32_t* q, float* out, int32_t* acc_out, int64_t B, int64_t N, int use_lut,
                      void* stream);
int fl_intlse_q10_6(const int16_t* q, float* out, int32_t* acc_out, int64_t B, int64_t N, void* stream);

/* ---------------------------------------------------------------------------
 * Sparse probabilistic-circuit sum layer: out[n, b] = log sum_e exp(logw_e +
 * child[c_e, b]) over node n's edges.  Node values are row-major [node][batch]
 * fp32.  q16 != 0 runs the IntLSE Q16.16 arithmetic with the reference's
 * edge-thread tree (bit-exact); q16 == 0 runs fp32.  A node without edges
 * gives -inf.
 *
 * fl_sparse_csr_fwd: CSR edges; offsets int64 [num_nodes + 1], child_ids
 *   int32 [nnz] (rows of child [num_children][batch]), logparams fp32 [nnz].
 *   Writes out [num_nodes][batch].  (The reference has no CSR entry point.)
 * fl_sparse_blocked_fwd: the pyjuice block layout, in place on node_mars:
 *   node block j (nids int64 [num_nblocks]) of block_size parents p writes
 *   node_mars[nids[j] + p, :] from children cids int64 [num_nblocks, num_edges]
 *   with weights params[pids[j, e] + p] (linear weights, log taken with a
 *   1e-45 floor, or log-weights when params_are_log != 0).  Replaces
 *   sparse_forward_float / sparse_forward_q16 (experiment_pyjuice/
 *   sparse_float_kernel.cu:110-167, sparse_q16_kernel.cu:139-202).
 * ------------------------------------------------------------------------- */
int fl_sparse_csr_fwd(const float* child, const int64_t* offsets, const int32_t* child_ids, const float* logparams,
                      float* out, int64_t num_nodes, int64_t batch, int q16, void* stream);
int fl_sparse_blocked_fwd(float* node_mars, const float* element_mars, const float* params, const int64_t* nids,
                          const int64_t* cids, const int64_t* pids, int64_t num_nblocks, int64_t num_edges,
                          int64_t block_size, int64_t batch, int q16, int params_are_log, void* stream);

/* ---------------------------------------------------------------------------
 * Sparse CSR backward ("flows"; the reference has no backward for its sparse
 * kernels).  For out = fl_sparse_csr_fwd(child, offsets, child_ids,
 * logparams) in fp32 and an upstream gradient grad_out [num_nodes, batch]:
 *   term[e, b]          = grad_out[n_e, b] * exp(logparams[e] + child[c_e, b] - out[n_e, b])
 *   grad_child[c, b]     = sum of term[e, b] over edges e with child_ids[e] = c
 *   grad_logparams[e]    = sum of term[e, b] over b
 * with term = 0 where out[n_e, b] is -inf.  The edges are given transposed
 * (CSC): csc_offsets int64 [num_children + 1]; csc_edges int32 [nnz], the
 * edge ids pointing at each child in increasing order; csc_nodes int32 [nnz],
 * the parent node of each of those edges.  child, grad_child: fp32
 * [num_children, batch]; out, grad_out: fp32 [num_nodes, batch]; both
 * gradients are written (not accumulated).  Deterministic: one wave owns each
 * child row and each edge.  grad_child is written once; grad_logparams[e] is
 * stored by the first 512-column tile of the batch and, when batch > 512,
 * increased by the later tiles with atomic adds from that same wave in tile
 * order, so the summation order is fixed.
 * ------------------------------------------------------------------------- */
int fl_sparse_csr_bwd(const float* child, const float* out, const float* grad_out, const float* logparams,
                      const int64_t* csc_offsets, const int32_t* csc_edges, const int32_t* csc_nodes,
                      float* grad_child, float* grad_logparams, int64_t num_children, int64_t batch, void* stream);

/* ---------------------------------------------------------------------------
 * Block-layout backward ("flows") of fl_sparse_blocked_fwd in fp32 (the
 * reference has no backward; this differentiates its block-layout forward,
 * experiment_pyjuice/sparse_float_kernel.cu:40-105).  With node_mars the
 * forward's output and node_flows the upstream flows, for block j, parent p
 * (node n = nids[j] + p), edge e (child c = cids[j, e], parameter
 * q = pids[j, e] + p) and column b:
 *   term = node_flows[n, b] * w_q * exp(element_mars[c, b] - node_mars[n, b])
 * (w_q = max(params[q], 1e-45), or exp(params[q]) with params_are_log; term
 * = 0 where node_mars is -inf), and
 *   edge_flows[j * num_edges + e, b] = sum over p of term   (written)
 *   element_flows[c, b]            += sum of edge_flows rows into c
 *   param_flows[q]                 += sum over b of term.
 * edge_flows is a caller workspace of num_nblocks * num_edges rows of batch
 * floats.  csc_offsets int64 [num_elements + 1] and csc_edges int32
 * [num_nblocks * num_edges] list, for each element row, the block edges
 * j * num_edges + e with cids[j, e] = c in increasing order.  Element flows
 * are summed in that order.  param_flows takes one add per (block, parent,
 * edge): an atomic add, whose order is free only where parameters are
 * shared, or, with params_disjoint (the caller's promise that the ranges
 * [pids[j, e], pids[j, e] + block_size) do not overlap), for blocks of at
 * most 32 parents, a plain read, add and write of each parameter.
 * ------------------------------------------------------------------------- */
int fl_sparse_blocked_bwd(const float* node_flows, const float* node_mars, const float* element_mars,
                          const float* params, const int64_t* nids, const int64_t* cids, const int64_t* pids,
                          int64_t num_nblocks, int64_t num_edges, int64_t block_size, int64_t batch,
                          int params_are_log, int params_disjoint, const int64_t* csc_offsets, const int32_t* csc_edges,
                          int64_t num_elements, float* edge_flows, float* element_flows, float* param_flows,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSELSE_AMD_H */
