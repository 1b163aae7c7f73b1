/* fuselse_amd measurement library: the kernels the benchmark's ceilings,
 * latencies and phase timings come from.  None of them has a counterpart in
 * the reference, and none is part of the row-LSE library's ABI
 * (include/fuselse_amd.h): they live in their own shared library,
 * fuselse_amd/libfuselse_amd_diag.so, which links libfuselse_amd.so.
 *
 * Conventions are those of fuselse_amd.h: an int status (FL_OK == 0),
 * fl_last_error() of libfuselse_amd.so for the message, device pointers,
 * and `stream` a hipStream_t (NULL: the null stream).  Every launch is
 * asynchronous on `stream`.
 */
#ifndef FUSELSE_AMD_DIAG_H
#define FUSELSE_AMD_DIAG_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------------------
 * Measurement aid (no counterpart in the reference): reads nbytes of x (a
 * multiple of 16, 16-byte aligned) from HBM with the forward kernels' load
 * form, 16-byte nontemporal buffer loads, in a flat grid-stride order over
 * `blocks` blocks of `threads` (64 or 256) threads with `unroll` (1, 2, 4 or
 * 8) loads per lane in flight, and nothing else.  The benchmark reports its
 * best rate over the forward's own input buffers as their read ceiling.
 * sink: one uint32 of device memory the kernel may write (it writes only for
 * a value no realistic input produces).
 * ------------------------------------------------------------------------- */
int fl_diag_read_stream(const void* x, int64_t nbytes, int blocks, int threads, int unroll, uint32_t* sink,
                        void* stream);

/* Measurement aid (no counterpart in the reference): copies nbytes of x to y
 * (a multiple of 16, both 16-byte aligned, not overlapping) with the fused
 * backward's forms, 16-byte nontemporal buffer loads and 16-byte buffer
 * stores written through to memory, in a flat grid-stride order over
 * `blocks` blocks of `threads` (64 or 256) threads with `unroll` (1, 2 or 4)
 * vectors per lane.  The benchmark reports its best rate over the backward's
 * own buffers as their copy ceiling. */
int fl_diag_copy_stream(const void* x, void* y, int64_t nbytes, int blocks, int threads, int unroll,
                        void* stream);

/* Measurement aid (no counterpart in the reference): one block of 64 * waves
 * threads (waves 1..16, on one CU) in which every wave runs `steps` (a
 * positive multiple of 16) dependent steps of one kind: 0 = v_add_u32, 1 = ds_read_u8 addressed by the
 * previous value, 2 = the Q10.6 pair step of fl_intlse_q10_6, 3 = the Q16.16
 * pair step with its LDS table, 4 = ds_read_b128 of the lane's own 16 bytes
 * (a conflict-free 16-byte LDS access), 5 = ds_write_b128 of the lane's own
 * 16 bytes followed by that read, 6 and 7 = the transposed 16-byte read and
 * the row-wise write+read of 64-column tiles in rows of 68 words, 8 and 9 =
 * the same in the layout the block-layout backward keeps its tiles in.  rec (device, 3 * waves uint64) receives per
 * wave: shader-clock cycles, 100 MHz real-time ticks, and the chain's final
 * value. */
int fl_diag_chain_latency(int kind, int steps, int waves, uint64_t* rec, void* stream);

/* ---------------------------------------------------------------------------
 * Per-block timestamps (100 MHz real time, s_memrealtime) of the one-block-
 * per-row streaming kernels over B contiguous fp32 rows of N elements (x
 * 16-byte aligned, N a multiple of 4, 1 <= B <= 2^24): one block of 256
 * threads per row, two register sets of two 16-byte vectors per lane in
 * flight, nontemporal buffer loads.
 *   fl_diag_fwd_block_times: the robust forward kernel of fl_lse_fwd_f32 in
 *     this geometry (the one fl_lse_fwd_f32 takes for 512 <= B < 768 rows of
 *     more than 4096 vectors), writing out[B] as that call does;
 *   fl_diag_read_rows_times: the same loads and loop with no arithmetic but
 *     an xor of the words (sink: one uint32 it writes only for a value no
 *     realistic input produces).
 * rec (device, 6 * B uint64) receives per row r: the block's start and end
 * (real-time ticks), its shader-clock cycles (s_memtime) between them, the
 * XCC id, the raw HW_ID register, and r.
 * ------------------------------------------------------------------------- */
int fl_diag_fwd_block_times(const float* x, float* out, int64_t B, int64_t N, uint64_t* rec, void* stream);
int fl_diag_read_rows_times(const float* x, int64_t B, int64_t N, uint64_t* rec, uint32_t* sink, void* stream);

/* The flat read of fl_diag_read_stream in one-wave blocks of 2 KB (block b
 * reads bytes [2048 b, 2048 b + 2048) of x; nbytes a positive multiple of
 * 2048, at most 2^31 bytes).  Blocks whose index b is a multiple of `every`
 * (>= 1) leave the record of fl_diag_fwd_block_times at index b / every (rec:
 * 6 uint64 per record, ceil(nbytes / 2048 / every) records, the last field
 * the block index b). */
int fl_diag_read_stream_times(const void* x, int64_t nbytes, int every, uint64_t* rec, uint32_t* sink, void* stream);

/* Phase timestamps of the IntLSE row kernels, as fl_intlse_q16_f32 (kind 0),
 * fl_intlse_q16_i32 (kind 1) and fl_intlse_q10_6 (kind 2) launch them for
 * these shapes (one block per row, the same prefetch depth; kind 2 only for
 * the 256-thread kernel, so B < 2048 or rows that kernel takes), writing out
 * as those calls do (1 <= B <= 2^24).  rec (device, 8 * B uint64) receives
 * per row, from the block's first thread (virtual threads 0-63): real-time
 * ticks at the block's start, after its first chunk is folded, at the end
 * of its chains, at the end of its tree and after the result is stored; the
 * shader-clock cycles from start to the result; the XCC id; the row. */
int fl_diag_intlse_phases(int kind, const void* x, float* out, int64_t B, int64_t N, uint64_t* rec, void* stream);

/* The plain half forward kernel that fl_lse_fwd_f16 (dtype 0) and
 * fl_lse_fwd_bf16 (dtype 1) launch for many mid-length rows (one 256-thread
 * block per row, four 16-byte vectors per lane per batch; 1 <= B <= 2^24),
 * with unused dynamic LDS reserved so that at most `cap` blocks share a CU
 * (cap 1..8; 0: no reservation, as many blocks as the registers allow).
 * Writes out[B] as those calls do (same bits for every cap).  The library
 * launches the fp16 kernel with cap 3 where it takes it, the bf16 one with
 * no reservation. */
int fl_diag_half_rows_cap(int dtype, const void* x, float* out, int64_t B, int64_t N, int cap, void* stream);

/* The row-pair maxima of the block-layout kernels (max_pair16 / max_pair32
 * in lse_common.hpp, gfx950's lane-swap moves) on one wave: v (device, 64
 * floats, lane l's value v[l]); out (device, 192 floats) receives fmaxf of
 * v over lanes {l, l ^ 16} at out[l], over {l, l ^ 32} at out[64 + l] and over
 * {l, l ^ 16, l ^ 32, l ^ 48} at out[128 + l]. */
int fl_diag_lane_pairs(const float* v, float* out, void* stream);

/* A gather copy: dst[i, :] = src[idx[i], :] for i < nrows (src, dst: fp32 rows
 * of batch columns, batch % 4 == 0, 16-byte aligned; idx: int64 [nrows],
 * valid rows of src).  Each 64-lane wave moves 16 bytes per lane of 8 * 64 / L
 * rows, L = lanes_per_row lanes on each row (16, 32 or 64), and `waves`
 * (1 or 4) waves of a workgroup take neighbouring column tiles of the same
 * rows.  With L = 16 and 4 waves (four rows of 256 bytes per load, 32 rows per
 * wave) it is the access pattern of the block-layout forward's single-chunk
 * kernel without its arithmetic, so its time at a layer's child ids is the
 * ceiling of that layer's forward traffic (the gathered child rows read once,
 * the parent rows written once).  policy: 0 plain loads and stores; 1
 * nontemporal loads (nt); 2 nontemporal stores (the forward's); 4 stores
 * written through to memory (sc1 nt, through a buffer resource over the
 * wave's destination rows); 5 both 1 and 4 (batch <= 2^20). */
int fl_diag_gather_rows(const float* src, const int64_t* idx, float* dst, int64_t nrows, int64_t batch,
                        int lanes_per_row, int waves, int policy, void* stream);

/* The memory pattern of fl_sparse_blocked_bwd's single pass for blocks of 32
 * parents and 32 edges, with one product and sum per column in place of its
 * arithmetic: F [nblocks * 32, batch] gets
 *   F[32 j + e, b] = x[cids[j, e], b] + sum_{ks < 8} o[n, b] * g[n, b],
 *   n = nids[j] + 4 ks + (e / 4) % 4,
 * from the same loads (child rows gathered by id, 256 bytes of each per
 * 64-column tile; the block's o and g rows with the nontemporal hint) and the
 * same edge-flow stores as the single pass, in its order.  One workgroup per
 * node block, `waves` (1, 2 or 4) waves taking interleaved column tiles;
 * lds_per_wave bytes of dynamic LDS per wave (the single pass holds 18432)
 * give it the single pass's occupancy.  batch % 64 == 0, 16-byte aligned
 * buffers; cids int64 [nblocks, 32], valid rows of x; nids valid row starts
 * of 32 rows in o and g.  Its time at a layer is the cost of the single
 * pass's memory traffic alone. */
int fl_diag_blocked_bwd_pattern(float* F, const float* g, const float* o, const float* x, const int64_t* nids,
                                const int64_t* cids, int64_t nblocks, int64_t batch, int waves, int lds_per_wave,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSELSE_AMD_DIAG_H */
