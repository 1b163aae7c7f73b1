// Float log-sum-exp kernels for gfx950: fp32 / fp16 / bf16 forward (plain and
// robust) and the fused fp32 backward.
//
// Forward: a single pass over HBM.  Each lane keeps an online (max, scaled
// sum) pair and folds a batch of 16-byte vectors at a time with a single
// rescale, so the steady state costs one v_exp_f32 per element.  Two loops:
// a software-pipelined one (the next batch's loads in flight while a batch
// folds; masked last batch) and a burst one (short rows).  Lanes merge
// through DPP / swizzle exchanges and waves through LDS.  Three geometries
// (launch_fwd picks geometry and loop per shape):
//   * group rows  : LPR lanes per row (4..64), 64/LPR rows per wave, for rows
//                   of up to 4096 vectors;
//   * block rows  : one 128..1024-thread block per row for longer rows and
//                   for few mid-length rows;
//   * split rows  : S blocks per row for few long rows, then a merge kernel
//                   (partials in a caller workspace);
// Backward: grad * exp2((x - lse) * log2 e), 16-byte loads and stores (fp32,
// fp16 or bf16 x and grad_x, fp32 arithmetic), grad[r] and lse[r]
// wave-uniform.
#include <stdint.h>

#include <mutex>

#include "../../include/fuselse_amd.h"
#include "fl_status.hpp"
#include "lse_common.hpp"
#include "lse_fwd_kernels.hpp"

namespace fl {

// ---------------------------------------------------------------------------
// Split rows, for few long rows (one block per row would leave most of the
// 256 CUs idle).  Two kernels on the caller's stream:
//   * lse_fwd_split_partials, grid (S, B): block k of row r folds the body
//     vectors [k*seg, (k+1)*seg) of row r (block 0 also its scalar head and
//     tail) and stores its partial (m, s) in part[r*S + k];
//   * lse_fwd_split_merge: LPR >= S lanes per row merge the S partials with a
//     fixed tree, so the result is deterministic.
// The kernel boundary orders the two.  (A single kernel whose last block per
// row merges needs a device-scope release per block, which on this GPU writes
// back the XCD's L2 each time and measured slower than the second launch.)
// ---------------------------------------------------------------------------
template <typename T, bool ROBUST, int THREADS, int U>
__global__ __launch_bounds__(THREADS) void lse_fwd_split_partials(const T* __restrict__ x, int64_t N, int64_t seg,
                                                                  float2* __restrict__ part) {
    constexpr int VE = Elem<T>::kVec;
    constexpr int WAVES = THREADS / 64;
    __shared__ float sh_m[WAVES], sh_s[WAVES];
    const int tid = threadIdx.x;
    const int S = (int)gridDim.x;
    const int k = (int)blockIdx.x;
    const int64_t row = blockIdx.y;
    const T* p = x + row * N;
    const RowSplit sp = split_row(p, N);
    float m = -kInf, s = 0.0f;
    if (k == 0) {
        if (tid < sp.head) fold_scalar<T, ROBUST>(m, s, p + tid);
        if (tid < sp.tail) fold_scalar<T, ROBUST>(m, s, p + sp.head + sp.nvec * VE + tid);
    }
    const int64_t v0 = (int64_t)k * seg;
    const int64_t v1 = v0 + seg < sp.nvec ? v0 + seg : sp.nvec;
    fold_body<T, ROBUST, THREADS, U>(m, s, reinterpret_cast<const char*>(p + sp.head + v0 * VE), (v1 - v0) * 16, tid * 16,
                                     tid, v1 - v0, batches<(int64_t)U * THREADS>(v1 - v0));
    group_merge<64>(m, s);
    if ((tid & 63) == 0) {
        sh_m[tid >> 6] = m;
        sh_s[tid >> 6] = s;
    }
    __syncthreads();
    if (tid < 64) {
        m = tid < WAVES ? sh_m[tid] : -kInf;
        s = tid < WAVES ? sh_s[tid] : 0.0f;
        group_merge<WAVES>(m, s);
        if (tid == 0) part[row * S + k] = make_float2(m, s);
    }
}

// LPR lanes per row (LPR >= S), 64/LPR rows per wave, 4 waves per block.
template <bool ROBUST, int LPR, typename OUT>
__global__ __launch_bounds__(256) void lse_fwd_split_merge(const float2* __restrict__ part, OUT out, int64_t B,
                                                           int S) {
    const int j = (int)(threadIdx.x % LPR);
    const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
    typename OUT::Row orow{};
    if (j == 0 && row < B) orow = out.begin(row);
    float m = -kInf, s = 0.0f;
    if (row < B && j < S) {
        const float2 pv = part[row * S + j];
        m = pv.x;
        s = pv.y;
    }
    group_merge<LPR>(m, s);
    if (j == 0 && row < B) out.end(row, orow, lse_finish<ROBUST>(m, s));
}

// The split is used for B < kSplitMaxRows and rows of more than 4096 body
// vectors, except for kOnePassRowsLo <= B <= kOnePassRowsHi: there
// each CU holds at most one 512-thread block of the one-pass kernel, which
// then streams without a partial second round of blocks and beats the split
// plus its merge.  S (<= 64) aims at kSplitBlocks blocks in all, with
// segments of at least kSplitMinVecs vectors, rounded to whole batches of the
// block.  Measured at N = 128256 fp32 (one-pass / split, us): B=96 15.9 /
// 11.9, 160 17.1 / 16.7, 192 18.1 / 19.1, 256 22.2 / 23.9, 288 30.4 / 27.0,
// 320 31.1 / 31.1.
constexpr int kSplitThreads = 256;
constexpr int kSplitU = 2;
constexpr int64_t kSplitMaxRows = 320;
constexpr int64_t kSplitBlocks = 2048;
constexpr int64_t kSplitMinVecs = 1024;
constexpr int64_t kOnePassRowsLo = 192, kOnePassRowsHi = 256;

struct SplitPlan {
    int64_t S, seg;
};

static SplitPlan split_plan(int64_t B, int64_t N, int64_t ve, int64_t max_rows, int64_t blocks, int64_t min_vecs,
                            int64_t fold) {
    const int64_t vecs = (N + ve - 1) / ve;  // >= the body vectors of any alignment
    if (B <= 0 || B >= max_rows || B > 65535 || vecs <= 4096) return {1, 0};
    if (B >= kOnePassRowsLo && B <= kOnePassRowsHi) return {1, 0};
    int64_t S = (blocks + B - 1) / B;
    if (S > 64) S = 64;
    if (S > vecs / min_vecs) S = vecs / min_vecs;
    if (S < 2) return {1, 0};
    int64_t seg = (vecs + S - 1) / S;
    seg = (seg + fold - 1) / fold * fold;
    S = (vecs + seg - 1) / seg;
    if (S < 2) return {1, 0};
    return {S, seg};
}

static SplitPlan default_split_plan(int64_t B, int64_t N, int64_t elem_bytes) {
    return split_plan(B, N, 16 / elem_bytes, kSplitMaxRows, kSplitBlocks, kSplitMinVecs,
                      (int64_t)kSplitThreads * kSplitU);
}

static int64_t split_ws_bytes(int64_t B, const SplitPlan& pl) {
    return pl.S < 2 ? 0 : B * pl.S * (int64_t)sizeof(float2);
}

template <bool ROBUST, typename OUT>
static void launch_split_merge(const float2* part, OUT out, int64_t B, int S, hipStream_t st) {
    int lpr = 4;
    while (lpr < S) lpr <<= 1;
    const int64_t rpb = 256 / lpr;
    const dim3 g((unsigned)((B + rpb - 1) / rpb)), blk(256);
    switch (lpr) {
    case 4: lse_fwd_split_merge<ROBUST, 4, OUT><<<g, blk, 0, st>>>(part, out, B, S); break;
    case 8: lse_fwd_split_merge<ROBUST, 8, OUT><<<g, blk, 0, st>>>(part, out, B, S); break;
    case 16: lse_fwd_split_merge<ROBUST, 16, OUT><<<g, blk, 0, st>>>(part, out, B, S); break;
    case 32: lse_fwd_split_merge<ROBUST, 32, OUT><<<g, blk, 0, st>>>(part, out, B, S); break;
    default: lse_fwd_split_merge<ROBUST, 64, OUT><<<g, blk, 0, st>>>(part, out, B, S); break;
    }
}

template <typename T, bool ROBUST, int THREADS, int U, typename OUT>
static void launch_split(const T* x, OUT out, int64_t B, int64_t N, const SplitPlan& pl, void* ws, hipStream_t st) {
    float2* part = static_cast<float2*>(ws);
    lse_fwd_split_partials<T, ROBUST, THREADS, U>
        <<<dim3((unsigned)pl.S, (unsigned)B), dim3(THREADS), 0, st>>>(x, N, pl.seg, part);
    launch_split_merge<ROBUST>(part, out, B, (int)pl.S, st);
}

static int64_t pow2_ceil(int64_t v) {
    int64_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

template <typename T, bool ROBUST, int LPR, int U, bool PIPE, typename OUT>
static void launch_group(const T* x, OUT out, int64_t B, int64_t N, hipStream_t st) {
    const int64_t rows_per_block = 4 * (64 / LPR);
    const int64_t grid = grid_stride_blocks((B + rows_per_block - 1) / rows_per_block, 256);
    lse_fwd_group_rows<T, ROBUST, LPR, U, PIPE, OUT><<<dim3((unsigned)grid), dim3(256), 0, st>>>(x, out, B, N);
}

// Dynamic LDS (bytes) for each block of a launch to reserve, unused, so that
// at most `cap` of its blocks share a CU: a little more than a (cap + 1)-th of
// the CU's LDS.  Read once per device; 0 (no reservation) where the device's
// LDS size cannot be read.  The kernels' own LDS is a few words.
constexpr int kLdsDevices = 64;
static std::mutex g_lds_mu;
static int g_lds_per_cu[kLdsDevices];  // guarded by g_lds_mu; 0 until read

static unsigned lds_reserve_for(int cap) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLdsDevices) return 0;
    int lds;
    {
        std::lock_guard<std::mutex> lock(g_lds_mu);
        if (g_lds_per_cu[dev] == 0) {
            int v = 0;
            if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
                v <= 0)
                return 0;
            g_lds_per_cu[dev] = v;
        }
        lds = g_lds_per_cu[dev];
    }
    const int r = lds / (cap + 1) + 64;
    return r <= 65536 ? (unsigned)r : 0u;  // a launch's dynamic LDS stays within 64 KB
}

// cap > 0: at most `cap` blocks per CU (lds_reserve_for).
template <typename T, bool ROBUST, int THREADS, int U, bool PIPE, typename OUT>
static void launch_block(const T* x, OUT out, int64_t B, int64_t N, hipStream_t st, int64_t keep_rows, int cap = 0) {
    const int64_t grid = grid_stride_blocks(B, THREADS);
    const unsigned lds = cap > 0 ? lds_reserve_for(cap) : 0u;
    if (keep_rows > 0)
        lse_fwd_block_rows<T, ROBUST, THREADS, U, PIPE, OUT, true>
            <<<dim3((unsigned)grid), dim3(THREADS), lds, st>>>(x, out, B, N, keep_rows);
    else
        lse_fwd_block_rows<T, ROBUST, THREADS, U, PIPE, OUT>
            <<<dim3((unsigned)grid), dim3(THREADS), lds, st>>>(x, out, B, N, 0);
}

// Geometry and loop per shape ("vectors" = 16-byte vectors per row), from
// same-process sweeps of both loops over 256..1024-thread blocks and 4..64
// lanes per row on MI355X.  The pipelined loop wins wherever a row is more
// than a few hundred vectors long: for fp16 / bf16, whose fold costs twice
// the ALU work per byte, by 3-10% on many rows and by up to 39% on few
// mid-length rows.  Short rows keep the burst loop, 2-10% ahead there.
// keep_rows > 0: the one-block-per-row launches load rows below it with
// kLoadKeepAux (the row-group launches keep nt).
template <typename T, bool ROBUST, typename OUT>
static void launch_fwd(const T* x, OUT out, int64_t B, int64_t N, hipStream_t st, int64_t keep_rows) {
    constexpr int VE = Elem<T>::kVec;
    constexpr bool kHalf = VE == 8;
    const int64_t vecs = (N + VE - 1) / VE;
    if (vecs > 4096) {
        // Long rows, one block per row.  fp16/bf16: 512 threads x 4 loads per
        // batch (1-1.5% ahead of x 2 at (2048, 128256)).  fp32 by row count
        // (N = 128256): 512 x 2 below 512 rows (22% ahead of the burst loop
        // at 256), 256 x 2 below 768 (0.8% ahead at 512), 1024 x 1 from 768
        // (best from 768 to 8184 rows, 1.5-4% ahead of 256 x 2 at 1024 and
        // of the burst loop at (2046, 256128) and (8184, 50257)).
        if constexpr (kHalf)
            launch_block<T, ROBUST, 512, 4, true, OUT>(x, out, B, N, st, keep_rows);
        else if (B < 512)
            launch_block<T, ROBUST, 512, 2, true, OUT>(x, out, B, N, st, keep_rows);
        else if (B < 768)
            launch_block<T, ROBUST, 256, 2, true, OUT>(x, out, B, N, st, keep_rows);
        else
            launch_block<T, ROBUST, 1024, 1, true, OUT>(x, out, B, N, st, keep_rows);
        return;
    }
    if (vecs > 1024 && B <= 1024) {
        // Few mid-length rows: a wave per row would leave the GPU
        // under-filled, so one block per row; 128 threads for fp16/bf16 up
        // to 2048 vectors (2-8% ahead of 256), 256 otherwise.
        if (kHalf && vecs <= 2048)
            launch_block<T, ROBUST, 128, 2, true, OUT>(x, out, B, N, st, keep_rows);
        else
            launch_block<T, ROBUST, 256, 2, true, OUT>(x, out, B, N, st, keep_rows);
        return;
    }
    if (vecs > 512) {
        // Many mid-length rows: fp32 takes a 256-thread block per row (4%
        // ahead of a wave per row at 1024 vectors, 2% at 4000).  fp16/bf16:
        // from 4096 rows of more than 2048 vectors, a 256-thread block per
        // row in batches of 4 (2-3% ahead of a wave per row at (4096, 32000)
        // and (8192, 24000), but 3% behind at (2048, 20000); 512 threads lose
        // 19% at 3000 vectors); 32 lanes per row for 1025..2048 vectors (3%
        // ahead at 2000); otherwise a wave per row.  The fp16 block kernel
        // (96 VGPRs: five blocks fit a CU) runs at most 3 blocks per CU: fewer
        // rows streamed at once per CU measured faster (medians of three
        // rounds, us, 5 / 4 / 3 / 2 blocks: (4096, 32000) 41.16 / 40.64 /
        // 40.49 / 42.30, (8192, 24000) 58.97 / 57.86 / 56.28 / 63.69,
        // (4096, 20000) 27.09 / 26.60 / 26.48 / 31.33).  bf16 (110 VGPRs,
        // four blocks) stays as it is: 3 blocks measured 0.8% and 2.6%
        // faster at the first two shapes and 4.1% slower at the third.
        if constexpr (!kHalf)
            launch_block<T, ROBUST, 256, 2, true, OUT>(x, out, B, N, st, keep_rows);
        else if (vecs > 2048 && B >= 4096)
            launch_block<T, ROBUST, 256, 4, true, OUT>(x, out, B, N, st, keep_rows,
                                                       __is_same(T, _Float16) ? 3 : 0);
        else if (vecs > 1024 && vecs <= 2048)
            launch_group<T, ROBUST, 32, 4, true, OUT>(x, out, B, N, st);
        else
            launch_group<T, ROBUST, 64, 4, true, OUT>(x, out, B, N, st);
        return;
    }
    if (vecs < 16) {
        // a few vectors per row: 4 lanes per row, one masked batch of 2
        // (22% ahead of the burst loop at 8 vectors)
        launch_group<T, ROBUST, 4, 2, true, OUT>(x, out, B, N, st);
        return;
    }
    // Short rows: LPR lanes per row, about 4 vectors per lane in one burst.
    int64_t lpr = pow2_ceil((vecs + 3) / 4);
    if (lpr < 4) lpr = 4;
    if (lpr > 64) lpr = 64;
    switch (lpr) {
    case 4: launch_group<T, ROBUST, 4, 4, false, OUT>(x, out, B, N, st); break;
    case 8: launch_group<T, ROBUST, 8, 4, false, OUT>(x, out, B, N, st); break;
    case 16: launch_group<T, ROBUST, 16, 4, false, OUT>(x, out, B, N, st); break;
    case 32: launch_group<T, ROBUST, 32, 4, false, OUT>(x, out, B, N, st); break;
    default: launch_group<T, ROBUST, 64, 4, false, OUT>(x, out, B, N, st); break;
    }
}

// Rows the keeping forward loads with kLoadKeepAux: the first three quarters
// of x, at most 240 MiB.  Same-process sweeps of the forward then the backward
// on the same batch (backward after the keeping forward, against after the nt
// forward): fp32 (512, 128256) 123.8 -> 118.6 us with 384 of 512 rows (all
// 512: 120.7, the forward alone 11% slower), fp32 (256, 128256) 67.1 ->
// 64.1 us with 192 of 256, bf16 (2048, 128256) 238.6 -> 232.8 us with 1024 of
// 2048 (250 MiB; 1536 rows: 235.5).  The backward's gain grows with the rows
// kept, the forward's cost faster beyond about three quarters of x.
constexpr int64_t kKeepMaxBytes = (int64_t)240 << 20;

static int64_t keep_rows_for(int64_t B, int64_t row_bytes) {
    if (row_bytes <= 0) return 0;
    int64_t budget = B * row_bytes / 4 * 3;
    if (budget > kKeepMaxBytes) budget = kKeepMaxBytes;
    return budget / row_bytes;
}

// ws == nullptr: the one-pass kernels for every shape.  Otherwise the split
// kernels where default_split_plan() chooses them, with ws_bytes checked
// against what that plan needs.  keep: the one-pass kernels load the rows
// keep_rows_for() gives with kLoadKeepAux (the split kernels ignore it).
// Argument checks other than x's are the caller's.
template <typename T, typename OUT>
static int fwd_launch(const char* name, const T* x, OUT out, int64_t B, int64_t N, int robust, void* ws,
                      size_t ws_bytes, hipStream_t st, bool keep = false) {
    FL_CHECK(x != nullptr || N == 0, "%s: x is NULL", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) % sizeof(T)) == 0, "%s: x is not element-aligned", name);
    const SplitPlan pl = ws ? default_split_plan(B, N, (int64_t)sizeof(T)) : SplitPlan{1, 0};
    if (pl.S >= 2) {
        const int64_t need = split_ws_bytes(B, pl);
        FL_CHECK((int64_t)ws_bytes >= need, "%s: workspace of %llu bytes, %lld needed", name,
                 (unsigned long long)ws_bytes, (long long)need);
        FL_CHECK((reinterpret_cast<uintptr_t>(ws) & 7u) == 0, "%s: workspace is not 8-byte aligned", name);
        if (robust)
            launch_split<T, true, kSplitThreads, kSplitU>(x, out, B, N, pl, ws, st);
        else
            launch_split<T, false, kSplitThreads, kSplitU>(x, out, B, N, pl, ws, st);
    } else {
        const int64_t keep_rows = keep ? keep_rows_for(B, N * (int64_t)sizeof(T)) : 0;
        if (robust)
            launch_fwd<T, true>(x, out, B, N, st, keep_rows);
        else
            launch_fwd<T, false>(x, out, B, N, st, keep_rows);
    }
    return launch_status(name);
}

template <typename T>
static int fwd_entry(const char* name, const T* x, float* out, int64_t B, int64_t N, int robust, void* ws,
                     size_t ws_bytes, void* stream, bool keep = false) {
    FL_CHECK(B >= 0 && N >= 0, "%s: negative shape (B=%lld, N=%lld)", name, (long long)B, (long long)N);
    if (B == 0) return ok();
    FL_CHECK(out != nullptr, "%s: out is NULL", name);
    return fwd_launch<T>(name, x, LseOut{out}, B, N, robust, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream),
                         keep);
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bwd_elem(float gv, float lse, float xv) {
    return gv * fexp2((xv - lse) * kLog2e);
}

// grad * exp(x - lse) over one vector of VE values, in place.  For |lse| < 64
// the exponent is one FMA, x*log2e - lse*log2e, whose shared rounding of
// lse*log2e costs at most 64*log2e*2^-24 (4e-6 relative); larger |lse| use
// the exact difference.
template <int VE>
__device__ __forceinline__ void bwd_vals(float gv, float lv, bool fma_ok, float (&v)[VE]) {
    if (fma_ok) {
        const float nb = -lv * kLog2e;
#pragma unroll
        for (int k = 0; k < VE; ++k) v[k] = gv * fexp2(__builtin_fmaf(v[k], kLog2e, nb));
    } else {
#pragma unroll
        for (int k = 0; k < VE; ++k) v[k] = bwd_elem(gv, lv, v[k]);
    }
}

// Backward targets.  LseGrad: grad_x = g * softmax.  SelGrad (selective
// log-softmax, logp = x[t] - lse): grad_x = g * (onehot(t) - softmax), i.e.
// the softmax term with -g plus g at column t; an index outside [0, N) adds
// nothing (its forward was NaN).
struct LseGrad {
    static constexpr bool kSel = false;
    __device__ __forceinline__ float coef(int64_t, float gv) const { return gv; }
    __device__ __forceinline__ int64_t target(int64_t) const { return -1; }
};
struct SelGrad {
    static constexpr bool kSel = true;
    const int64_t* __restrict__ index;
    __device__ __forceinline__ float coef(int64_t, float gv) const { return -gv; }
    __device__ __forceinline__ int64_t target(int64_t row) const { return index[row]; }
};

// SEL: adds gv to the element of r that sits at column t, if any; c0 is the
// column of r[0].
template <bool SEL, int VE>
__device__ __forceinline__ void add_at(float (&r)[VE], int64_t c0, int64_t t, float gv) {
    if constexpr (SEL) {
        const int64_t d = t - c0;
        if ((uint64_t)d < (uint64_t)VE) {
#pragma unroll
            for (int k = 0; k < VE; ++k) r[k] += d == k ? gv : 0.0f;
        }
    }
}

// One element at column c of a row (scalar head / tail / fallback paths).
template <typename T, typename GR>
__device__ __forceinline__ void bwd_one(T* gr, const T* xr, int64_t c, float gv, float lv, int64_t t, float g0) {
    Elem<T>::put(gr + c, bwd_elem(gv, lv, Elem<T>::scalar(xr + c)) + (GR::kSel && c == t ? g0 : 0.0f));
}

// Destination of a row body's 16-byte result vectors.  BUF: a buffer
// resource over the body, stored with kStoreStreamAux (rows under 2 GiB);
// otherwise plain nontemporal pointer stores.
template <typename T, bool BUF>
struct RowOut {
    T* body;
    __amdgpu_buffer_rsrc_t rsrc;
    __device__ __forceinline__ RowOut(T* b, int64_t nvec) : body(b) {
        if constexpr (BUF)
            rsrc = __builtin_amdgcn_make_buffer_rsrc(b, 0, (int)(nvec * 16), 0x00020000);
    }
    __device__ __forceinline__ void put(int64_t i, const float (&v)[Elem<T>::kVec]) const {
        if constexpr (BUF)
            Elem<T>::put_vec_buf(rsrc, (int)(i * 16), v);
        else
            Elem<T>::put_vec(body + i * Elem<T>::kVec, v);
    }
};

// One 16-byte vector i of a row body whose first column is head.
template <typename T, typename GR, bool BUF>
__device__ __forceinline__ void bwd_vec(const RowOut<T, BUF>& dst, const T* body_x, int64_t i, int64_t head, float gv,
                                        float lv, bool fma_ok, int64_t t, float g0) {
    constexpr int VE = Elem<T>::kVec;
    float v[VE];
    Elem<T>::vec(body_x + i * VE, v);
    bwd_vals<VE>(gv, lv, fma_ok, v);
    add_at<GR::kSel, VE>(v, head + VE * i, t, g0);
    dst.put(i, v);
}

// Long rows: grid = B * chunks_per_row blocks of 256 threads; a block covers
// 256*U consecutive vectors of one row.  x and grad_x share their alignment.
// With GRAN, the chunks of a row sit on absolute 256*U*16-byte boundaries of
// x: chunk k covers the body vectors [k*256*U - ph, (k+1)*256*U - ph), ph
// being the body's first vector's place in its granule, and the grid holds
// one more chunk per row.
template <typename T, int U, bool GRAN, typename GR, bool BUF>
__global__ __launch_bounds__(256) void lse_bwd_row_chunks(const float* __restrict__ g, const T* __restrict__ x,
                                                          const float* __restrict__ lse, T* __restrict__ gx,
                                                          int64_t N, int64_t chunks_per_row, GR gr_t,
                                                          int64_t block0) {
    constexpr int VE = Elem<T>::kVec;
    const int64_t blk = block0 + blockIdx.x;
    const int64_t row = blk / chunks_per_row;
    const int64_t chunk = blk - row * chunks_per_row;
    const int tid = threadIdx.x;
    const T* xr = x + row * N;
    T* gr = gx + row * N;
    const RowSplit sp = split_row(xr, N);
    const float g0 = g[row];
    const float gv = gr_t.coef(row, g0);
    const int64_t t = gr_t.target(row);
    const float lv = lse[row];
    if (chunk == 0) {
        if (tid < sp.head) bwd_one<T, GR>(gr, xr, tid, gv, lv, t, g0);
        if (tid < sp.tail) bwd_one<T, GR>(gr, xr, sp.head + sp.nvec * VE + tid, gv, lv, t, g0);
    }
    const T* xb = xr + sp.head;
    const RowOut<T, BUF> gb(gr + sp.head, sp.nvec);
    const bool fma_ok = __builtin_fabsf(lv) < 64.0f;
    const int64_t ph = GRAN ? (int64_t)((reinterpret_cast<uintptr_t>(xb) >> 4) & (256 * U - 1)) : 0;
    const int64_t i0 = chunk * 256 * U + tid - ph;
    if constexpr (U == 1) {
        if ((!GRAN || i0 >= 0) && i0 < sp.nvec) bwd_vec<T, GR>(gb, xb, i0, sp.head, gv, lv, fma_ok, t, g0);
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * 256;
            if ((!GRAN || i >= 0) && i < sp.nvec) bwd_vec<T, GR>(gb, xb, i, sp.head, gv, lv, fma_ok, t, g0);
        }
    }
}

// Rows of at least 1 KB, x and grad_x 16-byte aligned: the matrix is one
// flat run of 16-byte vectors, taken 64 at a time (1 KB) by one-wave blocks
// in order.  A block's vectors span at most two rows, and each lane takes its
// own row's gradient, LSE and target.  STRADDLE, for rows that are not whole
// vectors (the element count of the matrix still a multiple of the vector's):
// a vector may end one row and start the next, and its lane computes the
// elements of each row with that row's values.
template <typename T, typename GR, bool STRADDLE>
__global__ __launch_bounds__(64) void lse_bwd_flat(const float* __restrict__ g, const T* __restrict__ x,
                                                   const float* __restrict__ lse, T* __restrict__ gx, int64_t N,
                                                   int64_t total_vecs, GR gr_t, int64_t block0) {
    constexpr int VE = Elem<T>::kVec;
    const int64_t v0 = (block0 + (int64_t)blockIdx.x) * 64;
    const int64_t row0 = v0 * VE / N;
    const int l = threadIdx.x;
    const int64_t v = v0 + l;
    if (v >= total_vecs) return;
    const int64_t e = v * VE;
    const int64_t row = e >= (row0 + 1) * N ? row0 + 1 : row0;
    const float g0 = g[row];
    const float gv = gr_t.coef(row, g0);
    const int64_t t = gr_t.target(row);
    const float lv = lse[row];
    const int64_t left = total_vecs - v0;
    const int nrec = (left < 64 ? (int)left : 64) * 16;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(x + v0 * VE), 0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(gx + v0 * VE, 0, nrec, 0x00020000);
    float vals[VE];
    Elem<T>::cvt(__builtin_amdgcn_raw_buffer_load_b128(rx, l * 16, 0, kLoadStreamAux), vals);
    if constexpr (STRADDLE) {
        // elements of this vector in `row`; the rest start row + 1, which
        // exists: the vector lies inside the matrix
        const int64_t k0 = (row + 1) * N - e;
        if (k0 < VE) {
            float nxt[VE];
#pragma unroll
            for (int k = 0; k < VE; ++k) nxt[k] = vals[k];
            const float g1 = g[row + 1];
            const float lv1 = lse[row + 1];
            bwd_vals<VE>(gr_t.coef(row + 1, g1), lv1, __builtin_fabsf(lv1) < 64.0f, nxt);
            add_at<GR::kSel, VE>(nxt, -k0, gr_t.target(row + 1), g1);
            bwd_vals<VE>(gv, lv, __builtin_fabsf(lv) < 64.0f, vals);
            add_at<GR::kSel, VE>(vals, e - row * N, t, g0);
#pragma unroll
            for (int k = 0; k < VE; ++k) vals[k] = k < k0 ? vals[k] : nxt[k];
            Elem<T>::put_vec_buf(ry, l * 16, vals);
            return;
        }
    }
    bwd_vals<VE>(gv, lv, __builtin_fabsf(lv) < 64.0f, vals);
    add_at<GR::kSel, VE>(vals, e - row * N, t, g0);
    Elem<T>::put_vec_buf(ry, l * 16, vals);
}

// Short rows: LPR lanes per row, 256/LPR rows per block, grid-stride.
template <typename T, int LPR, typename GR, bool BUF>
__global__ __launch_bounds__(256) void lse_bwd_group_rows(const float* __restrict__ g, const T* __restrict__ x,
                                                          const float* __restrict__ lse, T* __restrict__ gx,
                                                          int64_t B, int64_t N, GR gr_t) {
    constexpr int VE = Elem<T>::kVec;
    constexpr int RPB = 256 / LPR;
    const int gi = threadIdx.x / LPR;
    const int j = threadIdx.x % LPR;
    for (int64_t row = (int64_t)blockIdx.x * RPB + gi; row < B; row += (int64_t)gridDim.x * RPB) {
        const T* xr = x + row * N;
        T* gr = gx + row * N;
        const RowSplit sp = split_row(xr, N);
        const float g0 = g[row];
        const float gv = gr_t.coef(row, g0);
        const int64_t t = gr_t.target(row);
        const float lv = lse[row];
        for (int64_t h = j; h < sp.head; h += LPR) bwd_one<T, GR>(gr, xr, h, gv, lv, t, g0);
        const int64_t t0 = sp.head + sp.nvec * VE;
        for (int64_t c = j; c < sp.tail; c += LPR) bwd_one<T, GR>(gr, xr, t0 + c, gv, lv, t, g0);
        const bool fma_ok = __builtin_fabsf(lv) < 64.0f;
        const RowOut<T, BUF> gb(gr + sp.head, sp.nvec);
        for (int64_t i = j; i < sp.nvec; i += LPR) bwd_vec<T, GR>(gb, xr + sp.head, i, sp.head, gv, lv, fma_ok, t, g0);
    }
}

// Fallback when x and grad_x differ in 16-byte alignment: scalar grid-stride.
template <typename T, typename GR>
__global__ __launch_bounds__(256) void lse_bwd_scalar(const float* __restrict__ g, const T* __restrict__ x,
                                                      const float* __restrict__ lse, T* __restrict__ gx,
                                                      int64_t B, int64_t N, GR gr_t) {
    for (int64_t row = blockIdx.y; row < B; row += gridDim.y) {
        const float g0 = g[row];
        const float gv = gr_t.coef(row, g0);
        const int64_t t = gr_t.target(row);
        const float lv = lse[row];
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < N; i += (int64_t)gridDim.x * 256)
            bwd_one<T, GR>(gx + row * N, x + row * N, i, gv, lv, t, g0);
    }
}

template <typename T, typename GR, bool BUF>
static void launch_bwd_vec(const float* g, const T* x, const float* lse, T* gx, int64_t B, int64_t N, GR gr_t,
                           hipStream_t st) {
    constexpr int VE = Elem<T>::kVec;
    const int64_t vecs = N / VE + 1;
    const int64_t row_bytes = N * (int64_t)sizeof(T);
    // Whole-vector rows of 1 KB or more: the flat kernel, in the order of the
    // fastest plain copy of the same buffers.  Against the row-chunk kernels
    // below: (512, 128256) 79.2 -> 78.3 us, bf16 (2048, 128256) 159.6 ->
    // 155.8, fp16 (16384, 8000) 86.1 -> 78.5, (262144, 256) 83.4 -> 80.8.
    // Rows that are not whole vectors take the flat kernel too when the
    // matrix is a whole number of vectors (some vectors then straddle two
    // rows): gpt-2's vocabulary, fp32 (8184, 50257), 514.8 -> 489.1 us (a
    // copy of the same bytes: 490.9), the selective backward 512.8 -> 489.6.
    if (row_bytes >= 1024 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        const int64_t total_vecs = B * N / VE;
        const int64_t blocks = (total_vecs + 63) / 64;
        if (row_bytes % 16 == 0) {
            for_grid_chunks(blocks, 64, [&](int64_t b0, int64_t nb) {
                lse_bwd_flat<T, GR, false><<<dim3((unsigned)nb), dim3(64), 0, st>>>(g, x, lse, gx, N, total_vecs, gr_t,
                                                                                    b0);
            });
            return;
        }
        if ((B * N) % VE == 0) {
            for_grid_chunks(blocks, 64, [&](int64_t b0, int64_t nb) {
                lse_bwd_flat<T, GR, true><<<dim3((unsigned)nb), dim3(64), 0, st>>>(g, x, lse, gx, N, total_vecs, gr_t,
                                                                                   b0);
            });
            return;
        }
    }
    if (vecs >= 1024) {
        // Rows that are not whole 16-byte vectors: one vector per lane, 256
        // per block (measured best with 128x2 and 1024x1).
        constexpr int U = 1;
        // Rows of at least 32 chunks whose starts do not all fall on 4 KB
        // boundaries take their chunks on absolute 4 KB boundaries: a chunk
        // that straddles one streams slower (fp32 rows of 128257: 87.2 ->
        // 81.3 us).  Shorter rows pay more for the extra chunk per row than
        // they gain (whole-vector rows, before the flat kernel took them:
        // fp32 (8192, 8000) 79.0 -> 81.5).
        const int64_t cpr0 = (vecs + 256 * U - 1) / (256 * U);
        const bool granules =
            cpr0 >= 32 && (((int64_t)N * (int64_t)sizeof(T)) % 4096 != 0 || (reinterpret_cast<uintptr_t>(x) & 4095u) != 0);
        // (a run-time switch measured 1-3% slower on every shape: a wave
        // handles one vector, so the kernel is two instantiations)
        if (granules)
            for_grid_chunks(B * (cpr0 + 1), 256, [&](int64_t b0, int64_t nb) {
                lse_bwd_row_chunks<T, U, true, GR, BUF>
                    <<<dim3((unsigned)nb), dim3(256), 0, st>>>(g, x, lse, gx, N, cpr0 + 1, gr_t, b0);
            });
        else
            for_grid_chunks(B * cpr0, 256, [&](int64_t b0, int64_t nb) {
                lse_bwd_row_chunks<T, U, false, GR, BUF>
                    <<<dim3((unsigned)nb), dim3(256), 0, st>>>(g, x, lse, gx, N, cpr0, gr_t, b0);
            });
        return;
    }
    int64_t lpr = pow2_ceil((vecs + 3) / 4);
    if (lpr < 4) lpr = 4;
    const int64_t rpb = 256 / lpr;
    const int64_t grid = grid_stride_blocks((B + rpb - 1) / rpb, 256);
    const dim3 gd((unsigned)grid), blk(256);
    switch (lpr) {
    case 4: lse_bwd_group_rows<T, 4, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    case 8: lse_bwd_group_rows<T, 8, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    case 16: lse_bwd_group_rows<T, 16, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    case 32: lse_bwd_group_rows<T, 32, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    case 64: lse_bwd_group_rows<T, 64, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    case 128: lse_bwd_group_rows<T, 128, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    default: lse_bwd_group_rows<T, 256, GR, BUF><<<gd, blk, 0, st>>>(g, x, lse, gx, B, N, gr_t); break;
    }
}

template <typename T, typename GR>
static void launch_bwd(const float* g, const T* x, const float* lse, T* gx, int64_t B, int64_t N, GR gr_t,
                       hipStream_t st) {
    const bool same_align = ((reinterpret_cast<uintptr_t>(x) ^ reinterpret_cast<uintptr_t>(gx)) & 15u) == 0;
    if (!same_align) {
        int64_t gxdim = (N + 255) / 256;
        if (gxdim > 1024) gxdim = 1024;
        int64_t gydim = B < 65535 ? B : 65535;
        lse_bwd_scalar<T><<<dim3((unsigned)gxdim, (unsigned)gydim), dim3(256), 0, st>>>(g, x, lse, gx, B, N, gr_t);
        return;
    }
    // buffer stores take 32-bit offsets: rows of 2 GiB or more keep pointer stores
    if (N * (int64_t)sizeof(T) < ((int64_t)1 << 31))
        launch_bwd_vec<T, GR, true>(g, x, lse, gx, B, N, gr_t, st);
    else
        launch_bwd_vec<T, GR, false>(g, x, lse, gx, B, N, gr_t, st);
}

template <typename T, typename GR>
static int bwd_entry(const char* name, const float* grad, const T* x, const float* lse, T* grad_x, int64_t B,
                     int64_t N, GR gr_t, void* stream) {
    FL_CHECK(B >= 0 && N >= 0, "%s: negative shape (B=%lld, N=%lld)", name, (long long)B, (long long)N);
    if (B == 0 || N == 0) return ok();
    FL_CHECK(grad && x && lse && grad_x, "%s: NULL pointer argument", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) % sizeof(T)) == 0 && (reinterpret_cast<uintptr_t>(grad_x) % sizeof(T)) == 0,
             "%s: x / grad_x are not element-aligned", name);
    launch_bwd<T>(grad, x, lse, grad_x, B, N, gr_t, reinterpret_cast<hipStream_t>(stream));
    return launch_status(name);
}

}  // namespace fl

using namespace fl;

extern "C" int fl_lse_fwd_f32(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<float>("fl_lse_fwd_f32", x, out, B, N, robust, nullptr, 0, stream);
}

extern "C" int fl_lse_fwd_f16(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<_Float16>("fl_lse_fwd_f16", static_cast<const _Float16*>(x), out, B, N, robust, nullptr, 0,
                               stream);
}

extern "C" int fl_lse_fwd_bf16(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<bf16_t>("fl_lse_fwd_bf16", static_cast<const bf16_t*>(x), out, B, N, robust, nullptr, 0,
                             stream);
}

extern "C" int fl_lse_fwd_f32_keep(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<float>("fl_lse_fwd_f32_keep", x, out, B, N, robust, nullptr, 0, stream, true);
}

extern "C" int fl_lse_fwd_f16_keep(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<_Float16>("fl_lse_fwd_f16_keep", static_cast<const _Float16*>(x), out, B, N, robust, nullptr,
                               0, stream, true);
}

extern "C" int fl_lse_fwd_bf16_keep(const void* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    return fwd_entry<bf16_t>("fl_lse_fwd_bf16_keep", static_cast<const bf16_t*>(x), out, B, N, robust, nullptr, 0,
                             stream, true);
}

extern "C" size_t fl_lse_fwd_workspace_bytes(int64_t B, int64_t N, int elem_bytes) {
    if (elem_bytes != 2 && elem_bytes != 4) return 0;
    return (size_t)split_ws_bytes(B, default_split_plan(B, N, elem_bytes));
}

extern "C" int fl_lse_fwd_f32_ws(const float* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    return fwd_entry<float>("fl_lse_fwd_f32_ws", x, out, B, N, robust, workspace, workspace_bytes, stream);
}

extern "C" int fl_lse_fwd_f16_ws(const void* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    return fwd_entry<_Float16>("fl_lse_fwd_f16_ws", static_cast<const _Float16*>(x), out, B, N, robust, workspace,
                               workspace_bytes, stream);
}

extern "C" int fl_lse_fwd_bf16_ws(const void* x, float* out, int64_t B, int64_t N, int robust, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    return fwd_entry<bf16_t>("fl_lse_fwd_bf16_ws", static_cast<const bf16_t*>(x), out, B, N, robust, workspace,
                             workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free split forward.  The split plan needs B * S partial pairs with
// B < kSplitMaxRows and S <= 64, at most 319 * 64 * 8 = 163,328 bytes, so one
// static 160 KiB array per GPU holds every plan's partials.  Host code never
// uses the array's name as an address (on the host it is only a stand-in for
// the symbol): each device's address comes from hipGetSymbolAddress, taken on
// the first call with a split shape made with that device current and kept
// only once it succeeded, so a call that failed (for instance one made under
// graph capture) leaves the next call to try again.  Every partial is written
// by the partials kernel before the merge kernel reads it, so the array needs
// no clearing between calls.  Calls on one GPU share the array: calls whose
// work can overlap (different streams of one device) race.
// ---------------------------------------------------------------------------
namespace fl {
constexpr int64_t kNoAllocPairs = 20480;  // 160 KiB of float2
static_assert((kSplitMaxRows - 1) * 64 <= kNoAllocPairs, "static scratch smaller than the largest split plan");
static __device__ __align__(256) float2 scratch[kNoAllocPairs];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // guarded by g_scratch_mu; NULL until an address was taken

// Device address of `scratch` on the current device, which must be the
// device of `stream` (the address is only valid there).
static int scratch_address(const char* name, hipStream_t stream, void** ptr) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(FL_ELAUNCH, "%s: hipGetDevice failed: %s", name, hipGetErrorString(e));
    FL_CHECK(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond the %d the library tracks", name, dev, kMaxDevices);
    if (stream != nullptr) {  // the null stream is the current device's
        int sdev = -1;
        const hipError_t se = hipStreamGetDevice(stream, &sdev);
        if (se != hipSuccess)
            return set_error(FL_EINVAL, "%s: hipStreamGetDevice failed: %s", name, hipGetErrorString(se));
        FL_CHECK(sdev == dev, "%s: the stream belongs to device %d, the current device is %d", name, sdev, dev);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t ge = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (ge != hipSuccess || p == nullptr)
            return set_error(FL_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                             hipGetErrorString(ge));
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return FL_OK;
}
}  // namespace fl

extern "C" int fl_lse_fwd_f32_noalloc(const float* x, float* out, int64_t B, int64_t N, int robust, void* stream) {
    const char* name = "fl_lse_fwd_f32_noalloc";
    FL_CHECK(B >= 0 && N >= 0, "%s: negative shape (B=%lld, N=%lld)", name, (long long)B, (long long)N);
    if (B == 0) return ok();
    FL_CHECK(out != nullptr, "%s: out is NULL", name);
    const int64_t need = split_ws_bytes(B, default_split_plan(B, N, (int64_t)sizeof(float)));
    if (need > (int64_t)sizeof(scratch))
        return set_error(FL_ERANGE, "%s: %lld bytes of partials needed, the static scratch holds %lld", name,
                         (long long)need, (long long)sizeof(scratch));
    void* ws = nullptr;
    if (need > 0) {
        const int rc = scratch_address(name, reinterpret_cast<hipStream_t>(stream), &ws);
        if (rc != FL_OK) return rc;
    }
    return fwd_launch<float>(name, x, LseOut{out}, B, N, robust, ws, sizeof(scratch),
                             reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fl_lse_bwd_f32(const float* grad, const float* x, const float* lse, float* grad_x, int64_t B,
                              int64_t N, void* stream) {
    return bwd_entry<float>("fl_lse_bwd_f32", grad, x, lse, grad_x, B, N, LseGrad{}, stream);
}

extern "C" int fl_lse_bwd_f16(const float* grad, const void* x, const float* lse, void* grad_x, int64_t B, int64_t N,
                              void* stream) {
    return bwd_entry<_Float16>("fl_lse_bwd_f16", grad, static_cast<const _Float16*>(x), lse,
                               static_cast<_Float16*>(grad_x), B, N, LseGrad{}, stream);
}

extern "C" int fl_lse_bwd_bf16(const float* grad, const void* x, const float* lse, void* grad_x, int64_t B,
                               int64_t N, void* stream) {
    return bwd_entry<bf16_t>("fl_lse_bwd_bf16", grad, static_cast<const bf16_t*>(x), lse,
                             static_cast<bf16_t*>(grad_x), B, N, LseGrad{}, stream);
}

extern "C" int fl_selective_logsoftmax_f32(const float* x, const int64_t* index, float* logp, float* lse, int64_t B,
                                           int64_t N, int robust, void* workspace, size_t workspace_bytes,
                                           void* stream) {
    const char* name = "fl_selective_logsoftmax_f32";
    FL_CHECK(B >= 0 && N >= 0, "%s: negative shape (B=%lld, N=%lld)", name, (long long)B, (long long)N);
    if (B == 0) return ok();
    FL_CHECK(index != nullptr && logp != nullptr, "%s: NULL pointer argument", name);
    return fwd_launch<float>(name, x, SelectOut<float>{x, index, logp, lse, N}, B, N, robust, workspace,
                             workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fl_selective_logsoftmax_bwd_f32(const float* grad, const float* x, const int64_t* index,
                                               const float* lse, float* grad_x, int64_t B, int64_t N, void* stream) {
    const char* name = "fl_selective_logsoftmax_bwd_f32";
    FL_CHECK(index != nullptr || B == 0 || N == 0, "%s: NULL pointer argument", name);
    return bwd_entry<float>(name, grad, x, lse, grad_x, B, N, SelGrad{index}, stream);
}
