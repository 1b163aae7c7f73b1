// Streaming row-LSE forward kernels for gfx950 (fp32 / fp16 / bf16 input,
// fp32 accumulation): the per-lane online (max, scaled sum) folds, the
// software-pipelined and burst loops, the row-output policies, and the
// one-block-per-row and row-group kernels.  lse_float.hip launches them; the
// measurement library instantiates the one-block-per-row kernel with a
// recording output policy.
#pragma once

#include <stdint.h>

#include "lse_common.hpp"

namespace fl {

template <typename T, bool ROBUST>
__device__ __forceinline__ void fold_scalar(float& m, float& s, const T* p) {
    float v[1] = {Elem<T>::scalar(p)};
    lse_fold<ROBUST, 1>(m, s, v);
}

// A wave-uniform 64-bit value in scalar registers.  Values the compiler
// computes inside a divergent branch are treated as divergent even when every
// lane holds the same; a buffer resource built from such a value would be
// issued once per distinct value (a waterfall loop).
__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// fp16 fold of raw vectors: the same fp32 operations on the same values as
// lse_fold over the widened elements, from the raw registers.  The maximum is
// taken over the packed halves (exact: widening is monotonic) and each
// exponent widens its element inside the FMA (v_fma_mix_f32).  A batch of 4
// vectors then holds its 16 raw registers, not 32 widened floats beside them.
template <bool ROBUST, int U>
__device__ __forceinline__ void fold_raw_f16(float& m, float& s, const u32x4 (&a)[U]) {
    f16x8 h[U];
#pragma unroll
    for (int u = 0; u < U; ++u) h[u] = __builtin_bit_cast(f16x8, a[u]);
    f16x8 mx = h[0];
#pragma unroll
    for (int u = 1; u < U; ++u) mx = __builtin_elementwise_maximum(mx, h[u]);
    const f16x4 m4 = __builtin_elementwise_maximum(__builtin_shufflevector(mx, mx, 0, 1, 2, 3),
                                               __builtin_shufflevector(mx, mx, 4, 5, 6, 7));
    const f16x2 m2 = __builtin_elementwise_maximum(__builtin_shufflevector(m4, m4, 0, 1),
                                               __builtin_shufflevector(m4, m4, 2, 3));
    const float b = lse_rebase<ROBUST>(m, s, fmaxf((float)m2[0], (float)m2[1]));
    // Only the fused exponent: the base is an fp16 value (|b| <= 65504) or
    // 0, or, in the plain fold of non-finite inputs, +-inf, where the fused
    // and the exact forms give the same 0 or NaN for every element.
    const float nb = -b * kLog2e;
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc += lse_exp_fused((float)h[u][k], nb);
    s += acc;
}

// Folds the raw vectors a[0..U) into (m, s) with one rescale.
template <typename T, bool ROBUST, int U>
__device__ __forceinline__ void fold_raw(float& m, float& s, const u32x4 (&a)[U]) {
    if constexpr (__is_same(T, _Float16)) {
        fold_raw_f16<ROBUST, U>(m, s, a);
    } else {
        constexpr int VE = Elem<T>::kVec;
        float v[U * VE];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float t[VE];
            Elem<T>::cvt(a[u], t);
#pragma unroll
            for (int k = 0; k < VE; ++k) v[u * VE + k] = t[k];
        }
        lse_fold<ROBUST, U * VE>(m, s, v);
    }
}

// Folds the vectors body[i], body[i + STRIDE], ... (i < nvec) into (m, s),
// U vectors per rescale, one burst of U loads at a time: each iteration
// issues its U loads and folds them once they land.  Where other waves cover
// the load latency (fp32 rows, short rows) this beats the pipelined loop
// below, whose extra loads in flight measured 2-10% slower there.  `nfull`,
// wave-uniform, counts the bursts that are whole for every lane of the wave;
// the lanes' remaining vectors then come as masked bursts, their loads past
// the end reading the lane's first remaining vector and folded as -inf (the
// robust fold, as in fold_last).  With a per-lane loop bound instead, the
// lanes of a row with whole and partial bursts ran them one after the other,
// each waiting for its loads: rows of 200 fp16 elements took 12.6 us at 65536
// rows against 8.0 us.
template <typename T, bool ROBUST, int STRIDE, int U>
__device__ __forceinline__ void fold_body_burst(float& m, float& s, const T* body, int64_t i, int64_t nvec,
                                                int64_t nfull) {
    constexpr int VE = Elem<T>::kVec;
    nfull = uniform64(nfull);
    for (int64_t b = 0; b < nfull; ++b, i += (int64_t)U * STRIDE) {
        u32x4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = load_stream<u32x4>(body + (i + (int64_t)u * STRIDE) * VE);
        fold_raw<T, ROBUST, U>(m, s, r);
    }
    for (; i < nvec; i += (int64_t)U * STRIDE) {
        u32x4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = i + (int64_t)u * STRIDE;
            const bool ok = j < nvec;
            // select on the raw vector: selecting the widened floats holds
            // both copies and costs a wave per SIMD of occupancy
            r[u] = load_stream<u32x4>(body + (ok ? j : i) * VE);
#pragma unroll
            for (int k = 0; k < 4; ++k) r[u][k] = ok ? r[u][k] : Elem<T>::kNegInfBits;
        }
        fold_raw<T, true, U>(m, s, r);
    }
}

// Loads batch t of a lane: its vectors t * STEP + l + u * STRIDE (u < U).
// The batch goes through a buffer resource based at the batch's start
// (wave-uniform, so it lives in scalar registers), which keeps the 32-bit
// offsets small for rows of any length; the resource's range check returns
// zeros, without a memory access, for the bytes past `region`.
template <int STRIDE, int U, int AUX = kLoadStreamAux>
__device__ __forceinline__ void load_batch(u32x4 (&a)[U], const char* base, int64_t region, int lane_off,
                                           int64_t t) {
    constexpr int64_t STEP_BYTES = (int64_t)U * STRIDE * 16;
    const int64_t left = region - t * STEP_BYTES;
    const int nrec = left <= 0 ? 0 : (left > 0x7fffffff ? 0x7fffffff : (int)left);
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base + t * STEP_BYTES), 0, nrec, 0x00020000);
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off + u * STRIDE * 16, 0, AUX);
}

// Folds the last batch: the lane's vectors at or past `count` (counted from
// the batch start) become -inf in their raw form, then the robust fold runs.
// It keeps (m, s) = (-inf, 0) for a lane with nothing yet and equals the
// plain fold on finite values, so both variants use it here.  Masking the raw
// bits first also leaves nothing in common with the whole-batch fold that the
// compiler could hoist above the loads that precede it.
template <typename T, int STRIDE, int U>
__device__ __forceinline__ void fold_last(float& m, float& s, const u32x4 (&a)[U], int l, int64_t count) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool ok = l + (int64_t)u * STRIDE < count;
        const uint32_t ninf = Elem<T>::kNegInfBits;
        v[u] = ok ? a[u] : u32x4{ninf, ninf, ninf, ninf};
    }
    fold_raw<T, true, U>(m, s, v);
}

// Folds the body vectors l, l + STRIDE, ... below `end` of this lane's row
// into (m, s), U vectors per rescale, for a lane l in [0, STRIDE).  Vector v
// of the row lies at base + lane_off + (v - l) * 16, with base wave-uniform;
// `region` bounds the bytes at base that may be read.  The caller passes
// `trips`, a wave-uniform batch count with (trips - 1) * U * STRIDE <= end <=
// trips * U * STRIDE for every row of the wave: batches 0 .. trips - 2 are
// whole for every lane and batch trips - 1 is masked.  The batches are
// software-pipelined: batch t + 1 is issued before batch t is folded, in two
// alternating register sets, so no register copy has to wait for a load in
// flight and each lane keeps 2U loads outstanding while it computes.  The
// sched_barrier after each issue keeps the scheduler from moving the fold
// (and its wait) above the new loads; the uniform trip count keeps every
// branch scalar.  AUX is the loads' cache policy.

template <typename T, bool ROBUST, int STRIDE, int U, int AUX = kLoadStreamAux>
__device__ __forceinline__ void fold_body(float& m, float& s, const char* base, int64_t region, int lane_off, int l,
                                          int64_t end, int64_t trips) {
    constexpr int64_t STEP = (int64_t)U * STRIDE;
    base = reinterpret_cast<const char*>(uniform64(reinterpret_cast<int64_t>(base)));
    region = uniform64(region);
    trips = uniform64(trips);
    if (trips <= 0) return;
    const int64_t count = end - (trips - 1) * STEP;
    u32x4 a[U], c[U];
    load_batch<STRIDE, U, AUX>(a, base, region, lane_off, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (trips == 1) {
        fold_last<T, STRIDE, U>(m, s, a, l, count);
        return;
    }
    int64_t t = 1;  // batches issued
    while (true) {
        load_batch<STRIDE, U, AUX>(c, base, region, lane_off, t);
        __builtin_amdgcn_sched_barrier(0);
        fold_raw<T, ROBUST, U>(m, s, a);
        if (t == trips - 1) {
            fold_last<T, STRIDE, U>(m, s, c, l, count);
            return;
        }
        ++t;
        load_batch<STRIDE, U, AUX>(a, base, region, lane_off, t);
        __builtin_amdgcn_sched_barrier(0);
        fold_raw<T, ROBUST, U>(m, s, c);
        if (t == trips - 1) {
            fold_last<T, STRIDE, U>(m, s, a, l, count);
            return;
        }
        ++t;
    }
}

template <int64_t STEP>
__device__ __forceinline__ int64_t batches(int64_t n) {
    return n > 0 ? (n + STEP - 1) / STEP : 0;
}

// ---------------------------------------------------------------------------
// Row outputs of the forward kernels.  begin(row) runs when a row starts, on
// the lane that later calls end(row, r, lse), so a policy's own loads are in
// flight during the row's reduction.
// ---------------------------------------------------------------------------
struct LseOut {
    float* __restrict__ out;
    struct Row {};
    __device__ __forceinline__ Row begin(int64_t) const { return {}; }
    __device__ __forceinline__ void end(int64_t row, Row, float lse) const { out[row] = lse; }
};

// Selective log-softmax: logp[row] = x[row, index[row]] - lse[row], and lse[row]
// when lse is not NULL.  An index outside [0, N) gives NaN (torch.gather would
// raise); the special values follow from the robust LSE (a +inf target in a
// row whose LSE is +inf gives NaN, as torch.log_softmax does).
template <typename T>
struct SelectOut {
    const T* __restrict__ x;
    const int64_t* __restrict__ index;
    float* __restrict__ logp;
    float* __restrict__ lse;
    int64_t N;
    struct Row {
        float xt;
    };
    __device__ __forceinline__ Row begin(int64_t row) const {
        const int64_t t = index[row];
        return {t >= 0 && t < N ? Elem<T>::scalar(x + row * N + t) : __builtin_nanf("")};
    }
    __device__ __forceinline__ void end(int64_t row, Row r, float l) const {
        if (lse) lse[row] = l;
        logp[row] = r.xt - l;
    }
};

// One block per row (grid-stride over rows).  KEEP: rows below keep_rows load
// with kLoadKeepAux instead of nt, for a backward that reads x next (a
// separate instantiation, so the other kernels are unchanged).
template <typename T, bool ROBUST, int THREADS, int U, bool PIPE, typename OUT, bool KEEP = false>
__global__ __launch_bounds__(THREADS) void lse_fwd_block_rows(const T* __restrict__ x, OUT out, int64_t B,
                                                              int64_t N, int64_t keep_rows) {
    constexpr int VE = Elem<T>::kVec;
    constexpr int WAVES = THREADS / 64;
    __shared__ float sh_m[WAVES], sh_s[WAVES];
    const int tid = threadIdx.x;
    for (int64_t row = blockIdx.x; row < B; row += gridDim.x) {
        typename OUT::Row orow{};
        if (tid == 0) orow = out.begin(row);
        const T* p = x + row * N;
        const RowSplit sp = split_row(p, N);
        float m = -kInf, s = 0.0f;
        if (tid < sp.head) fold_scalar<T, ROBUST>(m, s, p + tid);
        if (tid < sp.tail) fold_scalar<T, ROBUST>(m, s, p + sp.head + sp.nvec * VE + tid);
        if constexpr (PIPE && KEEP) {
            if (row < keep_rows)
                fold_body<T, ROBUST, THREADS, U, kLoadKeepAux>(m, s, reinterpret_cast<const char*>(p + sp.head),
                                                               sp.nvec * 16, tid * 16, tid, sp.nvec,
                                                               batches<(int64_t)U * THREADS>(sp.nvec));
            else
                fold_body<T, ROBUST, THREADS, U>(m, s, reinterpret_cast<const char*>(p + sp.head), sp.nvec * 16,
                                                 tid * 16, tid, sp.nvec, batches<(int64_t)U * THREADS>(sp.nvec));
        } else if constexpr (PIPE)
            fold_body<T, ROBUST, THREADS, U>(m, s, reinterpret_cast<const char*>(p + sp.head), sp.nvec * 16, tid * 16,
                                             tid, sp.nvec, batches<(int64_t)U * THREADS>(sp.nvec));
        else
            fold_body_burst<T, ROBUST, THREADS, U>(m, s, p + sp.head, tid, sp.nvec,
                                                   sp.nvec / ((int64_t)U * THREADS));
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
            if (tid == 0) out.end(row, orow, lse_finish<ROBUST>(m, s));
        }
        __syncthreads();
    }
}

// LPR lanes per row, 64/LPR rows per wave, WAVES waves per block
// (grid-stride over row groups).
template <typename T, bool ROBUST, int LPR, int U, bool PIPE, typename OUT>
__global__ __launch_bounds__(256) void lse_fwd_group_rows(const T* __restrict__ x, OUT out, int64_t B, int64_t N) {
    constexpr int VE = Elem<T>::kVec;
    constexpr int RPW = 64 / LPR;
    constexpr int WAVES = 4;
    constexpr int64_t E = (int64_t)sizeof(T);
    const int lane = threadIdx.x & 63;
    // The pipelined loop builds its buffer resource from the wave's first
    // row, so it needs the wave index in a scalar register; the burst loop
    // measured 2-3% faster (fp16, 256 vectors) with the plain index.
    const int wave = PIPE ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : (int)(threadIdx.x >> 6);
    const int g = lane / LPR;
    const int j = lane % LPR;
    const int64_t step = (int64_t)gridDim.x * WAVES * RPW;
    // Rows of one wave may differ in alignment by one body vector: N / VE
    // bounds every row's count, and the masked last batch covers the
    // difference.
    const int64_t trips = batches<(int64_t)U * LPR>(N / VE);
    // whole bursts for every lane of the wave: with x 16-byte aligned and rows
    // of whole vectors every body holds N / VE vectors, otherwise at least
    // (N - VE + 1) / VE whatever its alignment
    const bool whole_rows = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (N * E) % 16 == 0;
    const int64_t nv_lo = whole_rows ? N / VE : (N >= VE - 1 ? (N - VE + 1) / VE : 0);
    const int64_t nfull = nv_lo / ((int64_t)U * LPR);
    for (int64_t base = ((int64_t)blockIdx.x * WAVES + wave) * RPW; base < B; base += step) {
        const int64_t row = base + g;
        typename OUT::Row orow{};
        if (j == 0 && row < B) orow = out.begin(row);
        float m = -kInf, s = 0.0f;
        if (row < B) {
            const T* p = x + row * N;
            const RowSplit sp = split_row(p, N);
            for (int64_t h = j; h < sp.head; h += LPR) fold_scalar<T, ROBUST>(m, s, p + h);
            const T* tail = p + sp.head + sp.nvec * VE;
            for (int64_t t = j; t < sp.tail; t += LPR) fold_scalar<T, ROBUST>(m, s, tail + t);
            // The loads address the wave's rows [base, base + RPW) through one
            // resource at row `base`; a lane's offset within them stays below
            // RPW * N * E, which the launcher keeps under 2^31 (rows of at
            // most 4096 vectors).
            const int64_t rows = B - base < RPW ? B - base : RPW;
            const int lane_off = (int)(((int64_t)g * N + sp.head) * E) + j * 16;
            if constexpr (PIPE)
                fold_body<T, ROBUST, LPR, U>(m, s, reinterpret_cast<const char*>(x + base * N), rows * N * E, lane_off,
                                             j, sp.nvec, trips);
            else
                fold_body_burst<T, ROBUST, LPR, U>(m, s, p + sp.head, j, sp.nvec, nfull);
        }
        group_merge<LPR>(m, s);
        if (j == 0 && row < B) out.end(row, orow, lse_finish<ROBUST>(m, s));
    }
}

}  // namespace fl
