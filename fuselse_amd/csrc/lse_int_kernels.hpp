// IntLSE fixed-point kernels for gfx950: Q16.16 (fp32 input quantised in the
// kernel, or pre-quantised int32 input) and Q10.6 (int16 input).
//
// The reduction tree is part of the result (the pair op is commutative but not
// associative), so it follows the reference kernels exactly
// (intlse/gpu/lse_kernel.cu:67-159, lse_kernel_q10_6.cu:55-139):
//   * 256 virtual threads per row; virtual thread t folds, in order, its
//     alignment-prefix element (t < prefix), the 4-element vector chunks
//     t, t+256, t+512, ... (elements x, y, z, w), and its suffix element
//     (t < tail); the first element seeds the chain, an empty chain holds the
//     identity -0x3fffffff;
//   * a 32-lane xor butterfly (distances 16, 8, 4, 2, 1) inside each virtual
//     warp of 32;
//   * the 8 warp partials plus 24 identity lanes go through one more 32-lane
//     xor butterfly.
// On wave64 the 256 virtual threads are 4 waves of one 256-thread block; each
// wave's two 32-lane halves are two virtual warps and the xor exchanges are
// ds_swizzle bit-mask moves, which stay inside each half.
//
// Shift semantics: the reference computes M = (1 + frac) >> shift with a
// count that can exceed 31 (or be negative when the difference wraps); NVIDIA
// clamps counts >= 32 (read unsigned) to a zero result.  Here the count is
// clamped unsigned to 31, which gives the same zero for every count >= 17
// because the shifted value is below 2^17.
//
// The 64-entry correction tables live in LDS; the Q10.6 pair op, which depends
// only on the operand gap d and is the identity for d > 384, is read from a
// 386-entry LDS table of (M + LUT) built per block from the same formula.
// Both are built from immediates, without memory loads.
//
// This header holds the kernels; lse_int.hip launches them and the
// measurement library instantiates them with a recording clock policy.
#pragma once

#include <stdint.h>

#include <type_traits>

#include "lse_common.hpp"
#include "lse_pair.hpp"

namespace fl {

// cache-policy bits of the raw buffer loads: nontemporal (streamed once)
constexpr int kBufNT = 2;

// lse_kernel.cu:35-44 (Mitchell-error correction per 1/64 bin, Q16.16)
constexpr int kLutQ16[64] = {
       0,  571,  907, 1282, 1634, 1745, 2054, 2592,
    2900, 2859, 2895, 3015, 3222, 3522, 3922, 4426,
    4617, 4441, 4294, 4178, 4093, 4039, 4018, 4030,
    4076, 4157, 4272, 4424, 4613, 4838, 5102, 5404,
    5399, 5068, 4746, 4435, 4134, 3843, 3562, 3291,
    3031, 2781, 2541, 2312, 2094, 1886, 1689, 1502,
    1327, 1162, 1008,  865,  732,  611,  500,  401,
     312,  235,  168,  113,   69,   35,   13,    2,
};

// lse_kernel_q10_6.cu:27-32 (the same table at 6 fractional bits)
constexpr int kLutQ10[64] = {
    0, 1, 1, 1, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3, 4, 4,
    5, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 5, 5, 5, 5,
    5, 5, 5, 4, 4, 4, 3, 3, 3, 3, 2, 2, 2, 2, 2, 1,
    1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
};

// fl32(fl32(1.44269504089f) * 65536) = 94548.4609375 and
// fl32(0.69314718056f) / 65536, / 64 (lse_kernel.cu:28-30,156).
constexpr float kQ16Conv = 1.44269504089f * 65536.0f;
constexpr float kQ16Out = 0.69314718056f / 65536.0f;
constexpr float kQ10Out = 0.69314718056f / 64.0f;

// __float2int_rn semantics: round half to even, saturate, NaN -> 0
// (v_rndne_f32, then v_cvt_i32_f32, which clamps and maps NaN to 0).
__device__ __forceinline__ int q16_quant(float v) {
    const float r = __builtin_rintf(v * kQ16Conv);
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(r));
    return q;
}

// Element sources for the trees: fp32 quantised in the kernel, int32, int16.
// bload() fetches one 4-element chunk by raw buffer load, unpack() turns it
// into Q values, one() reads a single (prefix or suffix) element.
struct SrcF32 {
    using T = float;
    using Raw = f32x4;
    __device__ static __forceinline__ int cvt(float v) { return q16_quant(v); }
    __device__ static __forceinline__ float sload(__amdgpu_buffer_rsrc_t r, int voff) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
    }
    __device__ static __forceinline__ Raw bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(Raw, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kBufNT));
    }
    __device__ static __forceinline__ void unpack(Raw v, int (&q)[4]) {
        q[0] = q16_quant(v.x); q[1] = q16_quant(v.y); q[2] = q16_quant(v.z); q[3] = q16_quant(v.w);
    }
};
struct SrcI32 {
    using T = int32_t;
    using Raw = u32x4;
    __device__ static __forceinline__ int cvt(int32_t v) { return v; }
    __device__ static __forceinline__ int32_t sload(__amdgpu_buffer_rsrc_t r, int voff) {
        return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0);
    }
    __device__ static __forceinline__ Raw bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(Raw, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kBufNT));
    }
    __device__ static __forceinline__ void unpack(Raw v, int (&q)[4]) {
        q[0] = (int)v.x; q[1] = (int)v.y; q[2] = (int)v.z; q[3] = (int)v.w;
    }
};
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
struct SrcI16 {
    using T = int16_t;
    using Raw = u32x2;
    __device__ static __forceinline__ int cvt(int16_t v) { return (int)v; }
    __device__ static __forceinline__ int16_t sload(__amdgpu_buffer_rsrc_t r, int voff) {
        return (int16_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
    }
    __device__ static __forceinline__ Raw bload(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(Raw, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kBufNT));
    }
    __device__ static __forceinline__ void unpack(Raw v, int (&q)[4]) {
        q[0] = (int)(int16_t)(v.x & 0xFFFFu); q[1] = (int)(int16_t)(v.x >> 16);
        q[2] = (int)(int16_t)(v.y & 0xFFFFu); q[3] = (int)(int16_t)(v.y >> 16);
    }
};

// Clock policies of the row kernels: hooks at the start of a block, when its
// first chunk has been folded, at the end of its chains and of its tree, and
// once the row's result is stored.  The kernels the library launches take
// NoClock, whose hooks are empty; the measurement library records the times
// of each phase with its own policy.
struct NoClock {
    __device__ __forceinline__ void start() {}
    __device__ __forceinline__ void first() {}
    __device__ __forceinline__ void chain_end() {}
    __device__ __forceinline__ void tree_end() {}
    __device__ __forceinline__ void done(int64_t) {}
};

// The reference tree over one row per block (grid-stride over rows).
// ALIGN is the vector alignment the reference uses for the chunks (16 bytes
// for 4-byte elements, 8 for int16); PAIR folds two accumulators.
// SETUP builds the kernel's LDS table once the row's first loads are in
// flight (finish(), which ends with the block barrier); issue() runs before
// any row load and is free for setup work that must precede them.  The
// tables' source is held in registers as immediates, so building them waits
// for no memory access.
template <typename SRC, int ALIGN, int D, typename TAB, typename PAIR, typename SETUP, typename CLOCK>
__device__ __forceinline__ int tree_row(const typename SRC::T* row, int64_t n, const TAB* __restrict__ tab, PAIR pair,
                                        int* __restrict__ sh_warp, SETUP& setup, CLOCK& clk) {
    clk.start();
    setup.issue();
    using T = typename SRC::T;
    const int t = threadIdx.x;
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(row) & (ALIGN - 1));
    int64_t prefix = mis ? (int64_t)((ALIGN - mis) / sizeof(T)) : 0;
    if (prefix > n) prefix = n;
    const int64_t n4 = (n - prefix) / 4;
    const int64_t tail = n - prefix - 4 * n4;
    const T* body = row + prefix;

    // Vector chunks of virtual thread t are c = t + 256*k.  Every thread owns
    // k = 0 .. kmain-1 with kmain = n4 / 256 (a block-uniform count), and
    // threads t < n4 % 256 own one more, k = kmain.  The uniform part runs
    // with wave-uniform control flow; loads are raw buffer loads addressed by
    // a per-lane constant (t * chunk bytes) plus a scalar k * 256 * chunk
    // bytes, with the hardware range check returning zero past the body.
    constexpr int64_t CB = 4 * (int64_t)sizeof(T);  // chunk bytes
    const int64_t kmain = n4 / 256;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(body), 0, (int)(n4 * CB), 0x00020000);
    const int vofs = (int)(t * CB);
    auto chunk = [&](int64_t k) { return SRC::bload(rsrc, vofs, (int)(k * 256 * CB)); };

    // The loads the chain consumes outside the uniform loop (prefix element,
    // the extra chunk, suffix element) are issued before it, so no lane waits
    // a separate round trip for them at either end.  The extra chunk's load is
    // unconditional: past the body the range check returns zero, unused.
    // The scalar elements come through a buffer over the whole row: a lane
    // without one addresses past the row's end, where the range check returns
    // zero, so no lane branches around a load or selects its value (either
    // would wait for the load).  They stay raw until used, for the same reason.
    const __amdgpu_buffer_rsrc_t rrow = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(row), 0, (int)(n * (int64_t)sizeof(T)), 0x00020000);
    const bool has_pre = t < prefix;
    const T pre = SRC::sload(rrow, (int)((has_pre ? t : n) * (int64_t)sizeof(T)));
    const bool has_extra = t < n4 - kmain * 256;
    const typename SRC::Raw extra = chunk(kmain);
    const bool has_suf = t < tail;
    const T suf = SRC::sload(rrow, (int)((has_suf ? prefix + 4 * n4 + t : n) * (int64_t)sizeof(T)));

    int acc = kQNegInf;
    bool has = has_pre;
    auto fold_first = [&](const typename SRC::Raw& raw) {
        int qq[4];
        SRC::unpack(raw, qq);
        acc = has ? pair(acc, qq[0], tab) : qq[0];
        has = true;
        acc = pair(acc, qq[1], tab);
        acc = pair(acc, qq[2], tab);
        acc = pair(acc, qq[3], tab);
    };
    auto fold = [&](const typename SRC::Raw& raw) {
        int qq[4];
        SRC::unpack(raw, qq);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = pair(acc, qq[i], tab);
    };
    // Two register buffers of D chunks alternate: while one is folded the
    // other's loads are in flight.  Chunk 0 comes from the first buffer.
    // (loaded even when kmain == 0: the range check keeps the loads in the
    // body, and an unconditional load leaves no merge of register values that
    // would wait for it)
    typename SRC::Raw bufa[D], bufb[D];
#pragma unroll
    for (int d = 0; d < D; ++d) bufa[d] = chunk(d);
    setup.finish();
    if (has_pre) acc = SRC::cvt(pre);
    if (kmain > 0) {
        int64_t k = 0;
        for (;;) {
#pragma unroll
            for (int d = 0; d < D; ++d) bufb[d] = chunk(k + D + d);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (k + d < kmain) {
                    if (d == 0 && k == 0) {
                        fold_first(bufa[0]);
                        clk.first();
                    } else {
                        fold(bufa[d]);
                    }
                }
            }
            k += D;
            if (k >= kmain) break;
#pragma unroll
            for (int d = 0; d < D; ++d) bufa[d] = chunk(k + D + d);
#pragma unroll
            for (int d = 0; d < D; ++d)
                if (k + d < kmain) fold(bufb[d]);
            k += D;
            if (k >= kmain) break;
        }
    }
    if (has_extra) fold_first(extra);
    if (has_suf) {
        const int q = SRC::cvt(suf);
        acc = has ? pair(acc, q, tab) : q;
    }
    clk.chain_end();
    // virtual-warp butterfly (xor 16, 8, 4, 2, 1 inside each 32-lane half)
    acc = pair(acc, exact_xor<16>(acc), tab);
    acc = pair(acc, exact_xor<8>(acc), tab);
    acc = pair(acc, exact_xor<4>(acc), tab);
    acc = pair(acc, exact_xor<2>(acc), tab);
    acc = pair(acc, exact_xor<1>(acc), tab);
    if ((t & 31) == 0) sh_warp[t >> 5] = acc;
    __syncthreads();
    int v = kQNegInf;
    if (t < 64) {
        v = (t & 31) < 8 ? sh_warp[t & 31] : kQNegInf;
        v = pair(v, exact_xor<16>(v), tab);
        v = pair(v, exact_xor<8>(v), tab);
        v = pair(v, exact_xor<4>(v), tab);
        v = pair(v, exact_xor<2>(v), tab);
        v = pair(v, exact_xor<1>(v), tab);
    }
    clk.tree_end();
    __syncthreads();  // sh_warp is reused by the next row
    return v;
}

// A 64-entry table held across a wave's lanes: lane i gets tab[i], written
// lane by lane as immediates (v_writelane), with no memory access.  The
// tables' source used to be loaded from memory at the start of each block;
// those loads queued behind the whole CU's row loads (in flight at once at
// the kernel's start), so the table, and with it each block's first pair
// step, waited 2.5 us (median) to 8 us (99th percentile) at (1024, 32000).
__device__ __forceinline__ int lanes_table(const int (&tab)[64]) {
    int v = 0;
#pragma unroll
    for (int i = 0; i < 64; ++i) asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(tab[i]), "i"(i));
    return v;
}

// One row per block: with no loop over rows, no load issued for a later
// round (the prefetch runs past the end of a row's chunks) can be in flight
// when the next row would reuse its registers, so nothing waits for it.
template <bool USE_LUT>
struct Q16Setup {
    int* lut;
    int v;
    __device__ __forceinline__ void issue() {}
    __device__ __forceinline__ void finish() {
        if constexpr (USE_LUT) {
            __builtin_amdgcn_sched_barrier(0);
            if (threadIdx.x < 64) lut[threadIdx.x] = lanes_table(kLutQ16);
            __syncthreads();
        }
    }
};

template <typename SRC, bool USE_LUT, int D, typename CLOCK = NoClock>
__global__ __launch_bounds__(256) void intlse_q16_rows(const typename SRC::T* __restrict__ x, float* __restrict__ out,
                                                       int32_t* __restrict__ acc_out, int64_t N, CLOCK clk = {}) {
    __shared__ int lut[64];
    __shared__ int sh_warp[8];
    Q16Setup<USE_LUT> setup{lut, 0};
    auto pair = [](int a, int b, const int* t) { return q16_pair<USE_LUT>(a, b, t); };
    const int64_t row = blockIdx.x;
    const int v = tree_row<SRC, 16, D>(x + row * N, N, lut, pair, sh_warp, setup, clk);
    if (threadIdx.x == 0) {
        out[row] = (float)v * kQ16Out;
        if (acc_out) acc_out[row] = v;
    }
    clk.done(row);
}

// gap[d] = M + LUT[M & 63], M = (64 + ((-d) & 63)) >> ceil(d / 64), for
// d <= 384; gap[385] = 0.  Thread t builds entries t and t + 256, reading
// LUT[M & 63] from a lane-held copy of the table with a lane shuffle.
struct Q10Setup {
    uint8_t* gap;
    int l0, l1;
    __device__ static __forceinline__ int m_of(int d) {
        const int sub = -d;
        const uint32_t sh = (uint32_t)(-(sub >> 6));
        return (int)((64u | ((uint32_t)sub & 63u)) >> (sh < 31u ? sh : 31u));
    }
    __device__ __forceinline__ void issue() {}
    __device__ __forceinline__ void finish() {
        // keep the table work after the row's first loads are issued
        __builtin_amdgcn_sched_barrier(0);
        const int lutv = lanes_table(kLutQ10);
        const int d0 = threadIdx.x, d1 = threadIdx.x + 256;
        l0 = __shfl(lutv, m_of(d0) & 63, 64);
        l1 = __shfl(lutv, m_of(d1 <= 384 ? d1 : 384) & 63, 64);
        gap[d0] = (uint8_t)(m_of(d0) + l0);
        if (d1 <= 384)
            gap[d1] = (uint8_t)(m_of(d1) + l1);
        else if (d1 == 385)
            gap[d1] = 0;
        __syncthreads();
    }
};

template <int D, typename CLOCK = NoClock>
__global__ __launch_bounds__(256) void intlse_q10_6_rows(const int16_t* __restrict__ x, float* __restrict__ out,
                                                         int32_t* __restrict__ acc_out, int64_t N, CLOCK clk = {}) {
    __shared__ __align__(16) uint8_t gap[388];
    __shared__ int sh_warp[8];
    Q10Setup setup{gap, 0, 0};
    const int64_t row = blockIdx.x;
    const int v = tree_row<SrcI16, 8, D>(x + row * N, N, gap, q10_pair, sh_warp, setup, clk);
    if (threadIdx.x == 0) {
        out[row] = (float)v * kQ10Out;
        if (acc_out) acc_out[row] = v;
    }
    clk.done(row);
}

// Q10.6 rows whose bodies start on 16-byte boundaries (x 16-byte aligned, N a
// multiple of 8): 128 threads per row, thread l holding the virtual threads
// 2l and 2l+1 of the reference tree.  Their chunks are adjacent, so one
// 16-byte load fetches both; the two chains are folded interleaved.  The
// virtual-warp butterfly's distances 16, 8, 4, 2 become lane distances 8, 4,
// 2, 1 and distance 1 is the pair within the thread.  Every virtual thread
// folds the same elements in the same order as in tree_row, so the results
// are the same bits.  With half the waves per row, a row's chains are hidden
// behind fewer other waves, so the launcher takes this kernel only for many
// short rows: (8192, 4096) 15.5 -> 12.8 us and (2048, 32000) 23.9 -> 22.9,
// while (1024, 32000) measured the same and rows of 128256 elements 29-35%
// slower.
// chunk pairs per thread kept in flight ahead of the chains (2 measured ahead
// of 3 and 4: 12.80 against 13.74 and 14.55 us at (8192, 4096))
constexpr int kQ10PairedAhead = 2;

template <int D>
__global__ __launch_bounds__(128) void intlse_q10_6_rows_paired(const int16_t* __restrict__ x,
                                                                float* __restrict__ out,
                                                                int32_t* __restrict__ acc_out, int64_t N) {
    __shared__ __align__(16) uint8_t gap[388];
    __shared__ int sh_warp[8];
    const int l = threadIdx.x;
    const int va = 2 * l, vb = 2 * l + 1;
    const int16_t* row = x + (int64_t)blockIdx.x * N;
    // rows start 16-byte aligned, so the 8-byte alignment prefix is empty
    const int64_t n4 = N / 4;
    const int64_t tail = N - 4 * n4;
    const int64_t kmain = n4 / 256;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int16_t*>(row), 0, (int)(n4 * 8), 0x00020000);
    auto pairc = [&](int64_t k) {
        return __builtin_amdgcn_raw_buffer_load_b128(rsrc, l * 16, (int)(k * 2048), kBufNT);
    };
    // the extra chunks (k = kmain) and the suffix elements, issued before the chain
    const bool has_xa = va < n4 - kmain * 256, has_xb = vb < n4 - kmain * 256;
    const u32x2 xa = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, va * 8, (int)(kmain * 2048), kBufNT));
    const u32x2 xb = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, vb * 8, (int)(kmain * 2048), kBufNT));
    const __amdgpu_buffer_rsrc_t rrow =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int16_t*>(row), 0, (int)(N * 2), 0x00020000);
    const bool has_sa = va < tail, has_sb = vb < tail;
    const int16_t sa = SrcI16::sload(rrow, (int)((has_sa ? 4 * n4 + va : N) * 2));
    const int16_t sb = SrcI16::sload(rrow, (int)((has_sb ? 4 * n4 + vb : N) * 2));
    u32x4 bufa[D], bufb[D];
#pragma unroll
    for (int d = 0; d < D; ++d) bufa[d] = pairc(d);
    // the gap table (as Q10Setup, 128 threads), after the first loads are issued
    __builtin_amdgcn_sched_barrier(0);
    {
        const int lutv = lanes_table(kLutQ10);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = l + 128 * j;
            const int dc = d <= 384 ? d : 384;
            const int lv = __shfl(lutv, Q10Setup::m_of(dc) & 63, 64);
            if (d <= 384)
                gap[d] = (uint8_t)(Q10Setup::m_of(d) + lv);
            else if (d == 385)
                gap[d] = 0;
        }
        __syncthreads();
    }
    int a = kQNegInf, b = kQNegInf;
    bool has = false;  // no prefix: chunk 0 seeds both chains
    auto fold = [&](const u32x4& v, bool first) {
        int qa[4], qb[4];
        SrcI16::unpack(u32x2{v.x, v.y}, qa);
        SrcI16::unpack(u32x2{v.z, v.w}, qb);
        a = first ? qa[0] : q10_pair(a, qa[0], gap);
        b = first ? qb[0] : q10_pair(b, qb[0], gap);
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            a = q10_pair(a, qa[i], gap);
            b = q10_pair(b, qb[i], gap);
        }
    };
    if (kmain > 0) {
        int64_t k = 0;
        for (;;) {
#pragma unroll
            for (int d = 0; d < D; ++d) bufb[d] = pairc(k + D + d);
#pragma unroll
            for (int d = 0; d < D; ++d)
                if (k + d < kmain) fold(bufa[d], d == 0 && k == 0);
            k += D;
            if (k >= kmain) break;
#pragma unroll
            for (int d = 0; d < D; ++d) bufa[d] = pairc(k + D + d);
#pragma unroll
            for (int d = 0; d < D; ++d)
                if (k + d < kmain) fold(bufb[d], false);
            k += D;
            if (k >= kmain) break;
        }
        has = true;
    }
    // the extra chunk of each virtual thread, then its suffix element
    auto fold_one = [&](int& acc, bool h, const u32x2& raw) {
        int qq[4];
        SrcI16::unpack(raw, qq);
        acc = h ? q10_pair(acc, qq[0], gap) : qq[0];
        acc = q10_pair(acc, qq[1], gap);
        acc = q10_pair(acc, qq[2], gap);
        acc = q10_pair(acc, qq[3], gap);
    };
    if (has_xa) fold_one(a, has, xa);
    if (has_xb) fold_one(b, has, xb);
    const bool ha = has || has_xa, hb = has || has_xb;
    if (has_sa) a = ha ? q10_pair(a, (int)sa, gap) : (int)sa;
    if (has_sb) b = hb ? q10_pair(b, (int)sb, gap) : (int)sb;
    // virtual-warp butterfly: distances 16, 8, 4, 2 across lanes, 1 in-thread
    a = q10_pair(a, exact_xor<8>(a), gap);
    b = q10_pair(b, exact_xor<8>(b), gap);
    a = q10_pair(a, exact_xor<4>(a), gap);
    b = q10_pair(b, exact_xor<4>(b), gap);
    a = q10_pair(a, exact_xor<2>(a), gap);
    b = q10_pair(b, exact_xor<2>(b), gap);
    a = q10_pair(a, exact_xor<1>(a), gap);
    b = q10_pair(b, exact_xor<1>(b), gap);
    a = q10_pair(a, b, gap);  // distance 1: both virtual threads end with pair(a, b)
    if ((l & 15) == 0) sh_warp[l >> 4] = a;
    __syncthreads();
    if (l < 64) {
        int v = (l & 31) < 8 ? sh_warp[l & 31] : kQNegInf;
        v = q10_pair(v, exact_xor<16>(v), gap);
        v = q10_pair(v, exact_xor<8>(v), gap);
        v = q10_pair(v, exact_xor<4>(v), gap);
        v = q10_pair(v, exact_xor<2>(v), gap);
        v = q10_pair(v, exact_xor<1>(v), gap);
        if (l == 0) {
            out[blockIdx.x] = (float)v * kQ10Out;
            if (acc_out) acc_out[blockIdx.x] = v;
        }
    }
}

// Chunks per lane kept in flight ahead of the pair chain.  Every block starts
// its row at once and issues its first chunks together; a wave whose loads
// cannot issue yet (its CU's queue is full) also cannot start its chain, so
// a deep prefetch delays the first pair steps while a shallow one starves
// long rows.  Same-process sweeps of 1..8 chunks over 256..8192 rows of both
// formats put the best at about 20 KB in flight per CU: 1024 x 32000 Q10.6
// 15.9 -> 12.8 us and 512 x 128256 Q16.16 45.4 -> 41.3 us against 8 chunks.
inline int prefetch_chunks(int64_t rows, int64_t chunk_bytes) {
    const int64_t blocks_per_cu = (rows + 255) / 256 < 8 ? (rows + 255) / 256 : 8;
    const double t = 20480.0 / (double)(4 * blocks_per_cu * 64 * chunk_bytes);
    return t <= 2.5 ? 2 : t < 3.5 ? 3 : t < 5.0 ? 4 : 6;
}

// Launches KERNEL<D> with the prefetch depth for this shape.
template <typename LAUNCH>
inline void with_prefetch(int64_t rows, int64_t chunk_bytes, LAUNCH launch) {
    switch (prefetch_chunks(rows, chunk_bytes)) {
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 3: launch(std::integral_constant<int, 3>{}); break;
    case 4: launch(std::integral_constant<int, 4>{}); break;
    default: launch(std::integral_constant<int, 6>{}); break;
    }
}

}  // namespace fl
