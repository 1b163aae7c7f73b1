// The IntLSE pair operations (Q16.16 and Q10.6), shared by the row kernels
// and the latency measurement.  Both are commutative (symmetric in a, b) and
// follow the reference's integer arithmetic (intlse/gpu/lse_kernel.cu:46-57,
// lse_kernel_q10_6.cu:35-43) with the shift count clamped as described in
// lse_int.hip.
#pragma once

#include <stdint.h>

namespace fl {

constexpr int kQNegInf = -0x3fffffff;

// Q16.16 pair: max + M + LUT[(M >> 10) & 63], M = (2^16 + (sub & 0xFFFF)) >> -(sub >> 16).
template <bool USE_LUT>
__device__ __forceinline__ int q16_pair(int a, int b, const int* __restrict__ lut) {
    const int hi = a > b ? a : b;
    const int lo = a > b ? b : a;
    const int sub = (int)((uint32_t)lo - (uint32_t)hi);
    const uint32_t sh = (uint32_t)(-(sub >> 16));
    const uint32_t shc = sh < 31u ? sh : 31u;
    const uint32_t fr = 0x10000u | ((uint32_t)sub & 0xFFFFu);
    const int m = (int)(fr >> shc);
    const uint32_t r = (uint32_t)hi + (uint32_t)m;
    if constexpr (USE_LUT) {
        // LUT index (m >> 10) & 63 as a byte offset, (m >> 8) & 0xFC, taken as
        // ((fr >> 8) >> shc) & 0xFC so it does not wait for m.
        const uint32_t off = ((fr >> 8) >> shc) & 0xFCu;
        return (int)(r + (uint32_t)*reinterpret_cast<const int*>(reinterpret_cast<const char*>(lut) + off));
    } else {
        return (int)r;
    }
}

// Q10.6 pair through the gap table: max(a, b) + g[min(|a - b|, 385)],
// g[385] = 0.  Every table entry is at most 69, so the table is bytes and the
// clamped gap is the LDS address itself; the clamp is one v_med3_i32 of
// (a - b, b - a, 385), the median being min(|a - b|, 385).  The differences
// cannot overflow: inputs are int16, an accumulator exceeds the largest input
// by at most 64 * log2(N), and the identity -0x3fffffff stays below 2^30 in
// magnitude after any number of pair steps.  Measured 18% shorter per pair
// step than max/min, subtract, clamp and a word address.
__device__ __forceinline__ int q10_pair(int a, int b, const uint8_t* __restrict__ g) {
    const int hi = a > b ? a : b;
    const int u = a - b, nu = b - a;
    int d;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(d) : "v"(u), "v"(nu), "s"(385));
    return hi + (int)g[d];
}

}  // namespace fl
