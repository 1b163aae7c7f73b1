// Shared device helpers for the gfx950 log-sum-exp kernels: wave64 lane
// exchanges, the online (max, scaled-sum) state used by the float paths, and
// 16-byte vector loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fl_grid.hpp"

namespace fl {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kInf = __builtin_huge_valf();

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------
// Lane exchanges. exact_xor<K> returns the value held by lane (lane ^ K); for
// K < 32 it stays inside each 32-lane half (ds_swizzle bit-mask mode), which
// is the exchange pattern of a warp-32 xor butterfly.
// ---------------------------------------------------------------------------
template <int K>
__device__ __forceinline__ int exact_xor(int v) {
    static_assert(K == 1 || K == 2 || K == 4 || K == 8 || K == 16 || K == 32, "xor distance");
    if constexpr (K == 32) {
        return __shfl_xor(v, 32, 64);
    } else {
        return __builtin_amdgcn_ds_swizzle(v, 0x1F | (K << 10));
    }
}
template <int K>
__device__ __forceinline__ float exact_xor(float v) {
    return __builtin_bit_cast(float, exact_xor<K>(__builtin_bit_cast(int, v)));
}

// Maxima across the rows of a wave: max_pair16(v) is fmaxf of v at lanes l and
// l ^ 16, max_pair32(v) at l and l ^ 32.  gfx950's v_permlane16_swap_b32 and
// v_permlane32_swap_b32 exchange the rows inside the VGPRs, with no LDS round
// trip (ds_swizzle and ds_bpermute wait on the LDS unit).  With both operands
// v, the 16-lane swap returns rows {0, 0, 2, 2} and {1, 1, 3, 3} of v and the
// 32-lane swap halves {0, 0} and {1, 1}, so both lanes of a pair take fmaxf of
// the same two operands in the same order and hold the same bits.
__device__ __forceinline__ float max_pair16(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)s[0]), __builtin_bit_cast(float, (unsigned)s[1]));
}
__device__ __forceinline__ float max_pair32(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)s[0]), __builtin_bit_cast(float, (unsigned)s[1]));
}

// Partner exchange for commutative reductions whose operands are already
// uniform within aligned groups of K lanes: DPP moves for K <= 8 (quad
// permutes, then half-row and row mirrors, which pair the same groups as an
// xor once those groups are uniform), a swizzle for 16, a lane shuffle for 32.
template <int K>
__device__ __forceinline__ float reduce_partner(float v) {
    int iv = __builtin_bit_cast(int, v);
    int r;
    if constexpr (K == 1) r = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false);       // quad_perm 1,0,3,2
    else if constexpr (K == 2) r = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false);  // quad_perm 2,3,0,1
    else if constexpr (K == 4) r = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false); // row_half_mirror
    else if constexpr (K == 8) r = __builtin_amdgcn_update_dpp(0, iv, 0x140, 0xF, 0xF, false); // row_mirror
    else r = exact_xor<K>(iv);
    return __builtin_bit_cast(float, r);
}

// ---------------------------------------------------------------------------
// Online log-sum-exp state: m is the running maximum (natural units, NaN never
// enters it because fmaxf drops NaN), s = sum exp(x - base(m)) where base(m)
// is m when finite and 0 when m is +-inf.  With that base, a row of all -inf
// ends at (m=-inf, s=0) -> -inf, any +inf drives s to +inf -> +inf, and a NaN
// element makes s NaN -> NaN: torch.logsumexp's special values, which the
// reference's robust pair reproduces (fused_fp32_kernel.cu:34-40).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float lse_base(float m) { return __builtin_isfinite(m) ? m : 0.0f; }

// Rescale factor that moves a partial sum from base(mi) to base(m); an empty
// partial (mi = -inf) contributes nothing (0 * NaN still propagates NaN).
__device__ __forceinline__ float lse_rescale(float mi, float m) {
    return mi == -kInf ? 0.0f : fexp2((lse_base(mi) - lse_base(m)) * kLog2e);
}

__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
    float mn = fmaxf(m, m2);
    s = s * lse_rescale(m, mn) + s2 * lse_rescale(m2, mn);
    m = mn;
}

// The rescale of a fold whose new values have maximum cm: moves (m, s) to
// the maximum max(m, cm) and returns the base that the fold's exponents
// subtract.  ROBUST keeps the base finite so non-finite inputs follow the
// rules above; the plain variant assumes finite inputs (as the reference's
// non-robust kernel does).
template <bool ROBUST>
__device__ __forceinline__ float lse_rebase(float& m, float& s, float cm) {
    const float mn = fmaxf(m, cm);
    float b;
    if constexpr (ROBUST) {
        s *= lse_rescale(m, mn);
        b = lse_base(mn);
    } else {
        s *= fexp2((m - mn) * kLog2e);
        b = mn;
    }
    m = mn;
    return b;
}

// exp(v - b) = exp2(v*log2e - b*log2e) as one FMA per element.  The rounding
// of b*log2e shifts every exponent of a fold by the same delta <= |b|*2^-23,
// i.e. a relative error of the result of the same order as fp32 rounding of b
// itself.  For |b| >= 2^24 that shift could reach the exp2 range, so those
// lanes take the exact-difference form (lse_exp_exact).
__device__ __forceinline__ bool lse_fused_exp_ok(float b) { return __builtin_fabsf(b) < 0x1p24f; }
__device__ __forceinline__ float lse_exp_fused(float v, float nb) { return fexp2(__builtin_fmaf(v, kLog2e, nb)); }
__device__ __forceinline__ float lse_exp_exact(float v, float b) { return fexp2((v - b) * kLog2e); }

// Fold K new values into (m, s) with one rescale.
template <bool ROBUST, int K>
__device__ __forceinline__ void lse_fold(float& m, float& s, const float (&v)[K]) {
    float cm = v[0];
#pragma unroll
    for (int k = 1; k < K; ++k) cm = fmaxf(cm, v[k]);
    const float b = lse_rebase<ROBUST>(m, s, cm);
    float acc = 0.0f;
    if (lse_fused_exp_ok(b)) {
        const float nb = -b * kLog2e;
#pragma unroll
        for (int k = 0; k < K; ++k) acc += lse_exp_fused(v[k], nb);
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k) acc += lse_exp_exact(v[k], b);
    }
    s += acc;
}

template <bool ROBUST>
__device__ __forceinline__ float lse_finish(float m, float s) {
    float b = ROBUST ? lse_base(m) : m;
    return b + flog2(s) * kLn2;
}

// Merge (m, s) across aligned groups of W lanes; every lane of a group ends
// with the group result.  Two phases: a butterfly max, one rescale of each
// lane's sum to the group max, a butterfly sum.  This equals the tree of
// pairwise lse_merge steps up to rounding (the rescale factors compose, and
// lse_rescale keeps -inf partials at 0 and base(+inf) = 0 as each pairwise
// step would), with a dependent chain of cheap max and add steps and one
// exponential instead of two exponentials per level; the end-of-row merge is
// on the critical path of every block.
template <int W>
__device__ __forceinline__ void group_merge(float& m, float& s) {
    float mm = m;
    if constexpr (W >= 2) mm = fmaxf(mm, reduce_partner<1>(mm));
    if constexpr (W >= 4) mm = fmaxf(mm, reduce_partner<2>(mm));
    if constexpr (W >= 8) mm = fmaxf(mm, reduce_partner<4>(mm));
    if constexpr (W >= 16) mm = fmaxf(mm, reduce_partner<8>(mm));
    if constexpr (W >= 32) mm = fmaxf(mm, reduce_partner<16>(mm));
    if constexpr (W >= 64) mm = fmaxf(mm, reduce_partner<32>(mm));
    float ss = s * lse_rescale(m, mm);
    if constexpr (W >= 2) ss += reduce_partner<1>(ss);
    if constexpr (W >= 4) ss += reduce_partner<2>(ss);
    if constexpr (W >= 8) ss += reduce_partner<4>(ss);
    if constexpr (W >= 16) ss += reduce_partner<8>(ss);
    if constexpr (W >= 32) ss += reduce_partner<16>(ss);
    if constexpr (W >= 64) ss += reduce_partner<32>(ss);
    m = mm;
    s = ss;
}

// ---------------------------------------------------------------------------
// Element types: 16-byte vector loads widened to fp32.  Row data is streamed
// once, so vector loads carry the nontemporal hint (global_load ... nt), which
// measured 10% more read bandwidth than plain loads at (512, 128256).
// ---------------------------------------------------------------------------
template <typename V>
__device__ __forceinline__ V load_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
}
template <typename V>
__device__ __forceinline__ void store_stream(V v, void* p) {
    __builtin_nontemporal_store(v, reinterpret_cast<V*>(p));
}
struct bf16_t { uint16_t bits; };

// Cache policy of streamed 16-byte result stores through a buffer resource:
// device scope (sc1) and nontemporal (nt).  Written through to memory instead
// of left dirty in the XCD's L2, a row of results streams out in one pass;
// the (512, 128256) fp32 backward measured 79.9 us with it against 85.2 us
// with nt alone.
constexpr int kStoreStreamAux = 16 | 2;
// Streamed loads through a buffer resource: nontemporal (nt), as load_stream.
constexpr int kLoadStreamAux = 2;
// Loads of the rows a forward leaves for the backward that follows it: plain
// (no nt), so part of what they bring in stays in the Infinity Cache, the
// memory-side cache in front of HBM.  nt loads leave nothing there that a
// following read finds.
constexpr int kLoadKeepAux = 0;

// fp32 -> bfloat16 pairs with gfx950's v_cvt_pk_bf16_f32 (round to nearest
// even, NaN stays NaN): lo in bits 0-15, hi in bits 16-31.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16_pack2(float lo, float hi) {
    bf16x2_t v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

template <typename T> struct Elem;
template <> struct Elem<float> {
    static constexpr int kVec = 4;
    static constexpr uint32_t kNegInfBits = 0xFF800000u;  // -inf in each 32-bit word
    __device__ static __forceinline__ float scalar(const float* p) { return *p; }
    // cvt widens one raw 16-byte vector (as loaded by load_stream<u32x4>).
    // Each lane goes through a scalar temporary: this clang folds a bit_cast
    // whose operand is an ext-vector element to element 0.
    __device__ static __forceinline__ void cvt(u32x4 r, float (&o)[4]) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t e = r[k];
            o[k] = __builtin_bit_cast(float, e);
        }
    }
    __device__ static __forceinline__ void vec(const float* p, float (&o)[4]) {
        f32x4 v = load_stream<f32x4>(p);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    __device__ static __forceinline__ void put(float* p, float v) { *p = v; }
    __device__ static __forceinline__ void put_vec(float* p, const float (&v)[4]) {
        f32x4 t;
        t.x = v[0]; t.y = v[1]; t.z = v[2]; t.w = v[3];
        store_stream<f32x4>(t, p);
    }
    __device__ static __forceinline__ void put_vec_buf(__amdgpu_buffer_rsrc_t r, int off, const float (&v)[4]) {
        f32x4 t;
        t.x = v[0]; t.y = v[1]; t.z = v[2]; t.w = v[3];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), r, off, 0, kStoreStreamAux);
    }
};
template <> struct Elem<_Float16> {
    static constexpr int kVec = 8;
    static constexpr uint32_t kNegInfBits = 0xFC00FC00u;
    __device__ static __forceinline__ float scalar(const _Float16* p) { return (float)*p; }
    __device__ static __forceinline__ void cvt(u32x4 r, float (&o)[8]) {
        const f16x8 v = __builtin_bit_cast(f16x8, r);
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = (float)v[k];
    }
    __device__ static __forceinline__ void vec(const _Float16* p, float (&o)[8]) {
        f16x8 v = load_stream<f16x8>(p);
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = (float)v[k];
    }
    // fp32 -> binary16 with v_cvt_f16_f32 (round to nearest even)
    __device__ static __forceinline__ void put(_Float16* p, float v) { *p = (_Float16)v; }
    __device__ static __forceinline__ void put_vec(_Float16* p, const float (&v)[8]) {
        f16x8 t;
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = (_Float16)v[k];
        store_stream<f16x8>(t, p);
    }
    __device__ static __forceinline__ void put_vec_buf(__amdgpu_buffer_rsrc_t r, int off, const float (&v)[8]) {
        f16x8 t;
#pragma unroll
        for (int k = 0; k < 8; ++k) t[k] = (_Float16)v[k];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), r, off, 0, kStoreStreamAux);
    }
};
template <> struct Elem<bf16_t> {
    static constexpr int kVec = 8;
    static constexpr uint32_t kNegInfBits = 0xFF80FF80u;
    __device__ static __forceinline__ float scalar(const bf16_t* p) {
        return __builtin_bit_cast(float, (uint32_t)p->bits << 16);
    }
    __device__ static __forceinline__ void cvt(u32x4 v, float (&o)[8]) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[2 * k] = __builtin_bit_cast(float, v[k] << 16);
            o[2 * k + 1] = __builtin_bit_cast(float, v[k] & 0xFFFF0000u);
        }
    }
    __device__ static __forceinline__ void vec(const bf16_t* p, float (&o)[8]) { cvt(load_stream<u32x4>(p), o); }
    __device__ static __forceinline__ void put(bf16_t* p, float v) {
        p->bits = __builtin_bit_cast(uint16_t, (__bf16)v);
    }
    __device__ static __forceinline__ void put_vec(bf16_t* p, const float (&v)[8]) {
        store_stream<u32x4>(pack(v), p);
    }
    __device__ static __forceinline__ void put_vec_buf(__amdgpu_buffer_rsrc_t r, int off, const float (&v)[8]) {
        __builtin_amdgcn_raw_buffer_store_b128(pack(v), r, off, 0, kStoreStreamAux);
    }
    __device__ static __forceinline__ u32x4 pack(const float (&v)[8]) {
        u32x4 t;
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] = bf16_pack2(v[2 * k], v[2 * k + 1]);
        return t;
    }
};

// Split of a row into a scalar head (up to the first 16-byte boundary), a
// body of 16-byte vectors and a scalar tail.
struct RowSplit {
    int64_t head, nvec, tail;
};
template <typename T>
__device__ __forceinline__ RowSplit split_row(const T* row, int64_t n) {
    constexpr int64_t E = (int64_t)sizeof(T);
    uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(row) & 15u);
    int64_t head = mis ? (int64_t)((16u - mis) / E) : 0;
    if (head > n) head = n;
    int64_t nvec = (n - head) / Elem<T>::kVec;
    return {head, nvec, n - head - nvec * Elem<T>::kVec};
}

}  // namespace fl
