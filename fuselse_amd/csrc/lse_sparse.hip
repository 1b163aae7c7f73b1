// Sparse probabilistic-circuit sum-layer forward for gfx950: per sum node n
// and batch column b,
//     out[n, b] = log sum_e exp(logw_e + child[c_e, b])
// over the node's edges e, in fp32 or in the IntLSE Q16.16 arithmetic.
//
// Two edge layouts:
//   * CSR (offsets[n] .. offsets[n+1] index child ids and log-parameters);
//   * the pyjuice block layout of the reference (experiment_pyjuice/
//     sparse_float_kernel.cu:40-105, sparse_q16_kernel.cu:61-134): node block
//     j of block_size parents p shares the child ids cids[j, :]; parent p takes
//     weight params[pids[j, e] + p]; it writes node_mars[nids[j] + p, :].
// Node values are [node][batch] rows, so each edge gathers one contiguous
// child row.
//
// Mapping: one wave per (node, 256-column tile); lane l owns 4 columns (one
// 16-byte vector when the batch is a multiple of 4 and rows are 16-byte
// aligned, else 4 strided scalars).  Edge metadata is held one 64-edge window
// at a time across the lanes and broadcast per edge with readlane; child rows
// are loaded G = 4 edges at a time into two alternating register buffers, so
// the next group's loads are in flight while a group folds.
//
// fp32: an online (max, scaled sum) per column with one rescale per group.
// Q16.16: bit-exact with the reference's reduction: ET = 1, 2, 4, 8 chains
// for fan-in <= 8, 16, 32, above (sparse_q16_kernel.cu:161-165), chain et folds
// edges e = et, et + ET, ... in order starting from the identity -0x3fffffff,
// then an xor butterfly over the ET chains; each logit is quantised as
// rne_sat(fmaxf(logw + child, -20000) * 94548.4609375) and a result at or
// below the identity becomes -inf (sparse_q16_kernel.cu:113,129-131).
#include <math.h>
#include <stdint.h>

#include "../../include/fuselse_amd.h"
#include "fl_status.hpp"
#include "lse_blocked.hpp"
#include "lse_common.hpp"

namespace fl {
namespace sparse {

constexpr int kNegInfQ = -0x3fffffff;
constexpr float kConv = 1.44269504089f * 65536.0f;
constexpr float kOutScale = 0.69314718056f / 65536.0f;
constexpr int G = 4;      // edges per load group
constexpr int P = 4;      // columns per lane, forward kernels
constexpr int PB = 8;     // columns per lane, backward kernel

__constant__ int kLut[64] = {
       0,  571,  907, 1282, 1634, 1745, 2054, 2592,
    2900, 2859, 2895, 3015, 3222, 3522, 3922, 4426,
    4617, 4441, 4294, 4178, 4093, 4039, 4018, 4030,
    4076, 4157, 4272, 4424, 4613, 4838, 5102, 5404,
    5399, 5068, 4746, 4435, 4134, 3843, 3562, 3291,
    3031, 2781, 2541, 2312, 2094, 1886, 1689, 1502,
    1327, 1162, 1008,  865,  732,  611,  500,  401,
     312,  235,  168,  113,   69,   35,   13,    2,
};

__device__ __forceinline__ int pair(int a, int b, const int* __restrict__ lut) {
    const int hi = a > b ? a : b;
    const int lo = a > b ? b : a;
    const int sub = (int)((uint32_t)lo - (uint32_t)hi);
    const uint32_t sh = (uint32_t)(-(sub >> 16));
    const uint32_t shc = sh < 31u ? sh : 31u;
    const uint32_t fr = 0x10000u | ((uint32_t)sub & 0xFFFFu);
    const uint32_t m = fr >> shc;
    // (fr >> 8) >> shc == m >> 8 (logical shifts compose); byte 1 of m masked
    // is one instruction on this target
    const uint32_t off = (m >> 8) & 0xFCu;
    return (int)((uint32_t)hi + m + (uint32_t)*reinterpret_cast<const int*>(reinterpret_cast<const char*>(lut) + off));
}

__device__ __forceinline__ int quant(float logit) {
    const float r = __builtin_rintf(fmaxf(logit, -20000.0f) * kConv);
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(r));
    return q;
}

// The PP columns of lane l in the tile of 64*PP columns starting at b0.  With
// VEC, lane l holds the 16-byte vectors at b0 + 256*q + 4*l (q < PP/4): each
// vector load of the wave covers 1 KB of a row, contiguous.  Otherwise lane l
// holds the scalars b0 + l + 64*i.
template <bool VEC, int PP>
struct Cols {
    static_assert(!VEC || PP % 4 == 0, "vector columns come in fours");
    __device__ static __forceinline__ bool ok(int64_t b0, int l, int64_t batch, int i) {
        return VEC ? b0 + 256 * (i / 4) + 4 * l < batch : b0 + l + 64 * i < batch;
    }
    __device__ static __forceinline__ void load(const float* __restrict__ row, int64_t b0, int l, int64_t batch,
                                                float (&v)[PP]) {
        if constexpr (VEC) {
#pragma unroll
            for (int q = 0; q < PP / 4; ++q) {
                const int64_t c = b0 + 256 * q + 4 * l;
                if (c < batch) {
                    const f32x4 t = *reinterpret_cast<const f32x4*>(row + c);
                    v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
                } else {
                    v[4 * q] = v[4 * q + 1] = v[4 * q + 2] = v[4 * q + 3] = 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < PP; ++i) {
                const int64_t c = b0 + l + 64 * i;
                v[i] = c < batch ? row[c] : 0.0f;
            }
        }
    }
    __device__ static __forceinline__ void store(float* __restrict__ row, int64_t b0, int l, int64_t batch,
                                                 const float (&v)[PP]) {
        if constexpr (VEC) {
#pragma unroll
            for (int q = 0; q < PP / 4; ++q) {
                const int64_t c = b0 + 256 * q + 4 * l;
                if (c < batch) {
                    f32x4 t;
                    t.x = v[4 * q]; t.y = v[4 * q + 1]; t.z = v[4 * q + 2]; t.w = v[4 * q + 3];
                    store_stream<f32x4>(t, row + c);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < PP; ++i) {
                const int64_t c = b0 + l + 64 * i;
                if (c < batch) row[c] = v[i];
            }
        }
    }
};

// Lane-held metadata of edge (window start + lane).
struct EdgeMeta {
    int64_t cid;
    float logw;
};

__device__ __forceinline__ int64_t uniform64(int64_t v) {
    const int lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uint64_t)v);
    const int hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ int64_t bcast64(int64_t v, int lane) {
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, lane);
    const int hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ float bcastf(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// ---------------------------------------------------------------------------
// Layouts: node(n) returns a wave-uniform descriptor (edge count, output row);
// meta(d, e) the metadata of edge e of that node (called per lane).
// ---------------------------------------------------------------------------
struct CsrDesc {
    int64_t e0, k, n;
};
struct CsrLayout {
    const int64_t* offsets;
    const int32_t* cids;
    const float* logp;
    float* out;
    int64_t batch;
    __device__ __forceinline__ CsrDesc node(int64_t n) const {
        const int64_t e0 = uniform64(offsets[n]);
        return {e0, uniform64(offsets[n + 1]) - e0, n};
    }
    __device__ __forceinline__ EdgeMeta meta(const CsrDesc& d, int64_t e) const {
        return {(int64_t)cids[d.e0 + e], logp[d.e0 + e]};
    }
    __device__ __forceinline__ float* out_row(const CsrDesc& d) const { return out + d.n * batch; }
};

struct BlockDesc {
    int64_t base, k, p, row;
};
template <bool LOGP>
struct BlockLayout {
    float* node_mars;
    const float* params;
    const int64_t* nids;
    const int64_t* cids;
    const int64_t* pids;
    int64_t num_edges, block_size, batch;
    __device__ __forceinline__ BlockDesc node(int64_t jp) const {
        const int64_t j = jp / block_size;
        const int64_t p = jp - j * block_size;
        return {j * num_edges, num_edges, p, uniform64(nids[j]) + p};
    }
    __device__ __forceinline__ EdgeMeta meta(const BlockDesc& d, int64_t e) const {
        const float w = params[pids[d.base + e] + d.p];
        // log of the linear weight with the reference's 1e-45 floor
        // (sparse_float_kernel.cu:76), accurate libm log once per edge
        return {cids[d.base + e], LOGP ? w : logf(fmaxf(w, 1e-45f))};
    }
    __device__ __forceinline__ float* out_row(const BlockDesc& d) const { return node_mars + d.row * batch; }
};

// ---------------------------------------------------------------------------
// Per-node reductions over one 256-column tile.
// ---------------------------------------------------------------------------
// The 16-byte column vectors of lane l (as Cols<true, PP>) from the row
// segment starting at b0 (`row` points at it), through a buffer resource of
// `rec` bytes: vectors past the range read as zeros, without a memory access,
// and the load needs no branch.  The rows are gathered by id, and they take
// plain loads: with the nontemporal hint (which streamed dense rows read
// faster) the C5 layer's forward took 3339 us against 3139, its backward
// 7046 us against 6169.
template <int PP>
__device__ __forceinline__ void load_cols_buf(const float* row, int rec, int l, float (&v)[PP]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(row), 0, rec, 0x00020000);
#pragma unroll
    for (int q = 0; q < PP / 4; ++q) {
        const f32x4 t =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (256 * q + 4 * l) * 4, 0, 0));
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

// Bytes of a row from column b0 to the batch's end, clamped to a buffer range.
__device__ __forceinline__ int cols_bytes(int64_t batch, int64_t b0) {
    const int64_t left = (batch - b0) * 4;
    return left > 0x7fffffff ? 0x7fffffff : (int)left;
}

// Loads the child rows of window edges j .. j + GS - 1 (edges at or past wn
// are left for the fold to mask).  With VEC every load is issued: each edge's
// row goes through a buffer resource built from its wave-uniform child id,
// with an empty range for edges past wn and the range check covering the
// batch's end, so no load sits behind a branch.  A load behind a branch left
// the wait-count pass unable to count the loads in flight, and the fold of a
// group then waited for the next group's loads as well.
template <int GS, bool VEC, int PP>
__device__ __forceinline__ void load_group(float (&v)[GS][PP], const EdgeMeta& ew, int j, int wn,
                                           const float* __restrict__ child, int64_t batch, int64_t b0, int l) {
    if constexpr (VEC) {
        const int rec = cols_bytes(batch, b0);
#pragma unroll
        for (int g = 0; g < GS; ++g)
            load_cols_buf<PP>(child + bcast64(ew.cid, (j + g) & 63) * batch + b0, j + g < wn ? rec : 0, l, v[g]);
    } else {
#pragma unroll
        for (int g = 0; g < GS; ++g)
            if (j + g < wn) Cols<VEC, PP>::load(child + bcast64(ew.cid, j + g) * batch, b0, l, batch, v[g]);
    }
}

template <int PP>
__device__ __forceinline__ void fold_group_f32(const float (&v)[G][PP], const EdgeMeta& ew, int j, int wn,
                                               float (&m)[PP], float (&s)[PP]) {
    float lw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) lw[g] = j + g < wn ? bcastf(ew.logw, j + g) : -kInf;
#pragma unroll
    for (int i = 0; i < PP; ++i) {
        float col[G];
#pragma unroll
        for (int g = 0; g < G; ++g) col[g] = j + g < wn ? v[g][i] + lw[g] : -kInf;
        lse_fold<true, G>(m[i], s[i], col);
    }
}

// Edge g of a group starting at window edge j belongs to chain (j + g) % ET.
// Windows start at multiples of 64 and groups at multiples of G = 4, so for
// ET <= 4 the chain is g % ET, and for ET = 8 it is C0 + g with C0 = j % 8,
// 0 or 4: a wave-uniform choice between two static code paths.
template <int ET, int C0>
__device__ __forceinline__ void fold_group_q16_at(const float (&v)[G][P], const EdgeMeta& ew, int j, int wn,
                                                  int (&acc)[ET][P], const int* __restrict__ lut) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (j + g < wn) {
            const float lw = bcastf(ew.logw, j + g);
            const int c = (C0 + g) % ET;
#pragma unroll
            for (int i = 0; i < P; ++i) acc[c][i] = pair(acc[c][i], quant(lw + v[g][i]), lut);
        }
    }
}

template <int ET>
__device__ __forceinline__ void fold_group_q16(const float (&v)[G][P], const EdgeMeta& ew, int j, int wn,
                                               int (&acc)[ET][P], const int* __restrict__ lut) {
    if constexpr (ET == 8) {
        if (j & 4)
            fold_group_q16_at<ET, 4>(v, ew, j, wn, acc, lut);
        else
            fold_group_q16_at<ET, 0>(v, ew, j, wn, acc, lut);
    } else {
        fold_group_q16_at<ET, 0>(v, ew, j, wn, acc, lut);
    }
}

// Walks the node's edges in 64-edge windows; groups of GS edges alternate
// between two register buffers (loads of group g+1 in flight while group g
// folds).  FOLD(buf, j, wn, ew) folds group starting at window edge j.
template <int GS, bool VEC, int PP, typename LAYOUT, typename DESC, typename FOLD>
__device__ __forceinline__ void walk_edges(const LAYOUT& L, const DESC& d, const EdgeMeta& first,
                                           const float* __restrict__ child, int64_t batch, int64_t b0, int l,
                                           FOLD fold) {
    for (int64_t w0 = 0; w0 < d.k; w0 += 64) {
        const EdgeMeta ew = w0 == 0 ? first : (w0 + l < d.k ? L.meta(d, w0 + l) : EdgeMeta{0, 0.0f});
        const int wn = (int)(d.k - w0 < 64 ? d.k - w0 : 64);
        const int ng = (wn + GS - 1) / GS;
        float va[GS][PP], vb[GS][PP];
        load_group<GS, VEC, PP>(va, ew, 0, wn, child, batch, b0, l);
        for (int gi = 0; gi < ng; gi += 2) {
            // with VEC the prefetch is unconditional (a group past the window
            // reads empty ranges), keeping every load outside a branch
            if (VEC || gi + 1 < ng) load_group<GS, VEC, PP>(vb, ew, (gi + 1) * GS, wn, child, batch, b0, l);
            fold(va, gi * GS, wn, ew);
            if (gi + 1 >= ng) break;
            if (VEC || gi + 2 < ng) load_group<GS, VEC, PP>(va, ew, (gi + 2) * GS, wn, child, batch, b0, l);
            fold(vb, (gi + 1) * GS, wn, ew);
        }
    }
}

template <bool VEC, typename LAYOUT, typename DESC>
__device__ __forceinline__ void reduce_f32(const LAYOUT& L, const DESC& d, const EdgeMeta& first,
                                           const float* __restrict__ child, int64_t batch, int64_t b0, int l) {
    float m[P], s[P];
#pragma unroll
    for (int i = 0; i < P; ++i) { m[i] = -kInf; s[i] = 0.0f; }
    walk_edges<G, VEC, P>(L, d, first, child, batch, b0, l,
                           [&](const float (&v)[G][P], int j, int wn, const EdgeMeta& ew) {
                               fold_group_f32<P>(v, ew, j, wn, m, s);
                           });
    float res[P];
#pragma unroll
    for (int i = 0; i < P; ++i) res[i] = lse_finish<true>(m[i], s[i]);
    Cols<VEC, P>::store(L.out_row(d), b0, l, batch, res);
}

template <int ET, bool VEC, typename LAYOUT, typename DESC>
__device__ __forceinline__ void reduce_q16_et(const LAYOUT& L, const DESC& d, const EdgeMeta& first,
                                              const float* __restrict__ child, int64_t batch, int64_t b0, int l,
                                              const int* __restrict__ lut) {
    int acc[ET][P];
#pragma unroll
    for (int c = 0; c < ET; ++c)
#pragma unroll
        for (int i = 0; i < P; ++i) acc[c][i] = kNegInfQ;
    walk_edges<G, VEC, P>(L, d, first, child, batch, b0, l,
                          [&](const float (&v)[G][P], int j, int wn, const EdgeMeta& ew) {
                              fold_group_q16<ET>(v, ew, j, wn, acc, lut);
                          });
    float res[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        // xor butterfly over the chains, distances ET/2 .. 1; chain 0 ends with the result
        if constexpr (ET >= 8) {
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c][i] = pair(acc[c][i], acc[c + 4][i], lut);
        }
        if constexpr (ET >= 4) {
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[c][i] = pair(acc[c][i], acc[c + 2][i], lut);
        }
        if constexpr (ET >= 2) acc[0][i] = pair(acc[0][i], acc[1][i], lut);
        res[i] = acc[0][i] > kNegInfQ ? (float)acc[0][i] * kOutScale : -kInf;
    }
    Cols<VEC, P>::store(L.out_row(d), b0, l, batch, res);
}

template <bool VEC, typename LAYOUT, typename DESC>
__device__ __forceinline__ void reduce_q16(const LAYOUT& L, const DESC& d, const EdgeMeta& first,
                                           const float* __restrict__ child, int64_t batch, int64_t b0, int l,
                                           const int* __restrict__ lut) {
    if (d.k <= 8)
        reduce_q16_et<1, VEC>(L, d, first, child, batch, b0, l, lut);
    else if (d.k <= 16)
        reduce_q16_et<2, VEC>(L, d, first, child, batch, b0, l, lut);
    else if (d.k <= 32)
        reduce_q16_et<4, VEC>(L, d, first, child, batch, b0, l, lut);
    else
        reduce_q16_et<8, VEC>(L, d, first, child, batch, b0, l, lut);
}

// One single-wave block per (node, 256-column tile) pair, pairs numbered
// tile-fastest from pair0.  A block lives exactly as long as its own node's
// edge loop: with four nodes per block, a block held its slot until the
// largest of four power-law fan-ins was done, and the Q16 table needed a block
// barrier (C5: Q16 4.70 -> 3.79 ms, fp32 3.37 -> 3.32 ms).  One wave needs no
// barrier for the table: its LDS operations retire in order.  The pair index
// is block-uniform, so the node's descriptor comes through scalar loads.
template <bool Q16, bool VEC, typename LAYOUT>
__global__ __launch_bounds__(64) void sparse_kernel(LAYOUT L, const float* __restrict__ child, int64_t batch,
                                                    int64_t items, int64_t tiles, int64_t pair0) {
    __shared__ int lut[64];
    if constexpr (Q16) {
        lut[threadIdx.x] = kLut[threadIdx.x];
        __builtin_amdgcn_wave_barrier();
    }
    const int l = lane_id();
    const int64_t pair = pair0 + blockIdx.x;
    const int64_t item = pair / tiles;
    if (item >= items) return;
    const auto desc = L.node(item);
    const EdgeMeta first = l < desc.k ? L.meta(desc, l) : EdgeMeta{0, 0.0f};
    const int64_t b0 = (pair - item * tiles) * 64 * P;
    if constexpr (Q16)
        reduce_q16<VEC>(L, desc, first, child, batch, b0, l, lut);
    else
        reduce_f32<VEC>(L, desc, first, child, batch, b0, l);
}

template <bool Q16, typename LAYOUT>
static void launch(const LAYOUT& L, const float* child, const float* out_any, int64_t items, int64_t batch,
                   hipStream_t st) {
    const bool vec = (batch % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(child) | reinterpret_cast<uintptr_t>(out_any)) & 15) == 0;
    const int64_t tile = 64 * P;
    const int64_t tiles = (batch + tile - 1) / tile;
    const int64_t pairs = items * tiles;
    for_grid_chunks(pairs, 64, [&](int64_t p0, int64_t n) {
        if (vec)
            sparse_kernel<Q16, true, LAYOUT><<<dim3((unsigned)n), dim3(64), 0, st>>>(L, child, batch, items, tiles, p0);
        else
            sparse_kernel<Q16, false, LAYOUT><<<dim3((unsigned)n), dim3(64), 0, st>>>(L, child, batch, items, tiles, p0);
    });
}

// ---------------------------------------------------------------------------
// CSR backward (flows).  For out[n, b] = LSE_e(lw_e + child[c_e, b]) and an
// upstream gradient gout:
//   term[e, b]       = gout[n_e, b] * exp(lw_e + child[c_e, b] - out[n_e, b])
//   grad_child[c, b] = sum of term[e, b] over the edges e with c_e = c
//   grad_lw[e]       = sum of term[e, b] over b
// A term whose out[n_e, b] is -inf is 0: nothing flows through a node of
// probability 0 (torch's autograd of logsumexp would give NaN there).
// The kernel walks the transposed structure (CSC: for child c the edges that
// point at it, each with its parent node): one wave per child row, every
// 512-column tile of the batch in turn.  Each child row and each edge belongs
// to one wave.  grad_child is accumulated in registers and written once.
// grad_lw[e] is stored by the first column tile and, for batches over 512
// columns, increased by the later tiles with a no-return atomic add; all of
// these come from lane 0 of the one wave that owns edge e, in tile order, and
// same-address accesses of one lane are performed in program order, so the
// summation order is fixed and the result deterministic.
// ---------------------------------------------------------------------------
struct ParentMeta {
    int64_t node;
    int64_t edge;
    float lw;
};

__device__ __forceinline__ float wave_sum(float v) {
    v += reduce_partner<1>(v);
    v += reduce_partner<2>(v);
    v += reduce_partner<4>(v);
    v += reduce_partner<8>(v);
    v += reduce_partner<16>(v);
    v += reduce_partner<32>(v);
    return v;
}

// Parent edges per load group (two rows each), and columns per lane: 8 columns
// and single-edge groups measured 7.2 ms on the 1M-node C5 layer, against
// 7.8 ms for 4 columns and two-edge groups; the forward keeps 4 columns (8
// measured 3.8 ms against 3.45 ms).
constexpr int GB = 1;

template <bool VEC>
__device__ __forceinline__ void load_parents(float (&gv)[GB][PB], float (&ov)[GB][PB], const ParentMeta& pw, int j,
                                             int wn, const float* __restrict__ gout, const float* __restrict__ out,
                                             int64_t batch, int64_t b0, int l) {
    if constexpr (VEC) {
        // every load issued, as in load_group: parents past wn read empty ranges
        const int rec = cols_bytes(batch, b0);
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            const int64_t n = bcast64(pw.node, (j + g) & 63);
            const int r = j + g < wn ? rec : 0;
            load_cols_buf<PB>(gout + n * batch + b0, r, l, gv[g]);
            load_cols_buf<PB>(out + n * batch + b0, r, l, ov[g]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            if (j + g < wn) {
                const int64_t n = bcast64(pw.node, j + g);
                Cols<VEC, PB>::load(gout + n * batch, b0, l, batch, gv[g]);
                Cols<VEC, PB>::load(out + n * batch, b0, l, batch, ov[g]);
            }
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void flow_group(const float (&gv)[GB][PB], const float (&ov)[GB][PB], const ParentMeta& pw,
                                           int j, int wn, const float (&cv)[PB], float (&acc)[PB], bool first_tile,
                                           float* __restrict__ glogp, int64_t batch, int64_t b0, int l) {
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        if (j + g < wn) {
            const float lw = bcastf(pw.lw, j + g);
            float tsum = 0.0f;
#pragma unroll
            for (int i = 0; i < PB; ++i) {
                const bool live = Cols<VEC, PB>::ok(b0, l, batch, i) && ov[g][i] != -kInf;
                const float t = live ? gv[g][i] * fexp2((lw + cv[i] - ov[g][i]) * kLog2e) : 0.0f;
                acc[i] += t;
                tsum += t;
            }
            tsum = wave_sum(tsum);
            const int64_t e = bcast64(pw.edge, j + g);
            // later tiles add without reading back, so no load sits in the
            // edge loop; only this wave touches edge e, so the adds land in
            // tile order and the result is deterministic
            if (l == 0) {
                if (first_tile)
                    glogp[e] = tsum;
                else
                    __hip_atomic_fetch_add(glogp + e, tsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

template <bool VEC, int WPB>
__global__ __launch_bounds__(64 * WPB) void csr_bwd_kernel(const float* __restrict__ child, const float* __restrict__ out,
                                                      const float* __restrict__ gout, const float* __restrict__ logp,
                                                      const int64_t* __restrict__ csc_off,
                                                      const int32_t* __restrict__ csc_edge,
                                                      const int32_t* __restrict__ csc_node,
                                                      float* __restrict__ gchild, float* __restrict__ glogp,
                                                      int64_t children, int64_t batch, int64_t block0) {
    const int l = lane_id();
    const int64_t c =
        (block0 + (int64_t)blockIdx.x) * WPB + (WPB > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0);
    if (c >= children) return;
    const int64_t p0 = uniform64(csc_off[c]);
    const int64_t k = uniform64(csc_off[c + 1]) - p0;
    for (int64_t b0 = 0; b0 < batch; b0 += 64 * PB) {
        float cv[PB], acc[PB];
        if constexpr (VEC)
            load_cols_buf<PB>(child + c * batch + b0, cols_bytes(batch, b0), l, cv);
        else
            Cols<VEC, PB>::load(child + c * batch, b0, l, batch, cv);
#pragma unroll
        for (int i = 0; i < PB; ++i) acc[i] = 0.0f;
        for (int64_t w0 = 0; w0 < k; w0 += 64) {
            ParentMeta pw{0, 0, 0.0f};
            if (w0 + l < k) {
                const int64_t e = csc_edge[p0 + w0 + l];
                pw = {(int64_t)csc_node[p0 + w0 + l], e, logp[e]};
            }
            const int wn = (int)(k - w0 < 64 ? k - w0 : 64);
            const int ng = (wn + GB - 1) / GB;
            float ga[GB][PB], oa[GB][PB], gb[GB][PB], ob[GB][PB];
            load_parents<VEC>(ga, oa, pw, 0, wn, gout, out, batch, b0, l);
            int gi = 0;
            for (; gi + 1 < ng; gi += 2) {
                load_parents<VEC>(gb, ob, pw, (gi + 1) * GB, wn, gout, out, batch, b0, l);
                flow_group<VEC>(ga, oa, pw, gi * GB, wn, cv, acc, b0 == 0, glogp, batch, b0, l);
                if (VEC || gi + 2 < ng) load_parents<VEC>(ga, oa, pw, (gi + 2) * GB, wn, gout, out, batch, b0, l);
                flow_group<VEC>(gb, ob, pw, (gi + 1) * GB, wn, cv, acc, b0 == 0, glogp, batch, b0, l);
            }
            if (gi < ng) flow_group<VEC>(ga, oa, pw, gi * GB, wn, cv, acc, b0 == 0, glogp, batch, b0, l);
        }
        Cols<VEC, PB>::store(gchild + c * batch, b0, l, batch, acc);
    }
}

}  // namespace sparse
}  // namespace fl

using namespace fl;

extern "C" int fl_sparse_csr_bwd(const float* child, const float* out, const float* grad_out, const float* logparams,
                                 const int64_t* csc_offsets, const int32_t* csc_edges, const int32_t* csc_nodes,
                                 float* grad_child, float* grad_logparams, int64_t num_children, int64_t batch,
                                 void* stream) {
    const char* name = "fl_sparse_csr_bwd";
    FL_CHECK(num_children >= 0 && batch >= 0, "%s: negative size", name);
    if (num_children == 0 || batch == 0) return ok();
    FL_CHECK(child && out && grad_out && logparams && csc_offsets && csc_edges && csc_nodes && grad_child &&
                 grad_logparams,
             "%s: NULL pointer argument", name);
    const bool vec = (batch % 4 == 0) && ((reinterpret_cast<uintptr_t>(child) | reinterpret_cast<uintptr_t>(out) |
                                           reinterpret_cast<uintptr_t>(grad_out) |
                                           reinterpret_cast<uintptr_t>(grad_child)) & 15) == 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for_grid_chunks((num_children + 3) / 4, 256, [&](int64_t b0, int64_t nb) {
        if (vec)
            sparse::csr_bwd_kernel<true, 4><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
                child, out, grad_out, logparams, csc_offsets, csc_edges, csc_nodes, grad_child, grad_logparams,
                num_children, batch, b0);
        else
            sparse::csr_bwd_kernel<false, 4><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
                child, out, grad_out, logparams, csc_offsets, csc_edges, csc_nodes, grad_child, grad_logparams,
                num_children, batch, b0);
    });
    return launch_status(name);
}

extern "C" int fl_sparse_csr_fwd(const float* child, const int64_t* offsets, const int32_t* child_ids,
                                 const float* logparams, float* out, int64_t num_nodes, int64_t batch, int q16,
                                 void* stream) {
    const char* name = "fl_sparse_csr_fwd";
    FL_CHECK(num_nodes >= 0 && batch >= 0, "%s: negative size", name);
    if (num_nodes == 0 || batch == 0) return ok();
    FL_CHECK(child && offsets && out, "%s: NULL pointer argument", name);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const sparse::CsrLayout L{offsets, child_ids, logparams, out, batch};
    if (q16)
        sparse::launch<true>(L, child, out, num_nodes, batch, st);
    else
        sparse::launch<false>(L, child, out, num_nodes, batch, st);
    return launch_status(name);
}

extern "C" int fl_sparse_blocked_fwd(float* node_mars, const float* element_mars, const float* params,
                                     const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t num_nblocks,
                                     int64_t num_edges, int64_t block_size, int64_t batch, int q16, int params_are_log,
                                     void* stream) {
    const char* name = "fl_sparse_blocked_fwd";
    FL_CHECK(num_nblocks >= 0 && num_edges >= 0 && block_size >= 0 && batch >= 0, "%s: negative size", name);
    if (num_nblocks == 0 || block_size == 0 || batch == 0) return ok();
    FL_CHECK(node_mars && element_mars && params && nids && (num_edges == 0 || (cids && pids)),
             "%s: NULL pointer argument", name);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (!q16 && sparse::blocked_mfma_eligible(num_edges, block_size)) {
        sparse::launch_blocked_mfma(node_mars, element_mars, params, nids, cids, pids, num_nblocks, num_edges,
                                    block_size, batch, params_are_log != 0, st);
        return launch_status(name);
    }
    const int64_t items = num_nblocks * block_size;
    if (params_are_log) {
        const sparse::BlockLayout<true> L{node_mars, params, nids, cids, pids, num_edges, block_size, batch};
        if (q16) sparse::launch<true>(L, element_mars, node_mars, items, batch, st);
        else sparse::launch<false>(L, element_mars, node_mars, items, batch, st);
    } else {
        const sparse::BlockLayout<false> L{node_mars, params, nids, cids, pids, num_edges, block_size, batch};
        if (q16) sparse::launch<true>(L, element_mars, node_mars, items, batch, st);
        else sparse::launch<false>(L, element_mars, node_mars, items, batch, st);
    }
    return launch_status(name);
}
