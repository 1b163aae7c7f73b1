// pyjuice block-layout sum layer in fp32 on the matrix cores (gfx950).
//
// The layer (experiment_pyjuice/sparse_float_kernel.cu:40-105): node block j
// holds block_size parents p that share the child ids cids[j, e]; parent p
// weighs edge e with w[p, e] = params[pids[j, e] + p] and writes
//     node_mars[nids[j] + p, b] = log sum_e w[p, e] * exp(element_mars[cids[j, e], b]).
// With the column maximum m_b = max_e element_mars[cids[j, e], b] and the row
// maximum W_p = max_e w[p, e] this is
//     node_mars[nids[j] + p, b] = log W_p + m_b + log S[p, b],
//     S[p, b] = sum_e (w[p, e] / W_p) * exp(element_mars[cids[j, e], b] - m_b),
// a [block_size x num_edges] by [num_edges x batch] product of factors in
// [0, 1].  The reference computes each (p, b) as its own chain of pairwise
// log-sum-exps, gathering every child row once per parent; here each child
// value is loaded and exponentiated once per block and the product runs on
// v_mfma_f32_16x16x4_f32.
//
// Mapping: one wave per (node block, group of 16*MT parents, tile of 16*NT
// batch columns).  In each 16x16x4 product lane l supplies A[l%16][l/16]
// (parent row) and B[l/16][l%16] (edge row, column) and holds
// D[4*(l/16) + r][l%16], r < 4.  Column j of N-tile t = 4*q + u is batch
// column b0 + 64*q + 4*j + u, so lane l loads one 16-byte vector (columns
// b0 + 64*q + 4*(l%16) .. +3) of the child row of edge 4*ks + l/16 per q and
// that vector is its B operand for the four N-tiles 4*q .. 4*q + 3; the
// results of row p come back as the same four consecutive columns, one
// 16-byte store.  Edges are taken up to 32 at a time (2, 4 or 8 K-steps of
// 4); the row maxima of the weights and the column maxima of the child values
// are kept online across chunks, rescaling the accumulators, so every weight
// and child value is loaded once.
//
// Accuracy: every term is >= 0, so S carries only rounding of fp32 products
// and sums.  Terms below 2^-126 may flush to zero, losing at most
// num_edges * 2^-126 of S.  Where S < num_edges * 2^-102 (that loss could
// exceed 2^-24 of S), or S is not finite (non-finite inputs), the entry is
// recomputed by the exact online log-sum-exp over its edges, with the special
// values of the robust fold (NaN wins, +inf wins, -inf is the identity).
#include <math.h>
#include <stdint.h>
#include <type_traits>

#include "lse_blocked.hpp"
#include "lse_common.hpp"

namespace fl {
namespace sparse {

namespace {

constexpr int KSMAX = 8;        // K-steps of 4 edges per chunk, at most
constexpr int KCMAX = 4 * KSMAX;  // edges per chunk, at most

__device__ __forceinline__ float lane_read(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src * 4, __builtin_bit_cast(int, v)));
}

// The weight entering the linear product: the reference floors linear weights
// at 1e-45 before its log (sparse_float_kernel.cu:76).
template <bool LOGP>
__device__ __forceinline__ float weight_term(float w) {
    return LOGP ? w : fmaxf(w, 1e-45f);
}

// Child values of chunk edges c0 + 4*ks + kq at the lane's four columns;
// edges past ne read -inf (their addresses clamped to edge ne - 1), columns
// past the batch read 0 (never stored).  FULL: every edge of the chunk and
// every column of the tile is in range (a wave-uniform fact), so the values
// are taken as loaded.
template <int NK, int NT, bool VEC, bool FULL>
__device__ __forceinline__ void load_chunk(float (&x)[NK][NT], const float* __restrict__ child,
                                           const int64_t* __restrict__ cids, int64_t ebase, int64_t ne, int64_t c0,
                                           int kq, int64_t col, int64_t batch) {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
        const int64_t e = c0 + 4 * ks + kq;
        const bool ev = FULL || e < ne;
        const float* row = child + cids[ebase + (ev ? e : ne - 1)] * batch;
#pragma unroll
        for (int q = 0; q < NT / 4; ++q) {
            const int64_t cq = col + 64 * q;
            if constexpr (VEC) {
                const bool cv = FULL || cq < batch;
                const f32x4 v = *reinterpret_cast<const f32x4*>(row + (cv ? cq : 0));
                x[ks][4 * q] = ev ? (cv ? v.x : 0.0f) : -kInf;
                x[ks][4 * q + 1] = ev ? (cv ? v.y : 0.0f) : -kInf;
                x[ks][4 * q + 2] = ev ? (cv ? v.z : 0.0f) : -kInf;
                x[ks][4 * q + 3] = ev ? (cv ? v.w : 0.0f) : -kInf;
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const bool cv = FULL || cq + t < batch;
                    const float v = row[cv ? cq + t : 0];
                    x[ks][4 * q + t] = ev ? (cv ? v : 0.0f) : -kInf;
                }
            }
        }
    }
}

// Raw weights of chunk edges c0 + 4*ks + kq for parents p0 + 16*mt + jc
// (the lane's A-layout entries); invalid entries read as -inf (log weights)
// or 0 (linear weights), the identity of the row maximum.  FULL: every edge
// and parent is in range.
template <int MT, int NK, bool LOGP, bool FULL>
__device__ __forceinline__ void load_weights(float (&w)[MT][NK], const float* __restrict__ params,
                                             const int64_t* __restrict__ pids, int64_t ebase, int64_t ne, int64_t bs,
                                             int64_t c0, int64_t p0, int kq, int jc) {
#pragma unroll
    for (int ks = 0; ks < NK; ++ks) {
        const int64_t e = c0 + 4 * ks + kq;
        const bool ev = FULL || e < ne;
        const int64_t q = pids[ebase + (ev ? e : ne - 1)];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int64_t p = p0 + 16 * mt + jc;
            const bool pv = FULL || p < bs;
            const float v = weight_term<LOGP>(params[q + (pv ? p : bs - 1)]);
            w[mt][ks] = ev && pv ? v : (LOGP ? -kInf : 0.0f);
        }
    }
}

// Folds one chunk into the accumulators: online row maxima of the weights
// (A layout, wm) and column maxima of the child values (m), the accumulators
// rescaled to both (FIRST: nothing accumulated yet), then
// acc += (w / wm) x exp(x - m) on the matrix cores.
template <int MT, int NK, int NT, bool LOGP, bool FIRST>
__device__ __forceinline__ void fold_chunk(f32x4 (&acc)[MT][NT], float (&wm)[MT], float (&m)[NT],
                                           float (&x)[NK][NT], float (&w)[MT][NK], int kq) {
    float beta[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        float cw = w[mt][0];
#pragma unroll
        for (int ks = 1; ks < NK; ++ks) cw = fmaxf(cw, w[mt][ks]);
        cw = max_pair32(max_pair16(cw));
        const float nw = fmaxf(wm[mt], cw);
        if constexpr (LOGP) {
            beta[mt] = wm[mt] == -kInf ? 0.0f : fexp2((wm[mt] - nw) * kLog2e);
        } else {
            beta[mt] = wm[mt] / nw;
        }
        wm[mt] = nw;
    }
    // normalised weights, in place: w / wm (linear) or exp(w - wm) (log)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const float rinv = LOGP ? 0.0f : 1.0f / wm[mt];
#pragma unroll
        for (int ks = 0; ks < NK; ++ks)
            w[mt][ks] = LOGP ? (wm[mt] == -kInf ? 0.0f : fexp2((w[mt][ks] - wm[mt]) * kLog2e)) : w[mt][ks] * rinv;
    }
    float alpha[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float cm = x[0][t];
#pragma unroll
        for (int ks = 1; ks < NK; ++ks) cm = fmaxf(cm, x[ks][t]);
        cm = max_pair32(max_pair16(cm));
        const float mn = fmaxf(m[t], cm);
        alpha[t] = m[t] == -kInf ? 0.0f : fexp2((m[t] - mn) * kLog2e);
        m[t] = mn;
        // a column of -inf (and NaN) children so far is taken relative to 0:
        // its -inf terms are exp(-inf) = 0 and a NaN stays NaN, to reach the
        // exact fold (a select of 0 for every term of such a column would drop
        // a NaN that later chunks' finite children then hide)
        const float mz = mn == -kInf ? 0.0f : mn;
#pragma unroll
        for (int ks = 0; ks < NK; ++ks) x[ks][t] = fexp2((x[ks][t] - mz) * kLog2e);
    }
    if constexpr (!FIRST) {
        // D-layout row 16*mt + 4*kq + r takes the row factor of A-layout lane 4*kq + r
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float br = lane_read(beta[mt], 4 * kq + r);
#pragma unroll
                for (int t = 0; t < NT; ++t) acc[mt][t][r] *= br * alpha[t];
            }
    }
#pragma unroll
    for (int ks = 0; ks < NK; ++ks)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int t = 0; t < NT; ++t)
                acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[mt][ks], x[ks][t], acc[mt][t], 0, 0, 0);
}

// Loads and folds the NK K-steps of edges from c0.
template <int MT, int NK, int NT, bool VEC, bool LOGP, bool FIRST, bool FULL = false>
__device__ __forceinline__ void load_fold(f32x4 (&acc)[MT][NT], float (&wm)[MT], float (&m)[NT],
                                          const float* __restrict__ child, const float* __restrict__ params,
                                          const int64_t* __restrict__ cids, const int64_t* __restrict__ pids,
                                          int64_t ebase, int64_t ne, int64_t bs, int64_t c0, int64_t p0, int kq,
                                          int jc, int64_t col, int64_t batch) {
    float x[NK][NT], w[MT][NK];
    load_chunk<NK, NT, VEC, FULL>(x, child, cids, ebase, ne, c0, kq, col, batch);
    load_weights<MT, NK, LOGP, FULL>(w, params, pids, ebase, ne, bs, c0, p0, kq, jc);
    fold_chunk<MT, NK, NT, LOGP, FIRST>(acc, wm, m, x, w, kq);
}

// True where the product cannot resolve the entry: S outside [thr, 2^100],
// NaN and +inf included (S is a sum of products of non-negative factors, so
// never below +0).  The floats of [thr, 2^100] are one interval of unsigned
// bit patterns: one subtraction and one unsigned compare.
__device__ __forceinline__ bool unresolved(float s, uint32_t lo, uint32_t span) {
    return __builtin_bit_cast(uint32_t, s) - lo > span;
}

// Writes a tile's results, node_mars[nrow0 + p, c] = log W_p + m_c + log S, for
// the parents and columns in range (D layout: lane l holds rows
// p0 + 16*mt + 4*kq + r; lwm: log W in the A layout, row 16*mt + jc at lane
// jc, so D row 16*mt + 4*kq + r reads lane 4*kq + r).  Entries the product
// cannot resolve (rare: see the accuracy note above) are only flagged in the
// store loop; a lane with any recomputes them by the exact online log-sum-exp
// over the block's edges and stores them over the product's value.
template <int MT, int NT, bool VEC, bool LOGP>
__device__ __forceinline__ void store_tile(float* __restrict__ node_mars, const float* __restrict__ child,
                                           const float* __restrict__ params, const int64_t* __restrict__ cids,
                                           const int64_t* __restrict__ pids, int64_t ebase, int64_t ne, int64_t bs,
                                           int64_t batch, int64_t nrow0, int64_t p0, int kq, int64_t col,
                                           const f32x4 (&acc)[MT][NT], const float (&lwm)[MT],
                                           const float (&m)[NT]) {
    const float thr = (float)ne * 0x1p-102f;
    const uint32_t lo = __builtin_bit_cast(uint32_t, thr);
    const uint32_t span = __builtin_bit_cast(uint32_t, 0x1p100f) - lo;
    static_assert(MT * 4 * NT <= 64, "one bit per held entry");
    using Mask = typename std::conditional<MT * 4 * NT <= 32, uint32_t, uint64_t>::type;
    Mask redo = 0;  // bit (4*mt + r)*NT + t: entry left to the exact fold
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float lwr = lane_read(lwm[mt], 4 * kq + r);
            const int64_t p = p0 + 16 * mt + 4 * kq + r;
            if (p >= bs) continue;
            float* orow = node_mars + (nrow0 + p) * batch;
#pragma unroll
            for (int q = 0; q < NT / 4; ++q) {
                const int64_t cq = col + 64 * q;
                float res[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float s = acc[mt][4 * q + u][r];
                    res[u] = lwr + m[4 * q + u] + flog2(s) * kLn2;
                    const bool bad = unresolved(s, lo, span) && (VEC ? cq : cq + u) < batch;
                    redo |= bad ? (Mask)1 << ((4 * mt + r) * NT + 4 * q + u) : (Mask)0;
                }
                if constexpr (VEC) {
                    if (cq < batch) store_stream(f32x4{res[0], res[1], res[2], res[3]}, orow + cq);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (cq + u < batch) orow[cq + u] = res[u];
                }
            }
        }
    while (redo) {
        const int bit = __builtin_ctzll((uint64_t)redo);
        redo &= redo - 1;
        const int mr = bit / NT, t = bit % NT;
        const int64_t p = p0 + 16 * (mr >> 2) + 4 * kq + (mr & 3);
        const int64_t c = col + 64 * (t >> 2) + (t & 3);
        float mm = -kInf, ss = 0.0f;
        for (int64_t e = 0; e < ne; ++e) {
            const float w = params[pids[ebase + e] + p];
            const float lw = LOGP ? w : logf(fmaxf(w, 1e-45f));
            const float v[1] = {lw + child[cids[ebase + e] * batch + c]};
            lse_fold<true, 1>(mm, ss, v);
        }
        node_mars[(nrow0 + p) * batch + c] = lse_finish<true>(mm, ss);
    }
}

}  // namespace

// Waves per SIMD the register allocation must allow: four for a single chunk
// (the accumulators then live in VGPRs, not AGPRs: 101 registers instead of
// 86 + 44 for 32 parents, four waves instead of three) and for several chunks
// of 32 parents (128 registers instead of 132 + 52: four waves instead of
// two), three for several chunks of 16 parents; 64 parents with 32 edges keep
// the default allocation (three waves; four would spill), and several chunks
// never take 64 parents.
constexpr int fwd_min_waves(int mt, int nk, bool multi) {
    return mt == 4 ? (nk == 8 || multi ? 1 : 4) : multi ? (mt == 2 ? 4 : 3) : 4;
}

// One wave per (node block j, parent group g, column tile ct), W consecutive
// column tiles per workgroup (wave w of workgroup cg takes ct = W*cg + w);
// logical workgroup ids run cg fastest, then g, then j, and are dealt to the
// XCDs in contiguous ranges (physical workgroup w runs on XCD w % 8), so the
// column tiles and parent groups of one node block share an L2 for the
// block's weights and child rows.  NK: K-steps of the single chunk when ne <= 4*NK; MULTI: any
// ne, in chunks of 32 edges and a tail of 8, 16 or 32.
template <int MT, int NK, int NT, bool MULTI, bool VEC, bool LOGP, int W>
__global__ __launch_bounds__(64 * W, fwd_min_waves(MT, NK, MULTI)) void blocked_mfma_kernel(
    float* __restrict__ node_mars, const float* __restrict__ child, const float* __restrict__ params,
    const int64_t* __restrict__ nids, const int64_t* __restrict__ cids, const int64_t* __restrict__ pids, int64_t ne,
    int64_t bs, int64_t batch, int64_t ctiles, int64_t pgroups, int64_t items, int64_t id0) {
    const int64_t per_xcd = gridDim.x / 8;
    const int64_t id = id0 + (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (id >= items) return;
    const int64_t cgroups = (ctiles + W - 1) / W;
    const int64_t ct = id % cgroups * W + (int64_t)(threadIdx.x >> 6);
    if (ct >= ctiles) return;
    const int64_t jg = id / cgroups;
    const int64_t g = jg % pgroups;
    const int64_t j = jg / pgroups;
    const int l = lane_id();
    const int kq = l >> 4;
    const int jc = l & 15;
    const int64_t col = ct * 16 * NT + 4 * jc;  // N-tile t: column col + 64*(t/4) + t%4
    const int64_t ebase = j * ne;
    const int64_t p0 = g * 16 * MT;

    float m[NT], wm[MT];
    f32x4 acc[MT][NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        m[t] = -kInf;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) wm[mt] = LOGP ? -kInf : 0.0f;

    if constexpr (!MULTI) {
        // the masks of edges, parents and columns past their ends are all
        // true for a whole chunk of a whole tile: that case takes a copy of
        // the fold without them
        if (ne == 4 * NK && p0 + 16 * MT <= bs && (ct + 1) * 16 * NT <= batch)
            load_fold<MT, NK, NT, VEC, LOGP, true, true>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, 0, p0,
                                                         kq, jc, col, batch);
        else
            load_fold<MT, NK, NT, VEC, LOGP, true, false>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, 0, p0,
                                                          kq, jc, col, batch);
    } else {
        // full chunks of KCMAX edges, one at a time (a second buffer in flight
        // cost more in occupancy than it hid), then the rest in the smallest
        // chunk that holds it
        load_fold<MT, KSMAX, NT, VEC, LOGP, true>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, 0, p0, kq,
                                                  jc, col, batch);
        int64_t c0 = KCMAX;
        for (; c0 + KCMAX <= ne; c0 += KCMAX)
            load_fold<MT, KSMAX, NT, VEC, LOGP, false>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, c0, p0,
                                                       kq, jc, col, batch);
        const int64_t rest = ne - c0;
        if (rest > 16)
            load_fold<MT, KSMAX, NT, VEC, LOGP, false>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, c0, p0,
                                                       kq, jc, col, batch);
        else if (rest > 8)
            load_fold<MT, 4, NT, VEC, LOGP, false>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, c0, p0, kq,
                                                   jc, col, batch);
        else if (rest > 0)
            load_fold<MT, 2, NT, VEC, LOGP, false>(acc, wm, m, child, params, cids, pids, ebase, ne, bs, c0, p0, kq,
                                                   jc, col, batch);
    }

    float lwm[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) lwm[mt] = LOGP ? wm[mt] : logf(wm[mt]);
    store_tile<MT, NT, VEC, LOGP>(node_mars, child, params, cids, pids, ebase, ne, bs, batch, nids[j], p0, kq, col,
                                  acc, lwm, m);
}

// Parents per product row group: 16, 32 or 64.  Groups of 64 suit one chunk
// of edges (bs = 64, ne = 32: 197 us against 211 with two groups of 32); with
// several chunks their larger register set costs occupancy (bs = 64, ne = 64:
// 475 us against 401), so those take groups of 32.
static int blocked_mt(int64_t bs, int64_t ne) { return bs <= 16 ? 1 : bs <= 32 || ne > KCMAX ? 2 : 4; }

template <int MT, int NK, int NT, bool MULTI, bool VEC, bool LOGP, int W>
static void launch_kw(float* node_mars, const float* child, const float* params, const int64_t* nids,
                      const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                      int64_t batch, int64_t ctiles, hipStream_t st) {
    const int64_t pgroups = (bs + 16 * MT - 1) / (16 * MT);
    const int64_t items = nblocks * pgroups * ((ctiles + W - 1) / W);
    constexpr int64_t kMax = max_grid_blocks(64 * W);  // workgroups per launch, a multiple of 8
    for (int64_t id0 = 0; id0 < items; id0 += kMax) {
        const int64_t n = items - id0 < kMax ? items - id0 : kMax;
        const unsigned grid = (unsigned)((n + 7) / 8 * 8);
        blocked_mfma_kernel<MT, NK, NT, MULTI, VEC, LOGP, W><<<dim3(grid), dim3(64 * W), 0, st>>>(
            node_mars, child, params, nids, cids, pids, ne, bs, batch, ctiles, pgroups, items, id0);
    }
}

// Column tiles of one (node block, parent group) go to the waves of one
// workgroup, four at a time, so one CU reads 4 * 16 * NT consecutive columns
// of each child row and writes them of each parent row.  The rows are
// gathered, and a CU taking a kilobyte of a row at once instead of a quarter
// of it reads and writes the layer's bytes 13% faster: a copy with this
// kernel's loads and stores over the bench layer's child ids takes 159 us in
// four-wave workgroups against 183 us in one-wave ones.
template <int MT, int NK, int NT, bool MULTI, bool VEC, bool LOGP>
static void launch_k(float* node_mars, const float* child, const float* params, const int64_t* nids,
                     const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                     int64_t batch, hipStream_t st) {
    const int64_t ctiles = (batch + 16 * NT - 1) / (16 * NT);
    if (ctiles >= 4)
        launch_kw<MT, NK, NT, MULTI, VEC, LOGP, 4>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch,
                                                   ctiles, st);
    else
        launch_kw<MT, NK, NT, MULTI, VEC, LOGP, 1>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch,
                                                   ctiles, st);
}

template <int MT, bool VEC, bool LOGP>
static void launch_mt(float* node_mars, const float* child, const float* params, const int64_t* nids,
                      const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                      int64_t batch, hipStream_t st) {
    // 16x16 N-tiles per wave (16 * NT batch columns).  One parent group of 16
    // takes 128 columns (more bytes in flight per wave: bs = 16, ne = 32 at
    // batch 512, 337 -> 291 us); with 32 or 64 parents the larger accumulator
    // set cost occupancy and time (256 -> 388 us at bs = 32), so they take 64.
    constexpr int NT = MT == 1 ? 8 : 4;
    if (ne <= 8)
        launch_k<MT, 2, NT, false, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
    else if (ne <= 16)
        launch_k<MT, 4, NT, false, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
    else if (ne <= KCMAX)
        launch_k<MT, KSMAX, NT, false, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch,
                                                  st);
    else
        launch_k<MT, KSMAX, NT, true, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch,
                                                 st);
}

template <bool VEC, bool LOGP>
static void launch_vec_log(float* node_mars, const float* child, const float* params, const int64_t* nids,
                           const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                           int64_t batch, hipStream_t st) {
    switch (blocked_mt(bs, ne)) {
        case 1: launch_mt<1, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st); break;
        case 2: launch_mt<2, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st); break;
        default: launch_mt<4, VEC, LOGP>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st); break;
    }
}

// Block sizes from which the product form replaces the per-parent gather.
bool blocked_mfma_eligible(int64_t ne, int64_t bs) { return ne > 0 && bs >= kBlockedMfmaMinBs; }

void launch_blocked_mfma(float* node_mars, const float* child, const float* params, const int64_t* nids,
                         const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                         int64_t batch, bool params_are_log, hipStream_t st) {
    const bool vec = (batch % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(child) | reinterpret_cast<uintptr_t>(node_mars)) & 15) == 0;
    if (vec) {
        if (params_are_log) launch_vec_log<true, true>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
        else launch_vec_log<true, false>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
    } else {
        if (params_are_log) launch_vec_log<false, true>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
        else launch_vec_log<false, false>(node_mars, child, params, nids, cids, pids, nblocks, ne, bs, batch, st);
    }
}

}  // namespace sparse
}  // namespace fl
