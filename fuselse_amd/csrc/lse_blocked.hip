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
// Mapping: one wave per (node block, group of 16*MT parents, 64-column tile).
// In each 16x16x4 product lane l supplies A[l%16][l/16] (parent row) and
// B[l/16][l%16] (edge row, column) and holds D[4*(l/16) + r][l%16], r < 4.
// Column j of N-tile t is batch column b0 + 4*j + t, so lane l loads one
// 16-byte vector (columns b0 + 4*(l%16) .. +3) of the child row of edge
// 4*ks + l/16 and that vector is its B operand for the four N-tiles t; the
// results of row p come back as the same four consecutive columns, one
// 16-byte store.  Edges are taken 32 at a time (8 K-steps); the column
// maximum is kept online across chunks, rescaling the accumulators.
//
// Accuracy: every term is >= 0, so S carries only rounding of fp32 products
// and sums.  Terms below 2^-126 may flush to zero, losing at most
// num_edges * 2^-126 of S.  Where S < num_edges * 2^-102 (that loss could
// exceed 2^-24 of S), or S is not finite (non-finite inputs), the entry is
// recomputed by the exact online log-sum-exp over its edges, with the special
// values of the robust fold (NaN wins, +inf wins, -inf is the identity).
#include <math.h>
#include <stdint.h>

#include "lse_blocked.hpp"
#include "lse_common.hpp"

namespace fl {
namespace sparse {

namespace {

constexpr int KC = 32;      // edges per chunk
constexpr int KS = KC / 4;  // K-steps per chunk

__device__ __forceinline__ float xor16(float v) { return exact_xor<16>(v); }
__device__ __forceinline__ float xor32(float v) { return exact_xor<32>(v); }

// The weight entering the linear product: the reference floors linear weights
// at 1e-45 before its log (sparse_float_kernel.cu:76).
template <bool LOGP>
__device__ __forceinline__ float weight_term(float w) {
    return LOGP ? w : fmaxf(w, 1e-45f);
}

// Child values of chunk edges c0 + 4*ks + kq at the lane's four columns;
// edges past ne read -inf, columns past the batch read 0 (never stored).
template <bool VEC>
__device__ __forceinline__ void load_chunk(float (&x)[KS][4], const float* __restrict__ child,
                                           const int64_t* __restrict__ cids, int64_t ebase, int64_t ne, int64_t c0,
                                           int kq, int64_t col, int64_t batch) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int64_t e = c0 + 4 * ks + kq;
        const bool ev = e < ne;
        const float* row = child + cids[ebase + (ev ? e : ne - 1)] * batch;
        if constexpr (VEC) {
            const bool cv = col < batch;
            const f32x4 v = *reinterpret_cast<const f32x4*>(row + (cv ? col : 0));
            x[ks][0] = ev ? (cv ? v.x : 0.0f) : -kInf;
            x[ks][1] = ev ? (cv ? v.y : 0.0f) : -kInf;
            x[ks][2] = ev ? (cv ? v.z : 0.0f) : -kInf;
            x[ks][3] = ev ? (cv ? v.w : 0.0f) : -kInf;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bool cv = col + t < batch;
                const float v = row[cv ? col + t : 0];
                x[ks][t] = ev ? (cv ? v : 0.0f) : -kInf;
            }
        }
    }
}

// Raw weights of chunk edges c0 + 4*ks + kq for parents p0 + 16*mt + jc
// (the lane's A-layout entries); invalid entries read as -inf (log weights)
// or 0 (linear weights), the identity of the row maximum.
template <int MT, bool LOGP>
__device__ __forceinline__ void load_weights(float (&w)[MT][KS], const float* __restrict__ params,
                                             const int64_t* __restrict__ pids, int64_t ebase, int64_t ne, int64_t bs,
                                             int64_t c0, int64_t p0, int kq, int jc) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int64_t e = c0 + 4 * ks + kq;
        const bool ev = e < ne;
        const int64_t q = pids[ebase + (ev ? e : ne - 1)];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int64_t p = p0 + 16 * mt + jc;
            const bool pv = p < bs;
            const float v = weight_term<LOGP>(params[q + (pv ? p : bs - 1)]);
            w[mt][ks] = ev && pv ? v : (LOGP ? -kInf : 0.0f);
        }
    }
}

}  // namespace

// One wave per (node block j, parent group g, column tile ct); logical ids
// run ct fastest, then g, then j, and are dealt to the XCDs in contiguous
// ranges (physical workgroup w runs on XCD w % 8), so the column tiles and
// parent groups of one node block share an L2 for the block's weights and
// child rows.
template <int MT, bool VEC, bool LOGP, bool ONE>
__global__ __launch_bounds__(64) void blocked_mfma_kernel(float* __restrict__ node_mars,
                                                          const float* __restrict__ child,
                                                          const float* __restrict__ params,
                                                          const int64_t* __restrict__ nids,
                                                          const int64_t* __restrict__ cids,
                                                          const int64_t* __restrict__ pids, int64_t ne, int64_t bs,
                                                          int64_t batch, int64_t ctiles, int64_t pgroups,
                                                          int64_t items, int64_t id0) {
    const int64_t per_xcd = gridDim.x / 8;
    const int64_t id = id0 + (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (id >= items) return;
    const int64_t ct = id % ctiles;
    const int64_t jg = id / ctiles;
    const int64_t g = jg % pgroups;
    const int64_t j = jg / pgroups;
    const int l = lane_id();
    const int kq = l >> 4;
    const int jc = l & 15;
    const int64_t col = ct * 64 + 4 * jc;
    const int64_t ebase = j * ne;
    const int64_t p0 = g * 16 * MT;

    // Weights, A layout (row p0 + 16*mt + jc, edge c0 + 4*ks + kq), and their
    // row maxima over all edges.  With a single chunk (ONE) they are loaded
    // once; otherwise a first pass takes the maxima and each chunk reloads.
    float wr[MT][KS];
    float wmax[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) wmax[mt] = LOGP ? -kInf : 0.0f;
    for (int64_t c0 = 0; c0 < (ONE ? 1 : ne); c0 += KC) {
        load_weights<MT, LOGP>(wr, params, pids, ebase, ne, bs, c0, p0, kq, jc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) wmax[mt] = fmaxf(wmax[mt], wr[mt][ks]);
    }
    float rinv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        wmax[mt] = fmaxf(wmax[mt], xor16(wmax[mt]));
        wmax[mt] = fmaxf(wmax[mt], xor32(wmax[mt]));
        rinv[mt] = LOGP ? 0.0f : 1.0f / wmax[mt];
    }

    float m[4];
    f32x4 acc[MT][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        m[t] = -kInf;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    for (int64_t c0 = 0; c0 < ne; c0 += KC) {
        float x[KS][4];
        load_chunk<VEC>(x, child, cids, ebase, ne, c0, kq, col, batch);
        if (!ONE) load_weights<MT, LOGP>(wr, params, pids, ebase, ne, bs, c0, p0, kq, jc);
        float a[MT][KS];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const bool valid = c0 + 4 * ks + kq < ne && p0 + 16 * mt + jc < bs;
                const float wn = LOGP ? fexp2((wr[mt][ks] - wmax[mt]) * kLog2e) : wr[mt][ks] * rinv[mt];
                a[mt][ks] = valid ? wn : 0.0f;
            }
        // online column maximum; lanes l, l^16, l^32, l^48 share columns
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float cm = x[0][t];
#pragma unroll
            for (int ks = 1; ks < KS; ++ks) cm = fmaxf(cm, x[ks][t]);
            cm = fmaxf(cm, xor16(cm));
            cm = fmaxf(cm, xor32(cm));
            const float mn = fmaxf(m[t], cm);
            const float alpha = m[t] == -kInf ? 0.0f : fexp2((m[t] - mn) * kLog2e);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][t] *= alpha;
            m[t] = mn;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) x[ks][t] = mn == -kInf ? 0.0f : fexp2((x[ks][t] - mn) * kLog2e);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][ks], x[ks][t], acc[mt][t], 0, 0, 0);
    }

    // D layout: lane l holds rows p0 + 16*mt + 4*kq + r.  Their weight maxima
    // live in A-layout lane 4*kq + r.
    const float thr = (float)ne * 0x1p-102f;
    const int64_t nrow0 = nids[j];
    uint64_t redo = 0;  // bit 16*mt + 4*r + t: entry left to the exact fold
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const float lwm = LOGP ? wmax[mt] : logf(wmax[mt]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float lwr = __builtin_bit_cast(
                float, __builtin_amdgcn_ds_bpermute((4 * kq + r) * 4, __builtin_bit_cast(int, lwm)));
            const int64_t p = p0 + 16 * mt + 4 * kq + r;
            if (p >= bs) continue;
            float res[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float s = acc[mt][t][r];
                res[t] = lwr + m[t] + flog2(s) * kLn2;
                if (!(s >= thr && s <= 0x1p100f) && col + t < batch) redo |= (uint64_t)1 << (16 * mt + 4 * r + t);
            }
            float* orow = node_mars + (nrow0 + p) * batch;
            if constexpr (VEC) {
                if (col < batch) *reinterpret_cast<f32x4*>(orow + col) = f32x4{res[0], res[1], res[2], res[3]};
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (col + t < batch) orow[col + t] = res[t];
            }
        }
    }
    // Entries the product cannot resolve (rare: see the accuracy note above),
    // recomputed by the exact online log-sum-exp over the block's edges and
    // stored over the product's value by the same lane.
    while (redo) {
        const int bit = __builtin_ctzll(redo);
        redo &= redo - 1;
        const int64_t p = p0 + 16 * (bit >> 4) + 4 * kq + ((bit >> 2) & 3);
        const int64_t c = col + (bit & 3);
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

// Parents per product row group: 16, 32 or 64.
static int blocked_mt(int64_t bs) { return bs <= 16 ? 1 : bs <= 32 ? 2 : 4; }

template <int MT, bool VEC, bool LOGP>
static void launch_mt(float* node_mars, const float* child, const float* params, const int64_t* nids,
                      const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                      int64_t batch, hipStream_t st) {
    const int64_t ctiles = (batch + 63) / 64;
    const int64_t pgroups = (bs + 16 * MT - 1) / (16 * MT);
    const int64_t items = nblocks * pgroups * ctiles;
    constexpr int64_t kMax = (int64_t)1 << 30;  // workgroups per launch, a multiple of 8
    for (int64_t id0 = 0; id0 < items; id0 += kMax) {
        const int64_t n = items - id0 < kMax ? items - id0 : kMax;
        const unsigned grid = (unsigned)((n + 7) / 8 * 8);
        if (ne <= KC)
            blocked_mfma_kernel<MT, VEC, LOGP, true><<<dim3(grid), dim3(64), 0, st>>>(
                node_mars, child, params, nids, cids, pids, ne, bs, batch, ctiles, pgroups, items, id0);
        else
            blocked_mfma_kernel<MT, VEC, LOGP, false><<<dim3(grid), dim3(64), 0, st>>>(
                node_mars, child, params, nids, cids, pids, ne, bs, batch, ctiles, pgroups, items, id0);
    }
}

template <bool VEC, bool LOGP>
static void launch_vec_log(float* node_mars, const float* child, const float* params, const int64_t* nids,
                           const int64_t* cids, const int64_t* pids, int64_t nblocks, int64_t ne, int64_t bs,
                           int64_t batch, hipStream_t st) {
    switch (blocked_mt(bs)) {
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
