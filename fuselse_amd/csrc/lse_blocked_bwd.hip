// Backward ("flows") of the pyjuice block-layout fp32 sum layer, as products
// on the matrix cores (gfx950).  The reference has no sparse backward; this
// is the derivative of its block-layout forward (experiment_pyjuice/
// sparse_float_kernel.cu:40-105).  For node block j, parent p (node
// n = nids[j] + p), edge e (child c = cids[j, e], weight
// w[p, e] = params[pids[j, e] + p], floored at 1e-45 or given as a log) and
// batch column b, with g = node_flows, o = node_mars (the forward's output)
// and x = element_mars:
//     T[p, e, b] = g[n, b] * w[p, e] * exp(x[c, b] - o[n, b])   (0 where o = -inf)
//     edge flow   F[j, e, b] = sum over p of T
//     param flow  P[p, e]    = sum over b of T,  param_flows[pids[j, e] + p] += P
//     element_flows[c, b]   += sum of F[j, e, b] over the block edges (j, e) into c.
// For any per-column reference m_b and per-row reference W_p,
//     T = A[p, e] * X[e, b] * R[p, b],  A = w / W,  X = exp(x - m),
//     R = g * exp(log W + m - o),
// so F = X .* (A^T R) is a product over parents and P = A .* (R X^T) a
// product over the batch.  Each kernel takes m and W as the maxima over the
// 32-edge chunk it works on, so A, X <= 1, and R <= 2^24 |g| wherever
// log W + m - o <= 16.6.  Pairs (p, b) past that bound (a parent far below the
// scale of its heavy children, or non-finite values) are left out of the
// product and their terms computed one by one as T = g * exp(lw + x - o).
// A term lost to fp32 underflow in the product is below 2^-102 |g|.
//
// Kernels: edge flows (one wave per block, edge chunk and 64-column tile, the
// parents as the product's K), parameter flows (one wave per block, edge
// chunk and parent group, the batch as K, the sums added to param_flows once
// per (p, e)), and element flows (one wave per element row, its block edges
// summed in a fixed order through the transposed structure).  Blocks of at
// most 32 parents take both products in one pass instead (blocked_bwd_fused).
// The result does not depend on scheduling, except that parameters shared by
// several (block, parent, edge) triples receive their sums in any order.
#include <math.h>
#include <stdint.h>

#include "../../include/fuselse_amd.h"
#include "fl_status.hpp"
#include "lse_common.hpp"
#include "lse_tile_layout.hpp"

namespace fl {
namespace sparse {

namespace {

constexpr int CE = 32;          // edges per chunk
constexpr float kRMax = 16.6f;  // largest log W + m - o taken by the product

__device__ __forceinline__ float lane_read(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src * 4, __builtin_bit_cast(int, v)));
}
// maximum over the 16 lanes of a row (lanes 16*i .. 16*i + 15)
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, reduce_partner<1>(v));
    v = fmaxf(v, reduce_partner<2>(v));
    v = fmaxf(v, reduce_partner<4>(v));
    return fmaxf(v, reduce_partner<8>(v));
}

template <bool LOGP>
__device__ __forceinline__ float weight_term(float w) {
    return LOGP ? w : fmaxf(w, 1e-45f);
}
template <bool LOGP>
__device__ __forceinline__ float log_weight(float w) {
    return LOGP ? w : logf(fmaxf(w, 1e-45f));
}

// Four consecutive columns col .. col + 3 of a row; columns past the batch
// read `fill`.  With VEC, col is a multiple of 4 and rows are 16-byte aligned.
// ld4_raw issues the loads (columns past the batch read column 0) and
// ld4_fill puts `fill` in those columns, so a kernel can issue a tile's loads
// together behind a scheduling barrier before the first fill waits on one.
template <bool VEC>
__device__ __forceinline__ void ld4_raw(const float* __restrict__ row, int64_t col, int64_t batch, float (&v)[4]) {
    if constexpr (VEC) {
        const f32x4 t = *reinterpret_cast<const f32x4*>(row + (col < batch ? col : 0));
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = row[col + u < batch ? col + u : 0];
    }
}
// ld4_raw with the nontemporal hint when NT (rows of 16-byte vectors): for
// rows read once, which leave nothing in the caches that a later read finds.
template <bool VEC, bool NT>
__device__ __forceinline__ void ld4_raw_nt(const float* __restrict__ row, int64_t col, int64_t batch, float (&v)[4]) {
    if constexpr (VEC && NT) {
        const f32x4 t = load_stream<f32x4>(row + (col < batch ? col : 0));
        v[0] = t.x;
        v[1] = t.y;
        v[2] = t.z;
        v[3] = t.w;
    } else {
        ld4_raw<VEC>(row, col, batch, v);
    }
}
template <bool VEC>
__device__ __forceinline__ void ld4_fill(int64_t col, int64_t batch, float fill, float (&v)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = (VEC ? col : col + u) < batch ? v[u] : fill;
}
template <bool VEC>
__device__ __forceinline__ void ld4(const float* __restrict__ row, int64_t col, int64_t batch, float fill,
                                    float (&v)[4]) {
    ld4_raw<VEC>(row, col, batch, v);
    ld4_fill<VEC>(col, batch, fill, v);
}

// R = g * exp(lw + m - o) for one (p, b); `left` when the pair must take the
// one-by-one terms, 0 when the pair contributes nothing (o = -inf, padding).
__device__ __forceinline__ float r_factor(float lw, float m, float o, float g, bool valid, bool& left) {
    const float ex = lw + m - o;
    const float r = g * fexp2(ex * kLog2e);
    const bool dead = !valid || o == -kInf;
    const bool ok = ex <= kRMax && __builtin_isfinite(r);
    left = !dead && !ok;
    return dead || !ok ? 0.0f : r;
}

// XCD-contiguous logical id (physical workgroup w runs on XCD w % 8).
__device__ __forceinline__ int64_t logical_id(int64_t id0) {
    const int64_t per_xcd = gridDim.x / 8;
    return id0 + (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
}

}  // namespace

// x at a lane's cells of a 64-column tile (edges c0 + 16*et + 4*kq + r,
// columns col .. col + 3; edges past ne read -inf, columns past the batch 0)
// and the column maxima over the chunk's edges.  tile_x_raw issues the loads,
// tile_x_finish masks them and takes the maxima; tile_x does both with a
// scheduling barrier between, so every load is issued before the first use.
template <int ET, bool VEC>
__device__ __forceinline__ void tile_x_raw(const float* __restrict__ xm, const int64_t* __restrict__ cids,
                                           int64_t ebase, int64_t ne, int64_t c0, int kq, int64_t col,
                                           int64_t batch, float (&xv)[ET][4][4]) {
#pragma unroll
    for (int et = 0; et < ET; ++et)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t e = c0 + 16 * et + 4 * kq + r;
            ld4_raw<VEC>(xm + cids[ebase + (e < ne ? e : ne - 1)] * batch, col, batch, xv[et][r]);
        }
}
template <int ET, bool VEC>
__device__ __forceinline__ void tile_x_finish(int64_t ne, int64_t c0, int kq, int64_t col, int64_t batch,
                                              float (&xv)[ET][4][4], float (&m)[4]) {
#pragma unroll
    for (int et = 0; et < ET; ++et)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool ev = c0 + 16 * et + 4 * kq + r < ne;
            ld4_fill<VEC>(col, batch, 0.0f, xv[et][r]);
#pragma unroll
            for (int u = 0; u < 4; ++u) xv[et][r][u] = ev ? xv[et][r][u] : -kInf;
        }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        float mu = xv[0][0][u];
#pragma unroll
        for (int et = 0; et < ET; ++et)
#pragma unroll
            for (int r = 0; r < 4; ++r) mu = fmaxf(mu, xv[et][r][u]);
        m[u] = max_pair32(max_pair16(mu));
    }
}
template <int ET, bool VEC>
__device__ __forceinline__ void tile_x(const float* __restrict__ xm, const int64_t* __restrict__ cids, int64_t ebase,
                                       int64_t ne, int64_t c0, int kq, int64_t col, int64_t batch,
                                       float (&xv)[ET][4][4], float (&m)[4]) {
    tile_x_raw<ET, VEC>(xm, cids, ebase, ne, c0, kq, col, batch, xv);
    __builtin_amdgcn_sched_barrier(0);
    tile_x_finish<ET, VEC>(ne, c0, kq, col, batch, xv, m);
}

// Edge flows F[j, e, b] for edges c0 .. c0 + 16*ET - 1 and columns b0 .. b0 + 63.
// Product Z[e, b] = sum_p A[p, e] R[p, b]: lane l supplies A[e = c0 + 16*et + l%16]
// [p = pc0 + 4*ks + l/16] and R[p][b = b0 + 4*(l%16) + u] (N-tile u) and holds
// Z[e = c0 + 16*et + 4*(l/16) + r][b0 + 4*(l%16) + u], the same cells as its
// 16-byte vectors of x, so F = X .* Z needs no exchange.  KP: K-steps per
// parent chunk.
template <int ET, int KP, bool VEC, bool LOGP>
__global__ __launch_bounds__(64) void blocked_bwd_edges(float* __restrict__ edge_flows, const float* __restrict__ gf,
                                                        const float* __restrict__ om, const float* __restrict__ xm,
                                                        const float* __restrict__ params,
                                                        const int64_t* __restrict__ nids,
                                                        const int64_t* __restrict__ cids,
                                                        const int64_t* __restrict__ pids, int64_t ne, int64_t bs,
                                                        int64_t batch, int64_t ctiles, int64_t chunks, int64_t items,
                                                        int64_t id0) {
    __shared__ float ex[16 * ET][64];  // one-by-one terms: [edge - c0][column - b0]
    const int64_t id = logical_id(id0);
    if (id >= items) return;
    const int64_t ct = id % ctiles;
    const int64_t jc_ = id / ctiles;
    const int64_t c = jc_ % chunks;
    const int64_t j = jc_ / chunks;
    const int l = lane_id();
    const int kq = l >> 4;
    const int jc = l & 15;
    const int64_t b0 = ct * 64;
    const int64_t col = b0 + 4 * jc;
    const int64_t c0 = c * CE;
    const int64_t ebase = j * ne;
    const int64_t nrow0 = nids[j];

    // x at the lane's output cells; edges past ne read -inf, columns past the batch 0
    float xv[ET][4][4];
    float m[4];
    tile_x<ET, VEC>(xm, cids, ebase, ne, c0, kq, col, batch, xv, m);
#pragma unroll
    for (int et = 0; et < ET; ++et)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                xv[et][r][u] = __builtin_isfinite(m[u]) ? fexp2((xv[et][r][u] - m[u]) * kLog2e) : 0.0f;

    // the A operand's edges c0 + 16*et + jc
    int64_t qa[ET];
    bool eva[ET];
#pragma unroll
    for (int et = 0; et < ET; ++et) {
        const int64_t e = c0 + 16 * et + jc;
        eva[et] = e < ne;
        qa[et] = pids[ebase + (eva[et] ? e : ne - 1)];
    }

    f32x4 z[ET][4];
#pragma unroll
    for (int et = 0; et < ET; ++et)
#pragma unroll
        for (int u = 0; u < 4; ++u) z[et][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool any_left = false;

    for (int64_t pc0 = 0; pc0 < bs; pc0 += 4 * KP) {
        float a[KP][ET], rr[KP][4];
        uint32_t left = 0;  // bit 4*ks + u
        float wraw[KP][ET], ovk[KP][4], gvk[KP][4];
#pragma unroll
        for (int ks = 0; ks < KP; ++ks) {
            const int64_t p = pc0 + 4 * ks + kq;
            const int64_t pcl = p < bs ? p : bs - 1;
#pragma unroll
            for (int et = 0; et < ET; ++et) wraw[ks][et] = params[qa[et] + pcl];
            ld4_raw<VEC>(om + (nrow0 + pcl) * batch, col, batch, ovk[ks]);
            ld4_raw<VEC>(gf + (nrow0 + pcl) * batch, col, batch, gvk[ks]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KP; ++ks) {
            const int64_t p = pc0 + 4 * ks + kq;
            const bool pv = p < bs;
            float wv[ET];
#pragma unroll
            for (int et = 0; et < ET; ++et) {
                const float w = weight_term<LOGP>(wraw[ks][et]);
                wv[et] = eva[et] && pv ? w : (LOGP ? -kInf : 0.0f);
            }
            float wm = wv[0];
#pragma unroll
            for (int et = 1; et < ET; ++et) wm = fmaxf(wm, wv[et]);
            wm = row16_max(wm);  // over the chunk's edges
#pragma unroll
            for (int et = 0; et < ET; ++et)
                a[ks][et] = !pv ? 0.0f
                            : LOGP ? (wm == -kInf ? 0.0f : fexp2((wv[et] - wm) * kLog2e))
                                   : wv[et] / wm;
            const float lwm = LOGP ? wm : logf(wm);
            ld4_fill<VEC>(col, batch, -kInf, ovk[ks]);
            ld4_fill<VEC>(col, batch, 0.0f, gvk[ks]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                bool lf;
                rr[ks][u] = r_factor(lwm, m[u], ovk[ks][u], gvk[ks][u], pv, lf);
                left |= (uint32_t)lf << (4 * ks + u);
            }
        }
#pragma unroll
        for (int ks = 0; ks < KP; ++ks)
#pragma unroll
            for (int et = 0; et < ET; ++et)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    z[et][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ks][et], rr[ks][u], z[et][u], 0, 0, 0);

        if (__ballot(left != 0)) {
            if (!any_left) {
#pragma unroll
                for (int et = 0; et < ET; ++et)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int u = 0; u < 4; ++u) ex[16 * et + 4 * kq + r][4 * jc + u] = 0.0f;
                any_left = true;
                // one wave: its LDS operations complete in order
                __builtin_amdgcn_wave_barrier();
            }
            // One parent row of each quad at a time, so the lanes writing
            // ex hold different columns; a lane takes its pairs in order.
            for (int kk = 0; kk < 4; ++kk) {
                if (kq == kk) {
                    uint32_t lf = left;
                    while (lf) {
                        const int bit = __builtin_ctz(lf);
                        lf &= lf - 1;
                        const int64_t p = pc0 + 4 * (bit >> 2) + kk;
                        const int cu = 4 * jc + (bit & 3);
                        const int64_t n = nrow0 + p;
                        const float gg = gf[n * batch + b0 + cu];
                        const float oo = om[n * batch + b0 + cu];
                        for (int ee = 0; ee < 16 * ET && c0 + ee < ne; ++ee) {
                            const int64_t e = c0 + ee;
                            const float lw = log_weight<LOGP>(params[pids[ebase + e] + p]);
                            const float xx = xm[cids[ebase + e] * batch + b0 + cu];
                            ex[ee][cu] += gg * fexp2((lw + xx - oo) * kLog2e);
                        }
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }

    // F = X .* Z (+ one-by-one terms) at rows c0 + 16*et + 4*kq + r
#pragma unroll
    for (int et = 0; et < ET; ++et)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t e = c0 + 16 * et + 4 * kq + r;
            if (e >= ne) continue;
            float res[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float zz = z[et][u][r];
                res[u] = zz == 0.0f ? 0.0f : xv[et][r][u] * zz;
                if (any_left) res[u] += ex[16 * et + 4 * kq + r][4 * jc + u];
            }
            float* orow = edge_flows + (ebase + e) * batch;
            if constexpr (VEC) {
                if (col < batch) store_stream(f32x4{res[0], res[1], res[2], res[3]}, orow + col);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (col + u < batch) orow[col + u] = res[u];
            }
        }
}

// Parameter flows for parents p0 .. p0 + 16*MT - 1 and edges c0 .. c0 + 16*ET - 1.
// Product G[p, e] = sum_b R[p, b] X[e, b] over the whole batch, 4*CW columns
// per pass: lane l supplies R[p = p0 + 16*pt + l%16][b = b0 + CW*(l/16) + ks]
// and X[e = c0 + 16*et + l%16][same b] (its CW columns are CW/4 vectors of
// one row) and holds G[p0 + 16*pt + 4*(l/16) + r][c0 + 16*et + l%16].
template <int MT, int ET, int CW, bool VEC, bool LOGP>
__global__ __launch_bounds__(64) void blocked_bwd_params(float* __restrict__ param_flows, const float* __restrict__ gf,
                                                         const float* __restrict__ om, const float* __restrict__ xm,
                                                         const float* __restrict__ params,
                                                         const int64_t* __restrict__ nids,
                                                         const int64_t* __restrict__ cids,
                                                         const int64_t* __restrict__ pids, int64_t ne, int64_t bs,
                                                         int64_t batch, int64_t pgroups, int64_t chunks, int64_t items,
                                                         int64_t id0) {
    __shared__ float ex[16 * MT][16 * ET];  // one-by-one terms: [parent - p0][edge - c0]
    const int64_t id = logical_id(id0);
    if (id >= items) return;
    const int64_t g = id % pgroups;
    const int64_t jc_ = id / pgroups;
    const int64_t c = jc_ % chunks;
    const int64_t j = jc_ / chunks;
    const int l = lane_id();
    const int kq = l >> 4;
    const int jc = l & 15;
    const int64_t p0 = g * 16 * MT;
    const int64_t c0 = c * CE;
    const int64_t ebase = j * ne;
    const int64_t nrow0 = nids[j];

    // row maxima of the weights over the chunk's edges, for rows p0 + 16*pt + jc
    float wmx[MT], lwm[MT];
#pragma unroll
    for (int pt = 0; pt < MT; ++pt) {
        const int64_t p = p0 + 16 * pt + jc;
        const bool pv = p < bs;
        const int64_t pcl = pv ? p : bs - 1;
        float wm = LOGP ? -kInf : 0.0f;
#pragma unroll
        for (int i = 0; i < 4 * ET; ++i) {
            const int64_t e = c0 + kq + 4 * i;
            const bool ev = e < ne;
            const float w = weight_term<LOGP>(params[pids[ebase + (ev ? e : ne - 1)] + pcl]);
            wm = ev ? fmaxf(wm, w) : wm;
        }
        wmx[pt] = max_pair32(max_pair16(wm));
        lwm[pt] = LOGP ? wmx[pt] : logf(wmx[pt]);
    }
    const float* xrow[ET];
    bool evb[ET];
#pragma unroll
    for (int et = 0; et < ET; ++et) {
        const int64_t e = c0 + 16 * et + jc;
        evb[et] = e < ne;
        xrow[et] = xm + cids[ebase + (evb[et] ? e : ne - 1)] * batch;
    }
    const float* orow[MT];
    const float* grow[MT];
    bool pvr[MT];
#pragma unroll
    for (int pt = 0; pt < MT; ++pt) {
        const int64_t p = p0 + 16 * pt + jc;
        pvr[pt] = p < bs;
        const int64_t n = nrow0 + (pvr[pt] ? p : bs - 1);
        orow[pt] = om + n * batch;
        grow[pt] = gf + n * batch;
    }

    f32x4 acc[MT][ET];
#pragma unroll
    for (int pt = 0; pt < MT; ++pt)
#pragma unroll
        for (int et = 0; et < ET; ++et) acc[pt][et] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool any_left = false;

    for (int64_t b0 = 0; b0 < batch; b0 += 4 * CW) {
        const int64_t cb = b0 + CW * kq;  // K-step ks takes column cb + ks
        float xv[ET][CW], ovp[MT][CW], gvp[MT][CW];
#pragma unroll
        for (int q = 0; q < CW / 4; ++q) {
#pragma unroll
            for (int et = 0; et < ET; ++et)
                ld4_raw<VEC>(xrow[et], cb + 4 * q, batch, *reinterpret_cast<float(*)[4]>(&xv[et][4 * q]));
#pragma unroll
            for (int pt = 0; pt < MT; ++pt) {
                ld4_raw<VEC>(orow[pt], cb + 4 * q, batch, *reinterpret_cast<float(*)[4]>(&ovp[pt][4 * q]));
                ld4_raw<VEC>(grow[pt], cb + 4 * q, batch, *reinterpret_cast<float(*)[4]>(&gvp[pt][4 * q]));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < CW / 4; ++q)
#pragma unroll
            for (int et = 0; et < ET; ++et) {
                float(&v)[4] = *reinterpret_cast<float(*)[4]>(&xv[et][4 * q]);
                ld4_fill<VEC>(cb + 4 * q, batch, 0.0f, v);
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = evb[et] ? v[u] : -kInf;
            }
        float m[CW];
#pragma unroll
        for (int i = 0; i < CW; ++i) {
            float mi = xv[0][i];
#pragma unroll
            for (int et = 1; et < ET; ++et) mi = fmaxf(mi, xv[et][i]);
            m[i] = row16_max(mi);  // over the chunk's edges
        }
#pragma unroll
        for (int et = 0; et < ET; ++et)
#pragma unroll
            for (int i = 0; i < CW; ++i)
                xv[et][i] = __builtin_isfinite(m[i]) ? fexp2((xv[et][i] - m[i]) * kLog2e) : 0.0f;
        float rr[MT][CW];
        uint32_t left[MT];  // bit i: column cb + i
#pragma unroll
        for (int pt = 0; pt < MT; ++pt) {
            left[pt] = 0;
#pragma unroll
            for (int q = 0; q < CW / 4; ++q) {
                float(&ov)[4] = *reinterpret_cast<float(*)[4]>(&ovp[pt][4 * q]);
                float(&gv)[4] = *reinterpret_cast<float(*)[4]>(&gvp[pt][4 * q]);
                ld4_fill<VEC>(cb + 4 * q, batch, -kInf, ov);
                ld4_fill<VEC>(cb + 4 * q, batch, 0.0f, gv);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    bool lf;
                    rr[pt][4 * q + u] = r_factor(lwm[pt], m[4 * q + u], ov[u], gv[u], pvr[pt], lf);
                    left[pt] |= (uint32_t)lf << (4 * q + u);
                }
            }
        }
#pragma unroll
        for (int ks = 0; ks < CW; ++ks)
#pragma unroll
            for (int pt = 0; pt < MT; ++pt)
#pragma unroll
                for (int et = 0; et < ET; ++et)
                    acc[pt][et] = __builtin_amdgcn_mfma_f32_16x16x4f32(rr[pt][ks], xv[et][ks], acc[pt][et], 0, 0, 0);

        bool anyl = false;
#pragma unroll
        for (int pt = 0; pt < MT; ++pt) anyl = anyl || left[pt] != 0;
        if (__ballot(anyl)) {
            if (!any_left) {
#pragma unroll
                for (int pt = 0; pt < MT; ++pt)
#pragma unroll
                    for (int et = 0; et < ET; ++et)
#pragma unroll
                        for (int r = 0; r < 4; ++r) ex[16 * pt + 4 * kq + r][16 * et + jc] = 0.0f;
                any_left = true;
                __builtin_amdgcn_wave_barrier();
            }
            // One column quarter at a time, so the lanes writing ex hold
            // different parent rows; a lane takes its pairs in order.
            for (int kk = 0; kk < 4; ++kk) {
                if (kq == kk) {
#pragma unroll
                    for (int pt = 0; pt < MT; ++pt) {
                        uint32_t lf = left[pt];
                        while (lf) {
                            const int i = __builtin_ctz(lf);
                            lf &= lf - 1;
                            const int64_t p = p0 + 16 * pt + jc;
                            const int64_t b = cb + i;
                            const int64_t n = nrow0 + p;
                            const float gg = gf[n * batch + b];
                            const float oo = om[n * batch + b];
                            for (int ee = 0; ee < 16 * ET && c0 + ee < ne; ++ee) {
                                const int64_t e = c0 + ee;
                                const float lw = log_weight<LOGP>(params[pids[ebase + e] + p]);
                                const float xx = xm[cids[ebase + e] * batch + b];
                                ex[16 * pt + jc][ee] += gg * fexp2((lw + xx - oo) * kLog2e);
                            }
                        }
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }

    // param_flows[pids[j, e] + p] += (w / W) G + one-by-one terms, rows p0 + 16*pt + 4*kq + r
#pragma unroll
    for (int pt = 0; pt < MT; ++pt) {
        float wr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) wr[r] = lane_read(wmx[pt], 4 * kq + r);
#pragma unroll
        for (int et = 0; et < ET; ++et) {
            const int64_t e = c0 + 16 * et + jc;
            if (e >= ne) continue;
            const int64_t q = pids[ebase + e];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t p = p0 + 16 * pt + 4 * kq + r;
                if (p >= bs) continue;
                const float w = weight_term<LOGP>(params[q + p]);
                const float aw = LOGP ? (wr[r] == -kInf ? 0.0f : fexp2((w - wr[r]) * kLog2e)) : w / wr[r];
                const float gsum = acc[pt][et][r];
                float v = gsum == 0.0f ? 0.0f : aw * gsum;
                if (any_left) v += ex[16 * pt + 4 * kq + r][16 * et + jc];
                if (v != 0.0f)
                    __hip_atomic_fetch_add(param_flows + q + p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// Both products in one pass, for blocks of at most 32 parents: one wave per
// (block, edge chunk) walks the batch in 64-column tiles.  Per tile it loads
// x (the edge-flow cells), g and o once, runs the product over parents as
// blocked_bwd_edges does, then writes the tile's X and R to LDS and reads
// them back transposed for the product over the batch (rows padded to 68
// floats, so every LDS access is one aligned 16-byte vector per lane).  The
// weights are
// taken once per wave.  Pairs left out of the products are only counted in
// the tile loop; when there are any, a second pass over the tiles finds them
// again with the same arithmetic and adds their one-by-one terms (the code
// for them inside the loop cost 55 registers and half the occupancy).
// NKP: parent K-steps (4 parents each), MP = NKP / 4 rounded up: 16-parent
// tiles of the product over the batch.  NTP: the block's parent rows (o, g)
// take nontemporal loads, for layers of one edge chunk, where no other wave
// reads them again (one chunk at the bench layer: 473 -> 445 us; with two
// chunks the hint cost 4%, the other chunk's wave missing what the caches
// would have kept).  Compiled for at least two waves per SIMD: the
// accumulators then live in VGPRs (241 registers at 32 parents, where the
// default allocation took 197 + 48 AGPRs; 448 -> 443 us), 16 parents run
// three waves per SIMD instead of two, and rows that are not 16-byte vectors
// two instead of one.
template <int ET, int NKP, bool VEC, bool LOGP, bool NTP>
__global__ __launch_bounds__(64, 2) void blocked_bwd_fused(float* __restrict__ edge_flows,
                                                        float* __restrict__ param_flows,
                                                        const float* __restrict__ gf, const float* __restrict__ om,
                                                        const float* __restrict__ xm, const float* __restrict__ params,
                                                        const int64_t* __restrict__ nids,
                                                        const int64_t* __restrict__ cids,
                                                        const int64_t* __restrict__ pids, int64_t ne, int64_t bs,
                                                        int64_t batch, int64_t chunks, int64_t items, int64_t id0,
                                                        int disjoint) {
    constexpr int MP = (NKP + 3) / 4;
    constexpr int LD = kTileLD;  // tile row; columns placed by tile_col
    constexpr int KC = NKP < 4 ? NKP : 4;
    __shared__ __align__(16) float xt[16 * ET][LD];  // X of the tile: [edge - c0][column - b0]; one-by-one edge terms
    __shared__ __align__(16) float rt[16 * MP][LD];  // R of the tile: [parent][column - b0]
    // one-by-one parameter terms, [parent][edge - c0]: used only by the second
    // pass and the final adds, after the last read of rt, so they share its
    // storage (keeps a workgroup at 18 KB of LDS: eight per CU, as many as
    // the registers allow)
    static_assert(16 * MP * 16 * ET <= 16 * MP * LD, "parameter terms fit in the R tile");
    float(*gx)[16 * ET] = reinterpret_cast<float(*)[16 * ET]>(&rt[0][0]);
    const int64_t id = logical_id(id0);
    if (id >= items) return;
    const int64_t c = id % chunks;
    const int64_t j = id / chunks;
    const int l = lane_id();
    const int kq = l >> 4;
    const int jc = l & 15;
    const int64_t c0 = c * CE;
    const int64_t ebase = j * ne;
    const int64_t nrow0 = nids[j];
    // this lane's column word in the row-wise tile accesses (rows 16 et +
    // 4 kq + r: their swizzle depends on kq only) and its swizzle in the
    // transposed reads (rows 16 pt + jc)
    const int colw = tile_col(4 * kq, 4 * jc);
    const int swt = tile_swz(jc);

    // weights of the edge-flow product, A[p = 4*ks + kq][e = c0 + 16*et + jc], and
    // the row maxima (log) over the chunk's edges
    float a[NKP][ET], lwm[NKP];
    {
        int64_t qa[ET];
        bool eva[ET];
#pragma unroll
        for (int et = 0; et < ET; ++et) {
            const int64_t e = c0 + 16 * et + jc;
            eva[et] = e < ne;
            qa[et] = pids[ebase + (eva[et] ? e : ne - 1)];
        }
#pragma unroll
        for (int ks = 0; ks < NKP; ++ks) {
            const int64_t p = 4 * ks + kq;
            const bool pv = p < bs;
            const int64_t pcl = pv ? p : bs - 1;
            float wv[ET];
#pragma unroll
            for (int et = 0; et < ET; ++et) {
                const float w = weight_term<LOGP>(params[qa[et] + pcl]);
                wv[et] = eva[et] && pv ? w : (LOGP ? -kInf : 0.0f);
            }
            float wm = wv[0];
#pragma unroll
            for (int et = 1; et < ET; ++et) wm = fmaxf(wm, wv[et]);
            wm = row16_max(wm);
#pragma unroll
            for (int et = 0; et < ET; ++et)
                a[ks][et] = !pv ? 0.0f
                            : LOGP ? (wm == -kInf ? 0.0f : fexp2((wv[et] - wm) * kLog2e))
                                   : wv[et] / wm;
            lwm[ks] = LOGP ? wm : logf(wm);
        }
    }

    f32x4 gacc[MP][ET];
#pragma unroll
    for (int pt = 0; pt < MP; ++pt)
#pragma unroll
        for (int et = 0; et < ET; ++et) gacc[pt][et] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool any_left = false;

    for (int64_t b0 = 0; b0 < batch; b0 += 64) {
        const int64_t col = b0 + 4 * jc;
        // x, o and g of the whole tile are issued as one group: the tile
        // waits for memory once, not once per load phase
        float m[4];
        float ov[NKP][4], gv[NKP][4];
        {
            float xv[ET][4][4];
            tile_x_raw<ET, VEC>(xm, cids, ebase, ne, c0, kq, col, batch, xv);
#pragma unroll
            for (int ks = 0; ks < NKP; ++ks) {
                const int64_t p = 4 * ks + kq;
                const int64_t n = nrow0 + (p < bs ? p : bs - 1);
                ld4_raw_nt<VEC, NTP>(om + n * batch, col, batch, ov[ks]);
                ld4_raw_nt<VEC, NTP>(gf + n * batch, col, batch, gv[ks]);
            }
            __builtin_amdgcn_sched_barrier(0);
            tile_x_finish<ET, VEC>(ne, c0, kq, col, batch, xv, m);
#pragma unroll
            for (int et = 0; et < ET; ++et)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    f32x4 xe;
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        xe[u] = __builtin_isfinite(m[u]) ? fexp2((xv[et][r][u] - m[u]) * kLog2e) : 0.0f;
                    const int row = 16 * et + 4 * kq + r;
                    *reinterpret_cast<f32x4*>(&xt[row][colw]) = xe;
                }
        }  // the tile's X lives in xt from here

        f32x4 z[ET][4];
#pragma unroll
        for (int et = 0; et < ET; ++et)
#pragma unroll
            for (int u = 0; u < 4; ++u) z[et][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        bool left = false;
#pragma unroll
        for (int k0 = 0; k0 < NKP; k0 += KC) {
            float rr[KC][4];
#pragma unroll
            for (int kk = 0; kk < KC; ++kk) {
                const int ks = k0 + kk;
                const bool pv = 4 * ks + kq < bs;
                ld4_fill<VEC>(col, batch, -kInf, ov[ks]);
                ld4_fill<VEC>(col, batch, 0.0f, gv[ks]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    bool lf;
                    rr[kk][u] = r_factor(lwm[ks], m[u], ov[ks][u], gv[ks][u], pv, lf);
                    left = left || lf;
                }
                *reinterpret_cast<f32x4*>(&rt[4 * ks + kq][4 * (jc ^ tile_swz(4 * ks))]) =
                    f32x4{rr[kk][0], rr[kk][1], rr[kk][2], rr[kk][3]};
            }
#pragma unroll
            for (int kk = 0; kk < KC; ++kk)
#pragma unroll
                for (int et = 0; et < ET; ++et)
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        z[et][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[k0 + kk][et], rr[kk][u], z[et][u], 0, 0, 0);
        }
        any_left = any_left || __ballot(left) != 0;
        // rows of R past 4*NKP (up to the 16-row tiles) hold zeros
        if constexpr (4 * NKP < 16 * MP) {
#pragma unroll
            for (int i = 0; i < 4 * MP - NKP; ++i)
                *reinterpret_cast<f32x4*>(&rt[4 * (NKP + i) + kq][4 * (jc ^ tile_swz(4 * (NKP + i)))]) =
                    f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        __builtin_amdgcn_wave_barrier();
        // product over the batch: lane l supplies R[16*pt + l%16][16*(l/16) + ks]
        // and X[16*et + l%16][same column], K-steps ks in order, read four at a
        // time as one 16-byte vector per row
#pragma unroll 1
        for (int i = 0; i < 4; ++i) {
            f32x4 ra[MP], xb[ET];
#pragma unroll
            for (int pt = 0; pt < MP; ++pt)
                ra[pt] = *reinterpret_cast<const f32x4*>(&rt[16 * pt + jc][4 * ((4 * kq + i) ^ swt)]);
#pragma unroll
            for (int et = 0; et < ET; ++et)
                xb[et] = *reinterpret_cast<const f32x4*>(&xt[16 * et + jc][4 * ((4 * kq + i) ^ swt)]);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int pt = 0; pt < MP; ++pt)
#pragma unroll
                    for (int et = 0; et < ET; ++et)
                        gacc[pt][et] = __builtin_amdgcn_mfma_f32_16x16x4f32(ra[pt][t], xb[et][t], gacc[pt][et], 0, 0, 0);
        }
        // edge flows F = X .* Z at rows c0 + 16*et + 4*kq + r
#pragma unroll
        for (int et = 0; et < ET; ++et)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t e = c0 + 16 * et + 4 * kq + r;
                const int row = 16 * et + 4 * kq + r;
                const f32x4 xe = *reinterpret_cast<const f32x4*>(&xt[row][colw]);
                float res[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float zz = z[et][u][r];
                    res[u] = zz == 0.0f ? 0.0f : xe[u] * zz;
                }
                if (e >= ne) continue;
                float* orow = edge_flows + (ebase + e) * batch;
                if constexpr (VEC) {
                    if (col < batch) store_stream(f32x4{res[0], res[1], res[2], res[3]}, orow + col);
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (col + u < batch) orow[col + u] = res[u];
                }
            }
        __builtin_amdgcn_wave_barrier();
    }

    if (any_left) {
        // Second pass: the same column maxima and R tests find the pairs left
        // out; their terms go, one lane at a time and each lane's pairs in
        // order, into xt (edge terms of the tile, then added by each cell's
        // owner to its stored edge flow) and gx (parameter terms).
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");  // this wave's tile stores are visible
#pragma unroll
        for (int pt = 0; pt < MP; ++pt)
#pragma unroll
            for (int et = 0; et < ET; ++et)
#pragma unroll
                for (int r = 0; r < 4; ++r) gx[16 * pt + 4 * kq + r][16 * et + jc] = 0.0f;
        for (int64_t b0 = 0; b0 < batch; b0 += 64) {
            const int64_t col = b0 + 4 * jc;
            float m[4];
            {
                float xv[ET][4][4];
                tile_x<ET, VEC>(xm, cids, ebase, ne, c0, kq, col, batch, xv, m);
            }
            uint64_t left = 0;  // bit 4*ks + u
            // one K-step at a time (this pass is rare; its registers count
            // against the whole kernel), the row maximum taken again as the
            // first pass took it
#pragma unroll 1
            for (int ks = 0; ks < NKP; ++ks) {
                const int64_t p = 4 * ks + kq;
                const bool pv = p < bs;
                const int64_t pcl = pv ? p : bs - 1;
                float wm = LOGP ? -kInf : 0.0f;
#pragma unroll
                for (int et = 0; et < ET; ++et) {
                    const int64_t e = c0 + 16 * et + jc;
                    const bool ev = e < ne;
                    const float w = weight_term<LOGP>(params[pids[ebase + (ev ? e : ne - 1)] + pcl]);
                    wm = ev && pv ? fmaxf(wm, w) : wm;
                }
                wm = row16_max(wm);
                const float lw = LOGP ? wm : logf(wm);
                const int64_t n = nrow0 + pcl;
                float ov[4], gv[4];
                ld4<VEC>(om + n * batch, col, batch, -kInf, ov);
                ld4<VEC>(gf + n * batch, col, batch, 0.0f, gv);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    bool lf;
                    (void)r_factor(lw, m[u], ov[u], gv[u], pv, lf);
                    left |= (uint64_t)lf << (4 * ks + u);
                }
            }
            if (__ballot(left != 0) == 0) continue;
#pragma unroll
            for (int et = 0; et < ET; ++et)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    *reinterpret_cast<f32x4*>(&xt[16 * et + 4 * kq + r][colw]) =
                        f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            __builtin_amdgcn_wave_barrier();
            for (int ll = 0; ll < 64; ++ll) {
                if (l == ll) {
                    uint64_t lf = left;
                    while (lf) {
                        const int bit = __builtin_ctzll(lf);
                        lf &= lf - 1;
                        const int64_t p = 4 * (bit >> 2) + kq;
                        const int cu = 4 * jc + (bit & 3);
                        const int64_t n = nrow0 + p;
                        const float gg = gf[n * batch + b0 + cu];
                        const float oo = om[n * batch + b0 + cu];
                        for (int ee = 0; ee < 16 * ET && c0 + ee < ne; ++ee) {
                            const int64_t e = c0 + ee;
                            const float lw = log_weight<LOGP>(params[pids[ebase + e] + p]);
                            const float xx = xm[cids[ebase + e] * batch + b0 + cu];
                            const float t = gg * fexp2((lw + xx - oo) * kLog2e);
                            xt[ee][tile_col(ee, cu)] += t;
                            gx[p][ee] += t;
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
#pragma unroll
            for (int et = 0; et < ET; ++et)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t e = c0 + 16 * et + 4 * kq + r;
                    if (e >= ne) continue;
                    float* orow = edge_flows + (ebase + e) * batch;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const float t = xt[16 * et + 4 * kq + r][colw + u];
                        if (t != 0.0f && col + u < batch) orow[col + u] += t;
                    }
                }
            __builtin_amdgcn_wave_barrier();
        }
        __builtin_amdgcn_wave_barrier();
    }

    // param_flows[pids[j, e] + p] += (w / W) G + one-by-one terms, at
    // G[16*pt + 4*kq + r][c0 + 16*et + jc]; W, the row maximum over the chunk's
    // edges, is taken again from the same weights (lanes of a row hold all edges)
    int64_t q[ET];
#pragma unroll
    for (int et = 0; et < ET; ++et) {
        const int64_t e = c0 + 16 * et + jc;
        q[et] = pids[ebase + (e < ne ? e : ne - 1)];
    }
    float pfv[MP][4][ET];
#pragma unroll
    for (int pt = 0; pt < MP; ++pt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t p = 16 * pt + 4 * kq + r;
            const bool pv = p < bs;
            const int64_t pcl = pv ? p : bs - 1;
            float wv[ET];
#pragma unroll
            for (int et = 0; et < ET; ++et) {
                const int64_t e = c0 + 16 * et + jc;
                const bool ev = e < ne;
                const float w = weight_term<LOGP>(params[q[et] + pcl]);
                wv[et] = ev && pv ? w : (LOGP ? -kInf : 0.0f);
            }
            float wm = wv[0];
#pragma unroll
            for (int et = 1; et < ET; ++et) wm = fmaxf(wm, wv[et]);
            wm = row16_max(wm);
#pragma unroll
            for (int et = 0; et < ET; ++et) {
                const int64_t e = c0 + 16 * et + jc;
                float v = 0.0f;
                if (pv && e < ne) {
                    const float aw = LOGP ? (wm == -kInf ? 0.0f : fexp2((wv[et] - wm) * kLog2e)) : wv[et] / wm;
                    const float gsum = gacc[pt][et][r];
                    v = gsum == 0.0f ? 0.0f : aw * gsum;
                    if (any_left) v += gx[p][16 * et + jc];
                }
                pfv[pt][r][et] = v;
            }
        }
    if (disjoint) {
        // No parameter is shared by two (block, parent, edge) triples of the
        // layer, so this lane's cells are its own: a plain load, add and store,
        // every load issued before the first store.  The wave covers each block
        // edge's parents in one run, written back as whole lines.
        float old[MP][4][ET];
#pragma unroll
        for (int pt = 0; pt < MP; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int et = 0; et < ET; ++et)
                    old[pt][r][et] = pfv[pt][r][et] != 0.0f ? param_flows[q[et] + 16 * pt + 4 * kq + r] : 0.0f;
#pragma unroll
        for (int pt = 0; pt < MP; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int et = 0; et < ET; ++et)
                    if (pfv[pt][r][et] != 0.0f)
                        param_flows[q[et] + 16 * pt + 4 * kq + r] = old[pt][r][et] + pfv[pt][r][et];
    } else {
#pragma unroll
        for (int pt = 0; pt < MP; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int et = 0; et < ET; ++et)
                    if (pfv[pt][r][et] != 0.0f)
                        __hip_atomic_fetch_add(param_flows + q[et] + 16 * pt + 4 * kq + r, pfv[pt][r][et],
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// element_flows[c, b] += sum of edge_flows rows csc_edges[csc_offsets[c] ..
// csc_offsets[c + 1]) in that order: one wave per element row, 512 columns
// per pass (two 16-byte vectors per lane, both issued before either is
// used); the edge rows and the element row are read once, with the
// nontemporal hint (221 -> 210 us at the bench layer), and the sums stored
// with it.
template <bool VEC>
__global__ __launch_bounds__(256) void blocked_bwd_elements(float* __restrict__ element_flows,
                                                            const float* __restrict__ edge_flows,
                                                            const int64_t* __restrict__ csc_offsets,
                                                            const int32_t* __restrict__ csc_edges, int64_t nel,
                                                            int64_t batch, int64_t block0) {
    const int64_t c = (block0 + (int64_t)blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (c >= nel) return;
    const int64_t k0 = csc_offsets[c];
    const int64_t k1 = csc_offsets[c + 1];
    if (k0 >= k1) return;
    const int l = lane_id();
    float* er = element_flows + c * batch;
    for (int64_t b0 = 0; b0 < batch; b0 += 512) {
        const int64_t col[2] = {b0 + 4 * l, b0 + 256 + 4 * l};
        float s[2][4] = {};
        for (int64_t k = k0; k < k1; ++k) {
            const float* row = edge_flows + (int64_t)csc_edges[k] * batch;
            float v[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) ld4_raw_nt<VEC, true>(row, col[h], batch, v[h]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                ld4_fill<VEC>(col[h], batch, 0.0f, v[h]);
#pragma unroll
                for (int u = 0; u < 4; ++u) s[h][u] += v[h][u];
            }
        }
        float cur[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) ld4_raw_nt<VEC, true>(er, col[h], batch, cur[h]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            ld4_fill<VEC>(col[h], batch, 0.0f, cur[h]);
            if constexpr (VEC) {
                if (col[h] < batch)
                    store_stream(f32x4{cur[h][0] + s[h][0], cur[h][1] + s[h][1], cur[h][2] + s[h][2],
                                       cur[h][3] + s[h][3]},
                                 er + col[h]);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (col[h] + u < batch) er[col[h] + u] = cur[h][u] + s[h][u];
            }
        }
    }
}

namespace {

constexpr int64_t kMaxGroups = max_grid_blocks(64);  // workgroups per launch, a multiple of 8
// Columns per lane per pass of the parameter-flow product, and parent K-steps
// per chunk of the edge-flow product (at most).  Measured at 8192 blocks of
// 32 parents, 32 edges, batch 512: 16 columns and 8 K-steps 1280 us; 8 and 4
// 1084 us (4 waves per SIMD instead of 2 in both kernels); 4 columns 1191 us;
// 2 K-steps as 4.
constexpr int kParamCW = 8;
constexpr int kEdgeKPMax = 4;
// Largest block_size of the single-pass kernel.  It reads x, g and o once
// instead of twice (262144 nodes, 32 edges, batch 512: 8 parents 2213 ->
// 1667 us, 16: 1464 -> 1041 us, 24: 1284 -> 971 us, 32: 1088 -> 833 us
// against the two kernels).  Its loads are issued ahead of their first use
// behind scheduling barriers: without them the compiler waited on every load
// of a tile in turn (16 parents: 1312 us).
constexpr int64_t kFusedMaxBs = 32;

template <int ET, int KP, bool VEC, bool LOGP>
void launch_edges(float* edge_flows, const float* gf, const float* om, const float* xm, const float* params,
                  const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb, int64_t ne, int64_t bs,
                  int64_t batch, hipStream_t st) {
    const int64_t ctiles = (batch + 63) / 64;
    const int64_t chunks = (ne + CE - 1) / CE;
    const int64_t items = nb * chunks * ctiles;
    for (int64_t id0 = 0; id0 < items; id0 += kMaxGroups) {
        const int64_t n = items - id0 < kMaxGroups ? items - id0 : kMaxGroups;
        blocked_bwd_edges<ET, KP, VEC, LOGP><<<dim3((unsigned)((n + 7) / 8 * 8)), dim3(64), 0, st>>>(
            edge_flows, gf, om, xm, params, nids, cids, pids, ne, bs, batch, ctiles, chunks, items, id0);
    }
}

template <int MT, int ET, bool VEC, bool LOGP>
void launch_params(float* param_flows, const float* gf, const float* om, const float* xm, const float* params,
                   const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb, int64_t ne, int64_t bs,
                   int64_t batch, hipStream_t st) {
    const int64_t pgroups = (bs + 16 * MT - 1) / (16 * MT);
    const int64_t chunks = (ne + CE - 1) / CE;
    const int64_t items = nb * chunks * pgroups;
    for (int64_t id0 = 0; id0 < items; id0 += kMaxGroups) {
        const int64_t n = items - id0 < kMaxGroups ? items - id0 : kMaxGroups;
        blocked_bwd_params<MT, ET, kParamCW, VEC, LOGP><<<dim3((unsigned)((n + 7) / 8 * 8)), dim3(64), 0, st>>>(
            param_flows, gf, om, xm, params, nids, cids, pids, ne, bs, batch, pgroups, chunks, items, id0);
    }
}

template <int ET, bool VEC, bool LOGP>
void launch_et(float* edge_flows, float* param_flows, const float* gf, const float* om, const float* xm,
               const float* params, const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb,
               int64_t ne, int64_t bs, int64_t batch, hipStream_t st) {
    // parents per K chunk of the edge-flow product: 4 * KP
    if (bs <= 4)
        launch_edges<ET, 1, VEC, LOGP>(edge_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    else if (bs <= 8)
        launch_edges<ET, 2, VEC, LOGP>(edge_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    else if (bs <= 16)
        launch_edges<ET, 4, VEC, LOGP>(edge_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    else
        launch_edges<ET, kEdgeKPMax, VEC, LOGP>(edge_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch,
                                                st);
    // parents per group of the parameter-flow product: 16 * MT
    if (bs <= 16)
        launch_params<1, ET, VEC, LOGP>(param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    else
        launch_params<2, ET, VEC, LOGP>(param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
}

template <int ET, int NKP, bool VEC, bool LOGP>
void launch_fused(float* edge_flows, float* param_flows, const float* gf, const float* om, const float* xm,
                  const float* params, const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb,
                  int64_t ne, int64_t bs, int64_t batch, int disjoint, hipStream_t st) {
    const int64_t chunks = (ne + CE - 1) / CE;
    const int64_t items = nb * chunks;
    for (int64_t id0 = 0; id0 < items; id0 += kMaxGroups) {
        const int64_t n = items - id0 < kMaxGroups ? items - id0 : kMaxGroups;
        const dim3 grid((unsigned)((n + 7) / 8 * 8));
        if (chunks == 1)
            blocked_bwd_fused<ET, NKP, VEC, LOGP, true><<<grid, dim3(64), 0, st>>>(
                edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, ne, bs, batch, chunks, items, id0,
                disjoint);
        else
            blocked_bwd_fused<ET, NKP, VEC, LOGP, false><<<grid, dim3(64), 0, st>>>(
                edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, ne, bs, batch, chunks, items, id0,
                disjoint);
    }
}

template <int ET, bool VEC, bool LOGP>
void launch_fused_et(float* edge_flows, float* param_flows, const float* gf, const float* om, const float* xm,
                     const float* params, const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb,
                     int64_t ne, int64_t bs, int64_t batch, int disjoint, hipStream_t st) {
    if (bs <= 4)
        launch_fused<ET, 1, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, disjoint, st);
    else if (bs <= 8)
        launch_fused<ET, 2, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch,
                                       disjoint, st);
    else if (bs <= 16)
        launch_fused<ET, 4, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch,
                                       disjoint, st);
    else
        launch_fused<ET, 8, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch,
                                       disjoint, st);
}

template <bool VEC, bool LOGP>
void launch_all(float* edge_flows, float* param_flows, const float* gf, const float* om, const float* xm,
                const float* params, const int64_t* nids, const int64_t* cids, const int64_t* pids, int64_t nb,
                int64_t ne, int64_t bs, int64_t batch, int disjoint, hipStream_t st) {
    if (bs <= kFusedMaxBs) {
        if (ne <= 16)
            launch_fused_et<1, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs,
                                          batch, disjoint, st);
        else
            launch_fused_et<2, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs,
                                          batch, disjoint, st);
    } else if (ne <= 16) {
        launch_et<1, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    } else {
        launch_et<2, VEC, LOGP>(edge_flows, param_flows, gf, om, xm, params, nids, cids, pids, nb, ne, bs, batch, st);
    }
}

}  // namespace

}  // namespace sparse
}  // namespace fl

using namespace fl;

extern "C" int fl_sparse_blocked_bwd(const float* node_flows, const float* node_mars, const float* element_mars,
                                     const float* params, const int64_t* nids, const int64_t* cids,
                                     const int64_t* pids, int64_t num_nblocks, int64_t num_edges, int64_t block_size,
                                     int64_t batch, int params_are_log, int params_disjoint, const int64_t* csc_offsets,
                                     const int32_t* csc_edges, int64_t num_elements, float* edge_flows,
                                     float* element_flows, float* param_flows, void* stream) {
    const char* name = "fl_sparse_blocked_bwd";
    FL_CHECK(num_nblocks >= 0 && num_edges >= 0 && block_size >= 0 && batch >= 0 && num_elements >= 0,
             "%s: negative size", name);
    if (num_nblocks == 0 || num_edges == 0 || block_size == 0 || batch == 0) return ok();
    FL_CHECK(node_flows && node_mars && element_mars && params && nids && cids && pids && csc_offsets && csc_edges &&
                 edge_flows && element_flows && param_flows,
             "%s: NULL pointer argument", name);
    FL_CHECK(num_nblocks * num_edges < ((int64_t)1 << 31), "%s: block edges must be < 2^31", name);
    const bool vec = (batch % 4 == 0) &&
                     ((reinterpret_cast<uintptr_t>(node_flows) | reinterpret_cast<uintptr_t>(node_mars) |
                       reinterpret_cast<uintptr_t>(element_mars) | reinterpret_cast<uintptr_t>(edge_flows) |
                       reinterpret_cast<uintptr_t>(element_flows)) & 15) == 0;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t nb = num_nblocks, ne = num_edges, bs = block_size;
    if (vec) {
        if (params_are_log)
            sparse::launch_all<true, true>(edge_flows, param_flows, node_flows, node_mars, element_mars, params, nids,
                                           cids, pids, nb, ne, bs, batch, params_disjoint ? 1 : 0, st);
        else
            sparse::launch_all<true, false>(edge_flows, param_flows, node_flows, node_mars, element_mars, params,
                                            nids, cids, pids, nb, ne, bs, batch, params_disjoint ? 1 : 0, st);
    } else {
        if (params_are_log)
            sparse::launch_all<false, true>(edge_flows, param_flows, node_flows, node_mars, element_mars, params,
                                            nids, cids, pids, nb, ne, bs, batch, params_disjoint ? 1 : 0, st);
        else
            sparse::launch_all<false, false>(edge_flows, param_flows, node_flows, node_mars, element_mars, params,
                                             nids, cids, pids, nb, ne, bs, batch, params_disjoint ? 1 : 0, st);
    }
    if (num_elements > 0) {
        for_grid_chunks((num_elements + 3) / 4, 256, [&](int64_t b0, int64_t nb) {
            if (vec)
                sparse::blocked_bwd_elements<true><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
                    element_flows, edge_flows, csc_offsets, csc_edges, num_elements, batch, b0);
            else
                sparse::blocked_bwd_elements<false><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
                    element_flows, edge_flows, csc_offsets, csc_edges, num_elements, batch, b0);
        });
    }
    return launch_status(name);
}
