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
// child row of `batch` floats.
//
// Mapping: one wave per (node, batch tile of 64*VB columns); lane l owns
// columns 4*(l + 64 v) .. +3 (16-byte vectors) when the batch is a multiple of
// 4 and the rows are 16-byte aligned, else columns l + 64 v (scalars).  Edge
// metadata is loaded once per 64 edges into lanes and broadcast per edge with
// readlane, so the edge loop issues only the child-row loads, G edges at a
// time.
//
// fp32: an online (max, scaled sum) per column with one rescale per G edges.
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
#include "lse_common.hpp"

namespace fl {
namespace sparse {

constexpr int kNegInfQ = -0x3fffffff;
constexpr float kConv = 1.44269504089f * 65536.0f;
constexpr float kOutScale = 0.69314718056f / 65536.0f;
constexpr int G = 4;  // edges folded per group

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
    const uint32_t off = ((fr >> 8) >> shc) & 0xFCu;
    return (int)((uint32_t)hi + m + (uint32_t)*reinterpret_cast<const int*>(reinterpret_cast<const char*>(lut) + off));
}

__device__ __forceinline__ int quant(float logit) {
    const float r = __builtin_rintf(fmaxf(logit, -20000.0f) * kConv);
    int q;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(r));
    return q;
}

// Column ownership of one lane inside a batch tile.
template <bool VEC, int VB>
struct Cols {
    static constexpr int kPer = VEC ? 4 * VB : VB;  // columns per lane
    static constexpr int kTile = 64 * kPer;          // columns per wave tile
    // column index of slot i (i < kPer) for lane l in tile starting at b0
    __device__ static __forceinline__ int64_t col(int64_t b0, int l, int i) {
        return VEC ? b0 + 4 * (l + 64 * (i / 4)) + (i % 4) : b0 + l + 64 * i;
    }
    __device__ static __forceinline__ void load(const float* __restrict__ row, int64_t b0, int l, int64_t batch,
                                                float (&v)[kPer]) {
        if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int64_t c = b0 + 4 * (l + 64 * u);
                if (c < batch) {
                    f32x4 t = load_stream<f32x4>(row + c);
                    v[4 * u] = t.x; v[4 * u + 1] = t.y; v[4 * u + 2] = t.z; v[4 * u + 3] = t.w;
                } else {
                    v[4 * u] = v[4 * u + 1] = v[4 * u + 2] = v[4 * u + 3] = 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int64_t c = b0 + l + 64 * u;
                v[u] = c < batch ? row[c] : 0.0f;
            }
        }
    }
    __device__ static __forceinline__ void store(float* __restrict__ row, int64_t b0, int l, int64_t batch,
                                                 const float (&v)[kPer]) {
        if constexpr (VEC) {
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int64_t c = b0 + 4 * (l + 64 * u);
                if (c < batch) {
                    f32x4 t;
                    t.x = v[4 * u]; t.y = v[4 * u + 1]; t.z = v[4 * u + 2]; t.w = v[4 * u + 3];
                    store_stream<f32x4>(t, row + c);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < VB; ++u) {
                const int64_t c = b0 + l + 64 * u;
                if (c < batch) row[c] = v[u];
            }
        }
    }
};

// Edge metadata of one node held across the wave: lane l keeps edge
// (base + l) of the current 64-edge window; edge(e) broadcasts it.
struct EdgeWindow {
    int64_t cid;   // lane-held child id
    float logw;    // lane-held log-weight
};

__device__ __forceinline__ int64_t bcast64(int64_t v, int lane) {
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, lane);
    const int hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ float bcastf(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Q16.16 reduction of one node with ET chains: edges are taken in groups of
// GS = max(4, ET) so that edge g of a group always belongs to chain g % ET;
// every group start is a multiple of ET (windows are 64 edges).
template <int ET, bool VEC, int VB, typename META>
__device__ __forceinline__ void q16_chains(int64_t k, META meta, const float* __restrict__ child, int64_t batch,
                                           int64_t b0, const int* __restrict__ lut, float (&res)[Cols<VEC, VB>::kPer]) {
    using C = Cols<VEC, VB>;
    constexpr int P = C::kPer;
    constexpr int GS = ET > G ? ET : G;
    const int l = lane_id();
    int acc[ET][P];
#pragma unroll
    for (int c = 0; c < ET; ++c)
#pragma unroll
        for (int i = 0; i < P; ++i) acc[c][i] = kNegInfQ;
    for (int64_t w0 = 0; w0 < k; w0 += 64) {
        const EdgeWindow ew = w0 + l < k ? meta(w0, l) : EdgeWindow{0, 0.0f};
        const int wn = (int)(k - w0 < 64 ? k - w0 : 64);
        for (int j = 0; j < wn; j += GS) {
            const int gn = wn - j < GS ? wn - j : GS;
            float v[GS][P];
#pragma unroll
            for (int g = 0; g < GS; ++g)
                if (g < gn) C::load(child + bcast64(ew.cid, j + g) * batch, b0, l, batch, v[g]);
#pragma unroll
            for (int g = 0; g < GS; ++g) {
                if (g < gn) {
                    const float lw = bcastf(ew.logw, j + g);
#pragma unroll
                    for (int i = 0; i < P; ++i) acc[g % ET][i] = pair(acc[g % ET][i], quant(lw + v[g][i]), lut);
                }
            }
        }
    }
    // xor butterfly over the chains (distances ET/2 .. 1); chain 0 ends with the result
#pragma unroll
    for (int i = 0; i < P; ++i) {
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
}

// Reduce one node over a batch tile.  META(e0, lane) returns the EdgeWindow
// entry for edge e0 + lane (valid for e0 + lane < k).
template <bool Q16, bool VEC, int VB, typename META>
__device__ __forceinline__ void reduce_node(int64_t k, META meta, const float* __restrict__ child, int64_t batch,
                                            int64_t b0, float* __restrict__ out_row, const int* __restrict__ lut) {
    using C = Cols<VEC, VB>;
    constexpr int P = C::kPer;
    const int l = lane_id();
    float res[P];
    if constexpr (!Q16) {
        float m[P], s[P];
#pragma unroll
        for (int i = 0; i < P; ++i) { m[i] = -kInf; s[i] = 0.0f; }
        for (int64_t w0 = 0; w0 < k; w0 += 64) {
            const EdgeWindow ew = w0 + l < k ? meta(w0, l) : EdgeWindow{0, 0.0f};
            const int wn = (int)(k - w0 < 64 ? k - w0 : 64);
            int e = 0;
            for (; e + G <= wn; e += G) {
                float v[G][P];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const int64_t c = bcast64(ew.cid, e + g);
                    C::load(child + c * batch, b0, l, batch, v[g]);
                }
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float lw = bcastf(ew.logw, e + g);
#pragma unroll
                    for (int i = 0; i < P; ++i) v[g][i] += lw;
                }
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    float col[G];
#pragma unroll
                    for (int g = 0; g < G; ++g) col[g] = v[g][i];
                    lse_fold<true, G>(m[i], s[i], col);
                }
            }
            for (; e < wn; ++e) {
                float v[P];
                C::load(child + bcast64(ew.cid, e) * batch, b0, l, batch, v);
                const float lw = bcastf(ew.logw, e);
#pragma unroll
                for (int i = 0; i < P; ++i) {
                    float col[1] = {v[i] + lw};
                    lse_fold<true, 1>(m[i], s[i], col);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < P; ++i) res[i] = lse_finish<true>(m[i], s[i]);
    } else {
        const int et_n = k <= 8 ? 1 : k <= 16 ? 2 : k <= 32 ? 4 : 8;
        switch (et_n) {
        case 1: q16_chains<1, VEC, VB>(k, meta, child, batch, b0, lut, res); break;
        case 2: q16_chains<2, VEC, VB>(k, meta, child, batch, b0, lut, res); break;
        case 4: q16_chains<4, VEC, VB>(k, meta, child, batch, b0, lut, res); break;
        default: q16_chains<8, VEC, VB>(k, meta, child, batch, b0, lut, res); break;
        }
    }
    C::store(out_row, b0, l, batch, res);
}

template <bool Q16, bool VEC, int VB>
__global__ __launch_bounds__(256) void csr_kernel(const float* __restrict__ child, const int64_t* __restrict__ offsets,
                                                  const int32_t* __restrict__ cids, const float* __restrict__ logp,
                                                  float* __restrict__ out, int64_t num_nodes, int64_t batch,
                                                  int64_t tiles) {
    __shared__ int lut[64];
    if constexpr (Q16) {
        if (threadIdx.x < 64) lut[threadIdx.x] = kLut[threadIdx.x];
        __syncthreads();
    }
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * 4;
    for (int64_t w = wave; w < num_nodes * tiles; w += nwaves) {
        const int64_t n = w / tiles;
        const int64_t b0 = (w - n * tiles) * Cols<VEC, VB>::kTile;
        const int64_t e0 = offsets[n];
        const int64_t k = offsets[n + 1] - e0;
        auto meta = [&](int64_t w0, int l) { return EdgeWindow{(int64_t)cids[e0 + w0 + l], logp[e0 + w0 + l]}; };
        reduce_node<Q16, VEC, VB>(k, meta, child, batch, b0, out + n * batch, lut);
    }
}

// pyjuice block layout.  LOGP: params already hold log-weights.
template <bool Q16, bool VEC, int VB, bool LOGP>
__global__ __launch_bounds__(256) void blocked_kernel(float* __restrict__ node_mars, const float* __restrict__ element_mars,
                                                      const float* __restrict__ params, const int64_t* __restrict__ nids,
                                                      const int64_t* __restrict__ cids, const int64_t* __restrict__ pids,
                                                      int64_t num_nblocks, int64_t num_edges, int64_t block_size,
                                                      int64_t batch, int64_t tiles) {
    __shared__ int lut[64];
    if constexpr (Q16) {
        if (threadIdx.x < 64) lut[threadIdx.x] = kLut[threadIdx.x];
        __syncthreads();
    }
    const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * 4;
    const int64_t total = num_nblocks * block_size * tiles;
    for (int64_t w = wave; w < total; w += nwaves) {
        const int64_t jp = w / tiles;
        const int64_t b0 = (w - jp * tiles) * Cols<VEC, VB>::kTile;
        const int64_t j = jp / block_size;
        const int64_t p = jp - j * block_size;
        auto meta = [&](int64_t w0, int l) {
            const int64_t ge = j * num_edges + w0 + l;
            const float wv = params[pids[ge] + p];
            // log of the linear weight, clamped at the smallest fp32 denormal
            // (sparse_float_kernel.cu:76); accurate libm log, once per edge
            const float lw = LOGP ? wv : logf(fmaxf(wv, 1e-45f));
            return EdgeWindow{cids[ge], lw};
        };
        reduce_node<Q16, VEC, VB>(num_edges, meta, element_mars, batch, b0, node_mars + (nids[j] + p) * batch, lut);
    }
}

static int64_t grid_for(int64_t waves) {
    int64_t blocks = (waves + 3) / 4;
    const int64_t cap = (int64_t)1 << 20;  // grid-stride beyond ~1M blocks
    return blocks < 1 ? 1 : (blocks > cap ? cap : blocks);
}

template <bool Q16>
static void launch_csr(const float* child, const int64_t* off, const int32_t* cid, const float* lp, float* out,
                       int64_t nodes, int64_t batch, hipStream_t st) {
    const bool vec = (batch % 4 == 0) && ((reinterpret_cast<uintptr_t>(child) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec) {
        constexpr int VB = 2;
        const int64_t tiles = (batch + Cols<true, VB>::kTile - 1) / Cols<true, VB>::kTile;
        csr_kernel<Q16, true, VB><<<dim3((unsigned)grid_for(nodes * tiles)), dim3(256), 0, st>>>(child, off, cid, lp, out,
                                                                                                 nodes, batch, tiles);
    } else {
        constexpr int VB = 4;
        const int64_t tiles = (batch + Cols<false, VB>::kTile - 1) / Cols<false, VB>::kTile;
        csr_kernel<Q16, false, VB><<<dim3((unsigned)grid_for(nodes * tiles)), dim3(256), 0, st>>>(child, off, cid, lp,
                                                                                                  out, nodes, batch, tiles);
    }
}

template <bool Q16, bool LOGP>
static void launch_blocked(float* nm, const float* em, const float* params, const int64_t* nids, const int64_t* cids,
                           const int64_t* pids, int64_t nb, int64_t ne, int64_t bs, int64_t batch, hipStream_t st) {
    const bool vec = (batch % 4 == 0) && ((reinterpret_cast<uintptr_t>(nm) | reinterpret_cast<uintptr_t>(em)) & 15) == 0;
    if (vec) {
        constexpr int VB = 2;
        const int64_t tiles = (batch + Cols<true, VB>::kTile - 1) / Cols<true, VB>::kTile;
        blocked_kernel<Q16, true, VB, LOGP><<<dim3((unsigned)grid_for(nb * bs * tiles)), dim3(256), 0, st>>>(
            nm, em, params, nids, cids, pids, nb, ne, bs, batch, tiles);
    } else {
        constexpr int VB = 4;
        const int64_t tiles = (batch + Cols<false, VB>::kTile - 1) / Cols<false, VB>::kTile;
        blocked_kernel<Q16, false, VB, LOGP><<<dim3((unsigned)grid_for(nb * bs * tiles)), dim3(256), 0, st>>>(
            nm, em, params, nids, cids, pids, nb, ne, bs, batch, tiles);
    }
}

}  // namespace sparse
}  // namespace fl

using namespace fl;

extern "C" int fl_sparse_csr_fwd(const float* child, const int64_t* offsets, const int32_t* child_ids,
                                 const float* logparams, float* out, int64_t num_nodes, int64_t batch, int q16,
                                 void* stream) {
    const char* name = "fl_sparse_csr_fwd";
    FL_CHECK(num_nodes >= 0 && batch >= 0, "%s: negative size", name);
    if (num_nodes == 0 || batch == 0) return ok();
    FL_CHECK(child && offsets && out, "%s: NULL pointer argument", name);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (q16)
        sparse::launch_csr<true>(child, offsets, child_ids, logparams, out, num_nodes, batch, st);
    else
        sparse::launch_csr<false>(child, offsets, child_ids, logparams, out, num_nodes, batch, st);
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
    const int sel = (q16 ? 2 : 0) | (params_are_log ? 1 : 0);
    switch (sel) {
    case 0: sparse::launch_blocked<false, false>(node_mars, element_mars, params, nids, cids, pids, num_nblocks, num_edges, block_size, batch, st); break;
    case 1: sparse::launch_blocked<false, true>(node_mars, element_mars, params, nids, cids, pids, num_nblocks, num_edges, block_size, batch, st); break;
    case 2: sparse::launch_blocked<true, false>(node_mars, element_mars, params, nids, cids, pids, num_nblocks, num_edges, block_size, batch, st); break;
    default: sparse::launch_blocked<true, true>(node_mars, element_mars, params, nids, cids, pids, num_nblocks, num_edges, block_size, batch, st); break;
    }
    return launch_status(name);
}
