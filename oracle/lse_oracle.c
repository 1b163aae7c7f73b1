/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference's log-sum-exp
 * arithmetic.  Nothing in the shipped package links or loads this file; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker (or as the timed CPU baseline), never as the product.
 *
 * Each function names the reference lines it restates (paths relative to the
 * lingyunyao/fuselse tree).  What pins each function:
 *   or_q16_pair / or_q16_quant_*   : compiled reference intlse/cpu/lse_kernel_simd.c
 *                                    (oracle/_ref, bit-exact, N<64 scalar rows and
 *                                    N=2 sweeps), closed forms, log2 error bound.
 *   or_intlse_cpu_row[_neg_inf]    : compiled reference (oracle/_ref), bit-exact.
 *   or_q10_6_pair                  : closed forms, exhaustive log2 error bound,
 *                                    LUT = round(Q16 LUT / 1024) identity.
 *   or_q16_gpu_rows / or_q10_6_rows: hand-computed rows that fix the tree shape
 *                                    (single chain, all-equal rows, prefix/suffix
 *                                    layout, chunk t+256k striding in ascending k
 *                                    with x..w element order) plus the reference's
 *                                    published accuracy envelopes (mean |err| vs
 *                                    fp64 per N).
 *   or_sparse_q16_*                : closed forms (one edge, equal edges), a
 *                                    hand-computed row fixing the e mod ET edge
 *                                    striding, and the float oracle envelope.
 *   or_fuselse_cpu_rows            : compiled reference fuselse/cpu/fused_fp32_cpu.cpp
 *                                    (oracle/_ref, bit-exact, and the fixture
 *                                    tests/golden/fuselse_cpu_ref.npz written from it),
 *                                    fp64 envelope, N=2 textbook identity.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define Q16_FRAC 16
#define Q16_ONE (1 << Q16_FRAC)
#define Q16_MASK (Q16_ONE - 1)
#define Q10_FRAC 6
#define Q10_ONE (1 << Q10_FRAC)
#define Q10_MASK (Q10_ONE - 1)

/* Identity the GPU kernels seed empty chains with (lse_kernel.cu:85,
 * lse_kernel_q10_6.cu:81, sparse_q16_kernel.cu:19). */
#define GPU_NEG_INF (-0x3fffffff)
/* Sentinel of the CPU -inf variants (lse_kernel_simd.c:22). */
#define CPU_NEG_INF INT32_MIN

/* Correction table: Mitchell error of log2(1 + 2^z) per 1/64 bin of the
 * linear term, Q16.16 (lse_kernel.cu:35-44 = lse_kernel_simd.c:24-33). */
static const int32_t LUT_Q16[64] = {
       0,  571,  907, 1282, 1634, 1745, 2054, 2592,
    2900, 2859, 2895, 3015, 3222, 3522, 3922, 4426,
    4617, 4441, 4294, 4178, 4093, 4039, 4018, 4030,
    4076, 4157, 4272, 4424, 4613, 4838, 5102, 5404,
    5399, 5068, 4746, 4435, 4134, 3843, 3562, 3291,
    3031, 2781, 2541, 2312, 2094, 1886, 1689, 1502,
    1327, 1162, 1008,  865,  732,  611,  500,  401,
     312,  235,  168,  113,   69,   35,   13,    2,
};

/* The same table at 6 fractional bits (lse_kernel_q10_6.cu:27-32). */
static const int32_t LUT_Q10_6[64] = {
    0, 1, 1, 1, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3, 4, 4,
    5, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 5, 5, 5, 5,
    5, 5, 5, 4, 4, 4, 3, 3, 3, 3, 2, 2, 2, 2, 2, 1,
    1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
};

int32_t or_lut_q16(int i) { return LUT_Q16[i & 63]; }
int32_t or_lut_q10_6(int i) { return LUT_Q10_6[i & 63]; }

/* fl32(fl32(1.44269504089f) * 65536) and fl32(0.69314718056f) / 65536
 * (lse_kernel.cu:28-30,156). */
static float q16_conv(void) { return 1.44269504089f * (float)Q16_ONE; }
static float q16_out_scale(void) { return 0.69314718056f / (float)Q16_ONE; }
static float q10_out_scale(void) { return 0.69314718056f / (float)Q10_ONE; }

static inline int32_t wrap_sub(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a - (uint32_t)b);
}
static inline int32_t wrap_add3(int32_t a, int32_t b, int32_t c) {
    return (int32_t)((uint32_t)a + (uint32_t)b + (uint32_t)c);
}

/* Arithmetic right shift of a 32-bit value with the shift count read as an
 * unsigned 32-bit number and counts of 32 or more producing the sign fill:
 * the semantics of a variable `>>` on NVIDIA (PTX shr clamps the count) and
 * of AVX2 vpsravd. */
static inline int32_t sar_clamped(int32_t v, int32_t count) {
    uint32_t c = (uint32_t)count;
    if (c >= 32u) return v < 0 ? -1 : 0;
    return v >> c;
}
/* The same shift as x86 scalar `sar %cl` executes it: count taken mod 32. */
static inline int32_t sar_mod32(int32_t v, int32_t count) {
    return v >> ((uint32_t)count & 31u);
}

/* Q16.16 base-2 pair LSE, GPU / SIMD semantics (lse_kernel.cu:46-57,
 * sparse_q16_kernel.cu:43-51, lse_kernel_simd.c:60-83). */
int32_t or_q16_pair(int32_t x, int32_t y, int use_lut) {
    int32_t hi = x > y ? x : y;
    int32_t lo = x > y ? y : x;
    int32_t sub = wrap_sub(lo, hi);
    int32_t shift = -(sub >> Q16_FRAC);
    if (shift > 31) shift = 31; /* signed clamp (kept: negative counts pass) */
    int32_t m = sar_clamped(Q16_ONE + (sub & Q16_MASK), shift);
    int32_t c = use_lut ? LUT_Q16[(m >> 10) & 63] : 0;
    return wrap_add3(hi, m, c);
}

/* Q16.16 pair as the reference's scalar C helper runs on x86
 * (lse_kernel_simd.c:41-49): identical except for a negative count, which only
 * arises when the operands differ by more than 2^31 (wrapped subtraction). */
int32_t or_q16_pair_x86(int32_t x, int32_t y) {
    int32_t hi = x > y ? x : y;
    int32_t lo = x > y ? y : x;
    int32_t sub = wrap_sub(lo, hi);
    int32_t shift = -(sub >> Q16_FRAC);
    if (shift > 31) shift = 31;
    int32_t m = sar_mod32(Q16_ONE + (sub & Q16_MASK), shift);
    return wrap_add3(hi, m, LUT_Q16[(m >> 10) & 63]);
}

static inline int32_t q16_pair_x86_neg_inf(int32_t x, int32_t y) {
    if (x == CPU_NEG_INF) return y; /* lse_kernel_simd.c:51-55 */
    if (y == CPU_NEG_INF) return x;
    return or_q16_pair_x86(x, y);
}

static inline int32_t q16_pair_simd_neg_inf(int32_t x, int32_t y) {
    int32_t r = or_q16_pair(x, y, 1); /* lse_kernel_simd.c:85-92: blend y then x */
    if (x == CPU_NEG_INF) r = y;
    if (y == CPU_NEG_INF) r = x;
    return r;
}

/* Q10.6 base-2 pair LSE (lse_kernel_q10_6.cu:35-43). */
int32_t or_q10_6_pair(int32_t x, int32_t y) {
    int32_t hi = x > y ? x : y;
    int32_t lo = x > y ? y : x;
    int32_t sub = wrap_sub(lo, hi);
    int32_t shift = -(sub >> Q10_FRAC);
    if (shift > 31) shift = 31;
    int32_t m = sar_clamped(Q10_ONE + (sub & Q10_MASK), shift);
    return wrap_add3(hi, m, LUT_Q10_6[m & Q10_MASK]);
}

/* float -> int32, round to nearest even, saturating, NaN -> 0: the PTX
 * cvt.rni.s32.f32 behaviour of __float2int_rn. */
static inline int32_t rne_sat_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f < -2147483648.0f) return INT32_MIN;
    return (int32_t)nearbyintf(f); /* default rounding mode: nearest even */
}

/* GPU quantiser q = __float2int_rn(v * CONV) (lse_kernel.cu:99,114). */
int32_t or_q16_quant_gpu(float v) {
    volatile float p = v * q16_conv(); /* one fp32 rounding, no contraction */
    return rne_sat_i32(p);
}

/* Sparse quantiser __float2int_rn(fmaxf(logit, -20000) * CONV)
 * (sparse_q16_kernel.cu:113). fmaxf returns the non-NaN operand. */
int32_t or_q16_quant_sparse(float logit) {
    float c = fmaxf(logit, -20000.0f);
    volatile float p = c * q16_conv();
    return rne_sat_i32(p);
}

/* CPU scalar quantiser (lse_kernel_simd.c:35-39): saturate at +-2147483520,
 * else lroundf (half away from zero). */
int32_t or_q16_quant_cpu_scalar(float v) {
    volatile float f = v * q16_conv();
    if (f >= 2147483520.0f) return 2147483647;
    if (f <= -2147483520.0f) return -2147483647;
    return (int32_t)lroundf(f);
}

/* CPU SIMD quantiser (lse_kernel_simd.c:97-105): max_ps(f, lo) returns lo for
 * a NaN first operand, min_ps(., hi), then cvtps (nearest even). */
int32_t or_q16_quant_cpu_simd(float v) {
    volatile float f = v * q16_conv();
    const float lo = -2147483520.0f, hi = 2147483520.0f;
    float a = (f > lo) ? f : lo; /* maxps: second operand unless first > second */
    float b = (a < hi) ? a : hi; /* minps: second operand unless first < second */
    return (int32_t)nearbyintf(b);
}

/* ------------------------------------------------------------------------ */
/* CPU IntLSE AVX2 (lse_kernel_simd.c:164-315), eight lanes emulated.         */
/* ------------------------------------------------------------------------ */
#define SIMD_BLOCK 64

static float intlse_cpu_row(const float* in, int n, int neg_inf_variant) {
    if (n <= 0) return -INFINITY;          /* :167 */
    if (n == 1) return in[0];              /* :168 */
    const float oscale = q16_out_scale();
    if (n < SIMD_BLOCK) {                  /* :171-178, :242-255 */
        int32_t acc;
        if (neg_inf_variant) {
            acc = in[0] == -INFINITY ? CPU_NEG_INF : or_q16_quant_cpu_scalar(in[0]);
            for (int i = 1; i < n; i++) {
                int32_t q = in[i] == -INFINITY ? CPU_NEG_INF : or_q16_quant_cpu_scalar(in[i]);
                acc = q16_pair_x86_neg_inf(acc, q);
            }
            return acc == CPU_NEG_INF ? -INFINITY : (float)acc * oscale;
        }
        acc = or_q16_quant_cpu_scalar(in[0]);
        for (int i = 1; i < n; i++) acc = or_q16_pair_x86(acc, or_q16_quant_cpu_scalar(in[i]));
        return (float)acc * oscale;
    }
    int nblk = n / SIMD_BLOCK;
    int tail = nblk * SIMD_BLOCK;
    int32_t* part = (int32_t*)malloc(sizeof(int32_t) * 8 * (size_t)nblk);
    /* pass 1: per block, lane l folds elements l, l+8, ..., l+56 (:195-203) */
    for (int b = 0; b < nblk; b++) {
        const float* p = in + (size_t)b * SIMD_BLOCK;
        for (int l = 0; l < 8; l++) {
            int32_t acc = 0;
            for (int i = 0; i < SIMD_BLOCK; i += 8) {
                float v = p[i + l];
                int32_t q = or_q16_quant_cpu_simd(v);
                if (neg_inf_variant && v == -INFINITY) q = CPU_NEG_INF;
                if (i == 0) acc = q;
                else acc = neg_inf_variant ? q16_pair_simd_neg_inf(acc, q) : or_q16_pair(acc, q, 1);
            }
            part[b * 8 + l] = acc;
        }
    }
    /* pass 2: pairwise tree, odd leftover moves to the end (:205-213) */
    int cnt = nblk;
    while (cnt > 1) {
        int half = cnt / 2;
        for (int i = 0; i < half; i++)
            for (int l = 0; l < 8; l++) {
                int32_t a = part[(2 * i) * 8 + l], c = part[(2 * i + 1) * 8 + l];
                part[i * 8 + l] = neg_inf_variant ? q16_pair_simd_neg_inf(a, c) : or_q16_pair(a, c, 1);
            }
        if (cnt & 1) {
            memmove(&part[half * 8], &part[(cnt - 1) * 8], 8 * sizeof(int32_t));
            cnt = half + 1;
        } else {
            cnt = half;
        }
    }
    /* 8 -> 4 -> 2 -> 1 lane tree with the scalar helper (:125-148) */
    int32_t (*pf)(int32_t, int32_t) = neg_inf_variant ? q16_pair_x86_neg_inf : or_q16_pair_x86;
    int32_t a01 = pf(part[0], part[1]), a23 = pf(part[2], part[3]);
    int32_t a45 = pf(part[4], part[5]), a67 = pf(part[6], part[7]);
    int32_t acc = pf(pf(a01, a23), pf(a45, a67));
    free(part);
    /* scalar tail (:221-224, :299-304) */
    for (int i = tail; i < n; i++) {
        int32_t q;
        if (neg_inf_variant && in[i] == -INFINITY) q = CPU_NEG_INF;
        else q = or_q16_quant_cpu_scalar(in[i]);
        acc = pf(acc, q);
    }
    if (neg_inf_variant && acc == CPU_NEG_INF) return -INFINITY;
    return (float)acc * oscale;
}

void or_intlse_cpu_rows(const float* in, int64_t B, int64_t N, int neg_inf_variant, float* out) {
    for (int64_t b = 0; b < B; b++) out[b] = intlse_cpu_row(in + b * N, (int)N, neg_inf_variant);
}

/* ------------------------------------------------------------------------ */
/* GPU IntLSE tree (lse_kernel.cu:67-159, lse_kernel_q10_6.cu:55-139).        */
/* 256 virtual threads per row; thread t chains its alignment-prefix element, */
/* its vector chunks t, t+256, ... (lane order inside a chunk) and its suffix */
/* element, seeded with its first element; then a 32-lane xor butterfly per   */
/* virtual warp, and warp 0 folds the 8 warp partials padded with 24 copies   */
/* of the identity.                                                           */
/* ------------------------------------------------------------------------ */
#define VT 256

typedef int32_t (*pair_fn)(int32_t, int32_t);
static int32_t q16_lut(int32_t a, int32_t b) { return or_q16_pair(a, b, 1); }
static int32_t q16_nolut(int32_t a, int32_t b) { return or_q16_pair(a, b, 0); }

static void butterfly32(int32_t* v, pair_fn pf) {
    int32_t t[32];
    for (int off = 16; off > 0; off >>= 1) {
        for (int i = 0; i < 32; i++) t[i] = pf(v[i], v[i ^ off]);
        memcpy(v, t, sizeof(t));
    }
}

/* q(): fetch element i of the row already quantised. */
typedef int32_t (*elem_fn)(const void* row, int64_t i);
static int32_t el_f32(const void* row, int64_t i) { return or_q16_quant_gpu(((const float*)row)[i]); }
static int32_t el_i32(const void* row, int64_t i) { return ((const int32_t*)row)[i]; }
static int32_t el_i16(const void* row, int64_t i) { return (int32_t)((const int16_t*)row)[i]; }

static int32_t gpu_tree_row(const void* row, int64_t n, int prefix, elem_fn el, pair_fn pf) {
    int32_t acc[VT];
    int has[VT];
    for (int t = 0; t < VT; t++) { acc[t] = GPU_NEG_INF; has[t] = 0; }
#define FOLD(t, q) do { int32_t q_ = (q); if (!has[t]) { acc[t] = q_; has[t] = 1; } else acc[t] = pf(acc[t], q_); } while (0)
    for (int64_t i = 0; i < prefix; i++) FOLD((int)i, el(row, i));
    int64_t rem = n - prefix;
    int64_t n4 = rem / 4;
    for (int t = 0; t < VT; t++)
        for (int64_t c = t; c < n4; c += VT)
            for (int k = 0; k < 4; k++) FOLD(t, el(row, prefix + 4 * c + k));
    int64_t suf = prefix + 4 * n4;
    for (int64_t i = suf; i < n; i++) FOLD((int)(i - suf), el(row, i));
#undef FOLD
    int32_t part[8];
    for (int w = 0; w < 8; w++) {
        butterfly32(&acc[32 * w], pf);
        part[w] = acc[32 * w];
    }
    int32_t fin[32];
    for (int i = 0; i < 32; i++) fin[i] = i < 8 ? part[i] : GPU_NEG_INF;
    butterfly32(fin, pf);
    return fin[0];
}

/* base_mod: byte address of row 0 modulo 16; rows are contiguous. Returns the
 * float outputs; raw (if non-NULL) receives the Q accumulators. */
void or_q16_gpu_rows(const void* in, int in_is_int32, int64_t B, int64_t N, int base_mod,
                     int use_lut, float* out, int32_t* raw) {
    const float oscale = q16_out_scale();
    for (int64_t b = 0; b < B; b++) {
        const char* row = (const char*)in + b * N * 4;
        int mis = (int)((base_mod + b * N * 4) & 15);
        int prefix = mis ? (16 - mis) / 4 : 0;
        if (prefix > N) prefix = (int)N;
        int32_t r = gpu_tree_row(row, N, prefix, in_is_int32 ? el_i32 : el_f32,
                                 use_lut ? q16_lut : q16_nolut);
        if (raw) raw[b] = r;
        out[b] = (float)r * oscale;
    }
}

void or_q10_6_rows(const int16_t* in, int64_t B, int64_t N, int base_mod, float* out, int32_t* raw) {
    const float oscale = q10_out_scale();
    for (int64_t b = 0; b < B; b++) {
        const int16_t* row = in + b * N;
        int mis = (int)((base_mod + b * N * 2) & 7);
        int prefix = mis ? (8 - mis) / 2 : 0;
        if (prefix > N) prefix = (int)N;
        int32_t r = gpu_tree_row(row, N, prefix, el_i16, or_q10_6_pair);
        if (raw) raw[b] = r;
        out[b] = (float)r * oscale;
    }
}

/* Q10.6 quantiser of the reduced-bit harness (run_bench.py:50-53,100-103):
 * int16(clamp(round_half_even(fl32(x * fl32(log2(e) * 64))), -32768, 32767)). */
void or_to_q10_6(const float* x, int64_t n, int16_t* q) {
    const float conv = (float)(1.4426950408889634 * 64.0);
    for (int64_t i = 0; i < n; i++) {
        volatile float p = x[i] * conv;
        float r = nearbyintf(p);
        if (r < -32768.0f) r = -32768.0f;
        if (r > 32767.0f) r = 32767.0f;
        q[i] = (int16_t)r;
    }
}

/* Q16.16 int32 input recipe: sat_int32(rne(fl32(x * CONV))). */
void or_to_q16(const float* x, int64_t n, int32_t* q) {
    for (int64_t i = 0; i < n; i++) q[i] = or_q16_quant_gpu(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Sparse PC Q16.16 (sparse_q16_kernel.cu:61-134).                           */
/* ------------------------------------------------------------------------ */
static int edge_threads_for(int64_t fan_in) {   /* :161-165 (== float :127-131) */
    if (fan_in <= 8) return 1;
    if (fan_in <= 16) return 2;
    if (fan_in <= 32) return 4;
    return 8;
}
int or_edge_threads(int64_t fan_in) { return edge_threads_for(fan_in); }

/* One (node, b): ET chains over edges e = et, et+ET, ... seeded with the
 * identity, then an xor butterfly over ET lanes; lane 0 holds the result. */
static float sparse_q16_reduce(const float* logits, int64_t k, int32_t* raw) {
    int et_n = edge_threads_for(k);
    int32_t acc[8];
    for (int et = 0; et < et_n; et++) {
        acc[et] = GPU_NEG_INF;
        for (int64_t e = et; e < k; e += et_n) acc[et] = or_q16_pair(acc[et], or_q16_quant_sparse(logits[e]), 1);
    }
    int32_t t[8];
    for (int off = et_n / 2; off > 0; off >>= 1) {
        for (int i = 0; i < et_n; i++) t[i] = or_q16_pair(acc[i], acc[i ^ off], 1);
        memcpy(acc, t, sizeof(int32_t) * et_n);
    }
    if (raw) *raw = acc[0];
    return acc[0] > GPU_NEG_INF ? (float)acc[0] * q16_out_scale() : -INFINITY; /* :129-131 */
}

/* CSR layout: node n owns edges [off[n], off[n+1]); edge e reads
 * child[cid[e] * batch + b] and adds logparam[e] (one fp32 add). out is
 * [num_nodes][batch]. */
void or_sparse_q16_csr(const float* child, const int64_t* off, const int32_t* cid,
                       const float* logparam, int64_t num_nodes, int64_t batch, float* out) {
    float* logits = NULL;
    int64_t cap = 0;
    for (int64_t n = 0; n < num_nodes; n++) {
        int64_t k = off[n + 1] - off[n];
        if (k > cap) { cap = k; logits = (float*)realloc(logits, sizeof(float) * (size_t)cap); }
        for (int64_t b = 0; b < batch; b++) {
            for (int64_t e = 0; e < k; e++) {
                int64_t ge = off[n] + e;
                logits[e] = logparam[ge] + child[(int64_t)cid[ge] * batch + b];
            }
            out[n * batch + b] = sparse_q16_reduce(logits, k, NULL);
        }
    }
    free(logits);
}

/* pyjuice block layout (sparse_q16_kernel.cu:61-134) with log-weights already
 * taken: logw[j][p][e] = log(max(params[pids[j,e] + p], 1e-45)), supplied by
 * the caller. Writes node_mars[(nids[j] + p) * batch + b]. */
void or_sparse_q16_blocked(float* node_mars, const float* element_mars, const float* logw,
                           const int64_t* nids, const int64_t* cids, int64_t num_nblocks,
                           int64_t num_edges, int64_t block_size, int64_t batch) {
    float* logits = (float*)malloc(sizeof(float) * (size_t)(num_edges > 0 ? num_edges : 1));
    for (int64_t j = 0; j < num_nblocks; j++)
        for (int64_t p = 0; p < block_size; p++)
            for (int64_t b = 0; b < batch; b++) {
                for (int64_t e = 0; e < num_edges; e++)
                    logits[e] = logw[(j * block_size + p) * num_edges + e] +
                                element_mars[cids[j * num_edges + e] * batch + b];
                node_mars[(nids[j] + p) * batch + b] = sparse_q16_reduce(logits, num_edges, NULL);
            }
    free(logits);
}

/* ------------------------------------------------------------------------ */
/* FuseLSE CPU (fused_fp32_cpu.cpp:22-46) and the backward formula of the     */
/* GPU kernel (fused_fp32_kernel.cu:135-150), for the timed CPU baseline.     */
/* ------------------------------------------------------------------------ */
static inline float pair_float(float x, float y) {
    float xm = (x > y) ? x : y;
    float ym = (x > y) ? y : x;
    return xm + log1pf(expf(ym - xm));
}

void or_fuselse_cpu_rows(const float* in, int64_t B, int64_t N, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < B; b++) {
        const float* row = in + b * N;
        float acc = row[0];
        for (int64_t i = 1; i < N; i++) acc = pair_float(acc, row[i]);
        out[b] = acc;
    }
}

void or_lse_backward_rows(const float* g, const float* x, const float* lse, int64_t B, int64_t N,
                          float* gx) {
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < B; b++)
        for (int64_t i = 0; i < N; i++) gx[b * N + i] = g[b] * expf(x[b * N + i] - lse[b]);
}

void or_omp_set_threads(int n) {
#ifdef _OPENMP
    extern void omp_set_num_threads(int);
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

int or_omp_max_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* Batch helpers for the tests (elementwise over arrays).                    */
/* ------------------------------------------------------------------------ */
void or_q16_pair_batch(const int32_t* a, const int32_t* b, int64_t n, int mode, int32_t* out) {
    /* mode 0: GPU/SIMD with LUT, 1: GPU without LUT, 2: x86 scalar helper */
    for (int64_t i = 0; i < n; i++)
        out[i] = mode == 2 ? or_q16_pair_x86(a[i], b[i]) : or_q16_pair(a[i], b[i], mode == 0);
}

void or_q10_6_pair_batch(const int32_t* a, const int32_t* b, int64_t n, int32_t* out) {
    for (int64_t i = 0; i < n; i++) out[i] = or_q10_6_pair(a[i], b[i]);
}

void or_q16_quant_batch(const float* x, int64_t n, int mode, int32_t* out) {
    /* mode 0: GPU, 1: sparse (fmaxf -20000), 2: CPU scalar, 3: CPU SIMD */
    for (int64_t i = 0; i < n; i++) {
        switch (mode) {
        case 0: out[i] = or_q16_quant_gpu(x[i]); break;
        case 1: out[i] = or_q16_quant_sparse(x[i]); break;
        case 2: out[i] = or_q16_quant_cpu_scalar(x[i]); break;
        default: out[i] = or_q16_quant_cpu_simd(x[i]); break;
        }
    }
}
