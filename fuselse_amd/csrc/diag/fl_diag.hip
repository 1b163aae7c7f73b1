// The measurement library (libfuselse_amd_diag.so, include/fuselse_amd_diag.h):
// bandwidth and latency references and per-block timestamps of the library's
// kernels.  None of it has a counterpart in the reference.
//
// Read-bandwidth reference: streams a buffer from HBM with the forward
// kernels' load form (16-byte buffer loads with the nontemporal hint) in a
// flat grid-stride order, and does nothing else with the data.  Its rate over
// the forward's own input buffers, in the same run, is the read ceiling the
// forward is held against.
#include <stdint.h>

#include "../../../include/fuselse_amd.h"
#include "../../../include/fuselse_amd_diag.h"
#include "../fl_status.hpp"
#include "../lse_common.hpp"
#include "../lse_fwd_kernels.hpp"
#include "../lse_int_kernels.hpp"
#include "../lse_pair.hpp"
#include "../lse_tile_layout.hpp"

namespace fl {

// Block b reads chunks b, b + gridDim.x, ... of TPB * U * 16 bytes; lane t
// of the block reads bytes (t + u * TPB) * 16 of a chunk (u < U), so each
// group of U loads is issued back to back and every wave's loads are fully
// coalesced.  The xor of the words feeds a store that happens only when it
// equals a constant no realistic input produces, which keeps the loads live.
template <int TPB, int U>
__global__ __launch_bounds__(TPB) void read_stream_kernel(const char* __restrict__ x, int64_t nbytes,
                                                          uint32_t* __restrict__ sink) {
    constexpr int64_t CHUNK = TPB * U * 16;
    const int tid = threadIdx.x;
    uint32_t acc = 0;
    for (int64_t c = blockIdx.x; c * CHUNK < nbytes; c += gridDim.x) {
        const int64_t left = nbytes - c * CHUNK;
        const int nrec = left > CHUNK ? (int)CHUNK : (int)left;
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(x + c * CHUNK), 0, nrec, 0x00020000);
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (tid + u * TPB) * 16, 0, kLoadStreamAux);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Read+write reference (no counterpart in the reference): copies a buffer
// with the backward kernels' forms, 16-byte nontemporal buffer loads and
// 16-byte buffer stores written through to memory (sc1 nt), in a flat
// grid-stride order over chunks of TPB * U * 16 bytes.  Its rate is the copy ceiling the
// fused backward (one read and one write of the row) is held against.
template <int TPB, int U>
__global__ __launch_bounds__(TPB) void copy_stream_kernel(const char* __restrict__ x, char* __restrict__ y,
                                                          int64_t nbytes) {
    constexpr int64_t CHUNK = TPB * U * 16;
    const int tid = threadIdx.x;
    for (int64_t c = blockIdx.x; c * CHUNK < nbytes; c += gridDim.x) {
        const int64_t left = nbytes - c * CHUNK;
        const int nrec = left > CHUNK ? (int)CHUNK : (int)left;
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(x + c * CHUNK), 0, nrec, 0x00020000);
        const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(y + c * CHUNK, 0, nrec, 0x00020000);
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, (tid + u * TPB) * 16, 0, kLoadStreamAux);
#pragma unroll
        for (int u = 0; u < U; ++u) __builtin_amdgcn_raw_buffer_store_b128(v[u], ry, (tid + u * TPB) * 16, 0, kStoreStreamAux);
    }
}

// Dependent-chain latencies of the IntLSE pair steps (no counterpart in the
// reference).  Each wave of one block (one CU) runs `steps` (a multiple of
// 16) dependent steps
// of one kind and records the shader-clock cycles (s_memtime) and the 100 MHz
// real-time ticks (s_memrealtime) the chain took:
//   KIND 0: v_add_u32 of the previous value;
//   KIND 1: ds_read_u8 addressed by the previous value (a table of bytes);
//   KIND 2: the Q10.6 pair step of the row kernels (max, two subtracts, med3,
//           ds_read_u8 of the gap table, add), q10_pair;
//   KIND 3: the Q16.16 pair step with its LDS correction table, q16_pair;
//   KIND 4: ds_read_b128, lane l reading words 4l .. 4l+3 of the table
//           (no two lanes share a bank row), addressed by the previous value
//           (the table holds each slot's own index): the reference figure
//           for the LDS bank-conflict counter on 16-byte accesses;
//   KIND 5: ds_write_b128 of the lane's own 16-byte slot, then the KIND 4
//           read of it (the same figure for 16-byte writes);
//   KIND 6: ds_read_b128 at row l % 16, block 4 (l / 16) of rows of 68 words:
//           the transposed tile read with the rows padded in place;
//   KIND 7: ds_write_b128, then the read, at row 4 (l / 16), block l % 16 of the
//           same rows: the row-wise tile stores and reloads;
//   KIND 8, 9: KIND 6 and 7 in the layout the block-layout backward keeps
//           its tiles in (rows of kTileLD words, blocks placed by tile_col).
// The operand each step pairs with comes from the step index (a scalar
// value), so the only dependence is through the chain.  With 64 * w threads
// the block puts w / 4 waves on each of the CU's four SIMDs.
template <int KIND>
__device__ __forceinline__ int slot_word(int i) {
    if constexpr (KIND == 6) return 68 * (i & 15) + 16 * (i >> 4);
    else if constexpr (KIND == 7) return 68 * 4 * (i >> 4) + 4 * (i & 15);
    else if constexpr (KIND == 8) return sparse::kTileLD * (i & 15) + sparse::tile_col(i & 15, 16 * (i >> 4));
    else if constexpr (KIND == 9) return sparse::kTileLD * 4 * (i >> 4) + sparse::tile_col(4 * (i >> 4), 4 * (i & 15));
    else return 4 * i;
}

template <int KIND>
__global__ __launch_bounds__(1024) void chain_latency_kernel(int steps, uint64_t* __restrict__ rec) {
    __shared__ uint8_t tab8[512];  // first: its LDS address is the byte index
    __shared__ int lut[64];
    __shared__ __align__(16) uint32_t tabw[16 * sparse::kTileLD];  // 16-byte slots: slot_word(i) holds {i, i, 0, 0}
    for (int i = threadIdx.x; i < 512; i += blockDim.x) tab8[i] = (uint8_t)((i * 7) % 70);
    for (int i = threadIdx.x; i < 64; i += blockDim.x) lut[i] = (i * 613) & 0x1FFF;
    for (int i = threadIdx.x; i < 64; i += blockDim.x)
        *reinterpret_cast<u32x4*>(&tabw[slot_word<KIND>(i)]) = u32x4{(uint32_t)i, (uint32_t)i, 0u, 0u};
    __syncthreads();
    int a = KIND >= 4 ? (int)(threadIdx.x & 63) : (int)(threadIdx.x & 7);
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    // 16 steps per loop trip, fully unrolled, so the loop's own scalar
    // instructions and branch fall on one step in 16
    for (int k0 = 0; k0 < steps; k0 += 16) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int k = k0 + u;
            if constexpr (KIND == 0) {
                asm volatile("v_add_u32 %0, %0, %1" : "+v"(a) : "s"(k));
            } else if constexpr (KIND == 1) {
                a = tab8[a];  // table bytes are below 70, so the chain stays in the table
            } else if constexpr (KIND == 2) {
                a = q10_pair(a, (int)(((uint32_t)k * 2654435761u) >> 22) - 512, tab8);
            } else if constexpr (KIND == 3) {
                a = q16_pair<true>(a, (int)((uint32_t)k * 2654435761u) >> 6, lut);
            } else {
                u32x4* slot = reinterpret_cast<u32x4*>(&tabw[slot_word<KIND>(a)]);
                // the lane's own slot only: every wave writes the same words,
                // and slot a keeps holding a, so the chain stays on it
                if constexpr (KIND == 5 || KIND == 7 || KIND == 9) {
                    *slot = u32x4{(uint32_t)a, (uint32_t)k, 0u, 0u};
                    asm volatile("" ::: "memory");  // the read goes to LDS, not back from the stored registers
                }
                const u32x4 v = *slot;
                a = (int)(v.x | v.z);
            }
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        rec[3 * w + 0] = t1 - t0;
        rec[3 * w + 1] = r1 - r0;
        rec[3 * w + 2] = (uint64_t)(uint32_t)a;  // keeps the chain live
    }
}

// ---------------------------------------------------------------------------
// Per-block timestamps.  s_memrealtime reads the 100 MHz real-time counter,
// s_memtime the shader clock; XCC_ID (hardware register 20) names the XCD a
// wave runs on, HW_ID (register 4) its SIMD, CU, shader array and engine.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t rt_now() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint64_t clk_now() { return __builtin_amdgcn_s_memtime(); }
__device__ __forceinline__ uint32_t xcc_id() { return (uint32_t)__builtin_amdgcn_s_getreg((3 << 11) | 20); }
__device__ __forceinline__ uint32_t hw_id() { return (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4); }

__device__ __forceinline__ void put_block_record(uint64_t* rec, int64_t i, uint64_t t0, uint64_t c0) {
    const uint64_t t1 = rt_now();
    const uint64_t c1 = clk_now();
    uint64_t* r = rec + 6 * i;
    r[0] = t0;
    r[1] = t1;
    r[2] = c1 - c0;
    r[3] = xcc_id();
    r[4] = hw_id();
    r[5] = (uint64_t)i;
}

// The forward's row output with a record per row: begin() runs on the row's
// first thread before its loads, end() once the row's LSE is known.
struct TimedLseOut {
    float* __restrict__ out;
    uint64_t* __restrict__ rec;
    struct Row {
        uint64_t t0 = 0, c0 = 0;
    };
    __device__ __forceinline__ Row begin(int64_t) const { return {rt_now(), clk_now()}; }
    __device__ __forceinline__ void end(int64_t row, Row r, float lse) const {
        out[row] = lse;
        put_block_record(rec, row, r.t0, r.c0);
    }
};

// One 256-thread block per row, the forward's loads and software pipeline
// (two register sets of U vectors per lane) with an xor in place of the fold.
template <int U>
__global__ __launch_bounds__(256) void read_rows_kernel(const float* __restrict__ x, int64_t N,
                                                        uint64_t* __restrict__ rec, uint32_t* __restrict__ sink) {
    constexpr int STRIDE = 256;
    __shared__ uint32_t sh[4];
    const uint64_t t0 = rt_now();
    const uint64_t c0 = clk_now();
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t nvec = N / 4;
    const char* base = reinterpret_cast<const char*>(uniform64(reinterpret_cast<int64_t>(x + row * N)));
    const int64_t region = uniform64(nvec * 16);
    const int64_t trips = uniform64(batches<(int64_t)U * STRIDE>(nvec));
    uint32_t acc = 0;
    if (trips > 0) {
        u32x4 a[U], c[U];
        load_batch<STRIDE, U>(a, base, region, tid * 16, 0);
        __builtin_amdgcn_sched_barrier(0);
        int64_t t = 1;
        while (true) {
            if (t == trips) {
#pragma unroll
                for (int u = 0; u < U; ++u) acc ^= a[u][0] ^ a[u][1] ^ a[u][2] ^ a[u][3];
                break;
            }
            load_batch<STRIDE, U>(c, base, region, tid * 16, t);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= a[u][0] ^ a[u][1] ^ a[u][2] ^ a[u][3];
            if (++t == trips) {
#pragma unroll
                for (int u = 0; u < U; ++u) acc ^= c[u][0] ^ c[u][1] ^ c[u][2] ^ c[u][3];
                break;
            }
            load_batch<STRIDE, U>(a, base, region, tid * 16, t);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= c[u][0] ^ c[u][1] ^ c[u][2] ^ c[u][3];
            ++t;
        }
    }
    if ((tid & 63) == 0) sh[tid >> 6] = acc;
    __syncthreads();
    if (tid == 0) {
        if ((sh[0] ^ sh[1] ^ sh[2] ^ sh[3]) == 0x9E3779B9u) sink[0] = acc;
        put_block_record(rec, row, t0, c0);
    }
}

// The flat read in one-wave 2 KB blocks; blocks whose index is a multiple of
// `every` leave a record (at index b / every).  A record costs a block about a
// third of its lifetime, so sampling keeps the kernel's own timing.
__global__ __launch_bounds__(64) void read_stream_times_kernel(const char* __restrict__ x, int every,
                                                               uint64_t* __restrict__ rec, uint32_t* __restrict__ sink) {
    const uint64_t t0 = rt_now();
    const uint64_t c0 = clk_now();
    const int64_t b = blockIdx.x;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(x + b * 2048), 0, 2048, 0x00020000);
    const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(r, threadIdx.x * 16, 0, kLoadStreamAux);
    const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(r, (threadIdx.x + 64) * 16, 0, kLoadStreamAux);
    const uint32_t acc = v0[0] ^ v0[1] ^ v0[2] ^ v0[3] ^ v1[0] ^ v1[1] ^ v1[2] ^ v1[3];
    if (acc == 0x9E3779B9u) sink[0] = acc;
    // every lane's loads have landed once its xor is done; the record waits
    // for lane 0's, which retire in order with the wave's others
    if (threadIdx.x == 0 && b % every == 0) {
        put_block_record(rec, b / every, t0, c0);
        rec[6 * (b / every) + 5] = (uint64_t)b;
    }
}

// The IntLSE kernels' phase clock: times of the wave's own phases, recorded
// by the block's first thread.
struct RecClock {
    uint64_t* rec;
    uint64_t t0 = 0, c0 = 0, t1 = 0, t2 = 0, t3 = 0;
    __device__ __forceinline__ void start() {
        t0 = rt_now();
        c0 = clk_now();
    }
    __device__ __forceinline__ void first() { t1 = rt_now(); }
    __device__ __forceinline__ void chain_end() { t2 = rt_now(); }
    __device__ __forceinline__ void tree_end() { t3 = rt_now(); }
    __device__ __forceinline__ void done(int64_t row) {
        if (threadIdx.x == 0) {
            const uint64_t t4 = rt_now();
            const uint64_t c1 = clk_now();
            uint64_t* r = rec + 8 * row;
            r[0] = t0;
            r[1] = t1;
            r[2] = t2;
            r[3] = t3;
            r[4] = t4;
            r[5] = c1 - c0;
            r[6] = xcc_id();
            r[7] = (uint64_t)row;
        }
    }
};

}  // namespace fl

using namespace fl;

extern "C" int fl_diag_chain_latency(int kind, int steps, int waves, uint64_t* rec, void* stream) {
    const char* name = "fl_diag_chain_latency";
    FL_CHECK(kind >= 0 && kind <= 9, "%s: kind must be 0..9", name);
    FL_CHECK(steps > 0 && steps % 16 == 0, "%s: steps must be a positive multiple of 16", name);
    FL_CHECK(waves >= 1 && waves <= 16, "%s: waves must be 1..16", name);
    FL_CHECK(rec != nullptr, "%s: rec is NULL", name);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 blk(64 * waves);
    switch (kind) {
    case 0: chain_latency_kernel<0><<<1, blk, 0, st>>>(steps, rec); break;
    case 1: chain_latency_kernel<1><<<1, blk, 0, st>>>(steps, rec); break;
    case 2: chain_latency_kernel<2><<<1, blk, 0, st>>>(steps, rec); break;
    case 3: chain_latency_kernel<3><<<1, blk, 0, st>>>(steps, rec); break;
    case 4: chain_latency_kernel<4><<<1, blk, 0, st>>>(steps, rec); break;
    case 5: chain_latency_kernel<5><<<1, blk, 0, st>>>(steps, rec); break;
    case 6: chain_latency_kernel<6><<<1, blk, 0, st>>>(steps, rec); break;
    case 7: chain_latency_kernel<7><<<1, blk, 0, st>>>(steps, rec); break;
    case 8: chain_latency_kernel<8><<<1, blk, 0, st>>>(steps, rec); break;
    default: chain_latency_kernel<9><<<1, blk, 0, st>>>(steps, rec); break;
    }
    return launch_status(name);
}

extern "C" int fl_diag_read_stream(const void* x, int64_t nbytes, int blocks, int threads, int unroll,
                                   uint32_t* sink, void* stream) {
    const char* name = "fl_diag_read_stream";
    FL_CHECK(nbytes >= 0 && nbytes % 16 == 0, "%s: nbytes must be a non-negative multiple of 16", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0, "%s: x is not 16-byte aligned", name);
    FL_CHECK(blocks > 0 && blocks <= (1 << 20), "%s: blocks out of range", name);
    FL_CHECK(sink != nullptr, "%s: sink is NULL", name);
    if (nbytes == 0) return ok();
    FL_CHECK(x != nullptr, "%s: x is NULL", name);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    FL_CHECK(threads == 64 || threads == 256, "%s: threads must be 64 or 256", name);
    const char* xs = static_cast<const char*>(x);
    if (threads == 64) {
        switch (unroll) {
        case 1: read_stream_kernel<64, 1><<<blocks, 64, 0, st>>>(xs, nbytes, sink); break;
        case 2: read_stream_kernel<64, 2><<<blocks, 64, 0, st>>>(xs, nbytes, sink); break;
        case 4: read_stream_kernel<64, 4><<<blocks, 64, 0, st>>>(xs, nbytes, sink); break;
        case 8: read_stream_kernel<64, 8><<<blocks, 64, 0, st>>>(xs, nbytes, sink); break;
        default: return set_error(FL_EINVAL, "%s: unroll must be 1, 2, 4 or 8", name);
        }
    } else {
        switch (unroll) {
        case 1: read_stream_kernel<256, 1><<<blocks, 256, 0, st>>>(xs, nbytes, sink); break;
        case 2: read_stream_kernel<256, 2><<<blocks, 256, 0, st>>>(xs, nbytes, sink); break;
        case 4: read_stream_kernel<256, 4><<<blocks, 256, 0, st>>>(xs, nbytes, sink); break;
        case 8: read_stream_kernel<256, 8><<<blocks, 256, 0, st>>>(xs, nbytes, sink); break;
        default: return set_error(FL_EINVAL, "%s: unroll must be 1, 2, 4 or 8", name);
        }
    }
    return launch_status(name);
}

extern "C" int fl_diag_copy_stream(const void* x, void* y, int64_t nbytes, int blocks, int threads, int unroll,
                                   void* stream) {
    const char* name = "fl_diag_copy_stream";
    FL_CHECK(nbytes >= 0 && nbytes % 16 == 0, "%s: nbytes must be a non-negative multiple of 16", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0,
             "%s: x and y must be 16-byte aligned", name);
    FL_CHECK(blocks > 0 && blocks <= (1 << 24), "%s: blocks out of range", name);
    if (nbytes == 0) return ok();
    FL_CHECK(x != nullptr && y != nullptr, "%s: x or y is NULL", name);
    FL_CHECK(blocks <= max_grid_blocks(threads), "%s: %d blocks of %d threads exceed one dispatch", name, blocks,
             threads);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const char* xs = static_cast<const char*>(x);
    char* ys = static_cast<char*>(y);
    FL_CHECK(threads == 64 || threads == 256, "%s: threads must be 64 or 256", name);
    FL_CHECK(unroll == 1 || unroll == 2 || unroll == 4, "%s: unroll must be 1, 2 or 4", name);
    if (threads == 64) {
        switch (unroll) {
        case 1: copy_stream_kernel<64, 1><<<blocks, 64, 0, st>>>(xs, ys, nbytes); break;
        case 2: copy_stream_kernel<64, 2><<<blocks, 64, 0, st>>>(xs, ys, nbytes); break;
        default: copy_stream_kernel<64, 4><<<blocks, 64, 0, st>>>(xs, ys, nbytes); break;
        }
    } else {
        switch (unroll) {
        case 1: copy_stream_kernel<256, 1><<<blocks, 256, 0, st>>>(xs, ys, nbytes); break;
        case 2: copy_stream_kernel<256, 2><<<blocks, 256, 0, st>>>(xs, ys, nbytes); break;
        default: copy_stream_kernel<256, 4><<<blocks, 256, 0, st>>>(xs, ys, nbytes); break;
        }
    }
    return launch_status(name);
}

extern "C" int fl_diag_fwd_block_times(const float* x, float* out, int64_t B, int64_t N, uint64_t* rec, void* stream) {
    const char* name = "fl_diag_fwd_block_times";
    FL_CHECK(B >= 1 && B <= ((int64_t)1 << 24) && N >= 4 && N % 4 == 0, "%s: B in [1, 2^24], N a positive multiple of 4",
             name);
    FL_CHECK(x && out && rec, "%s: NULL pointer argument", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0, "%s: x is not 16-byte aligned", name);
    lse_fwd_block_rows<float, true, 256, 2, true, TimedLseOut>
        <<<dim3((unsigned)B), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(x, TimedLseOut{out, rec}, B, N, 0);
    return launch_status(name);
}

extern "C" int fl_diag_read_rows_times(const float* x, int64_t B, int64_t N, uint64_t* rec, uint32_t* sink,
                                       void* stream) {
    const char* name = "fl_diag_read_rows_times";
    FL_CHECK(B >= 1 && B <= ((int64_t)1 << 24) && N >= 4 && N % 4 == 0, "%s: B in [1, 2^24], N a positive multiple of 4",
             name);
    FL_CHECK(x && rec && sink, "%s: NULL pointer argument", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0, "%s: x is not 16-byte aligned", name);
    FL_CHECK(N * 4 < ((int64_t)1 << 31), "%s: rows of 2 GiB or more", name);
    read_rows_kernel<2><<<dim3((unsigned)B), dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>(x, N, rec, sink);
    return launch_status(name);
}

extern "C" int fl_diag_read_stream_times(const void* x, int64_t nbytes, int every, uint64_t* rec, uint32_t* sink,
                                         void* stream) {
    const char* name = "fl_diag_read_stream_times";
    FL_CHECK(nbytes > 0 && nbytes % 2048 == 0 && nbytes <= ((int64_t)1 << 31),
             "%s: nbytes must be a positive multiple of 2048, at most 2^31", name);
    FL_CHECK(every >= 1, "%s: every must be positive", name);
    FL_CHECK(x && rec && sink, "%s: NULL pointer argument", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0, "%s: x is not 16-byte aligned", name);
    read_stream_times_kernel<<<dim3((unsigned)(nbytes / 2048)), dim3(64), 0, reinterpret_cast<hipStream_t>(stream)>>>(
        static_cast<const char*>(x), every, rec, sink);
    return launch_status(name);
}

extern "C" int fl_diag_intlse_phases(int kind, const void* x, float* out, int64_t B, int64_t N, uint64_t* rec,
                                     void* stream) {
    const char* name = "fl_diag_intlse_phases";
    FL_CHECK(kind >= 0 && kind <= 2, "%s: kind must be 0, 1 or 2", name);
    FL_CHECK(B >= 1 && B <= max_grid_blocks(256) && N >= 1, "%s: B in [1, %lld], N >= 1", name,
             (long long)max_grid_blocks(256));
    FL_CHECK(x && out && rec, "%s: NULL pointer argument", name);
    const int64_t esize = kind == 2 ? 2 : 4;
    FL_CHECK((reinterpret_cast<uintptr_t>(x) % esize) == 0, "%s: x is not element-aligned", name);
    FL_CHECK(N * esize < ((int64_t)1 << 31), "%s: rows of 2 GiB or more", name);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 g((unsigned)B);
    const RecClock clk{rec};
    if (kind == 0)
        with_prefetch(B, 16, [&](auto d) {
            intlse_q16_rows<SrcF32, true, d.value, RecClock><<<g, dim3(256), 0, st>>>(static_cast<const float*>(x), out,
                                                                                      nullptr, N, clk);
        });
    else if (kind == 1)
        with_prefetch(B, 16, [&](auto d) {
            intlse_q16_rows<SrcI32, true, d.value, RecClock><<<g, dim3(256), 0, st>>>(static_cast<const int32_t*>(x),
                                                                                      out, nullptr, N, clk);
        });
    else
        with_prefetch(B, 8, [&](auto d) {
            intlse_q10_6_rows<d.value, RecClock><<<g, dim3(256), 0, st>>>(static_cast<const int16_t*>(x), out, nullptr,
                                                                          N, clk);
        });
    return launch_status(name);
}

extern "C" int fl_diag_half_rows_cap(int dtype, const void* x, float* out, int64_t B, int64_t N, int cap,
                                     void* stream) {
    const char* name = "fl_diag_half_rows_cap";
    FL_CHECK(dtype == 0 || dtype == 1, "%s: dtype must be 0 (fp16) or 1 (bf16)", name);
    FL_CHECK(cap >= 0 && cap <= 8, "%s: cap must be in [0, 8]", name);
    FL_CHECK(B >= 1 && B <= max_grid_blocks(256) && N >= 1, "%s: B in [1, %lld], N >= 1", name,
             (long long)max_grid_blocks(256));
    FL_CHECK(x && out, "%s: NULL pointer argument", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 1u) == 0, "%s: x is not element-aligned", name);
    unsigned lds = 0;
    if (cap > 0) {
        int dev = 0, per_cu = 0;
        FL_CHECK(hipGetDevice(&dev) == hipSuccess &&
                     hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) ==
                         hipSuccess &&
                     per_cu > 0,
                 "%s: cannot read the device's LDS per CU", name);
        lds = (unsigned)(per_cu / (cap + 1) + 64);
        FL_CHECK(lds <= 65536, "%s: cap %d needs %u bytes of LDS per block", name, cap, lds);
    }
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == 0)
        lse_fwd_block_rows<_Float16, false, 256, 4, true, LseOut><<<dim3((unsigned)B), dim3(256), lds, st>>>(
            static_cast<const _Float16*>(x), LseOut{out}, B, N, 0);
    else
        lse_fwd_block_rows<bf16_t, false, 256, 4, true, LseOut><<<dim3((unsigned)B), dim3(256), lds, st>>>(
            static_cast<const bf16_t*>(x), LseOut{out}, B, N, 0);
    return launch_status(name);
}

namespace {
// one wave: lane l holds v[l]; out[l] = max_pair16(v)[l], out[64 + l] =
// max_pair32(v)[l], out[128 + l] = max_pair32(max_pair16(v))[l]
__global__ __launch_bounds__(64) void lane_pairs_kernel(const float* __restrict__ v, float* __restrict__ out) {
    const int l = threadIdx.x;
    const float x = v[l];
    out[l] = max_pair16(x);
    out[64 + l] = max_pair32(x);
    out[128 + l] = max_pair32(max_pair16(x));
}
}  // namespace

extern "C" int fl_diag_lane_pairs(const float* v, float* out, void* stream) {
    const char* name = "fl_diag_lane_pairs";
    FL_CHECK(v && out, "%s: NULL pointer argument", name);
    lane_pairs_kernel<<<dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream)>>>(v, out);
    return launch_status(name);
}

namespace {
// One wave per (group of 8 * 64 / L destination rows, 4 * L-column tile), W
// consecutive tiles of one row group per workgroup (wave w of workgroup cg
// takes tile W * cg + w), workgroup ids dealt to the XCDs in contiguous
// ranges: lane l copies columns 4 * L * ct + 4 * (l % L) .. + 3 of rows
// (8 * 64 / L) * g + (64 / L) * ks + l / L, ks < 8, the loads of a tile issued
// before its first store.  With L = 16 this is the block-layout forward's
// access pattern (child rows gathered by id, 16 bytes per lane, four rows of
// 256 bytes per load, one block's 32 outputs per wave; W = 4 as the library
// launches it) with no arithmetic; L = 32 and 64 read the same bytes as two
// rows of 512 or one row of 1024 bytes per load.
template <int L, int W, int POL>
__global__ __launch_bounds__(64 * W) void gather_rows_kernel(const float* __restrict__ src,
                                                             const int64_t* __restrict__ idx, float* __restrict__ dst,
                                                             int64_t nrows, int64_t batch, int64_t ctiles,
                                                             int64_t items, int64_t id0) {
    constexpr int RI = 64 / L;  // rows per load
    const int64_t per_xcd = gridDim.x / 8;
    const int64_t id = id0 + (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (id >= items) return;
    const int64_t cgroups = (ctiles + W - 1) / W;
    const int64_t ct = id % cgroups * W + (int64_t)(threadIdx.x >> 6);
    if (ct >= ctiles) return;
    const int64_t g = id / cgroups;
    const int l = lane_id();
    const int64_t col = ct * 4 * L + 4 * (l % L);
    const bool cv = col < batch;
    f32x4 v[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        const int64_t i = g * 8 * RI + RI * ks + l / L;
        const int64_t row = idx[i < nrows ? i : nrows - 1];
        const float* p = src + row * batch + (cv ? col : 0);
        v[ks] = (POL & 1) ? load_stream<f32x4>(p) : *reinterpret_cast<const f32x4*>(p);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the wave's destination rows as one buffer resource (stores written
    // through to memory, sc1 nt: POL & 4)
    const int64_t r0 = g * 8 * RI;
    const int64_t rn = nrows - r0 < 8 * RI ? nrows - r0 : 8 * RI;
    const __amdgpu_buffer_rsrc_t rd =
        __builtin_amdgcn_make_buffer_rsrc(dst + r0 * batch, 0, (int)(rn * batch * 4), 0x00020000);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        const int64_t i = g * 8 * RI + RI * ks + l / L;
        if (i < nrows && cv) {
            if constexpr (POL & 4)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[ks]), rd,
                                                       (int)(((i - r0) * batch + col) * 4), 0, kStoreStreamAux);
            else if constexpr (POL & 2)
                store_stream(v[ks], dst + i * batch + col);
            else
                *reinterpret_cast<f32x4*>(dst + i * batch + col) = v[ks];
        }
    }
}

template <int L, int W, int POL>
void launch_gather_rows(const float* src, const int64_t* idx, float* dst, int64_t nrows, int64_t batch,
                        hipStream_t st) {
    const int64_t ctiles = (batch + 4 * L - 1) / (4 * L);
    const int64_t items = (nrows + 8 * 64 / L - 1) / (8 * 64 / L) * ((ctiles + W - 1) / W);
    constexpr int64_t kMax = max_grid_blocks(64 * W);
    for (int64_t id0 = 0; id0 < items; id0 += kMax) {
        const int64_t n = items - id0 < kMax ? items - id0 : kMax;
        gather_rows_kernel<L, W, POL><<<dim3((unsigned)((n + 7) / 8 * 8)), dim3(64 * W), 0, st>>>(
            src, idx, dst, nrows, batch, ctiles, items, id0);
    }
}

template <int W, int POL>
void launch_gather_lanes(const float* src, const int64_t* idx, float* dst, int64_t nrows, int64_t batch, int lanes,
                         hipStream_t st) {
    if (lanes == 16) launch_gather_rows<16, W, POL>(src, idx, dst, nrows, batch, st);
    else if (lanes == 32) launch_gather_rows<32, W, POL>(src, idx, dst, nrows, batch, st);
    else launch_gather_rows<64, W, POL>(src, idx, dst, nrows, batch, st);
}

template <int POL>
void launch_gather_pol(const float* src, const int64_t* idx, float* dst, int64_t nrows, int64_t batch, int lanes,
                       int waves, hipStream_t st) {
    if (waves == 4) launch_gather_lanes<4, POL>(src, idx, dst, nrows, batch, lanes, st);
    else launch_gather_lanes<1, POL>(src, idx, dst, nrows, batch, lanes, st);
}
}  // namespace

extern "C" int fl_diag_gather_rows(const float* src, const int64_t* idx, float* dst, int64_t nrows, int64_t batch,
                                   int lanes_per_row, int waves, int policy, void* stream) {
    const char* name = "fl_diag_gather_rows";
    FL_CHECK(nrows >= 0 && batch >= 0, "%s: negative size", name);
    FL_CHECK(lanes_per_row == 16 || lanes_per_row == 32 || lanes_per_row == 64, "%s: lanes_per_row must be 16, 32 or 64",
             name);
    if (nrows == 0 || batch == 0) return ok();
    FL_CHECK(src && idx && dst, "%s: NULL pointer argument", name);
    FL_CHECK(batch % 4 == 0 && ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0,
             "%s: rows must be 16-byte vectors (batch %% 4 == 0, 16-byte aligned buffers)", name);
    FL_CHECK(waves == 1 || waves == 4, "%s: waves must be 1 or 4", name);
    FL_CHECK(policy >= 0 && policy <= 5 && policy != 3, "%s: policy must be 0, 1, 2, 4 or 5", name);
    FL_CHECK(batch <= ((int64_t)1 << 31) / (4 * 8 * 64), "%s: batch too large for the destination resource", name);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (policy) {
        case 0: launch_gather_pol<0>(src, idx, dst, nrows, batch, lanes_per_row, waves, st); break;
        case 1: launch_gather_pol<1>(src, idx, dst, nrows, batch, lanes_per_row, waves, st); break;
        case 2: launch_gather_pol<2>(src, idx, dst, nrows, batch, lanes_per_row, waves, st); break;
        case 4: launch_gather_pol<4>(src, idx, dst, nrows, batch, lanes_per_row, waves, st); break;
        default: launch_gather_pol<5>(src, idx, dst, nrows, batch, lanes_per_row, waves, st); break;
    }
    return launch_status(name);
}

namespace {
// The memory pattern of the block-layout backward's single pass at 32
// parents and 32 edges (one edge chunk), with its arithmetic reduced to one
// product and sum per column: wave w of a workgroup (one workgroup per node
// block j) takes the 64-column tiles w, w + W, ...; per tile, lane
// (kq = l / 16, jc = l % 16) loads columns b0 + 4 jc .. + 3 of the gathered
// child rows cids[j, 16 et + 4 kq + r] (et < 2, r < 4) with plain loads and
// of the parent rows nids[j] + 4 ks + kq (ks < 8) of o and g with the
// nontemporal hint, all issued before the first use, and stores with the
// nontemporal hint
//   F[32 j + e, b] = x[cids[j, e], b] + sum_ks o[n, b] g[n, b],
//   n = nids[j] + 4 ks + (e / 4) % 4,
// the single pass's loads and edge-flow stores in the same order.  Dynamic
// LDS (lds_per_wave bytes per wave) sets the occupancy the single pass has.
template <int W>
__global__ __launch_bounds__(64 * W) void bwd_pattern_kernel(float* __restrict__ F, const float* __restrict__ g,
                                                             const float* __restrict__ o, const float* __restrict__ x,
                                                             const int64_t* __restrict__ nids,
                                                             const int64_t* __restrict__ cids, int64_t batch,
                                                             int64_t block0) {
    const int64_t j = block0 + blockIdx.x;
    const int w = threadIdx.x >> 6;
    const int l = lane_id(), kq = l >> 4, jc = l & 15;
    const int64_t nrow0 = nids[j];
    int64_t xr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xr[i] = cids[j * 32 + 16 * (i >> 2) + 4 * kq + (i & 3)];
    for (int64_t b0 = 64 * w; b0 < batch; b0 += 64 * W) {
        const int64_t col = b0 + 4 * jc;
        f32x4 xv[8], ov[8], gv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = *reinterpret_cast<const f32x4*>(x + xr[i] * batch + col);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int64_t n = nrow0 + 4 * ks + kq;
            ov[ks] = load_stream<f32x4>(o + n * batch + col);
            gv[ks] = load_stream<f32x4>(g + n * batch + col);
        }
        __builtin_amdgcn_sched_barrier(0);
        f32x4 sum = ov[0] * gv[0];
#pragma unroll
        for (int ks = 1; ks < 8; ++ks) sum += ov[ks] * gv[ks];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            store_stream(xv[i] + sum, F + (j * 32 + 16 * (i >> 2) + 4 * kq + (i & 3)) * batch + col);
    }
}
}  // namespace

extern "C" int fl_diag_blocked_bwd_pattern(float* F, const float* g, const float* o, const float* x,
                                           const int64_t* nids, const int64_t* cids, int64_t nblocks,
                                           int64_t batch, int waves, int lds_per_wave, void* stream) {
    const char* name = "fl_diag_blocked_bwd_pattern";
    FL_CHECK(nblocks >= 0 && batch >= 0, "%s: negative size", name);
    if (nblocks == 0 || batch == 0) return ok();
    FL_CHECK(F && g && o && x && nids && cids, "%s: NULL pointer argument", name);
    FL_CHECK(batch % 64 == 0 && ((reinterpret_cast<uintptr_t>(F) | reinterpret_cast<uintptr_t>(g) |
                                  reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(x)) & 15) == 0,
             "%s: batch must be a multiple of 64 and the buffers 16-byte aligned", name);
    FL_CHECK(waves == 1 || waves == 2 || waves == 4, "%s: waves must be 1, 2 or 4", name);
    FL_CHECK(lds_per_wave >= 0 && lds_per_wave <= 40960, "%s: lds_per_wave must be in [0, 40960]", name);
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const size_t lds = (size_t)lds_per_wave * waves;
    constexpr int64_t kMax = max_grid_blocks(256);
    for (int64_t b0 = 0; b0 < nblocks; b0 += kMax) {
        const unsigned n = (unsigned)(nblocks - b0 < kMax ? nblocks - b0 : kMax);
        if (waves == 1)
            bwd_pattern_kernel<1><<<dim3(n), dim3(64), lds, st>>>(F, g, o, x, nids, cids, batch, b0);
        else if (waves == 2)
            bwd_pattern_kernel<2><<<dim3(n), dim3(128), lds, st>>>(F, g, o, x, nids, cids, batch, b0);
        else
            bwd_pattern_kernel<4><<<dim3(n), dim3(256), lds, st>>>(F, g, o, x, nids, cids, batch, b0);
    }
    return launch_status(name);
}
