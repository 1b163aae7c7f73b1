// Read-bandwidth reference for the measurements (no counterpart in the
// reference): streams a buffer from HBM with the forward kernels' load form
// (16-byte buffer loads with the nontemporal hint) in a flat grid-stride
// order, and does nothing else with the data.  Its rate over the forward's own
// input buffers, in the same run, is the read ceiling the forward is held
// against.
#include <stdint.h>

#include "../../include/fuselse_amd.h"
#include "fl_status.hpp"
#include "lse_common.hpp"

namespace fl {

// Block b reads chunks b, b + gridDim.x, ... of 256 * U * 16 bytes; lane t of
// the block reads bytes t * 16 + u * 4096 of a chunk (u < U), so each group of
// U loads is issued back to back and every wave's loads are fully coalesced.
// The xor of the words feeds a store that happens only when it equals a
// constant no realistic input produces, which keeps the loads live.
template <int U>
__global__ __launch_bounds__(256) void read_stream_kernel(const char* __restrict__ x, int64_t nbytes,
                                                          uint32_t* __restrict__ sink) {
    constexpr int64_t CHUNK = 256 * U * 16;
    const int tid = threadIdx.x;
    uint32_t acc = 0;
    for (int64_t c = blockIdx.x; c * CHUNK < nbytes; c += gridDim.x) {
        const int64_t left = nbytes - c * CHUNK;
        const int nrec = left > CHUNK ? (int)CHUNK : (int)left;
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(x + c * CHUNK), 0, nrec, 0x00020000);
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, tid * 16 + u * 4096, 0, kLoadStreamAux);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace fl

using namespace fl;

extern "C" int fl_diag_read_stream(const void* x, int64_t nbytes, int blocks, int unroll, uint32_t* sink,
                                   void* stream) {
    const char* name = "fl_diag_read_stream";
    FL_CHECK(nbytes >= 0 && nbytes % 16 == 0, "%s: nbytes must be a non-negative multiple of 16", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) & 15u) == 0, "%s: x is not 16-byte aligned", name);
    FL_CHECK(blocks > 0 && blocks <= (1 << 20), "%s: blocks out of range", name);
    FL_CHECK(sink != nullptr, "%s: sink is NULL", name);
    if (nbytes == 0) return ok();
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    switch (unroll) {
    case 1: read_stream_kernel<1><<<blocks, 256, 0, st>>>(static_cast<const char*>(x), nbytes, sink); break;
    case 2: read_stream_kernel<2><<<blocks, 256, 0, st>>>(static_cast<const char*>(x), nbytes, sink); break;
    case 4: read_stream_kernel<4><<<blocks, 256, 0, st>>>(static_cast<const char*>(x), nbytes, sink); break;
    case 8: read_stream_kernel<8><<<blocks, 256, 0, st>>>(static_cast<const char*>(x), nbytes, sink); break;
    default: return set_error(FL_EINVAL, "%s: unroll must be 1, 2, 4 or 8", name);
    }
    return launch_status(name);
}
