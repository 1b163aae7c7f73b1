// The matrix-core form of the pyjuice block-layout fp32 sum layer
// (lse_blocked.hip), called by fl_sparse_blocked_fwd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fl {
namespace sparse {

// Smallest block_size that takes the product form.  Measured at batch 512,
// 32 edges per block: block_size 2, 1528 -> 823 us; 4, 1567 -> 422 us against
// the per-parent gather.  block_size 1 keeps the per-parent kernel.
constexpr int64_t kBlockedMfmaMinBs = 2;

bool blocked_mfma_eligible(int64_t num_edges, int64_t block_size);

void launch_blocked_mfma(float* node_mars, const float* element_mars, const float* params, const int64_t* nids,
                         const int64_t* cids, const int64_t* pids, int64_t num_nblocks, int64_t num_edges,
                         int64_t block_size, int64_t batch, bool params_are_log, hipStream_t st);

}  // namespace sparse
}  // namespace fl
