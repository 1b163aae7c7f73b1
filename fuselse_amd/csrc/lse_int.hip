// IntLSE fixed-point launchers for gfx950: Q16.16 (fp32 input quantised in the
// kernel, or pre-quantised int32 input) and Q10.6 (int16 input).  The kernels
// and the reduction tree they follow are in lse_int_kernels.hpp.
#include <stdint.h>

#include <type_traits>

#include "../../include/fuselse_amd.h"
#include "fl_status.hpp"
#include "lse_int_kernels.hpp"

namespace fl {

// Calls launch(grid, x, out, acc) for consecutive chunks of rows (one block
// per row), each within one dispatch for blocks of up to 256 threads.
template <typename T, typename LAUNCH>
static void for_row_chunks(const T* x, float* out, int32_t* acc, int64_t B, int64_t N, LAUNCH launch) {
    for_grid_chunks(B, 256, [&](int64_t r0, int64_t rows) {
        launch(dim3((unsigned)rows), x + r0 * N, out + r0, acc ? acc + r0 : nullptr);
    });
}

template <typename T>
static int int_entry_check(const char* name, const T* x, float* out, int64_t B, int64_t N) {
    FL_CHECK(B >= 0 && N >= 0, "%s: negative shape (B=%lld, N=%lld)", name, (long long)B, (long long)N);
    if (B == 0) return ok();
    FL_CHECK(out != nullptr, "%s: out is NULL", name);
    FL_CHECK(x != nullptr || N == 0, "%s: x is NULL", name);
    FL_CHECK((reinterpret_cast<uintptr_t>(x) % sizeof(T)) == 0, "%s: x is not element-aligned", name);
    if (N * (int64_t)sizeof(T) >= ((int64_t)1 << 31))
        return set_error(FL_ERANGE, "%s: rows of %lld elements exceed the 2 GiB buffer range", name, (long long)N);
    return ok();
}

}  // namespace fl

using namespace fl;

extern "C" int fl_intlse_q16_f32(const float* x, float* out, int32_t* acc_out, int64_t B, int64_t N, int use_lut,
                                 void* stream) {
    const char* name = "fl_intlse_q16_f32";
    if (int rc = int_entry_check(name, x, out, B, N)) return rc;
    if (B == 0) return ok();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for_row_chunks(x, out, acc_out, B, N, [&](dim3 g, const float* xc, float* oc, int32_t* ac) {
        with_prefetch(g.x, 16, [&](auto d) {
            if (use_lut)
                intlse_q16_rows<SrcF32, true, d.value><<<g, dim3(256), 0, st>>>(xc, oc, ac, N);
            else
                intlse_q16_rows<SrcF32, false, d.value><<<g, dim3(256), 0, st>>>(xc, oc, ac, N);
        });
    });
    return launch_status(name);
}

extern "C" int fl_intlse_q16_i32(const int32_t* q, float* out, int32_t* acc_out, int64_t B, int64_t N, int use_lut,
                                 void* stream) {
    const char* name = "fl_intlse_q16_i32";
    if (int rc = int_entry_check(name, q, out, B, N)) return rc;
    if (B == 0) return ok();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for_row_chunks(q, out, acc_out, B, N, [&](dim3 g, const int32_t* qc, float* oc, int32_t* ac) {
        with_prefetch(g.x, 16, [&](auto d) {
            if (use_lut)
                intlse_q16_rows<SrcI32, true, d.value><<<g, dim3(256), 0, st>>>(qc, oc, ac, N);
            else
                intlse_q16_rows<SrcI32, false, d.value><<<g, dim3(256), 0, st>>>(qc, oc, ac, N);
        });
    });
    return launch_status(name);
}

extern "C" int fl_intlse_q10_6(const int16_t* q, float* out, int32_t* acc_out, int64_t B, int64_t N, void* stream) {
    const char* name = "fl_intlse_q10_6";
    if (int rc = int_entry_check(name, q, out, B, N)) return rc;
    if (B == 0) return ok();
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool paired = (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && N % 8 == 0 && N > 0 && N <= 32768 && B >= 2048;
    for_row_chunks(q, out, acc_out, B, N, [&](dim3 g, const int16_t* qc, float* oc, int32_t* ac) {
        if (paired)
            intlse_q10_6_rows_paired<kQ10PairedAhead><<<g, dim3(128), 0, st>>>(qc, oc, ac, N);
        else
            with_prefetch(g.x, 8, [&](auto d) { intlse_q10_6_rows<d.value><<<g, dim3(256), 0, st>>>(qc, oc, ac, N); });
    });
    return launch_status(name);
}
