// RMSNorm entry points used inside the library.
#pragma once

#include "common.hpp"

namespace glt {

// RMSNorm backward (glt_rmsnorm_bwd's result, bit for bit) on a persistent
// grid of `grid` workgroups, one per CU, for a caller that runs it beside
// another kernel. Eligible when rmsnorm_bwd_rows_ok holds (rows of at most
// 4096 elements, a multiple of 8, 16-byte aligned buffers).
bool rmsnorm_bwd_rows_ok(const float* dy, const uint16_t* x, const uint16_t* w, const float* dx, int M, int D);
glt_status rmsnorm_bwd_rows(const float* dy, const uint16_t* x, const uint16_t* w, const float* var, float* dx, int M,
                            int D, float eps, int grid, hipStream_t st);

}  // namespace glt
