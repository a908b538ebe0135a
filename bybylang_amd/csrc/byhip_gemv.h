// byhip_gemv.h - the Q4 decode GEMV launcher (internal to libbybyhip.so).
#pragma once

#include "byhip_internal.h"

namespace byhip {

// Whether the GEMV takes these weights for M rows of activations of x_dtype (K and the group a
// multiple of 32, activations fitting the per-lane register tile, 32-bit buffer offsets).
bool q4_gemv_eligible(const byhip_q4w* w, int M, int x_dtype);
// Queues y[M, N] = x[M, K] . W^T (M <= 8 runs as launches of up to 4 activation rows).
void launch_q4_gemv(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M);

}  // namespace byhip
