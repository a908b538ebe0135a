// byhip_gemv.h - the Q4 decode GEMV launcher (internal to libbybyhip.so).
#pragma once

#include "byhip_internal.h"

namespace byhip {

// Whether the GEMV takes these weights for M rows of activations of x_dtype (K and the group a
// multiple of 32, 32-bit buffer offsets, and, when K is cut into slices, their fp32 partial sums
// within `work_bytes` of scratch).
bool q4_gemv_eligible(const byhip_q4w* w, int M, int x_dtype, size_t work_bytes = kWorkspaceBytes);
// Activation rows one GEMV launch takes (at most 4; 0: not even one row fits).
int gemv_rows_per_launch(int K, int M, int x_dtype);
// Queues y[M, N] = x[M, K] . W^T (M <= 8 runs as launches of up to 4 activation rows). K of any
// multiple of 32: rows longer than one launch's register tile or staging run in K slices whose
// fp32 partial sums go to `work` (null: the library workspace) and are added in slice order.
void launch_q4_gemv(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M,
                    void* work = nullptr, size_t work_bytes = 0);

// The fused decode GEMV of sessionMatmulQ4Fused: BYHIP_OK when the kernel takes these weights for
// this mode (1..3 weights for mode 0, gate and up of equal N for mode 1, equal K / group / groups
// per row and scale formats, the decode layout present), else BYHIP_UNSUPPORTED.
int q4_fused_check(int mode, const byhip_q4w* const* ws, int n_ws);
// Queues it (fp32 input, outputs, residual and norm weights; res / gamma null when absent).
void launch_q4_gemv_fused(int mode, const float* x, const byhip_q4w* const* ws, int n_ws, float* const* outs,
                          const float* res, const float* gamma, float eps);

}  // namespace byhip
