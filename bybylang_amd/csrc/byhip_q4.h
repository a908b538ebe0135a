// byhip_q4.h - Q4 kernel choice shared by the router and the tuner (internal to libbybyhip.so).
#pragma once

#include "byhip_internal.h"

namespace byhip {

// A choice of Q4 kernel for one call shape: what byhip_q4_prepare stores and byhip_q4_matmul
// follows. tile / splits pick the MFMA GEMM's tile (1..4) and split-K (0: the default choice).
enum Q4PlanKind : int {
    kPlanGeneric = 1,  // the exact per-element kernel (the tuner's parity baseline)
    kPlanGemv = 2,     // the decode GEMV
    kPlanPipe = 3,     // the LDS-staged pipelined MFMA GEMM (benchmark format)
    kPlanSkinny = 4,   // the skinny MFMA GEMM (M <= 32)
    kPlanGemm = 5,     // the general LDS-staged MFMA GEMM
    kPlanBig = 6,      // the 128 x 256 prefill tile
    kPlanWide = 7,     // the wide tile (128 columns; 16, 32 or 64 rows)
    kPlanExact = 8,    // the exact fp32 MFMA GEMM
    kPlanStream = 9,   // the small-M streaming GEMM (M <= 32, one column strip per CU over all of K)
    kPlanLast = kPlanStream
};
struct Q4Plan {
    int kind = 0;
    int tile = 0;
    int splits = 0;
};

// Queues y = x . W^T with the kernel the plan names; false, queueing nothing, when that kernel
// does not take this call (the arguments were validated by the caller).
bool q4_run_plan(const Q4Plan& p, const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M);
// byhip_q4_matmul's routing with the kernels' scratch (split-K partials, per-row activation shifts)
// in `work` (work_bytes) instead of the library workspace; tuned plans are not consulted.
void q4_matmul_run_scratch(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, void* work,
                           size_t work_bytes);
// The plan byhip_q4_prepare chose for these weights, this M's class and activation dtype, if any.
bool q4_lookup_plan(const byhip_q4w* w, int M, int x_dtype, Q4Plan* out);

}  // namespace byhip
