// byhip_gemm.h - host-side launchers of the MFMA GEMM kernels (internal to libbybyhip.so).
#pragma once

#include <cstddef>
#include <cstdint>

namespace byhip {

// Weight formats of the LDS-staged fp16 MFMA GEMM (y[M, N] = x[M, K] . W^T, fp32 accumulation).
enum class BFormat {
    Q4Fast,     // Q4 nibbles, integer zero points, fp16 scales: (q - z) * s rounded once to fp16
    Q4Generic,  // Q4 nibbles, any zeros / scales / group: ((float)q - z) * s rounded to fp16
    Fp4Km,      // FP4-KM nibbles + scale bytes + 272-float decode table
    F16         // IEEE halves [N, K]
};

struct GemmArgs {
    const void* x = nullptr;  // [M, K], x_dtype BYHIP_F32 (split into two fp16 terms) or BYHIP_F16
    int x_dtype = 0;
    void* y = nullptr;        // [M, N], y_dtype
    int y_dtype = 0;
    int M = 0, K = 0, N = 0;
    // Q4
    const uint8_t* wq = nullptr;
    size_t row_bytes = 0;
    const void* scales = nullptr;
    int scale_f16 = 0;
    const float* zeros = nullptr;  // null: zero_value for every group
    float zero_value = 0.0f;
    int group = 0;                 // 0: one group per row
    int gpr = 0;
    const void* sblk = nullptr;    // fp16 scales per 32-value chunk in blocks of 8 columns,
                                   // [ceil(N/8)][K/32][8] (byhip_q4w::sblk), or null
    // FP4-KM
    const uint8_t* blob = nullptr;
    size_t scale_base = 0;
    const float* lut = nullptr;    // the 272 floats (16 values, 256 scales)
    // F16
    const uint16_t* w16 = nullptr;
    // Split-K (set by the launcher): block z of the grid covers K steps [z * split_steps, ...) and
    // writes fp32 partial sums to part[z][M][N]; a second kernel adds them in z order into y.
    float* part = nullptr;
    int split_steps = 0;
};

// Queues the GEMM on the library stream; K % 32 == 0 is required (callers check).
void launch_gemm(BFormat fmt, const GemmArgs& a);

// The Q4 GEMM kernels by explicit choice (a tuned plan's candidates): kQ4Pipe, the LDS-staged
// pipelined kernel with `tile` 1..4 (64x128, 64x64, 32x128, 32x64) and `splits`; kQ4Skinny (M <= 32,
// `splits`); kQ4General, the general LDS-staged kernel; kQ4Big, the 128 x 256 prefill tile, and
// kQ4Wide, the 64 x 128 skinny tile (`splits`). tile / splits 0 keep the default choice.
// Returns false, queueing nothing, when that kernel does not take the call.
enum { kQ4Pipe = 1, kQ4Skinny = 2, kQ4General = 3, kQ4Big = 4, kQ4Wide = 5 };
bool launch_q4_choice(BFormat fmt, const GemmArgs& a, int kind, int tile, int splits);

// Native MXFP4 GEMM (E2M1 x E2M1 with E8M0 block scales): x and w in the FP4-KM packing.
// K % 128 == 0 is required.
void launch_mxfp4(const uint8_t* x, const uint8_t* x_scales, const uint8_t* w,
                  const uint8_t* w_scales, void* y, int y_dtype, int M, int K, int N);

}  // namespace byhip
