// byhip_gemm.h - host-side launchers of the MFMA GEMM kernels (internal to libbybyhip.so).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <utility>

#include "byhip_kernels.h"

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
    const uint8_t* wpf = nullptr;  // the prefill copy of the nibbles and its scales
    const void* spf = nullptr;     // (byhip_q4w::wpf, spf), or null
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
    // Device scratch the launches may use (split-K partials, per-row activation exponents), in
    // stream order: null means the library workspace (kWorkspaceBytes, allocated at init).
    void* work = nullptr;
    size_t work_bytes = 0;
    // Set by the fp32-activation launch of the fp16 MFMA kernel: per-row exponents t (x * 2^t is
    // split into fp16 hi + lo; the row's sums are scaled by 2^-t).
    const int* row_shift = nullptr;
    // The wide tile on fp32 activations: x holds the high fp16 plane of the shifted activations and
    // x_lo the low one (x * 2^t = hi + lo, t per row in row_shift).
    const void* x_lo = nullptr;
    // A device-side route choice: when gate is set, the general fp16 MFMA GEMM, the exact GEMM and
    // their split-K sum do nothing unless *gate == gate_want (the flag a classification kernel
    // earlier on the stream wrote), so two routes can be queued and only the chosen one runs.
    const int* gate = nullptr;
    int gate_want = 0;
};

// Whether 8-output chunks may leave as 16-byte stores: every row of y (or of the split-K
// partials) starts 16-byte aligned.
template <int YT>
__device__ __forceinline__ bool out8_vector_ok(const GemmArgs& a, const float* part) {
    constexpr int es = YT == BYHIP_F32 ? 4 : 2;
    return part ? a.N % 4 == 0 : ((uintptr_t)a.y % 16 == 0 && (size_t)a.N * es % 16 == 0);
}

// Outputs v[0..7] of row m, columns n .. n + 7, to y (or to the split-K partials `part`): one
// 16-byte store (fp16 / bf16) or two (fp32) when `vec` and all 8 columns exist, else one store per
// column inside N.
template <int YT>
__device__ __forceinline__ void store_out8(const GemmArgs& a, float* part, bool vec, int m, int n, const float (&v)[8]) {
    if (vec && n + 8 <= a.N) {
        if (part || YT == BYHIP_F32) {
            float* dst = part ? part + (size_t)m * a.N + n : static_cast<float*>(a.y) + (size_t)m * a.N + n;
            reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
        } else {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (YT == BYHIP_F16)
                    w[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * e]) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * e + 1]) << 16);
                else
                    w[e] = f32x2_to_bf16x2_bits(v[2 * e], v[2 * e + 1]);
            }
            *reinterpret_cast<uint4*>(static_cast<uint8_t*>(a.y) + ((size_t)m * a.N + n) * 2) =
                make_uint4(w[0], w[1], w[2], w[3]);
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (n + e >= a.N) break;
        if (part) part[(size_t)m * a.N + n + e] = v[e];
        else store_y<YT>(a.y, (size_t)m * a.N + n + e, v[e]);
    }
}

// LDS slot swizzle of the activation slices (rows of 128 bytes, eight 16-byte chunks): chunk k of
// row r sits at slot k ^ x_swizzle(r), row bits 2, 1, 3 giving slot bits 0, 1, 2. With the fragment
// reads (lane (c, g) reads chunk 2 g + kk of row 16 i + c, 16 bytes) this layout measured free of
// LDS bank conflicts on the MI355X (a standalone probe of that read pattern with the hardware's
// conflict counter): 2.3-2.5 ns per wave-wide read per CU, as fast as contiguous reads, against
// 3.7-4.0 ns and 4 conflict cycles per read with the slot k ^ (r / 2 % 8) used before.
__host__ __device__ constexpr int x_swizzle(int r) {
    return ((r >> 2) & 1) | (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
}

// Calls f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>) in order.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Floats between consecutive split-K partials (16-byte aligned).
__host__ __device__ __forceinline__ size_t splitk_stride(int M, int N) { return ((size_t)M * N + 3) & ~(size_t)3; }
// Split-K for a grid of `tiles` blocks over `nsteps` K steps: when the tiles leave CUs idle, K is
// split so that the grid holds about `per_cu` blocks per CU, each split keeping at least
// `min_steps` steps; the partials must fit the scratch (a.work, or the workspace). BYHIP_Q4_SPLIT
// forces the number of splits, as does `forced` > 0. Sets a.part / a.split_steps and returns the
// number of splits (1: none).
int choose_split(GemmArgs& a, long tiles, int nsteps, int min_steps, int forced, int per_cu = 2);
// y = the sum of the split-K partials in slice order.
void launch_splitk_sum(const GemmArgs& a, int splits);

// Queues the GEMM on the library stream; K % 32 == 0 is required (callers check). fp16 MFMA: the
// weights are rounded once to fp16 (exact for F16 weights and for FP4-KM tables whose products
// are halves; Q4 rounds (q - z) * s).
void launch_gemm(BFormat fmt, const GemmArgs& a);
// Whether launch_gemm(Q4Fast, a) takes a call with fp32 activations on the wide tile over two fp16
// activation planes (the prefill copy's format conditions, and BYHIP_Q4_F32_WIDE not 0).
bool q4_f32_wide_takes(const GemmArgs& a);
// Whether launch_gemm(Q4Fast, a) takes the small-M streaming GEMM (fp16 activations, M up to 32 or
// BYHIP_Q4_SKINNY_MAX_M, the prefill copy; BYHIP_Q4_STREAM=0 switches it off).
bool q4_stream_takes(const GemmArgs& a);
// Queues the 16- or 32-row wide tile on fp16 activations with each Q4 weight as two fp16 terms that
// add up to it exactly (the weights' prefill copy, M <= 32); false, queueing nothing, when it does
// not take the call.
bool launch_q4_wide_exact_weights(const GemmArgs& a);

// The exact route: each weight formed in fp32 exactly as the reference forms it (Q4
// ((float)q - z) * s with any scales, zeros and group size; FP4-KM lut[nibble] * lut[16 + byte];
// F16 halves), fp32 activations as they are (fp16 widened), fp32 products and accumulation in
// v_mfma_f32_16x16x4_f32. Any K (Q4; FP4-KM and F16 need K % 32 == 0), M, N.
void launch_gemm_exact(BFormat fmt, const GemmArgs& a);

// The Q4 GEMM kernels by explicit choice (a tuned plan's candidates): kQ4Pipe, the LDS-staged
// pipelined kernel with `tile` 1..4 (64x128, 64x64, 32x128, 32x64) and `splits`; kQ4Skinny (M <= 32,
// `splits`); kQ4General, the general LDS-staged kernel; kQ4Big, the 128 x 256 prefill tile, and
// kQ4Wide, the 64 x 128 skinny tile (`splits`); kQ4Stream, the small-M streaming GEMM (`splits`).
// tile / splits 0 keep the default choice.
// Returns false, queueing nothing, when that kernel does not take the call.
enum { kQ4Pipe = 1, kQ4Skinny = 2, kQ4General = 3, kQ4Big = 4, kQ4Wide = 5, kQ4Stream = 6 };
bool launch_q4_choice(BFormat fmt, const GemmArgs& a, int kind, int tile, int splits);

// The small-M streaming Q4 GEMM (q4_gemm_stream): up to 32 rows of fp16 activations on weights
// with the prefill copy, one block per CU owning a strip of columns over all of K. q4_stream_ok
// says whether it takes the call; launch_q4_stream splits K only when `split_choice` (or
// BYHIP_Q4_SPLIT) asks for it.
bool q4_stream_ok(const GemmArgs& a);
// Column fragments per block of the streaming GEMM for this call with `row_blocks` blocks per
// strip, and the row blocks it launches (2 for 17 to 32 rows unless BYHIP_Q4_STREAM_HALVES=0).
int stream_fn(const GemmArgs& a, int row_blocks);
int stream_row_blocks(const GemmArgs& a);
void launch_q4_stream(const GemmArgs& a, int split_choice = 0);

// Native MXFP4 GEMM (E2M1 x E2M1 with E8M0 block scales): x and w in the FP4-KM packing.
// K % 128 == 0 is required.
void launch_mxfp4(const uint8_t* x, const uint8_t* x_scales, const uint8_t* w,
                  const uint8_t* w_scales, void* y, int y_dtype, int M, int K, int N);

}  // namespace byhip
