// byhip_mxfp4.hip - native MXFP4 GEMM on gfx950's scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// y[M, N] = x[M, K] . W^T with both operands E2M1 (fp4) and one E8M0 scale per 32 values, fp32
// accumulation. Operand layout (checked on the device): lane l holds the 32 values of row (or
// column) l%16, K block l/16 of the 128-deep step as 16 bytes, low nibble first, and its scale in
// byte 0 of the scale register. One FP4-KM group (16 bytes + 1 scale byte, session_vm.nim:384-388)
// is therefore exactly one lane's operand. FP4-KM stores element j and j+16 in byte j rather than
// elements 2j and 2j+1, so the MFMA sees the 32 values of a group in a permuted order; x uses the
// same packing, both operands carry the same permutation, and the dot product is unchanged.
//
// A 256-thread block computes a 128 x 128 tile; each wave owns 64 x 64 (4 x 4 fragments, 16 MFMAs per
// 128-deep step). Operands are staged through LDS: per step 128 rows x 64 bytes for each side plus
// 4 scale bytes per row.
#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

constexpr int TM = 128, TN = 128;
constexpr int KSTEP = 128;           // values per step (4 groups)
constexpr int ROWB = KSTEP / 2;      // 64 bytes of nibbles per row per step
constexpr int LDB = ROWB + 16;       // padded LDS row (bytes)

template <int YT>
__global__ __launch_bounds__(256) void mxfp4_gemm(const uint8_t* __restrict__ x,
                                                  const uint8_t* __restrict__ xs,
                                                  const uint8_t* __restrict__ w,
                                                  const uint8_t* __restrict__ ws,
                                                  void* __restrict__ y, int M, int K, int N) {
    __shared__ __attribute__((aligned(16))) uint8_t As[TM * LDB];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[TN * LDB];
    __shared__ uint32_t Asc[TM];
    __shared__ uint32_t Bsc[TN];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
    const size_t kb = (size_t)K >> 1, kg = (size_t)K >> 5;

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    const int srow = tid >> 1, shalf = tid & 1;  // staging: 32 bytes (2 groups) per thread
    for (int k0 = 0; k0 < K; k0 += KSTEP) {
        {
            const int m = m0 + srow;
            uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
            if (m < M) {
                const uint4* p = reinterpret_cast<const uint4*>(x + (size_t)m * kb + (k0 >> 1) + 32 * shalf);
                v0 = p[0];
                v1 = p[1];
            }
            uint4* d = reinterpret_cast<uint4*>(&As[srow * LDB + 32 * shalf]);
            d[0] = v0;
            d[1] = v1;
            const int n = n0 + srow;
            uint4 u0 = make_uint4(0, 0, 0, 0), u1 = u0;
            if (n < N) {
                const uint4* p = reinterpret_cast<const uint4*>(w + (size_t)n * kb + (k0 >> 1) + 32 * shalf);
                u0 = p[0];
                u1 = p[1];
            }
            uint4* e = reinterpret_cast<uint4*>(&Bs[srow * LDB + 32 * shalf]);
            e[0] = u0;
            e[1] = u1;
            if (shalf == 0) {
                Asc[srow] = m < M ? *reinterpret_cast<const uint32_t*>(xs + (size_t)m * kg + (k0 >> 5)) : 0u;
                Bsc[srow] = n < N ? *reinterpret_cast<const uint32_t*>(ws + (size_t)n * kg + (k0 >> 5)) : 0u;
            }
        }
        __syncthreads();
        i8v av[4], bv[4];
        int sa[4], sb[4];
        const int grp = lane >> 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = wm * 64 + i * 16 + (lane & 15);
            const uint4 u = *reinterpret_cast<const uint4*>(&As[r * LDB + 16 * grp]);
            av[i] = (i8v){(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
            sa[i] = (int)((Asc[r] >> (8 * grp)) & 0xFFu);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = wn * 64 + j * 16 + (lane & 15);
            const uint4 u = *reinterpret_cast<const uint4*>(&Bs[c * LDB + 16 * grp]);
            bv[j] = (i8v){(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
            sb[j] = (int)((Bsc[c] >> (8 * grp)) & 0xFFu);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av[i], bv[j], acc[i][j], 4, 4, 0,
                                                                             sa[i], 0, sb[j]);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                if (m < M && n < N) store_y<YT>(y, (size_t)m * N + n, acc[i][j][r]);
            }
        }
}

}  // namespace

void launch_mxfp4(const uint8_t* x, const uint8_t* x_scales, const uint8_t* w,
                  const uint8_t* w_scales, void* y, int y_dtype, int M, int K, int N) {
    if (K % KSTEP != 0) fail("byhip: internal: MXFP4 GEMM needs K %% 128 == 0 (K=%d)", K);
    if (M <= 0 || N <= 0) return;
    const dim3 grid((N + TN - 1) / TN, (M + TM - 1) / TM);
    switch (y_dtype) {
    case BYHIP_F32:
        hipLaunchKernelGGL(mxfp4_gemm<BYHIP_F32>, grid, dim3(256), 0, stream(), x, x_scales, w, w_scales,
                           y, M, K, N);
        break;
    case BYHIP_F16:
        hipLaunchKernelGGL(mxfp4_gemm<BYHIP_F16>, grid, dim3(256), 0, stream(), x, x_scales, w, w_scales,
                           y, M, K, N);
        break;
    default:
        hipLaunchKernelGGL(mxfp4_gemm<BYHIP_BF16>, grid, dim3(256), 0, stream(), x, x_scales, w, w_scales,
                           y, M, K, N);
        break;
    }
    BYHIP_LAUNCHED("mxfp4_gemm");
}

}  // namespace byhip
