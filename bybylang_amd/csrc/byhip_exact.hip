// byhip_exact.hip - the exact fp32 GEMM for the quantized weight formats (gfx950).
//
// y[M, N] = x[M, K] . W^T where every weight is formed in fp32 exactly as the reference forms it:
//   Q4      ((float)q - zero) * scale, any scales, zeros and group size (cpu_vm.c:467-470,
//           cpu_kernels_impl.inc:309-314)
//   FP4-KM  lut[nibble] * lut[16 + scale byte] (cpu_vm.c:611-618)
//   F16     the half widened (cpu_vm.c:571-575)
// Activations are used in fp32 (fp16 ones widened exactly); products and sums are fp32, in
// v_mfma_f32_16x16x4_f32. This is the route for data the fp16 MFMA kernels cannot hold exactly:
// Q4 weights outside fp16's range, FP4-KM tables whose products are not halves, and the micro-VM's
// Q4 GEMV op (fp32 arithmetic in the reference) above the decode GEMV's rows. It differs from the
// reference only in the order of the fp32 additions.
//
// Block: BM x 64 outputs, 4 waves; wave w owns columns 16w .. 16w+15 and all BM rows (BM / 16
// fragments). K steps of 64: each thread stages BM / 4 activations and 16 weights of one column
// (formed in fp32) into LDS, then each wave issues 16 MFMAs per fragment.
// Operand layout of v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][g] and B[g][l % 16] for its
// lane group g = l / 16; the result lane l holds C[4g + i][l % 16], i = 0..3. In MFMA kk (0..15) of a
// step, lane group g supplies K position 16g + kk, so one 16-byte LDS read gives a lane four MFMAs'
// worth of an operand; both operands use that order, so every product pairs the same k.
// Split-K: when the tiles leave CUs idle, block z covers K steps [z * split_steps, ...) and writes
// fp32 partials that splitk_sum adds in slice order.
#include <algorithm>

#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

constexpr int EBK = 64;        // K values per step
constexpr int ELD = EBK + 4;   // floats per LDS row: 16-byte aligned rows, 4-bank skew per row

// FX activations of row m from position k (zeros past M and K), widened to fp32.
template <bool XF32, int FX>
__device__ __forceinline__ void exact_x(const GemmArgs& a, int m, int k, float* v) {
    const bool row = m < a.M;
    const size_t base = (size_t)m * a.K;
#pragma unroll
    for (int e = 0; e < FX; ++e) {
        const bool ok = row && k + e < a.K;
        if constexpr (XF32) v[e] = ok ? static_cast<const float*>(a.x)[base + k + e] : 0.0f;
        else v[e] = ok ? (float)static_cast<const _Float16*>(a.x)[base + k + e] : 0.0f;
    }
}

// The 16 weights of column n at K positions k .. k+15 (k % 16 == 0), formed as the reference forms
// them; zeros past N and K.
template <BFormat F>
__device__ __forceinline__ void exact_w(const GemmArgs& a, int n, int k, const float* lut_s, float* w) {
#pragma unroll
    for (int e = 0; e < 16; ++e) w[e] = 0.0f;
    if (n >= a.N || k >= a.K) return;
    if constexpr (F == BFormat::Fp4Km) {
        // FP4-KM group g = k / 32: byte j holds element j (low nibble) and j + 16 (high nibble)
        const int g = k >> 5, hi = (k >> 4) & 1;
        const uint4 d = *reinterpret_cast<const uint4*>(a.blob + (size_t)n * (a.K >> 1) + (size_t)g * 16);
        const float s = lut_s[16 + a.blob[a.scale_base + (size_t)n * (a.K >> 5) + g]];
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (dw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            w[j] = lut_s[hi ? byte >> 4 : byte & 15u] * s;
        }
    } else if constexpr (F == BFormat::F16) {
        const _Float16* p = reinterpret_cast<const _Float16*>(a.w16) + (size_t)n * a.K + k;
#pragma unroll
        for (int e = 0; e < 16; ++e) w[e] = (float)p[e];
    } else {
        // Q4: nibble k at byte k / 2 of the row, even k in the low nibble
        const uint8_t* row = a.wq + (size_t)n * a.row_bytes;
        uint32_t b[8];
        if (a.row_bytes % 4 == 0 && reinterpret_cast<uintptr_t>(a.wq) % 4 == 0) {
            const uint32_t* r32 = reinterpret_cast<const uint32_t*>(row + (k >> 1));
            const uint32_t w0 = r32[0], w1 = (size_t)(k >> 1) + 4 < a.row_bytes ? r32[1] : 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                b[i] = (w0 >> (8 * i)) & 0xFFu;
                b[4 + i] = (w1 >> (8 * i)) & 0xFFu;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) b[i] = (size_t)(k >> 1) + i < a.row_bytes ? row[(k >> 1) + i] : 0u;
        }
        const size_t rowg = (size_t)n * a.gpr;
        int g = a.group ? k / a.group : 0;
        int next = a.group ? (g + 1) * a.group : 0x7FFFFFFF;
        auto scale_at = [&](int gg) {
            return a.scale_f16 ? (float)static_cast<const _Float16*>(a.scales)[rowg + gg]
                               : static_cast<const float*>(a.scales)[rowg + gg];
        };
        float s = scale_at(g), z = a.zeros ? a.zeros[rowg + g] : a.zero_value;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            if (k + e >= a.K) break;
            if (k + e >= next) {
                ++g;
                next += a.group;
                s = scale_at(g);
                z = a.zeros ? a.zeros[rowg + g] : a.zero_value;
            }
            const uint32_t q = (b[e >> 1] >> (4 * (e & 1))) & 15u;
            w[e] = ((float)q - z) * s;
        }
    }
}

__device__ __forceinline__ void store_any(void* y, int y_dtype, size_t idx, float v) {
    if (y_dtype == BYHIP_F32) store_y<BYHIP_F32>(y, idx, v);
    else if (y_dtype == BYHIP_F16) store_y<BYHIP_F16>(y, idx, v);
    else store_y<BYHIP_BF16>(y, idx, v);
}

template <BFormat F, bool XF32, int BM>
__global__ __launch_bounds__(256) void gemm_f32_exact(GemmArgs a) {
    if (a.gate && *a.gate != a.gate_want) return;  // the other route was chosen (whole grid)
    constexpr int FM = BM / 16;      // row fragments per wave
    constexpr int FX = BM / 4;       // activations a thread stages per step
    constexpr int XT = EBK / FX;     // threads per activation row
    __shared__ __attribute__((aligned(16))) float xs[BM * ELD];
    __shared__ __attribute__((aligned(16))) float ws[64 * ELD];
    __shared__ float lut_s[F == BFormat::Fp4Km ? 272 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int n0 = blockIdx.x * 64, m0 = blockIdx.y * BM;
    const int total = (a.K + EBK - 1) / EBK;
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nsteps = a.part ? min(a.split_steps, total - s_first) : total;

    if constexpr (F == BFormat::Fp4Km) {
        for (int i = tid; i < 272; i += 256) lut_s[i] = a.lut[i];
        __syncthreads();
    }

    f4 acc[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) acc[i] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    const int xrow = tid / XT, xseg = tid % XT;  // the activation row this thread stages, FX values
    const int wcol = tid >> 2, wseg = tid & 3;   // the weight column, 16 values
    for (int s = 0; s < nsteps; ++s) {
        const int k0 = (s_first + s) * EBK;
        float xv[FX], wv[16];
        exact_x<XF32, FX>(a, m0 + xrow, k0 + xseg * FX, xv);
        exact_w<F>(a, n0 + wcol, k0 + wseg * 16, lut_s, wv);
#pragma unroll
        for (int t = 0; t < FX / 4; ++t)
            *reinterpret_cast<float4*>(&xs[xrow * ELD + xseg * FX + 4 * t]) =
                make_float4(xv[4 * t], xv[4 * t + 1], xv[4 * t + 2], xv[4 * t + 3]);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            *reinterpret_cast<float4*>(&ws[wcol * ELD + wseg * 16 + 4 * t]) =
                make_float4(wv[4 * t], wv[4 * t + 1], wv[4 * t + 2], wv[4 * t + 3]);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 b = *reinterpret_cast<const float4*>(&ws[(16 * wid + c) * ELD + 16 * g + 4 * q]);
            float4 av[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                av[i] = *reinterpret_cast<const float4*>(&xs[(16 * i + c) * ELD + 16 * g + 4 * q]);
            const float bj[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const float aj[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(aj[j], bj[j], acc[i], 0, 0, 0);
                }
        }
        __syncthreads();
    }

    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
    const int n = n0 + 16 * wid + c;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * i + 4 * g + r;
            if (m < a.M && n < a.N) {
                if (part) part[(size_t)m * a.N + n] = acc[i][r];
                else store_any(a.y, a.y_dtype, (size_t)m * a.N + n, acc[i][r]);
            }
        }
}

template <BFormat F, bool XF32>
void launch_exact_bm(const GemmArgs& a, int bm, dim3 grid) {
    switch (bm) {
    case 16: launch("gemm_f32_exact", (gemm_f32_exact<F, XF32, 16>), grid, dim3(256), 0, a); break;
    case 32: launch("gemm_f32_exact", (gemm_f32_exact<F, XF32, 32>), grid, dim3(256), 0, a); break;
    default: launch("gemm_f32_exact", (gemm_f32_exact<F, XF32, 64>), grid, dim3(256), 0, a); break;
    }
    BYHIP_LAUNCHED("gemm_f32_exact");
}

template <BFormat F>
void launch_exact_x(const GemmArgs& a, int bm, dim3 grid) {
    if (a.x_dtype == BYHIP_F32) launch_exact_bm<F, true>(a, bm, grid);
    else launch_exact_bm<F, false>(a, bm, grid);
}

}  // namespace

void launch_gemm_exact(BFormat fmt, const GemmArgs& a0) {
    GemmArgs a = a0;
    if (a.M <= 0 || a.N <= 0 || a.K <= 0) return;
    if (fmt != BFormat::Q4Fast && fmt != BFormat::Q4Generic && a.K % 32 != 0)
        fail("byhip: internal: the exact FP4-KM / F16 GEMM needs K %% 32 == 0 (K=%d)", a.K);
    const int bm = a.M <= 16 ? 16 : (a.M <= 32 ? 32 : 64);
    if ((a.M + bm - 1) / bm > 65535) fail("byhip: M=%d too large for one launch", a.M);
    const long tiles = (long)((a.N + 63) / 64) * ((a.M + bm - 1) / bm);
    const int nsteps = (a.K + EBK - 1) / EBK;
    const int splits = choose_split(a, tiles, nsteps, 4, 0, 2);
    const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)((a.M + bm - 1) / bm), (unsigned)splits);
    switch (fmt) {
    case BFormat::Fp4Km: launch_exact_x<BFormat::Fp4Km>(a, bm, grid); break;
    case BFormat::F16: launch_exact_x<BFormat::F16>(a, bm, grid); break;
    default: launch_exact_x<BFormat::Q4Generic>(a, bm, grid); break;
    }
    if (a.part) launch_splitk_sum(a, splits);
}

}  // namespace byhip
