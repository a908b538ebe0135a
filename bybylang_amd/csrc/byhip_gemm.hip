// byhip_gemm.hip - LDS-staged fp16 MFMA GEMM for the quantized weight formats (gfx950).
//
// y[M, N] = x[M, K] . W^T with W dequantized to fp16 while it is staged in LDS, fp32 accumulation
// in v_mfma_f32_16x16x32_f16. A 256-thread block computes a 64 x 128 tile; its four waves each own a
// 32 x 64 quarter (2 x 4 fragments). Per K step of 64 (two 32-value groups) every thread stages 16
// activations and one weight group (32 values) of one output column.
//
// Operand layout of v_mfma_f32_16x16x32_f16 (checked on the device): lane l holds A[l%16][8(l/16)..+7]
// and B[8(l/16)..+7][l%16]; the result lane l holds C[4(l/16)..+3][l%16].
//
// The order of the 32 values inside a group is free as long as both operands use the same one (a dot
// product does not depend on the order of its terms). Each weight format stages its group in the
// order its packing yields cheaply, and the activations are staged in that same order:
//   Q4Fast  nibble pairs (k, k+4) of each 8-value word, from one AND-OR against 0x6400
//   Fp4Km   byte j -> (element j, element j+16), the FP4-KM packing (session_vm.nim:384-388)
//   others  natural order.
// fp32 activations are split into hi = fp16(x) and lo = fp16(x - hi) and multiplied twice, which
// keeps ~22 bits of x; fp16 activations are used as they are.
#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

constexpr int BM = 64, BN = 128, BK = 64;
constexpr int LDA = BK + 8;  // halves per LDS row (16-byte pad)

template <BFormat F>
struct FormatTraits {
    // 0: natural, 1: (k, k+4) pairs in each 8, 2: (j, j+16) pairs in each 32
    static constexpr int kPerm = F == BFormat::Q4Fast ? 1 : (F == BFormat::Fp4Km ? 2 : 0);
};

__device__ __forceinline__ void split_store(_Float16* hi, _Float16* lo, const float* v, int n) {
    for (int i = 0; i < n; ++i) {
        const _Float16 h = (_Float16)v[i];
        hi[i] = h;
        if (lo) lo[i] = (_Float16)(v[i] - (float)h);
    }
}

// Stages 16 activation values of one row (positions 16*seg .. +15 of the K step) into LDS in the
// format's order.
template <int PERM, bool XF32>
__device__ __forceinline__ void stage_a(const GemmArgs& a, int m, int k0, int seg, _Float16* hi,
                                        _Float16* lo) {
    int eu, ev;  // first elements (relative to k0) of the two 8-value chunks this thread reads
    if (PERM == 2) {
        const int g = seg >> 1, s = seg & 1;
        eu = 32 * g + 8 * s;
        ev = eu + 16;
    } else {
        eu = 16 * seg;
        ev = eu + 8;
    }
    float u[8], v[8];
    const bool row_ok = m < a.M;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int k = k0 + (c == 0 ? eu : ev);
        float* dst = c == 0 ? u : v;
        if (row_ok && k < a.K) {
            if constexpr (XF32) {
                const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(a.x) + (size_t)m * a.K + k);
                const float4 p0 = p[0], p1 = p[1];
                dst[0] = p0.x; dst[1] = p0.y; dst[2] = p0.z; dst[3] = p0.w;
                dst[4] = p1.x; dst[5] = p1.y; dst[6] = p1.z; dst[7] = p1.w;
            } else {
                const h8 h = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + (size_t)m * a.K + k);
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[i] = (float)h[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) dst[i] = 0.0f;
        }
    }
    float o[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (PERM == 0) {
            o[i] = u[i];
            o[8 + i] = v[i];
        } else if (PERM == 1) {
            // positions 2i, 2i+1 of each 8 hold elements i, i+4 (i < 4)
            const int src = i >> 1, hiHalf = i & 1;
            o[i] = u[src + 4 * hiHalf];
            o[8 + i] = v[src + 4 * hiHalf];
        } else {
            o[2 * i] = u[i];
            o[2 * i + 1] = v[i];
        }
    }
    _Float16 th[16], tl[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        th[i] = (_Float16)o[i];
        tl[i] = (_Float16)(o[i] - (float)th[i]);
    }
    *reinterpret_cast<h8*>(hi) = *reinterpret_cast<h8*>(&th[0]);
    *reinterpret_cast<h8*>(hi + 8) = *reinterpret_cast<h8*>(&th[8]);
    if constexpr (XF32) {
        *reinterpret_cast<h8*>(lo) = *reinterpret_cast<h8*>(&tl[0]);
        *reinterpret_cast<h8*>(lo + 8) = *reinterpret_cast<h8*>(&tl[8]);
    }
}

// Stages one 32-value weight group of column n (K positions k0g .. k0g+31) into LDS (32 halves).
template <BFormat F>
__device__ __forceinline__ void stage_b(const GemmArgs& a, int n, int k0g, const float* lut_s,
                                        _Float16* dst) {
    uint32_t outw[16];
    if (n >= a.N || k0g >= a.K) {
#pragma unroll
        for (int i = 0; i < 16; ++i) outw[i] = 0u;
    } else if constexpr (F == BFormat::Q4Fast) {
        const uint4 d = *reinterpret_cast<const uint4*>(a.wq + (size_t)n * a.row_bytes + (k0g >> 1));
        const int chunk = k0g >> 5;
        const int g = a.group ? chunk / (a.group >> 5) : 0;
        const _Float16 s = static_cast<const _Float16*>(a.scales)[(size_t)n * a.gpr + g];
        const _Float16 zb = (_Float16)(1024.0f + a.zero_value);
        const h2 zz = {zb, zb}, ss = {s, s};
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const h2 q = bits_h2(((dw[w] >> (4 * i)) & 0x000F000Fu) | 0x64006400u);
                outw[4 * w + i] = h2_bits((q - zz) * ss);
            }
    } else if constexpr (F == BFormat::Q4Generic) {
        const uint4 d = *reinterpret_cast<const uint4*>(a.wq + (size_t)n * a.row_bytes + (k0g >> 1));
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
        int g = a.group ? k0g / a.group : 0;
        int next = a.group ? (g + 1) * a.group : 0x7FFFFFFF;
        const size_t rowg = (size_t)n * a.gpr;
        auto scale_at = [&](int gg) {
            return a.scale_f16 ? (float)static_cast<const _Float16*>(a.scales)[rowg + gg]
                               : static_cast<const float*>(a.scales)[rowg + gg];
        };
        float s = scale_at(g), z = a.zeros ? a.zeros[rowg + g] : a.zero_value;
        _Float16 t[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            if (k0g + e >= next) {
                ++g;
                next += a.group;
                s = scale_at(g);
                z = a.zeros ? a.zeros[rowg + g] : a.zero_value;
            }
            const uint32_t q = (dw[e >> 3] >> (4 * (e & 7))) & 15u;
            t[e] = (_Float16)(((float)q - z) * s);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            outw[i] = (uint32_t)h_bits(t[2 * i]) | ((uint32_t)h_bits(t[2 * i + 1]) << 16);
    } else if constexpr (F == BFormat::Fp4Km) {
        const size_t kb = (size_t)a.K >> 1;
        const uint4 d = *reinterpret_cast<const uint4*>(a.blob + (size_t)n * kb + (k0g >> 1));
        const uint8_t sb = a.blob[a.scale_base + (size_t)n * (a.K >> 5) + (k0g >> 5)];
        const float s = lut_s[16 + sb];
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (dw[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            const _Float16 lo = (_Float16)(lut_s[byte & 15u] * s);
            const _Float16 hi = (_Float16)(lut_s[byte >> 4] * s);
            outw[j] = (uint32_t)h_bits(lo) | ((uint32_t)h_bits(hi) << 16);
        }
    } else {  // F16
        const uint4* p = reinterpret_cast<const uint4*>(a.w16 + (size_t)n * a.K + k0g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 u = p[i];
            outw[4 * i] = u.x; outw[4 * i + 1] = u.y; outw[4 * i + 2] = u.z; outw[4 * i + 3] = u.w;
        }
    }
    uint4* o = reinterpret_cast<uint4*>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_uint4(outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]);
}

template <BFormat F, bool XF32, int YT>
__global__ __launch_bounds__(256) void gemm_f16_mfma(GemmArgs a) {
    constexpr int PERM = FormatTraits<F>::kPerm;
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDA];
    __shared__ __attribute__((aligned(16))) _Float16 Al[XF32 ? BM * LDA : 8];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDA];
    __shared__ float lut_s[F == BFormat::Fp4Km ? 272 : 1];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;

    if constexpr (F == BFormat::Fp4Km) {
        for (int i = tid; i < 272; i += 256) lut_s[i] = a.lut[i];
        __syncthreads();
    }

    f4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    const int arow = tid >> 2, aseg = tid & 3;
    const int bcol = tid >> 1, bhalf = tid & 1;
    for (int k0 = 0; k0 < a.K; k0 += BK) {
        stage_a<PERM, XF32>(a, m0 + arow, k0, aseg, &As[arow * LDA + 16 * aseg],
                            XF32 ? &Al[arow * LDA + 16 * aseg] : nullptr);
        stage_b<F>(a, n0 + bcol, k0 + 32 * bhalf, lut_s, &Bs[bcol * LDA + 32 * bhalf]);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            h8 av[2], al[2], bv[4];
            const int kc = kk + 8 * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 32 + i * 16 + (lane & 15);
                av[i] = *reinterpret_cast<const h8*>(&As[r * LDA + kc]);
                if constexpr (XF32) al[i] = *reinterpret_cast<const h8*>(&Al[r * LDA + kc]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = wn * 64 + j * 16 + (lane & 15);
                bv[j] = *reinterpret_cast<const h8*>(&Bs[c * LDA + kc]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
                    if constexpr (XF32)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bv[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                if (m < a.M && n < a.N) store_y<YT>(a.y, (size_t)m * a.N + n, acc[i][j][r]);
            }
        }
}

template <BFormat F, bool XF32>
void launch_fx(const GemmArgs& a) {
    const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
    switch (a.y_dtype) {
    case BYHIP_F32:
        hipLaunchKernelGGL((gemm_f16_mfma<F, XF32, BYHIP_F32>), grid, dim3(256), 0, stream(), a);
        break;
    case BYHIP_F16:
        hipLaunchKernelGGL((gemm_f16_mfma<F, XF32, BYHIP_F16>), grid, dim3(256), 0, stream(), a);
        break;
    default:
        hipLaunchKernelGGL((gemm_f16_mfma<F, XF32, BYHIP_BF16>), grid, dim3(256), 0, stream(), a);
        break;
    }
    BYHIP_LAUNCHED("gemm_f16_mfma");
}

template <BFormat F>
void launch_f(const GemmArgs& a) {
    if (a.x_dtype == BYHIP_F32) launch_fx<F, true>(a);
    else launch_fx<F, false>(a);
}

}  // namespace

void launch_gemm(BFormat fmt, const GemmArgs& a) {
    if (a.K % 32 != 0) fail("byhip: internal: GEMM needs K %% 32 == 0 (K=%d)", a.K);
    if (a.M <= 0 || a.N <= 0) return;
    if (a.M > 65535 * BM) fail("byhip: M=%d too large for one launch", a.M);
    switch (fmt) {
    case BFormat::Q4Fast: launch_f<BFormat::Q4Fast>(a); break;
    case BFormat::Q4Generic: launch_f<BFormat::Q4Generic>(a); break;
    case BFormat::Fp4Km: launch_f<BFormat::Fp4Km>(a); break;
    case BFormat::F16: launch_f<BFormat::F16>(a); break;
    }
}

}  // namespace byhip
