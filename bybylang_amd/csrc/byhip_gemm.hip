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
// fp32 activations: each row is first brought onto fp16's range by an exact power of two (undone
// on the output), then split into hi = fp16(x) and lo = fp16(x - hi), ~22 bits of x; with Q4
// weights the weight's fp16 remainder is staged as well and the products hi*w_hi + lo*w_hi +
// hi*w_lo keep the fp32 weight, so fp32 activations meet the reference's fp32 tolerance. fp16
// activations are used as they are, against the weight rounded once to fp16.
#include <algorithm>
#include <utility>

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
    // fp32 activations: the row's power-of-two shift onto fp16's range (exact)
    const int sh = XF32 && row_ok ? a.row_shift[m] : 0;
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
#pragma unroll
                for (int i = 0; i < 8; ++i) dst[i] = __builtin_amdgcn_ldexpf(dst[i], sh);
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
// WLO (Q4 formats with fp32 activations): also the remainder w - fp16(w) as halves into dst_lo, so
// that hi + lo holds the fp32 weight to ~22 bits (for Q4Fast exactly: (q - z) * s has at most 15
// significant bits, and the remainder at most 4 at or above 2^-24, the weights being fp16-safe).
template <BFormat F, bool WLO>
__device__ __forceinline__ void stage_b(const GemmArgs& a, int n, int k0g, const float* lut_s,
                                        _Float16* dst, _Float16* dst_lo) {
    uint32_t outw[16], outl[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) outl[i] = 0u;
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
                const h2 qz = q - zz, hi = qz * ss;
                outw[4 * w + i] = h2_bits(hi);
                if constexpr (WLO) {
                    // (q - z) * s exactly in fp32, less its fp16 rounding: exact in fp16
                    const float sf = (float)s;
                    const _Float16 l0 = (_Float16)((float)qz[0] * sf - (float)hi[0]);
                    const _Float16 l1 = (_Float16)((float)qz[1] * sf - (float)hi[1]);
                    outl[4 * w + i] = (uint32_t)h_bits(l0) | ((uint32_t)h_bits(l1) << 16);
                }
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
        _Float16 t[32], tl[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            if (k0g + e >= next) {
                ++g;
                next += a.group;
                s = scale_at(g);
                z = a.zeros ? a.zeros[rowg + g] : a.zero_value;
            }
            const uint32_t q = (dw[e >> 3] >> (4 * (e & 7))) & 15u;
            const float wf = ((float)q - z) * s;  // the reference's weight
            t[e] = (_Float16)wf;
            tl[e] = WLO ? (_Float16)(wf - (float)t[e]) : (_Float16)0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            outw[i] = (uint32_t)h_bits(t[2 * i]) | ((uint32_t)h_bits(t[2 * i + 1]) << 16);
            outl[i] = (uint32_t)h_bits(tl[2 * i]) | ((uint32_t)h_bits(tl[2 * i + 1]) << 16);
        }
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
    if constexpr (WLO) {
        uint4* ol = reinterpret_cast<uint4*>(dst_lo);
#pragma unroll
        for (int i = 0; i < 4; ++i) ol[i] = make_uint4(outl[4 * i], outl[4 * i + 1], outl[4 * i + 2], outl[4 * i + 3]);
    }
}

template <BFormat F, bool XF32, int YT>
__global__ __launch_bounds__(256) void gemm_f16_mfma(GemmArgs a) {
    if (a.gate && *a.gate != a.gate_want) return;  // the other route was chosen (whole grid)
    constexpr int PERM = FormatTraits<F>::kPerm;
    // fp32 activations with Q4 weights: the weights' fp16 remainders too (F16 weights and FP4-KM
    // tables of halves are exact in one fp16 term)
    constexpr bool WLO = XF32 && (F == BFormat::Q4Fast || F == BFormat::Q4Generic);
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDA];
    __shared__ __attribute__((aligned(16))) _Float16 Al[XF32 ? BM * LDA : 8];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDA];
    __shared__ __attribute__((aligned(16))) _Float16 Bl[WLO ? BN * LDA : 8];
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
    // split-K: block z covers the K steps [z * split_steps, (z + 1) * split_steps)
    const int k_begin = a.part ? (int)blockIdx.z * a.split_steps * BK : 0;
    const int k_end = a.part ? min(a.K, k_begin + a.split_steps * BK) : a.K;
    for (int k0 = k_begin; k0 < k_end; k0 += BK) {
        stage_a<PERM, XF32>(a, m0 + arow, k0, aseg, &As[arow * LDA + 16 * aseg],
                            XF32 ? &Al[arow * LDA + 16 * aseg] : nullptr);
        stage_b<F, WLO>(a, n0 + bcol, k0 + 32 * bhalf, lut_s, &Bs[bcol * LDA + 32 * bhalf],
                        WLO ? &Bl[bcol * LDA + 32 * bhalf] : nullptr);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            h8 av[2], al[2], bv[4], bl[4];
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
                if constexpr (WLO) bl[j] = *reinterpret_cast<const h8*>(&Bl[c * LDA + kc]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
                    if constexpr (XF32)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bv[j], acc[i][j], 0, 0, 0);
                    if constexpr (WLO)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bl[j], acc[i][j], 0, 0, 0);
                }
        }
        __syncthreads();
    }

    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + wn * 64 + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                if (m < a.M && n < a.N) {
                    // fp32 activations: undo the row's shift (exact unless the result over- or
                    // underflows, as the reference's own sum would)
                    const float v = XF32 ? __builtin_amdgcn_ldexpf(acc[i][j][r], -a.row_shift[m]) : acc[i][j][r];
                    if (part) part[(size_t)m * a.N + n] = v;
                    else store_y<YT>(a.y, (size_t)m * a.N + n, v);
                }
            }
        }
}

// Per-row shift t of fp32 activations: the row's largest magnitude brought into [2^14, 2^15) (one
// block per row), so the fp16 hi + lo split of x * 2^t neither overflows nor loses the row's large
// values to fp16 subnormals.
__global__ __launch_bounds__(256) void row_range_shift(const float* __restrict__ x, int K, int* __restrict__ out) {
    __shared__ float part[4];
    const float* r = x + (size_t)blockIdx.x * K;
    float mx = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) mx = fmaxf(mx, fabsf(r[k]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = fp16_range_shift(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])));
}

// fp32 activations for the wide tile: the row's shift t as row_range_shift finds it, and the
// shifted row as two fp16 planes, hi = fp16(x 2^t) and lo = fp16(x 2^t - hi) (about 22 bits of x).
// One block per row, K % 4 == 0, 16-byte aligned rows. The first kSplitHeld float4 of each thread
// (K <= 8192) are loaded at once and stay in registers between the maximum and the split; the
// rest of a longer row is read again.
constexpr int kSplitHeld = 8;
__global__ __launch_bounds__(256) void split_rows_f16(const float* __restrict__ x, int K, int* __restrict__ shifts,
                                                     _Float16* __restrict__ hi, _Float16* __restrict__ lo) {
    __shared__ float part[4];
    __shared__ int shift;
    const size_t row = (size_t)blockIdx.x * K;
    const float4* r = reinterpret_cast<const float4*>(x + row);
    const int nq = K / 4;
    float4 held[kSplitHeld];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < kSplitHeld; ++u) {
        const int k = (int)threadIdx.x + 256 * u;
        held[u] = k < nq ? r[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < kSplitHeld; ++u)
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(held[u].x), fabsf(held[u].y))), fmaxf(fabsf(held[u].z), fabsf(held[u].w)));
    for (int k = (int)threadIdx.x + 256 * kSplitHeld; k < nq; k += 256) {
        const float4 v = r[k];
        mx = fmaxf(fmaxf(mx, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        shift = fp16_range_shift(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])));
        shifts[blockIdx.x] = shift;
    }
    __syncthreads();
    const int t = shift;
    auto split = [&](int k, const float4 v) {
        const float s[4] = {__builtin_amdgcn_ldexpf(v.x, t), __builtin_amdgcn_ldexpf(v.y, t),
                            __builtin_amdgcn_ldexpf(v.z, t), __builtin_amdgcn_ldexpf(v.w, t)};
        uint16_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const _Float16 he = (_Float16)s[e];
            h[e] = h_bits(he);
            l[e] = h_bits((_Float16)(s[e] - (float)he));
        }
        reinterpret_cast<uint2*>(hi + row)[k] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
        reinterpret_cast<uint2*>(lo + row)[k] = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    };
#pragma unroll
    for (int u = 0; u < kSplitHeld; ++u) {
        const int k = (int)threadIdx.x + 256 * u;
        if (k < nq) split(k, held[u]);
    }
    for (int k = (int)threadIdx.x + 256 * kSplitHeld; k < nq; k += 256) split(k, r[k]);
}

// Pipelined Q4 GEMM for the benchmark format: fp16 activations, fp16 scales, one integral zero,
// group 0 or 32 * 2^j, K % 64 == 0. A 256-thread block computes a BM x BN tile (BM 32 or 64, BN 64
// or 128, chosen per shape) in K steps of 64 (two 32-value groups); its four waves each own a
// 32-row slice of BN / (4 / (BM / 32)) columns, as 16 x 16 fragments of v_mfma_f32_16x16x32_f16.
// LDS holds two steps (double buffer, one barrier per step); each thread's global loads run three
// steps ahead in registers (three register sets rotate), so a step's MFMAs overlap the
// dequantization of the next step and the loads of later ones.
//   x: each thread stages BM / 4 values of one row, permuted to the weights' (k, k+4) pair order.
//   W: each thread dequantizes BN / 4 values of one column. A nibble at bits 0-3 of a half ORed
//      into 0x6400 is the fp16 1024 + q, at bits 4-7 into 0x5400 it is 64 + q; minus 1024 + z or
//      64 + z that is q - z exactly, times the fp16 scale (one rounding), as Q4Fast does.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
constexpr int PBK = 64;
constexpr int PLD = PBK + 8;  // halves per LDS row (16-byte pad)

template <int BM, int BN>
struct PipeShape {
    static constexpr int WGM = BM / 32, WGN = 4 / WGM;   // wave grid
    static constexpr int WN = BN / WGN, FN = WN / 16;     // columns and fragments per wave
    static constexpr int XV = BM / 4;                     // activations staged per thread (8 or 16)
    static constexpr int XT = PBK / XV;                   // threads per activation row
    static constexpr int WV = BN / 4;                     // weights dequantized per thread (16 or 32)
    static constexpr int WT = PBK / WV;                   // threads per weight column
    static_assert(WGM * WGN == 4 && FN >= 1, "tile shape");
};

struct PipeRegs {
    uint4 x0, x1;  // up to 16 activations of one row
    uint4 w;       // up to 32 nibbles of one column
    uint32_t s;    // their fp16 scale
};

// (a.lo, b.lo) and (a.hi, b.hi) halves of two dwords.
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
// 8 activations (x0..x7) reordered to (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ uint4 perm8(uint4 v) {
    return make_uint4(pair_lo(v.x, v.z), pair_hi(v.x, v.z), pair_lo(v.y, v.w), pair_hi(v.y, v.w));
}

template <int BM, int BN, int YT>
__global__ __launch_bounds__(256) void q4_gemm_pipe(GemmArgs a) {
    using S = PipeShape<BM, BN>;
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * PLD];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * PLD];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid / S::WGN, wn = wid % S::WGN;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = a.K;
    // K steps of this block: all of them, or split_steps from blockIdx.z * split_steps (split-K)
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nsteps = a.part ? min(a.split_steps, K / PBK - s_first) : K / PBK;

    // Rows past M / N read zeros through the buffer range checks (offsets stay below 2^32: the
    // launcher checks the sizes).
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.M * K * 2));
    const rsrc_t wr = make_rsrc(a.wq, (uint32_t)((size_t)a.N * a.row_bytes));
    const rsrc_t sr = make_rsrc(a.scales, (uint32_t)((size_t)a.N * a.gpr * 2));
    const int arow = tid / S::XT, aseg = tid % S::XT;    // values aseg*XV .. +XV-1 of the step
    const int bcol = tid / S::WT, bseg = tid % S::WT;    // values bseg*WV .. +WV-1 of the step
    const uint32_t xoff = (uint32_t)(m0 + arow) * (uint32_t)K * 2u + (uint32_t)(2 * S::XV * aseg);
    const uint32_t woff = (uint32_t)(n0 + bcol) * (uint32_t)a.row_bytes + (uint32_t)(S::WV / 2 * bseg);
    const uint32_t soff = (uint32_t)(n0 + bcol) * (uint32_t)a.gpr;
    const int gshift = a.group ? __builtin_ctz((unsigned)a.group >> 5) : 0;  // group: 0 or 32 * 2^j

    auto gload = [&](PipeRegs& r, int s) {
        const int k0 = (s_first + min(s, nsteps - 1)) * PBK;
        const v4u u0 = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + 2u * k0, 0, 0);
        r.x0 = make_uint4(u0[0], u0[1], u0[2], u0[3]);
        if constexpr (S::XV == 16) {
            const v4u u1 = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff + 2u * k0 + 16u, 0, 0);
            r.x1 = make_uint4(u1[0], u1[1], u1[2], u1[3]);
        }
        if constexpr (S::WV == 32) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wr, woff + (uint32_t)(k0 >> 1), 0, 0);
            r.w = make_uint4(v[0], v[1], v[2], v[3]);
        } else {
            const v2u v = __builtin_amdgcn_raw_buffer_load_b64(wr, woff + (uint32_t)(k0 >> 1), 0, 0);
            r.w = make_uint4(v[0], v[1], 0u, 0u);
        }
        const int g = a.group ? ((k0 + bseg * S::WV) >> 5) >> gshift : 0;
        r.s = __builtin_amdgcn_raw_buffer_load_b16(sr, 2u * (soff + (uint32_t)g), 0, 0);
    };
    const _Float16 zlo = (_Float16)(1024.0f + a.zero_value), zhi = (_Float16)(64.0f + a.zero_value);
    const h2 zz_lo = {zlo, zlo}, zz_hi = {zhi, zhi};
    // The magic words live in VGPRs so each AND-OR is one v_and_or_b32.
    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));
    auto stage = [&](const PipeRegs& r, int buf) {
        uint4* da = reinterpret_cast<uint4*>(&As[buf][arow * PLD + S::XV * aseg]);
        da[0] = perm8(r.x0);
        if constexpr (S::XV == 16) da[1] = perm8(r.x1);
        // weights: word d holds values k..k+7; pair i = (k+i, k+i+4)
        const _Float16 sc = bits_h((uint16_t)r.s);
        const h2 ss = {sc, sc};
        const uint32_t dw[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
        uint4* db = reinterpret_cast<uint4*>(&Bs[buf][bcol * PLD + S::WV * bseg]);
#pragma unroll
        for (int w = 0; w < S::WV / 8; ++w) {
            const uint32_t d8 = dw[w] >> 8;
            const h2 q0 = bits_h2((dw[w] & 0x000F000Fu) | mag_lo);
            const h2 q1 = bits_h2((dw[w] & 0x00F000F0u) | mag_hi);
            const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo);
            const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi);
            db[w] = make_uint4(h2_bits((q0 - zz_lo) * ss), h2_bits((q1 - zz_hi) * ss),
                               h2_bits((q2 - zz_lo) * ss), h2_bits((q3 - zz_hi) * ss));
        }
    };

    f4 acc[2][S::FN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < S::FN; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    const int kc = 8 * (lane >> 4);
    auto mma = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < PBK; kk += 32) {
            h8 av[2], bv[S::FN];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                av[i] = *reinterpret_cast<const h8*>(&As[buf][(wm * 32 + i * 16 + (lane & 15)) * PLD + kk + kc]);
#pragma unroll
            for (int j = 0; j < S::FN; ++j)
                bv[j] = *reinterpret_cast<const h8*>(&Bs[buf][(wn * S::WN + j * 16 + (lane & 15)) * PLD + kk + kc]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < S::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
    };

    PipeRegs r0, r1, r2;
    gload(r0, 0);
    gload(r1, 1);
    gload(r2, 2);
    stage(r0, 0);
    __syncthreads();
    // Step s: MFMAs on buffer s % 2; stage step s + 1 (registers loaded three steps ago) into the
    // other buffer; load step s + 3 into the registers step s used.
    auto step = [&](int s, PipeRegs& rs, PipeRegs& rn, bool more) {
        mma(s & 1);
        // Keeps each accumulator in its AGPRs across steps (otherwise the allocator rotates them
        // through copies at the loop head).
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < S::FN; ++j) asm volatile("" : "+a"(acc[i][j]));
        if (more) stage(rn, (s + 1) & 1);
        gload(rs, s + 3);
        __syncthreads();
    };
    int s = 0;
    for (; s + 3 < nsteps; s += 3) {  // every step here has a successor
        step(s, r0, r1, true);
        step(s + 1, r1, r2, true);
        step(s + 2, r2, r0, true);
    }
    if (s < nsteps) step(s, r0, r1, s + 1 < nsteps);
    if (s + 1 < nsteps) step(s + 1, r1, r2, s + 2 < nsteps);
    if (s + 2 < nsteps) step(s + 2, r2, r0, false);

    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < S::FN; ++j) {
            const int n = n0 + wn * S::WN + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
                if (m < a.M && n < a.N) {
                    if (part) part[(size_t)m * a.N + n] = acc[i][j][r];
                    else store_y<YT>(a.y, (size_t)m * a.N + n, acc[i][j][r]);
                }
            }
        }
}

// y = sum over z of part[z] (z in order, so the result does not depend on block timing), four
// consecutive outputs per thread; nothing when `gate` is set and *gate != want (GemmArgs::gate).
// The same sum, one output per thread: four times the blocks, for outputs too few to fill the CUs
// four to a thread.
template <int YT>
__global__ __launch_bounds__(256) void splitk_sum1(const float* __restrict__ part, int splits, int M, int N,
                                                   void* y, const int* gate, int want) {
    if (gate && *gate != want) return;
    const size_t mn = (size_t)M * N, stride = splitk_stride(M, N);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    float t = 0.0f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < splits) v[u] = part[(size_t)(z0 + u) * stride + i];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (z0 + u < splits) t = z0 + u == 0 ? v[0] : t + v[u];
    }
    store_y<YT>(y, i, t);
}

template <int YT>
__global__ __launch_bounds__(256) void splitk_sum(const float* __restrict__ part, int splits, int M, int N,
                                                  void* y, const int* gate, int want) {
    if (gate && *gate != want) return;
    const size_t mn = (size_t)M * N, stride = splitk_stride(M, N);
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;
    if (i + 4 <= mn) {
        // The slices are loaded eight at a time before they are added, so their latencies overlap.
        float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int z0 = 0; z0 < splits; z0 += 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (z0 + u < splits) v[u] = *reinterpret_cast<const float4*>(part + (size_t)(z0 + u) * stride + i);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (z0 + u < splits) {
                    if (z0 + u == 0) t = v[0];
                    else { t.x += v[u].x; t.y += v[u].y; t.z += v[u].z; t.w += v[u].w; }
                }
        }
        store_y<YT>(y, i, t.x);
        store_y<YT>(y, i + 1, t.y);
        store_y<YT>(y, i + 2, t.z);
        store_y<YT>(y, i + 3, t.w);
    } else {
        for (size_t e = i; e < mn; ++e) {
            float t = part[e];
            for (int z = 1; z < splits; ++z) t += part[(size_t)z * stride + e];
            store_y<YT>(y, e, t);
        }
    }
}

// Skinny Q4 GEMM for small M (the decode-batch and short-prefill shapes): weights are read once,
// straight from HBM into MFMA operand registers, so the kernel streams them like the GEMV while the
// MFMAs do the row products. Same format conditions as q4_gemm_pipe, K % 128 == 0, M <= 32; the
// wide 64 x 128 tile below serves prefill shapes.
//   Block: 4 waves on the same 16 FN columns (FN fragments of 16) and BM rows (BM / 16
//   fragments);
//   the block's K steps of 128 are dealt round-robin to its waves, and the four partial tiles are
//   added through LDS at the end (wave order 0 + 1 + 2 + 3).
//   K order: in MFMA kk (0..3) of a step, lane group g (lanes 16g..16g+15) supplies the values
//   32g + 8kk + (0, 4, 1, 5, 2, 6, 3, 7) of the step. A lane's weights for a step are then one
//   16-byte load (one 32-value group) and one scale, from the blocked scale copy when the
//   weights have one (a fragment's 16 columns x 4 chunks are then 2 lines); the (k, k+4) order is
//   what the AND-OR
//   dequantization yields, and perm8 gives the activations the same order. Both operands use it,
//   so every product pairs the same k.
//   Activations: each wave moves its step's BM x 128 slice straight from global memory into its
//   own LDS buffer (16 lanes read a row's 256 bytes, so every load is a run of whole lines), with
//   16-byte chunk c of row r at slot c ^ (r & 15) (the fragment reads take 16 rows, one chunk
//   each). Each wave reads only what it loaded, so no barrier is
//   needed; the double buffer and a vmcnt wait order the direct loads and the reads.
//   Shapes: BM x 16 FN with FN = 4 column fragments and BM 16 or 32 (two blocks per CU). The
//   64 x 128 prefill tile with the same operand layout is q4_gemm_wide.
template <int FN>
struct SkinnyW {
    v4u w[FN];       // 32 nibbles of one column per fragment
    uint32_t s[FN];  // their fp16 scale
};

// Partial tiles staged in LDS in output layout: rows of 16 FN + 4 floats, so that the accumulator
// writes (lanes: 16 columns x 4 row groups) hit 64 distinct banks.
constexpr int out_pitch(int FN) { return 16 * FN + 4; }

template <int BM, int FN>
struct SkinnyLds {
    static constexpr int kX = 4 * 2 * BM * 256;                 // 4 waves x 2 buffers x BM rows x 256 bytes
    static constexpr int kRed = 4 * BM * out_pitch(FN) * 4;      // 4 partial tiles of the block
    static constexpr int kBytes = kX > kRed ? kX : kRed;
};

template <int BM, int FN, int YT>
__global__ __launch_bounds__(256, 2) void q4_gemm_skinny(GemmArgs a) {
    static_assert(FN <= 4 && BM <= 32, "q4_gemm_skinny: 16 or 32 rows, at most 4 column fragments");
    constexpr int FM = BM / 16;  // row fragments
    constexpr int XDMA = BM / 4;                           // direct loads per step (4 rows each)
    constexpr int XBUF = BM * 256;                         // bytes of one activation buffer
    __shared__ __attribute__((aligned(16))) uint8_t lds[SkinnyLds<BM, FN>::kBytes];

    // wid is wave-uniform; readfirstlane tells the compiler so, which keeps the step logic in
    // scalar registers and branches.
    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * (16 * FN), m0 = blockIdx.y * BM;
    const int K = a.K;
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nsteps = a.part ? min(a.split_steps, K / 128 - s_first) : K / 128;  // the block's steps

    // Rows past M and columns past N read zeros through the range checks (the launcher keeps the
    // offsets below 2^31).
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.M * K * 2));
    const rsrc_t wr = make_rsrc(a.wq, (uint32_t)((size_t)a.N * a.row_bytes));
    // Scales: from the blocked copy when there is one (a lane group's 4 chunks of 8 columns are 64
    // contiguous bytes, so a fragment's load touches 2 lines rather than 16), else row-major.
    const bool sblk = a.sblk != nullptr;
    const uint32_t G = (uint32_t)K >> 5;
    const rsrc_t sr = sblk ? make_rsrc(a.sblk, (uint32_t)(((size_t)a.N + 7) / 8 * 8 * G * 2))
                           : make_rsrc(a.scales, (uint32_t)((size_t)a.N * a.gpr * 2));
    const int gshift = a.group ? __builtin_ctz((unsigned)a.group >> 5) : 0;
    // Direct load u of a step: lane -> row 4u + lane / 16, LDS slot lane % 16 holding chunk
    // slot ^ (row & 15) of that row. Loads u and u + 4 differ by 16 rows and share the slot
    // pattern, so four lane offsets serve them all; the rest of every offset is wave-uniform and
    // travels in the scalar offset, as does each column fragment's row of weights and scales.
    uint32_t xo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = 4 * q + (lane >> 4), chunk = (lane & 15) ^ (r & 15);
        xo[q] = (uint32_t)(m0 + r) * (uint32_t)K * 2u + 16u * chunk;
    }
    const uint32_t xrow16 = 16u * (uint32_t)K * 2u;  // 16 activation rows
    const uint32_t wo = (uint32_t)(n0 + c) * (uint32_t)a.row_bytes + 16u * g;
    const uint32_t so = sblk ? 2u * ((((uint32_t)n0 >> 3) + ((uint32_t)c >> 3)) * G * 8u + 8u * g + (c & 7))
                             : (uint32_t)(n0 + c) * (uint32_t)a.gpr;
    const uint32_t wfrag = 16u * (uint32_t)a.row_bytes;                              // per fragment
    const uint32_t sfrag = sblk ? 32u * G : 32u * (uint32_t)a.gpr;
    uint8_t* const xbuf = lds + wid * 2 * XBUF;

    // Step t of this wave is block step (wid + 4t + rot) mod nsteps: the rotation by the block
    // index staggers where blocks start along K.
    const int nt = nsteps > wid ? (nsteps - wid + 3) / 4 : 0;
    const int rot = nsteps > 0 ? (int)(blockIdx.x % (unsigned)nsteps) : 0;
    auto kstep = [&](int t) {
        const int v = wid + 4 * t + rot;
        return v >= nsteps ? v - nsteps : v;
    };
    // Every step issues the same loads: XDMA direct activation loads, then FN weight and FN scale
    // loads. A step past the wave's last one (t >= nt) adds 2^31 through the scalar offset, which
    // every resource rejects: it reads zeros without touching memory, so the loads need no branch
    // around them and every step leaves the same number in flight.
    auto load = [&](SkinnyW<FN>& r, uint8_t* __restrict__ dst, int t) {
        const bool ok = t < nt;
        const uint32_t k0 = (uint32_t)(s_first + (ok ? kstep(t) : 0)) * 128u;
        const uint32_t oob = ok ? 0u : 0x80000000u;
        const uint32_t grp = a.group ? ((k0 >> 5) + g) >> gshift : 0u;
        const uint32_t soff = sblk ? so + 16u * (k0 >> 5) : 2u * (so + grp);
#pragma unroll
        for (int u = 0; u < XDMA; ++u)
            lds_dma16(xr, dst + 1024 * u, xo[u & 3] + 2u * k0, oob + (uint32_t)(u >> 2) * xrow16);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            r.w[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, wo + (k0 >> 1), oob + (uint32_t)j * wfrag, 2);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            r.s[j] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff, oob + (uint32_t)j * sfrag, 0);
    };

    const _Float16 zlo = (_Float16)(1024.0f + a.zero_value), zhi = (_Float16)(64.0f + a.zero_value);
    const h2 zz_lo = {zlo, zlo}, zz_hi = {zhi, zhi};
    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));

    f4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const SkinnyW<FN>& r, const uint8_t* __restrict__ src) {
        h2 ss[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const _Float16 sc = bits_h((uint16_t)r.s[j]);
            ss[j] = (h2){sc, sc};
        }
        // The step's activation fragments for all four MFMA columns (kk), read ahead of the math.
        constexpr int XA = 4;
        uint4 xv[XA][FM];
        auto xread = [&](int kk) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
                xv[kk % XA][i] = *reinterpret_cast<const uint4*>(src + 256 * (16 * i + c) + 16 * ((4 * g + kk) ^ c));
        };
#pragma unroll
        for (int kk = 0; kk < XA; ++kk) xread(kk);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            h8 bw[FN], ax[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint4 u = perm8(xv[kk % XA][i]);
                ax[i] = *reinterpret_cast<const h8*>(&u);
            }
            if (kk + XA < 4) xread(kk + XA);
            auto dequant = [&](int j) {
                const uint32_t d = r.w[j][kk], d8 = d >> 8;
                const h2 q0 = bits_h2((d & 0x000F000Fu) | mag_lo);
                const h2 q1 = bits_h2((d & 0x00F000F0u) | mag_hi);
                const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo);
                const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi);
                const uint4 u = make_uint4(h2_bits((q0 - zz_lo) * ss[j]), h2_bits((q1 - zz_hi) * ss[j]),
                                           h2_bits((q2 - zz_lo) * ss[j]), h2_bits((q3 - zz_hi) * ss[j]));
                bw[j] = *reinterpret_cast<const h8*>(&u);
            };
#pragma unroll
            for (int j = 0; j < FN; ++j) dequant(j);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax[i], bw[j], acc[i][j], 0, 0, 0);
        }
    };

    // Two register sets and two LDS buffers: the loads of the wave's next step are in flight while
    // this one computes. The scheduling barriers keep each step's loads ahead of its math in issue
    // order; the wait leaves exactly the next step's loads in flight, so this step's activations
    // have landed in LDS (the compiler cannot see that dependence) and its weights and scales are
    // in registers.
    SkinnyW<FN> ra, rb;
    load(ra, xbuf, 0);
    auto step = [&](int t, const SkinnyW<FN>& cur, SkinnyW<FN>& nxt, const uint8_t* __restrict__ xcur,
                    uint8_t* __restrict__ xnxt) {
        __builtin_amdgcn_sched_barrier(0);
        load(nxt, xnxt, t + 1);
        wait_vmcnt<XDMA + 2 * FN>();
        __builtin_amdgcn_sched_barrier(0);
        compute(cur, xcur);
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int t = 0; t < nt; t += 2) {
        step(t, ra, rb, xbuf, xbuf + XBUF);
        if (t + 1 >= nt) break;
        step(t + 1, rb, ra, xbuf + XBUF, xbuf);
    }

    // Partial tiles of the four waves -> LDS (over the activation buffers, once every wave is done
    // with them and every direct load has landed) -> sum in wave order -> y or the split-K partials.
    wait_vmcnt<0>();
    __syncthreads();
    constexpr int P = out_pitch(FN), TN = 16 * FN;
    float* red = reinterpret_cast<float*>(lds);  // [4 waves][BM rows][P]
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(wid * BM + 16 * i + 4 * g + r) * P + 16 * j + c] = acc[i][j][r];
    __syncthreads();
    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
    const bool vec = out8_vector_ok<YT>(a, part);
    // chunk u of 8 outputs: row u / (TN / 8), columns 8 (u % (TN / 8))
    for (int u = threadIdx.x; u < BM * TN / 8; u += 256) {
        const int row = u / (TN / 8), col = (u % (TN / 8)) * 8;
        const float* src = red + row * P + col;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            const float4 s0 = *reinterpret_cast<const float4*>(src + e);
            const float4 s1 = *reinterpret_cast<const float4*>(src + BM * P + e);
            const float4 s2 = *reinterpret_cast<const float4*>(src + 2 * BM * P + e);
            const float4 s3 = *reinterpret_cast<const float4*>(src + 3 * BM * P + e);
            v[e] = s0.x + s1.x + s2.x + s3.x;
            v[e + 1] = s0.y + s1.y + s2.y + s3.y;
            v[e + 2] = s0.z + s1.z + s2.z + s3.z;
            v[e + 3] = s0.w + s1.w + s2.w + s3.w;
        }
        if (m0 + row < a.M) store_out8<YT>(a, part, vec, m0 + row, n0 + col, v);
    }
}

// Wide Q4 GEMM for prefill shapes whose 64 x 128 tiles alone fill the CUs, on the weights' prefill
// copy (byhip_q4w::wpf, spf). Eight waves, two per SIMD.
//   Block: waves w and w + 4 (one SIMD) form group p = w % 4, which takes the block's K sub-steps
//   p, p + 4, ... (64 values each); wave w of the group owns columns 64 h .. 64 h + 63 (h = w / 4)
//   and all 64 rows, as 4 x 4 fragments of v_mfma_f32_16x16x32_f16 (64 accumulators per lane).
//   K order: in MFMA kk (0, 1) of a sub-step, lane group g supplies the values 16 g + 8 kk .. + 7 in
//   natural order, for the weights (the prefill copy's nibble order makes one AND-OR against the
//   exponent words yield them so) and the activations alike: no permutation.
//   Weights: per fragment and sub-step a lane's 16 nibbles are 8 contiguous bytes of a 512-byte
//   block, so a load touches whole lines; its four fragments' scales are one 8-byte load.
//   Activations: the group's sub-step slice (64 rows x 128 bytes, one line per row) moves straight
//   from global memory into LDS, each wave of the group loading 32 rows, 16-byte chunk k of row r
//   at slot k ^ x_swizzle(r), so the fragment reads (16 rows, one chunk each) are free of bank
//   conflicts. D buffers per group (wide_depth).
//   Sub-step t of a group runs in two halves around one block barrier: the kk = 0 MFMAs beside
//   the fragment reads of t's kk = 1 activations, the dequantization of t's kk = 1 weights and the
//   loads of t + D - 1 (weights into the register set t - 1 finished with, activations into buffer
//   (t - 1) % D, whose reads of t - 1 all returned before the previous barrier); the wait for this
//   wave's loads of t + 1 and the barrier (which publishes every wave's direct loads of t + 1); the
//   kk = 1 MFMAs beside the fragment reads of t + 1's kk = 0 activations and the dequantization of
//   t + 1's kk = 0 weights. The dequantization VALU work thus runs between MFMAs of the same wave
//   (interleaved by scheduling groups), and loads have D - 1.5 sub-steps to land. With the
//   loads of a sub-step split over both halves and all fragment reads in the second, the kernel was
//   6 % slower at K = 14336. Every group runs the same number of sub-steps (the barrier needs the same
//   count in every wave), the largest group's; a sub-step past a group's last reads zeros through
//   an out-of-range offset and adds nothing. The last D - 1 sub-steps issue no loads (their waits
//   count down instead).
//   Tile order: with the tile count a multiple of 8, the workgroups that share an XCD (every 8th
//   workgroup id) take a contiguous run of tiles in groups of 4 row tiles, so each XCD's L2 holds
//   the activations of 4 row tiles and the weights of the column tiles it needs, rather than
//   every row tile's activations.
//   Output: the groups' partial tiles go to LDS in output layout (rows of 132 floats, so the
//   accumulator writes hit 64 distinct banks), and each thread adds 8 neighbouring outputs in
//   group order (0 + 1 + 2 + 3) and writes them with 16-byte stores.
constexpr int kWideBN = 128;
constexpr int kWideSub = 64;                         // K values per sub-step
constexpr int kWidePitch = out_pitch(kWideBN / 16);  // floats per row of a staged partial tile

// Operands of the wide tile: fp16 activations and weights rounded once to fp16 (kWideHalf); fp32
// activations as a high and a low fp16 plane and the weights as two fp16 terms that add up to them
// exactly (kWideF32); fp16 activations and the weights' two terms (kWideExactW).
enum WideKind { kWideHalf = 1, kWideF32 = 2, kWideExactW = 3 };
__host__ __device__ constexpr int wide_xplanes(int v) { return v == kWideF32 ? 2 : 1; }
__host__ __device__ constexpr int wide_wplanes(int v) { return v == kWideHalf ? 1 : 2; }

// Sizes for FM row fragments (BM = 16 FM rows: 64 for prefill, 32 or 16 for small M), D
// activation buffers per group (loads D - 1 sub-steps ahead) and operand kind V.
template <int FM, int D, int V = kWideHalf>
struct WideShape {
    static constexpr int XS = wide_xplanes(V);
    static constexpr int kBM = 16 * FM;
    static constexpr int kXBuf = XS * kBM * kWideSub * 2;     // one activation buffer (all planes)
    static constexpr int kLoads = XS * FM + 4 + 1;            // loads per wave and sub-step
    static constexpr int kLdsX = 4 * D * kXBuf;               // 4 groups x D buffers
    static constexpr int kLdsRed = 4 * kBM * kWidePitch * 4;  // 4 partial tiles
    static constexpr int kLds = kLdsX > kLdsRed ? kLdsX : kLdsRed;
};
// Pipeline depth (activation buffers per group): four at every tile height. Deeper pipelines were
// slower at 32 rows (c4's M = 32 gate+up: 17.1 us with four buffers, 18.8 with five or six, 19.6
// with eight; qkv 10.0, 10.7, 11.2, 12.1).
constexpr int wide_depth(int) { return 4; }

// One wave's prefill-copy operands of one sub-step: per fragment 16 nibbles (two words), and the
// four fragments' fp16 scales.
struct WideW {
    v2u w[4];
    v2u s;
};

// A sub-step's kind: whether it issues the loads of the sub-step a pipeline depth minus one ahead,
// how many of this wave's loads may stay in flight at its mid-step wait, and whether it may lie
// past the last sub-step (then it only waits and syncs).
template <bool L, int W, bool G = false>
struct WideStep {
    static constexpr bool load = L;
    static constexpr int wait = W;
    static constexpr bool guard = G;
};

template <int FM, int YT, int D = wide_depth(FM), int V = kWideHalf>
__global__ __launch_bounds__(512, 1) void q4_gemm_wide(GemmArgs a) {
    static_assert(FM == 1 || FM == 2 || FM == 4, "q4_gemm_wide: 16, 32 or 64 rows");
    constexpr int XS = wide_xplanes(V), WS = wide_wplanes(V);  // activation and weight planes
    static_assert(V == kWideHalf || FM <= 2, "q4_gemm_wide: two operand planes up to 32 rows");
    constexpr int FN = 4;
    using S = WideShape<FM, D, V>;
    constexpr int BM = S::kBM, kXBuf = S::kXBuf, kLoads = S::kLoads;
    static_assert(D >= 4 && S::kLds <= 160 * 1024 && (D - 2) * kLoads <= 63,
                  "q4_gemm_wide: the buffers must fit LDS and the loads in flight the wait counter");
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLds];

    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p = wid & 3, h = wid >> 2;
    const int c = lane & 15, g = lane >> 4;
    int bx = blockIdx.x, by = blockIdx.y;
    {
        const int gx = gridDim.x, gy = gridDim.y, tiles = gx * gy, id = bx + gx * by;
        const int j = tiles % 8 == 0 ? (id % 8) * (tiles / 8) + id / 8 : id;
        const int grp = j / (4 * gx), rows = min(4, gy - 4 * grp), r = j % (4 * gx);
        by = 4 * grp + r % rows;
        bx = r / rows;
    }
    const int n0 = bx * kWideBN, m0 = by * BM;
    const int K = a.K;
    const uint32_t nsub_all = (uint32_t)K / kWideSub;
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nsub = a.part ? min(a.split_steps, (int)nsub_all - s_first) : (int)nsub_all;  // the block's
    const int nt_all = (nsub + 3) / 4;                     // sub-steps every group runs
    const int nt = nsub > p ? (nsub - p + 3) / 4 : 0;     // the group's own sub-steps

    // Rows past M and columns past N read zeros through the range checks (the launcher keeps the
    // offsets below 2^31; the prefill copy pads N to whole fragments).
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.M * K * 2));
    const rsrc_t xlr = make_rsrc(XS == 2 ? a.x_lo : a.x, XS == 2 ? (uint32_t)((size_t)a.M * K * 2) : 0u);
    const rsrc_t wr = make_rsrc(a.wpf, (uint32_t)(((size_t)a.N + 15) / 16 * nsub_all * 512));
    const rsrc_t sr = make_rsrc(a.spf, (uint32_t)(((size_t)a.N + 63) / 64 * nsub_all * 256));
    // Direct load q (0 .. FM - 1) of wave h: rows 8 FM h + 8 q + lane / 8 of the tile, LDS slot
    // lane % 8 (with two planes, the low plane's rows follow the high plane's in the buffer).
    uint32_t xo[FM];
#pragma unroll
    for (int q = 0; q < FM; ++q) {
        const int r = 8 * FM * h + 8 * q + (lane >> 3), chunk = (lane & 7) ^ x_swizzle(r);
        xo[q] = (uint32_t)(m0 + r) * (uint32_t)K * 2u + 16u * chunk;
    }
    const uint32_t wfrag = nsub_all * 512u;  // per fragment
    const uint32_t wo = (uint32_t)(n0 + 64 * h) / 16u * wfrag + 8u * lane;
    const uint32_t so = (uint32_t)(n0 + 64 * h) / 64u * nsub_all * 256u + 8u * (16u * (uint32_t)(g >> 1) + c);
    uint8_t* const xgrp = lds + p * D * kXBuf;  // the group's buffers
    // Fragment reads: lane (c, g) reads row 16 i + c, chunk 2 g + kk, at slot
    // (2 g + kk) ^ x_swizzle(c) (x_swizzle(16 i + c) is x_swizzle(c)): one lane offset per kk, the
    // fragment a constant 2048 i.
    const int rd0 = 128 * c + 16 * ((2 * g) ^ x_swizzle(c)), rd1 = 128 * c + 16 * ((2 * g + 1) ^ x_swizzle(c));

    // The loads of the group's sub-step t (block sub-step p + 4 t): its activations into buffer t % D
    // (FM direct loads), its weights and scales into a register set (5 loads); the sub-step's offset
    // goes in the scalar offset. A sub-step past the group's last (t >= nt) adds 2^31 there, which
    // every resource rejects: it reads zeros without touching memory.
    // The lambdas are always inlined: left to the inliner, the 32-row tile on two activation
    // planes kept its operand arrays in scratch memory.
    // Buffer indices are compile-time constants at every call (t % D in the unrolled loop): the
    // compiler then sees that reads of one buffer do not alias direct loads into another and waits
    // for no direct load before them (with a run-time index it waited for nearly all in flight).
    auto load_x = [&](int t, int buf) __attribute__((always_inline)) {
        const bool ok = t < nt;
        const uint32_t u = (uint32_t)(s_first + (ok ? p + 4 * t : 0));
        const uint32_t oob = ok ? 0u : 0x80000000u;
        uint8_t* const dst = xgrp + buf * kXBuf;
#pragma unroll
        for (int q = 0; q < FM; ++q) lds_dma16(xr, dst + 1024 * (FM * h + q), xo[q], oob + 128u * u);
        if constexpr (XS == 2) {
#pragma unroll
            for (int q = 0; q < FM; ++q) lds_dma16(xlr, dst + 128 * BM + 1024 * (FM * h + q), xo[q], oob + 128u * u);
        }
    };
    auto load_ws = [&](WideW& r, int t) __attribute__((always_inline)) {
        const bool ok = t < nt;
        const uint32_t u = (uint32_t)(s_first + (ok ? p + 4 * t : 0));
        const uint32_t oob = ok ? 0u : 0x80000000u;
#pragma unroll
        for (int j = 0; j < FN; ++j)
            r.w[j] = __builtin_amdgcn_raw_buffer_load_b64(wr, wo, oob + 512u * u + (uint32_t)j * wfrag, 0);
        r.s = __builtin_amdgcn_raw_buffer_load_b64(sr, so, oob + 256u * u, 0);
    };

    const _Float16 zlo = (_Float16)(1024.0f + a.zero_value), zhi = (_Float16)(64.0f + a.zero_value);
    const h2 zz_lo = {zlo, zlo}, zz_hi = {zhi, zhi};
    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));

    f4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    // Weights of MFMA kk of a sub-step: (q - zero) * scale in fp16, exact in the subtraction. With
    // two weight planes also the weight's low term: the product (q - zero) * scale has at most
    // 15 significant bits, so hi = fp16 of it (one rounding) and lo = fma(q - zero, scale, -hi),
    // which an fp16 holds exactly, add up to it: plane [1] of bw.
    auto dequant = [&](const WideW& r, int kk, h8 (&bw)[WS][FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const _Float16 sc = bits_h((uint16_t)(r.s[j >> 1] >> (16 * (j & 1))));
            const h2 ss = {sc, sc};
            const uint32_t d = r.w[j][kk], d8 = d >> 8;
            const h2 q0 = bits_h2((d & 0x000F000Fu) | mag_lo) - zz_lo;
            const h2 q1 = bits_h2((d & 0x00F000F0u) | mag_hi) - zz_hi;
            const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo) - zz_lo;
            const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi) - zz_hi;
            const h2 w0 = q0 * ss, w1 = q1 * ss, w2 = q2 * ss, w3 = q3 * ss;
            const uint4 u = make_uint4(h2_bits(w0), h2_bits(w1), h2_bits(w2), h2_bits(w3));
            bw[0][j] = *reinterpret_cast<const h8*>(&u);
            if constexpr (WS == 2) {
                const uint4 l = make_uint4(h2_bits(__builtin_elementwise_fma(q0, ss, -w0)),
                                           h2_bits(__builtin_elementwise_fma(q1, ss, -w1)),
                                           h2_bits(__builtin_elementwise_fma(q2, ss, -w2)),
                                           h2_bits(__builtin_elementwise_fma(q3, ss, -w3)));
                bw[WS - 1][j] = *reinterpret_cast<const h8*>(&l);
            }
        }
    };
    // The kk half of the activation fragments in buffer buf (plane [1]: the low plane).
    auto read_x = [&](int buf, int kk, h8 (&x)[XS][FM]) __attribute__((always_inline)) {
        const uint8_t* src = xgrp + buf * kXBuf + (kk ? rd1 : rd0);
#pragma unroll
        for (int i = 0; i < FM; ++i) x[0][i] = *reinterpret_cast<const h8*>(src + 2048 * i);
        if constexpr (XS == 2) {
#pragma unroll
            for (int i = 0; i < FM; ++i) x[XS - 1][i] = *reinterpret_cast<const h8*>(src + 128 * BM + 2048 * i);
        }
    };
    // x . w, with two activation planes also x_lo . w_hi, with two weight planes also x_hi . w_lo
    // (x_lo . w_lo is below fp32's resolution of the sum).
    auto mfmas = [&](const h8 (&x)[XS][FM], const h8 (&b)[WS][FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[0][i], b[0][j], acc[i][j], 0, 0, 0);
                if constexpr (XS == 2)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[XS - 1][i], b[0][j], acc[i][j], 0, 0, 0);
                if constexpr (WS == 2)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[0][i], b[WS - 1][j], acc[i][j], 0, 0, 0);
            }
    };

    // Sub-steps 0 .. D - 2 are loaded here (activations, then weights), sub-step t + D - 1 in
    // sub-step t.
    WideW rs[D];
    h8 ax0[XS][FM], ax1[XS][FM], bw0[WS][FN], bw1[WS][FN];
    static_for<D - 1>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        load_x(k, k);
        load_ws(rs[k], k);
    });
    wait_vmcnt<(D - 2) * kLoads>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read_x(0, 0, ax0);
    dequant(rs[0], 0, bw0);

    // Sub-step t = base + k (base a multiple of D) with register sets rs[k] (t's operands),
    // rs[k + 1] (t + 1's) and rs[k - 1] (refilled with t + D - 1's weights, once t's last fragments
    // are dequantized), all indices mod D; t + D - 1's activations go to buffer k - 1, which every
    // wave's reads of t - 1 freed before the previous barrier. At the mid-step wait the loads of
    // t + 2 .. t + D - 1 may stay in flight, those that were issued.
    constexpr int kMfmas = (XS + WS - 1) * FM * FN;                                 // per K half
    constexpr int kValuPerMfma = (FN * (WS == 2 ? 18 : 14) + kMfmas - 1) / kMfmas;  // a K half's dequantization
    auto step = [&](int t, auto kc, auto kind) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value, k1 = (k + 1) % D, kp = (k + D - 1) % D;
        constexpr int kWait = decltype(kind)::wait;
        const bool live = !decltype(kind)::guard || t < nt_all;
        __builtin_amdgcn_sched_barrier(0);
        if (live) {
            mfmas(ax0, bw0);
            read_x(k, 1, ax1);
            dequant(rs[k], 1, bw1);
            if constexpr (decltype(kind)::load) {
                load_ws(rs[kp], t + D - 1);
                load_x(t + D - 1, kp);
            }
#pragma unroll
            for (int m = 0; m < kMfmas; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                        // one MFMA
                if (m < XS * FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);       // a fragment read
                if (m < kLoads) __builtin_amdgcn_sched_group_barrier(0x0010, 1, 0);        // a load
                __builtin_amdgcn_sched_group_barrier(0x0002, kValuPerMfma, 0);             // its share of the VALU
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kWait>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (live) {
            mfmas(ax1, bw1);
            read_x(k1, 0, ax0);
            dequant(rs[k1], 0, bw0);
#pragma unroll
            for (int m = 0; m < kMfmas; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                  // one MFMA
                if (m < XS * FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0); // a fragment read
                __builtin_amdgcn_sched_group_barrier(0x0002, kValuPerMfma, 0);       // its share of the VALU
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // D sub-steps per iteration and no exit between them (an exit there made the register
    // allocator keep extra copies of the accumulators and spill). Of the last D only the first
    // issues loads (the weights of the last sub-step); the loads of the sub-steps up to D - 1 past
    // them are in flight (those past nt_all read zeros), and their waits count down; the ones past
    // nt_all only wait and sync.
    int t = 0;
    for (; t + D < nt_all; t += D)
        static_for<D>([&](auto kc) { step(t + decltype(kc)::value, kc, WideStep<true, (D - 2) * kLoads>{}); });
    static_for<D>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        step(t + k, kc, WideStep<k == 0, (D - 2 - k > 0 ? D - 2 - k : 0) * kLoads, (k > 0)>{});
    });

    // Partial tiles -> LDS in output layout, once every wave's loads have landed (the last ones
    // read zeros into the buffers) and every wave is done with the activation buffers -> sums in
    // group order -> y or the split-K partials.
    wait_vmcnt<0>();
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);  // [4 groups][BM rows][kWidePitch]
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                red[(p * BM + 16 * i + 4 * g + r) * kWidePitch + 64 * h + 16 * j + c] = acc[i][j][r];
    __syncthreads();
    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
    const bool vec = out8_vector_ok<YT>(a, part);
#pragma unroll
    for (int k = 0; k < (BM * 16 + 511) / 512; ++k) {
        const int u = (int)threadIdx.x + 512 * k;  // chunk of 8 outputs: row u / 16, columns 8 (u % 16)
        if (BM * 16 < 512 && u >= BM * 16) break;
        const int row = u >> 4, col = (u & 15) * 8;
        const int m = m0 + row, n = n0 + col;
        float v[8];
        const float* src = red + row * kWidePitch + col;
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            const float4 s0 = *reinterpret_cast<const float4*>(src + e);
            const float4 s1 = *reinterpret_cast<const float4*>(src + BM * kWidePitch + e);
            const float4 s2 = *reinterpret_cast<const float4*>(src + 2 * BM * kWidePitch + e);
            const float4 s3 = *reinterpret_cast<const float4*>(src + 3 * BM * kWidePitch + e);
            v[e] = s0.x + s1.x + s2.x + s3.x;
            v[e + 1] = s0.y + s1.y + s2.y + s3.y;
            v[e + 2] = s0.z + s1.z + s2.z + s3.z;
            v[e + 3] = s0.w + s1.w + s2.w + s3.w;
        }
        if (m < a.M) {
            if constexpr (XS == 2) {  // fp32 activations: undo the row's power-of-two shift
                const int sh = a.row_shift[m];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = __builtin_amdgcn_ldexpf(v[e], -sh);
            }
            store_out8<YT>(a, part, vec, m, n, v);
        }
    }
}

// Tall Q4 GEMM for large prefill shapes: a 128 x 256 tile per block on the prefill copy, so that
// each activation byte reaches the CU once per 256 columns and each weight byte once per 128 rows
// (about half the operand bytes per output of the 64 x 128 wide tile).
//   Block: eight waves, two per SIMD; wave w owns columns 32 w .. 32 w + 31 (2 fragments) and all
//   128 rows (8 fragments), 64 accumulators; every wave runs every 64-value sub-step, so each
//   dequantized fragment feeds 8 MFMAs (about 2 VALU per MFMA) and each activation fragment read
//   from LDS feeds 2.
//   Operands as in the wide tile: natural K order from the copy's nibble order; a wave's weights
//   for a sub-step are two 8-byte loads and its 2 fragments' scales one 4-byte load; the block's
//   activation slice (128 rows x 128 bytes, 16 KB) moves straight into LDS, each wave loading 16
//   rows, XOR-swizzled as in the wide tile. Four buffers.
//   Sub-step t runs in two halves around one block barrier, as in the wide tile: the kk = 0 MFMAs
//   beside the fragment reads of t's kk = 1 activations, the dequantization of t's kk = 1 weights
//   and the loads of t + 3; the wait for this wave's loads of t + 1 and the barrier; the kk = 1
//   MFMAs beside the reads of t + 1's kk = 0 activations and the dequantization of t + 1's kk = 0
//   weights. Of the last four sub-steps only the first issues loads, and those past the last only
//   wait and sync. (Six or eight buffers, loads five or seven sub-steps ahead: no faster.)
//   Output: each wave stages its 128 x 32 block in LDS (rows of 36 floats: the accumulator writes
//   hit 64 distinct banks) and writes it as 16-byte stores of 8 outputs; no cross-wave sums.
//   Split-K: block z covers the sub-steps [z * split_steps, ...) and writes fp32 partials.
constexpr int kTallBM = 128, kTallBN = 256;
constexpr int kTallXBuf = kTallBM * kWideSub * 2;           // one activation buffer (16 KB)
constexpr int kTallLoads = 2 + 2 + 1;                       // loads per wave and sub-step
constexpr int kTallPitch = 32 + 4;                          // floats per row of a wave's staged block
constexpr int kTallLdsOut = 8 * kTallBM * kTallPitch * 4;  // the eight waves' staged blocks
constexpr int kTallDepth = 4;                               // activation buffers and operand sets
constexpr int tall_lds(int depth) { return depth * kTallXBuf > kTallLdsOut ? depth * kTallXBuf : kTallLdsOut; }

// One wave's prefill-copy operands of one sub-step: per fragment 16 nibbles (two words), and the
// two fragments' fp16 scales.
struct TallW {
    v2u w[2];
    uint32_t s;
};

template <int YT, int D = kTallDepth>
__global__ __launch_bounds__(512, 1) void q4_gemm_tall(GemmArgs a) {
    static_assert(D >= 3 && D * kTallXBuf <= 160 * 1024, "q4_gemm_tall: 3 to 10 buffers");
    constexpr int FM = 8, FN = 2;
    __shared__ __attribute__((aligned(16))) uint8_t lds[tall_lds(D)];

    const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    int bx = blockIdx.x, by = blockIdx.y;
    {
        // the wide tile's XCD-grouped tile order
        const int gx = gridDim.x, gy = gridDim.y, tiles = gx * gy, id = bx + gx * by;
        const int j = tiles % 8 == 0 ? (id % 8) * (tiles / 8) + id / 8 : id;
        const int grp = j / (4 * gx), rows = min(4, gy - 4 * grp), r = j % (4 * gx);
        by = 4 * grp + r % rows;
        bx = r / rows;
    }
    const int n0 = bx * kTallBN, m0 = by * kTallBM, col0 = n0 + 32 * wid;
    const int K = a.K;
    const uint32_t nsub_all = (uint32_t)K / kWideSub;
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nt = a.part ? min(a.split_steps, (int)nsub_all - s_first) : (int)nsub_all;  // the block's sub-steps

    // Rows past M and columns past N read zeros through the range checks (the launcher keeps the
    // offsets below 2^31; the prefill copy pads N to whole fragments).
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.M * K * 2));
    const rsrc_t wr = make_rsrc(a.wpf, (uint32_t)(((size_t)a.N + 15) / 16 * nsub_all * 512));
    const rsrc_t sr = make_rsrc(a.spf, (uint32_t)(((size_t)a.N + 63) / 64 * nsub_all * 256));
    // Direct load q (0, 1) of wave w: rows 16 w + 8 q + lane / 8 of the tile, LDS slot lane % 8.
    uint32_t xo[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 16 * wid + 8 * q + (lane >> 3), chunk = (lane & 7) ^ x_swizzle(r);
        xo[q] = (uint32_t)(m0 + r) * (uint32_t)K * 2u + 16u * chunk;
    }
    const uint32_t wfrag = nsub_all * 512u;  // per fragment
    const uint32_t wo = (uint32_t)col0 / 16u * wfrag + 8u * lane;
    // the wave's 2 fragments are fragments 2 (w % 2) and 2 (w % 2) + 1 of their quad
    const uint32_t so = (uint32_t)col0 / 64u * nsub_all * 256u + 8u * (16u * (uint32_t)(g >> 1) + c) + 4u * (wid & 1);
    const int rd0 = 128 * c + 16 * ((2 * g) ^ x_swizzle(c)), rd1 = 128 * c + 16 * ((2 * g + 1) ^ x_swizzle(c));

    // Loads of sub-step t (the sub-step's offset in the scalar offset; past the last, 2^31 there
    // reads zeros): its activations into buffer t % D, its weights and scales into a register set.
    auto load_x = [&](int t, int buf) {
        const bool ok = t < nt;
        const uint32_t u = (uint32_t)(s_first + (ok ? t : 0));
        const uint32_t oob = ok ? 0u : 0x80000000u;
        uint8_t* const dst = lds + buf * kTallXBuf;
#pragma unroll
        for (int q = 0; q < 2; ++q) lds_dma16(xr, dst + 1024 * (2 * wid + q), xo[q], oob + 128u * u);
    };
    auto load_ws = [&](TallW& r, int t) {
        const bool ok = t < nt;
        const uint32_t u = (uint32_t)(s_first + (ok ? t : 0));
        const uint32_t oob = ok ? 0u : 0x80000000u;
#pragma unroll
        for (int j = 0; j < FN; ++j)
            r.w[j] = __builtin_amdgcn_raw_buffer_load_b64(wr, wo, oob + 512u * u + (uint32_t)j * wfrag, 0);
        r.s = __builtin_amdgcn_raw_buffer_load_b32(sr, so, oob + 256u * u, 0);
    };

    const _Float16 zlo = (_Float16)(1024.0f + a.zero_value), zhi = (_Float16)(64.0f + a.zero_value);
    const h2 zz_lo = {zlo, zlo}, zz_hi = {zhi, zhi};
    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));

    f4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    // Weights of MFMA kk of a sub-step: (q - zero) * scale in fp16, exact in the subtraction.
    auto dequant = [&](const TallW& r, int kk, h8 (&bw)[FN]) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const _Float16 sc = bits_h((uint16_t)(r.s >> (16 * j)));
            const h2 ss = {sc, sc};
            const uint32_t d = r.w[j][kk], d8 = d >> 8;
            const h2 q0 = bits_h2((d & 0x000F000Fu) | mag_lo);
            const h2 q1 = bits_h2((d & 0x00F000F0u) | mag_hi);
            const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo);
            const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi);
            const uint4 u = make_uint4(h2_bits((q0 - zz_lo) * ss), h2_bits((q1 - zz_hi) * ss),
                                       h2_bits((q2 - zz_lo) * ss), h2_bits((q3 - zz_hi) * ss));
            bw[j] = *reinterpret_cast<const h8*>(&u);
        }
    };
    // The kk half of the activation fragments in buffer buf.
    auto read_x = [&](int buf, int kk, h8 (&x)[FM]) {
        const uint8_t* src = lds + buf * kTallXBuf + (kk ? rd1 : rd0);
#pragma unroll
        for (int i = 0; i < FM; ++i) x[i] = *reinterpret_cast<const h8*>(src + 2048 * i);
    };
    auto mfmas = [&](const h8 (&x)[FM], const h8 (&b)[FN]) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[i], b[j], acc[i][j], 0, 0, 0);
    };

    // Sub-steps 0 .. D - 2 are loaded here (activations, then weights), sub-step t + D - 1 in
    // sub-step t.
    TallW rs[D];
    h8 ax0[FM], ax1[FM], bw0[FN], bw1[FN];
    static_for<D - 1>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        load_x(k, k);
        load_ws(rs[k], k);
    });
    wait_vmcnt<(D - 2) * kTallLoads>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read_x(0, 0, ax0);
    dequant(rs[0], 0, bw0);

    constexpr int kValuPerMfma = (FN * 14 + FM * FN - 1) / (FM * FN);  // a K half's dequantization
    // Sub-step t = base + k (base a multiple of D) with register sets rs[k] (t's operands),
    // rs[k + 1] (t + 1's) and rs[k - 1] (refilled with t + D - 1's weights), all indices mod D;
    // t + D - 1's activations go to buffer k - 1, which every wave's reads of t - 1 freed before the
    // previous barrier. At the mid-step wait the loads of t + 2 .. t + D - 1 may stay in flight,
    // those issued.
    auto step = [&](int t, auto kc, auto kind) {
        constexpr int k = decltype(kc)::value, k1 = (k + 1) % D, kp = (k + D - 1) % D;
        constexpr int kWait = decltype(kind)::wait;
        const bool live = !decltype(kind)::guard || t < nt;
        __builtin_amdgcn_sched_barrier(0);
        if (live) {
            mfmas(ax0, bw0);
            read_x(k, 1, ax1);
            dequant(rs[k], 1, bw1);
            if constexpr (decltype(kind)::load) {
                load_ws(rs[kp], t + D - 1);
                load_x(t + D - 1, kp);
            }
#pragma unroll
            for (int m = 0; m < FM * FN; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                       // one MFMA
                if (m < FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);           // a fragment read
                if (m < kTallLoads) __builtin_amdgcn_sched_group_barrier(0x0010, 1, 0);  // a load
                __builtin_amdgcn_sched_group_barrier(0x0002, kValuPerMfma, 0);            // its share of the VALU
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kWait>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (live) {
            mfmas(ax1, bw1);
            read_x(k1, 0, ax0);
            dequant(rs[k1], 0, bw0);
#pragma unroll
            for (int m = 0; m < FM * FN; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);               // one MFMA
                if (m < FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);   // a fragment read
                __builtin_amdgcn_sched_group_barrier(0x0002, kValuPerMfma, 0);    // its share of the VALU
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // D sub-steps per iteration, no exit between them; of the last D only the first issues loads
    // (the weights of the last sub-step), their waits count down, and the ones past nt only wait
    // and sync.
    int t = 0;
    for (; t + D < nt; t += D)
        static_for<D>([&](auto kc) { step(t + decltype(kc)::value, kc, WideStep<true, (D - 2) * kTallLoads>{}); });
    static_for<D>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        step(t + k, kc, WideStep<k == 0, (D - 2 - k > 0 ? D - 2 - k : 0) * kTallLoads, (k > 0)>{});
    });

    // Each wave's 128 x 32 block -> LDS (once every wave is done with the activation buffers and
    // every direct load has landed) -> 16-byte stores of 8 outputs (y or the split-K partials).
    wait_vmcnt<0>();
    __syncthreads();
    float* stage = reinterpret_cast<float*>(lds) + wid * kTallBM * kTallPitch;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) stage[(16 * i + 4 * g + r) * kTallPitch + 16 * j + c] = acc[i][j][r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
    const bool vec = out8_vector_ok<YT>(a, part);
#pragma unroll
    for (int k = 0; k < kTallBM * 4 / 64; ++k) {
        const int u = lane + 64 * k;  // chunk of 8 outputs: row u / 4, columns 8 (u % 4)
        const int row = u >> 2, col = (u & 3) * 8;
        const int m = m0 + row;
        float v[8];
        const float* src = stage + row * kTallPitch + col;
        const float4 s0 = *reinterpret_cast<const float4*>(src);
        const float4 s1 = *reinterpret_cast<const float4*>(src + 4);
        v[0] = s0.x; v[1] = s0.y; v[2] = s0.z; v[3] = s0.w;
        v[4] = s1.x; v[5] = s1.y; v[6] = s1.z; v[7] = s1.w;
        if (m < a.M) store_out8<YT>(a, part, vec, m, col0 + col, v);
    }
}

// Whether the pipelined Q4 kernel takes these arguments.
bool q4_pipe_ok(const GemmArgs& a) {
    const bool pow2_group = a.group % 32 == 0 && ((a.group >> 5) & ((a.group >> 5) - 1)) == 0;
    return a.x_dtype == BYHIP_F16 && a.K % PBK == 0 && a.scale_f16 && !a.zeros &&
           (a.group == 0 || pow2_group) && a.row_bytes % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && reinterpret_cast<uintptr_t>(a.wq) % 16 == 0 &&
           (uint64_t)(a.M + 64) * a.K * 2 < kOutOfRange && (uint64_t)(a.N + 128) * a.row_bytes < kOutOfRange &&
           (uint64_t)(a.N + 128) * a.gpr * 2 < kOutOfRange;
}

template <int BM, int FN>
void launch_q4_skinny_shape(const GemmArgs& a, int splits) {
    const dim3 grid((a.N + 16 * FN - 1) / (16 * FN), (a.M + BM - 1) / BM, splits);
    switch (a.y_dtype) {
    case BYHIP_F32: launch("q4_gemm_skinny", (q4_gemm_skinny<BM, FN, BYHIP_F32>), grid, dim3(256), 0, a); break;
    case BYHIP_F16: launch("q4_gemm_skinny", (q4_gemm_skinny<BM, FN, BYHIP_F16>), grid, dim3(256), 0, a); break;
    default: launch("q4_gemm_skinny", (q4_gemm_skinny<BM, FN, BYHIP_BF16>), grid, dim3(256), 0, a); break;
    }
    BYHIP_LAUNCHED("q4_gemm_skinny");
}

template <int FM, int V = kWideHalf>
void launch_q4_wide_shape(const GemmArgs& a, int splits) {
    const dim3 grid((a.N + kWideBN - 1) / kWideBN, (a.M + 16 * FM - 1) / (16 * FM), splits);
    constexpr int D = wide_depth(FM);
    switch (a.y_dtype) {
    case BYHIP_F32: launch("q4_gemm_wide", (q4_gemm_wide<FM, BYHIP_F32, D, V>), grid, dim3(512), 0, a); break;
    case BYHIP_F16: launch("q4_gemm_wide", (q4_gemm_wide<FM, BYHIP_F16, D, V>), grid, dim3(512), 0, a); break;
    default: launch("q4_gemm_wide", (q4_gemm_wide<FM, BYHIP_BF16, D, V>), grid, dim3(512), 0, a); break;
    }
    BYHIP_LAUNCHED("q4_gemm_wide");
}

// Rows per tile: 16 or 32 when M fits, else 64.
int wide_rows(int M) { return M <= 16 ? 16 : M <= 32 ? 32 : 64; }

void launch_q4_wide(const GemmArgs& a, int splits) {
    switch (wide_rows(a.M)) {
    case 16: launch_q4_wide_shape<1>(a, splits); break;
    case 32: launch_q4_wide_shape<2>(a, splits); break;
    default: launch_q4_wide_shape<4>(a, splits); break;
    }
}

template <int BM, int BN>
void launch_q4_pipe_shape(const GemmArgs& a, int splits) {
    const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, splits);
    switch (a.y_dtype) {
    case BYHIP_F32: launch("q4_gemm_pipe", (q4_gemm_pipe<BM, BN, BYHIP_F32>), grid, dim3(256), 0, a); break;
    case BYHIP_F16: launch("q4_gemm_pipe", (q4_gemm_pipe<BM, BN, BYHIP_F16>), grid, dim3(256), 0, a); break;
    default: launch("q4_gemm_pipe", (q4_gemm_pipe<BM, BN, BYHIP_BF16>), grid, dim3(256), 0, a); break;
    }
    BYHIP_LAUNCHED("q4_gemm_pipe");
}

}  // namespace

int choose_split(GemmArgs& a, long tiles, int nsteps, int min_steps, int forced, int per_cu) {
    const long cus = compute_units();
    long splits = forced > 0 ? forced : env_int("BYHIP_Q4_SPLIT", 0);
    if (splits < 1)
        splits = tiles >= cus ? 1 : std::min<long>((per_cu * cus + tiles - 1) / tiles, nsteps / min_steps);
    void* work = a.work ? a.work : workspace();
    const size_t work_bytes = a.work ? a.work_bytes : kWorkspaceBytes;
    const long fit = (long)(work_bytes / (splitk_stride(a.M, a.N) * sizeof(float)));
    splits = std::max<long>(1, std::min<long>({splits, (long)nsteps, fit}));
    if (splits == 1) return 1;
    a.split_steps = (int)((nsteps + splits - 1) / splits);
    a.part = static_cast<float*>(work);
    return (nsteps + a.split_steps - 1) / a.split_steps;  // no empty split
}

void launch_splitk_sum(const GemmArgs& a, int splits) {
    const size_t quads = ((size_t)a.M * a.N + 3) / 4;
    const dim3 grid((unsigned)((quads + 255) / 256));
    if (grid.x < (unsigned)compute_units()) {  // fp32 route M = 9 .. 32: 0.2-0.4 us faster
        const dim3 g1((unsigned)(((size_t)a.M * a.N + 255) / 256));
        switch (a.y_dtype) {
        case BYHIP_F32: launch("splitk_sum1", splitk_sum1<BYHIP_F32>, g1, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
        case BYHIP_F16: launch("splitk_sum1", splitk_sum1<BYHIP_F16>, g1, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
        default: launch("splitk_sum1", splitk_sum1<BYHIP_BF16>, g1, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
        }
        BYHIP_LAUNCHED("splitk_sum1");
        return;
    }
    switch (a.y_dtype) {
    case BYHIP_F32: launch("splitk_sum", splitk_sum<BYHIP_F32>, grid, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
    case BYHIP_F16: launch("splitk_sum", splitk_sum<BYHIP_F16>, grid, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
    default: launch("splitk_sum", splitk_sum<BYHIP_BF16>, grid, dim3(256), 0, a.part, splits, a.M, a.N, a.y, a.gate, a.gate_want); break;
    }
    BYHIP_LAUNCHED("splitk_sum");
}

namespace {

// Tile choice: 64 x 128, or 32 x 128 when M <= 32, split along K when the tiles leave CUs idle.
// BYHIP_Q4_TILE=1..4 forces 64x128, 64x64, 32x128, 32x64; a tuned plan passes tile / splits (0:
// the default choice).
void launch_q4_pipe(const GemmArgs& a0, int tile_choice = 0, int split_choice = 0) {
    GemmArgs a = a0;
    int tile = tile_choice > 0 ? tile_choice : env_int("BYHIP_Q4_TILE", 0);
    if (tile < 1 || tile > 4) tile = a.M <= 32 ? 3 : 1;
    const int bm = tile <= 2 ? 64 : 32, bn = tile % 2 ? 128 : 64;
    const long tiles = (long)((a.N + bn - 1) / bn) * ((a.M + bm - 1) / bm);
    const int splits = choose_split(a, tiles, a.K / PBK, 4, split_choice);
    switch (tile) {
    case 1: launch_q4_pipe_shape<64, 128>(a, splits); break;
    case 2: launch_q4_pipe_shape<64, 64>(a, splits); break;
    case 3: launch_q4_pipe_shape<32, 128>(a, splits); break;
    default: launch_q4_pipe_shape<32, 64>(a, splits); break;
    }
    if (a.part) launch_splitk_sum(a, splits);
}

// Whether the skinny kernel takes the call: the pipelined kernel's conditions, K % 128 == 0, all
// operand offsets below 2^31, and M up to 32 (BYHIP_Q4_SKINNY_MAX_M lowers the limit).
bool q4_skinny_ok(const GemmArgs& a) {
    constexpr uint64_t kLim = 0x80000000u;  // offsets stay below 2^31 (the kernel's out-of-range steps)
    return a.K % 128 == 0 && a.M <= std::min(32, env_int("BYHIP_Q4_SKINNY_MAX_M", 32)) && q4_pipe_ok(a) &&
           (uint64_t)(a.M + 64) * a.K * 2 < kLim && (uint64_t)(a.N + 64) * a.row_bytes < kLim &&
           (uint64_t)(a.N + 64) * a.gpr * 2 < kLim;
}

// Whether the wide tile takes the call: the weights' prefill copy (K % 64 == 0), the pipelined
// kernel's conditions and all operand offsets, including the rows and columns a tile reaches past
// M and N, below 2^31.
bool q4_wide_ok(const GemmArgs& a) {
    constexpr uint64_t kLim = 0x80000000u;
    return a.wpf && a.spf && a.K % kWideSub == 0 && q4_pipe_ok(a) && (uint64_t)(a.M + 64) * a.K * 2 < kLim &&
           (uint64_t)(a.N + 128) * a.row_bytes < kLim && (uint64_t)(a.N + 128) * a.gpr * 2 < kLim;
}

// Whether the 128 x 256 tile (the tall kernel) takes the call: the wide tile's conditions (the
// prefill copy among them), with the rows and columns a 128 x 256 tile reaches past M and N.
bool q4_big_ok(const GemmArgs& a) {
    constexpr uint64_t kLim = 0x80000000u;
    return q4_wide_ok(a) && (uint64_t)(a.M + kTallBM) * a.K * 2 < kLim && (uint64_t)(a.N + kTallBN) * a.row_bytes < kLim;
}

int q4_big_splits(const GemmArgs& a);

// The 128 x 256 tile (the tall kernel) with one block per CU, K split as q4_big_splits says (or
// `split_choice`).
void launch_q4_big(const GemmArgs& a0, int split_choice = 0) {
    GemmArgs a = a0;
    const long tiles = (long)((a.N + kTallBN - 1) / kTallBN) * ((a.M + kTallBM - 1) / kTallBM);
    const int forced = split_choice > 0 ? split_choice : q4_big_splits(a);
    const int splits = choose_split(a, tiles, a.K / kWideSub, 8, forced);
    const dim3 grid((a.N + kTallBN - 1) / kTallBN, (a.M + kTallBM - 1) / kTallBM, splits);
    switch (a.y_dtype) {
    case BYHIP_F32: launch("q4_gemm_tall", q4_gemm_tall<BYHIP_F32>, grid, dim3(512), 0, a); break;
    case BYHIP_F16: launch("q4_gemm_tall", q4_gemm_tall<BYHIP_F16>, grid, dim3(512), 0, a); break;
    default: launch("q4_gemm_tall", q4_gemm_tall<BYHIP_BF16>, grid, dim3(512), 0, a); break;
    }
    BYHIP_LAUNCHED("q4_gemm_tall");
    if (a.part) launch_splitk_sum(a, splits);
}

// K splits for the wide tile: the count that minimises the estimated time
// ceil(tiles * s / CUs) x (sub-steps per split + 16), the 16 standing for a block's fixed cost (its
// first loads' latency, the epilogue), with at least 8 sub-steps per split and each split a multiple
// of 4 sub-steps (one per group and round); fewer splits win unless more save over 3 %.
int wide_splits(const GemmArgs& a, long tiles) {
    const int nsub = a.K / kWideSub;
    const long cus = compute_units();
    int best = 1;
    double best_t = 1e300;
    for (int s = 1; s <= std::max(1, nsub / 8); ++s) {
        const int steps = ((nsub + s - 1) / s + 3) / 4 * 4;
        const int splits = (nsub + steps - 1) / steps;
        if (splits != s) continue;  // the same split as a smaller s
        const double t = (double)((tiles * s + cus - 1) / cus) * (steps + 16);
        if (t < 0.97 * best_t) {
            best = s;
            best_t = t;
        }
    }
    return best;
}

// Rows per block: 16 or 32 (the smallest that holds M) with 64 columns and two blocks per CU, or
// the wide tile (q4_gemm_wide: 128 columns, 16, 32 or 64 rows, eight waves) with one block per CU.
void launch_q4_skinny(const GemmArgs& a0, int split_choice = 0, bool wide = false) {
    GemmArgs a = a0;
    const int bm = wide ? wide_rows(a.M) : a.M <= 16 ? 16 : 32, cols = wide ? 128 : 64;
    const long tiles = (long)((a.N + cols - 1) / cols) * ((a.M + bm - 1) / bm);
    // the wide kernel counts 64-value sub-steps, the skinny one 128-value steps
    int splits;
    if (wide) {
        const int forced = split_choice > 0 ? split_choice : env_int("BYHIP_Q4_SPLIT", 0);
        splits = choose_split(a, tiles, a.K / kWideSub, 1, forced > 0 ? forced : wide_splits(a, tiles), 1);
        if (a.part) {
            // whole rounds of the four groups
            a.split_steps = (a.split_steps + 3) / 4 * 4;
            splits = (a.K / kWideSub + a.split_steps - 1) / a.split_steps;
        }
        if (splits == 1) a.part = nullptr;
    } else {
        splits = choose_split(a, tiles, a.K / 128, 8, split_choice, 2);
    }
    if (wide) launch_q4_wide(a, splits);
    else if (bm == 16) launch_q4_skinny_shape<16, 4>(a, splits);
    else launch_q4_skinny_shape<32, 4>(a, splits);
    if (a.part) launch_splitk_sum(a, splits);
}

// Whether a small-M call (the skinny kernel's range) takes the wide tile: when the weights have the
// prefill copy and the wide grid keeps at least 16 sub-steps per K split. Measured on MI355X (M = 9
// to 32, weights streamed from HBM): the wide tile is 8-30 % faster on K x N = 4096 x 6144,
// 4096 x 28672 and 14336 x 4096, and 15-25 % slower on 4096 x 4096, whose 32 column tiles need 8
// splits of 8 sub-steps.
bool q4_small_wide(const GemmArgs& a) {
    if (!q4_wide_ok(a)) return false;
    const long tiles = (long)((a.N + kWideBN - 1) / kWideBN) * ((a.M + wide_rows(a.M) - 1) / wide_rows(a.M));
    const int splits = wide_splits(a, tiles), nsub = a.K / kWideSub;
    return (nsub + splits - 1) / splits >= 16;
}

// Whether the wide tile takes a call with fp32 activations: the weights' prefill copy (its format
// conditions), K % 64 == 0, 16-byte aligned activation rows, and the operand offsets below 2^31.
bool q4_wide_f32_ok(const GemmArgs& a) {
    constexpr uint64_t kLim = 0x80000000u;
    return a.x_dtype == BYHIP_F32 && a.wpf && a.spf && a.K % kWideSub == 0 && a.scale_f16 && !a.zeros &&
           reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && (uint64_t)(a.M + 32) * a.K * 2 < kLim &&
           (uint64_t)(a.N + 128) * a.row_bytes < kLim && (uint64_t)(a.N + 128) * a.gpr * 2 < kLim;
}

// The 16- or 32-row wide tile with operand kind V (two weight planes) on a.x (and a.x_lo): K split
// as for the fp16 tile (whole rounds of the four K groups), then splitk_sum.
template <int V>
void launch_q4_wide_planes(GemmArgs a, int split_choice) {
    const int bm = a.M <= 16 ? 16 : 32;
    const long tiles = (long)((a.N + kWideBN - 1) / kWideBN) * ((a.M + bm - 1) / bm);
    const int forced = split_choice > 0 ? split_choice : env_int("BYHIP_Q4_SPLIT", 0);
    int splits = choose_split(a, tiles, a.K / kWideSub, 1, forced > 0 ? forced : wide_splits(a, tiles), 1);
    if (a.part) {
        a.split_steps = (a.split_steps + 3) / 4 * 4;
        splits = (a.K / kWideSub + a.split_steps - 1) / a.split_steps;
    }
    if (splits == 1) a.part = nullptr;
    if (bm == 16) launch_q4_wide_shape<1, V>(a, splits);
    else launch_q4_wide_shape<2, V>(a, splits);
    if (a.part) launch_splitk_sum(a, splits);
}

// The wide tile on fp32 activations: per row a power-of-two shift onto fp16's range and the shifted
// row as two fp16 planes (split_rows_f16, into the scratch), then the 16- or 32-row tile with three
// MFMAs per product (hi . w_hi + lo . w_hi + hi . w_lo), every fp32 weight and about 22 bits of
// each activation kept. False, queueing nothing, when the planes do not fit the scratch.
bool launch_q4_wide_f32(const GemmArgs& a0, int split_choice = 0) {
    GemmArgs a = a0;
    uint8_t* const work = static_cast<uint8_t*>(a.work ? a.work : workspace());
    const size_t work_bytes = a.work ? a.work_bytes : kWorkspaceBytes;
    const size_t shift_bytes = ((size_t)a.M * sizeof(int) + 255) / 256 * 256;
    const size_t plane = ((size_t)a.M * a.K * 2 + 255) / 256 * 256;
    if (shift_bytes + 2 * plane > work_bytes) return false;
    int* const shifts = reinterpret_cast<int*>(work);
    _Float16* const hi = reinterpret_cast<_Float16*>(work + shift_bytes);
    _Float16* const lo = reinterpret_cast<_Float16*>(work + shift_bytes + plane);
    launch("split_rows_f16", split_rows_f16, dim3((unsigned)a.M), dim3(256), 0, static_cast<const float*>(a.x), a.K,
                       shifts, hi, lo);
    BYHIP_LAUNCHED("split_rows_f16");
    a.x = hi;
    a.x_lo = lo;
    a.row_shift = shifts;
    a.work = work + shift_bytes + 2 * plane;
    a.work_bytes = work_bytes - shift_bytes - 2 * plane;
    launch_q4_wide_planes<kWideF32>(a, split_choice);
    return true;
}

// Splits launch_q4_big chooses: K is split when the tiles fill at most half the CUs, into as many
// slices as keep the grid within one block per CU (each slice at least 8 sub-steps).
int q4_big_splits(const GemmArgs& a) {
    const long tiles = (long)((a.N + kTallBN - 1) / kTallBN) * ((a.M + kTallBM - 1) / kTallBM);
    const int forced = env_int("BYHIP_Q4_SPLIT", 0);
    if (forced > 0) return forced;
    return (int)std::max<long>(1, std::min<long>(compute_units() / tiles, a.K / kWideSub / 8));
}

// The Q4 prefill kernel (M above the skinny kernel's range) for the benchmark format, from
// measurements on MI355X (c4's projections, weights streamed from HBM):
//   the 64 x 128 wide tile when its tiles alone fill the CUs while 128 x 256 tiles would leave
//   more than half of them idle (M = 512, N = K = 4096: 20.6 us against 31.0 for the 128 x 256
//   tile split 4 ways);
//   else, for M > 64, the 128 x 256 tile (the tall kernel), which reads about half the operand
//   bytes per output, unless the split-K it needs to fill the CUs moves partial sums (8 bytes per
//   output and split: written, then read) of more than 100 bytes per tile and K value. It wins on
//   gate+up (K = 4096, N = 28672) at M = 256 (no split: 55 against 80 us) and M = 512 (110
//   against 142), and loses at M = 256 on qkv (N = 6144: 26.7 against 17.7), o (26.4 against
//   20.4) and down (K = 14336: 41.6 against 36.6), and at M = 128 on all four; the wide tile also
//   takes M <= 64 (half-empty large tiles);
//   the pipelined kernel where neither takes the call (no prefill copy, offsets past 2^31).
// BYHIP_Q4_PREFILL forces one: 1 the pipelined kernel, 2 the 128 x 256 tile, 3 the wide tile,
// when it takes the call. Returns kQ4Pipe / kQ4Big / kQ4Wide, or 0 for the general kernel.
int q4_prefill_kind(const GemmArgs& a) {
    const int forced = env_int("BYHIP_Q4_PREFILL", 0);
    const bool big = q4_big_ok(a), wide = q4_wide_ok(a), pipe = q4_pipe_ok(a);
    if (forced == 1) return pipe ? kQ4Pipe : 0;
    if (forced == 2 && big) return kQ4Big;
    if (forced == 3 && wide) return kQ4Wide;
    const long cus = compute_units();
    const long big_tiles = (long)((a.N + kTallBN - 1) / kTallBN) * ((a.M + kTallBM - 1) / kTallBM);
    const long wide_tiles = (long)((a.N + 127) / 128) * ((a.M + 63) / 64);
    if (wide && wide_tiles >= cus && 2 * big_tiles < cus) return kQ4Wide;
    if (big && (a.M > 64 || !wide)) {
        const double splits = q4_big_splits(a);
        const double partial = splits > 1 ? 8.0 * a.M * a.N * splits : 0.0;
        if (!wide || partial <= 100.0 * big_tiles * a.K) return kQ4Big;
    }
    if (wide) return kQ4Wide;
    return pipe ? kQ4Pipe : 0;
}

template <BFormat F, bool XF32>
void launch_fx(const GemmArgs& a0) {
    // K split (fp32 partial sums, added by splitk_sum) when the tiles leave CUs idle: at M = 16,
    // K = N = 4096 the 32 tiles alone keep 32 of the 256 CUs busy
    GemmArgs a = a0;
    const long tiles = (long)((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
    const int splits = choose_split(a, tiles, (a.K + BK - 1) / BK, 8, 0, 1);
    const dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM, splits);
    switch (a.y_dtype) {
    case BYHIP_F32:
        launch("gemm_f16_mfma", (gemm_f16_mfma<F, XF32, BYHIP_F32>), grid, dim3(256), 0, a);
        break;
    case BYHIP_F16:
        launch("gemm_f16_mfma", (gemm_f16_mfma<F, XF32, BYHIP_F16>), grid, dim3(256), 0, a);
        break;
    default:
        launch("gemm_f16_mfma", (gemm_f16_mfma<F, XF32, BYHIP_BF16>), grid, dim3(256), 0, a);
        break;
    }
    BYHIP_LAUNCHED("gemm_f16_mfma");
    if (a.part) launch_splitk_sum(a, splits);
}

template <BFormat F>
void launch_f(const GemmArgs& a0) {
    if (a0.x_dtype != BYHIP_F32) {
        launch_fx<F, false>(a0);
        return;
    }
    // fp32 activations: the per-row shifts first, into the scratch
    GemmArgs a = a0;
    void* work = a.work ? a.work : workspace();
    const size_t work_bytes = a.work ? a.work_bytes : kWorkspaceBytes;
    if ((size_t)a.M * sizeof(int) > work_bytes) fail("byhip: M=%d rows of fp32 activations exceed the scratch", a.M);
    int* shifts = static_cast<int*>(work);
    launch("row_range_shift", row_range_shift, dim3((unsigned)a.M), dim3(256), 0, static_cast<const float*>(a.x), a.K,
                       shifts);
    BYHIP_LAUNCHED("row_range_shift");
    a.row_shift = shifts;
    // the split-K partial sums, if any, go after the shifts
    const size_t used = ((size_t)a.M * sizeof(int) + 255) / 256 * 256;
    a.work = static_cast<uint8_t*>(work) + used;
    a.work_bytes = work_bytes > used ? work_bytes - used : 0;
    launch_fx<F, true>(a);
}

}  // namespace

bool launch_q4_choice(BFormat fmt, const GemmArgs& a, int kind, int tile, int splits) {
    if (a.K % 32 != 0 || a.M <= 0 || a.N <= 0 || a.M > 65535 * BM) return false;
    switch (kind) {
    case kQ4Pipe:
        if (fmt != BFormat::Q4Fast || !q4_pipe_ok(a)) return false;
        launch_q4_pipe(a, tile, splits);
        return true;
    case kQ4Skinny: {
        constexpr uint64_t kLim = 0x80000000u;
        if (fmt != BFormat::Q4Fast || a.K % 128 != 0 || a.M > 32 || !q4_pipe_ok(a) ||
            (uint64_t)(a.M + 64) * a.K * 2 >= kLim || (uint64_t)(a.N + 64) * a.row_bytes >= kLim ||
            (uint64_t)(a.N + 64) * a.gpr * 2 >= kLim)
            return false;
        launch_q4_skinny(a, splits);
        return true;
    }
    case kQ4Big:
        if (fmt != BFormat::Q4Fast || !q4_big_ok(a)) return false;
        launch_q4_big(a, splits);
        return true;
    case kQ4Wide:
        if (fmt != BFormat::Q4Fast) return false;
        if (q4_wide_f32_ok(a)) return launch_q4_wide_f32(a, splits);
        if (!q4_wide_ok(a)) return false;
        launch_q4_skinny(a, splits, true);
        return true;
    case kQ4Stream:
        if (fmt != BFormat::Q4Fast || !q4_stream_ok(a)) return false;
        launch_q4_stream(a, splits);
        return true;
    case kQ4General:
        if (fmt == BFormat::Q4Fast) launch_f<BFormat::Q4Fast>(a);
        else if (fmt == BFormat::Q4Generic) launch_f<BFormat::Q4Generic>(a);
        else return false;
        return true;
    default:
        return false;
    }
}

bool q4_f32_wide_takes(const GemmArgs& a) { return q4_wide_f32_ok(a) && env_int("BYHIP_Q4_F32_WIDE", 1) != 0; }

// Whether a call takes the small-M streaming GEMM: fp16 activations, up to 32 rows (or the lower
// limit BYHIP_Q4_SKINNY_MAX_M sets for the small-M kernels), weights with the prefill copy, at most
// two column fragments per 32-row block and K up to 8192, where it beats the split-K kernels (it
// loses to the wide tile at 4096 x 28672 and 14336 x 4096, measured at M = 32). BYHIP_Q4_STREAM=0 leaves
// such calls to the skinny kernel and the wide tile, 1 gives it every shape it takes.
bool q4_stream_takes(const GemmArgs& a) {
    const int forced = env_int("BYHIP_Q4_STREAM", -1);
    if (forced == 0 || a.M > env_int("BYHIP_Q4_SKINNY_MAX_M", 32) || !q4_stream_ok(a)) return false;
    return forced == 1 || (stream_fn(a, 1) <= 2 && a.K <= 8192);
}

bool launch_q4_wide_exact_weights(const GemmArgs& a) {
    if (a.M > 32 || !q4_wide_ok(a)) return false;
    launch_q4_wide_planes<kWideExactW>(a, 0);
    return true;
}

void launch_gemm(BFormat fmt, const GemmArgs& a) {
    if (a.K % 32 != 0) fail("byhip: internal: GEMM needs K %% 32 == 0 (K=%d)", a.K);
    if (a.M <= 0 || a.N <= 0) return;
    if (a.M > 65535 * BM) fail("byhip: M=%d too large for one launch", a.M);
    switch (fmt) {
    case BFormat::Q4Fast:
        // fp32 activations: the wide tile on two fp16 planes where the scratch holds them
        if (q4_f32_wide_takes(a) && launch_q4_wide_f32(a)) break;
        if (q4_stream_takes(a)) {
            launch_q4_stream(a);
            break;
        }
        if (q4_skinny_ok(a)) {
            launch_q4_skinny(a, 0, q4_small_wide(a));
            break;
        }
        switch (q4_prefill_kind(a)) {
        case kQ4Big: launch_q4_big(a); break;
        case kQ4Wide: launch_q4_skinny(a, 0, true); break;
        case kQ4Pipe: launch_q4_pipe(a); break;
        default: launch_f<BFormat::Q4Fast>(a); break;
        }
        break;
    case BFormat::Q4Generic: launch_f<BFormat::Q4Generic>(a); break;
    case BFormat::Fp4Km: launch_f<BFormat::Fp4Km>(a); break;
    case BFormat::F16: launch_f<BFormat::F16>(a); break;
    }
}

}  // namespace byhip
