// byhip_q4.hip - resident Q4 weights and the Q4 block-dequant GEMV / GEMM entry points.
//
// Semantics: y[m, n] = sum_k x[m, k] * ((float)q[n, k] - zero[n, g]) * scale[n, g], g = k / group
// (group 0: g = 0), q the nibble k of row n with even k in the low nibble: the reference's
// cpu_kernels_impl.inc:293-319, gpubackend.nim:288-311 and cpu_vm.c:420-482, accumulated in fp32.
//
// Decode GEMV (M <= 8): q4_gemv_dot2 streams each weight row once with 16-byte loads (one 32-value
// chunk per lane), turns nibble pairs into fp16 with one AND-OR against the 0x6400 exponent
// (1024 + q exactly), subtracts 1024 (exact), and feeds v_dot2_f32_f16 against fp16 x pairs held in
// registers. Products are exact in fp32; the zero point is applied once per chunk as
// s * (sum x*q - z * sum x), so the result differs from the reference's serial fmaf chain only by
// fp32 summation order. fp32 activations are split into two fp16 terms (hi + lo, ~22 bits).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

constexpr int kGemvRows = 4;  // weight rows a wave keeps in flight per batch

template <int M, int CPL, bool XF32, bool SF16, bool ZU, int YT>
__global__ __launch_bounds__(256) void q4_gemv_dot2(
    const void* __restrict__ xv, const uint8_t* __restrict__ wq, const void* __restrict__ sv,
    const float* __restrict__ zeros, float zero_value, void* __restrict__ y, int K, int N,
    int group_chunks, int gpr, int row_bytes) {
    constexpr int XS = XF32 ? 2 : 1;
    constexpr int R = kGemvRows;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nwaves = gridDim.x * 4;
    const int G = K >> 5;  // 32-value chunks per row

    // x chunks of this lane, as fp16 pairs (x[8j+i], x[8j+i+4]) matching the nibble pairs below.
    uint32_t xp[M][CPL][16];
    uint32_t xq[XS == 2 ? M : 1][XS == 2 ? CPL : 1][16];
    float sx[M][CPL];
    int gi[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ci = lane + kWave * c;
        gi[c] = group_chunks ? ci / group_chunks : 0;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float s = 0.0f;
            if (ci < G) {
                if constexpr (XF32) {
                    const float4* p =
                        reinterpret_cast<const float4*>(static_cast<const float*>(xv) + (size_t)m * K + ci * 32);
                    float v[32];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        float4 u = p[t];
                        v[4 * t] = u.x; v[4 * t + 1] = u.y; v[4 * t + 2] = u.z; v[4 * t + 3] = u.w;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float a = v[8 * j + i], b = v[8 * j + i + 4];
                            const _Float16 ha = (_Float16)a, hb = (_Float16)b;
                            const _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
                            xp[m][c][4 * j + i] = (uint32_t)h_bits(ha) | ((uint32_t)h_bits(hb) << 16);
                            if constexpr (XS == 2)
                                xq[m][c][4 * j + i] = (uint32_t)h_bits(la) | ((uint32_t)h_bits(lb) << 16);
                        }
#pragma unroll
                    for (int t = 0; t < 32; ++t) s += v[t];
                } else {
                    const uint4* p = reinterpret_cast<const uint4*>(
                        static_cast<const _Float16*>(xv) + (size_t)m * K + ci * 32);
                    uint32_t d[16];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        uint4 u = p[t];
                        d[4 * t] = u.x; d[4 * t + 1] = u.y; d[4 * t + 2] = u.z; d[4 * t + 3] = u.w;
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t A = d[4 * j], B = d[4 * j + 1], C = d[4 * j + 2], D = d[4 * j + 3];
                        xp[m][c][4 * j + 0] = (A & 0xFFFFu) | (C << 16);
                        xp[m][c][4 * j + 1] = (A >> 16) | (C & 0xFFFF0000u);
                        xp[m][c][4 * j + 2] = (B & 0xFFFFu) | (D << 16);
                        xp[m][c][4 * j + 3] = (B >> 16) | (D & 0xFFFF0000u);
                    }
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
                        const h2 h = bits_h2(d[t]);
                        s += (float)h[0] + (float)h[1];
                    }
                }
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    xp[m][c][t] = 0u;
                    if constexpr (XS == 2) xq[m][c][t] = 0u;
                }
            }
            sx[m][c] = s;
        }
    }

    for (int n0 = wave * R; n0 < N; n0 += nwaves * R) {
        uint4 wv[R][CPL];
        float sc[R][CPL], zp[R][CPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int n = n0 + r, ci = lane + kWave * c;
                if (n < N && ci < G) {
                    wv[r][c] = *reinterpret_cast<const uint4*>(wq + (size_t)n * row_bytes + ci * 16);
                    const size_t si = (size_t)n * gpr + gi[c];
                    if constexpr (SF16)
                        sc[r][c] = (float)static_cast<const _Float16*>(sv)[si];
                    else
                        sc[r][c] = static_cast<const float*>(sv)[si];
                    zp[r][c] = ZU ? zero_value : zeros[si];
                } else {
                    wv[r][c] = make_uint4(0u, 0u, 0u, 0u);
                    sc[r][c] = 0.0f;
                    zp[r][c] = 0.0f;
                }
            }
        float acc[M][R];
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t dw[4] = {wv[r][c].x, wv[r][c].y, wv[r][c].z, wv[r][c].w};
                h2 q[16];
#pragma unroll
                for (int w = 0; w < 4; ++w)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        q[4 * w + i] =
                            bits_h2(((dw[w] >> (4 * i)) & 0x000F000Fu) | 0x64006400u) - (h2){1024, 1024};
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float p = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        p = __builtin_amdgcn_fdot2(bits_h2(xp[m][c][e]), q[e], p, false);
                        if constexpr (XS == 2) p = __builtin_amdgcn_fdot2(bits_h2(xq[m][c][e]), q[e], p, false);
                    }
                    acc[m][r] = fmaf(sc[r][c], p - zp[r][c] * sx[m][c], acc[m][r]);
                }
            }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float t = wave_sum(acc[m][r]);
                if (lane == 0 && n0 + r < N) store_y<YT>(y, (size_t)m * N + n0 + r, t);
            }
    }
}

// Any shape: one wave per weight row, lanes strided over k, the reference's per-element weight
// ((float)q - z) * s and one fmaf per element (cpu_vm.c:467-470).
template <bool XF32, bool SF16, bool ZU, int YT>
__global__ __launch_bounds__(256) void q4_generic(
    const void* __restrict__ xv, const uint8_t* __restrict__ wq, const void* __restrict__ sv,
    const float* __restrict__ zeros, float zero_value, void* __restrict__ y, int M, int K, int N,
    int group, int gpr, size_t row_bytes) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;  // the whole wave leaves together
    for (int m = 0; m < M; ++m) {
        float acc = 0.0f;
        for (int k = lane; k < K; k += kWave) {
            const uint32_t b = wq[(size_t)n * row_bytes + (k >> 1)];
            const uint32_t q = (b >> ((k & 1) * 4)) & 15u;
            const int g = group > 0 ? k / group : 0;
            const size_t si = (size_t)n * gpr + g;
            const float s = SF16 ? (float)static_cast<const _Float16*>(sv)[si] : static_cast<const float*>(sv)[si];
            const float z = ZU ? zero_value : zeros[si];
            const float w = ((float)q - z) * s;
            const float xv_k = XF32 ? static_cast<const float*>(xv)[(size_t)m * K + k]
                                    : (float)static_cast<const _Float16*>(xv)[(size_t)m * K + k];
            acc = fmaf(xv_k, w, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) store_y<YT>(y, (size_t)m * N + n, acc);
    }
}

__global__ void q4_unpack(const uint8_t* __restrict__ wq, size_t row_bytes, int K, int N,
                          const void* __restrict__ sv, int sf16, const float* __restrict__ zeros,
                          float zero_value, size_t n_groups_total, uint8_t* __restrict__ codes,
                          float* __restrict__ scales, float* __restrict__ zs) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)N * K;
    if (i < total) {
        const size_t n = i / K, k = i % K;
        const uint32_t b = wq[n * row_bytes + (k >> 1)];
        codes[i] = (uint8_t)((b >> ((k & 1) * 4)) & 15u);
    }
    if (i < n_groups_total) {
        scales[i] = sf16 ? (float)static_cast<const _Float16*>(sv)[i] : static_cast<const float*>(sv)[i];
        zs[i] = zeros ? zeros[i] : zero_value;
    }
}

// ── host side ───────────────────────────────────────────────────────────────────────────────

// binary32 -> binary16 round to nearest even, on the host (scale classification).
uint16_t host_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

float host_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 113;
            while (!(m & 0x400u)) { m <<= 1; --e; }
            bits = sign | (e << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

void validate_q4_shape(int K, int N, int group, int gpr) {
    if (K <= 0 || N <= 0) fail("byhip: Q4 weights need K > 0 and N > 0 (K=%d N=%d)", K, N);
    if (group < 0 || gpr <= 0) fail("byhip: Q4 group_size %d / groups_per_row %d invalid", group, gpr);
    const int used = group > 0 ? (K - 1) / group + 1 : 1;
    if (used > gpr)
        fail("byhip: K=%d with group_size %d needs %d groups per row, got %d", K, group, used, gpr);
}

byhip_q4w* build_resident(const uint8_t* wq_rows, const float* scales, const float* zeros, int K,
                          int N, int group, int gpr) {
    const size_t row_bytes = (size_t)(K + 1) / 2;
    const size_t ng = (size_t)N * gpr;
    bool sf16 = true;
    for (size_t i = 0; i < ng && sf16; ++i) {
        const float s = scales[i];
        sf16 = std::isfinite(s) && host_f16_to_f32(host_f32_to_f16(s)) == s;
    }
    bool zu = true;
    for (size_t i = 1; i < ng && zu; ++i) zu = memcmp(&zeros[i], &zeros[0], 4) == 0;
    const size_t wq_bytes = (size_t)N * row_bytes;
    const size_t s_bytes = ng * (sf16 ? 2 : 4);
    const size_t z_bytes = zu ? 0 : ng * 4;
    const size_t total = align256(wq_bytes) + align256(s_bytes) + align256(z_bytes);
    uint8_t* base = static_cast<uint8_t*>(device_alloc(total));
    byhip_q4w* w = new byhip_q4w{};
    w->K = K; w->N = N; w->group = group; w->gpr = gpr; w->row_bytes = row_bytes;
    w->wq = base;
    w->scales = base + align256(wq_bytes);
    w->zeros = zu ? nullptr : reinterpret_cast<float*>(base + align256(wq_bytes) + align256(s_bytes));
    w->scale_f16 = sf16;
    w->zero_uniform = zu;
    w->zero_value = zu ? zeros[0] : 0.0f;
    w->bytes = total;
    try {
        BYHIP_HIP(hipMemcpyAsync(w->wq, wq_rows, wq_bytes, hipMemcpyHostToDevice, stream()));
        if (sf16) {
            std::vector<uint16_t> h(ng);
            for (size_t i = 0; i < ng; ++i) h[i] = host_f32_to_f16(scales[i]);
            BYHIP_HIP(hipMemcpyAsync(w->scales, h.data(), s_bytes, hipMemcpyHostToDevice, stream()));
            BYHIP_HIP(hipStreamSynchronize(stream()));
        } else {
            BYHIP_HIP(hipMemcpyAsync(w->scales, scales, s_bytes, hipMemcpyHostToDevice, stream()));
        }
        if (!zu) BYHIP_HIP(hipMemcpyAsync(w->zeros, zeros, z_bytes, hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipStreamSynchronize(stream()));
    } catch (...) {
        device_free(base);
        delete w;
        throw;
    }
    return w;
}

int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return (s && *s) ? atoi(s) : dflt;
}

template <int M, int CPL, bool XF32, bool SF16, bool ZU>
void launch_dot2_y(const void* x, const byhip_q4w* w, void* y, int y_dtype) {
    const int rows_per_block = 4 * kGemvRows;
    const int want = (w->N + rows_per_block - 1) / rows_per_block;
    const int cap = compute_units() * env_int("BYHIP_GEMV_BLOCKS_PER_CU", 4);
    const int grid = std::max(1, std::min(want, cap));
    const int group_chunks = w->group / 32;
    switch (y_dtype) {
    case BYHIP_F32:
        hipLaunchKernelGGL((q4_gemv_dot2<M, CPL, XF32, SF16, ZU, BYHIP_F32>), dim3(grid), dim3(256), 0,
                           stream(), x, w->wq, w->scales, w->zeros, w->zero_value, y, w->K, w->N,
                           group_chunks, w->gpr, (int)w->row_bytes);
        break;
    case BYHIP_F16:
        hipLaunchKernelGGL((q4_gemv_dot2<M, CPL, XF32, SF16, ZU, BYHIP_F16>), dim3(grid), dim3(256), 0,
                           stream(), x, w->wq, w->scales, w->zeros, w->zero_value, y, w->K, w->N,
                           group_chunks, w->gpr, (int)w->row_bytes);
        break;
    default:
        hipLaunchKernelGGL((q4_gemv_dot2<M, CPL, XF32, SF16, ZU, BYHIP_BF16>), dim3(grid), dim3(256), 0,
                           stream(), x, w->wq, w->scales, w->zeros, w->zero_value, y, w->K, w->N,
                           group_chunks, w->gpr, (int)w->row_bytes);
        break;
    }
    BYHIP_LAUNCHED("q4_gemv_dot2");
}

template <int M, int CPL, bool XF32>
void launch_dot2_sz(const void* x, const byhip_q4w* w, void* y, int y_dtype) {
    if (w->scale_f16) {
        if (w->zero_uniform) launch_dot2_y<M, CPL, XF32, true, true>(x, w, y, y_dtype);
        else launch_dot2_y<M, CPL, XF32, true, false>(x, w, y, y_dtype);
    } else {
        if (w->zero_uniform) launch_dot2_y<M, CPL, XF32, false, true>(x, w, y, y_dtype);
        else launch_dot2_y<M, CPL, XF32, false, false>(x, w, y, y_dtype);
    }
}

// x registers per lane: M * CPL * 16 dwords per fp16 term; at most 8 chunk-rows are compiled.
template <int M, int CPL, bool XF32>
void launch_dot2_fit(const void* x, const byhip_q4w* w, void* y, int y_dtype) {
    if constexpr (M * CPL * (XF32 ? 2 : 1) <= 8) launch_dot2_sz<M, CPL, XF32>(x, w, y, y_dtype);
    else fail("byhip: internal: GEMV register tile out of range");
}

template <int M, bool XF32>
void launch_dot2_cpl(int cpl, const void* x, const byhip_q4w* w, void* y, int y_dtype) {
    switch (cpl) {
    case 1: launch_dot2_fit<M, 1, XF32>(x, w, y, y_dtype); break;
    case 2: launch_dot2_fit<M, 2, XF32>(x, w, y, y_dtype); break;
    case 4: launch_dot2_fit<M, 4, XF32>(x, w, y, y_dtype); break;
    default: launch_dot2_fit<M, 8, XF32>(x, w, y, y_dtype); break;
    }
}

// Chunks of 32 values per lane the GEMV keeps in registers for K (a power of two up to 8).
int gemv_cpl(int K) {
    const int G = K / 32;
    int cpl = 1;
    while (cpl * kWave < G) cpl *= 2;
    return cpl;
}

bool dot2_eligible(const byhip_q4w* w, int M, int x_dtype) {
    if (w->K % 32 != 0 || (w->group != 0 && w->group % 32 != 0)) return false;
    const int xs = x_dtype == BYHIP_F32 ? 2 : 1;
    const int cpl = gemv_cpl(w->K);
    const int m = std::min(M, 4);
    return cpl <= 8 && m * xs * cpl <= 8;
}

void launch_dot2(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    const int cpl = gemv_cpl(w->K);
    const size_t xb = dtype_bytes(x_dtype), yb = dtype_bytes(y_dtype);
    for (int m0 = 0; m0 < M; m0 += 4) {
        const int mm = std::min(4, M - m0);
        const void* xm = static_cast<const uint8_t*>(x) + (size_t)m0 * w->K * xb;
        void* ym = static_cast<uint8_t*>(y) + (size_t)m0 * w->N * yb;
        if (x_dtype == BYHIP_F32) {
            switch (mm) {
            case 1: launch_dot2_cpl<1, true>(cpl, xm, w, ym, y_dtype); break;
            case 2: launch_dot2_cpl<2, true>(cpl, xm, w, ym, y_dtype); break;
            case 3: launch_dot2_cpl<3, true>(cpl, xm, w, ym, y_dtype); break;
            default: launch_dot2_cpl<4, true>(cpl, xm, w, ym, y_dtype); break;
            }
        } else {
            switch (mm) {
            case 1: launch_dot2_cpl<1, false>(cpl, xm, w, ym, y_dtype); break;
            case 2: launch_dot2_cpl<2, false>(cpl, xm, w, ym, y_dtype); break;
            case 3: launch_dot2_cpl<3, false>(cpl, xm, w, ym, y_dtype); break;
            default: launch_dot2_cpl<4, false>(cpl, xm, w, ym, y_dtype); break;
            }
        }
    }
}

template <bool XF32, bool SF16, bool ZU>
void launch_generic_y(const void* x, const byhip_q4w* w, void* y, int y_dtype, int M) {
    const int grid = (w->N + 3) / 4;
    switch (y_dtype) {
    case BYHIP_F32:
        hipLaunchKernelGGL((q4_generic<XF32, SF16, ZU, BYHIP_F32>), dim3(grid), dim3(256), 0, stream(), x,
                           w->wq, w->scales, w->zeros, w->zero_value, y, M, w->K, w->N, w->group,
                           w->gpr, w->row_bytes);
        break;
    case BYHIP_F16:
        hipLaunchKernelGGL((q4_generic<XF32, SF16, ZU, BYHIP_F16>), dim3(grid), dim3(256), 0, stream(), x,
                           w->wq, w->scales, w->zeros, w->zero_value, y, M, w->K, w->N, w->group,
                           w->gpr, w->row_bytes);
        break;
    default:
        hipLaunchKernelGGL((q4_generic<XF32, SF16, ZU, BYHIP_BF16>), dim3(grid), dim3(256), 0, stream(), x,
                           w->wq, w->scales, w->zeros, w->zero_value, y, M, w->K, w->N, w->group,
                           w->gpr, w->row_bytes);
        break;
    }
    BYHIP_LAUNCHED("q4_generic");
}

void launch_generic(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    const bool xf = x_dtype == BYHIP_F32;
    if (xf) {
        if (w->scale_f16) {
            if (w->zero_uniform) launch_generic_y<true, true, true>(x, w, y, y_dtype, M);
            else launch_generic_y<true, true, false>(x, w, y, y_dtype, M);
        } else {
            if (w->zero_uniform) launch_generic_y<true, false, true>(x, w, y, y_dtype, M);
            else launch_generic_y<true, false, false>(x, w, y, y_dtype, M);
        }
    } else {
        if (w->scale_f16) {
            if (w->zero_uniform) launch_generic_y<false, true, true>(x, w, y, y_dtype, M);
            else launch_generic_y<false, true, false>(x, w, y, y_dtype, M);
        } else {
            if (w->zero_uniform) launch_generic_y<false, false, true>(x, w, y, y_dtype, M);
            else launch_generic_y<false, false, false>(x, w, y, y_dtype, M);
        }
    }
}

// Zero points the fp16 MFMA path subtracts exactly: integers with |1024 + z| representable.
bool zeros_integral(const byhip_q4w* w) {
    if (!w->zero_uniform) return false;  // per-group zeros: the generic dequant handles them
    const float z = w->zero_value;
    return std::floor(z) == z && z >= -1024.0f && z <= 1024.0f;
}

void q4_matmul_impl(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    if (!w) fail("byhip: null Q4 weights");
    if (x_dtype != BYHIP_F32 && x_dtype != BYHIP_F16) fail("byhip: Q4 activations must be F32 or F16");
    if (y_dtype != BYHIP_F32 && y_dtype != BYHIP_F16 && y_dtype != BYHIP_BF16)
        fail("byhip: Q4 output must be F32, F16 or BF16");
    if (M <= 0) fail("byhip: Q4 matmul needs M > 0 (M=%d)", M);
    check_span(x, (size_t)M * w->K * dtype_bytes(x_dtype), "Q4 activations");
    check_span(y, (size_t)M * w->N * dtype_bytes(y_dtype), "Q4 output");
    const int mode = env_int("BYHIP_Q4_ROUTE", 0);  // 0 auto, 1 GEMV, 2 GEMM, 3 generic
    // The vector kernels read 16-byte words of weights and activations.
    const bool aligned = reinterpret_cast<uintptr_t>(w->wq) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (!aligned) {
        launch_generic(x, x_dtype, w, y, y_dtype, M);
        return;
    }
    const bool gemm_ok = w->K % 32 == 0;
    if (mode == 3 || (mode == 0 && !gemm_ok && !dot2_eligible(w, M, x_dtype))) {
        launch_generic(x, x_dtype, w, y, y_dtype, M);
        return;
    }
    const bool want_gemv = mode == 1 || (mode == 0 && M <= 8);
    if (want_gemv && dot2_eligible(w, M, x_dtype)) {
        launch_dot2(x, x_dtype, w, y, y_dtype, M);
        return;
    }
    // Decode shapes the GEMV does not take (groups not a multiple of 32, very long K) stay on the
    // exact per-element kernel rather than rounding weights to fp16 for the MFMA.
    if (!gemm_ok || (mode <= 1 && M <= 8)) {
        launch_generic(x, x_dtype, w, y, y_dtype, M);
        return;
    }
    GemmArgs a;
    a.x = x; a.x_dtype = x_dtype; a.y = y; a.y_dtype = y_dtype;
    a.M = M; a.K = w->K; a.N = w->N;
    a.wq = w->wq; a.row_bytes = w->row_bytes; a.scales = w->scales; a.scale_f16 = w->scale_f16;
    a.zeros = w->zeros; a.zero_value = w->zero_value; a.group = w->group; a.gpr = w->gpr;
    const bool fast = w->scale_f16 && zeros_integral(w) && (w->group == 0 || w->group % 32 == 0);
    launch_gemm(fast ? BFormat::Q4Fast : BFormat::Q4Generic, a);
}

}  // namespace

void q4_matmul_run(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    q4_matmul_impl(x, x_dtype, w, y, y_dtype, M);
}

}  // namespace byhip

using namespace byhip;

extern "C" {

int byhip_q4_resident_upload(const uint8_t* wq, size_t wq_bytes, size_t wq_off, const float* scales,
                             const float* zeros, int K, int N, int group_size, int groups_per_row,
                             byhip_q4w** out) {
    return guard([&] {
        enter_compute();
        if (!out) fail("byhip: null output handle");
        *out = nullptr;
        validate_q4_shape(K, N, group_size, groups_per_row);
        if (!wq || !scales || !zeros) fail("byhip: null Q4 weight array");
        const size_t need = (size_t)N * ((size_t)(K + 1) / 2);
        if (wq_off > wq_bytes || wq_bytes - wq_off < need)
            fail("byhip: Q4 weights need %zu bytes at offset %zu, buffer holds %zu", need, wq_off,
                 wq_bytes);
        *out = build_resident(wq + wq_off, scales, zeros, K, N, group_size, groups_per_row);
    });
}

int byhip_q4_resident_from_device(const void* d_wq, size_t wq_off, const void* d_scales,
                                  const void* d_zeros, int K, int N, int group_size,
                                  int groups_per_row, byhip_q4w** out) {
    return guard([&] {
        enter_compute();
        if (!out) fail("byhip: null output handle");
        *out = nullptr;
        validate_q4_shape(K, N, group_size, groups_per_row);
        const size_t wq_bytes = (size_t)N * ((size_t)(K + 1) / 2);
        const size_t ng = (size_t)N * groups_per_row;
        check_span(static_cast<const uint8_t*>(d_wq) + wq_off, wq_bytes, "Q4 packed weights");
        check_span(d_scales, ng * 4, "Q4 scales");
        check_span(d_zeros, ng * 4, "Q4 zeros");
        std::vector<uint8_t> wq(wq_bytes);
        std::vector<float> sc(ng), ze(ng);
        BYHIP_HIP(hipStreamSynchronize(stream()));
        BYHIP_HIP(hipMemcpy(wq.data(), static_cast<const uint8_t*>(d_wq) + wq_off, wq_bytes,
                            hipMemcpyDeviceToHost));
        BYHIP_HIP(hipMemcpy(sc.data(), d_scales, ng * 4, hipMemcpyDeviceToHost));
        BYHIP_HIP(hipMemcpy(ze.data(), d_zeros, ng * 4, hipMemcpyDeviceToHost));
        *out = build_resident(wq.data(), sc.data(), ze.data(), K, N, group_size, groups_per_row);
    });
}

int byhip_q4_resident_free(byhip_q4w* w) {
    return guard([&] {
        enter_compute();
        if (!w) return;
        BYHIP_HIP(hipStreamSynchronize(stream()));
        device_free(w->wq);
        delete w;
    });
}

int byhip_q4_resident_info(const byhip_q4w* w, byhip_q4w_info* out) {
    return guard([&] {
        if (!w || !out) fail("byhip: null argument");
        out->K = w->K; out->N = w->N; out->group_size = w->group; out->groups_per_row = w->gpr;
        out->scale_is_f16 = w->scale_f16; out->zero_uniform = w->zero_uniform;
        out->zero_value = w->zero_value; out->device_bytes = w->bytes;
    });
}

int byhip_q4_matmul(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    return guard([&] {
        enter_compute();
        q4_matmul_impl(x, x_dtype, w, y, y_dtype, M);
    });
}

int byhip_gpu_matmul_q4(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                        float* c, int M, int K, int N, int group_size, int groups_per_row) {
    return guard([&] {
        enter_compute();
        if (M <= 0) fail("byhip: Q4 matmul needs M > 0 (M=%d)", M);
        if (!a || !c) fail("byhip: null Q4 activation or output");
        validate_q4_shape(K, N, group_size, groups_per_row);
        if (!wq || !scales || !zeros) fail("byhip: null Q4 weight array");
        byhip_q4w* w = build_resident(wq, scales, zeros, K, N, group_size, groups_per_row);
        void* dx = nullptr;
        void* dy = nullptr;
        try {
            dx = device_alloc((size_t)M * K * 4);
            dy = device_alloc((size_t)M * N * 4);
            BYHIP_HIP(hipMemcpyAsync(dx, a, (size_t)M * K * 4, hipMemcpyHostToDevice, stream()));
            q4_matmul_impl(dx, BYHIP_F32, w, dy, BYHIP_F32, M);
            BYHIP_HIP(hipMemcpyAsync(c, dy, (size_t)M * N * 4, hipMemcpyDeviceToHost, stream()));
            BYHIP_HIP(hipStreamSynchronize(stream()));
        } catch (...) {
            (void)hipStreamSynchronize(stream());
            device_free(dx);
            device_free(dy);
            device_free(w->wq);
            delete w;
            throw;
        }
        device_free(dx);
        device_free(dy);
        device_free(w->wq);
        delete w;
    });
}

int byhip_debug_unpack_q4(const byhip_q4w* w, uint8_t* codes, float* scales, float* zeros) {
    return guard([&] {
        enter_compute();
        if (!w || !codes || !scales || !zeros) fail("byhip: null argument");
        const size_t total = (size_t)w->N * w->K, ng = (size_t)w->N * w->gpr;
        uint8_t* dc = static_cast<uint8_t*>(device_alloc(total));
        float* ds = static_cast<float*>(device_alloc(ng * 4));
        float* dz = static_cast<float*>(device_alloc(ng * 4));
        const size_t n = std::max(total, ng);
        const int grid = (int)((n + 255) / 256);
        hipLaunchKernelGGL(q4_unpack, dim3(grid), dim3(256), 0, stream(), w->wq, w->row_bytes, w->K,
                           w->N, w->scales, w->scale_f16, w->zeros, w->zero_value, ng, dc, ds, dz);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(stream());
        if (e == hipSuccess) e = hipMemcpy(codes, dc, total, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(scales, ds, ng * 4, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(zeros, dz, ng * 4, hipMemcpyDeviceToHost);
        device_free(dc);
        device_free(ds);
        device_free(dz);
        BYHIP_HIP(e);
    });
}

}  // extern "C"
