// byhip_q4.hip - resident Q4 weights and the Q4 block-dequant GEMV / GEMM entry points.
//
// Semantics: y[m, n] = sum_k x[m, k] * ((float)q[n, k] - zero[n, g]) * scale[n, g], g = k / group
// (group 0: g = 0), q the nibble k of row n with even k in the low nibble: the reference's
// cpu_kernels_impl.inc:293-319, gpubackend.nim:288-311 and cpu_vm.c:420-482, accumulated in fp32.
//
// Decode GEMV (M <= 8): byhip_gemv.hip. Larger M: the fp16 MFMA GEMM of byhip_gemm.hip for weights
// whose products stay in fp16's range, else the exact fp32 GEMM of byhip_exact.hip. Decode shapes
// the GEMV does not take (K or the group not a multiple of 32, unaligned buffers): q4_generic below,
// which forms the reference's per-element weight ((float)q - z) * s in fp32.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "byhip_gemm.h"
#include "byhip_gemv.h"
#include "byhip_q4.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

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

// Codes, scales and zeros back from the device layout. A (row, group) whose group holds data is
// read from the decode copy when there is one (the layout the GEMV reads), else from the rows.
__global__ void q4_unpack(const uint8_t* __restrict__ wq, size_t row_bytes, int K, int N,
                          const void* __restrict__ sv, int sf16, const float* __restrict__ zeros,
                          float zero_value, const void* __restrict__ sblk,
                          const float* __restrict__ zblk, int group, int gpr,
                          uint8_t* __restrict__ codes, float* __restrict__ scales,
                          float* __restrict__ zs) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)N * K;
    if (i < total) {
        const size_t n = i / K, k = i % K;
        const uint32_t b = wq[n * row_bytes + (k >> 1)];
        codes[i] = (uint8_t)((b >> ((k & 1) * 4)) & 15u);
    }
    if (i < (size_t)N * gpr) {
        const size_t n = i / gpr, g = i % gpr, G = (size_t)K / 32;
        const size_t ch = group ? g * (size_t)group / 32 : 0;
        const bool from_blk = sblk && (group ? g * (size_t)group < (size_t)K : g == 0) && ch < G;
        const size_t j = from_blk ? ((n / 8) * G + ch) * 8 + n % 8 : i;
        const void* s = from_blk ? sblk : sv;
        scales[i] = sf16 ? (float)static_cast<const _Float16*>(s)[j] : static_cast<const float*>(s)[j];
        const float* z = from_blk ? zblk : zeros;
        zs[i] = z ? z[j] : zero_value;
    }
}

// Classification of the scales and zeros of a resident upload, per block b, in flags[8b .. 8b+7]:
//   0  every scale is finite and converts to fp16 exactly
//   1  every zero equals zeros[0] bit for bit
//   2  every scale and zero is finite
//   3  the largest |scale| (float bits)
//   4  the smallest nonzero |scale| (float bits; +inf when every scale is zero)
//   5, 6  the smallest and largest zero (float bits)
// The host combines the blocks.
__global__ __launch_bounds__(256) void q4_classify(const float* __restrict__ sc, const float* __restrict__ ze,
                                                   size_t ng, int* __restrict__ flags) {
    __shared__ float red[4][4];
    const uint32_t z0 = __builtin_bit_cast(uint32_t, ze[0]);
    int ok_s = 1, ok_z = 1, fin = 1;
    float smax = 0.0f, smin = __builtin_inff(), zmin = __builtin_inff(), zmax = -__builtin_inff();
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < ng; i += (size_t)gridDim.x * 256) {
        const float s = sc[i], z = ze[i];
        ok_s &= (__builtin_isfinite(s) && (float)(_Float16)s == s) ? 1 : 0;
        ok_z &= __builtin_bit_cast(uint32_t, z) == z0 ? 1 : 0;
        fin &= (__builtin_isfinite(s) && __builtin_isfinite(z)) ? 1 : 0;
        const float as = fabsf(s);
        smax = fmaxf(smax, as);
        if (as > 0.0f) smin = fminf(smin, as);
        zmin = fminf(zmin, z);
        zmax = fmaxf(zmax, z);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        smax = fmaxf(smax, __shfl_xor(smax, o, kWave));
        smin = fminf(smin, __shfl_xor(smin, o, kWave));
        zmin = fminf(zmin, __shfl_xor(zmin, o, kWave));
        zmax = fmaxf(zmax, __shfl_xor(zmax, o, kWave));
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        red[0][w] = smax; red[1][w] = smin; red[2][w] = zmin; red[3][w] = zmax;
    }
    ok_s = __syncthreads_and(ok_s);
    ok_z = __syncthreads_and(ok_z);
    fin = __syncthreads_and(fin);
    if (threadIdx.x == 0) {
        int* f = flags + 8 * blockIdx.x;
        f[0] = ok_s;
        f[1] = ok_z;
        f[2] = fin;
        f[3] = __builtin_bit_cast(int, fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3])));
        f[4] = __builtin_bit_cast(int, fminf(fminf(red[1][0], red[1][1]), fminf(red[1][2], red[1][3])));
        f[5] = __builtin_bit_cast(int, fminf(fminf(red[2][0], red[2][1]), fminf(red[2][2], red[2][3])));
        f[6] = __builtin_bit_cast(int, fmaxf(fmaxf(red[3][0], red[3][1]), fmaxf(red[3][2], red[3][3])));
        f[7] = 0;
    }
}

// The resident scale and zero layouts from fp32 device arrays [N * gpr]: plain scales (fp16 when
// sf16), plain zeros (unless uniform), and the decode copy [ceil(N/8)][K/32][8] (padded rows 0).
__global__ __launch_bounds__(256) void q4_pack_scales(const float* __restrict__ sc, const float* __restrict__ ze,
                                                      int N, int gpr, int group, int G, int sf16, int zu,
                                                      void* __restrict__ scales, float* __restrict__ zeros,
                                                      void* __restrict__ sblk, float* __restrict__ zblk) {
    const size_t ng = (size_t)N * gpr, nb = sblk ? (size_t)(N + 7) / 8 * 8 * G : 0;
    const size_t total = ng > nb ? ng : nb;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        if (i < ng) {
            if (sf16) static_cast<_Float16*>(scales)[i] = (_Float16)sc[i];
            else static_cast<float*>(scales)[i] = sc[i];
            if (!zu) zeros[i] = ze[i];
        }
        if (i < nb) {
            // entry i = ((n / 8) * G + ch) * 8 + n % 8
            const size_t n = (i / ((size_t)G * 8)) * 8 + i % 8, ch = (i / 8) % G;
            float s = 0.0f, z = 0.0f;
            if (n < (size_t)N) {
                const size_t src = n * gpr + (group ? ch * 32 / (size_t)group : 0);
                s = sc[src];
                z = ze[src];
            }
            if (sf16) static_cast<_Float16*>(sblk)[i] = (_Float16)s;
            else static_cast<float*>(sblk)[i] = s;
            if (!zu) zblk[i] = z;
        }
    }
}

// The prefill copy (byhip_q4w::wpf, spf) from the nibble rows already on the device and the fp32
// scales [N * gpr]: word i of wpf holds, for fragment f, sub-step u, lane l = c + 16 g and half d,
// the nibbles of column 16 f + c at K positions p0 .. p0 + 7 (p0 = 64 u + 16 g + 8 d), position
// p0 + k at bits 4 (k / 2) for even k and 16 + 4 (k / 2) for odd k; half i of spf the scale of
// column 64 q + 16 j + c at K position 64 u + 32 t. Columns past N are zeros.
__global__ __launch_bounds__(256) void q4_pack_prefill(const uint8_t* __restrict__ wq, size_t row_bytes,
                                                       const float* __restrict__ sc, int N, int K, int gpr,
                                                       int group, uint32_t* __restrict__ wpf,
                                                       _Float16* __restrict__ spf) {
    const size_t nsub = (size_t)K / 64;
    const size_t nw = (size_t)(N + 15) / 16 * nsub * 128, ns = (size_t)(N + 63) / 64 * nsub * 128;
    const size_t total = nw > ns ? nw : ns;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        if (i < nw) {
            const size_t d = i & 1, l = (i >> 1) & 63, u = (i >> 7) % nsub, f = (i >> 7) / nsub;
            const size_t n = 16 * f + (l & 15), p0 = 64 * u + 16 * (l >> 4) + 8 * d;
            uint32_t v = 0;
            if (n < (size_t)N) {
                const uint32_t b = *reinterpret_cast<const uint32_t*>(wq + n * row_bytes + p0 / 2);
#pragma unroll
                for (int k = 0; k < 8; ++k) v |= ((b >> (4 * k)) & 15u) << ((k & 1) ? 16 + 4 * (k >> 1) : 4 * (k >> 1));
            }
            wpf[i] = v;
        }
        if (i < ns) {
            const size_t j = i & 3, c = (i >> 2) & 15, t = (i >> 6) & 1, u = (i >> 7) % nsub, q = (i >> 7) / nsub;
            const size_t n = 64 * q + 16 * j + c, p = 64 * u + 32 * t;
            spf[i] = n < (size_t)N ? (_Float16)sc[n * gpr + (group ? p / (size_t)group : 0)] : (_Float16)0.0f;
        }
    }
}

// ── host side ───────────────────────────────────────────────────────────────────────────────

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

float bits_float(int v) {
    float f;
    memcpy(&f, &v, sizeof f);
    return f;
}

void validate_q4_shape(int K, int N, int group, int gpr) {
    if (K <= 0 || N <= 0) fail("byhip: Q4 weights need K > 0 and N > 0 (K=%d N=%d)", K, N);
    if (group < 0 || gpr <= 0) fail("byhip: Q4 group_size %d / groups_per_row %d invalid", group, gpr);
    const int used = group > 0 ? (K - 1) / group + 1 : 1;
    if (used > gpr)
        fail("byhip: K=%d with group_size %d needs %d groups per row, got %d", K, group, used, gpr);
}

// The resident layout from nibble rows at wq_src (host memory, or device memory when wq_on_device)
// and fp32 scales / zeros [N * gpr] in device memory. The scale format and the uniform zero are
// decided on the device (q4_classify) and the layouts written there (q4_pack_scales), so the host
// does no per-element work; only the block flags and zeros[0] come back.
byhip_q4w* build_resident_dev(const void* wq_src, bool wq_on_device, const float* d_sc, const float* d_ze,
                              int K, int N, int group, int gpr) {
    const size_t row_bytes = (size_t)(K + 1) / 2;
    const size_t ng = (size_t)N * gpr;
    const int cblocks = (int)std::min<size_t>((ng + 255) / 256, 1024);
    int* d_flags = static_cast<int*>(device_alloc((size_t)cblocks * 8 * sizeof(int)));
    std::vector<int> flags((size_t)cblocks * 8);
    float zero0 = 0.0f;
    try {
        launch("q4_classify", q4_classify, dim3(cblocks), dim3(256), 0, d_sc, d_ze, ng, d_flags);
        BYHIP_LAUNCHED("q4_classify");
        BYHIP_HIP(hipMemcpyAsync(flags.data(), d_flags, flags.size() * sizeof(int), hipMemcpyDeviceToHost, stream()));
        BYHIP_HIP(hipMemcpyAsync(&zero0, d_ze, sizeof(float), hipMemcpyDeviceToHost, stream()));
        BYHIP_HIP(hipStreamSynchronize(stream()));
    } catch (...) {
        device_free(d_flags);
        throw;
    }
    device_free(d_flags);
    bool sf16 = true, zu = true, finite = true;
    float smax = 0.0f, smin = INFINITY, zmin = INFINITY, zmax = -INFINITY;
    for (int b = 0; b < cblocks; ++b) {
        const int* f = &flags[8 * b];
        sf16 = sf16 && f[0];
        zu = zu && f[1];
        finite = finite && f[2];
        smax = std::fmax(smax, bits_float(f[3]));
        smin = std::fmin(smin, bits_float(f[4]));
        zmin = std::fmin(zmin, bits_float(f[5]));
        zmax = std::fmax(zmax, bits_float(f[6]));
    }
    // The fp16 MFMA kernels round (q - z) * s to fp16 (one rounding, 2^-11 relative): they take the
    // weights only when every such product stays in fp16's normal range, so none overflows and
    // none loses more than that to subnormals. Otherwise the exact fp32 route runs them.
    const float qz = std::fmax(std::fmax(std::fabs(zmin), std::fabs(zmax)),
                               std::fmax(std::fabs(15.0f - zmin), std::fabs(15.0f - zmax)));
    const bool f16_safe = finite && (double)smax * qz <= 65504.0 && (smin == INFINITY || smin >= 0x1p-14f);
    const size_t wq_bytes = (size_t)N * row_bytes;
    const size_t s_bytes = ng * (sf16 ? 2 : 4);
    const size_t z_bytes = zu ? 0 : ng * 4;
    // Decode copy: per 32-value chunk, rows in blocks of 8 (see byhip_q4w::sblk).
    const bool blk = K % 32 == 0 && (group == 0 || group % 32 == 0);
    const size_t G = (size_t)K / 32, n_pad = ((size_t)N + 7) / 8 * 8;
    const size_t sb_bytes = blk ? n_pad * G * (sf16 ? 2 : 4) : 0;
    const size_t zb_bytes = blk && !zu ? n_pad * G * 4 : 0;
    // Prefill copy (byhip_q4w::wpf, spf) for the fp16 MFMA prefill kernels.
    const bool pf = f16_safe && sf16 && zu && K % 64 == 0 && (group == 0 || group % 32 == 0) && row_bytes % 4 == 0;
    const size_t nsub = (size_t)K / 64;
    const size_t wpf_bytes = pf ? ((size_t)N + 15) / 16 * nsub * 512 : 0;
    const size_t spf_bytes = pf ? ((size_t)N + 63) / 64 * nsub * 256 : 0;
    const size_t o_s = align256(wq_bytes), o_z = o_s + align256(s_bytes), o_sb = o_z + align256(z_bytes),
                 o_zb = o_sb + align256(sb_bytes), o_wpf = o_zb + align256(zb_bytes),
                 o_spf = o_wpf + align256(wpf_bytes), total = o_spf + align256(spf_bytes);
    uint8_t* base = static_cast<uint8_t*>(device_alloc(total));
    byhip_q4w* w = new byhip_q4w{};
    w->K = K; w->N = N; w->group = group; w->gpr = gpr; w->row_bytes = row_bytes;
    w->wq = base;
    w->scales = base + o_s;
    w->zeros = zu ? nullptr : reinterpret_cast<float*>(base + o_z);
    w->scale_f16 = sf16;
    w->zero_uniform = zu;
    w->zero_value = zu ? zero0 : 0.0f;
    w->bytes = total;
    w->sblk = blk ? base + o_sb : nullptr;
    w->zblk = blk && !zu ? reinterpret_cast<float*>(base + o_zb) : nullptr;
    w->blk_scale_f16 = sf16;
    w->f16_safe = f16_safe;
    w->wpf = pf ? base + o_wpf : nullptr;
    w->spf = pf ? base + o_spf : nullptr;
    try {
        BYHIP_HIP(hipMemcpyAsync(w->wq, wq_src, wq_bytes, wq_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                 stream()));
        const size_t work = std::max(ng, blk ? n_pad * G : (size_t)0);
        const int pblocks = (int)std::min<size_t>((work + 255) / 256, (size_t)compute_units() * 16);
        launch("q4_pack_scales", q4_pack_scales, dim3(pblocks), dim3(256), 0, d_sc, d_ze, N, gpr, group, (int)G,
                           (int)sf16, (int)zu, w->scales, w->zeros, w->sblk, w->zblk);
        BYHIP_LAUNCHED("q4_pack_scales");
        if (pf) {
            const size_t pw = std::max(((size_t)N + 15) / 16 * nsub * 128, ((size_t)N + 63) / 64 * nsub * 128);
            const int fblocks = (int)std::min<size_t>((pw + 255) / 256, (size_t)compute_units() * 16);
            launch("q4_pack_prefill", q4_pack_prefill, dim3(fblocks), dim3(256), 0, w->wq, row_bytes, d_sc, N, K,
                               gpr, group, reinterpret_cast<uint32_t*>(w->wpf), static_cast<_Float16*>(w->spf));
            BYHIP_LAUNCHED("q4_pack_prefill");
        }
        BYHIP_HIP(hipStreamSynchronize(stream()));  // the source may be pageable host memory
    } catch (...) {
        device_free(base);
        delete w;
        throw;
    }
    return w;
}

// The same from host scale and zero arrays: they go to the device as they are, then as above.
byhip_q4w* build_resident(const uint8_t* wq_rows, const float* scales, const float* zeros, int K, int N,
                          int group, int gpr) {
    const size_t ng = (size_t)N * gpr;
    float* d = static_cast<float*>(device_alloc(2 * ng * sizeof(float)));
    byhip_q4w* w = nullptr;
    try {
        BYHIP_HIP(hipMemcpyAsync(d, scales, ng * 4, hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipMemcpyAsync(d + ng, zeros, ng * 4, hipMemcpyHostToDevice, stream()));
        w = build_resident_dev(wq_rows, false, d, d + ng, K, N, group, gpr);
    } catch (...) {
        device_free(d);
        throw;
    }
    device_free(d);
    return w;
}

template <bool XF32, bool SF16, bool ZU>
void launch_generic_y(const void* x, const byhip_q4w* w, void* y, int y_dtype, int M) {
    const int grid = (w->N + 3) / 4;
    switch (y_dtype) {
    case BYHIP_F32:
        launch("q4_generic", (q4_generic<XF32, SF16, ZU, BYHIP_F32>), dim3(grid), dim3(256), 0, x,
                           w->wq, w->scales, w->zeros, w->zero_value, y, M, w->K, w->N, w->group,
                           w->gpr, w->row_bytes);
        break;
    case BYHIP_F16:
        launch("q4_generic", (q4_generic<XF32, SF16, ZU, BYHIP_F16>), dim3(grid), dim3(256), 0, x,
                           w->wq, w->scales, w->zeros, w->zero_value, y, M, w->K, w->N, w->group,
                           w->gpr, w->row_bytes);
        break;
    default:
        launch("q4_generic", (q4_generic<XF32, SF16, ZU, BYHIP_BF16>), dim3(grid), dim3(256), 0, x,
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

GemmArgs q4_gemm_args(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    GemmArgs a;
    a.x = x; a.x_dtype = x_dtype; a.y = y; a.y_dtype = y_dtype;
    a.M = M; a.K = w->K; a.N = w->N;
    a.wq = w->wq; a.row_bytes = w->row_bytes; a.scales = w->scales; a.scale_f16 = w->scale_f16;
    a.zeros = w->zeros; a.zero_value = w->zero_value; a.group = w->group; a.gpr = w->gpr;
    a.sblk = w->blk_scale_f16 ? w->sblk : nullptr;
    a.wpf = w->wpf;
    a.spf = w->spf;
    return a;
}

// Weights the fp16 MFMA kernels take in the Q4Fast form: fp16 scales, an integral uniform zero,
// group 0 or a multiple of 32.
bool q4_fast(const byhip_q4w* w) {
    return w->scale_f16 && zeros_integral(w) && (w->group == 0 || w->group % 32 == 0);
}

// Routes y = x . W^T. Decode shapes (M <= 8) take the GEMV, whose arithmetic is exact (fp32 scales,
// zeros and sums; fp32 activations kept to ~22 bits over their whole range), or the per-element
// kernel when the GEMV does not take the shape. Exception: fp32 activations on weights with the
// prefill copy take the wide tile over two fp16 activation planes (the weights kept exactly, ~22
// bits of x) from M = 3, and at M = 2 when one GEMV launch does not hold both rows. The GEMV's time
// grows with its rows while the tile's barely moves (fp32, K x N = 4096 x 14336, M = 1 / 2 / 3 /
// 4 / 8: GEMV 11.6 / 14.0 / 25.6 / 27.6 / 54.2 us, tile 15.6 / 15.8 / 15.9 / 16.1 / 16.6;
// 14336 x 4096: GEMV 13.7 / 27.2 / 40.6 / 53.9 / 107.0, tile 18.6 / 19.2 / 19.3 / 19.5 / 20.7).
// fp16 activations take the wide tile with each weight as two fp16 terms that add up to it (the
// weights exact, as in the GEMV) past 4 rows, or past the rows one GEMV launch holds (fp16,
// M = 2 / 4 / 5 / 8: 4096 x 14336 GEMV 9.9 / 13.8 / 21.1 / 27.2 us, tile 12.6 / 12.6 / 12.7 /
// 12.7; 14336 x 4096, one row per GEMV launch, GEMV 15.9 / 31.0 / 38.5 / 60.8, tile 12.5 / 12.8 /
// 12.9 / 13.0; 4096 x 6144 GEMV 6.3 / 9.0 / 13.7 / 17.9, tile 9.6 / 9.6 / 9.7 / 9.9).
// BYHIP_Q4_DECODE_TILE=0 keeps them on the GEMV, 1 puts them on the tile from M = 2.
// Larger M takes the fp16 MFMA kernels when the weights are fp16-safe (each (q - z) * s rounded
// once to fp16, byhip_q4w::f16_safe) and `exact` is not asked for, else the exact fp32 GEMM. BYHIP_Q4_ROUTE forces a route: 1 GEMV, 2 GEMM (fp16
// when safe, else exact), 3 per-element, 4 exact GEMM.
void q4_matmul_impl(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, bool exact,
                    void* work, size_t work_bytes) {
    if (!w) fail("byhip: null Q4 weights");
    if (x_dtype != BYHIP_F32 && x_dtype != BYHIP_F16) fail("byhip: Q4 activations must be F32 or F16");
    if (y_dtype != BYHIP_F32 && y_dtype != BYHIP_F16 && y_dtype != BYHIP_BF16)
        fail("byhip: Q4 output must be F32, F16 or BF16");
    if (M <= 0) fail("byhip: Q4 matmul needs M > 0 (M=%d)", M);
    check_span(x, (size_t)M * w->K * dtype_bytes(x_dtype), "Q4 activations");
    check_span(y, (size_t)M * w->N * dtype_bytes(y_dtype), "Q4 output");
    const int mode = env_int("BYHIP_Q4_ROUTE", 0);
    GemmArgs ga = q4_gemm_args(x, x_dtype, w, y, y_dtype, M);
    ga.work = work;
    ga.work_bytes = work_bytes;
    // A plan chosen by byhip_q4_prepare for this shape, unless a route is forced or exactness asked.
    Q4Plan plan;
    if (mode == 0 && !exact && !work && q4_lookup_plan(w, M, x_dtype, &plan) &&
        q4_run_plan(plan, x, x_dtype, w, y, y_dtype, M))
        return;
    // The vector kernels read 16-byte words of weights and activations.
    const bool aligned = reinterpret_cast<uintptr_t>(w->wq) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const bool gemv = aligned && q4_gemv_eligible(w, M, x_dtype, work ? work_bytes : kWorkspaceBytes);
    if (mode == 3) return launch_generic(x, x_dtype, w, y, y_dtype, M);
    if (mode == 4) return launch_gemm_exact(BFormat::Q4Generic, ga);
    if (mode == 0 && M > 1 && M <= 8 && x_dtype == BYHIP_F32 && !exact && w->f16_safe && aligned &&
        w->K % 32 == 0 && q4_fast(w) && q4_f32_wide_takes(ga) &&
        !(M == 2 && gemv && gemv_rows_per_launch(w->K, M, x_dtype) >= 2))
        return launch_gemm(BFormat::Q4Fast, ga);
    {
        const int dt = env_int("BYHIP_Q4_DECODE_TILE", -1);
        if (mode == 0 && M > 1 && M <= 8 && x_dtype == BYHIP_F16 && !exact && w->f16_safe && aligned &&
            q4_fast(w) &&
            (dt == 1 || (dt < 0 && (M > 4 || !gemv || gemv_rows_per_launch(w->K, M, x_dtype) < M))) &&
            launch_q4_wide_exact_weights(ga))
            return;
    }
    if (gemv && (mode == 1 || (mode == 0 && M <= 8)))
        return launch_q4_gemv(x, x_dtype, w, y, y_dtype, M, work, work_bytes);
    // Decode shapes the GEMV does not take (K or the group not a multiple of 32, unaligned rows or
    // activations, offsets past 32 bits) stay on the exact per-element kernel.
    if (M <= 8 && mode != 2) return launch_generic(x, x_dtype, w, y, y_dtype, M);
    if (!exact && w->f16_safe && aligned && w->K % 32 == 0)
        return launch_gemm(q4_fast(w) ? BFormat::Q4Fast : BFormat::Q4Generic, ga);
    launch_gemm_exact(BFormat::Q4Generic, ga);
}

}  // namespace

void q4_matmul_run(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, bool exact) {
    q4_matmul_impl(x, x_dtype, w, y, y_dtype, M, exact, nullptr, 0);
}

void q4_matmul_run_scratch(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, void* work,
                           size_t work_bytes) {
    q4_matmul_impl(x, x_dtype, w, y, y_dtype, M, false, work, work_bytes);
}

bool q4_run_plan(const Q4Plan& p, const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    const bool aligned = reinterpret_cast<uintptr_t>(w->wq) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    switch (p.kind) {
    case kPlanGeneric:
        launch_generic(x, x_dtype, w, y, y_dtype, M);
        return true;
    case kPlanExact:
        launch_gemm_exact(BFormat::Q4Generic, q4_gemm_args(x, x_dtype, w, y, y_dtype, M));
        return true;
    case kPlanGemv:
        if (!aligned || M > 8 || !q4_gemv_eligible(w, M, x_dtype)) return false;
        launch_q4_gemv(x, x_dtype, w, y, y_dtype, M);
        return true;
    case kPlanPipe:
    case kPlanSkinny:
    case kPlanGemm:
    case kPlanBig:
    case kPlanStream:
    case kPlanWide: {
        // fp16 MFMA kernels: only for weights whose products stay in fp16's normal range
        if (!aligned || w->K % 32 != 0 || !w->f16_safe) return false;
        const int kind = p.kind == kPlanPipe     ? kQ4Pipe
                         : p.kind == kPlanSkinny ? kQ4Skinny
                         : p.kind == kPlanBig    ? kQ4Big
                         : p.kind == kPlanWide   ? kQ4Wide
                         : p.kind == kPlanStream ? kQ4Stream
                                                 : kQ4General;
        return launch_q4_choice(q4_fast(w) ? BFormat::Q4Fast : BFormat::Q4Generic,
                                q4_gemm_args(x, x_dtype, w, y, y_dtype, M), kind, p.tile, p.splits);
    }
    default:
        return false;
    }
}

}  // namespace byhip

using namespace byhip;

extern "C" {

int byhip_q4_resident_upload(const uint8_t* wq, size_t wq_bytes, size_t wq_off, const float* scales,
                             const float* zeros, int K, int N, int group_size, int groups_per_row,
                             byhip_q4w** out) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_q4_resident_upload");
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
        no_host_sync("byhip_q4_resident_from_device");
        if (!out) fail("byhip: null output handle");
        *out = nullptr;
        validate_q4_shape(K, N, group_size, groups_per_row);
        const size_t wq_bytes = (size_t)N * ((size_t)(K + 1) / 2);
        const size_t ng = (size_t)N * groups_per_row;
        check_span(static_cast<const uint8_t*>(d_wq) + wq_off, wq_bytes, "Q4 packed weights");
        check_span(d_scales, ng * 4, "Q4 scales");
        check_span(d_zeros, ng * 4, "Q4 zeros");
        *out = build_resident_dev(static_cast<const uint8_t*>(d_wq) + wq_off, true,
                                  static_cast<const float*>(d_scales), static_cast<const float*>(d_zeros), K, N,
                                  group_size, groups_per_row);
    });
}

int byhip_q4_resident_free(byhip_q4w* w) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_q4_resident_free");
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
        out->zero_value = w->zero_value; out->device_bytes = w->bytes; out->f16_safe = w->f16_safe;
    });
}

int byhip_q4_matmul(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M) {
    return guard([&] {
        enter_compute();
        note_device_write(y);
        q4_matmul_impl(x, x_dtype, w, y, y_dtype, M, false, nullptr, 0);
    });
}

int byhip_q4_matmul_fused(int mode, const float* a, byhip_q4w* const* ws, int n_ws, float* const* outs,
                          int n_outs, const float* res, int has_res, const float* gamma, float eps,
                          int has_norm) {
    return guard([&] {
        enter_compute();
        if (!a) fail("byhip: null fused GEMV input");
        if (!ws || !outs) unsupported("byhip: fused GEMV without weights or outputs");
        // The reference's encoders return false for these (gpubackend.nim:3200-3206, 3219-3225).
        if (n_ws < 1 || n_ws > 3 || n_outs < n_ws || (mode == 1 && n_ws != 2) || (mode != 0 && mode != 1))
            unsupported("byhip: fused GEMV takes 1..3 weights in mode 0, gate and up in mode 1 (mode=%d, %d weights, %d outputs)",
                        mode, n_ws, n_outs);
        if (has_res && !res) unsupported("byhip: fused GEMV residual requested without a buffer");
        if (has_norm && !gamma) unsupported("byhip: fused GEMV norm requested without weights");
        // The reference wants an allocated output per weight, also in mode 1, where only outs[0]
        // is written (gpubackend.nim:3204-3206).
        for (int i = 0; i < n_ws; ++i)
            if (!outs[i]) unsupported("byhip: fused GEMV output %d is not allocated", i);
        const int n_out = mode == 1 ? 1 : n_ws;
        if (q4_fused_check(mode, ws, n_ws) != BYHIP_OK)
            unsupported("byhip: fused GEMV does not take these weights (K, group, groups per row and "
                        "scale formats must match, K %% 32 == 0, equal N for gate and up)");
        const int K = ws[0]->K;
        int max_n = 0;
        for (int i = 0; i < n_ws; ++i) max_n = std::max(max_n, ws[i]->N);
        check_span(a, (size_t)K * 4, "fused GEMV input");
        for (int i = 0; i < n_out; ++i) check_span(outs[i], (size_t)ws[i]->N * 4, "fused GEMV output");
        if (has_res) check_span(res, (size_t)(mode == 1 ? ws[0]->N : max_n) * 4, "fused GEMV residual");
        if (has_norm) check_span(gamma, (size_t)K * 4, "fused GEMV norm weights");
        for (int i = 0; i < n_out; ++i) note_device_write(outs[i]);
        launch_q4_gemv_fused(mode, a, ws, n_ws, outs, has_res ? res : nullptr, has_norm ? gamma : nullptr, eps);
    });
}

int byhip_gpu_matmul_q4(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                        float* c, int M, int K, int N, int group_size, int groups_per_row) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_gpu_matmul_q4");
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
            q4_matmul_impl(dx, BYHIP_F32, w, dy, BYHIP_F32, M, false, nullptr, 0);
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
        no_host_sync("byhip_debug_unpack_q4");
        if (!w || !codes || !scales || !zeros) fail("byhip: null argument");
        const size_t total = (size_t)w->N * w->K, ng = (size_t)w->N * w->gpr;
        uint8_t* dc = static_cast<uint8_t*>(device_alloc(total));
        float* ds = static_cast<float*>(device_alloc(ng * 4));
        float* dz = static_cast<float*>(device_alloc(ng * 4));
        const size_t n = std::max(total, ng);
        const int grid = (int)((n + 255) / 256);
        try {
            launch("q4_unpack", q4_unpack, dim3(grid), dim3(256), 0, w->wq, w->row_bytes, w->K,
                               w->N, w->scales, w->scale_f16, w->zeros, w->zero_value, w->sblk, w->zblk,
                               w->group, w->gpr, dc, ds, dz);
        } catch (...) {
            device_free(dc);
            device_free(ds);
            device_free(dz);
            throw;
        }
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
