// byhip_gemv.hip - the Q4 decode GEMV (M <= 8) for resident or slot-bound Q4 weights (gfx950).
//
// y[m, n] = sum_k x[m, k] * ((float)q[n, k] - zero[n, g]) * scale[n, g] with fp32 accumulation
// (cpu_kernels_impl.inc:293-319, cpu_vm.c:420-482).
//
// Work split: a wave owns R consecutive weight rows (4 or 8 when a row is at most two 32-value chunks
// per lane); lane l holds chunks l, l + 64, ... of every row, each chunk one 16-byte load of 32
// nibbles.
// Per wave the loads go out in this order, all before the first wait: the block's activations, the
// scales (one load per chunk covers the wave's rows: the resident layout blocks them by 8), then the
// weight rows; the wait counter completes in issue order, so row r is processed as soon as it
// lands.
//
// Activations are staged once per 256-thread block in LDS: each 32-value chunk as 16 fp16 pairs
// (x[8j+i], x[8j+i+4]) matching the nibble pairs below, with its sums of x.
//
// Nibble pairs become fp16 with one AND-OR against an exponent word: 0x6400 | q is 1024 + q and
// 0x5400 | (q << 4) is 64 + q, both exact; v_dot2_f32_f16 multiplies them with the x pairs (exact
// products, fp32 accumulation). With fp16 activations the biased halves go into the dot products
// and the bias (1024 and 64 times the chunk's sums of x over the low and high nibble pairs) is
// removed once per chunk; the fp32 sum then carries about 2^-13 of the bias as rounding, well below
// the fp16 output's own. With fp32 activations the bias is subtracted from the halves first (exact)
// and x is split into two fp16 terms (hi + lo, ~22 bits). The zero point enters once per chunk as
// s * (sum x*q - z * sum x).
//
// fp32 range: each 32-value chunk of fp32 activations is multiplied by an exact power of two 2^t
// that brings its largest magnitude into [2^14, 2^15) before the split, and the chunk's partial is
// multiplied by 2^-t (folded into its scale). So any finite fp32 input keeps its ~22 bits: nothing
// overflows fp16, and only values more than 2^28 below the chunk's largest reach fp16 subnormals
// (an absolute error below 2^-39 of that largest value). Non-finite inputs give non-finite outputs.
#include <algorithm>

#include "byhip_gemm.h"
#include "byhip_gemv.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Weight rows a wave keeps in flight: 8 rows of up to two chunks per lane, fewer when each row
// needs more chunks (16 chunk loads in flight per lane at most). A single activation row takes 2:
// more waves, so the dequantization and reduction left after the last loads land are spread
// thinner. Measured on MI355X at K = 4096, N = 14336 in a standalone copy of this kernel: 7.54 us
// with 2 rows per wave, 7.85 with 4, 8.05 with 8, 8.13 with 1 (too many waves to launch), while
// the weight loads alone take 6.35-6.7 us; this kernel in the library: 7.6-7.7 us with 2 rows.
// With several activation rows the larger batch wins.
constexpr int gemv_rows(int m, int cpl) { return cpl >= 8 ? 2 : (m == 1 ? 2 : (cpl >= 4 ? 4 : 8)); }

struct GemvArgs {
    const void* x;
    const uint8_t* wq;
    const void* scales;  // resident: [ceil(N/8)][K/32][8]; slots: [N][gpr]
    const float* zeros;  // same layout as scales (fp32); null when the zero point is uniform
    float zero_value;
    void* y;
    int K, N, group_chunks, gpr, row_bytes, n_pad;
    // K slices (blockIdx.y): slice z takes chunks z * slice_chunks .. of the Gt 32-value chunks of
    // a row and, when there are several, writes fp32 partial sums to y + z * ystride (split-K);
    // ldx is the activation row stride in elements.
    int Gt, slice_chunks, ldx;
    size_t ystride;
};

template <int NB>
__device__ __forceinline__ void load_bytes(rsrc_t r, uint32_t off, uint32_t* w) {
    if constexpr (NB == 4) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    } else if constexpr (NB == 8) {
        const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        w[0] = v[0]; w[1] = v[1];
    } else if constexpr (NB == 16) {
        const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    } else {
        static_assert(NB == 32, "scale block width");
        const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        const v4u u = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0);
        w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
        w[4] = u[0]; w[5] = u[1]; w[6] = u[2]; w[7] = u[3];
    }
}

template <int M, int CPL, bool XF32, bool SF16, bool ZU, bool BLK, int YT>
__global__ __launch_bounds__(256) void q4_gemv(GemvArgs a) {
    constexpr int XS = XF32 ? 2 : 1;
    // A single fp32 row reads its activations from LDS where each weight row uses them: past 4
    // chunks per lane they do not fit the register tile, and below it holding them took the
    // registers of 3 waves per SIMD (K = 4096: 107 VGPRs, 4 waves per SIMD, against 7 reading
    // LDS; 11.6 -> 9.7 us at N = 14336, 5.3 -> 4.8 at N = 4096, together with XHALF).
    constexpr bool XLDS = M * CPL * XS > 8 || (XF32 && M == 1);
    static_assert(!XLDS || M == 1, "the launcher slices rows so that only one-row launches read x from LDS");
    constexpr int R = gemv_rows(M, CPL);
    constexpr uint32_t XB = XF32 ? 4 : 2;  // bytes per activation
    constexpr int XW = XF32 ? 8 : 4;       // 16-byte activation loads per 32-value chunk
    // activation chunks a thread stages: M * G <= M * 64 * CPL chunks over 256 threads (at most 512)
    constexpr int XC = (M * CPL + 3) / 4 < 2 ? (M * CPL + 3) / 4 : 2;
    // fp32 activations with at most 256 half chunks: each thread stages half a chunk (16 values),
    // the pair of lanes sharing the chunk's maximum and sum, so that the staging holds 16 values
    // per thread instead of 32 (with x read from LDS, the staging was the register peak at M = 1,
    // K <= 4096)
    constexpr bool XHALF = XF32 && M * CPL <= 2;
    constexpr int XWL = XHALF ? XW / 2 : XW;  // 16-byte activation loads a thread issues per chunk
    constexpr uint32_t SB = SF16 ? 2u : 4u;
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int N = a.N, Gt = a.Gt;
    // this block's K slice: chunks c0 .. c0 + G - 1 of a row
    const int c0 = blockIdx.y * a.slice_chunks;
    const int G = min(a.slice_chunks, Gt - c0);
    const int n0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + (tid >> 6)) * R);
    const bool rows_live = n0 < N;  // uniform in the wave; every wave takes part in the barrier

    // Staged chunk idx (= m G + chunk) as four 16-byte pieces, piece t at uint4 index t M G + idx:
    // a wave's reads of piece t (64 consecutive chunks) and the staging writes then touch
    // consecutive 16-byte units, which read with no LDS bank conflict; with each chunk's 64 bytes
    // contiguous, the lanes' 16-byte reads were 64 bytes apart, 12 conflict cycles per read
    // (both measured on the MI355X with the hardware's conflict counter).
    uint32_t* xh = lds;                                   // [4][M][G][4] fp16 pairs
    uint32_t* xl = xh + M * G * 16;                       // [4][M][G][4] low terms (fp32 x only)
    float* sums = reinterpret_cast<float*>(xl + (XS == 2 ? M * G * 16 : 0));  // [M][G]{bias, sum}

    const rsrc_t wr = make_rsrc(a.wq, (uint32_t)N * (uint32_t)a.row_bytes);
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)M * (uint32_t)a.ldx * XB);
    const uint32_t srows = BLK ? (uint32_t)a.n_pad : (uint32_t)N;
    const rsrc_t sr = make_rsrc(a.scales, srows * (uint32_t)(BLK ? Gt : a.gpr) * SB);
    const rsrc_t zr = make_rsrc(ZU ? a.scales : a.zeros, ZU ? 0u : srows * (uint32_t)(BLK ? Gt : a.gpr) * 4u);

    // This lane's chunks of the slice (chunks past its end are clamped onto its last one and their
    // scale is zeroed): lch is the chunk within the slice (the staging index), coff its byte offset
    // in the weight row.
    uint32_t coff[CPL], gsel[CPL];
    int lch[CPL];
    bool cv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ci = lane + kWave * c;
        cv[c] = ci < G;
        const int cc = min(ci, G - 1);
        lch[c] = cc;
        coff[c] = (uint32_t)(c0 + cc) * 16u;
        gsel[c] = BLK ? (uint32_t)(c0 + cc) : (uint32_t)(a.group_chunks ? (c0 + cc) / a.group_chunks : 0);
    }

    // 1. the activations this thread stages. fp16: 16-byte pieces tid, tid + 256, ... of the M x G
    // chunks' 4 M G pieces, so that a wave's loads cover 1 KB of consecutive bytes (whole lines;
    // loading a chunk's 64 bytes per lane touched four times the lines). fp32: chunks tid and
    // tid + 256 (with XHALF half hf = tid & 1 of chunk tid / 2).
    constexpr bool XPIECE = !XF32;
    constexpr int XP = XPIECE ? M * CPL : 1;  // pieces per thread: 4 M G <= 256 M CPL
    uint4 xpc[XP];
    if constexpr (XPIECE) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int pc = tid + 256 * i, idx = pc >> 2, m = idx / G, ci = idx - m * G;
            xpc[i] = buf_load16(xr, idx < M * G ? (uint32_t)m * (uint32_t)a.ldx * XB + (uint32_t)(c0 + ci) * 64u + 16u * (pc & 3)
                                                : kOutOfRange);
        }
    }
    uint4 xraw[XPIECE ? 1 : XC][XWL];
    const int hf = XHALF ? (tid & 1) : 0;
#pragma unroll
    for (int i = 0; i < (XPIECE ? 0 : XC); ++i) {
        const int idx = XHALF ? tid >> 1 : tid + 256 * i;
        const int m = idx / G, ci = idx - m * G;
        const uint32_t base = idx < M * G ? (uint32_t)m * (uint32_t)a.ldx * XB + (uint32_t)(c0 + ci) * 32u * XB + 64u * (uint32_t)hf
                                          : kOutOfRange;
#pragma unroll
        for (int t = 0; t < XWL; ++t) xraw[i][t] = buf_load16(xr, base == kOutOfRange ? kOutOfRange : base + 16u * t);
    }

    // 2. scales and zeros of the wave's R rows
    uint32_t sraw[R][CPL], zraw[R][CPL];
    // first row of the batch; a wave past the end reads the last (aligned) batch and stores nothing
    const int nb = BLK ? min(n0, a.n_pad - R) : min(n0, N - 1);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if constexpr (BLK) {
            // rows n0 .. n0+R-1 of chunk c sit together: [(n0/8) * G + chunk] * 8 + n0 % 8
            const uint32_t e = ((uint32_t)(nb >> 3) * (uint32_t)Gt + gsel[c]) * 8u + (uint32_t)(nb & 7);
            uint32_t sw[R * SB / 4];
            load_bytes<R * SB>(sr, e * SB, sw);
#pragma unroll
            for (int r = 0; r < R; ++r)
                sraw[r][c] = SF16 ? ((sw[r >> 1] >> (16 * (r & 1))) & 0xFFFFu) : sw[r];
            if constexpr (!ZU) {
                uint32_t zw[R];
                load_bytes<R * 4>(zr, e * 4u, zw);
#pragma unroll
                for (int r = 0; r < R; ++r) zraw[r][c] = zw[r];
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t g = (uint32_t)min(nb + r, N - 1) * (uint32_t)a.gpr + gsel[c];
                if constexpr (SF16)
                    sraw[r][c] = __builtin_amdgcn_raw_buffer_load_b16(sr, g * SB, 0, 0);
                else
                    sraw[r][c] = __builtin_amdgcn_raw_buffer_load_b32(sr, g * SB, 0, 0);
                if constexpr (!ZU) zraw[r][c] = __builtin_amdgcn_raw_buffer_load_b32(zr, g * 4u, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. the weight rows in row order (streamed once: non-temporal); the row offset is
    // wave-uniform and travels in the scalar offset
    uint4 wv[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t roff = (uint32_t)min(nb + r, N - 1) * (uint32_t)a.row_bytes;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wr, coff[c], roff, 2);
            wv[r][c] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load is out before the first wait

    // 4. stage the activations: fp16 pairs matching the nibble pairs, and the chunk sums
    if constexpr (XHALF) {
        // values 16 hf .. 16 hf + 15 of chunk idx: pieces 2 hf and 2 hf + 1 (both lanes of a pair
        // take the branch together, so each reads its partner's maximum and sum)
        const int idx = tid >> 1;
        if (idx < M * G) {
            float v[16];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v[4 * t] = __builtin_bit_cast(float, xraw[0][t].x);
                v[4 * t + 1] = __builtin_bit_cast(float, xraw[0][t].y);
                v[4 * t + 2] = __builtin_bit_cast(float, xraw[0][t].z);
                v[4 * t + 3] = __builtin_bit_cast(float, xraw[0][t].w);
            }
            float mx = 0.0f;
#pragma unroll
            for (int t = 0; t < 16; ++t) mx = fmaxf(mx, fabsf(v[t]));
            mx = fmaxf(mx, __shfl_xor(mx, 1, kWave));
            const int sh = fp16_range_shift(mx);
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                v[t] = __builtin_amdgcn_ldexpf(v[t], sh);
                s += v[t];
            }
            s += __shfl_xor(s, 1, kWave);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t p[4], lo[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float u = v[8 * j + q], w = v[8 * j + q + 4];
                    const _Float16 hu = (_Float16)u, hw = (_Float16)w;
                    const _Float16 lu = (_Float16)(u - (float)hu), lw = (_Float16)(w - (float)hw);
                    p[q] = (uint32_t)h_bits(hu) | ((uint32_t)h_bits(hw) << 16);
                    lo[q] = (uint32_t)h_bits(lu) | ((uint32_t)h_bits(lw) << 16);
                }
                const int t = 2 * hf + j;
                reinterpret_cast<uint4*>(xh)[idx + t * M * G] = make_uint4(p[0], p[1], p[2], p[3]);
                reinterpret_cast<uint4*>(xl)[idx + t * M * G] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            }
            if (hf == 0) {
                sums[2 * idx] = __builtin_amdgcn_ldexpf(1.0f, -sh);  // the back-scale rides in the bias slot
                sums[2 * idx + 1] = s;
            }
        }
    }
    if constexpr (XPIECE) {
        // piece t of chunk idx holds x[8 t .. 8 t + 7]: its pairs (x[8t+q], x[8t+q+4]) are piece t
        // of the staged chunk, and its sums over the low- and high-nibble pairs are added over the
        // chunk's four lanes (exact products with 1, fp32 accumulation)
        const h2 one = {1, 1};
#pragma unroll
        for (int i = 0; i < XP; ++i) {
            const int pc = tid + 256 * i, idx = pc >> 2, t = pc & 3;
            const uint32_t A = xpc[i].x, B = xpc[i].y, C = xpc[i].z, D = xpc[i].w;
            const uint32_t p0 = __builtin_amdgcn_perm(C, A, 0x05040100u), p1 = __builtin_amdgcn_perm(C, A, 0x07060302u);
            const uint32_t p2 = __builtin_amdgcn_perm(D, B, 0x05040100u), p3 = __builtin_amdgcn_perm(D, B, 0x07060302u);
            float sl = __builtin_amdgcn_fdot2(bits_h2(p0), one, 0.0f, false);
            sl = __builtin_amdgcn_fdot2(bits_h2(p2), one, sl, false);
            float sh = __builtin_amdgcn_fdot2(bits_h2(p1), one, 0.0f, false);
            sh = __builtin_amdgcn_fdot2(bits_h2(p3), one, sh, false);
            sl += __shfl_xor(sl, 1, kWave);
            sh += __shfl_xor(sh, 1, kWave);
            sl += __shfl_xor(sl, 2, kWave);
            sh += __shfl_xor(sh, 2, kWave);
            if (idx < M * G) {
                reinterpret_cast<uint4*>(xh)[t * M * G + idx] = make_uint4(p0, p1, p2, p3);
                if (t == 0) {
                    sums[2 * idx] = 1024.0f * sl + 64.0f * sh;
                    sums[2 * idx + 1] = sl + sh;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < (XHALF || XPIECE ? 0 : XC); ++i) {
        const int idx = tid + 256 * i;
        if (idx < M * G) {
            uint32_t p[16], lo[16];
            float bias = 0.0f, s = 0.0f;
            if constexpr (XF32) {
                float v[32];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    v[4 * t] = __builtin_bit_cast(float, xraw[i][t].x);
                    v[4 * t + 1] = __builtin_bit_cast(float, xraw[i][t].y);
                    v[4 * t + 2] = __builtin_bit_cast(float, xraw[i][t].z);
                    v[4 * t + 3] = __builtin_bit_cast(float, xraw[i][t].w);
                }
                // the chunk onto fp16's range: x * 2^sh; the partial is scaled back by 2^-sh
                float mx = 0.0f;
#pragma unroll
                for (int t = 0; t < 32; ++t) mx = fmaxf(mx, fabsf(v[t]));
                const int sh = fp16_range_shift(mx);
#pragma unroll
                for (int t = 0; t < 32; ++t) v[t] = __builtin_amdgcn_ldexpf(v[t], sh);
                bias = __builtin_amdgcn_ldexpf(1.0f, -sh);  // the back-scale rides in the bias slot
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float u = v[8 * j + q], w = v[8 * j + q + 4];
                        const _Float16 hu = (_Float16)u, hw = (_Float16)w;
                        const _Float16 lu = (_Float16)(u - (float)hu), lw = (_Float16)(w - (float)hw);
                        p[4 * j + q] = (uint32_t)h_bits(hu) | ((uint32_t)h_bits(hw) << 16);
                        lo[4 * j + q] = (uint32_t)h_bits(lu) | ((uint32_t)h_bits(lw) << 16);
                    }
#pragma unroll
                for (int t = 0; t < 32; ++t) s += v[t];
            } else {
                uint32_t d[16];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    d[4 * t] = xraw[i][t].x; d[4 * t + 1] = xraw[i][t].y;
                    d[4 * t + 2] = xraw[i][t].z; d[4 * t + 3] = xraw[i][t].w;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t A = d[4 * j], B = d[4 * j + 1], C = d[4 * j + 2], D = d[4 * j + 3];
                    p[4 * j + 0] = __builtin_amdgcn_perm(C, A, 0x05040100u);
                    p[4 * j + 1] = __builtin_amdgcn_perm(C, A, 0x07060302u);
                    p[4 * j + 2] = __builtin_amdgcn_perm(D, B, 0x05040100u);
                    p[4 * j + 3] = __builtin_amdgcn_perm(D, B, 0x07060302u);
                }
                // sums over the low-nibble pairs (p[4j], p[4j+2]) and high-nibble pairs (p[4j+1],
                // p[4j+3]): exact products with 1, fp32 accumulation
                const h2 one = {1, 1};
                float sl = 0.0f, sh = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sl = __builtin_amdgcn_fdot2(bits_h2(p[4 * j + 0]), one, sl, false);
                    sl = __builtin_amdgcn_fdot2(bits_h2(p[4 * j + 2]), one, sl, false);
                    sh = __builtin_amdgcn_fdot2(bits_h2(p[4 * j + 1]), one, sh, false);
                    sh = __builtin_amdgcn_fdot2(bits_h2(p[4 * j + 3]), one, sh, false);
                }
                s = sl + sh;
                bias = 1024.0f * sl + 64.0f * sh;
            }
            uint4* dh = reinterpret_cast<uint4*>(xh) + idx;
#pragma unroll
            for (int t = 0; t < 4; ++t) dh[t * M * G] = make_uint4(p[4 * t], p[4 * t + 1], p[4 * t + 2], p[4 * t + 3]);
            if constexpr (XS == 2) {
                uint4* dl = reinterpret_cast<uint4*>(xl) + idx;
#pragma unroll
                for (int t = 0; t < 4; ++t) dl[t * M * G] = make_uint4(lo[4 * t], lo[4 * t + 1], lo[4 * t + 2], lo[4 * t + 3]);
            }
            sums[2 * idx] = bias;
            sums[2 * idx + 1] = s;
        }
    }
    __syncthreads();
    if (!rows_live) return;

    // The staged activation pairs of (row m, lane chunk c): held in registers for the whole row
    // loop when they fit (XLDS false), else read from LDS where each row uses them.
    constexpr int XM = XLDS ? 1 : M, XCP = XLDS ? 1 : CPL;
    uint32_t xp[XM][XCP][16];
    uint32_t xq[XS == 2 ? XM : 1][XS == 2 ? XCP : 1][16];
    float bias[M][CPL], sx[M][CPL];
    auto read_x = [&](int m, int c, uint32_t* hp, uint32_t* lp) {
        const int idx = m * G + lch[c];
        const uint4* sh = reinterpret_cast<const uint4*>(xh) + idx;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint4 u = sh[t * M * G];
            hp[4 * t] = u.x; hp[4 * t + 1] = u.y; hp[4 * t + 2] = u.z; hp[4 * t + 3] = u.w;
        }
        if constexpr (XS == 2) {
            const uint4* sl = reinterpret_cast<const uint4*>(xl) + idx;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint4 u = sl[t * M * G];
                lp[4 * t] = u.x; lp[4 * t + 1] = u.y; lp[4 * t + 2] = u.z; lp[4 * t + 3] = u.w;
            }
        }
    };
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int idx = m * G + lch[c];
            if constexpr (!XLDS) read_x(m, c, xp[m][c], xq[XS == 2 ? m : 0][XS == 2 ? c : 0]);
            bias[m][c] = sums[2 * idx];
            sx[m][c] = sums[2 * idx + 1];
        }

    // Nibble n at bits 0-3 of a half: 0x6400 | n is the fp16 1024 + n; at bits 4-7: 0x5400 | (n << 4)
    // is the fp16 64 + n. The magic words live in VGPRs so the AND-OR is one v_and_or_b32.
    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));
    const h2 bias_lo = {1024, 1024}, bias_hi = {64, 64};

    // 5. rows in load order; each row is reduced over the wave and stored before the next
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t dw[4] = {wv[r][c].x, wv[r][c].y, wv[r][c].z, wv[r][c].w};
            h2 q[16];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t d8 = dw[w] >> 8;
                q[4 * w + 0] = bits_h2((dw[w] & 0x000F000Fu) | mag_lo);
                q[4 * w + 1] = bits_h2((dw[w] & 0x00F000F0u) | mag_hi);
                q[4 * w + 2] = bits_h2((d8 & 0x000F000Fu) | mag_lo);
                q[4 * w + 3] = bits_h2((d8 & 0x00F000F0u) | mag_hi);
                if constexpr (XS == 2) {  // fp32 activations: remove the bias exactly here
                    q[4 * w + 0] -= bias_lo;
                    q[4 * w + 1] -= bias_hi;
                    q[4 * w + 2] -= bias_lo;
                    q[4 * w + 3] -= bias_hi;
                }
            }
            float s = SF16 ? (float)bits_h((uint16_t)sraw[r][c]) : __builtin_bit_cast(float, sraw[r][c]);
            s = cv[c] ? s : 0.0f;
            const float z = ZU ? a.zero_value : __builtin_bit_cast(float, zraw[r][c]);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint32_t* hp = xp[XLDS ? 0 : m][XLDS ? 0 : c];
                const uint32_t* lp = xq[XS == 2 && !XLDS ? m : 0][XS == 2 && !XLDS ? c : 0];
                if constexpr (XLDS) read_x(m, c, xp[0][0], xq[0][0]);
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    p = __builtin_amdgcn_fdot2(bits_h2(hp[e]), q[e], p, false);
                    if constexpr (XS == 2) p = __builtin_amdgcn_fdot2(bits_h2(lp[e]), q[e], p, false);
                }
                // fp32 x: the bias slot holds the chunk's back-scale 2^-sh
                if constexpr (XS == 2) acc[m] = fmaf(s * bias[m][c], p - z * sx[m][c], acc[m]);
                else acc[m] = fmaf(s, (p - bias[m][c]) - z * sx[m][c], acc[m]);
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float t = wave_sum_lane63(acc[m]);
            if (lane == 63 && n0 + r < N) store_y<YT>(a.y, blockIdx.y * a.ystride + (size_t)m * N + n0 + r, t);
        }
    }
}

template <int M, int CPL, bool XF32, bool SF16, bool ZU, bool BLK>
void launch_y(const GemvArgs& a, int y_dtype) {
    constexpr int R = gemv_rows(M, CPL);
    const int G = a.slice_chunks;
    const size_t lds = (size_t)M * G * 16 * 4 * (XF32 ? 2 : 1) + (size_t)M * G * 2 * 4;
    // one batch of rows per wave; one block row per K slice
    const dim3 grid((a.N + 4 * R - 1) / (4 * R), (a.Gt + G - 1) / G);
    switch (y_dtype) {
    case BYHIP_F32:
        launch("q4_gemv", (q4_gemv<M, CPL, XF32, SF16, ZU, BLK, BYHIP_F32>), grid, dim3(256), lds, a);
        break;
    case BYHIP_F16:
        launch("q4_gemv", (q4_gemv<M, CPL, XF32, SF16, ZU, BLK, BYHIP_F16>), grid, dim3(256), lds, a);
        break;
    default:
        launch("q4_gemv", (q4_gemv<M, CPL, XF32, SF16, ZU, BLK, BYHIP_BF16>), grid, dim3(256), lds, a);
        break;
    }
    BYHIP_LAUNCHED("q4_gemv");
}

template <int M, int CPL, bool XF32>
void launch_szb(const GemvArgs& a, const byhip_q4w* w, bool blk, int y_dtype) {
    if constexpr (M > 1 && M * CPL * (XF32 ? 2 : 1) > 8) {
        fail("byhip: internal: GEMV register tile out of range");
    } else {
        const bool sf = blk ? w->blk_scale_f16 : w->scale_f16;
        const bool zu = w->zero_uniform;
#define BYHIP_GEMV_CASE(SF, ZU_, BLK_) \
    if (sf == SF && zu == ZU_ && blk == BLK_) return launch_y<M, CPL, XF32, SF, ZU_, BLK_>(a, y_dtype);
        BYHIP_GEMV_CASE(true, true, true)
        BYHIP_GEMV_CASE(true, false, true)
        BYHIP_GEMV_CASE(false, true, true)
        BYHIP_GEMV_CASE(false, false, true)
        BYHIP_GEMV_CASE(true, true, false)
        BYHIP_GEMV_CASE(true, false, false)
        BYHIP_GEMV_CASE(false, true, false)
        BYHIP_GEMV_CASE(false, false, false)
#undef BYHIP_GEMV_CASE
    }
}

template <int M, bool XF32>
void launch_cpl(int cpl, const GemvArgs& a, const byhip_q4w* w, bool blk, int y_dtype) {
    switch (cpl) {
    case 1: launch_szb<M, 1, XF32>(a, w, blk, y_dtype); break;
    case 2: launch_szb<M, 2, XF32>(a, w, blk, y_dtype); break;
    case 4: launch_szb<M, 4, XF32>(a, w, blk, y_dtype); break;
    default: launch_szb<M, 8, XF32>(a, w, blk, y_dtype); break;
    }
}

// Chunks of 32 values per lane the GEMV keeps in registers for K (a power of two up to 8).
int gemv_cpl(int K) {
    const int G = K / 32;
    int cpl = 1;
    while (cpl * kWave < G) cpl *= 2;
    return cpl;
}

// The GEMV's K slices. One slice holds all of K when the per-lane register tile (8 chunks of 32
// values per lane: 512 chunks) and the block's staging take it: with fp32 activations each staged
// chunk needs 136 bytes of the 64 KB of LDS (481 chunks, K = 15,392). Longer rows are cut into
// equal slices that do fit; each slice's blocks write fp32 partial sums and splitk_sum adds them
// in slice order.
struct GemvSlices {
    int slices, chunks;
};
GemvSlices gemv_slices(int K, int x_dtype) {
    const int G = K / 32, maxc = x_dtype == BYHIP_F32 ? 481 : 512;
    if (G <= maxc) return {1, G};
    const int s = (G + maxc - 1) / maxc;
    return {s, (G + s - 1) / s};
}

// ---- fused decode GEMV (sessionMatmulQ4Fused, gpubackend.nim:3185-3231) ----------------------
//
// M = 1, fp32 input and outputs, resident weights with the blocked scale copy. The shader it
// replaces (q4_autotune.nim:194-330) computes, per output row, sum_k ((q - z) * s) * x[k] with
// x[k] = a[k] * gamma[k] under RMSNorm, scales the sum by inv = 1 / sqrt(sum a^2 / K + eps), and
// in mode 1 returns silu(gate) * up; the residual is added last.
//   mode 0: up to three matrices share the input; a wave's batch of 4 rows lies in one matrix
//   (batches are numbered per matrix), so the matrix is wave-uniform.
//   mode 1: a wave loads 4 rows of gate and the same 4 rows of up.
// The input is staged once per block as in q4_gemv (fp16 hi/lo pairs in the (k, k+4) order of the
// nibble pairs, and the chunk sums for the zero point), after the norm weight is applied; the
// block also sums a^2 for the norm factor (partials per thread, added in a fixed order).
struct FusedMat {
    const uint8_t* wq;
    const void* sblk;   // [ceil(N/8)][K/32][8] scales (fp16 or fp32)
    const float* zblk;  // same layout, fp32 zeros; null when the zero point is uniform
    float zero_value;
    float* y;
    int N, n_pad, batch0;  // batch0: the first row batch of this matrix in the wave numbering
    int part_off;          // K slices: this matrix's rows in each slice's plane of partial sums
};

struct FusedArgs {
    const float* x;
    const float* res;    // null: no residual
    const float* gamma;  // null: no RMSNorm
    float eps;
    int K, row_bytes, nmats, batches;
    // K slices (blockIdx.y): slice z takes chunks z * slice_chunks .. of the Gt chunks. With several
    // slices the waves store their raw dot products to part[z * pstride + part_off + row], and
    // block 0 of each slice its sum of a^2 to ssq[z]; fused_finish applies the rest.
    int Gt, slice_chunks;
    float* part;
    float* ssq;
    size_t pstride;
    FusedMat m[3];
};

// Rows per wave and matrix: 2 when a row takes 8 chunks per lane (the weights a wave keeps in
// flight) and up to K = 4096, else 4. At K = 4096 two rows gave more waves with shorter tails:
// gate+up (2 x 14336 rows) 106 VGPRs against 129, 4 waves per SIMD instead of 3, 17.5 -> 16.7 us;
// QKV 6.35 -> 6.0 us, O 4.72 -> 4.65.
constexpr int fused_rows(int cpl) { return cpl >= 8 || cpl <= 2 ? 2 : 4; }

template <int CPL, bool SF16, bool ZU, int MODE>
__global__ __launch_bounds__(256) void q4_gemv_fused(FusedArgs a) {
    constexpr int R = fused_rows(CPL);
    constexpr int NM = MODE == 1 ? 2 : 1;  // matrices a wave reads
    constexpr uint32_t SB = SF16 ? 2u : 4u;
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int K = a.K, Gt = a.Gt;
    // this block's K slice: chunks c0 .. c0 + G - 1
    const int c0 = blockIdx.y * a.slice_chunks;
    const int G = min(a.slice_chunks, Gt - c0);
    // chunk idx as four 16-byte pieces, piece t at uint4 index t G + idx (conflict-free reads, as
    // in q4_gemv)
    uint32_t* xh = lds;                                      // [4][G][4] fp16 pairs, high terms
    uint32_t* xl = xh + G * 16;                              // [4][G][4] low terms
    float* sums = reinterpret_cast<float*>(xl + G * 16);     // [G] sum of the scaled x over the chunk
    float* facs = sums + G;                                  // [G] the chunk's back-scale 2^-sh
    float* ssq_part = facs + G;                              // [256]

    const int wb = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (tid >> 6));
    const bool live = wb < a.batches;  // uniform in the wave; every wave takes part in the barrier
    int mi = 0;
    if (MODE == 0) {
        if (a.nmats > 1 && wb >= a.m[1].batch0) mi = 1;
        if (a.nmats > 2 && wb >= a.m[2].batch0) mi = 2;
    }
    const FusedMat& fm0 = a.m[mi];
    const int n0 = (wb - fm0.batch0) * R;  // first matrix-local row of the wave

    // This lane's chunks of the slice (chunks past its end are clamped onto its last one and their
    // scale is zeroed): lch is the chunk within the slice (the staging index), coff its byte offset
    // in the weight row.
    uint32_t coff[CPL];
    int lch[CPL];
    bool cv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ci = lane + kWave * c;
        cv[c] = ci < G;
        lch[c] = min(ci, G - 1);
        coff[c] = (uint32_t)(c0 + lch[c]) * 16u;
    }

    // 1. the first input chunk this thread stages (chunk tid; chunk tid + 256 follows after the
    // weight loads are out) and its norm weights
    // Up to 2 chunks per lane (G <= 128) each thread stages half a chunk, values 16 hf .. 16 hf + 15
    // of chunk tid / 2, and the two lanes of a chunk exchange its maximum and sum: the staging
    // registers (the kernel's peak, beside the weights in flight) hold 16 values instead of 32.
    constexpr bool HALF = CPL <= 2;
    constexpr int XW = HALF ? 4 : 8;  // 16-byte loads per staged piece
    const int hf = HALF ? (tid & 1) : 0;
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)K * 4u);
    const rsrc_t gr = make_rsrc(a.gamma ? a.gamma : a.x, a.gamma ? (uint32_t)K * 4u : 0u);
    auto load_chunk = [&](int idx, uint4* xraw, uint4* graw) {
        const uint32_t base = idx < G ? (uint32_t)(c0 + idx) * 128u + 64u * (uint32_t)hf : kOutOfRange;
#pragma unroll
        for (int t = 0; t < XW; ++t) xraw[t] = buf_load16(xr, base == kOutOfRange ? kOutOfRange : base + 16u * t);
        if (a.gamma) {
#pragma unroll
            for (int t = 0; t < XW; ++t) graw[t] = buf_load16(gr, base == kOutOfRange ? kOutOfRange : base + 16u * t);
        }
    };
    uint4 xraw[XW], graw[XW];
    load_chunk(HALF ? tid >> 1 : tid, xraw, graw);

    // 2. scales and zeros, 3. weight rows of the wave's batch (per matrix), all before the first wait
    uint32_t sraw[NM][R][CPL], zraw[NM][R][CPL];
    uint4 wv[NM][R][CPL];
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        const FusedMat& fm = MODE == 1 ? a.m[j] : fm0;
        const rsrc_t sr = make_rsrc(fm.sblk, (uint32_t)fm.n_pad * (uint32_t)Gt * SB);
        const rsrc_t zr = make_rsrc(ZU ? fm.sblk : fm.zblk, ZU ? 0u : (uint32_t)fm.n_pad * (uint32_t)Gt * 4u);
        const int nb = min(n0, fm.n_pad - R);  // R divides 8 and n0, so the rows sit in one block of 8
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t e = ((uint32_t)(nb >> 3) * (uint32_t)Gt + (uint32_t)(c0 + lch[c])) * 8u + (uint32_t)(nb & 7);
            uint32_t sw[R * SB / 4];
            load_bytes<R * SB>(sr, e * SB, sw);
#pragma unroll
            for (int r = 0; r < R; ++r) sraw[j][r][c] = SF16 ? ((sw[r >> 1] >> (16 * (r & 1))) & 0xFFFFu) : sw[r];
            if constexpr (!ZU) {
                uint32_t zw[R];
                load_bytes<R * 4>(zr, e * 4u, zw);
#pragma unroll
                for (int r = 0; r < R; ++r) zraw[j][r][c] = zw[r];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NM; ++j) {
        const FusedMat& fm = MODE == 1 ? a.m[j] : fm0;
        const rsrc_t wr = make_rsrc(fm.wq, (uint32_t)fm.N * (uint32_t)a.row_bytes);
        // chunk-major, the order step 5 consumes them in
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t roff = (uint32_t)min(n0 + r, fm.N - 1) * (uint32_t)a.row_bytes;
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wr, coff[c], roff, 2);
                wv[j][r][c] = make_uint4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load is out before the first wait

    // 4. stage the input: x = a * gamma under the norm, fp16 hi/lo pairs, chunk sums, sum of a^2
    float ssq = 0.0f;
    auto stage_chunk = [&](int idx, const uint4* xraw, const uint4* graw) {
        if (idx >= G) return;
        constexpr int NV = 4 * XW;  // values this thread holds
        float v[NV];
#pragma unroll
        for (int t = 0; t < XW; ++t) {
            v[4 * t] = __builtin_bit_cast(float, xraw[t].x);
            v[4 * t + 1] = __builtin_bit_cast(float, xraw[t].y);
            v[4 * t + 2] = __builtin_bit_cast(float, xraw[t].z);
            v[4 * t + 3] = __builtin_bit_cast(float, xraw[t].w);
        }
        if (a.gamma) {
#pragma unroll
            for (int t = 0; t < XW; ++t) {
                const float gm[4] = {__builtin_bit_cast(float, graw[t].x), __builtin_bit_cast(float, graw[t].y),
                                     __builtin_bit_cast(float, graw[t].z), __builtin_bit_cast(float, graw[t].w)};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ssq = fmaf(v[4 * t + e], v[4 * t + e], ssq);
                    v[4 * t + e] *= gm[e];
                }
            }
        }
        // the chunk onto fp16's range (x * 2^sh), as in q4_gemv
        float mx = 0.0f;
#pragma unroll
        for (int t = 0; t < NV; ++t) mx = fmaxf(mx, fabsf(v[t]));
        if constexpr (HALF) mx = fmaxf(mx, __shfl_xor(mx, 1, kWave));
        const int sh = fp16_range_shift(mx);
#pragma unroll
        for (int t = 0; t < NV; ++t) v[t] = __builtin_amdgcn_ldexpf(v[t], sh);
        uint32_t p[NV / 2], lo[NV / 2];
#pragma unroll
        for (int j = 0; j < NV / 8; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float u = v[8 * j + q], w = v[8 * j + q + 4];
                const _Float16 hu = (_Float16)u, hw = (_Float16)w;
                const _Float16 lu = (_Float16)(u - (float)hu), lw = (_Float16)(w - (float)hw);
                p[4 * j + q] = (uint32_t)h_bits(hu) | ((uint32_t)h_bits(hw) << 16);
                lo[4 * j + q] = (uint32_t)h_bits(lu) | ((uint32_t)h_bits(lw) << 16);
            }
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < NV; ++t) s += v[t];
        if constexpr (HALF) s += __shfl_xor(s, 1, kWave);
        uint4* dh = reinterpret_cast<uint4*>(xh) + idx;
        uint4* dl = reinterpret_cast<uint4*>(xl) + idx;
#pragma unroll
        for (int t = 0; t < NV / 8; ++t) {
            const int piece = (NV / 8) * hf + t;  // 0 .. 3
            dh[piece * G] = make_uint4(p[4 * t], p[4 * t + 1], p[4 * t + 2], p[4 * t + 3]);
            dl[piece * G] = make_uint4(lo[4 * t], lo[4 * t + 1], lo[4 * t + 2], lo[4 * t + 3]);
        }
        if (hf == 0) {
            sums[idx] = s;
            facs[idx] = __builtin_amdgcn_ldexpf(1.0f, -sh);
        }
    };
    stage_chunk(HALF ? tid >> 1 : tid, xraw, graw);
    // K > 8192 (8 chunks per lane): the second input chunk of each thread (chunks 256 ..) is
    // loaded after the weight loads, so its wait is the wait for all of them; the wave first runs
    // its chunks below 256 (c < 4), staged before the first barrier, while its later weights
    // stream in, then stages the second chunk and runs c >= 4 after a second barrier. Each row's
    // sum keeps the chunk order.
    constexpr bool TWO = CPL == 8;
    if constexpr (TWO) load_chunk(tid + 256, xraw, graw);
    else ssq_part[tid] = ssq;
    __syncthreads();
    if constexpr (!TWO) {
        if (!live) return;
    }
    // norm factor: the 256 partials in a fixed order (lane l adds l, l + 64, l + 128, l + 192)
    float inv = 1.0f;
    auto norm_factor = [&]() {
        if (a.gamma) {
            const float t = (ssq_part[lane] + ssq_part[lane + 64]) + (ssq_part[lane + 128] + ssq_part[lane + 192]);
            const float total = wave_sum_lane63(t);
            inv = 1.0f / sqrtf(total / (float)K + a.eps);  // meaningful on lane 63, which stores
            // K slices: the slice's sum of a^2, once per slice
            if (a.part && blockIdx.x == 0 && tid == 63) a.ssq[blockIdx.y] = total;
        }
    };
    if constexpr (!TWO) norm_factor();

    uint32_t mag_lo, mag_hi;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(mag_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(mag_hi));
    const h2 bias_lo = {1024, 1024}, bias_hi = {64, 64};

    // 5. chunks in load order, each chunk's input pairs read from LDS once for all the wave's rows;
    // then the wave sums (lane 63) and the epilogue on lane 63
    float acc[NM][R];
#pragma unroll
    for (int j = 0; j < NM; ++j)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[j][r] = 0.0f;
    auto run_chunks = [&](auto c_lo, auto c_hi) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NM; ++j) {
            const FusedMat& fm = MODE == 1 ? a.m[j] : fm0;
#pragma unroll
            for (int c = decltype(c_lo)::value; c < decltype(c_hi)::value; ++c) {
                const int idx = lch[c];
                const uint4* sh = reinterpret_cast<const uint4*>(xh) + idx;
                const uint4* sl = reinterpret_cast<const uint4*>(xl) + idx;
                const float sxc = sums[idx], fac = facs[idx];
                // piece by piece (4 input pairs and their low terms at a time), every row's dot product
                // in the same order as one row at a time: the input registers are 8, not 32
                float p[R];
#pragma unroll
                for (int r = 0; r < R; ++r) p[r] = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint4 u = sh[w * G], l = sl[w * G];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t d = w == 0 ? wv[j][r][c].x : w == 1 ? wv[j][r][c].y : w == 2 ? wv[j][r][c].z : wv[j][r][c].w;
                        const uint32_t d8 = d >> 8;
                        const h2 q0 = bits_h2((d & 0x000F000Fu) | mag_lo) - bias_lo;
                        const h2 q1 = bits_h2((d & 0x00F000F0u) | mag_hi) - bias_hi;
                        const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo) - bias_lo;
                        const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi) - bias_hi;
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(u.x), q0, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(l.x), q0, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(u.y), q1, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(l.y), q1, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(u.z), q2, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(l.z), q2, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(u.w), q3, p[r], false);
                        p[r] = __builtin_amdgcn_fdot2(bits_h2(l.w), q3, p[r], false);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float sc = SF16 ? (float)bits_h((uint16_t)sraw[j][r][c]) : __builtin_bit_cast(float, sraw[j][r][c]);
                    sc = cv[c] ? sc : 0.0f;
                    const float z = ZU ? fm.zero_value : __builtin_bit_cast(float, zraw[j][r][c]);
                    acc[j][r] = fmaf(sc * fac, p[r] - z * sxc, acc[j][r]);
                }
            }
        }
    };
    if constexpr (TWO) {
        if (live) run_chunks(std::integral_constant<int, 0>{}, std::integral_constant<int, 4>{});
        stage_chunk(tid + 256, xraw, graw);
        ssq_part[tid] = ssq;
        __syncthreads();
        if (!live) return;
        norm_factor();
        run_chunks(std::integral_constant<int, 4>{}, std::integral_constant<int, CPL>{});
    } else {
        run_chunks(std::integral_constant<int, 0>{}, std::integral_constant<int, CPL>{});
    }
    float dots[NM][R];
#pragma unroll
    for (int j = 0; j < NM; ++j)
#pragma unroll
        for (int r = 0; r < R; ++r) dots[j][r] = wave_sum_lane63(acc[j][r]);
    if (lane == 63 && a.part) {
        float* pp = a.part + blockIdx.y * a.pstride;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = n0 + r;
            if (row >= fm0.N) continue;
#pragma unroll
            for (int j = 0; j < NM; ++j) pp[(MODE == 1 ? a.m[j].part_off : fm0.part_off) + row] = dots[j][r];
        }
    } else if (lane == 63) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = n0 + r;
            if (row >= fm0.N) continue;
            float v = dots[0][r] * inv;
            if constexpr (MODE == 1) {
                const float u = dots[1][r] * inv;
                v = v / (1.0f + expf(-v)) * u;
            }
            if (a.res) v += a.res[row];
            fm0.y[row] = v;
        }
    }
}

// The end of a K-sliced fused GEMV: for every output row (the matrices' rows one after another),
// the slices' dot products added in slice order, scaled by the norm factor from the slices' sums
// of a^2 (added in slice order), then silu(gate) * up in mode 1 and the residual, as the unsliced
// kernel's epilogue does.
template <int MODE>
__global__ __launch_bounds__(256) void fused_finish(FusedArgs a, int slices, int rows) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows) return;
    int mi = 0;
    if (MODE == 0) {
        if (a.nmats > 1 && i >= a.m[1].part_off) mi = 1;
        if (a.nmats > 2 && i >= a.m[2].part_off) mi = 2;
    }
    const FusedMat& fm = a.m[mi];
    const int row = i - fm.part_off;
    float inv = 1.0f;
    if (a.gamma) {
        float total = 0.0f;
        for (int z = 0; z < slices; ++z) total += a.ssq[z];
        inv = 1.0f / sqrtf(total / (float)a.K + a.eps);
    }
    float d = 0.0f, u = 0.0f;
    for (int z = 0; z < slices; ++z) {
        d += a.part[z * a.pstride + i];
        if (MODE == 1) u += a.part[z * a.pstride + a.m[1].part_off + row];
    }
    float v = d * inv;
    if (MODE == 1) {
        u *= inv;
        v = v / (1.0f + expf(-v)) * u;
    }
    if (a.res) v += a.res[row];
    fm.y[row] = v;
}

template <int CPL, int MODE>
void launch_fused_sz(const FusedArgs& a, bool sf16, bool zu) {
    const int G = a.slice_chunks;
    const size_t lds = (size_t)G * 16 * 4 * 2 + (size_t)G * 4 * 2 + 256 * 4;
    const dim3 grid((a.batches + 3) / 4, (a.Gt + G - 1) / G);
#define BYHIP_FUSED_CASE(SF, ZU_) \
    if (sf16 == SF && zu == ZU_) { launch("q4_gemv_fused", (q4_gemv_fused<CPL, SF, ZU_, MODE>), grid, dim3(256), lds, a); }
    BYHIP_FUSED_CASE(true, true)
    else BYHIP_FUSED_CASE(true, false)
    else BYHIP_FUSED_CASE(false, true)
    else BYHIP_FUSED_CASE(false, false)
#undef BYHIP_FUSED_CASE
    BYHIP_LAUNCHED("q4_gemv_fused");
}

}  // namespace

// Activation rows one GEMV launch takes (at most 4): the rows' staged activations fit the register
// tile (rows x chunks per lane x fp16 terms <= 8, except a single row, which then reads them from
// LDS), the block's staging (at most 512 chunks) and 64 KB of LDS. 0: not even one row fits.
int gemv_rows_per_launch(int K, int M, int x_dtype) {
    const int G = gemv_slices(K, x_dtype).chunks;
    const int xs = x_dtype == BYHIP_F32 ? 2 : 1, cpl = gemv_cpl(G * 32);
    for (int m = std::min(M, 4); m >= 1; --m) {
        const size_t lds = (size_t)m * G * (64 * xs + 8);
        if ((m == 1 || m * xs * cpl <= 8) && m * G <= 512 && lds <= 65536) return m;
    }
    return 0;
}

bool q4_gemv_eligible(const byhip_q4w* w, int M, int x_dtype, size_t work_bytes) {
    if (w->K % 32 != 0 || (w->group != 0 && w->group % 32 != 0)) return false;
    // 32-bit buffer offsets (below the out-of-range marker) for weights, scales and activations
    const uint64_t lim = kOutOfRange - 64;
    const bool fits = (uint64_t)w->N * w->row_bytes < lim && (uint64_t)(w->N + 8) * (w->K / 32 + w->gpr) * 4 < lim &&
                      (uint64_t)4 * w->K * 4 < lim;
    const bool aligned = reinterpret_cast<uintptr_t>(w->wq) % 16 == 0;
    // the partial sums of a sliced K fit the scratch
    const GemvSlices sl = gemv_slices(w->K, x_dtype);
    const bool room = sl.slices == 1 || (size_t)sl.slices * splitk_stride(M, w->N) * sizeof(float) <= work_bytes;
    return fits && aligned && room && gemv_rows_per_launch(w->K, M, x_dtype) > 0;
}

void launch_q4_gemv(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, void* work,
                    size_t work_bytes) {
    const GemvSlices sl = gemv_slices(w->K, x_dtype);
    const int cpl = gemv_cpl(sl.chunks * 32);
    const size_t xb = dtype_bytes(x_dtype), yb = dtype_bytes(y_dtype);
    const bool blk = w->sblk != nullptr;
    const int step = gemv_rows_per_launch(w->K, M, x_dtype);
    if (step < 1) fail("byhip: internal: GEMV launched on a shape it does not take (K=%d)", w->K);
    // several slices: fp32 partials [slice][M][N] in the scratch, then splitk_sum into y
    float* part = nullptr;
    if (sl.slices > 1) {
        part = static_cast<float*>(work ? work : workspace());
        const size_t room = work ? work_bytes : kWorkspaceBytes;
        if ((size_t)sl.slices * splitk_stride(M, w->N) * sizeof(float) > room)
            fail("byhip: internal: GEMV partial sums exceed the scratch");
    }
    const int yd = part ? BYHIP_F32 : y_dtype;
    for (int m0 = 0; m0 < M; m0 += step) {
        const int mm = std::min(step, M - m0);
        GemvArgs a;
        a.x = static_cast<const uint8_t*>(x) + (size_t)m0 * w->K * xb;
        a.wq = w->wq;
        a.scales = blk ? w->sblk : w->scales;
        a.zeros = blk ? w->zblk : w->zeros;
        a.zero_value = w->zero_value;
        a.y = part ? static_cast<void*>(part + (size_t)m0 * w->N) : static_cast<uint8_t*>(y) + (size_t)m0 * w->N * yb;
        a.K = w->K; a.N = w->N; a.gpr = w->gpr; a.row_bytes = (int)w->row_bytes;
        a.group_chunks = w->group / 32;
        a.n_pad = (w->N + 7) / 8 * 8;
        a.Gt = w->K / 32; a.slice_chunks = sl.chunks; a.ldx = w->K;
        a.ystride = part ? splitk_stride(M, w->N) : 0;
        if (x_dtype == BYHIP_F32) {
            switch (mm) {
            case 1: launch_cpl<1, true>(cpl, a, w, blk, yd); break;
            case 2: launch_cpl<2, true>(cpl, a, w, blk, yd); break;
            case 3: launch_cpl<3, true>(cpl, a, w, blk, yd); break;
            default: launch_cpl<4, true>(cpl, a, w, blk, yd); break;
            }
        } else {
            switch (mm) {
            case 1: launch_cpl<1, false>(cpl, a, w, blk, yd); break;
            case 2: launch_cpl<2, false>(cpl, a, w, blk, yd); break;
            case 3: launch_cpl<3, false>(cpl, a, w, blk, yd); break;
            default: launch_cpl<4, false>(cpl, a, w, blk, yd); break;
            }
        }
    }
    if (part) {
        GemmArgs ga;
        ga.M = M; ga.N = w->N; ga.y = y; ga.y_dtype = y_dtype; ga.part = part;
        launch_splitk_sum(ga, sl.slices);
    }
}


// The fused GEMV's K slices: one when a block stages the whole input (fp16 hi/lo pairs and chunk
// sums, 136 bytes per chunk, with the norm partials in 64 KB of LDS: 474 chunks; gate and up keep
// at most 4 chunks per lane: 256), else equal slices that fit.
GemvSlices fused_slices(int K, int mode) {
    const int G = K / 32, maxc = mode == 1 ? 256 : 474;
    if (G <= maxc) return {1, G};
    const int s = (G + maxc - 1) / maxc;
    return {s, (G + s - 1) / s};
}

// Floats of one slice's plane of partial dot products: every matrix's rows (gate then up in mode 1),
// 16-byte aligned.
size_t fused_rows_total(const byhip_q4w* const* ws, int n_ws) {
    size_t rows = 0;
    for (int i = 0; i < n_ws; ++i) rows += ws[i]->N;
    return (rows + 3) & ~(size_t)3;
}

int q4_fused_check(int mode, const byhip_q4w* const* ws, int n_ws) {
    if (mode != 0 && mode != 1) return BYHIP_UNSUPPORTED;
    if (n_ws < 1 || n_ws > 3 || (mode == 1 && n_ws != 2)) return BYHIP_UNSUPPORTED;
    const byhip_q4w* w0 = ws[0];
    for (int i = 0; i < n_ws; ++i) {
        const byhip_q4w* w = ws[i];
        if (!w) return BYHIP_UNSUPPORTED;
        if (w->K != w0->K || w->group != w0->group || w->gpr != w0->gpr) return BYHIP_UNSUPPORTED;
        if (!w->sblk || w->blk_scale_f16 != w0->blk_scale_f16 || w->zero_uniform != w0->zero_uniform)
            return BYHIP_UNSUPPORTED;
        // 32-bit buffer offsets for weights and the blocked scales, 16-byte aligned rows
        const uint64_t lim = kOutOfRange - 64;
        if ((uint64_t)w->N * w->row_bytes >= lim || (uint64_t)(w->N + 8) * (w->K / 32) * 4 >= lim ||
            reinterpret_cast<uintptr_t>(w->wq) % 16 != 0)
            return BYHIP_UNSUPPORTED;
    }
    if (w0->K % 32 != 0 || (w0->group != 0 && w0->group % 32 != 0)) return BYHIP_UNSUPPORTED;
    if (mode == 1 && ws[1]->N != w0->N) return BYHIP_UNSUPPORTED;
    // a sliced K's partial sums and sums of squares fit the workspace
    const GemvSlices sl = fused_slices(w0->K, mode);
    if (sl.slices > 1 && (size_t)sl.slices * (fused_rows_total(ws, n_ws) + 1) * sizeof(float) > kWorkspaceBytes)
        return BYHIP_UNSUPPORTED;
    return BYHIP_OK;
}

void launch_q4_gemv_fused(int mode, const float* x, const byhip_q4w* const* ws, int n_ws, float* const* outs,
                          const float* res, const float* gamma, float eps) {
    FusedArgs a{};
    const GemvSlices sl = fused_slices(ws[0]->K, mode);
    const int cpl = gemv_cpl(sl.chunks * 32);
    const int rows = fused_rows(cpl);
    a.x = x; a.res = res; a.gamma = gamma; a.eps = eps;
    a.K = ws[0]->K; a.row_bytes = (int)ws[0]->row_bytes; a.nmats = n_ws;
    a.Gt = ws[0]->K / 32; a.slice_chunks = sl.chunks;
    if (sl.slices > 1) {
        a.pstride = fused_rows_total(ws, n_ws);
        a.part = static_cast<float*>(workspace());
        a.ssq = a.part + (size_t)sl.slices * a.pstride;
    }
    int batches = 0, off = 0;
    for (int i = 0; i < n_ws; ++i) {
        const byhip_q4w* w = ws[i];
        FusedMat& m = a.m[i];
        m.wq = w->wq; m.sblk = w->sblk; m.zblk = w->zblk; m.zero_value = w->zero_value;
        m.y = mode == 1 ? outs[0] : outs[i];
        m.N = w->N; m.n_pad = (w->N + 7) / 8 * 8;
        m.batch0 = mode == 1 ? 0 : batches;
        m.part_off = off;
        off += w->N;
        if (mode == 0 || i == 0) batches += (w->N + rows - 1) / rows;
    }
    a.batches = batches;
    const bool sf = ws[0]->blk_scale_f16, zu = ws[0]->zero_uniform;
    switch (cpl) {
    case 1: mode ? launch_fused_sz<1, 1>(a, sf, zu) : launch_fused_sz<1, 0>(a, sf, zu); break;
    case 2: mode ? launch_fused_sz<2, 1>(a, sf, zu) : launch_fused_sz<2, 0>(a, sf, zu); break;
    case 4: mode ? launch_fused_sz<4, 1>(a, sf, zu) : launch_fused_sz<4, 0>(a, sf, zu); break;
    default: launch_fused_sz<8, 0>(a, sf, zu); break;  // mode 1 slices stop at 4 chunks per lane
    }
    if (sl.slices > 1) {
        const int out_rows = mode == 1 ? ws[0]->N : off;
        const dim3 grid((unsigned)((out_rows + 255) / 256));
        if (mode == 1)
            launch("fused_finish", fused_finish<1>, grid, dim3(256), 0, a, sl.slices, out_rows);
        else
            launch("fused_finish", fused_finish<0>, grid, dim3(256), 0, a, sl.slices, out_rows);
    }
}

}  // namespace byhip
