// byhip_mxfp4.hip - native MXFP4 GEMM on gfx950's scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// y[M, N] = x[M, K] . W^T with both operands E2M1 (fp4) and one E8M0 scale per 32 values, fp32
// accumulation. Operand layout (checked on the device): lane l holds the 32 values of row (or
// column) l%16, K block l/16 of the 128-deep step as 16 bytes, low nibble first, and its scale in
// the byte of the scale register that op_sel names. One FP4-KM group (16 bytes + 1 scale byte,
// session_vm.nim:384-388) is therefore exactly one lane's operand. FP4-KM stores element j and
// j+16 in byte j rather than elements 2j and 2j+1, so the MFMA sees the 32 values of a group in a
// permuted order; x uses the same packing, both operands carry the same permutation, and the dot
// product is unchanged.
//
// Tiling: a 256-thread block computes a 256 x 256 tile, each wave a 128 x 128 quarter as 8 x 8
// fragments (64 accumulators of 4 floats). Per 128-deep K step the block moves 256 rows x 64 bytes
// of x and of W straight from global memory into LDS (gfx950's 16-byte buffer_load ... lds, no
// staging registers), 4 lanes per 64-byte row segment, into a swizzled layout; the scale bytes
// follow once per 4 steps, 16 bytes per row. Steps are loaded in pairs, the two 64-byte halves of
// each row's 128-byte line a few loads apart, which halves the line fetches. Four LDS stages
// overlap, during the MFMAs of step s, the LDS reads of step s + 1 and the direct loads of the
// next pair, with one LDS barrier per step; the loads and reads are spread over the step's MFMAs
// in quarters. The output tile leaves through LDS so that global stores are 16 bytes per lane
// along rows.
//
// Tile order: blocks are handed to the 8 XCDs round-robin; block b works on tile
// (b % 8) * ceil(T/8) + b / 8 in column-major tile order, so each XCD owns a run of column tiles and
// its L2 serves the x and W slices its CUs share.
#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

constexpr int TM = 256, TN = 256;
constexpr int KSTEP = 128;            // values per step (4 groups)
constexpr int kXcds = 8;

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

struct MxArgs {
    const uint8_t* x;
    const uint8_t* xs;
    const uint8_t* w;
    const uint8_t* ws;
    void* y;
    int M, K, N, tiles_m, tiles, per_xcd;
};

// LDS layout.
//   Data stages (kStages), each the 16 x fragments then the 16 W fragments of one K step. Fragment F
//   (tile rows 16 F .. 16 F + 15) is 1 KB: row r's four 16-byte K blocks sit at 64 r + 16 (c ^ swz(r)),
//   so a direct load in which 4 neighbouring lanes read one row's 64 contiguous bytes lands each
//   chunk where the MFMA operand read (lane 16 j + i takes row i, block j) finds it.
//   Scale buffers (2), one per 4-step period: 256 x rows of 16 bytes, then 256 W rows; byte 4 t + g
//   of a row is the scale of group g of step t of the period (the row's 16 scale bytes in memory).
//   After the K loop the stages hold the output tile on its way to global memory.
constexpr int kFragBytes = 1024;
constexpr int kOpBytes = 16 * kFragBytes;
constexpr int kStageBytes = 2 * kOpBytes;
constexpr int kStages = 4;
constexpr int kScaleOpBytes = 256 * 16;
constexpr int kScaleBufBytes = 2 * kScaleOpBytes;
constexpr int kScaleBase = kStages * kStageBytes;
constexpr int kLdsBytes = kScaleBase + 2 * kScaleBufBytes;   // 144 KB
constexpr int kPairDma = 16;                                 // direct loads per lane per 2 steps
constexpr int kScaleDma = 2;                                 // per lane per 4-step period
constexpr int kOutPitch = 128 + 4;                           // floats per staged output row
constexpr int kOutWaveBytes = 32 * kOutPitch * 4;            // 32 rows per wave and pass

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 2)) & 3; }

__device__ __forceinline__ i8v operand(uint4 u) {
    return (i8v){(int)u.x, (int)u.y, (int)u.z, (int)u.w, 0, 0, 0, 0};
}

// One wave's operands of one K step: 8 x fragments, 8 W fragments and their scale bytes, one per
// register in byte 0 (a byte load each, so no ALU op combines them and nothing waits for them
// before the MFMAs that use them).
struct Frags {
    uint4 a[8], b[8];
    int sa[8], sb[8];
};

// acc += a . b with the scale bytes of the two fragments (byte 0 of sa and sb: op_sel 0).
__device__ __forceinline__ f4 mx_mfma(uint4 a, uint4 b, f4 acc, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(operand(a), operand(b), acc, 4, 4, 0, sa, 0, sb);
}

// Workgroup barrier after this wave's LDS reads and all but the newest N direct loads have
// completed: the memory clobber keeps the compiler from moving LDS accesses across it, and the
// direct loads issued last stay in flight.
template <int N>
__device__ __forceinline__ void stage_barrier() {
    wait_vmcnt<N>();
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int YT>
__global__ __launch_bounds__(256) void mxfp4_gemm(MxArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int t = (blockIdx.x % kXcds) * a.per_xcd + blockIdx.x / kXcds;
    if (t >= a.tiles) return;  // whole block
    const int m0 = (t % a.tiles_m) * TM, n0 = (t / a.tiles_m) * TN;
    const int M = a.M, N = a.N, K = a.K;
    const uint32_t kb = (uint32_t)K >> 1, kg = (uint32_t)K >> 5;

    const rsrc_t xr = make_rsrc(a.x, (uint32_t)M * kb);
    const rsrc_t wr = make_rsrc(a.w, (uint32_t)N * kb);
    const rsrc_t xsr = make_rsrc(a.xs, (uint32_t)M * kg);
    const rsrc_t wsr = make_rsrc(a.ws, (uint32_t)N * kg);

    // Direct loads of wave w: per step, fragments 4 w .. 4 w + 3 of x and of W, lane l reading
    // row l / 4 of the fragment, chunk (l % 4) ^ swz(row); per period, the 16 scale bytes of rows
    // 64 w + l. The lane's row offset is loop-invariant in voffset and the step's K offset goes in
    // soffset; the buffer range check covers their sum, so rows past M or N (offsets from M * K / 2
    // up, below 2^32 by the launcher's check) load zeros. The scale window of a row may run into the
    // next row or past the buffer end (K % 512 != 0): those bytes belong to steps past the last
    // and are never read, and the range check is per dword.
    const int fr = lane & 15, grp = lane >> 4;
    const int drow = lane >> 2;
    const uint32_t dchunk = 16u * (uint32_t)((lane & 3) ^ swz(drow));
    uint32_t xo[4], wo[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        xo[q] = (uint32_t)(m0 + 16 * (4 * wid + q) + drow) * kb + dchunk;
        wo[q] = (uint32_t)(n0 + 16 * (4 * wid + q) + drow) * kb + dchunk;
    }
    const uint32_t xso = (uint32_t)(m0 + tid) * kg, wso = (uint32_t)(n0 + tid) * kg;

    const int nsteps = K / KSTEP;
    // Steps past the last re-read the last one (cache hits) into a stage nobody reads again.
    // Period p = steps 4 p .. 4 p + 3. A period past the last reads bytes nobody uses into the
    // buffer the last period does not occupy.
    auto dma_scales = [&](int p, uint8_t* buf) {
        const int pofs = 16 * p;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (lds_void*)(buf + wid * 1024), 16, xso, pofs, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (lds_void*)(buf + kScaleOpBytes + wid * 1024), 16, wso, pofs, 0, 0);
    };
    // Steps e and e + 1 (e even) are the two 64-byte halves of each row's 128-byte line. They are
    // loaded as one batch of 16 direct loads, k = 0 .. 15 in issue order [x e][x e + 1][W e][W e + 1]
    // (4 each), the halves of a row 4 loads apart so that the second request finds the line the
    // first one brought in.
    auto dma_batch = [&](int k, int e, uint8_t* st0, uint8_t* st1) {
        const int op = k >> 3, half = (k >> 2) & 1, q = k & 3;
        const int kofs = min(e + half, nsteps - 1) * (KSTEP / 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            op ? wr : xr, (lds_void*)((half ? st1 : st0) + op * kOpBytes + (4 * wid + q) * kFragBytes), 16,
            op ? wo[q] : xo[q], kofs, 0, 0);
    };
    auto dma_pair = [&](int e, uint8_t* st0, uint8_t* st1) {
#pragma unroll
        for (int k = 0; k < kPairDma; ++k) dma_batch(k, e, st0, st1);
    };

    const int rd = 64 * fr + 16 * (grp ^ swz(fr));
    const int sa_row = 16 * (16 * 8 * wm + fr) + grp;
    const int sb_row = kScaleOpBytes + 16 * (16 * 8 * wn + fr) + grp;
    // T = position of the step inside its period (selects the scale byte).
    auto lread = [&](Frags& f, const uint8_t* stage, const uint8_t* sbuf, int T) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            f.a[i] = *reinterpret_cast<const uint4*>(stage + (8 * wm + i) * kFragBytes + rd);
            f.b[i] = *reinterpret_cast<const uint4*>(stage + kOpBytes + (8 * wn + i) * kFragBytes + rd);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f.sa[2 * k] = sbuf[sa_row + 512 * k + 4 * T];
            f.sa[2 * k + 1] = sbuf[sa_row + 512 * k + 256 + 4 * T];
            f.sb[2 * k] = sbuf[sb_row + 512 * k + 4 * T];
            f.sb[2 * k + 1] = sbuf[sb_row + 512 * k + 256 + 4 * T];
        }
    };

    // quarter 0: W fragments 0-3 and all scales; 1: W 4-7; 2: x 0-3; 3: x 4-7.
    auto lread_q = [&](Frags& f, const uint8_t* stage, const uint8_t* sbuf, int T, int g) {
        const int op = g >> 1, i0 = 4 * (g & 1);
#pragma unroll
        for (int i = i0; i < i0 + 4; ++i) {
            if (op == 0)
                f.b[i] = *reinterpret_cast<const uint4*>(stage + kOpBytes + (8 * wn + i) * kFragBytes + rd);
            else
                f.a[i] = *reinterpret_cast<const uint4*>(stage + (8 * wm + i) * kFragBytes + rd);
        }
        if (g == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                f.sa[2 * k] = sbuf[sa_row + 512 * k + 4 * T];
                f.sa[2 * k + 1] = sbuf[sa_row + 512 * k + 256 + 4 * T];
                f.sb[2 * k] = sbuf[sb_row + 512 * k + 4 * T];
                f.sb[2 * k + 1] = sbuf[sb_row + 512 * k + 256 + 4 * T];
            }
        }
    };

    f4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    auto stage_at = [&](int s) { return lds + (s & (kStages - 1)) * kStageBytes; };
    auto sbuf_at = [&](int s) { return lds + kScaleBase + ((s >> 2) & 1) * kScaleBufBytes; };

    // Pipeline, at the start of step s: `cur` holds step s's operands and LDS stage (s + 1) % 4 with
    // the scales of step s + 1 is complete. Step s reads step s + 1's operands into `nxt` while its
    // MFMAs run. An odd step s also issues the batch of steps s + 3 and s + 4 (stages (s + 3) % 4
    // and s % 4, read two steps and one step ago), preceded, when s % 4 == 1, by the scales of
    // period (s + 3) / 4. Every step ends by waiting for the loads the next step reads, the newest
    // ones staying in flight, and one LDS barrier:
    //   even s: stage s + 2 = the first half of the last batch; only [W s + 3] may be pending;
    //   odd s:  stage s + 2 = the second half of the previous batch; this step's batch may be.
    // The pointers given to a step are distinct regions; __restrict__ lets the compiler see that
    // the step's LDS reads cannot alias its direct loads, so it does not wait for them first.
    Frags f0, f1;
    [&](uint8_t* __restrict__ sc, uint8_t* __restrict__ s0, uint8_t* __restrict__ s1,
        uint8_t* __restrict__ s2, uint8_t* __restrict__ s3) {
        dma_scales(0, sc);
        dma_pair(0, s0, s1);
        dma_pair(2, s2, s3);
        stage_barrier<kPairDma>();  // scales and steps 0, 1; steps 2, 3 stay in flight
        lread(f0, s0, sc, 0);
    }(sbuf_at(0), stage_at(0), stage_at(1), stage_at(2), stage_at(3));

    // P = s % 4 (compile time): odd positions issue a batch, position 1 with scales.
    auto step = [&](auto Pc, int s, Frags& cur, Frags& nxt, uint8_t* __restrict__ d0,
                    uint8_t* __restrict__ d1, uint8_t* __restrict__ sdst,
                    const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc) {
        constexpr int P = decltype(Pc)::value;
        constexpr int T1 = (P + 1) & 3;
        constexpr bool batch = P & 1, scales = P == 1;
        // loads issued after the ones step s + 1 reads: this step's batch and scales
        constexpr int V = (batch ? kPairDma : 0) + (scales ? kScaleDma : 0);
        if constexpr (batch) {
            if (scales) dma_scales((s + 3) >> 2, sdst);
#pragma unroll
            for (int k = 0; k < 4; ++k) dma_batch(k, s + 3, d0, d1);
        }
        lread_q(nxt, src, ssrc, T1, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = mx_mfma(cur.a[i], cur.b[j], acc[i][j], cur.sa[i], cur.sb[j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (batch) {
#pragma unroll
            for (int k = 4; k < 8; ++k) dma_batch(k, s + 3, d0, d1);
        }
        lread_q(nxt, src, ssrc, T1, 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 2; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = mx_mfma(cur.a[i], cur.b[j], acc[i][j], cur.sa[i], cur.sb[j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (batch) {
#pragma unroll
            for (int k = 8; k < 12; ++k) dma_batch(k, s + 3, d0, d1);
        }
        lread_q(nxt, src, ssrc, T1, 2);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 4; i < 6; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = mx_mfma(cur.a[i], cur.b[j], acc[i][j], cur.sa[i], cur.sb[j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (batch) {
#pragma unroll
            for (int k = 12; k < 16; ++k) dma_batch(k, s + 3, d0, d1);
        }
        lread_q(nxt, src, ssrc, T1, 3);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 6; i < 8; ++i) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[i][j] = mx_mfma(cur.a[i], cur.b[j], acc[i][j], cur.sa[i], cur.sb[j]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        stage_barrier<batch ? V : kPairDma / 4>();
        __builtin_amdgcn_sched_barrier(0);
    };
    // d0 / d1 (stages (s + 3) % 4 and s % 4) and sdst (the buffer of period (s + 3) / 4, which
    // step s + 1 does not read) are only written by odd steps.
#define MX_STEP(P, S, CUR, NXT)                                                                   \
    step(std::integral_constant<int, P>{}, S, CUR, NXT, stage_at((S) + 3), stage_at((S) + 4),       \
         sbuf_at((S) + 3), stage_at((S) + 1), sbuf_at((S) + 1))
    int s = 0;
    for (; s + 3 < nsteps; s += 4) {
        MX_STEP(0, s, f0, f1);
        MX_STEP(1, s + 1, f1, f0);
        MX_STEP(2, s + 2, f0, f1);
        MX_STEP(3, s + 3, f1, f0);
    }
    if (s < nsteps) MX_STEP(0, s, f0, f1);
    if (s + 1 < nsteps) MX_STEP(1, s + 1, f1, f0);
    if (s + 2 < nsteps) MX_STEP(2, s + 2, f0, f1);
#undef MX_STEP
    stage_barrier<0>();  // every direct load has landed and every wave is done with the stages

    // Output: per wave, 4 passes of 32 rows (fragment rows 2 p, 2 p + 1) staged as fp32 in the
    // wave's own LDS region, then written back a full row segment per lane group: 16-byte stores.
    float* ostage = reinterpret_cast<float*>(lds + wid * kOutWaveBytes);
    const int ro = m0 + wm * 128, co = n0 + wn * 128;
    constexpr int es = YT == BYHIP_F32 ? 4 : 2;
    const bool wide = ((uintptr_t)a.y % 16 == 0) && ((size_t)N * es % 16 == 0);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    ostage[(16 * ii + 4 * grp + r) * kOutPitch + 16 * j + fr] = acc[2 * p + ii][j][r];
        __builtin_amdgcn_wave_barrier();
        // 16 output bytes per lane: 4 floats (f32) or 8 halves.
        constexpr int per = 16 / es;                 // elements per lane
        constexpr int lanes_per_row = 128 / per;     // 32 (f32) or 16
        constexpr int rows_per_pass = 64 / lanes_per_row;
#pragma unroll
        for (int u = 0; u < 32 / rows_per_pass; ++u) {
            const int rr = u * rows_per_pass + lane / lanes_per_row;
            const int cc = (lane % lanes_per_row) * per;
            const int m = ro + 32 * p + rr, n = co + cc;
            const float* src = ostage + rr * kOutPitch + cc;
            float v[per];
#pragma unroll
            for (int e = 0; e < per; e += 4) {
                const float4 q = *reinterpret_cast<const float4*>(src + e);
                v[e] = q.x; v[e + 1] = q.y; v[e + 2] = q.z; v[e + 3] = q.w;
            }
            if (m >= M) continue;
            if (wide && n + per <= N) {
                uint4 o;
                if constexpr (YT == BYHIP_F32) {
                    o = make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                                   __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
                } else {
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        uint32_t lo, hi;
                        if constexpr (YT == BYHIP_F16) {
                            lo = __builtin_bit_cast(uint16_t, (_Float16)v[2 * e]);
                            hi = __builtin_bit_cast(uint16_t, (_Float16)v[2 * e + 1]);
                        } else {
                            lo = f32_to_bf16_bits(v[2 * e]);
                            hi = f32_to_bf16_bits(v[2 * e + 1]);
                        }
                        w[e] = lo | (hi << 16);
                    }
                    o = make_uint4(w[0], w[1], w[2], w[3]);
                }
                // streamed out (nontemporal): nothing reads the output back in this kernel
                const v4u ov = {o.x, o.y, o.z, o.w};
                __builtin_nontemporal_store(ov, reinterpret_cast<v4u*>(static_cast<uint8_t*>(a.y) + ((size_t)m * N + n) * es));
            } else {
#pragma unroll
                for (int e = 0; e < per; ++e)
                    if (n + e < N) store_y<YT>(a.y, (size_t)m * N + n + e, v[e]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace

void launch_mxfp4(const uint8_t* x, const uint8_t* x_scales, const uint8_t* w,
                  const uint8_t* w_scales, void* y, int y_dtype, int M, int K, int N) {
    if (K % KSTEP != 0) fail("byhip: internal: MXFP4 GEMM needs K %% 128 == 0 (K=%d)", K);
    if (M <= 0 || N <= 0) return;
    // Buffer offsets of the rows a tile reaches past M or N must stay below 2^32.
    if ((uint64_t)(M + TM) * (K / 2) >= kOutOfRange || (uint64_t)(N + TN) * (K / 2) >= kOutOfRange)
        fail("byhip: MXFP4 operands above 4 GiB are not supported");
    MxArgs a;
    a.x = x; a.xs = x_scales; a.w = w; a.ws = w_scales; a.y = y;
    a.M = M; a.K = K; a.N = N;
    a.tiles_m = (M + TM - 1) / TM;
    a.tiles = a.tiles_m * ((N + TN - 1) / TN);
    a.per_xcd = (a.tiles + kXcds - 1) / kXcds;
    const dim3 grid(kXcds * a.per_xcd);
    switch (y_dtype) {
    case BYHIP_F32: hipLaunchKernelGGL(mxfp4_gemm<BYHIP_F32>, grid, dim3(256), 0, stream(), a); break;
    case BYHIP_F16: hipLaunchKernelGGL(mxfp4_gemm<BYHIP_F16>, grid, dim3(256), 0, stream(), a); break;
    default: hipLaunchKernelGGL(mxfp4_gemm<BYHIP_BF16>, grid, dim3(256), 0, stream(), a); break;
    }
    BYHIP_LAUNCHED("mxfp4_gemm");
}

}  // namespace byhip
