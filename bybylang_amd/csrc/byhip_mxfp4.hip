// byhip_mxfp4.hip - native MXFP4 GEMM on gfx950's scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4).
//
// y[M, N] = x[M, K] . W^T with both operands E2M1 (fp4) and one E8M0 scale per 32 values, fp32
// accumulation. Operand layout (checked on the device): lane l holds the 32 values of row (or
// column) l%32 of one 32-value K block as 16 bytes, low nibble first, and its scale in the byte of
// the scale register that op_sel names; the two lane halves cover two K blocks, so one MFMA is 64
// deep. One FP4-KM group (16 bytes + 1 scale byte, session_vm.nim:384-388) is therefore exactly
// one lane's operand. FP4-KM stores element j and j+16 in byte j rather than elements 2j and 2j+1,
// so the MFMA sees the 32 values of a group in a permuted order; x uses the same packing, both
// operands carry the same permutation, and the dot product is unchanged.
//
// Why 32x32x64: on the MI355X the 16x16x128 form sustains about 4.6 PFLOP/s with one wave per
// SIMD and the 32x32x64 form about 6.8 (register-only throughput, measured during development).
//
// Tiling: a 256-thread block computes a 256 x 256 tile, each wave a 128 x 128 quarter as 4 x 4
// fragments of 32 x 32 (16 accumulators of 16 floats). A K step is 128 deep: per fragment two
// MFMAs, one per 64-deep half. The block moves x and W straight from global memory into LDS
// (gfx950's 16-byte buffer_load ... lds, no staging registers). One direct load covers 8 rows x
// 128 bytes, whole cache lines: two steps of each row. Fetching whole lines doubles what a CU pulls
// per cycle against half lines (136 against 67 GB/s per CU from L2 in a standalone probe). The
// scale bytes follow once per 4 steps, 16 bytes per row. LDS holds two regions of two steps each;
// during the MFMAs of step s the wave reads step s + 1's operands, and odd steps issue the loads
// of the pair after next. One LDS barrier per pair. Reads and loads sit between the MFMAs, so the
// MFMA pipe is fed while they issue. The output tile leaves through LDS so that global stores are
// 16 bytes per lane along rows.
//
// The MFMAs are inline assembly, which keeps the 256 accumulators in place in AGPRs (the
// compiler's own MFMA shuffled them through VGPRs in this loop). The compiler then does not know
// them as MFMAs, so the code covers what it would otherwise track: the accumulators are zeroed and
// settled before the first MFMA, each step's operand registers stay reserved until the step ends,
// and the results are waited out before they are read. Register dependencies of the operands
// (LDS reads feeding an MFMA) are tracked by the compiler as for any instruction.
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
typedef float f16v __attribute__((ext_vector_type(16)));

struct MxArgs {
    const uint8_t* x;
    const uint8_t* xs;
    const uint8_t* w;
    const uint8_t* ws;
    void* y;
    int M, K, N, tiles_m, tiles, per_xcd;
};

// LDS layout.
//   Data regions (2), each two K steps e, e + 1 (e even) of the 256 x rows (32 KB) then the 256 W
//   rows. Rows come in blocks of 8 (1 KB): step e's 64 bytes of each row in the first 512 bytes,
//   step e + 1's in the second, row r of the block at 64 (r % 8) + 16 (c ^ swz(r % 16)) for K
//   block c. A direct load (8 lanes per row: 4 per step half) fills one block, and the swizzle
//   makes the MFMA operand reads, 16 neighbouring rows per 16 lanes, free of bank conflicts.
//   Scale buffers (2), one per 4-step period: 256 x rows of 16 bytes, then 256 W rows; byte 4 t + c
//   of a row is the scale of block c of step t of the period (the row's 16 scale bytes in memory).
//   After the K loop the regions hold the output tile on its way to global memory.
constexpr int kGroupBytes = 1024;                            // 8 rows x 2 steps
constexpr int kOpRegionBytes = 32 * kGroupBytes;             // one operand's 256 rows, two steps
constexpr int kRegionBytes = 2 * kOpRegionBytes;
constexpr int kScaleOpBytes = 256 * 16;
constexpr int kScaleBufBytes = 2 * kScaleOpBytes;
constexpr int kScaleBase = 2 * kRegionBytes;
constexpr int kLdsBytes = kScaleBase + 2 * kScaleBufBytes;   // 144 KB
constexpr int kPairDma = 16;                                 // direct loads per lane per 2 steps
constexpr int kOutPitch = 128 + 8;                           // floats per staged output row
constexpr int kOutWaveBytes = 32 * kOutPitch * 4;            // 32 rows per wave and pass

__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 2)) & 3; }

// One wave's operands of one K step: 4 x fragments and 4 W fragments of 32 rows, each as two
// 64-deep halves, and per fragment the scale bytes of both halves (bytes 0 and 1 of one register,
// one 16-bit LDS read).
struct Frags {
    v4u a[4][2], b[4][2];
    int sa[4], sb[4];
};

// acc += a . b over one 64-deep half H: v_mfma_scale_f32_32x32x64_f8f6f4 with both operands fp4
// (cbsz = blgp = 4), the scales in byte H of sa and sb. Lane l holds row (or column) l % 32 and
// 32 values of the half; the result is column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4 for
// r = 0..15. Written as assembly so that the accumulators stay in place in AGPRs.
template <int H>
__device__ __forceinline__ void mx_mfma(f16v& acc, v4u av, v4u bv, int sa, int sb) {
    if constexpr (H == 0)
        asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel_hi:[0,0,0] cbsz:4 blgp:4"
                     : "+a"(acc) : "v"(av), "v"(bv), "v"(sa), "v"(sb));
    else
        asm volatile("v_mfma_scale_f32_32x32x64_f8f6f4 %0, %1, %2, %0, %3, %4 op_sel:[1,1,0] op_sel_hi:[0,0,0] cbsz:4 blgp:4"
                     : "+a"(acc) : "v"(av), "v"(bv), "v"(sa), "v"(sb));
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

    // wid is wave-uniform; readfirstlane tells the compiler so, which keeps each direct load's LDS
    // address (M0) in scalar code instead of a v_readfirstlane per load.
    const int tid = threadIdx.x, lane = tid & 63, wid = __builtin_amdgcn_readfirstlane(tid >> 6);
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

    // Direct loads of wave w: per pair of steps, load q (0..7) covers x (and W) tile rows
    // 64 w + 8 q .. + 7, lane l reading row 8 q + (l % 32) / 4, step half l / 32, K block
    // (l % 4) ^ swz(row); per period, the 16 scale bytes of rows 64 w + l. The lane's row offset is
    // loop-invariant in voffset and the pair's K offset goes in soffset; the buffer range check
    // covers their sum, so rows past M or N (offsets from M * K / 2 up, below 2^32 by the launcher's
    // check) load zeros. A step past the last (the second half of a pair when K / 128 is odd) reads
    // the start of the next row, or zeros, into a half nobody reads. The scale window of a row may
    // run into the next row or past the buffer end (K % 512 != 0): those bytes belong to steps past
    // the last and are never read, and the range check is per dword.
    const int drow = (lane & 31) >> 2;
    uint32_t xo[8], wo[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int R = 64 * wid + 8 * q + drow;  // tile row
        const uint32_t c = 16u * (uint32_t)((lane & 3) ^ swz(R & 15)) + 64u * (uint32_t)(lane >> 5);
        xo[q] = (uint32_t)(m0 + R) * kb + c;
        wo[q] = (uint32_t)(n0 + R) * kb + c;
    }
    const uint32_t xso = (uint32_t)(m0 + tid) * kg, wso = (uint32_t)(n0 + tid) * kg;

    const int nsteps = K / KSTEP;
    // Pairs past the last re-read the last one (cache hits) into a region nobody reads again.
    // Period p = steps 4 p .. 4 p + 3. A period past the last reads bytes nobody uses into the
    // buffer the last period does not occupy.
    auto dma_scales = [&](int p, uint8_t* buf) {
        const int pofs = 16 * p;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (lds_void*)(buf + wid * 1024), 16, xso, pofs, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wsr, (lds_void*)(buf + kScaleOpBytes + wid * 1024), 16, wso, pofs, 0, 0);
    };
    // Steps e and e + 1 (e even) are the two 64-byte halves of each row's 128-byte line: one direct
    // load brings 8 whole lines (8 rows), step e to the first 512 bytes of its LDS block and step
    // e + 1 to the second. A batch is 16 loads, k = 0 .. 15: x rows 64 w + 8 k .., then W rows.
    auto dma_batch = [&](int k, int e, uint8_t* reg) {
        const int op = k >> 3, q = k & 7;
        const int kofs = min(e, nsteps - 1) * (KSTEP / 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            op ? wr : xr, (lds_void*)(reg + op * kOpRegionBytes + (8 * wid + q) * kGroupBytes), 16,
            op ? wo[q] : xo[q], kofs, 0, 0);
    };
    auto dma_pair = [&](int e, uint8_t* reg) {
#pragma unroll
        for (int k = 0; k < kPairDma; ++k) dma_batch(k, e, reg);
    };

    // Operand reads. Fragment F of the wave (rows 32 F .. 32 F + 31 of its 128) spans row blocks
    // 4 F .. 4 F + 3; lane l takes row l % 32 and, for half h, K block 2 (l / 32) + h of the step.
    // The blocks of a lane's two halves are neighbours, so its two scale bytes are one 16-bit read.
    const int lq = lane >> 5;
    int rd[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
        rd[h] = kGroupBytes * ((lane & 31) >> 3) + 64 * (lane & 7) + 16 * ((2 * lq + h) ^ swz(lane & 15));
    const int sa_row = 16 * (128 * wm + (lane & 31)) + 2 * lq;
    const int sb_row = kScaleOpBytes + 16 * (128 * wn + (lane & 31)) + 2 * lq;
    auto read_frag = [&](Frags& f, const uint8_t* stage, int op, int F, int h) {
        if (op == 0)
            f.a[F][h] = *reinterpret_cast<const v4u*>(stage + (16 * wm + 4 * F) * kGroupBytes + rd[h]);
        else
            f.b[F][h] = *reinterpret_cast<const v4u*>(stage + kOpRegionBytes + (16 * wn + 4 * F) * kGroupBytes + rd[h]);
    };
    // T = position of the step inside its period (selects the scale bytes).
    auto read_scale = [&](Frags& f, const uint8_t* sbuf, int T, int op, int F) {
        if (op == 0)
            f.sa[F] = *reinterpret_cast<const uint16_t*>(sbuf + sa_row + 512 * F + 4 * T);
        else
            f.sb[F] = *reinterpret_cast<const uint16_t*>(sbuf + sb_row + 512 * F + 4 * T);
    };
    auto lread = [&](Frags& f, const uint8_t* stage, const uint8_t* sbuf, int T) {
#pragma unroll
        for (int k = 0; k < 16; ++k) read_frag(f, stage, k & 1, (k >> 1) & 3, k >> 3);
#pragma unroll
        for (int k = 0; k < 8; ++k) read_scale(f, sbuf, T, k & 1, k >> 1);
    };

    f16v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // The MFMAs below are assembly: the zeroed accumulators must be in their registers, and a few
    // cycles old, before the first one reads them.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i][j]));
    asm volatile("s_nop 7" ::: "memory");

    // step s: LDS region (s / 2) % 2, second half of each 1 KB block when s is odd
    auto region_at = [&](int s) { return lds + ((s >> 1) & 1) * kRegionBytes; };
    auto stage_at = [&](int s) { return region_at(s) + (s & 1) * 512; };
    auto sbuf_at = [&](int s) { return lds + kScaleBase + ((s >> 2) & 1) * kScaleBufBytes; };

    // Pipeline, at the start of step s: `cur` holds step s's operands and the LDS data of step s + 1
    // with its scales is complete. Step s reads step s + 1's operands into `nxt` while its MFMAs
    // run. An odd step s also issues the batch of the pair s + 3, s + 4 into the region of the pair
    // s - 1, s (read during steps s - 2 and s - 1), and, when s % 4 == 1, the scales of period
    // (s + 3) / 4 into the buffer period (s - 1) / 4 has left. An even step s ends by waiting for
    // every load (the batch issued one step before: the pair s + 2, s + 3) and one LDS barrier.
    // After it, that pair is visible to all waves, and every wave is done with the pair s, s + 1,
    // whose region the next batch overwrites. Odd steps need no barrier: the step after reads the
    // second half of a pair already waited for.
    // The pointers given to a step are distinct regions; __restrict__ lets the compiler see that
    // the step's LDS reads cannot alias its direct loads, so it does not wait for them first.
    Frags f0, f1;
    [&](uint8_t* __restrict__ sc, uint8_t* __restrict__ s0, uint8_t* r0, uint8_t* r1) {
        dma_scales(0, sc);
        dma_pair(0, r0);
        dma_pair(2, r1);
        stage_barrier<kPairDma>();  // scales and steps 0, 1; steps 2, 3 stay in flight
        lread(f0, s0, sc, 0);
    }(sbuf_at(0), stage_at(0), region_at(0), region_at(2));

    // P = s % 4 (compile time): odd positions issue a batch, position 1 with scales. The step's
    // 32 MFMAs (half 0, then half 1, each over the 4 x 4 fragments) have the other instructions
    // placed between them: the 16 operand reads after MFMAs 0..15, the 8 scale reads after MFMAs
    // 16..23, a direct load after every even MFMA (the scales after MFMA 1), so that the MFMA pipe
    // is fed while they issue. Spreading the loads over the whole step (rather than MFMAs 8..23)
    // keeps the address unit from backing up into the MFMA issue: 65.8 us against 66.9 at
    // config 3, where the clock, not the cycle count, is the limit.
    auto step = [&](auto Pc, int s, Frags& cur, Frags& nxt, uint8_t* __restrict__ dreg,
                    uint8_t* __restrict__ sdst,
                    const uint8_t* __restrict__ src, const uint8_t* __restrict__ ssrc) {
        constexpr int P = decltype(Pc)::value;
        constexpr int T1 = (P + 1) & 3;
        constexpr bool batch = P & 1, scales = P == 1;
#pragma unroll
        for (int m = 0; m < 32; ++m) {
            const int i = (m >> 2) & 3, j = m & 3;
            if (m < 16)
                mx_mfma<0>(acc[i][j], cur.a[i][0], cur.b[j][0], cur.sa[i], cur.sb[j]);
            else
                mx_mfma<1>(acc[i][j], cur.a[i][1], cur.b[j][1], cur.sa[i], cur.sb[j]);
            __builtin_amdgcn_sched_barrier(0);
            if (m < 16) read_frag(nxt, src, m & 1, (m >> 1) & 3, m >> 3);
            if (m >= 16 && m < 24) read_scale(nxt, ssrc, T1, m & 1, (m - 16) >> 1);
            if constexpr (batch) {
                if (scales && m == 1) dma_scales((s + 3) >> 2, sdst);
                if ((m & 1) == 0) dma_batch(m >> 1, s + 3, dreg);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // The MFMAs above read their operands as they issue, but the compiler sees assembly: keep
        // every operand register of this step out of reach of the reads into `nxt` until here.
#pragma unroll
        for (int i = 0; i < 4; ++i)
            asm volatile("" ::"v"(cur.a[i][0]), "v"(cur.a[i][1]), "v"(cur.b[i][0]), "v"(cur.b[i][1]),
                         "v"(cur.sa[i]), "v"(cur.sb[i]));
        if constexpr (!batch) stage_barrier<0>();
        __builtin_amdgcn_sched_barrier(0);
    };
    // dreg (the region of the pair s + 3, s + 4) and sdst (the buffer of period (s + 3) / 4, which
    // step s + 1 does not read) are only written by odd steps.
#define MX_STEP(P, S, CUR, NXT)                                                                   \
    step(std::integral_constant<int, P>{}, S, CUR, NXT, region_at((S) + 3), sbuf_at((S) + 3),     \
         stage_at((S) + 1), sbuf_at((S) + 1))
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
    // The compiler does not see the MFMAs' results arrive late: wait out the longest MFMA latency
    // before the accumulators are read.
    asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i][j]));
    stage_barrier<0>();  // every direct load has landed and every wave is done with the stages

    // Output: per wave, 4 passes of 32 rows (fragment row F = p) staged as fp32 in the wave's own
    // LDS region, then written back a full row segment per lane group: 16-byte stores.
    float* ostage = reinterpret_cast<float*>(lds + wid * kOutWaveBytes);
    const int ro = m0 + wm * 128, co = n0 + wn * 128;
    constexpr int es = YT == BYHIP_F32 ? 4 : 2;
    const bool wide = ((uintptr_t)a.y % 16 == 0) && ((size_t)N * es % 16 == 0);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                ostage[(8 * (r >> 2) + 4 * lq + (r & 3)) * kOutPitch + 32 * j + (lane & 31)] = acc[p][j][r];
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
                        if constexpr (YT == BYHIP_F16) {
                            const uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)v[2 * e]);
                            const uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)v[2 * e + 1]);
                            w[e] = lo | (hi << 16);
                        } else {
                            w[e] = f32x2_to_bf16x2_bits(v[2 * e], v[2 * e + 1]);
                        }
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
    // Buffer offsets of the rows a tile reaches past M or N (plus the second half of a last pair
    // of steps) must stay below 2^32.
    if ((uint64_t)(M + TM) * (K / 2) + 128 >= kOutOfRange || (uint64_t)(N + TN) * (K / 2) + 128 >= kOutOfRange)
        fail("byhip: MXFP4 operands above 4 GiB are not supported");
    MxArgs a;
    a.x = x; a.xs = x_scales; a.w = w; a.ws = w_scales; a.y = y;
    a.M = M; a.K = K; a.N = N;
    a.tiles_m = (M + TM - 1) / TM;
    a.tiles = a.tiles_m * ((N + TN - 1) / TN);
    a.per_xcd = (a.tiles + kXcds - 1) / kXcds;
    const dim3 grid(kXcds * a.per_xcd);
    switch (y_dtype) {
    case BYHIP_F32: launch("mxfp4_gemm", mxfp4_gemm<BYHIP_F32>, grid, dim3(256), 0, a); break;
    case BYHIP_F16: launch("mxfp4_gemm", mxfp4_gemm<BYHIP_F16>, grid, dim3(256), 0, a); break;
    default: launch("mxfp4_gemm", mxfp4_gemm<BYHIP_BF16>, grid, dim3(256), 0, a); break;
    }
    BYHIP_LAUNCHED("mxfp4_gemm");
}

}  // namespace byhip
