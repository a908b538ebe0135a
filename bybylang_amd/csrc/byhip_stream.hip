// byhip_stream.hip - the small-M streaming Q4 GEMM (gfx950): y[M, N] = x[M, K] . W^T for 9 .. 32
// rows of fp16 activations on resident weights with the prefill copy (cpu_kernels_impl.inc:293-319
// semantics; each weight rounded once to fp16, fp32 accumulation in v_mfma_f32_16x16x32_f16).
//
// At small M the weights dominate the bytes, and a GEMM tile that covers only part of K (split-K)
// pays a second launch for the partial sums, while a tile that covers all of K but few columns
// leaves most CUs idle. Here one block per CU owns a strip of 16 FN output columns over the whole
// K, so every weight byte streams from HBM once and the grid fills the chip at any N. From 17 rows
// a strip has two 16-row blocks on one XCD (the second read of its weights hits that XCD's L2):
//   Block: eight waves (two per SIMD). Wave w takes the block's 64-value sub-steps w, w + 8, ...
//   (counted from a per-block starting sub-step, wrapping around) for all BM rows and all FN
//   column fragments, with private LDS buffers, so the K loop has no block barrier; the eight
//   partial tiles are added in wave order at the end.
//   Per sub-step a wave moves the BM activation rows' 128-byte slices straight into one of its
//   four LDS buffers (1 KB direct loads, whole lines, XOR-swizzled as in the wide tile so the
//   fragment reads are free of bank conflicts), loads each fragment's 512 contiguous bytes of the
//   prefill copy (8 bytes per lane) and its fp16 scale, three sub-steps ahead.
//   The activations are the same for every block and come from L2: per CU that is BM x K x 2 bytes
//   (128 KB per 16-row block at K = 4096). The weight and scale loads are inline assembly, outside
//   the compiler's wait-count tracking, which had drained the loads ahead in every sub-step; the K
//   loop's explicit waits cover them. Measured at M = 32 (weights rotated past the Infinity Cache,
//   against the split-K kernels and their sum launch): K x N = 4096 x 4096 6.6 us against 8.8,
//   4096 x 6144 8.0 against 10.4, but 4096 x 28672 (seven fragments per block, dequantization-
//   heavy) 21.3 against 17.1 and 14336 x 4096 15.5-15.9 against 13.1 (the last two before the load
//   change). The router therefore takes it for at most two fragments per 32-row block and K up to
//   8192.
#include <algorithm>

#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {
namespace {

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

constexpr int kStreamWaves = 8;  // per block, one block per CU
constexpr int kSub = 64;         // K values per sub-step (the prefill copy's unit)
constexpr int kMaxFN = 8;        // column fragments per block

// LDS buffers and register sets per wave: loads three sub-steps ahead. Eight buffers of 16 rows
// (every sub-step of a wave at K = 4096 in flight at once) measured slower in a timing copy at
// M = 32 (qkv 12.0 against 9.9 us, o 9.7 against 8.1: the first data arrive later).
constexpr int kStreamDepth = 4;

template <int FM, int FN, int D = kStreamDepth>
struct StreamShape {
    static constexpr int kBM = 16 * FM;
    static constexpr int kXBuf = kBM * kSub * 2;        // one sub-step's activation slices
    static constexpr int kXLoads = kBM / 8;             // 1 KB direct loads per sub-step
    static constexpr int kLoads = kXLoads + 2 * FN;     // with the weights and the scales
    static constexpr int kLdsX = kStreamWaves * D * kXBuf;
    static constexpr int kPitch = 16 * FN + 4;          // floats per row of a staged partial tile
    static constexpr int kLdsRed = kStreamWaves * kBM * kPitch * 4;
    static constexpr int kLds = kLdsX > kLdsRed ? kLdsX : kLdsRed;
};

// One wave's weights of one sub-step: per fragment 16 nibbles (two words) and the fp16 scale of the
// lane's 32-value group.
template <int FN>
struct StreamW {
    v2u w[FN];
    uint32_t s[FN];
};

template <int FM, int FN, int YT, int D = kStreamDepth>
__global__ __launch_bounds__(512, 1) void q4_gemm_stream(GemmArgs a) {
    using S = StreamShape<FM, FN, D>;
    constexpr int BM = S::kBM, L = S::kLoads;
    static_assert(S::kLds <= 160 * 1024 && (D - 1) * L <= 63,
                  "q4_gemm_stream: the buffers must fit LDS and the loads in flight the wait counter");
    __shared__ __attribute__((aligned(16))) uint8_t lds[S::kLds];

    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int f0 = blockIdx.x * FN;  // the block's first column fragment
    const int m0 = (int)blockIdx.y * BM;  // the block's first activation row
    if (16 * f0 >= a.N) return;  // a block of the grid's rounding (whole block, before any barrier)
    const int K = a.K;
    const uint32_t nsub_all = (uint32_t)K / kSub;
    const int s_first = a.part ? (int)blockIdx.z * a.split_steps : 0;
    const int nsub = a.part ? min(a.split_steps, (int)nsub_all - s_first) : (int)nsub_all;
    const int nt = nsub > w ? (nsub - w + kStreamWaves - 1) / kStreamWaves : 0;  // this wave's sub-steps
    // Every block reads the same activations: each starts its K walk at its own sub-step (and wraps
    // around), so that the blocks sharing an L2 do not all request the same lines at once.
    const int rot = (int)((blockIdx.x * 5u) % (uint32_t)max(nsub, 1));
    // sub-step of the wave's t-th (t < nt): (w + 8 t + rot) mod nsub, from the split's first
    auto sub_of = [&](int t) __attribute__((always_inline)) {
        int v = w + kStreamWaves * t + rot;
        v -= v >= nsub ? nsub : 0;
        v -= v >= nsub ? nsub : 0;
        return (uint32_t)(s_first + v);
    };

    // Rows past M and sub-steps past the wave's last read zeros: their per-lane offsets lie past the
    // resources' sizes (the launcher keeps every offset below 2^31, and the out-of-range marker 2^31
    // goes into the per-lane offset). Fragments past N are read at the last fragment and never
    // stored.
    const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.M * K * 2));
    const rsrc_t wr = make_rsrc(a.wpf, (uint32_t)(((size_t)a.N + 15) / 16 * nsub_all * 512));
    const rsrc_t sr = make_rsrc(a.spf, (uint32_t)(((size_t)a.N + 63) / 64 * nsub_all * 256));
    // Direct load q: rows 8 q + lane / 8, LDS slot lane % 8 holding chunk (lane % 8) ^ x_swizzle(row).
    uint32_t xo[S::kXLoads];
#pragma unroll
    for (int q = 0; q < S::kXLoads; ++q) {
        const int r = 8 * q + (lane >> 3), chunk = (lane & 7) ^ x_swizzle(r);
        xo[q] = (uint32_t)(m0 + r) * (uint32_t)K * 2u + 16u * chunk;
    }
    const uint32_t wfrag = nsub_all * 512u, squad = nsub_all * 256u;
    // the lane's scale in a quad's [2][16][4] block: its 32-value group g / 2, column c
    const uint32_t soff = 2u * (4u * (16u * (uint32_t)(g >> 1) + (uint32_t)c));
    uint8_t* const xw = lds + w * D * S::kXBuf;  // this wave's buffers
    // Fragment reads: lane (c, g) reads row 16 i + c, chunk 2 g + kk, at slot (2 g + kk) ^ x_swizzle(c).
    const int rd0 = 128 * c + 16 * ((2 * g) ^ x_swizzle(c)), rd1 = 128 * c + 16 * ((2 * g + 1) ^ x_swizzle(c));

    const int flast = (a.N + 15) / 16 - 1;
    auto load_x = [&](int t, int buf) __attribute__((always_inline)) {
        const bool ok = t < nt;
        const uint32_t u = ok ? sub_of(t) : (uint32_t)s_first;
        const uint32_t oob = ok ? 0u : 0x80000000u;
        uint8_t* const dst = xw + buf * S::kXBuf;
#pragma unroll
        for (int q = 0; q < S::kXLoads; ++q) lds_dma16(xr, dst + 1024 * q, xo[q] + oob, 128u * u);
    };
    auto load_ws = [&](StreamW<FN>& r, int t) __attribute__((always_inline)) {
        const bool ok = t < nt;
        const uint32_t u = ok ? sub_of(t) : (uint32_t)s_first;
        const uint32_t oob = ok ? 0u : 0x80000000u;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const uint32_t f = (uint32_t)min(f0 + j, flast);
            // Default cache policy: marking these loads nontemporal measured slower here (M = 32:
            // 4096 x 4096 6.8 -> 8.3 us, 14336 x 4096 15.5 -> 20.3). Issued as assembly, so the
            // compiler's wait-count pass does not see them: through the K loop's back edge it
            // placed waits of vmcnt 2 to 11 before their first use, which drained the loads of
            // the sub-steps ahead in every sub-step. The K loop's explicit waits cover them (loads
            // complete in issue order: a register set is read only after the wait that follows
            // its sub-step's loads), and the sets stay live past the final wait.
            asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen"
                         : "=v"(r.w[j]) : "v"(8u * lane + oob), "s"(wr), "s"(f * wfrag + 512u * u));
            asm volatile("buffer_load_ushort %0, %1, %2, %3 offen"
                         : "=v"(r.s[j]) : "v"(soff + 2u * (f & 3u) + oob), "s"(sr), "s"((f >> 2) * squad + 256u * u));
        }
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

    // (q - zero) * scale in fp16 for MFMA kk (word kk of each fragment): the nibble pairs of the
    // prefill copy's order come out in natural K order from one AND-OR against the fp16 exponent
    // words (0x6400 | q is 1024 + q, 0x5400 | q << 4 is 64 + q), the bias and zero go in one exact
    // subtraction, and the product is rounded once.
    auto dequant = [&](const StreamW<FN>& r, int kk, h8 (&bw)[FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const _Float16 sc = bits_h((uint16_t)r.s[j]);
            const h2 ss = {sc, sc};
            const uint32_t d = r.w[j][kk], d8 = d >> 8;
            const h2 q0 = bits_h2((d & 0x000F000Fu) | mag_lo) - zz_lo;
            const h2 q1 = bits_h2((d & 0x00F000F0u) | mag_hi) - zz_hi;
            const h2 q2 = bits_h2((d8 & 0x000F000Fu) | mag_lo) - zz_lo;
            const h2 q3 = bits_h2((d8 & 0x00F000F0u) | mag_hi) - zz_hi;
            const uint4 u = make_uint4(h2_bits(q0 * ss), h2_bits(q1 * ss), h2_bits(q2 * ss), h2_bits(q3 * ss));
            bw[j] = *reinterpret_cast<const h8*>(&u);
        }
    };
    auto read_x = [&](int buf, int kk, h8 (&x)[FM]) __attribute__((always_inline)) {
        const uint8_t* src = xw + buf * S::kXBuf + (kk ? rd1 : rd0);
#pragma unroll
        for (int i = 0; i < FM; ++i) x[i] = *reinterpret_cast<const h8*>(src + 2048 * i);
    };

    // Sub-steps 0 .. D - 2 are loaded here, sub-step t + D - 1 in sub-step t into the buffer and
    // register set that sub-step t - 1 used (its fragment reads and weights were consumed by its
    // MFMAs). Loads past the wave's last sub-step read zeros, so every wait has the same count. A
    // sub-step runs in two halves: the kk = 0 MFMAs beside the kk = 1 fragment reads, the kk = 1
    // dequantization and the loads of t + D - 1; the wait for t + 1's loads (those of t + 2 ..
    // t + D - 1 stay in flight); the kk = 1 MFMAs beside t + 1's kk = 0 reads and dequantization.
    // Scheduling groups place each MFMA next to its share of the other work.
    StreamW<FN> rs[D];
    static_for<D - 1>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        load_x(k, k);
        load_ws(rs[k], k);
    });
    h8 x0[FM], x1[FM], b0[FN], b1[FN];
    // The weight loads are not tracked by the compiler, so their results look ready at once: after
    // the wait that covers a register set, the set passes through an empty asm statement, which no
    // use of it can be placed before.
    auto landed = [&](StreamW<FN>& r) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(r.w[j]), "+v"(r.s[j]));
    };
    wait_vmcnt<(D - 2) * L>();
    landed(rs[0]);
    read_x(0, 0, x0);
    dequant(rs[0], 0, b0);
    constexpr int kMfmas = FM * FN;  // per half
    constexpr int kValu = (14 * FN + kMfmas - 1) / kMfmas;
    auto step = [&](int t, auto kc) __attribute__((always_inline)) {
        constexpr int k = decltype(kc)::value, k1 = (k + 1) % D, kp = (k + D - 1) % D;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0[i], b0[j], acc[i][j], 0, 0, 0);
        read_x(k, 1, x1);
        dequant(rs[k], 1, b1);
        load_x(t + D - 1, kp);
        load_ws(rs[kp], t + D - 1);
#pragma unroll
        for (int m = 0; m < kMfmas; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                   // one MFMA
            if (m < FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);       // a fragment read
            if (m < L) __builtin_amdgcn_sched_group_barrier(0x0010, 1, 0);        // a load
            __builtin_amdgcn_sched_group_barrier(0x0002, kValu, 0);               // its share of the VALU
        }
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(D - 2) * L>();
        landed(rs[k1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1[i], b1[j], acc[i][j], 0, 0, 0);
        read_x(k1, 0, x0);
        dequant(rs[k1], 0, b0);
#pragma unroll
        for (int m = 0; m < kMfmas; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);                   // one MFMA
            if (m < FM) __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);       // a fragment read
            __builtin_amdgcn_sched_group_barrier(0x0002, kValu, 0);               // its share of the VALU
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Whole groups of D sub-steps, so the loop body has no branch around a step (a step past the
    // wave's last reads zeros, whose products add nothing): the register sets then keep one place
    // through the back edge and every step issues the same loads.
    for (int t0 = 0; t0 < nt; t0 += D) {
        static_for<D>([&](auto kc) {
            const int t = t0 + decltype(kc)::value;
            step(t, kc);
        });
    }

    // Partial tiles -> LDS in output layout once every load has landed (those past the last
    // sub-step wrote zeros into the buffers and registers) and every wave is done with its buffers
    // -> the eight partials added in wave order -> y or the split-K partials. The register sets
    // are kept live until the loads into them have landed.
    wait_vmcnt<0>();
#pragma unroll
    for (int k = 0; k < D; ++k)
#pragma unroll
        for (int j = 0; j < FN; ++j) asm volatile("" ::"v"(rs[k].w[j]), "v"(rs[k].s[j]));
    __syncthreads();
    constexpr int P = S::kPitch;
    float* red = reinterpret_cast<float*>(lds);  // [waves][BM rows][P]
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(w * BM + 16 * i + 4 * g + r) * P + 16 * j + c] = acc[i][j][r];
    __syncthreads();
    float* part = a.part ? a.part + (size_t)blockIdx.z * splitk_stride(a.M, a.N) : nullptr;
    const bool vec = out8_vector_ok<YT>(a, part);
    constexpr int kChunks = BM * 2 * FN;  // 8 outputs each
    for (int u = threadIdx.x; u < kChunks; u += 512) {
        const int row = u / (2 * FN), col = (u % (2 * FN)) * 8;
        if (m0 + row >= a.M) continue;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kStreamWaves; ++ww) {
            const float* src = red + (ww * BM + row) * P + col;
            const float4 s0 = *reinterpret_cast<const float4*>(src);
            const float4 s1 = *reinterpret_cast<const float4*>(src + 4);
            v[0] += s0.x; v[1] += s0.y; v[2] += s0.z; v[3] += s0.w;
            v[4] += s1.x; v[5] += s1.y; v[6] += s1.z; v[7] += s1.w;
        }
        store_out8<YT>(a, part, vec, m0 + row, 16 * f0 + col, v);
    }
}

template <int FM, int FN>
void launch_stream_y(const GemmArgs& a, dim3 grid) {
    switch (a.y_dtype) {
    case BYHIP_F32: launch("q4_gemm_stream", (q4_gemm_stream<FM, FN, BYHIP_F32>), grid, dim3(512), 0, a); break;
    case BYHIP_F16: launch("q4_gemm_stream", (q4_gemm_stream<FM, FN, BYHIP_F16>), grid, dim3(512), 0, a); break;
    default: launch("q4_gemm_stream", (q4_gemm_stream<FM, FN, BYHIP_BF16>), grid, dim3(512), 0, a); break;
    }
}

template <int FM>
void launch_stream_fm(const GemmArgs& a, int fn, dim3 grid) {
    switch (fn) {
    case 1: launch_stream_y<FM, 1>(a, grid); break;
    case 2: launch_stream_y<FM, 2>(a, grid); break;
    case 3: launch_stream_y<FM, 3>(a, grid); break;
    case 4: launch_stream_y<FM, 4>(a, grid); break;
    case 5: launch_stream_y<FM, 5>(a, grid); break;
    case 6: launch_stream_y<FM, 6>(a, grid); break;
    case 7: launch_stream_y<FM, 7>(a, grid); break;
    default: launch_stream_y<FM, 8>(a, grid); break;
    }
}

}  // namespace

// Row blocks: 17 to 32 rows run as two blocks of 16 rows over the same strip (each reads half the
// activations; the two share an XCD, so the second read of the strip's weights comes from its L2),
// unless BYHIP_Q4_STREAM_HALVES=0 keeps one block of 32 rows.
int stream_row_blocks(const GemmArgs& a) {
    return a.M > 16 && env_int("BYHIP_Q4_STREAM_HALVES", 1) != 0 ? 2 : 1;
}

// Column fragments per block with `row_blocks` blocks per strip: the fewest that give every CU at
// most one block.
int stream_fn(const GemmArgs& a, int row_blocks) {
    const long cus = compute_units(), nfr = (a.N + 15) / 16;
    return (int)std::min<long>(kMaxFN, std::max<long>(1, (nfr * row_blocks + cus - 1) / cus));
}

bool q4_stream_ok(const GemmArgs& a) {
    constexpr uint64_t kLim = 0x80000000u;  // offsets stay below 2^31 (the kernel's out-of-range steps)
    return a.x_dtype == BYHIP_F16 && a.wpf && a.spf && a.M >= 1 && a.M <= 32 && a.K % kSub == 0 &&
           (uint64_t)32 * a.K * 2 < kLim && (uint64_t)(a.N + 16 * kMaxFN) * a.K / 2 < kLim &&
           (uint64_t)(a.N + 64 * kMaxFN) / 64 * (a.K / kSub) * 256 < kLim;
}

// One strip of stream_fn column fragments (at most 8) per block and row block, so each CU streams
// one strip of the weights. Block (x, y) takes strip x and rows 16 y .. 16 y + 15 (or all 32 rows in
// one block). Blocks go to the XCDs round-robin in dispatch order (x first), so with two row blocks
// the strip count is rounded up to a multiple of 8 (the extra blocks exit at once) and the two
// blocks of a strip land on one XCD. K is split (fp32 partials, then splitk_sum) only when asked
// (`split_choice`, or BYHIP_Q4_SPLIT).
void launch_q4_stream(const GemmArgs& a0, int split_choice) {
    GemmArgs a = a0;
    const long nfr = (a.N + 15) / 16;
    const int rb = stream_row_blocks(a);
    const int fn = stream_fn(a, rb);
    const long strips = (nfr + fn - 1) / fn;
    const long blocks = rb == 2 ? (strips + 7) / 8 * 8 : strips;
    const int forced = split_choice > 0 ? split_choice : env_int("BYHIP_Q4_SPLIT", 0);
    const int splits = forced > 1 ? choose_split(a, strips * rb, a.K / kSub, kStreamWaves, forced, 1) : 1;
    if (splits == 1) a.part = nullptr;
    const dim3 grid((unsigned)blocks, (unsigned)rb, (unsigned)splits);
    if (a.M <= 16 || rb == 2) launch_stream_fm<1>(a, fn, grid);
    else launch_stream_fm<2>(a, fn, grid);
    BYHIP_LAUNCHED("q4_gemm_stream");
    if (a.part) launch_splitk_sum(a, splits);
}

}  // namespace byhip
