// byhip_fp4.hip - FP4-KM tile GEMM, native MXFP4, FP16 tile GEMM, the micro-VM program route and
// the tile GEMM parity gate.
//
// FP4-KM (cpu_vm.c:583-628): weight = lut[nibble] * lut[16 + scale byte] with the 272-float decode
// table; nibble bytes [N, K/2] (byte j of a group: element j low, j + 16 high), scale bytes
// [N, K/32] at scale_base. fp32/fp16 activations take the fp16 MFMA GEMM with the weights decoded
// through the table in LDS; activations already in MXFP4 take the scaled MFMA when the table is
// exactly E2M1 and 2^(e-127).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "byhip_gemm.h"
#include "byhip_internal.h"
#include "byhip_kernels.h"

namespace byhip {

void q4_matmul_run(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M, bool exact);

namespace {

constexpr float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                             -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// The decode table is E2M1 followed by E8M0 (2^(e-127)) exactly: bitwise for the 16 values, and
// for scale bytes 0..254; byte 255 (NaN in E8M0) must decode to a non-finite value.
bool lut_is_mx(const float* t) {
    for (int i = 0; i < 16; ++i)
        if (memcmp(&t[i], &kE2M1[i], 4) != 0) return false;
    for (int e = 0; e < 255; ++e)
        if (t[16 + e] != std::ldexp(1.0f, e - 127)) return false;
    return !std::isfinite(t[16 + 255]);
}

void check_dtype_y(int y_dtype) {
    if (y_dtype != BYHIP_F32 && y_dtype != BYHIP_F16 && y_dtype != BYHIP_BF16)
        fail("byhip: output must be F32, F16 or BF16");
}

__global__ void fp4km_unpack(const uint8_t* __restrict__ blob, size_t scale_base,
                             const float* __restrict__ lut, int K, int N, uint8_t* __restrict__ codes,
                             float* __restrict__ weights) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K) return;
    const size_t n = i / K, k = i % K, g = k >> 5, j = k & 31;
    const uint8_t byte = blob[n * ((size_t)K >> 1) + g * 16 + (j & 15)];
    const uint8_t code = j < 16 ? (byte & 15) : (byte >> 4);
    const uint8_t sb = blob[scale_base + n * ((size_t)K >> 5) + g];
    codes[i] = code;
    weights[i] = lut[code] * lut[16 + sb];
}

}  // namespace

// Whether every product lut[i] * lut[16 + b] (i < 16, b < 256), formed in fp32 as the reference
// forms it, is a finite fp16 value: then the fp16 MFMA kernel holds every weight exactly. The last
// table classified is remembered (a model keeps one table).
bool table_products_are_halves(const float* t) {
    static std::mutex mu;
    static float last[272];
    static bool have = false, last_ok = false;
    std::lock_guard<std::mutex> lk(mu);
    if (have && memcmp(last, t, sizeof last) == 0) return last_ok;
    bool ok = true;
    for (int b = 0; b < 256 && ok; ++b)
        for (int i = 0; i < 16; ++i) {
            const float p = t[i] * t[16 + b];
            if (!std::isfinite(p) || (float)(_Float16)p != p) {
                ok = false;
                break;
            }
        }
    memcpy(last, t, sizeof last);
    have = true;
    last_ok = ok;
    return ok;
}

// Device-side form of table_products_are_halves: thread b checks the 16 products with scale entry
// b (finite, and exact in fp16), and the block's AND goes to *flag (1: the products are halves).
__global__ __launch_bounds__(256) void fp4km_classify(const float* __restrict__ t, int* flag) {
    const float s = t[16 + threadIdx.x];
    bool ok = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float p = t[i] * s;
        ok = ok && __builtin_isfinite(p) && (float)(_Float16)p == p;
    }
    ok = __syncthreads_and(ok);
    if (threadIdx.x == 0) *flag = ok ? 1 : 0;
}

void fp4km_run(const void* x, int x_dtype, const uint8_t* blob, size_t blob_bytes, size_t scale_base,
               const float* lut, size_t lut_floats, size_t lut_base, void* y, int y_dtype, int M,
               int K, int N) {
    check_dtype_y(y_dtype);
    if (M <= 0 || K <= 0 || N <= 0 || K % 32 != 0)
        fail("byhip: unsupported tile GEMM (format 0 K %d N %d M %d)", K, N, M);
    if ((size_t)N * (K / 2) > blob_bytes || scale_base + (size_t)N * (K / 32) > blob_bytes ||
        lut_base + 272 > lut_floats)
        fail("byhip: tile GEMM input out of range");
    check_span(blob, blob_bytes, "tile GEMM weights");
    check_span(lut + lut_base, 272 * 4, "tile GEMM decode table");
    check_span(y, (size_t)M * N * dtype_bytes(y_dtype), "tile GEMM output");
    if (x_dtype == BYHIP_MXFP4_KM) {
        if (K % 128 != 0) unsupported("byhip: MXFP4 activations need K %% 128 == 0 (K=%d)", K);
        if (scale_base % 4 != 0 || reinterpret_cast<uintptr_t>(blob) % 16 != 0)
            unsupported("byhip: MXFP4 route needs 16-byte aligned weights and word-aligned scales");
        float t[272];
        read_small(lut, lut_base * 4, t, sizeof t);
        if (!lut_is_mx(t)) unsupported("byhip: decode table is not E2M1 / E8M0; MXFP4 route unavailable");
        const size_t xbytes = (size_t)M * (K / 2) + (size_t)M * (K / 32);
        check_span(x, xbytes, "MXFP4 activations");
        const uint8_t* xb = static_cast<const uint8_t*>(x);
        launch_mxfp4(xb, xb + (size_t)M * (K / 2), blob, blob + scale_base, y, y_dtype, M, K, N);
        return;
    }
    if (x_dtype != BYHIP_F32 && x_dtype != BYHIP_F16) fail("byhip: tile GEMM activations must be F32, F16 or MXFP4_KM");
    check_span(x, (size_t)M * K * dtype_bytes(x_dtype), "tile GEMM activations");
    GemmArgs a;
    a.x = x; a.x_dtype = x_dtype; a.y = y; a.y_dtype = y_dtype; a.M = M; a.K = K; a.N = N;
    a.blob = blob; a.scale_base = scale_base; a.lut = lut + lut_base;
    // The fp16 MFMA kernel when every decoded weight is a half, otherwise the exact fp32 GEMM. The
    // table is classified on the host from its host copy, outside recordings; otherwise on the
    // device, by a kernel that writes the choice to a flag, with both routes queued behind it and
    // each gated on the flag, so that a recording replays the right route for whatever table the
    // buffer holds at replay, and no call waits for the device to read the table.
    const bool aligned = reinterpret_cast<uintptr_t>(blob) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (aligned && env_int("BYHIP_TILE_EXACT", 0) == 0) {
        float t[272];
        if (!session_recording() && mirror_read(lut, lut_base * 4, t, sizeof t)) {
            if (table_products_are_halves(t)) {
                launch_gemm(BFormat::Fp4Km, a);
                return;
            }
        } else {
            int* flag = device_flags();
            launch("fp4km_classify", fp4km_classify, dim3(1), dim3(256), 0, static_cast<const float*>(lut + lut_base),
                   flag);
            GemmArgs g = a;
            g.gate = flag;
            g.gate_want = 1;
            launch_gemm(BFormat::Fp4Km, g);
            g.gate_want = 0;
            launch_gemm_exact(BFormat::Fp4Km, g);
            return;
        }
    }
    if (reinterpret_cast<uintptr_t>(blob) % 16 != 0)
        unsupported("byhip: tile GEMM needs 16-byte aligned weights");
    launch_gemm_exact(BFormat::Fp4Km, a);
}

void f16_run(const void* x, int x_dtype, const uint16_t* w, size_t w_halves, void* y, int y_dtype,
             int M, int K, int N) {
    check_dtype_y(y_dtype);
    if (M <= 0 || K <= 0 || N <= 0 || K % 32 != 0)
        fail("byhip: unsupported tile GEMM (format 1 K %d N %d M %d)", K, N, M);
    if ((size_t)N * K > w_halves) fail("byhip: tile GEMM input out of range");
    if (x_dtype != BYHIP_F32 && x_dtype != BYHIP_F16) fail("byhip: FP16 tile GEMM activations must be F32 or F16");
    check_span(w, (size_t)N * K * 2, "FP16 weights");
    check_span(x, (size_t)M * K * dtype_bytes(x_dtype), "tile GEMM activations");
    check_span(y, (size_t)M * N * dtype_bytes(y_dtype), "tile GEMM output");
    GemmArgs a;
    a.x = x; a.x_dtype = x_dtype; a.y = y; a.y_dtype = y_dtype; a.M = M; a.K = K; a.N = N;
    a.w16 = w;
    // Halves are exact in the fp16 MFMA kernel (fp32 activations as two fp16 terms); it reads
    // 16-byte words, so unaligned operands take the exact kernel, which reads element by element.
    if (reinterpret_cast<uintptr_t>(w) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0)
        launch_gemm(BFormat::F16, a);
    else
        launch_gemm_exact(BFormat::F16, a);
}

}  // namespace byhip

using namespace byhip;

namespace {

uint32_t reg_a(uint32_t w) { return ((w >> 8) & 0x1Fu) | (((w >> 23) & 0x7u) << 5); }

bool tile_op_noop(uint32_t op) { return op == 0x00 || op == 0x50 || (op >= 0xB1 && op <= 0xB8); }

// The tile GEMM parity gate's closed-form data (vulkanTileGemmReady, vulkan_driver.nim:2697-2731):
// every product is exact in fp16 inputs and every sum exact in fp32, so the expected values are exact.
bool run_ready_gate(bool f16) {
    const int M = 37, K = 128, N = 80;
    std::vector<float> x(M * K), table(272, 0.0f), expected(M * N);
    for (int i = 0; i < M * K; ++i) x[i] = (float)((i * 7 + 3) % 33 - 16) / 64.0f;
    std::vector<uint8_t> wbytes;
    if (f16) {
        std::vector<float> wv(N * K);
        for (int i = 0; i < N * K; ++i) wv[i] = (float)((i * 5 + 1) % 29 - 14) / 16.0f;
        wbytes.resize((size_t)N * K * 2);
        for (int i = 0; i < N * K; ++i) {
            // values are k/16 with |k| <= 14: exact halves
            _Float16 h = (_Float16)wv[i];
            memcpy(&wbytes[2 * i], &h, 2);
        }
        for (int r = 0; r < M; ++r)
            for (int c = 0; c < N; ++c) {
                double s = 0.0;
                for (int k = 0; k < K; ++k) s += (double)x[r * K + k] * wv[c * K + k];
                expected[r * N + c] = (float)s;
            }
    } else {
        for (int i = 0; i < 16; ++i) table[i] = kE2M1[i];
        for (int i = 0; i < 256; ++i) table[16 + i] = std::ldexp(1.0f, i % 5 - 3);
        const int groups = K / 32;
        wbytes.resize((size_t)N * (K / 2) + (size_t)N * groups);
        for (int i = 0; i < N * (K / 2); ++i) wbytes[i] = (uint8_t)((i * 37 + 11) % 256);
        for (int i = 0; i < N * groups; ++i) wbytes[N * (K / 2) + i] = (uint8_t)((i * 13 + 5) % 256);
        for (int r = 0; r < M; ++r)
            for (int c = 0; c < N; ++c) {
                double s = 0.0;
                for (int g = 0; g < groups; ++g) {
                    const double sc = table[16 + wbytes[N * (K / 2) + c * groups + g]];
                    for (int j = 0; j < 16; ++j) {
                        const uint8_t b = wbytes[c * (K / 2) + g * 16 + j];
                        s += (double)x[r * K + g * 32 + j] * table[b & 15] * sc;
                        s += (double)x[r * K + g * 32 + 16 + j] * table[b >> 4] * sc;
                    }
                }
                expected[r * N + c] = (float)s;
            }
    }
    void* dx = device_alloc(x.size() * 4);
    void* dw = device_alloc(wbytes.size());
    void* dl = device_alloc(272 * 4);
    void* dy = device_alloc((size_t)M * N * 4);
    bool ok = false;
    try {
        BYHIP_HIP(hipMemcpyAsync(dx, x.data(), x.size() * 4, hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipMemcpyAsync(dw, wbytes.data(), wbytes.size(), hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipMemcpyAsync(dl, table.data(), 272 * 4, hipMemcpyHostToDevice, stream()));
        if (f16)
            f16_run(dx, BYHIP_F32, static_cast<const uint16_t*>(dw), wbytes.size() / 2, dy, BYHIP_F32, M, K, N);
        else
            fp4km_run(dx, BYHIP_F32, static_cast<const uint8_t*>(dw), wbytes.size(), (size_t)N * (K / 2),
                      static_cast<const float*>(dl), 272, 0, dy, BYHIP_F32, M, K, N);
        std::vector<float> got((size_t)M * N);
        BYHIP_HIP(hipStreamSynchronize(stream()));
        BYHIP_HIP(hipMemcpy(got.data(), dy, got.size() * 4, hipMemcpyDeviceToHost));
        double worst = 0.0;
        for (size_t i = 0; i < got.size(); ++i) {
            const double e = std::fabs((double)got[i] - expected[i]) / std::fmax(1.0, std::fabs((double)expected[i]));
            worst = (e != e) ? INFINITY : std::fmax(worst, e);
        }
        ok = worst <= 1e-3;
    } catch (...) {
        device_free(dx); device_free(dw); device_free(dl); device_free(dy);
        throw;
    }
    device_free(dx); device_free(dw); device_free(dl); device_free(dy);
    return ok;
}

}  // namespace

extern "C" {

int byhip_fp4km_tile_gemm(const void* x, int x_dtype, const uint8_t* blob, size_t blob_bytes,
                          size_t scale_base, const float* lut, size_t lut_floats, size_t lut_base,
                          void* y, int y_dtype, int M, int K, int N) {
    return guard([&] {
        enter_compute();
        note_device_write(y);
        fp4km_run(x, x_dtype, blob, blob_bytes, scale_base, lut, lut_floats, lut_base, y, y_dtype, M, K, N);
    });
}

int byhip_mxfp4_gemm(const uint8_t* x, const uint8_t* w, void* y, int y_dtype, int M, int K, int N) {
    return guard([&] {
        enter_compute();
        check_dtype_y(y_dtype);
        if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0)
            fail("byhip: MXFP4 GEMM needs M, N > 0 and K %% 128 == 0 (M=%d K=%d N=%d)", M, K, N);
        const size_t xb = (size_t)M * (K / 2), wb = (size_t)N * (K / 2);
        check_span(x, xb + (size_t)M * (K / 32), "MXFP4 activations");
        check_span(w, wb + (size_t)N * (K / 32), "MXFP4 weights");
        check_span(y, (size_t)M * N * dtype_bytes(y_dtype), "MXFP4 output");
        if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
            fail("byhip: MXFP4 operands must be 16-byte aligned");
        note_device_write(y);
        launch_mxfp4(x, x + xb, w, w + wb, y, y_dtype, M, K, N);
    });
}

int byhip_f16_tile_gemm(const void* x, int x_dtype, const uint16_t* w, size_t w_halves, void* y,
                        int y_dtype, int M, int K, int N) {
    return guard([&] {
        enter_compute();
        note_device_write(y);
        f16_run(x, x_dtype, w, w_halves, y, y_dtype, M, K, N);
    });
}

int byhip_tile_gemm_ready(int f16, int tensor_core) {
    static int cache[2] = {-1, -1};
    int result = BYHIP_ERROR;
    const int rc = guard([&] {
        enter_compute();
        no_host_sync("byhip_tile_gemm_ready");
        (void)tensor_core;  // every HIP route is an MFMA route
        int& c = cache[f16 ? 1 : 0];
        if (c < 0) c = run_ready_gate(f16 != 0) ? 1 : 0;
        result = c;
    });
    return rc == BYHIP_OK ? result : rc;
}

int byhip_program_dispatch(const uint32_t* words, int n_words, void* mem, size_t mem_len,
                           const void* u8, size_t u8_len, const void* lut, size_t lut_len,
                           const void* input, size_t input_len, int rows) {
    return guard([&] {
        enter_compute();
        // The reference's checks in its order (cpu_vm.c:178-188, 420-628), with its messages.
        if (!words || n_words <= 0 || !mem || mem_len == 0) fail("invalid CPU VM arguments");
        note_device_write(mem);
        const uint32_t w0 = words[0], op = w0 & 0xFFu, fmt = reg_a(w0);
        if (op != 0xB0 && op != 0xAC && op != 0xAA && op != 0xAB)
            unsupported("byhip: program op 0x%02x is not a tile GEMM / Q4 / FP4 shape op", op);
        if (n_words < 6)
            fail(op == 0xB0 ? "CPU VM truncated tile GEMM header"
                            : (op == 0xAC ? "CPU VM truncated FP4 shape op" : "CPU VM truncated Q4 shape op"));
        uint32_t M = words[1];
        const uint32_t K = words[2], N = words[3];
        const float* in = static_cast<const float*>(input ? input : mem);
        const size_t in_len = input ? input_len : mem_len;

        // Shape and slot validation; then `stop`, the first output (row-major) at which the
        // reference stops with `msg` (it checks each output's inputs before storing it), or -1.
        int64_t stop = -1;
        char msg[160] = "";
        auto stop_at = [&](int64_t at, const char* text) {
            if (stop < 0 || at < stop) {
                stop = at;
                snprintf(msg, sizeof msg, "%s", text);
            }
        };
        auto store_stop = [&](const char* what) {
            if ((uint64_t)M * N > mem_len) {
                char t[96];
                snprintf(t, sizeof t, "CPU VM %s out of range: %lld", what, (long long)mem_len);
                if (stop < 0 || (int64_t)mem_len < stop) stop_at((int64_t)mem_len, t);
            }
        };
        const uint32_t group = words[4], n_groups = words[5];
        if (op == 0xB0) {
            if (fmt > 1u || !K || K % 32u || !N)
                fail("CPU VM unsupported tile GEMM (format %u K %u N %u)", fmt, K, N);
            if (!u8 || (fmt == 0u && !lut)) fail("CPU VM tile GEMM slot is missing");
            if (M == 0) M = rows > 0 ? (uint32_t)rows : (uint32_t)(in_len / K);
            const bool range = fmt == 1u ? (uint64_t)N * K * 2 > u8_len
                                         : ((uint64_t)N * (K / 2) > u8_len || (uint64_t)words[4] + (uint64_t)N * (K / 32) > u8_len ||
                                            (uint64_t)words[5] + 272 > lut_len);
            if (range || (uint64_t)M * K > in_len) fail("CPU VM tile GEMM input out of range");
            store_stop("tile_gemm_store");
        } else if (op == 0xAC) {
            if (!M || !K || K % 64u || N < 16u || group != 32u || n_groups != K / 32u)
                fail("CPU VM unsupported FP4 cooperative shape");
            if (!u8 || !lut) fail("CPU VM FP4 cooperative slot is missing");
            const uint64_t scale_bytes = (uint64_t)N * (K / 2);
            const uint64_t lut_base = (scale_bytes + (uint64_t)N * n_groups + 3u) / 4u;
            if (scale_bytes + (uint64_t)N * n_groups > u8_len || lut_base + 272 > lut_len || (uint64_t)M * K > in_len)
                fail("CPU VM FP4 cooperative input out of range");
            store_stop("fp4_coop_store");
        } else {
            const bool coop = op == 0xAA;
            if (!M || !N || !K || !group || K % group || n_groups != K / group ||
                (coop && (N < 16u || K % 64u || group % 2u)) || (!coop && (K % 8u || group % 8u)))
                fail(coop ? "CPU VM unsupported Q4 cooperative shape" : "CPU VM unsupported Q4 GEMV shape");
            if (!u8 || !lut) fail("CPU VM Q4 cooperative slot is missing");
            // Output (r, c) reads bytes c * K/2 + k/2, zeros at zero_base + c * groups + k / group
            // (past every scale it reads) and x[r * K + k]: its largest indices decide it.
            const uint64_t rb = K / 2u, scale_base = ((uint64_t)N * rb + 3u) / 4u;
            const uint64_t zero_base = scale_base + (uint64_t)N * n_groups;
            auto first_col = [](uint64_t at0, uint64_t per_col, uint64_t len) {
                return at0 >= len ? (uint64_t)0 : (len - at0 + per_col - 1) / per_col;
            };
            const uint64_t c_in = std::min(first_col((K - 1u) / 2u, rb, u8_len),
                                           first_col(zero_base + (K - 1u) / group, n_groups, lut_len));
            const uint64_t r_x = in_len / K;  // the first row whose activations run past the input
            int64_t in_stop = -1;
            if (r_x == 0 || c_in == 0) in_stop = 0;
            else if (c_in < N) in_stop = (int64_t)c_in;
            else if (r_x < M) in_stop = (int64_t)(r_x * N);
            if (in_stop >= 0) stop_at(in_stop, "CPU VM Q4 cooperative input out of range");
            store_stop("q4_coop_store");
        }
        for (int pc = 6; pc < n_words; ++pc) {
            const uint32_t o = words[pc] & 0xFFu;
            if (o == 0x01) break;
            if (!tile_op_noop(o)) unsupported("byhip: op 0x%02x after a shape op has no HIP route", o);
        }

        // The outputs the reference computes before it stops (all of them when it does not):
        // whole rows, then the first columns of the next row.
        const uint64_t total = (uint64_t)M * N, done = stop < 0 ? total : std::min<uint64_t>((uint64_t)stop, total);
        auto run = [&](uint32_t Mx, uint32_t Nx, const float* xp, float* yp) {
            if (!Mx || !Nx) return;
            if (op == 0xB0 && fmt == 1u) {
                f16_run(xp, BYHIP_F32, static_cast<const uint16_t*>(u8), u8_len / 2, yp, BYHIP_F32, Mx, K, Nx);
            } else if (op == 0xB0) {
                fp4km_run(xp, BYHIP_F32, static_cast<const uint8_t*>(u8), u8_len, words[4],
                          static_cast<const float*>(lut), lut_len, words[5], yp, BYHIP_F32, Mx, K, Nx);
            } else if (op == 0xAC) {
                const size_t scale_bytes = (size_t)N * (K / 2);
                const size_t lut_base = (scale_bytes + (size_t)N * n_groups + 3u) / 4u;
                fp4km_run(xp, BYHIP_F32, static_cast<const uint8_t*>(u8), u8_len, scale_bytes,
                          static_cast<const float*>(lut), lut_len, lut_base, yp, BYHIP_F32, Mx, K, Nx);
            } else {
                // The Q4 shape ops are fp32 arithmetic in the reference: the exact routes.
                const size_t rb = K / 2u, scale_base = ((size_t)N * rb + 3u) / 4u;
                const size_t zero_base = scale_base + (size_t)N * n_groups;
                check_span(u8, (size_t)Nx * rb, "Q4 nibbles");
                check_span(static_cast<const float*>(lut) + scale_base, ((size_t)N * n_groups + (size_t)Nx * n_groups) * 4,
                           "Q4 scales and zeros");
                byhip_q4w w{};
                w.K = (int)K; w.N = (int)Nx; w.group = (int)group; w.gpr = (int)n_groups; w.row_bytes = rb;
                w.wq = const_cast<uint8_t*>(static_cast<const uint8_t*>(u8));
                w.scales = const_cast<float*>(static_cast<const float*>(lut) + scale_base);
                w.zeros = const_cast<float*>(static_cast<const float*>(lut) + zero_base);
                w.scale_f16 = 0;
                w.zero_uniform = 0;
                q4_matmul_run(xp, BYHIP_F32, &w, yp, BYHIP_F32, (int)Mx, true);
            }
        };
        float* y = static_cast<float*>(mem);
        const uint32_t full = (uint32_t)(done / N), rem = (uint32_t)(done % N);
        run(full, N, in, y);
        run(rem ? 1u : 0u, rem, in + (size_t)full * K, y + (size_t)full * N);
        if (stop >= 0) fail("%s", msg);
    });
}

int byhip_debug_unpack_fp4km(const uint8_t* blob, size_t scale_base, const float* lut, size_t lut_base,
                             int K, int N, uint8_t* codes, float* weights) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_debug_unpack_fp4km");
        if (!blob || !lut || !codes || !weights || K <= 0 || N <= 0 || K % 32)
            fail("byhip: invalid FP4-KM unpack arguments");
        check_span(blob, scale_base + (size_t)N * (K / 32), "FP4-KM blob");
        const size_t total = (size_t)N * K;
        uint8_t* dc = static_cast<uint8_t*>(device_alloc(total));
        float* dw = static_cast<float*>(device_alloc(total * 4));
        try {
            launch("fp4km_unpack", fp4km_unpack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, blob,
                               scale_base, lut + lut_base, K, N, dc, dw);
        } catch (...) {
            device_free(dc);
            device_free(dw);
            throw;
        }
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(stream());
        if (e == hipSuccess) e = hipMemcpy(codes, dc, total, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(weights, dw, total * 4, hipMemcpyDeviceToHost);
        device_free(dc);
        device_free(dw);
        BYHIP_HIP(e);
    });
}

}  // extern "C"
