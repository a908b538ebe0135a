/* byby_oracle.h - CPU restatement of the reference's quantized tile-GEMM arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (bybylang_amd/, include/) links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
 * it, and only as the checker or as the timed CPU baseline, never as the thing measured or
 * shipped.
 *
 * Every function restates one loop of the reference (bobbyshop-vui/bybylang) and cites the
 * file:line it follows. Loop order, fused/unfused multiply-adds and float evaluation order follow
 * the reference so results are bit-identical; build with -O3 -ffp-contract=off so the compiler
 * does not contract a*b+c where the reference does not.
 *
 * Pinning (how each function is checked, beyond retyping its formula):
 *   - golden fixtures in tests/golden/ written from the reference's own C (cpu_vm.c,
 *     cpu_kernels.c) compiled into oracle/_ref/ (bit-exact comparisons);
 *   - oracle/_ref itself when it is built (bit-exact, random shapes);
 *   - closed forms: power-of-two data whose sums are exact in fp32, fp64 brute force within the
 *     accumulated-rounding bound, the E2M1 table, planted mistakes that must be detected.
 */
#ifndef BYBY_ORACLE_H
#define BYBY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opcodes of the shape-op programs (session_vm.nim:98-118). */
enum {
    ORC_OP_NOP = 0x00, ORC_OP_HALT = 0x01, ORC_OP_BARRIER_TG = 0x50,
    ORC_OP_Q4_COOP_GEMM = 0xAA, ORC_OP_Q4_GEMV = 0xAB, ORC_OP_FP4_COOP_GEMM = 0xAC,
    ORC_OP_TILE_GEMM = 0xB0, ORC_OP_TILE_ZERO = 0xB1, ORC_OP_TILE_K_BEGIN = 0xB2,
    ORC_OP_TILE_K_END = 0xB3, ORC_OP_TILE_LOAD_A = 0xB4, ORC_OP_TILE_DECODE_FP4 = 0xB5,
    ORC_OP_TILE_MMA = 0xB6, ORC_OP_TILE_STORE = 0xB7, ORC_OP_TILE_LOAD_B_F16 = 0xB8
};

/* IEEE binary16 -> binary32, cpu_vm.c:53-69. */
float orc_half_to_float(uint16_t h);
/* binary32 -> binary16, round to nearest even (generators; checked against every half). */
uint16_t orc_float_to_half(float f);

/* Q4 shape ops OP_Q4_GEMV (coop = 0) and OP_Q4_COOP_GEMM (coop = 1), cpu_vm.c:420-482.
 * qdata = the u8 slot (nibbles [N, K/2], even k in the low nibble); params = the lut slot read as
 * floats: scales [N, n_groups] at float (N*K/2+3)/4, zeros right after them. x = input slot
 * [M, K], out = mem slot [M, N]. Rows [row_begin, row_end) only (the full op is 0..M); the
 * per-output arithmetic does not depend on the split. Returns 0, or -1 with the reference's
 * error text in err. */
int orc_q4_shape_op(int coop, uint32_t M, uint32_t K, uint32_t N, uint32_t group_size,
                    uint32_t n_groups, const uint8_t* qdata, int64_t q_len,
                    const float* params, int64_t params_len, const float* x, int64_t x_len,
                    float* out, int64_t out_len, uint32_t row_begin, uint32_t row_end,
                    char* err, int err_len);

/* Legacy OP_FP4_COOP_GEMM (one blob: nibbles, scale bytes, word pad, 272-float table),
 * cpu_vm.c:483-540. */
int orc_fp4_coop_gemm(uint32_t M, uint32_t K, uint32_t N, uint32_t group_size, uint32_t n_groups,
                      const uint8_t* qdata, int64_t q_len, const float* params, int64_t params_len,
                      const float* x, int64_t x_len, float* out, int64_t out_len,
                      char* err, int err_len);

/* OP_TILE_GEMM, format 0 (FP4-KM) and format 1 (FP16 halves [N, K]), cpu_vm.c:541-628.
 * M = 0 takes the row count from x_len / K (cpu_vm.c:566,595). Rows [row_begin, row_end) of the
 * resolved M (pass row_end = UINT32_MAX for all rows). */
int orc_tile_gemm(uint32_t format, uint32_t M, uint32_t K, uint32_t N, uint64_t scale_base,
                  uint64_t lut_base, const uint8_t* packed, int64_t packed_len,
                  const float* lut, int64_t lut_len, const float* x, int64_t x_len,
                  float* out, int64_t out_len, uint32_t row_begin, uint32_t row_end,
                  char* err, int err_len);

/* Host reference of the FP4-KM tile GEMM, unfused sum += x * (t * s), tile_gemm.nim:663-677. */
void orc_tile_gemm_reference(const float* x, const uint8_t* packed, const float* table,
                             int rows, int K, int N, int64_t scale_base, int64_t lut_base,
                             float* out);

/* CPU_FN(matmul_q4): sum += a * (q - z) * s evaluated left to right, no contraction,
 * cpu_kernels_impl.inc:293-319 (reached through nimf_cpu_matmul_q4, cpu_kernels.c:423-430). */
void orc_matmul_q4(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                   float* c, int M, int K, int N, int group_size, int groups_per_row,
                   int row_begin, int row_end);

/* cpuMatmulQ4Ref: sum += a * ((q - z) * s), gpubackend.nim:288-311. */
void orc_matmul_q4_ref(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                       float* c, int M, int K, int N, int group_size, int groups_per_row);

/* The fused decode GEMV (M = 1) of sessionMatmulQ4Fused (gpubackend.nim:3185-3231) with the
 * arithmetic of its shader matmul_q4_fused (backends/vulkan/q4_autotune.nim:194-330):
 *   x[k] = a[k] * gamma[k] with RMSNorm (gamma != NULL), else a[k];
 *   per output row: acc = sum over k of fma(w, x[k], acc), w = ((float)q - z) * s;
 *   with RMSNorm, acc *= inv, inv = 1 / sqrt(ssq / K + eps), ssq = sum of fma(a, a, ssq);
 *   mode 0: n_mats (1..3) matrices share x, out[i][row] = acc_i;
 *   mode 1: matrices 0 (gate) and 1 (up), out[0][row] = silu(g) * u, silu(v) = v / (1 + exp(-v));
 *   residual[row] (matrix-local row) is added last when residual != NULL.
 * Sums run over k in order (the shader's lane partition and tree reduction reorder them; the
 * checks allow fp32 accumulation differences). Returns 0, or -1 for the argument combinations the
 * reference rejects (n_mats outside 1..3, mode 1 without exactly two matrices, another mode). */
int orc_q4_fused(int mode, int n_mats, const float* a, int K, int group_size, int groups_per_row,
                 const uint8_t* const* wq, const float* const* scales, const float* const* zeros,
                 const int* N, float* const* out, const float* residual, const float* gamma,
                 float eps);

/* A shape-op program run the way nimf_cpu_vm_run_slots (cpu_vm.c:178) runs it: the first
 * instruction is one of the five-word shape ops, the rest may only be the tile ops (no-ops on the
 * CPU, cpu_vm.c:629-631), threadgroup barriers, NOPs and HALT. Slot lengths are in the units the
 * reference uses (mem/lut/input floats, packed bytes). */
int orc_run_shape_program(const uint32_t* code, int n_words, float* mem, int mem_len,
                          const uint8_t* packed, int packed_len, const float* lut, int lut_len,
                          const float* in_f32, int in_len, char* err, int err_len);

/* Q4 unpack (bit-exact checks): codes[n*K + k] = nibble k of row n; g = k / group. */
void orc_unpack_q4(const uint8_t* wq, int K, int N, uint8_t* codes);
/* FP4-KM unpack: codes[n*K + k] = the 4-bit code of element k of row n (byte j of group g holds
 * element j low, j + 16 high: session_vm.nim:384-388); scale_bytes[n*(K/32)+g] copied out. */
void orc_unpack_fp4km(const uint8_t* packed, int64_t scale_base, int K, int N, uint8_t* codes,
                      uint8_t* scale_bytes);

/* Generators of tests/t_fp4_tile_gemm.nim. xorshift32 (30-33); one seed shared by every case in
 * the order the test makes them. */
uint32_t orc_xorshift32(uint32_t* state);
/* makeCase (35-44): x [M*K], packed [N*K/2 + N*K/32], table [272]. */
void orc_make_fp4_case(uint32_t* state, int M, int K, int N, float* x, uint8_t* packed,
                       float* table);
/* makeF16Case (210-223): x [M*K], w [N*K] (exact halves), halves [N*K*2] little endian. */
void orc_make_f16_case(uint32_t* state, int M, int K, int N, float* x, float* w,
                       uint8_t* halves);

#ifdef __cplusplus
}
#endif
#endif
