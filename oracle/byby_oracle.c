/* byby_oracle.c - CPU restatement of the reference's quantized tile-GEMM arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); the product never links it.
 * Build: -O3 -std=c11 -ffp-contract=off (the reference builds its C with -O3 -std=c11,
 * backends/cpu/cpu_backend.nim:22-24, which in ISO C mode also leaves a*b+c uncontracted).
 * Every loop cites the reference loop it restates; see byby_oracle.h for how each is pinned.
 */
#include "byby_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

static void set_err(char* err, int err_len, const char* msg) {
    if (err && err_len > 0) snprintf(err, (size_t)err_len, "%s", msg);
}

/* cpu_vm.c:53-69: sign, then zero / subnormal (renormalised) / inf-nan / normal. */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0u) {
        if (m == 0u) {
            bits = sign;
        } else {
            uint32_t e32 = 113u; /* 127 - 15 + 1: exponent of the leading subnormal bit */
            while ((m & 0x400u) == 0u) { m <<= 1; e32--; }
            bits = sign | (e32 << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31u) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* Round-to-nearest-even binary32 -> binary16 (used by generators only). */
uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal or zero */
        if (ax < 0x33000000u) return sign;                    /* below 2^-25: rounds to zero */
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); half subnormal unit 2^-24 */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u, m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* OP_Q4_GEMV / OP_Q4_COOP_GEMM, cpu_vm.c:420-482. Validation text and order follow 426-432 and
 * 441-445; the index arithmetic is uint32 as in 448-463; the k loop is one serial fmaf chain
 * (470). */
int orc_q4_shape_op(int coop, uint32_t M, uint32_t K, uint32_t N, uint32_t group_size,
                    uint32_t n_groups, const uint8_t* qdata, int64_t q_len,
                    const float* params, int64_t params_len, const float* x, int64_t x_len,
                    float* out, int64_t out_len, uint32_t row_begin, uint32_t row_end,
                    char* err, int err_len) {
    if (err && err_len > 0) err[0] = '\0';
    if (!M || !N || !K || !group_size || K % group_size || n_groups != K / group_size ||
        (coop && (N < 16u || K % 64u || group_size % 2u)) ||
        (!coop && (K % 8u || group_size % 8u))) {
        set_err(err, err_len, coop ? "CPU VM unsupported Q4 cooperative shape"
                                   : "CPU VM unsupported Q4 GEMV shape");
        return -1;
    }
    if (!qdata || !params || x_len < 0) {
        set_err(err, err_len, "CPU VM Q4 cooperative slot is missing");
        return -1;
    }
    const uint32_t row_bytes = K / 2u;
    const uint32_t scale_base = (N * row_bytes + 3u) / 4u;
    const uint32_t zero_base = scale_base + N * n_groups;
    if (row_end > M) row_end = M;
    for (uint32_t row = row_begin; row < row_end; ++row) {
        for (uint32_t col = 0; col < N; ++col) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < K; ++k) {
                const uint32_t byte_idx = col * row_bytes + (k >> 1u);
                const uint32_t grp = col * n_groups + k / group_size;
                const uint32_t scale_idx = scale_base + grp, zero_idx = zero_base + grp;
                const uint32_t x_idx = row * K + k;
                if (byte_idx >= (uint32_t)q_len || scale_idx >= (uint32_t)params_len ||
                    zero_idx >= (uint32_t)params_len || x_idx >= (uint32_t)x_len) {
                    set_err(err, err_len, "CPU VM Q4 cooperative input out of range");
                    return -1;
                }
                const uint32_t q = ((uint32_t)qdata[byte_idx] >> ((k & 1u) * 4u)) & 15u;
                const float w = ((float)q - params[zero_idx]) * params[scale_idx];
                sum = fmaf(x[x_idx], w, sum);
            }
            const int64_t o = (int64_t)row * N + col;
            if (o >= out_len) {
                if (err && err_len > 0)
                    snprintf(err, (size_t)err_len, "CPU VM q4_coop_store out of range: %lld",
                             (long long)o);
                return -1;
            }
            out[o] = sum;
        }
    }
    return 0;
}

/* One FP4-KM output: per group g the scale lut[16 + scale byte], then 16 fmaf over the low
 * nibbles (elements j) and 16 over the high nibbles (elements j + 16): cpu_vm.c:611-618 (and the
 * identical legacy loop 527-534). */
static float fp4km_dot(const uint8_t* qdata, uint64_t scale_base, const float* fp4,
                       const float* xr, uint32_t K, uint32_t col) {
    const uint64_t row_bytes = K / 2u, n_groups = K / 32u;
    const float* scales = fp4 + 16;
    float sum = 0.0f;
    for (uint64_t g = 0; g < n_groups; ++g) {
        const float scale = scales[qdata[scale_base + (uint64_t)col * n_groups + g]];
        const uint8_t* bytes = qdata + (uint64_t)col * row_bytes + g * 16u;
        const float* xg = xr + g * 32u;
        for (uint32_t j = 0; j < 16u; ++j) sum = fmaf(xg[j], fp4[bytes[j] & 15u] * scale, sum);
        for (uint32_t j = 0; j < 16u; ++j) sum = fmaf(xg[16u + j], fp4[bytes[j] >> 4] * scale, sum);
    }
    return sum;
}

/* Legacy OP_FP4_COOP_GEMM, cpu_vm.c:483-540: scale bytes right after the nibbles, the table at
 * float (nibbles + scale bytes + 3) / 4 of the same blob (504-506). */
int orc_fp4_coop_gemm(uint32_t M, uint32_t K, uint32_t N, uint32_t group_size, uint32_t n_groups,
                      const uint8_t* qdata, int64_t q_len, const float* params, int64_t params_len,
                      const float* x, int64_t x_len, float* out, int64_t out_len,
                      char* err, int err_len) {
    if (err && err_len > 0) err[0] = '\0';
    if (!M || !K || K % 64u || N < 16u || group_size != 32u || n_groups != K / 32u) {
        set_err(err, err_len, "CPU VM unsupported FP4 cooperative shape");
        return -1;
    }
    if (!qdata || !params) {
        set_err(err, err_len, "CPU VM FP4 cooperative slot is missing");
        return -1;
    }
    const uint64_t row_bytes = K / 2u;
    const uint64_t scale_bytes = (uint64_t)N * row_bytes;
    const uint64_t lut_base = (scale_bytes + (uint64_t)N * n_groups + 3u) / 4u;
    if ((int64_t)(scale_bytes + (uint64_t)N * n_groups) > q_len ||
        (int64_t)(lut_base + 272u) > params_len || (int64_t)M * (int64_t)K > x_len) {
        set_err(err, err_len, "CPU VM FP4 cooperative input out of range");
        return -1;
    }
    for (uint32_t row = 0; row < M; ++row) {
        for (uint32_t col = 0; col < N; ++col) {
            const int64_t o = (int64_t)row * N + col;
            if (o >= out_len) {
                if (err && err_len > 0)
                    snprintf(err, (size_t)err_len, "CPU VM fp4_coop_store out of range: %lld",
                             (long long)o);
                return -1;
            }
            out[o] = fp4km_dot(qdata, scale_bytes, params + lut_base, x + (uint64_t)row * K, K, col);
        }
    }
    return 0;
}

/* OP_TILE_GEMM, cpu_vm.c:541-628 (format check 546-549, FP16 550-582, FP4-KM 583-628). */
int orc_tile_gemm(uint32_t format, uint32_t M, uint32_t K, uint32_t N, uint64_t scale_base,
                  uint64_t lut_base, const uint8_t* packed, int64_t packed_len,
                  const float* lut, int64_t lut_len, const float* x, int64_t x_len,
                  float* out, int64_t out_len, uint32_t row_begin, uint32_t row_end,
                  char* err, int err_len) {
    if (err && err_len > 0) err[0] = '\0';
    if (format > 1u || !K || K % 32u || !N) {
        if (err && err_len > 0)
            snprintf(err, (size_t)err_len, "CPU VM unsupported tile GEMM (format %u K %u N %u)",
                     format, K, N);
        return -1;
    }
    if (format == 1u) {
        if (!packed || x_len < 0) {
            set_err(err, err_len, "CPU VM tile GEMM slot is missing");
            return -1;
        }
        if (M == 0) M = (uint32_t)(x_len / (int64_t)K);
        if ((int64_t)N * (int64_t)K * 2 > packed_len || (int64_t)M * (int64_t)K > x_len) {
            set_err(err, err_len, "CPU VM tile GEMM input out of range");
            return -1;
        }
        if (row_end > M) row_end = M;
        for (uint32_t row = row_begin; row < row_end; ++row) {
            for (uint32_t col = 0; col < N; ++col) {
                const uint8_t* w = packed + (uint64_t)col * K * 2u;
                const float* xr = x + (uint64_t)row * K;
                float sum = 0.0f;
                for (uint32_t k = 0; k < K; ++k) {
                    const uint16_t h = (uint16_t)(w[2u * k] | ((uint16_t)w[2u * k + 1u] << 8));
                    sum = fmaf(xr[k], orc_half_to_float(h), sum);
                }
                const int64_t o = (int64_t)row * N + col;
                if (o >= out_len) {
                    if (err && err_len > 0)
                        snprintf(err, (size_t)err_len,
                                 "CPU VM tile_gemm_store out of range: %lld", (long long)o);
                    return -1;
                }
                out[o] = sum;
            }
        }
        return 0;
    }
    if (!packed || !lut || x_len < 0) {
        set_err(err, err_len, "CPU VM tile GEMM slot is missing");
        return -1;
    }
    if (M == 0) M = (uint32_t)(x_len / (int64_t)K);
    const uint64_t row_bytes = K / 2u, n_groups = K / 32u;
    if ((int64_t)(N * row_bytes) > packed_len ||
        (int64_t)(scale_base + (uint64_t)N * n_groups) > packed_len ||
        (int64_t)(lut_base + 272u) > lut_len || (int64_t)M * (int64_t)K > x_len) {
        set_err(err, err_len, "CPU VM tile GEMM input out of range");
        return -1;
    }
    if (row_end > M) row_end = M;
    for (uint32_t row = row_begin; row < row_end; ++row) {
        for (uint32_t col = 0; col < N; ++col) {
            const int64_t o = (int64_t)row * N + col;
            if (o >= out_len) {
                if (err && err_len > 0)
                    snprintf(err, (size_t)err_len, "CPU VM tile_gemm_store out of range: %lld",
                             (long long)o);
                return -1;
            }
            out[o] = fp4km_dot(packed, scale_base, lut + lut_base, x + (uint64_t)row * K, K, col);
        }
    }
    return 0;
}

/* tile_gemm.nim:663-677: the low element then the high element of each byte, unfused. */
void orc_tile_gemm_reference(const float* x, const uint8_t* packed, const float* table,
                             int rows, int K, int N, int64_t scale_base, int64_t lut_base,
                             float* out) {
    const int groups = K / 32;
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < N; ++c) {
            float sum = 0.0f;
            for (int g = 0; g < groups; ++g) {
                const float scale = table[lut_base + 16 + packed[scale_base + (int64_t)c * groups + g]];
                for (int j = 0; j < 16; ++j) {
                    const uint8_t b = packed[(int64_t)c * (K / 2) + g * 16 + j];
                    const float lo = table[lut_base + (b & 15)] * scale;
                    const float hi = table[lut_base + (b >> 4)] * scale;
                    sum += x[(int64_t)r * K + g * 32 + j] * lo;
                    sum += x[(int64_t)r * K + g * 32 + 16 + j] * hi;
                }
            }
            out[(int64_t)r * N + c] = sum;
        }
    }
}

/* cpu_kernels_impl.inc:293-319. */
void orc_matmul_q4(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                   float* c, int M, int K, int N, int group_size, int groups_per_row,
                   int row_begin, int row_end) {
    if (M <= 0 || K <= 0 || N <= 0) return;
    const int bytes_per_row = (K + 1) / 2;
    if (row_end > M) row_end = M;
    for (int m = row_begin; m < row_end; ++m) {
        const float* arow = a + (size_t)m * K;
        for (int n = 0; n < N; ++n) {
            const uint8_t* wrow = wq + (size_t)n * bytes_per_row;
            const int rg = n * groups_per_row;
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) {
                const int g = group_size > 0 ? k / group_size : 0;
                const float sc = scales[rg + g], zp = zeros[rg + g];
                const uint8_t byte = wrow[k >> 1];
                const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0F);
                sum += arow[k] * ((float)nib - zp) * sc;
            }
            c[(size_t)m * N + n] = sum;
        }
    }
}

/* sessionMatmulQ4Fused (gpubackend.nim:3185-3231), shader q4_autotune.nim:194-330. */
static float fused_row_dot(const float* x, const uint8_t* wq, const float* scales, const float* zeros,
                           int row, int K, int group_size, int groups_per_row) {
    const uint8_t* wrow = wq + (size_t)row * (size_t)((K + 1) / 2);
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) {
        const int gi = row * groups_per_row + (group_size > 0 ? k / group_size : 0);
        const uint8_t byte = wrow[k >> 1];
        const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0F);
        const float w = ((float)nib - zeros[gi]) * scales[gi];
        acc = fmaf(w, x[k], acc);
    }
    return acc;
}

int orc_q4_fused(int mode, int n_mats, const float* a, int K, int group_size, int groups_per_row,
                 const uint8_t* const* wq, const float* const* scales, const float* const* zeros,
                 const int* N, float* const* out, const float* residual, const float* gamma,
                 float eps) {
    if (n_mats < 1 || n_mats > 3 || (mode == 1 && n_mats != 2) || (mode != 0 && mode != 1))
        return -1;
    float* x = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
    if (!x) return -1;
    float ssq = 0.0f;
    for (int k = 0; k < K; ++k) {
        if (gamma) {
            ssq = fmaf(a[k], a[k], ssq);
            x[k] = a[k] * gamma[k];
        } else {
            x[k] = a[k];
        }
    }
    const float inv = gamma ? 1.0f / sqrtf(ssq / (float)K + eps) : 1.0f;
    if (mode == 0) {
        for (int i = 0; i < n_mats; ++i)
            for (int row = 0; row < N[i]; ++row) {
                float v = fused_row_dot(x, wq[i], scales[i], zeros[i], row, K, group_size,
                                        groups_per_row) * inv;
                if (residual) v += residual[row];
                out[i][row] = v;
            }
    } else {
        for (int row = 0; row < N[0]; ++row) {
            const float g = fused_row_dot(x, wq[0], scales[0], zeros[0], row, K, group_size,
                                          groups_per_row) * inv;
            const float u = fused_row_dot(x, wq[1], scales[1], zeros[1], row, K, group_size,
                                          groups_per_row) * inv;
            float v = g / (1.0f + expf(-g)) * u;
            if (residual) v += residual[row];
            out[0][row] = v;
        }
    }
    free(x);
    return 0;
}

/* gpubackend.nim:288-311. */
void orc_matmul_q4_ref(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                       float* c, int M, int K, int N, int group_size, int groups_per_row) {
    const int bytes_per_row = (K + 1) / 2;
    for (int m = 0; m < M; ++m) {
        for (int n = 0; n < N; ++n) {
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) {
                const int g = group_size > 0 ? k / group_size : 0;
                const float sc = scales[n * groups_per_row + g], zp = zeros[n * groups_per_row + g];
                const uint8_t b = wq[(size_t)n * bytes_per_row + (k >> 1)];
                const uint8_t nib = (k & 1) == 0 ? (uint8_t)(b & 0x0F) : (uint8_t)((b >> 4) & 0x0F);
                const float wval = ((float)nib - zp) * sc;
                sum += a[(size_t)m * K + k] * wval;
            }
            c[(size_t)m * N + n] = sum;
        }
    }
}

static int tile_op_is_noop(uint32_t op) {
    return op == ORC_OP_NOP || op == ORC_OP_BARRIER_TG || (op >= ORC_OP_TILE_ZERO && op <= ORC_OP_TILE_LOAD_B_F16);
}

/* nimf_cpu_vm_run_slots (cpu_vm.c:178) for shape-op programs: argument checks 181-185, the shape
 * op on lane 0 of threadgroup 0 (420-628; the slot bases are 0 because no OP_BASE_* precedes the
 * header), the trailing tile ops as no-ops (629-631). */
int orc_run_shape_program(const uint32_t* code, int n_words, float* mem, int mem_len,
                          const uint8_t* packed, int packed_len, const float* lut, int lut_len,
                          const float* in_f32, int in_len, char* err, int err_len) {
    if (err && err_len > 0) err[0] = '\0';
    if (!code || n_words <= 0 || !mem || mem_len <= 0) {
        set_err(err, err_len, "invalid CPU VM arguments");
        return -1;
    }
    const float* x = in_f32 ? in_f32 : mem;
    const int64_t x_len = in_f32 ? in_len : mem_len;
    const uint32_t w0 = code[0], op = w0 & 0xFFu;
    const uint32_t fmt = ((w0 >> 8) & 0x1Fu) | (((w0 >> 23) & 0x7u) << 5);
    int rc = 0;
    if (op == ORC_OP_Q4_GEMV || op == ORC_OP_Q4_COOP_GEMM || op == ORC_OP_FP4_COOP_GEMM ||
        op == ORC_OP_TILE_GEMM) {
        if (n_words < 6) {
            set_err(err, err_len, op == ORC_OP_TILE_GEMM ? "CPU VM truncated tile GEMM header"
                                  : op == ORC_OP_FP4_COOP_GEMM ? "CPU VM truncated FP4 shape op"
                                                               : "CPU VM truncated Q4 shape op");
            return -1;
        }
        if (op == ORC_OP_TILE_GEMM)
            rc = orc_tile_gemm(fmt, code[1], code[2], code[3], code[4], code[5], packed, packed_len,
                               lut, lut_len, x, x_len, mem, mem_len, 0u, UINT32_MAX, err, err_len);
        else if (op == ORC_OP_FP4_COOP_GEMM)
            rc = orc_fp4_coop_gemm(code[1], code[2], code[3], code[4], code[5], packed, packed_len,
                                   lut, lut_len, x, x_len, mem, mem_len, err, err_len);
        else
            rc = orc_q4_shape_op(op == ORC_OP_Q4_COOP_GEMM, code[1], code[2], code[3], code[4],
                                 code[5], packed, packed_len, lut, lut_len, x, x_len, mem, mem_len,
                                 0u, code[1], err, err_len);
        if (rc != 0) return rc;
    } else {
        set_err(err, err_len, "oracle runs shape-op programs only");
        return -1;
    }
    for (int pc = 6; pc < n_words; ++pc) {
        const uint32_t o = code[pc] & 0xFFu;
        if (o == ORC_OP_HALT) return 0;
        if (!tile_op_is_noop(o)) {
            if (err && err_len > 0)
                snprintf(err, (size_t)err_len, "oracle: op 0x%02x after a shape op", o);
            return -1;
        }
    }
    return 0;
}

void orc_unpack_q4(const uint8_t* wq, int K, int N, uint8_t* codes) {
    const int bytes_per_row = (K + 1) / 2;
    for (int n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k) {
            const uint8_t b = wq[(size_t)n * bytes_per_row + (k >> 1)];
            codes[(size_t)n * K + k] = (k & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
        }
}

void orc_unpack_fp4km(const uint8_t* packed, int64_t scale_base, int K, int N, uint8_t* codes,
                      uint8_t* scale_bytes) {
    const int groups = K / 32;
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < groups; ++g) {
            const uint8_t* b = packed + (size_t)n * (K / 2) + (size_t)g * 16;
            for (int j = 0; j < 16; ++j) {
                codes[(size_t)n * K + g * 32 + j] = b[j] & 15;
                codes[(size_t)n * K + g * 32 + 16 + j] = b[j] >> 4;
            }
            scale_bytes[(size_t)n * groups + g] = packed[scale_base + (int64_t)n * groups + g];
        }
}

/* t_fp4_tile_gemm.nim:30-33. */
uint32_t orc_xorshift32(uint32_t* s) {
    uint32_t v = *s;
    v ^= v << 13;
    v ^= v >> 17;
    v ^= v << 5;
    *s = v;
    return v;
}

/* t_fp4_tile_gemm.nim:35-44. */
void orc_make_fp4_case(uint32_t* state, int M, int K, int N, float* x, uint8_t* packed,
                       float* table) {
    static const float fp4[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                  -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
    for (int i = 0; i < M * K; ++i)
        x[i] = (float)((int)(orc_xorshift32(state) % 2001u) - 1000) / 1000.0f;
    const int nbytes = N * (K / 2) + N * (K / 32);
    for (int i = 0; i < nbytes; ++i) packed[i] = (uint8_t)(orc_xorshift32(state) & 255u);
    for (int i = 0; i < 16; ++i) table[i] = fp4[i];
    for (int i = 0; i < 256; ++i) table[16 + i] = (float)(1 + (i % 13)) / 64.0f;
}

/* t_fp4_tile_gemm.nim:210-223 (halfBits 198-208 for exact halves). */
void orc_make_f16_case(uint32_t* state, int M, int K, int N, float* x, float* w,
                       uint8_t* halves) {
    for (int i = 0; i < M * K; ++i)
        x[i] = (float)((int)(orc_xorshift32(state) % 2001u) - 1000) / 1000.0f;
    for (int i = 0; i < N * K; ++i)
        w[i] = (float)((int)(orc_xorshift32(state) % 2001u) - 1000) / 1024.0f;
    for (int i = 0; i < N * K; ++i) {
        const uint16_t h = orc_float_to_half(w[i]);
        halves[2 * i] = (uint8_t)(h & 255u);
        halves[2 * i + 1] = (uint8_t)(h >> 8);
    }
}
