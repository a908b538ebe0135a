/* ref_shim.c - exports three entry points of the reference's CPU backend for the checker.
 *
 * TEST INFRASTRUCTURE ONLY. The reference declares its kernels with hidden visibility
 * (backends/cpu/cpu_kernels.h:16-18, 86, 118), so a shared object built from its sources exports
 * nothing; this file is linked into that same object (oracle/_ref/libbybyref.so) and forwards to
 * the two functions the quantized tile-GEMM path uses, and to the RMSNorm of the unfused sequence
 * that the fused decode GEMV replaces. It contains no arithmetic of its own.
 */
#include "cpu_kernels.h"

#define REFSHIM_EXPORT __attribute__((visibility("default")))

REFSHIM_EXPORT int refshim_vm_run_slots(uint32_t* code, int n_words, float* mem, int mem_len,
                                        const uint8_t* packed, int packed_len, const float* lut,
                                        int lut_len, const float* in_f32, int in_len,
                                        int n_threads, int tg_floats, int tg_size, char* err,
                                        int err_len) {
    return nimf_cpu_vm_run_slots(code, n_words, mem, mem_len, packed, packed_len, lut, lut_len,
                                 in_f32, in_len, n_threads, tg_floats, tg_size, err, err_len);
}

REFSHIM_EXPORT void refshim_matmul_q4(float* a, uint8_t* wq, float* scales, float* zeros, float* c,
                                      int M, int K, int N, int group_size, int groups_per_row) {
    nimf_cpu_matmul_q4(a, wq, scales, zeros, c, M, K, N, group_size, groups_per_row);
}

REFSHIM_EXPORT void refshim_rmsnorm(float* x, float* gamma, float* out, int rows, int cols, float eps) {
    nimf_cpu_rmsnorm(x, gamma, out, rows, cols, eps);
}
