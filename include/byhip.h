/* byhip.h - C ABI of the MI355X (gfx950) backend for BybyLang's quantized tile-GEMM path.
 *
 * libbybyhip.so is the drop-in boundary that a `backends/hip/hip_backend.nim` binds with
 * `importc, cdecl`, the way backends/cpu/cpu_backend.nim:22-26,102-160 binds the CPU C code. Every
 * entry point names the reference interface it replaces (file:line in bobbyshop-vui/bybylang).
 *
 * Conventions (mirroring the reference's native shims):
 *  - Return value: BYHIP_OK (0) on success. BYHIP_UNSUPPORTED (1) is the "false" an encoder
 *    returns for a shape or device it does not handle, after which the caller may take another
 *    route (gpubackend.nim:1444-1445). BYHIP_ERROR (-1) is a failure; byhip_last_error() gives
 *    the message, as nimf_cpu_vm_run_slots fills err/err_len (backends/cpu/cpu_vm.c:178-188).
 *    The library never computes on the CPU: a failure is returned, and the caller's policy
 *    (handleGpuFailure, gpubackend.nim:80-105) decides between raising and its own fallback.
 *  - Memory: device pointers and byte or element counts; no framework types. Work is queued on
 *    the library's stream for the current device and runs asynchronously; results are valid after
 *    byhip_session_end() or byhip_synchronize().
 *  - One host thread drives a session at a time (the reference's global session state,
 *    backends/vulkan/vulkan_driver.nim:1668).
 */
#ifndef BYHIP_H
#define BYHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BYHIP_OK 0
#define BYHIP_UNSUPPORTED 1
#define BYHIP_ERROR (-1)

/* Element types of activations and outputs (the reference's session path is fp32 in and out). */
enum byhip_dtype {
    BYHIP_F32 = 0,
    BYHIP_F16 = 1,
    BYHIP_BF16 = 2,
    /* Activations in the FP4-KM packing of the weights: E2M1 nibbles [M, K/2] (byte j of a
     * 32-value group holds element j low and j + 16 high, session_vm.nim:384-388) followed by one
     * E8M0 scale byte per group [M, K/32]. Only byhip_mxfp4_gemm and byhip_fp4km_tile_gemm read
     * it. */
    BYHIP_MXFP4_KM = 3
};

typedef struct byhip_device_info {
    int device;
    int compute_units;
    int wavefront_size;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    size_t total_global_mem;
    size_t lds_bytes_per_block;
    char arch_name[64];
    char name[128];
} byhip_device_info;

/* ── Lifecycle and errors ─────────────────────────────────────────────────────────────────── */

/* Selects and initialises `device` (creates the library stream). Replaces the backends'
 * ensureInit / ensureGpuInit (gpubackend.nim detectBackend 131-141; the device ordinal follows
 * BYBY_VULKAN_DEVICE, distributed.nim:144-145, as BYBY_HIP_DEVICE). Idempotent. */
int byhip_init(int device);
int byhip_device_info_get(byhip_device_info* out);
/* Thread-local text of the last failure; "" when none. Backs sessionGetLastError
 * (gpubackend.nim:2647-2667). */
const char* byhip_last_error(void);
void byhip_clear_error(void);
/* The next `count` compute or session entry points fail with "byhip: injected fault" before
 * touching the device, so the host can exercise failure handling (handleGpuFailure,
 * gpubackend.nim:80-105) without a GPU fault. */
void byhip_fault_inject(int count);
int byhip_version(void);

/* ── Device memory ────────────────────────────────────────────────────────────────────────── */

int byhip_alloc(size_t bytes, void** dptr);
int byhip_free(void* dptr);
/* Host -> device copy of `bytes` at byte `dst_off`; stream-ordered. */
int byhip_upload(void* dptr, size_t dst_off, const void* src, size_t bytes);
/* Device -> host copy; waits for the stream first (a read is valid only after the session's
 * work, gpubackend.nim:2669). */
int byhip_read(const void* dptr, size_t src_off, void* dst, size_t bytes);
int byhip_memset(void* dptr, int value, size_t bytes);
int byhip_synchronize(void);
/* The library stream (hipStream_t) of the current device, for callers that time or order their
 * own work against it. */
void* byhip_stream(void);

/* ── Session (gpubackend.nim:894-903 SessionHandle and its lifecycle) ─────────────────────── */

/* sessionBegin (gpubackend.nim:1042): fails if a session is already open
 * (vulkan_driver.nim:1668). */
int byhip_session_begin(void);
/* sessionUpload (gpubackend.nim:1133): a new device buffer holding `n` floats. */
int byhip_session_upload(const float* data, size_t n, void** out);
/* Byte variant (vulkanSessionUploadBytesPrivate, vulkan_driver.nim:2146). */
int byhip_session_upload_bytes(const void* data, size_t bytes, void** out);
/* sessionAllocScratch (gpubackend.nim:1295): `n` floats, zero-filled. */
int byhip_session_alloc_scratch(size_t n, void** out);
/* sessionEnd (gpubackend.nim:2422): waits for the queued work and reports device errors;
 * deferred frees run here (vulkan_driver.nim:1817-1819). */
int byhip_session_end(void);
/* sessionCommitContinue (gpubackend.nim:2444-2467): no wait; the session stays open. */
int byhip_session_commit_continue(void);
/* sessionRecoverQueue (gpubackend.nim:2593): drops an open session after a failed end. */
int byhip_session_recover(void);
/* sessionRead (gpubackend.nim:2669): `n` floats from a session buffer. */
int byhip_session_read(const void* h, float* dst, size_t n);
/* sessionFree (gpubackend.nim:2694): deferred to the end of an open session. */
int byhip_session_free(void* h);
/* sessionGpuSeconds / sessionSetGpuTiming (gpubackend.nim:2617-2632): hipEvent time between
 * begin and end of the timed sessions since the last reset. */
int byhip_session_set_gpu_timing(int on);
double byhip_session_gpu_seconds(void);

/* Record / replay as HIP graphs (gpubackend.nim:2502-2552, vulkan_driver.nim:1659-2030).
 * sessionCanRecord: always 1 on this backend. */
int byhip_session_can_record(void);
/* sessionBeginRecording: opens a session whose queued work is captured; it must be
 * self-contained (entry points that wait for the device, upload or clear memory fail while
 * recording). byhip_session_end() keeps it as a graph, runs it once and waits. */
int byhip_session_begin_recording(void);
/* sessionLastRecording: id kept by the last byhip_session_end(), or -1. */
int byhip_session_last_recording(void);
/* sessionReplay: launches recording `id` `times` times back to back (outside a session), then
 * waits; counted by byhip_session_gpu_seconds() when timing is on. */
int byhip_session_replay(int id, int times);
/* A measurement form of sessionReplay with no counterpart in the reference: launches recording
 * `pre_id` `pre_times` times (untimed), then recording `id` `times` times right behind it, and
 * counts only the latter in byhip_session_gpu_seconds(). All launches are queued before the one
 * wait, so the timed events never include the host's launch latency. */
int byhip_session_replay_after(int pre_id, int pre_times, int id, int times);
/* Measurement marks, with no counterpart in the reference: byhip_session_mark(0) and (1) launch
 * (or, inside a recording, record) a one-thread kernel that stores the GPU's constant-rate
 * realtime counter into the library's begin and end slots. byhip_session_replay_marked(id)
 * launches a recording holding both marks once, waits, and counts the time between the two
 * stores in byhip_session_gpu_seconds() (timing on). Outside recordings and sessions, mark(0)
 * clears the slots before its kernel, and byhip_session_take_marks() waits for the stream and
 * counts the same interval for directly launched work. The slots are the library's: one marked
 * interval at a time. */
int byhip_session_mark(int which);
int byhip_session_replay_marked(int id);
int byhip_session_take_marks(void);
/* sessionFreeRecording. */
int byhip_session_free_recording(int id);
/* A measurement switch with no counterpart in the reference: recordings begun while it is on keep
 * their kernel launches (kernel, launch shape and arguments by value) instead of capturing a HIP
 * graph; ending one launches them in order, and every replay launches them again, directly on the
 * library stream. Same results as the graph form; it exists so that profilers which trace direct
 * dispatches see exactly the replayed kernels (off by default). */
int byhip_session_set_direct_replay(int on);

/* ── Q4 block-dequant GEMV / GEMM ─────────────────────────────────────────────────────────── */

/* Resident Q4 weights: the ResidentWeightHandle of gpubackend.nim:2813-2825. */
typedef struct byhip_q4w byhip_q4w;

typedef struct byhip_q4w_info {
    int K, N, group_size, groups_per_row;
    int scale_is_f16;   /* scales held as fp16 (every scale was exactly representable) */
    int zero_uniform;   /* one zero point for every group (its value in zero_value) */
    float zero_value;
    size_t device_bytes;
    /* every (q - zero) * scale lies in fp16's normal range (or is 0): the fp16 MFMA kernels may
     * take these weights at M > 8; otherwise the exact fp32 GEMM does */
    int f16_safe;
} byhip_q4w_info;

/* residentUploadQ4 (gpubackend.nim:2883-2919) and residentUploadQ4Mapped (2961-2998): host wq
 * (`wq_bytes` bytes, the packed rows [N, (K+1)/2] start at byte `wq_off`; even k in the low
 * nibble), scales and zeros fp32 [N * groups_per_row]. The weights are copied once into the device
 * layout (fp16 scales when exact, one zero when uniform). group_size 0 means one group per row,
 * as in cpu_kernels_impl.inc:309. */
int byhip_q4_resident_upload(const uint8_t* wq, size_t wq_bytes, size_t wq_off,
                             const float* scales, const float* zeros, int K, int N,
                             int group_size, int groups_per_row, byhip_q4w** out);
/* The same from device-resident fp32 scale/zero arrays and nibble rows (e.g. session buffers). */
int byhip_q4_resident_from_device(const void* d_wq, size_t wq_off, const void* d_scales,
                                  const void* d_zeros, int K, int N, int group_size,
                                  int groups_per_row, byhip_q4w** out);
/* residentFreeQ4 (gpubackend.nim:3233-3253). */
int byhip_q4_resident_free(byhip_q4w* w);
int byhip_q4_resident_info(const byhip_q4w* w, byhip_q4w_info* out);

/* sessionMatmulQ4 (gpubackend.nim:3000-3061): y[M, N] = x[M, K] . W^T on device buffers,
 * computing sum_k x[m,k] * (q[n,k] - zero[n,g]) * scale[n,g] (cpu_kernels_impl.inc:293-319,
 * cpu_vm.c:420-482) with fp32 accumulation. x_dtype: BYHIP_F32 or BYHIP_F16; y_dtype: BYHIP_F32,
 * BYHIP_F16 or BYHIP_BF16. M <= 8 runs the decode GEMV; larger M the fp16 MFMA GEMMs when the
 * weights are fp16-safe (byhip_q4w_info.f16_safe), else the exact fp32 GEMM. fp32 activations
 * keep the reference's fp32 tolerance on every route (1e-4 of max(1, |y|max)); fp16 activations
 * at M > 8 use weights rounded once to fp16. */
int byhip_q4_matmul(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M);

/* No counterpart in the reference: byhip_q4_matmul for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results; tuned plans are not consulted. The kernels' scratch (split-K
 * partial sums, per-row shifts of fp32 activations) is a 16 MiB device array inside the library,
 * one per GPU, set up by byhip_init: the call allocates nothing. More than 4,194,304 rows of fp32
 * activations at M > 8 are rejected (BYHIP_ERROR). Calls on one GPU share the array: calls that
 * overlap (other threads or streams) race on it. */
int byhip_q4_matmul_static(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype, int M);

/* residentPrepareQ4 (gpubackend.nim:2871-2880; vulkanPrepareQ4Tuned, q4_autotune.nim:387-543):
 * chooses the kernel byhip_q4_matmul uses for these weights, this M's class (1; 2..32; 33..128;
 * more, tuned at M = 1, 32, 64 and 256) and activation dtype (BYHIP_F32 is the reference's session
 * dtype).
 * Every candidate runs once on deterministic input and must match the exact per-element kernel
 * within 1e-4 of the output's magnitude (3e-3 for kernels that round weights to fp16 for the MFMA)
 * with finite outputs; the survivors are timed and the fastest by at least 3% is kept, in memory
 * and in a plan file under BYHIP_CACHE_DIR (else $XDG_CACHE_HOME/bybylang_amd or
 * ~/.cache/bybylang_amd) keyed by the device and the library's kernel sources, so a later process
 * reuses it (q4_autotune.nim:32-50). Returns BYHIP_UNSUPPORTED when tuning is off
 * (BYHIP_Q4_TUNED=0 or BYHIP_GPU_AUTOTUNE=0) or a session is open, as the reference does. */
int byhip_q4_prepare(const byhip_q4w* w, int M, int x_dtype);
/* The plan in place for these weights, M class and dtype: its name and whether it came from the
 * plan file (1) or was tuned in this process (0); BYHIP_UNSUPPORTED when there is none. */
int byhip_q4_plan_info(const byhip_q4w* w, int M, int x_dtype, char* name, int name_len, int* from_cache);
/* Forgets this process's plans (the plan file stays; the next prepare reads it again). */
int byhip_q4_plans_reset(void);

/* sessionMatmulQ4Fused (gpubackend.nim:3185-3231; its shader, q4_autotune.nim:194-330): the fused
 * decode GEMV, M = 1, on fp32 device buffers.
 *   mode 0: ws[0..n_ws-1] (1..3 resident weights of equal K, group and groups per row) share `a`
 *           (K floats); outs[i] receives ws[i]'s N rows.
 *   mode 1: ws = {gate, up} of equal N; outs[0][row] = silu(gate . x) * (up . x), with
 *           silu(v) = v / (1 + exp(-v)). As in the reference, outs holds an allocated buffer per
 *           weight (n_outs >= 2); only outs[0] is written.
 *   has_norm: `a` is the raw vector; RMSNorm with weights `gamma` (K floats) and `eps` is applied
 *           inside the kernel: x = a * gamma, each dot product times 1 / sqrt(sum a^2 / K + eps).
 *   has_res: res[row] (matrix-local row) is added to each output.
 * Returns BYHIP_UNSUPPORTED, with the outputs untouched, for the combinations the reference's
 * encoders reject (n_ws outside 1..3, n_outs < n_ws, mode 1 without exactly two weights, a missing
 * output, residual or norm buffer) and for weights this kernel does not take (mismatched shapes
 * or scale formats, K % 32 != 0); any K that is a multiple of 32 is taken (long rows in K slices).
 * The caller then runs the unfused sequence, as the reference's callers do. */
int byhip_q4_matmul_fused(int mode, const float* a, byhip_q4w* const* ws, int n_ws, float* const* outs,
                          int n_outs, const float* res, int has_res, const float* gamma, float eps,
                          int has_norm);
/* gpuMatmulQ4 (gpubackend.nim:806-843): host fp32 in, host fp32 out; uploads the weights on every
 * call and waits, like vulkanMatmulQ4 (vulkan_driver.nim:1012-1161). */
int byhip_gpu_matmul_q4(const float* a, const uint8_t* wq, const float* scales, const float* zeros,
                        float* c, int M, int K, int N, int group_size, int groups_per_row);

/* ── FP4-KM tile GEMM and MXFP4 ───────────────────────────────────────────────────────────── */

/* OP_TILE_GEMM format 0 (cpu_vm.c:583-628, tile_gemm.nim:1-26): y[M, N] = x[M, K] . W^T with W
 * the FP4-KM blob in `blob` (nibbles [N, K/2] from byte 0, scale bytes [N, K/32] from byte
 * `scale_base`) and the 272-float decode table at float `lut_base` of `lut` (16 FP4 values, then
 * 256 scale values): weight = lut[nibble] * lut[16 + scale byte]. x_dtype BYHIP_F32 / BYHIP_F16,
 * or BYHIP_MXFP4_KM when the table is exactly E2M1 and 2^(e-127) (then the native scaled MFMA runs;
 * otherwise BYHIP_UNSUPPORTED). `blob_bytes` and `lut_floats` bound the reads as the CPU VM bounds
 * them (cpu_vm.c:600-604). Replaces sessionFp4GemmTensorCore / sessionFp4GemmTiledEnc /
 * sessionFp4GemmMetal (gpubackend.nim:1442-1472). */
int byhip_fp4km_tile_gemm(const void* x, int x_dtype, const uint8_t* blob, size_t blob_bytes,
                          size_t scale_base, const float* lut, size_t lut_floats, size_t lut_base,
                          void* y, int y_dtype, int M, int K, int N);
/* Native MXFP4 GEMM (the FP4 configuration of the benchmark): x and w both in the FP4-KM packing
 * with E8M0 scale bytes (x: nibbles [M, K/2] then scales [M, K/32]; w: nibbles [N, K/2] then scales
 * [N, K/32] at byte N*K/2), E2M1 values, fp32 accumulation, y_dtype F32/F16/BF16. */
int byhip_mxfp4_gemm(const uint8_t* x, const uint8_t* w, void* y, int y_dtype, int M, int K, int N);
/* OP_TILE_GEMM format 1 (cpu_vm.c:550-582): W IEEE halves [N, K]; sessionF16GemmTile
 * (gpubackend.nim:1474-1481). */
int byhip_f16_tile_gemm(const void* x, int x_dtype, const uint16_t* w, size_t w_halves,
                        void* y, int y_dtype, int M, int K, int N);
/* sessionTileGemmReady (gpubackend.nim:1483-1488, vulkanTileGemmReady vulkan_driver.nim:2681-2762):
 * the parity gate on closed-form data whose sums are exact, run once per process and format;
 * returns 1 (passed), 0 (failed) or BYHIP_ERROR. `tensor_core` selects the MFMA route. */
int byhip_tile_gemm_ready(int f16, int tensor_core);

/* ── Micro-VM route (session_vm_dispatch.nim:128-158, slot_layout.nim:11-73) ───────────────── */

/* Runs a shape-op micro-kernel program on the five slots the reference binds (mem, u8, lut,
 * input, u32; slot_layout.nim:23-37): OP_TILE_GEMM (formats 0 and 1), OP_FP4_COOP_GEMM,
 * OP_Q4_GEMV and OP_Q4_COOP_GEMM, decoded with the rules of nimf_cpu_vm_run_slots
 * (cpu_vm.c:420-628) and tileGemmShape (tile_gemm.nim:68-78). Slots are device pointers; lengths
 * are in the reference's units (mem, lut, input: floats; u8: bytes). `rows` > 0 overrides an
 * M = 0 header (a dispatch's row count); with rows = 0, M = 0 means input_len / K. A rejected
 * program returns BYHIP_ERROR with the reference's own message ("CPU VM unsupported tile GEMM
 * (format 0 K 48 N 16)", "CPU VM q4_coop_store out of range: 64", ...), checked in its order, and
 * leaves in `mem` the outputs the reference writes before it stops. The Q4 shape ops run the exact
 * routes (fp32 arithmetic, as in the reference). The program's remaining words may only be tile
 * ops, barriers, NOPs and HALT (else BYHIP_UNSUPPORTED). */
int byhip_program_dispatch(const uint32_t* words, int n_words, void* mem, size_t mem_len,
                           const void* u8, size_t u8_len, const void* lut, size_t lut_len,
                           const void* input, size_t input_len, int rows);

/* ── Debug (bit-exact unpack checks) ──────────────────────────────────────────────────────── */

/* Unpacks resident Q4 weights on the device into host arrays: codes [N*K] (0..15), scales and
 * zeros [N * groups_per_row] as fp32, from the device layout. */
int byhip_debug_unpack_q4(const byhip_q4w* w, uint8_t* codes, float* scales, float* zeros);
/* Unpacks an FP4-KM blob on the device: codes [N*K] in element order (k), decoded weights
 * [N*K] = lut[code] * lut[16 + scale byte] as fp32. */
int byhip_debug_unpack_fp4km(const uint8_t* blob, size_t scale_base, const float* lut,
                             size_t lut_base, int K, int N, uint8_t* codes, float* weights);
/* A plain device copy of `bytes` (16-byte multiples): the reference point for HBM bandwidth and
 * for scaling hardware traffic counters. No counterpart in the reference. */
int byhip_debug_copy(void* dst, const void* src, size_t bytes);
/* A plain streaming read of `bytes` (16-byte multiples; nontemporal 16-byte loads, eight per lane
 * in flight, 16 waves per CU): the reference point for what the kernels' reads can reach. Each
 * wave stores a fold of what it read into `sink`, which must hold 16 * CUs 32-bit words.
 * No counterpart in the reference. */
int byhip_debug_read(const void* src, size_t bytes, void* sink, size_t sink_bytes);
/* The number of device allocations the library has made since the process started (its buffers,
 * resident weights, workspace and internal temporaries): a test checks with it that an entry
 * point allocates nothing. No counterpart in the reference. */
unsigned long long byhip_debug_alloc_count(void);

#ifdef __cplusplus
}
#endif
#endif
