// byhip_internal.h - shared declarations of libbybyhip.so (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "byhip.h"

namespace byhip {

// A failure that the C ABI reports as BYHIP_ERROR with its message.
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};
// A shape or device the entry point does not handle: reported as BYHIP_UNSUPPORTED, the "false"
// of the reference's encoders.
struct Unsupported : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
[[noreturn]] void unsupported(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void check_hip(hipError_t e, const char* what, const char* file, int line);
#define BYHIP_HIP(call) ::byhip::check_hip((call), #call, __FILE__, __LINE__)
// Checks the launch just queued (invalid configuration and the like).
#define BYHIP_LAUNCHED(name) ::byhip::check_hip(hipGetLastError(), name, __FILE__, __LINE__)

void set_error(const std::string& msg);

hipStream_t stream();

// A kernel launch kept with its arguments by value, run on the stream it is given.
using Relaunch = std::function<void(hipStream_t)>;
// Whether the open session is recorded for direct replay: its launches are then kept (keep_launch)
// instead of queued, run in order when the session ends, and run again at every replay.
bool keeping_launches();
void keep_launch(Relaunch l);

template <typename... P, std::size_t... I>
void launch_tuple(const char* name, void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t s,
                  std::tuple<P...>& t, std::index_sequence<I...>) {
    void* argv[sizeof...(P) + 1] = {static_cast<void*>(&std::get<I>(t))..., nullptr};
    check_hip(hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, (unsigned)lds, s), name,
              __FILE__, __LINE__);
}

// Every kernel of the library is launched through here: on the library stream now, or, inside a
// session recorded for direct replay, kept for the recording's launches.
template <typename... P, typename... A>
void launch(const char* name, void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, A&&... args) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    std::tuple<P...> t(static_cast<P>(std::forward<A>(args))...);
    if (keeping_launches()) {
        keep_launch([=](hipStream_t s) mutable {
            launch_tuple(name, kernel, grid, block, lds, s, t, std::index_sequence_for<P...>{});
        });
        return;
    }
    launch_tuple(name, kernel, grid, block, lds, stream(), t, std::index_sequence_for<P...>{});
}

// Every entry point: injected fault first, then the device must be initialised.
void enter_compute();
// Entry points that wait for the device or write memory outside a kernel call this first: they
// cannot be part of a recorded session (stream capture).
void no_host_sync(const char* what);
hipStream_t stream();
int compute_units();
// Device scratch for kernels that need it (split-K partial sums), allocated once at init so that
// no GEMM call allocates (calls may be captured into a recording). Work queued on the library
// stream uses it in stream order.
constexpr size_t kWorkspaceBytes = 32u << 20;
void* workspace();
// Takes the device address of byhip_q4_matmul_static's scratch array on `device` (current).
void static_scratch_setup(int device);
// Whether a session (or a recording) is open.
bool session_open();
// Properties of the initialised device.
const hipDeviceProp_t& device_props();

// Allocation registry of buffers the library handed out: byte size (0 = not ours) and, for small
// host uploads, a host copy (decode tables are classified on the host without a device read).
size_t alloc_bytes(const void* p);
const std::vector<uint8_t>* host_mirror(const void* p);
void* device_alloc(size_t bytes);
void device_free(void* p);
// Bounds check of a device pointer the library allocated: [p, p + need) inside its allocation.
void check_span(const void* p, size_t need, const char* what);
// Reads `bytes` at `p` to the host, from the mirror when there is one, else with a stream wait.
void read_small(const void* p, size_t off, void* dst, size_t bytes);
// The same, but returns false instead of waiting when there is no host copy and a session is being
// recorded (a recording cannot wait for the device).
bool try_read_small(const void* p, size_t off, void* dst, size_t bytes);
// Reads from the host copy only (false when there is none): no device access, no wait.
bool mirror_read(const void* p, size_t off, void* dst, size_t bytes);
// A kernel of the library writes the buffer holding p: its host copy no longer holds its contents.
void note_device_write(const void* p);
// Whether a session is being recorded (graph capture or kept launches).
bool session_recording();
// A small device array of the library (64 ints), for flags that one kernel writes and later
// kernels on the stream read (the FP4-KM route's table classification).
int* device_flags();

template <class F>
int guard(F&& f) {
    try {
        f();
        return BYHIP_OK;
    } catch (const Unsupported& e) {
        set_error(e.what());
        return BYHIP_UNSUPPORTED;
    } catch (const std::exception& e) {
        set_error(e.what());
        return BYHIP_ERROR;
    } catch (...) {
        set_error("byhip: unknown exception");
        return BYHIP_ERROR;
    }
}

// Integer value of environment variable `name` (tuning overrides), or dflt when unset or empty.
inline int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    return (s && *s) ? atoi(s) : dflt;
}

inline size_t dtype_bytes(int dt) {
    switch (dt) {
    case BYHIP_F32: return 4;
    case BYHIP_F16: case BYHIP_BF16: return 2;
    default: return 0;
    }
}

}  // namespace byhip

// byhip_q4w: resident Q4 weights in the device layout.
struct byhip_q4w {
    int K, N, group, gpr;       // group 0: one group per row (cpu_kernels_impl.inc:309)
    size_t row_bytes;           // (K + 1) / 2
    uint8_t* wq;                // nibble rows [N, row_bytes], from byte 0
    void* scales;               // [N * gpr], fp16 when scale_f16 else fp32
    float* zeros;               // [N * gpr] fp32, or null when zero_uniform
    int scale_f16;
    int zero_uniform;
    float zero_value;
    size_t bytes;               // device bytes held
    // Decode copy of the scales (and non-uniform zeros) per 32-value chunk in blocks of 8 rows,
    // [ceil(N/8)][K/32][8] (fp16 scales when scale_f16, fp32 zeros), so one 16-byte load gives a
    // lane the scales of 8 consecutive rows. Present when K and the group are multiples of 32
    // (or the group is 0); null otherwise.
    void* sblk = nullptr;
    float* zblk = nullptr;
    int blk_scale_f16 = 0;
    // Every (q - z) * s lies in fp16's normal range (or is 0), so the fp16 MFMA kernels may take
    // these weights (rounding each product once); else the exact fp32 route runs them. Weights
    // built from micro-VM slots are not classified (0).
    int f16_safe = 0;
    // Prefill copy, in the order the wide prefill kernel's lanes load it, built when the weights
    // are fp16-safe with fp16 scales, one uniform zero, K % 64 == 0 and groups of a multiple of 32
    // (or one per row); null otherwise. Per 16-column fragment f and 64-value K sub-step u, 512
    // contiguous bytes: lane l = c + 16 g holds column 16 f + c, K positions 64 u + 16 g .. + 15 as
    // two words, each holding positions 0..7 of its 8 as nibbles (0, 2, 4, 6, 1, 3, 5, 7) from bit 0,
    // so that one AND-OR against the fp16 exponent words yields them in natural order. Scales: per
    // 64 columns and sub-step, [2][16][4] fp16: the scales of columns 16 j + c (j = 0..3) for K
    // positions 64 u + 32 t (t = g / 2), 8 bytes per lane.
    uint8_t* wpf = nullptr;     // [ceil(N/16)][K/64][64][8]
    void* spf = nullptr;        // [ceil(N/64)][K/64][2][16][4] fp16
};
