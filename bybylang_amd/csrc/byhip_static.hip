// byhip_static.hip - byhip_q4_matmul_static: the Q4 matmul entry point that allocates nothing.
//
// It computes what byhip_q4_matmul computes, on the same kernels and routes (tuned plans aside),
// for callers that cannot allocate device memory: code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc. The kernels' scratch (split-K partial sums, the per-row
// shifts of fp32 activations) is `scratch`, a file-scope device array of kStaticScratchBytes that
// each GPU holds until the process ends, in place of the library workspace. Its device address is
// taken once per device at byhip_init (hipGetSymbolAddress) and only that address is handed to the
// kernels. Every call on a GPU shares that GPU's array, and every kernel writes the scratch it
// reads before reading it (nothing needs to start at zero); calls that overlap on one GPU (from
// several threads, or other streams) race on it.
#include "byhip_internal.h"
#include "byhip_q4.h"

namespace byhip {
constexpr size_t kStaticScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
}  // namespace byhip

static __device__ __align__(256) unsigned char scratch[byhip::kStaticScratchBytes];

namespace byhip {
namespace {
void* g_scratch[kMaxDevices] = {};  // scratch's device address, per device
}  // namespace

void static_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) fail("byhip: device %d past the static scratch table", device);
    void* p = nullptr;
    BYHIP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail("byhip: the static scratch has no device address");
    g_scratch[device] = p;
}

}  // namespace byhip

using namespace byhip;

extern "C" int byhip_q4_matmul_static(const void* x, int x_dtype, const byhip_q4w* w, void* y, int y_dtype,
                                      int M) {
    return guard([&] {
        enter_compute();
        int device = -1;
        BYHIP_HIP(hipGetDevice(&device));
        void* p = device >= 0 && device < kMaxDevices ? g_scratch[device] : nullptr;
        if (!p) fail("byhip: no static scratch on device %d (call byhip_init first)", device);
        if (!w) fail("byhip: null Q4 weights");
        // fp32 activations at M > 8 keep one 32-bit shift per row in the scratch
        if (x_dtype == BYHIP_F32 && M > 8 && (size_t)M * sizeof(int) > kStaticScratchBytes)
            fail("byhip: byhip_q4_matmul_static takes at most %zu rows of fp32 activations (M=%d)",
                 kStaticScratchBytes / sizeof(int), M);
        note_device_write(y);
        q4_matmul_run_scratch(x, x_dtype, w, y, y_dtype, M, p, kStaticScratchBytes);
    });
}
