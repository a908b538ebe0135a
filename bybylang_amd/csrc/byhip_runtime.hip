// byhip_runtime.hip - device, stream, memory, errors and the session lifecycle of libbybyhip.so.
//
// Mirrors the reference's session semantics (gpubackend.nim:894-903, 1042-2721): one open session
// at a time, uploads into device buffers, work queued on one stream, sessionEnd = wait + error
// check, frees deferred while a session is open, GPU time from events around each session.
#include "byhip_internal.h"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>

namespace byhip {
namespace {

struct Alloc {
    size_t bytes = 0;
    std::vector<uint8_t> mirror;  // host copy of a small upload (<= kMirrorBytes)
};

constexpr size_t kMirrorBytes = 64 * 1024;

struct State {
    std::recursive_mutex mu;
    bool inited = false;
    int device = -1;
    hipStream_t stream = nullptr;
    hipDeviceProp_t prop{};
    std::unordered_map<const void*, Alloc> allocs;
    void* workspace = nullptr;  // kWorkspaceBytes, allocated by byhip_init, kept until exit
    // session
    bool session_open = false;
    std::vector<void*> deferred_frees;
    bool timing = false;
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;
    double gpu_seconds = 0.0;
    double realtime_hz = 0.0;  // rate of the counter the timing marks read
    // record / replay (sessionBeginRecording .. sessionFreeRecording, gpubackend.nim:2502-2552)
    bool recording = false;
    // Recordings made while `direct` is set keep their kernel launches (with their arguments) and
    // replay them by launching them again; the others are HIP graphs.
    bool direct = false;
    bool direct_open = false;          // the open recording keeps its launches
    std::vector<Relaunch> kept;        // launches of the open direct recording
    struct Recording {
        hipGraphExec_t exec = nullptr;  // graph recordings
        std::vector<Relaunch> launches; // direct recordings
        bool live = false;              // false once freed
    };
    std::vector<Recording> recordings;  // id -> recording
    int last_recording = -1;
    int* gate = nullptr;   // pinned host word the replay gate waits on (hipHostMalloc, coherent)
    int* flags = nullptr;  // device_flags(): 64 ints, allocated by byhip_init
    int gate_open = 0;     // value that opens the next gate
};

State& st() {
    static State s;
    return s;
}

thread_local std::string t_last_error;

// Timing marks: one thread stores the GPU's constant-rate realtime counter (s_memrealtime, at
// hipDeviceAttributeWallClockRate) with an ordinary vector store.
__device__ unsigned long long g_marks[2];
__global__ void timing_mark(int which) { g_marks[which] = __builtin_amdgcn_s_memrealtime(); }

// Replay gate: one thread waits until the host has stored `open` into a pinned word, or until
// `max_ticks` of the realtime counter have passed (the wait always ends). A direct replay puts it
// ahead of its launches and opens it once every launch is queued, so the replayed kernels run back
// to back however slowly the host launches them (a kernel-trace profiler slows each launch).
__global__ void replay_gate(const int* word, int open, unsigned long long max_ticks) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != open &&
           __builtin_amdgcn_s_memrealtime() - t0 < max_ticks)
        __builtin_amdgcn_s_sleep(8);
}
std::atomic<int> g_fault_inject{0};

}  // namespace

void set_error(const std::string& msg) { t_last_error = msg; }

void fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw Error(buf);
}

void unsupported(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw Unsupported(buf);
}

void check_hip(hipError_t e, const char* what, const char* file, int line) {
    if (e != hipSuccess) {
        const char* base = strrchr(file, '/');
        fail("byhip: %s failed: %s (%s:%d)", what, hipGetErrorString(e), base ? base + 1 : file,
             line);
    }
}

void enter_compute() {
    int pending = g_fault_inject.load();
    while (pending > 0) {
        if (g_fault_inject.compare_exchange_weak(pending, pending - 1))
            fail("byhip: injected fault");
    }
    if (!st().inited) fail("byhip: not initialised (call byhip_init first)");
}

hipStream_t stream() { return st().stream; }
int compute_units() { return st().prop.multiProcessorCount; }
void* workspace() { return st().workspace; }
bool session_open() { return st().session_open || st().recording; }
bool keeping_launches() { return st().recording && st().direct_open; }
void keep_launch(Relaunch l) { st().kept.push_back(std::move(l)); }
const hipDeviceProp_t& device_props() { return st().prop; }

void no_host_sync(const char* what) {
    if (st().recording)
        fail("byhip: %s waits for the device and is not allowed while a session is recorded", what);
}

size_t alloc_bytes(const void* p) {
    State& s = st();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    auto it = s.allocs.find(p);
    return it == s.allocs.end() ? 0 : it->second.bytes;
}

const std::vector<uint8_t>* host_mirror(const void* p) {
    State& s = st();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    auto it = s.allocs.find(p);
    if (it == s.allocs.end() || it->second.mirror.empty()) return nullptr;
    return &it->second.mirror;
}

std::atomic<unsigned long long> g_alloc_count{0};  // device allocations since the process started

void* device_alloc(size_t bytes) {
    State& s = st();
    void* p = nullptr;
    BYHIP_HIP(hipMalloc(&p, bytes ? bytes : 1));
    g_alloc_count.fetch_add(1);
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    s.allocs[p].bytes = bytes;
    return p;
}

void device_free(void* p) {
    if (!p) return;
    State& s = st();
    {
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        s.allocs.erase(p);
    }
    BYHIP_HIP(hipFree(p));
}

void check_span(const void* p, size_t need, const char* what) {
    if (!p) fail("byhip: %s is null", what);
    State& s = st();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    // Find the allocation holding p (p may point inside one, e.g. a slot at an offset).
    for (const auto& kv : s.allocs) {
        const uint8_t* base = static_cast<const uint8_t*>(kv.first);
        const uint8_t* q = static_cast<const uint8_t*>(p);
        if (q >= base && q < base + (kv.second.bytes ? kv.second.bytes : 1)) {
            size_t avail = kv.second.bytes - static_cast<size_t>(q - base);
            if (need > avail)
                fail("byhip: %s needs %zu bytes but its buffer holds %zu", what, need, avail);
            return;
        }
    }
    // Not one of ours (memory from another allocator): the caller vouches for the size.
}

bool mirror_read(const void* p, size_t off, void* dst, size_t bytes) {
    State& s = st();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    auto it = s.allocs.find(p);
    if (it == s.allocs.end() || off + bytes > it->second.mirror.size()) return false;
    memcpy(dst, it->second.mirror.data() + off, bytes);
    return true;
}

void note_device_write(const void* p) {
    if (!p) return;
    State& s = st();
    std::lock_guard<std::recursive_mutex> lk(s.mu);
    for (auto& kv : s.allocs) {
        const uint8_t* base = static_cast<const uint8_t*>(kv.first);
        const uint8_t* q = static_cast<const uint8_t*>(p);
        if (q >= base && q < base + (kv.second.bytes ? kv.second.bytes : 1)) {
            kv.second.mirror.clear();
            return;
        }
    }
}

bool session_recording() { return st().recording; }

int* device_flags() { return st().flags; }

bool try_read_small(const void* p, size_t off, void* dst, size_t bytes) {
    if (const std::vector<uint8_t>* m = host_mirror(p)) {
        if (off + bytes <= m->size()) {
            memcpy(dst, m->data() + off, bytes);
            return true;
        }
    }
    if (st().recording) return false;
    BYHIP_HIP(hipStreamSynchronize(stream()));
    BYHIP_HIP(hipMemcpy(dst, static_cast<const uint8_t*>(p) + off, bytes, hipMemcpyDeviceToHost));
    return true;
}

void read_small(const void* p, size_t off, void* dst, size_t bytes) {
    if (const std::vector<uint8_t>* m = host_mirror(p)) {
        if (off + bytes <= m->size()) {
            memcpy(dst, m->data() + off, bytes);
            return;
        }
    }
    no_host_sync("reading a device buffer");
    BYHIP_HIP(hipStreamSynchronize(stream()));
    BYHIP_HIP(hipMemcpy(dst, static_cast<const uint8_t*>(p) + off, bytes, hipMemcpyDeviceToHost));
}

}  // namespace byhip

using namespace byhip;

extern "C" {

int byhip_version(void) { return 1; }

const char* byhip_last_error(void) { return t_last_error.c_str(); }

void byhip_clear_error(void) { t_last_error.clear(); }

void byhip_fault_inject(int count) { g_fault_inject.store(count > 0 ? count : 0); }

int byhip_init(int device) {
    return guard([&] {
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.inited) {
            if (device != s.device)
                fail("byhip: already initialised on device %d (asked for %d)", s.device, device);
            return;
        }
        int count = 0;
        hipError_t e = hipGetDeviceCount(&count);
        if (e != hipSuccess || count <= 0) fail("byhip: no HIP device is available");
        if (device < 0 || device >= count) fail("byhip: device %d out of range (%d)", device, count);
        BYHIP_HIP(hipSetDevice(device));
        BYHIP_HIP(hipGetDeviceProperties(&s.prop, device));
        if (strncmp(s.prop.gcnArchName, "gfx950", 6) != 0)
            fail("byhip: built for gfx950, device %d is %s", device, s.prop.gcnArchName);
        BYHIP_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
        BYHIP_HIP(hipEventCreate(&s.ev_begin));
        BYHIP_HIP(hipEventCreate(&s.ev_end));
        int khz = 0;
        BYHIP_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
        s.realtime_hz = khz * 1e3;
        BYHIP_HIP(hipMalloc(&s.workspace, kWorkspaceBytes));
        BYHIP_HIP(hipMalloc(reinterpret_cast<void**>(&s.flags), 64 * sizeof(int)));
        g_alloc_count.fetch_add(2);
        BYHIP_HIP(hipHostMalloc(reinterpret_cast<void**>(&s.gate), sizeof(int), hipHostMallocCoherent));
        *s.gate = 0;
        static_scratch_setup(device);
        s.device = device;
        s.inited = true;
    });
}

int byhip_device_info_get(byhip_device_info* out) {
    return guard([&] {
        enter_compute();
        if (!out) fail("byhip: null device info");
        const hipDeviceProp_t& p = st().prop;
        memset(out, 0, sizeof *out);
        out->device = st().device;
        out->compute_units = p.multiProcessorCount;
        out->wavefront_size = p.warpSize;
        out->clock_khz = p.clockRate;
        out->memory_clock_khz = p.memoryClockRate;
        out->memory_bus_width = p.memoryBusWidth;
        out->total_global_mem = p.totalGlobalMem;
        out->lds_bytes_per_block = p.sharedMemPerBlock;
        snprintf(out->arch_name, sizeof out->arch_name, "%s", p.gcnArchName);
        snprintf(out->name, sizeof out->name, "%s", p.name);
    });
}

int byhip_alloc(size_t bytes, void** dptr) {
    return guard([&] {
        enter_compute();
        if (!dptr) fail("byhip: null output pointer");
        *dptr = device_alloc(bytes);
    });
}

int byhip_free(void* dptr) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_free");
        BYHIP_HIP(hipStreamSynchronize(stream()));
        device_free(dptr);
    });
}

int byhip_upload(void* dptr, size_t dst_off, const void* src, size_t bytes) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_upload");
        if (!bytes) return;
        if (!src) fail("byhip: null upload source");
        check_span(static_cast<uint8_t*>(dptr) + dst_off, bytes, "upload destination");
        BYHIP_HIP(hipMemcpyAsync(static_cast<uint8_t*>(dptr) + dst_off, src, bytes,
                                 hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipStreamSynchronize(stream()));  // the source is pageable host memory
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        auto it = s.allocs.find(dptr);
        if (it != s.allocs.end()) {
            std::vector<uint8_t>& m = it->second.mirror;
            if (!m.empty()) {
                if (dst_off + bytes <= m.size())
                    memcpy(m.data() + dst_off, src, bytes);
                else
                    m.clear();
            }
        }
    });
}

int byhip_read(const void* dptr, size_t src_off, void* dst, size_t bytes) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_read");
        if (!bytes) return;
        if (!dst) fail("byhip: null read destination");
        check_span(static_cast<const uint8_t*>(dptr) + src_off, bytes, "read source");
        BYHIP_HIP(hipStreamSynchronize(stream()));
        BYHIP_HIP(hipMemcpy(dst, static_cast<const uint8_t*>(dptr) + src_off, bytes,
                            hipMemcpyDeviceToHost));
    });
}

int byhip_memset(void* dptr, int value, size_t bytes) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_memset");
        if (!bytes) return;
        check_span(dptr, bytes, "memset destination");
        BYHIP_HIP(hipMemsetAsync(dptr, value, bytes, stream()));
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        auto it = s.allocs.find(dptr);
        if (it != s.allocs.end()) it->second.mirror.clear();
    });
}

int byhip_synchronize(void) {
    return guard([&] {
        enter_compute();
        no_host_sync("byhip_synchronize");
        BYHIP_HIP(hipStreamSynchronize(stream()));
    });
}

void* byhip_stream(void) { return st().inited ? static_cast<void*>(st().stream) : nullptr; }

// ── Session ──────────────────────────────────────────────────────────────────────────────────

int byhip_session_begin(void) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: a session is already open");
        s.session_open = true;
        if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_begin, s.stream));
    });
}

static void* session_new_buffer(const void* data, size_t bytes, bool zero) {
    void* p = device_alloc(bytes);
    if (data && bytes) {
        BYHIP_HIP(hipMemcpyAsync(p, data, bytes, hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipStreamSynchronize(stream()));
        if (bytes <= kMirrorBytes) {
            State& s = st();
            std::lock_guard<std::recursive_mutex> lk(s.mu);
            std::vector<uint8_t>& m = s.allocs[p].mirror;
            m.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + bytes);
        }
    } else if (zero && bytes) {
        BYHIP_HIP(hipMemsetAsync(p, 0, bytes, stream()));
    }
    return p;
}

int byhip_session_upload(const float* data, size_t n, void** out) {
    return guard([&] {
        enter_compute();
        no_host_sync("sessionUpload");
        if (!out) fail("byhip: null output handle");
        if (n && !data) fail("byhip: null upload data");
        *out = session_new_buffer(data, n * sizeof(float), false);
    });
}

int byhip_session_upload_bytes(const void* data, size_t bytes, void** out) {
    return guard([&] {
        enter_compute();
        no_host_sync("sessionUpload");
        if (!out) fail("byhip: null output handle");
        if (bytes && !data) fail("byhip: null upload data");
        *out = session_new_buffer(data, bytes, false);
    });
}

int byhip_session_alloc_scratch(size_t n, void** out) {
    return guard([&] {
        enter_compute();
        no_host_sync("sessionAllocScratch");
        if (!out) fail("byhip: null output handle");
        *out = session_new_buffer(nullptr, n * sizeof(float), true);
    });
}

// Launches recording `id` once on the library stream.
static void launch_recording(State& s, int id) {
    State::Recording& r = s.recordings[id];
    if (r.exec) {
        BYHIP_HIP(hipGraphLaunch(r.exec, s.stream));
    } else {
        for (Relaunch& l : r.launches) l(s.stream);
    }
}

static bool recording_live(const State& s, int id) {
    return id >= 0 && id < (int)s.recordings.size() && s.recordings[id].live;
}

// Holds the stream behind a replay gate while a direct recording's launches are queued, and opens
// it when it goes out of scope (also when a launch fails). Graph replays need none.
struct ReplayGate {
    State& s;
    bool held = false;
    ReplayGate(State& st_, bool direct) : s(st_) {
        if (!direct) return;
        const int open = ++s.gate_open;
        const unsigned long long max_ticks = (unsigned long long)(0.2 * s.realtime_hz);  // 200 ms
        launch("replay_gate", replay_gate, dim3(1), dim3(1), 0, (const int*)s.gate, open, max_ticks);
        held = true;
    }
    ~ReplayGate() {
        if (held) __atomic_store_n(s.gate, s.gate_open, __ATOMIC_RELEASE);
    }
};

static bool is_direct(const State& s, int id) { return s.recordings[id].exec == nullptr; }

// Ends a recorded session: the captured work becomes an executable graph (or, recorded for direct
// replay, the list of its kept launches), which is launched once (the session's work happens, as
// a kept Vulkan command buffer is also submitted) and kept.
static void end_recording(State& s) {
    State::Recording rec;
    rec.live = true;
    const bool direct = s.direct_open;
    s.recording = false;
    s.session_open = false;
    if (direct) {
        rec.launches.swap(s.kept);
    } else {
        hipGraph_t graph = nullptr;
        hipError_t e = hipStreamEndCapture(s.stream, &graph);
        if (e != hipSuccess || !graph) {
            (void)hipGetLastError();
            fail("byhip: the recorded session could not be kept: %s", hipGetErrorString(e));
        }
        e = hipGraphInstantiate(&rec.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) fail("byhip: instantiating the recorded session failed: %s", hipGetErrorString(e));
    }
    s.recordings.push_back(std::move(rec));
    s.last_recording = (int)s.recordings.size() - 1;
    {
        ReplayGate gate(s, direct);
        if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_begin, s.stream));
        launch_recording(s, s.last_recording);
        if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_end, s.stream));
    }
    hipError_t e = hipStreamSynchronize(s.stream);
    std::vector<void*> frees;
    frees.swap(s.deferred_frees);
    if (e != hipSuccess) fail("byhip: session failed on the device: %s", hipGetErrorString(e));
    if (s.timing) {
        float ms = 0.0f;
        BYHIP_HIP(hipEventElapsedTime(&ms, s.ev_begin, s.ev_end));
        s.gpu_seconds += ms * 1e-3;
    }
    for (void* p : frees) device_free(p);
}

int byhip_session_end(void) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (!s.session_open) fail("byhip: no session is open");
        if (s.recording) {
            end_recording(s);
            return;
        }
        s.last_recording = -1;
        if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_end, s.stream));
        hipError_t e = hipStreamSynchronize(s.stream);
        s.session_open = false;
        std::vector<void*> frees;
        frees.swap(s.deferred_frees);
        if (e != hipSuccess) fail("byhip: session failed on the device: %s", hipGetErrorString(e));
        if (s.timing) {
            float ms = 0.0f;
            BYHIP_HIP(hipEventElapsedTime(&ms, s.ev_begin, s.ev_end));
            s.gpu_seconds += ms * 1e-3;
        }
        for (void* p : frees) device_free(p);
    });
}

int byhip_session_commit_continue(void) {
    return guard([&] {
        enter_compute();
        if (!st().session_open) fail("byhip: no session is open");
        // HIP submits queued work as it is enqueued; nothing to flush and nothing to wait for.
    });
}

int byhip_session_recover(void) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.recording) {
            if (!s.direct_open) {
                hipGraph_t g = nullptr;
                (void)hipStreamEndCapture(s.stream, &g);
                if (g) (void)hipGraphDestroy(g);
            }
            s.kept.clear();
            s.recording = false;
        }
        (void)hipStreamSynchronize(s.stream);
        (void)hipGetLastError();
        s.session_open = false;
        std::vector<void*> frees;
        frees.swap(s.deferred_frees);
        for (void* p : frees) device_free(p);
    });
}

int byhip_session_read(const void* h, float* dst, size_t n) {
    return byhip_read(h, 0, dst, n * sizeof(float));
}

int byhip_session_free(void* h) {
    return guard([&] {
        enter_compute();
        if (!h) return;
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) {
            s.deferred_frees.push_back(h);
            return;
        }
        BYHIP_HIP(hipStreamSynchronize(s.stream));
        device_free(h);
    });
}

int byhip_session_set_gpu_timing(int on) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        s.timing = on != 0;
        s.gpu_seconds = 0.0;
    });
}

double byhip_session_gpu_seconds(void) { return st().gpu_seconds; }

int byhip_session_can_record(void) { return 1; }

int byhip_session_begin_recording(void) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: a session is already open");
        s.direct_open = s.direct;
        s.kept.clear();
        if (!s.direct_open) BYHIP_HIP(hipStreamBeginCapture(s.stream, hipStreamCaptureModeThreadLocal));
        s.session_open = true;
        s.recording = true;
    });
}

int byhip_session_last_recording(void) { return st().last_recording; }

int byhip_session_set_direct_replay(int on) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        s.direct = on != 0;
    });
}

int byhip_session_replay(int id, int times) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: replay runs outside a session");
        if (!recording_live(s, id)) fail("byhip: no recording %d", id);
        if (times < 1) fail("byhip: replay count %d", times);
        {
            ReplayGate gate(s, is_direct(s, id));
            if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_begin, s.stream));
            for (int i = 0; i < times; ++i) launch_recording(s, id);
            if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_end, s.stream));
        }
        BYHIP_HIP(hipStreamSynchronize(s.stream));
        if (s.timing) {
            float ms = 0.0f;
            BYHIP_HIP(hipEventElapsedTime(&ms, s.ev_begin, s.ev_end));
            s.gpu_seconds += ms * 1e-3;
        }
    });
}

int byhip_session_replay_after(int pre_id, int pre_times, int id, int times) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: replay runs outside a session");
        for (int r : {pre_id, id})
            if (!recording_live(s, r)) fail("byhip: no recording %d", r);
        if (pre_times < 1 || times < 1) fail("byhip: replay counts %d, %d", pre_times, times);
        // Everything is queued before the first wait: while the lead-in runs, the host has already
        // queued the begin event and the timed launches behind it.
        {
            ReplayGate gate(s, is_direct(s, pre_id) || is_direct(s, id));
            for (int i = 0; i < pre_times; ++i) launch_recording(s, pre_id);
            if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_begin, s.stream));
            for (int i = 0; i < times; ++i) launch_recording(s, id);
            if (s.timing) BYHIP_HIP(hipEventRecord(s.ev_end, s.stream));
        }
        BYHIP_HIP(hipStreamSynchronize(s.stream));
        if (s.timing) {
            float ms = 0.0f;
            BYHIP_HIP(hipEventElapsedTime(&ms, s.ev_begin, s.ev_end));
            s.gpu_seconds += ms * 1e-3;
        }
    });
}

namespace {

// Zeroes both mark slots on the library stream (outside recordings only: no copy is captured).
void clear_marks(State& s) {
    const unsigned long long unset[2] = {0, 0};
    BYHIP_HIP(hipMemcpyToSymbolAsync(HIP_SYMBOL(g_marks), unset, sizeof unset, 0, hipMemcpyHostToDevice, s.stream));
}

// Waits for the stream, reads both slots and counts end - begin (timing on); fails unless the
// stream stored a begin and a later end since the slots were cleared.
void take_marks(State& s, const char* what) {
    unsigned long long t[2] = {0, 0};
    BYHIP_HIP(hipMemcpyFromSymbolAsync(t, HIP_SYMBOL(g_marks), sizeof t, 0, hipMemcpyDeviceToHost, s.stream));
    BYHIP_HIP(hipStreamSynchronize(s.stream));
    if (!t[0] || !t[1] || t[1] < t[0]) fail("byhip: %s holds no pair of timing marks", what);
    if (s.timing) s.gpu_seconds += (double)(t[1] - t[0]) / s.realtime_hz;
}

}  // namespace

int byhip_session_mark(int which) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (which != 0 && which != 1) fail("byhip: mark %d (0: begin, 1: end)", which);
        if (!s.recording && s.session_open) fail("byhip: marks go into a recording or outside a session");
        if (!s.recording && which == 0) clear_marks(s);
        launch("timing_mark", timing_mark, dim3(1), dim3(1), 0, which);
        BYHIP_LAUNCHED("timing_mark");
    });
}

int byhip_session_take_marks() {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: marks are taken outside a session");
        take_marks(s, "the stream");
    });
}

int byhip_session_replay_marked(int id) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (s.session_open) fail("byhip: replay runs outside a session");
        if (!recording_live(s, id)) fail("byhip: no recording %d", id);
        clear_marks(s);
        {
            ReplayGate gate(s, is_direct(s, id));
            launch_recording(s, id);
        }
        char what[48];
        snprintf(what, sizeof what, "recording %d", id);
        take_marks(s, what);
    });
}

int byhip_session_free_recording(int id) {
    return guard([&] {
        enter_compute();
        State& s = st();
        std::lock_guard<std::recursive_mutex> lk(s.mu);
        if (!recording_live(s, id)) return;
        BYHIP_HIP(hipStreamSynchronize(s.stream));
        State::Recording& r = s.recordings[id];
        if (r.exec) BYHIP_HIP(hipGraphExecDestroy(r.exec));
        r = State::Recording();
    });
}

}  // extern "C"

// ── A plain copy kernel (bandwidth and HBM-counter calibration) ─────────────────────────────

namespace {
__global__ __launch_bounds__(256) void copy_words(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                  size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}
// Streaming read: each wave reads runs of 8 x 1 KB (a 16-byte nontemporal load per lane, eight in
// flight), grid-stride; the tail words one per thread. Each wave stores its fold of the words to its
// own sink slot, which keeps the loads.
constexpr int kReadDepth = 8;
__global__ __launch_bounds__(256) void read_words(const uint4* __restrict__ src, size_t n, uint32_t* sink) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u* s4 = reinterpret_cast<const v4u*>(src);
    const size_t wave = (size_t)blockIdx.x * 4 + threadIdx.x / 64, nwaves = (size_t)gridDim.x * 4;
    const size_t lane = threadIdx.x & 63, run = 64 * kReadDepth;
    uint32_t acc = 0;
    for (size_t seg = wave; seg < n / run; seg += nwaves) {
        v4u v[kReadDepth];
#pragma unroll
        for (int d = 0; d < kReadDepth; ++d) v[d] = __builtin_nontemporal_load(s4 + seg * run + 64 * d + lane);
#pragma unroll
        for (int d = 0; d < kReadDepth; ++d) acc ^= v[d][0] + v[d][1] + v[d][2] + v[d][3];
    }
    for (size_t i = n / run * run + (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        acc ^= src[i].x;
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if (lane == 0) sink[wave] = acc;
}
}  // namespace

extern "C" int byhip_debug_read(const void* src, size_t bytes, void* sink, size_t sink_bytes) {
    return guard([&] {
        enter_compute();
        if (bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
            fail("byhip: read needs a 16-byte aligned pointer and size");
        const unsigned grid = (unsigned)compute_units() * 4;  // 16 waves per CU
        if (sink_bytes < (size_t)grid * 4 * sizeof(uint32_t))
            fail("byhip: read sink needs %zu bytes", (size_t)grid * 4 * sizeof(uint32_t));
        check_span(src, bytes, "read source");
        check_span(sink, (size_t)grid * 4 * sizeof(uint32_t), "read sink");
        if (bytes == 0) return;
        launch("read_words", read_words, dim3(grid), dim3(256), 0, static_cast<const uint4*>(src),
                           bytes / 16, static_cast<uint32_t*>(sink));
        BYHIP_LAUNCHED("read_words");
    });
}

extern "C" unsigned long long byhip_debug_alloc_count(void) { return g_alloc_count.load(); }

extern "C" int byhip_debug_copy(void* dst, const void* src, size_t bytes) {
    return guard([&] {
        enter_compute();
        if (bytes % 16 || reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(src) % 16)
            fail("byhip: copy needs 16-byte aligned pointers and sizes");
        check_span(dst, bytes, "copy destination");
        check_span(src, bytes, "copy source");
        const size_t n = bytes / 16;
        const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, (size_t)compute_units() * 16);
        if (n == 0) return;
        launch("copy_words", copy_words, dim3(grid), dim3(256), 0, static_cast<const uint4*>(src),
                           static_cast<uint4*>(dst), n);
        BYHIP_LAUNCHED("copy_words");
    });
}
