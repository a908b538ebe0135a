// byhip_tune.hip - per-shape Q4 kernel plans: selection with a parity gate, kept on disk.
//
// byhip_q4_prepare follows residentPrepareQ4 (gpubackend.nim:2871-2880) and vulkanPrepareQ4Tuned
// (backends/vulkan/q4_autotune.nim:387-543): for the weights' shape and an M class (1: decode;
// 2..32; 33..128; more), every kernel choice that takes the call runs once on deterministic input
// and must match the exact per-element kernel (the reference's arithmetic) within 1e-4 of the
// output's magnitude, 3e-3 for kernels that round weights to fp16 for the MFMA (the reference's
// tolerance for its tensor-core kernels), with finite outputs. The survivors are timed in three
// rounds in alternating order, each run with cold caches; the median decides, and a kernel
// replaces the current best only when it is at least 3% faster. The choice is kept in memory for byhip_q4_matmul and in a plan
// file keyed by the device and the library's kernel sources (q4_autotune.nim:32-50), so a later
// process reuses it without tuning.
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "byhip_internal.h"
#include "byhip_q4.h"

#ifndef BYHIP_SOURCE_HASH
#define BYHIP_SOURCE_HASH "unknown"
#endif

namespace byhip {
namespace {

struct PlanEntry {
    Q4Plan plan;
    std::string name;
    bool from_cache = false;
};

struct Tuner {
    std::mutex mu;
    std::map<std::string, PlanEntry> plans;  // this process's plans
    bool cache_loaded = false;
    std::map<std::string, PlanEntry> cached;  // the plan file's entries
};

Tuner& tuner() {
    static Tuner t;
    return t;
}

// M classes, each tuned at its representative M: decode; up to 32 rows (the skinny kernel's
// range); up to 128 (tuned at 64, the reference's prefill M); larger prefill (tuned at 256: a tile
// and split chosen at 64 rows can be slower at a few hundred).
int m_class(int M) { return M == 1 ? 1 : (M <= 32 ? 32 : (M <= 128 ? 64 : 256)); }

std::string plan_key(const byhip_q4w* w, int M, int x_dtype) {
    char buf[160];
    snprintf(buf, sizeof buf, "%d_%d_g%d_%d_f%d%d_m%d_x%d", w->K, w->N, w->group, w->gpr, w->scale_f16,
             w->zero_uniform, m_class(M), x_dtype);
    return buf;
}

std::string plan_name(const Q4Plan& p) {
    static const char* tiles[] = {"auto", "64x128", "64x64", "32x128", "32x64"};
    char buf[64];
    switch (p.kind) {
    case kPlanGeneric: return "generic";
    case kPlanGemv: return "gemv";
    case kPlanPipe:
        snprintf(buf, sizeof buf, "pipe-%s-s%d", tiles[p.tile >= 0 && p.tile <= 4 ? p.tile : 0], p.splits);
        return buf;
    case kPlanSkinny:
        snprintf(buf, sizeof buf, "skinny-s%d", p.splits);
        return buf;
    case kPlanGemm: return "gemm";
    case kPlanBig:
        snprintf(buf, sizeof buf, "big-s%d", p.splits);
        return buf;
    case kPlanWide:
        snprintf(buf, sizeof buf, "wide-s%d", p.splits);
        return buf;
    case kPlanExact: return "exact";
    case kPlanStream:
        snprintf(buf, sizeof buf, "stream-s%d", p.splits);
        return buf;
    default: return "none";
    }
}

uint64_t fnv1a(const std::string& s) {
    uint64_t h = 14695981039346656037ull;
    for (unsigned char c : s) h = (h ^ c) * 1099511628211ull;
    return h;
}

// The device and the kernels a plan was chosen for (a plan from another build or device is not
// reused).
std::string cache_signature() {
    const hipDeviceProp_t& p = device_props();
    const char* tuned = getenv("BYHIP_Q4_TUNED");
    std::ostringstream o;
    o << "v1|" << p.gcnArchName << "|" << p.name << "|cus=" << p.multiProcessorCount << "|clk=" << p.clockRate
      << "|mem=" << p.totalGlobalMem << "|tuned=" << (tuned ? tuned : "1") << "|source=" << BYHIP_SOURCE_HASH;
    return o.str();
}

std::string cache_path() {
    std::string dir;
    if (const char* d = getenv("BYHIP_CACHE_DIR")) dir = d;
    else if (const char* x = getenv("XDG_CACHE_HOME")) dir = std::string(x) + "/bybylang_amd";
    else if (const char* h = getenv("HOME")) dir = std::string(h) + "/.cache/bybylang_amd";
    else return "";
    char name[64];
    snprintf(name, sizeof name, "/q4-plans-%016llx.txt", (unsigned long long)fnv1a(cache_signature()));
    return dir + name;
}

// Plan file: the signature line, then one line per plan: key kind tile splits name.
void load_cache(Tuner& t) {
    if (t.cache_loaded) return;
    t.cache_loaded = true;
    const std::string path = cache_path();
    if (path.empty()) return;
    std::ifstream f(path);
    if (!f) return;
    std::string line;
    if (!std::getline(f, line) || line != "signature " + cache_signature()) return;
    while (std::getline(f, line)) {
        std::istringstream in(line);
        std::string key, name;
        PlanEntry e;
        if (!(in >> key >> e.plan.kind >> e.plan.tile >> e.plan.splits >> name)) continue;
        if (e.plan.kind < kPlanGeneric || e.plan.kind > kPlanLast || name != plan_name(e.plan)) continue;
        e.name = name;
        e.from_cache = true;
        t.cached[key] = e;
    }
}

void save_cache(Tuner& t) {
    const std::string path = cache_path();
    if (path.empty()) return;
    // create the directory and its parents (an existing one is fine)
    const std::string dir = path.substr(0, path.rfind('/'));
    for (size_t i = 1; i <= dir.size(); ++i)
        if (i == dir.size() || dir[i] == '/') (void)mkdir(dir.substr(0, i).c_str(), 0755);
    const std::string tmp = path + ".tmp" + std::to_string((long)getpid());
    {
        std::ofstream f(tmp);
        if (!f) return;
        f << "signature " << cache_signature() << "\n";
        for (const auto& kv : t.cached)
            f << kv.first << " " << kv.second.plan.kind << " " << kv.second.plan.tile << " "
              << kv.second.plan.splits << " " << kv.second.name << "\n";
        if (!f) return;
    }
    std::rename(tmp.c_str(), path.c_str());  // a reader sees the old or the new file, never a part
}

bool tuning_enabled() {
    const char* a = getenv("BYHIP_Q4_TUNED");
    const char* b = getenv("BYHIP_GPU_AUTOTUNE");
    return !(a && strcmp(a, "0") == 0) && !(b && strcmp(b, "0") == 0);
}

constexpr size_t kScrubBytes = (size_t)512 << 20;
constexpr int kScrubBlocks = 1024;

// Reads every 16-byte word of `buf` (n words), so that the caches and address translations hold
// other, clean data, as after other weights streamed through; each block's XOR of what it read
// goes to sink[block] (the reads are then not dead code).
__global__ __launch_bounds__(256) void scrub_read(const uint4* __restrict__ buf, size_t n, uint32_t* sink) {
    uint32_t v = 0;
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += (size_t)kScrubBlocks * 256) {
        const uint4 q = buf[i];
        v ^= q.x ^ q.y ^ q.z ^ q.w;
    }
    __shared__ uint32_t red[256];
    red[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = 0;
        for (int i = 0; i < 256; ++i) r ^= red[i];
        sink[blockIdx.x] = r;
    }
}

struct Candidate {
    Q4Plan plan;
    float tol;
};

std::vector<Candidate> candidates(int mt, int x_dtype) {
    std::vector<Candidate> c;
    if (mt == 1) {
        c.push_back({{kPlanGemv, 0, 0}, 1e-4f});
        return c;
    }
    if (x_dtype == BYHIP_F16) {
        for (int tile = 1; tile <= 4; ++tile)
            for (int sp : {0, 1, 2, 4}) c.push_back({{kPlanPipe, tile, sp}, 3e-3f});
        if (mt <= 32) {
            for (int sp : {0, 1, 2, 4}) c.push_back({{kPlanSkinny, 0, sp}, 3e-3f});
            for (int sp : {0, 1, 2, 4, 8}) c.push_back({{kPlanWide, 0, sp}, 3e-3f});
            for (int sp : {0, 2}) c.push_back({{kPlanStream, 0, sp}, 3e-3f});
        }
        if (mt > 32) {
            for (int sp : {0, 1, 2, 4}) c.push_back({{kPlanBig, 0, sp}, 3e-3f});
            for (int sp : {0, 1, 2}) c.push_back({{kPlanWide, 0, sp}, 3e-3f});
        }
    } else {
        // fp32 activations: the wide tile on two fp16 planes keeps the fp32 tolerance
        for (int sp : {0, 1, 2, 4}) c.push_back({{kPlanWide, 0, sp}, 1e-4f});
    }
    c.push_back({{kPlanGemm, 0, 0}, 3e-3f});
    c.push_back({{kPlanExact, 0, 0}, 1e-4f});
    return c;
}

// Parity, then timing and the choice, for one key.
PlanEntry tune(const byhip_q4w* w, int M, int x_dtype) {
    const int mt = m_class(M);
    const size_t xb = x_dtype == BYHIP_F32 ? 4 : 2;
    const size_t nx = (size_t)mt * w->K, ny = (size_t)mt * w->N;
    // Deterministic input in the reference's pattern (q4_autotune.nim:454-455): k/64 values, exact
    // in fp16 as well.
    std::vector<float> xf(nx);
    for (size_t i = 0; i < nx; ++i) xf[i] = (float)((long)(i * 17 % 101) - 50) / 64.0f;
    std::vector<uint16_t> xh;
    if (x_dtype == BYHIP_F16) {
        xh.resize(nx);
        for (size_t i = 0; i < nx; ++i) {
            const _Float16 h = (_Float16)xf[i];
            memcpy(&xh[i], &h, 2);
        }
    }
    void* dx = device_alloc(nx * xb);
    float* dy = static_cast<float*>(device_alloc(ny * 4));
    void* scrub = nullptr;  // kScrubBytes to read, then the blocks' sink words
    if (hipMalloc(&scrub, kScrubBytes + kScrubBlocks * sizeof(uint32_t)) != hipSuccess) {  // else warm timing
        (void)hipGetLastError();
        scrub = nullptr;
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    PlanEntry best_entry;
    try {
        BYHIP_HIP(hipMemcpyAsync(dx, x_dtype == BYHIP_F16 ? (const void*)xh.data() : (const void*)xf.data(),
                                 nx * xb, hipMemcpyHostToDevice, stream()));
        BYHIP_HIP(hipEventCreate(&e0));
        BYHIP_HIP(hipEventCreate(&e1));
        if (scrub) BYHIP_HIP(hipMemsetAsync(scrub, 0x5A, kScrubBytes, stream()));
        auto run_once = [&](const Q4Plan& p, std::vector<float>& out) {
            if (!q4_run_plan(p, dx, x_dtype, w, dy, BYHIP_F32, mt)) return false;
            out.resize(ny);
            BYHIP_HIP(hipMemcpyAsync(out.data(), dy, ny * 4, hipMemcpyDeviceToHost, stream()));
            BYHIP_HIP(hipStreamSynchronize(stream()));
            return true;
        };
        // Each timed run starts cold: a scrub buffer twice the Infinity Cache is read first (outside
        // the events), so the weights come from HBM as they do when a model's layers stream
        // through, and the caches hold clean lines as they do then (a rewrite would leave dirty
        // lines whose write-back slows the timed kernel); repeated runs on the same weights would
        // otherwise time cache hits.
        auto time_ms = [&](const Q4Plan& p, int reps) {
            float total = 0.0f;
            for (int r = 0; r < reps; ++r) {
                if (scrub) {
                    launch("scrub_read", scrub_read, dim3(kScrubBlocks), dim3(256), 0,
                                       static_cast<const uint4*>(scrub), kScrubBytes / 16,
                                       reinterpret_cast<uint32_t*>(static_cast<char*>(scrub) + kScrubBytes));
                    BYHIP_LAUNCHED("scrub_read");
                }
                BYHIP_HIP(hipEventRecord(e0, stream()));
                q4_run_plan(p, dx, x_dtype, w, dy, BYHIP_F32, mt);
                BYHIP_HIP(hipEventRecord(e1, stream()));
                BYHIP_HIP(hipEventSynchronize(e1));
                float ms = 0.0f;
                BYHIP_HIP(hipEventElapsedTime(&ms, e0, e1));
                total += ms;
            }
            return total / (float)reps;
        };

        std::vector<Q4Plan> valid{{kPlanGeneric, 0, 0}};
        std::vector<float> ref, out;
        run_once(valid[0], ref);
        float mag = 0.0f;
        for (float v : ref) {
            if (!std::isfinite(v)) fail("byhip: Q4 tuning: the reference kernel gave a non-finite output");
            mag = std::max(mag, std::fabs(v));
        }
        for (const Candidate& c : candidates(mt, x_dtype)) {
            if (!run_once(c.plan, out)) continue;  // this kernel does not take the shape
            float err = 0.0f;
            bool finite = true;
            for (size_t i = 0; i < ny; ++i) {
                finite = finite && std::isfinite(out[i]);
                err = std::max(err, std::fabs(out[i] - ref[i]));
            }
            if (finite && err <= std::max(1e-5f, mag * c.tol)) valid.push_back(c.plan);
            else if (getenv("BYHIP_Q4_TUNE_VERBOSE"))
                fprintf(stderr, "[q4-tune:hip] parity reject %s: err=%g max=%g\n", plan_name(c.plan).c_str(), err, mag);
        }
        const int reps = mt == 1 ? 32 : (mt <= 64 ? 4 : 2);
        std::vector<std::vector<float>> samples(valid.size());
        for (int round = 0; round < 3; ++round)
            for (size_t j = 0; j < valid.size(); ++j) {
                const size_t i = round % 2 == 0 ? j : valid.size() - 1 - j;
                samples[i].push_back(time_ms(valid[i], reps));
            }
        size_t best = 0;
        for (auto& s : samples) std::sort(s.begin(), s.end());
        if (getenv("BYHIP_Q4_TUNE_VERBOSE"))
            for (size_t i = 0; i < valid.size(); ++i)
                fprintf(stderr, "[q4-tune:hip]   %s %.4f ms\n", plan_name(valid[i]).c_str(), samples[i][1]);
        for (size_t i = 1; i < valid.size(); ++i)
            if (samples[i][1] < samples[best][1] * 0.97f) best = i;
        best_entry.plan = valid[best];
        best_entry.name = plan_name(valid[best]);
        fprintf(stderr, "[q4-tune:hip] %dx%d M=%d x=%s: %s %.4f ms (reference %.4f ms; %zu validated candidates)\n",
                w->K, w->N, mt, x_dtype == BYHIP_F32 ? "f32" : "f16", best_entry.name.c_str(), samples[best][1],
                samples[0][1], valid.size());
    } catch (...) {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (scrub) (void)hipFree(scrub);
        device_free(dx);
        device_free(dy);
        throw;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (scrub) (void)hipFree(scrub);
    device_free(dx);
    device_free(dy);
    return best_entry;
}

}  // namespace

bool q4_lookup_plan(const byhip_q4w* w, int M, int x_dtype, Q4Plan* out) {
    Tuner& t = tuner();
    std::lock_guard<std::mutex> lk(t.mu);
    if (t.plans.empty()) return false;
    auto it = t.plans.find(plan_key(w, M, x_dtype));
    if (it == t.plans.end()) return false;
    *out = it->second.plan;
    return true;
}

}  // namespace byhip

using namespace byhip;

extern "C" {

int byhip_q4_prepare(const byhip_q4w* w, int M, int x_dtype) {
    return guard([&] {
        enter_compute();
        if (!w) fail("byhip: null Q4 weights");
        if (M <= 0) fail("byhip: Q4 prepare needs M > 0 (M=%d)", M);
        if (x_dtype != BYHIP_F32 && x_dtype != BYHIP_F16) fail("byhip: Q4 activations must be F32 or F16");
        // As the reference: off when tuning is disabled, and not inside an open session.
        if (!tuning_enabled()) unsupported("byhip: Q4 tuning is off (BYHIP_Q4_TUNED / BYHIP_GPU_AUTOTUNE = 0)");
        if (session_open()) unsupported("byhip: Q4 tuning is not available inside a session");
        Tuner& t = tuner();
        const std::string key = plan_key(w, M, x_dtype);
        {
            std::lock_guard<std::mutex> lk(t.mu);
            if (t.plans.count(key)) return;
            load_cache(t);
            auto it = t.cached.find(key);
            if (it != t.cached.end()) {
                t.plans[key] = it->second;
                fprintf(stderr, "[q4-tune:hip] %dx%d M=%d: cache hit %s\n", w->K, w->N, m_class(M),
                        it->second.name.c_str());
                return;
            }
        }
        PlanEntry e = tune(w, M, x_dtype);
        std::lock_guard<std::mutex> lk(t.mu);
        t.plans[key] = e;
        PlanEntry saved = e;
        saved.from_cache = true;
        t.cached[key] = saved;
        save_cache(t);
    });
}

int byhip_q4_plan_info(const byhip_q4w* w, int M, int x_dtype, char* name, int name_len, int* from_cache) {
    return guard([&] {
        if (!w) fail("byhip: null Q4 weights");
        Tuner& t = tuner();
        std::lock_guard<std::mutex> lk(t.mu);
        auto it = t.plans.find(plan_key(w, M, x_dtype));
        if (it == t.plans.end()) unsupported("byhip: no Q4 plan for this shape");
        if (name && name_len > 0) snprintf(name, (size_t)name_len, "%s", it->second.name.c_str());
        if (from_cache) *from_cache = it->second.from_cache ? 1 : 0;
    });
}

int byhip_q4_plans_reset(void) {
    return guard([&] {
        Tuner& t = tuner();
        std::lock_guard<std::mutex> lk(t.mu);
        t.plans.clear();
        t.cached.clear();
        t.cache_loaded = false;
    });
}

}  // extern "C"
