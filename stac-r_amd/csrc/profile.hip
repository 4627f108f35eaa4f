// Per-kernel timing hook (benchmarking aid).  When enabled, every kernel the library launches is
// bracketed by a pair of HIP events on its own stream.  A short device-side sleep is enqueued
// before the start event so the GPU is still busy while the host enqueues start/kernel/stop: the
// measured interval is then the kernel's execution, not host launch gaps.  A session is process
// wide: it records the launches of every thread (a framework may launch from several, such as
// an autograd worker), each thread's start/stop pair under one lock.
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <string.h>
#include <vector>

#include "internal.h"

namespace {

struct Rec {
    const char *name;
    hipEvent_t start, stop;
};

struct Session {
    std::atomic<bool> on{false};
    std::mutex mu;
    size_t max = 0;
    uint64_t sleep_ticks = 0;
    std::vector<Rec> recs;  // capacity reserved at begin: never reallocated while recording
};

Session g_session;
thread_local long t_open = -1;  // this thread's record awaiting its stop event

// Sleeps one wave until `ticks` of the constant wall clock have passed; the loop is bounded so it
// ends even if the clock were to misbehave.
__global__ void k_gpu_sleep(uint64_t ticks)
{
    const uint64_t t0 = wall_clock64();
    for (int i = 0; i < (1 << 16); ++i) {
        if (wall_clock64() - t0 >= ticks) break;
        __builtin_amdgcn_s_sleep(32);
    }
}

}  // namespace

bool stacr_prof_on() { return g_session.on.load(std::memory_order_acquire); }

void stacr_prof_before(hipStream_t s)
{
    t_open = -1;
    std::lock_guard<std::mutex> lock(g_session.mu);
    if (!g_session.on.load(std::memory_order_relaxed) || g_session.recs.size() >= g_session.max) return;
    Rec r{nullptr, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess) return;
    if (hipEventCreate(&r.stop) != hipSuccess) {
        (void)hipEventDestroy(r.start);
        return;
    }
    if (g_session.sleep_ticks) k_gpu_sleep<<<1, 64, 0, s>>>(g_session.sleep_ticks);
    (void)hipEventRecord(r.start, s);
    g_session.recs.push_back(r);
    t_open = (long)g_session.recs.size() - 1;
}

void stacr_prof_after(const char *name, hipStream_t s)
{
    if (t_open < 0) return;
    std::lock_guard<std::mutex> lock(g_session.mu);
    if ((size_t)t_open < g_session.recs.size()) {
        g_session.recs[(size_t)t_open].name = name;
        (void)hipEventRecord(g_session.recs[(size_t)t_open].stop, s);
    }
    t_open = -1;
}

extern "C" {

int stacr_profile_begin(int max_launches, double sleep_us)
{
    std::lock_guard<std::mutex> lock(g_session.mu);
    if (g_session.on.load(std::memory_order_relaxed)) return stacr_fail(STACR_ERR_INVALID, "profiling already active");
    if (max_launches < 1) return stacr_fail(STACR_ERR_INVALID, "max_launches must be positive");
    int dev = 0, khz = 0;
    int rc = stacr_hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    rc = stacr_hip_check(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "wall clock rate");
    if (rc) return rc;
    g_session.sleep_ticks = sleep_us > 0 ? (uint64_t)(sleep_us * (double)khz / 1000.0) : 0;
    g_session.max = (size_t)max_launches;
    g_session.recs.clear();
    g_session.recs.reserve(g_session.max);
    g_session.on.store(true, std::memory_order_release);
    return STACR_OK;
}

int stacr_profile_end(int max_kernels, char *names, double *total_ms, int *launches, int *n_kernels)
{
    std::lock_guard<std::mutex> lock(g_session.mu);
    if (!g_session.on.load(std::memory_order_relaxed)) return stacr_fail(STACR_ERR_INVALID, "profiling is not active");
    g_session.on.store(false, std::memory_order_release);
    std::map<std::string, std::pair<double, int>> agg;
    std::vector<std::string> order;
    int rc = STACR_OK;
    for (Rec &r : g_session.recs) {
        if (!rc) rc = stacr_hip_check(hipEventSynchronize(r.stop), "hipEventSynchronize");
        float ms = 0.f;
        if (!rc && r.name) rc = stacr_hip_check(hipEventElapsedTime(&ms, r.start, r.stop), "hipEventElapsedTime");
        if (!rc && r.name) {
            auto it = agg.find(r.name);
            if (it == agg.end()) {
                agg[r.name] = {0.0, 0};
                order.push_back(r.name);
            }
            agg[r.name].first += ms;
            agg[r.name].second += 1;
        }
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_session.recs.clear();
    if (rc) return rc;
    int n = 0;
    for (const std::string &name : order) {
        if (n >= max_kernels) break;
        if (names) {
            strncpy(names + 64 * n, name.c_str(), 63);
            names[64 * n + 63] = 0;
        }
        if (total_ms) total_ms[n] = agg[name].first;
        if (launches) launches[n] = agg[name].second;
        ++n;
    }
    if (n_kernels) *n_kernels = n;
    return STACR_OK;
}

}  // extern "C"
