// Per-kernel timing hook (benchmarking aid).  When enabled, every kernel the library launches is
// bracketed by a pair of HIP events on its own stream.  A short device-side sleep is enqueued
// before the start event so the GPU is still busy while the host enqueues start/kernel/stop: the
// measured interval is then the kernel's execution, not host launch gaps.  Not thread-safe; meant
// for a single benchmarking thread.
#include <map>
#include <string>
#include <string.h>
#include <vector>

#include "internal.h"

namespace {

struct Rec {
    const char *name;
    hipEvent_t start, stop;
};

bool g_on = false;
bool g_open = false;
size_t g_max = 0;
uint64_t g_sleep_ticks = 0;
std::vector<Rec> g_recs;

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

bool stacr_prof_on() { return g_on; }

void stacr_prof_before(hipStream_t s)
{
    g_open = false;
    if (g_recs.size() >= g_max) return;
    Rec r{nullptr, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess) return;
    if (hipEventCreate(&r.stop) != hipSuccess) {
        (void)hipEventDestroy(r.start);
        return;
    }
    if (g_sleep_ticks) k_gpu_sleep<<<1, 64, 0, s>>>(g_sleep_ticks);
    (void)hipEventRecord(r.start, s);
    g_recs.push_back(r);
    g_open = true;
}

void stacr_prof_after(const char *name, hipStream_t s)
{
    if (!g_open) return;
    g_recs.back().name = name;
    (void)hipEventRecord(g_recs.back().stop, s);
    g_open = false;
}

extern "C" {

int stacr_profile_begin(int max_launches, double sleep_us)
{
    if (g_on) return stacr_fail(STACR_ERR_INVALID, "profiling already active");
    if (max_launches < 1) return stacr_fail(STACR_ERR_INVALID, "max_launches must be positive");
    int dev = 0, khz = 0;
    int rc = stacr_hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    rc = stacr_hip_check(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "wall clock rate");
    if (rc) return rc;
    g_sleep_ticks = sleep_us > 0 ? (uint64_t)(sleep_us * (double)khz / 1000.0) : 0;
    g_max = (size_t)max_launches;
    g_recs.clear();
    g_recs.reserve(g_max);
    g_on = true;
    return STACR_OK;
}

int stacr_profile_end(int max_kernels, char *names, double *total_ms, int *launches, int *n_kernels)
{
    if (!g_on) return stacr_fail(STACR_ERR_INVALID, "profiling is not active");
    g_on = false;
    std::map<std::string, std::pair<double, int>> agg;
    std::vector<std::string> order;
    int rc = STACR_OK;
    for (Rec &r : g_recs) {
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
    g_recs.clear();
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
