// profile.cpp - optional per-kernel timing with HIP events.
//
// When enabled, every launch site brackets its kernel with two events on the
// launch stream; sqa_profile_get() synchronises and sums the elapsed times.
// This is the device-timer counterpart of the engine's host-side phase timers
// (SQWEN_PROFILE, src/engine/runner.rs:1602-1705 of the reference). Off by
// default; when off a launch site costs one relaxed flag test.
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace sqa {
namespace {
struct Rec {
    hipEvent_t a, b;
    const char *name;
};
std::mutex g_mu;
std::atomic<bool> g_on{false};
std::vector<Rec> g_pool;    // created events, reused
size_t g_used = 0;
size_t g_cap = 0;
}  // namespace

bool profile_on() { return g_on.load(std::memory_order_relaxed); }

// Returns a record slot (or -1 when full/off) and records its start event.
int profile_start(const char *name, hipStream_t s) {
    if (!profile_on()) return -1;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_used >= g_cap) return -1;
    Rec &r = g_pool[g_used];
    r.name = name;
    if (hipEventRecord(r.a, s) != hipSuccess) return -1;
    return (int)g_used++;
}

void profile_stop(int slot, hipStream_t s) {
    if (slot < 0) return;
    std::lock_guard<std::mutex> lock(g_mu);
    (void)hipEventRecord(g_pool[slot].b, s);
}

}  // namespace sqa

using namespace sqa;

extern "C" {

int sqa_profile_begin(int32_t max_records) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (max_records < 0) return set_error(SQA_ERR_RANGE, "profile_begin: negative size");
    // Timing-only events without the system-scope fence: with the default flags
    // every record writes back and invalidates the caches, which adds ~1.5 us to
    // each bracketed kernel (an empty kernel of the decode launch shape reads
    // 6.1 us between default events, 4.6 us between these, 1.5 us in a kernel
    // trace) and slows the kernel that follows.
    while ((int32_t)g_pool.size() < max_records) {
        Rec r{};
        if (hipEventCreateWithFlags(&r.a, hipEventDisableSystemFence) != hipSuccess ||
            hipEventCreateWithFlags(&r.b, hipEventDisableSystemFence) != hipSuccess)
            return set_error(SQA_ERR_HIP, "profile_begin: hipEventCreate failed");
        g_pool.push_back(r);
    }
    g_cap = (size_t)max_records;
    g_used = 0;
    g_on.store(true);
    return SQA_OK;
}

int sqa_profile_end(void) {
    g_on.store(false);
    return SQA_OK;
}

int sqa_profile_get(const char *kernel, double *total_ms, int64_t *count) {
    if (!kernel || !total_ms || !count) return set_error(SQA_ERR_INVALID, "profile_get: null argument");
    std::lock_guard<std::mutex> lock(g_mu);
    double tot = 0.0;
    int64_t n = 0;
    for (size_t i = 0; i < g_used; ++i) {
        if (std::string(g_pool[i].name) != kernel) continue;
        if (hipEventSynchronize(g_pool[i].b) != hipSuccess)
            return set_error(SQA_ERR_HIP, "profile_get: event sync failed");
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g_pool[i].a, g_pool[i].b) != hipSuccess)
            return set_error(SQA_ERR_HIP, "profile_get: elapsed time failed");
        tot += ms;
        ++n;
    }
    *total_ms = tot;
    *count = n;
    return SQA_OK;
}

}  // extern "C"
