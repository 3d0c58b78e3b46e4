// xq_profile.hip — optional per-kernel device timing with HIP events.
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "xq_kernels.h"

namespace xq {

namespace {
struct Pending {
    const char* name;
    hipEvent_t start, stop;
};
struct Total {
    double ms = 0.0;
    int64_t n = 0;
};
std::atomic<int> g_on{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::map<std::string, Total> g_totals;
thread_local int g_no_alloc = 0;
}  // namespace

NoAllocScope::NoAllocScope() { ++g_no_alloc; }
NoAllocScope::~NoAllocScope() { --g_no_alloc; }

bool prof_events(hipStream_t stream, hipEvent_t* start, hipEvent_t* stop) {
    if (!g_on.load(std::memory_order_relaxed) || g_no_alloc) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
    if (hipEventCreate(start) != hipSuccess) return false;
    if (hipEventCreate(stop) != hipSuccess) {
        (void)hipEventDestroy(*start);
        return false;
    }
    return true;
}

void prof_commit(const char* name, hipEvent_t start, hipEvent_t stop) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_pending.push_back({name, start, stop});
}

}  // namespace xq

extern "C" {

void xq_profile_enable(int32_t on) { xq::g_on.store(on ? 1 : 0); }

void xq_profile_reset(void) {
    std::lock_guard<std::mutex> lk(xq::g_mu);
    for (auto& p : xq::g_pending) {
        (void)hipEventSynchronize(p.stop);
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    xq::g_pending.clear();
    xq::g_totals.clear();
}

int32_t xq_profile_read(char* names, double* total_ms, int64_t* launches, int32_t max) {
    std::lock_guard<std::mutex> lk(xq::g_mu);
    for (auto& p : xq::g_pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            auto& t = xq::g_totals[p.name];
            t.ms += ms;
            t.n += 1;
        }
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    xq::g_pending.clear();
    int32_t i = 0;
    for (auto& kv : xq::g_totals) {
        if (i >= max) break;
        if (names) {
            memset(names + 32 * i, 0, 32);
            strncpy(names + 32 * i, kv.first.c_str(), 31);
        }
        if (total_ms) total_ms[i] = kv.second.ms;
        if (launches) launches[i] = kv.second.n;
        ++i;
    }
    return i;
}

}  // extern "C"
