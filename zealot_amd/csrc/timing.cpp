// timing.cpp -- optional hipEvent bracketing of the library's kernel launches.
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "zk_common.h"

namespace zk {
namespace {

struct Record {
    const char *name;
    hipEvent_t start, stop;
};

std::atomic<bool> g_on{false};
thread_local int g_suspended = 0;
std::mutex g_mu;
std::vector<Record> g_records;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

TimingSuspend::TimingSuspend() { ++g_suspended; }
TimingSuspend::~TimingSuspend() { --g_suspended; }

KernelTimer::KernelTimer(const char *name, hipStream_t stream) : name_(name), stream_(stream) {
    if (!g_on.load(std::memory_order_relaxed) || g_suspended) return;
    std::lock_guard<std::mutex> g(g_mu);
    start_ = take_event();
    stop_ = take_event();
    if (start_ && stop_ && hipEventRecord(start_, stream_) == hipSuccess) {
        active_ = true;
    } else {
        if (start_) g_pool.push_back(start_);
        if (stop_) g_pool.push_back(stop_);
        start_ = stop_ = nullptr;
    }
}

KernelTimer::~KernelTimer() {
    if (!active_) return;
    std::lock_guard<std::mutex> g(g_mu);
    if (hipEventRecord(stop_, stream_) == hipSuccess) {
        g_records.push_back({name_, start_, stop_});
    } else {
        g_pool.push_back(start_);
        g_pool.push_back(stop_);
    }
}

}  // namespace zk

extern "C" {

int zk_timing_enable(int on) {
    zk::g_on.store(on != 0);
    return ZK_OK;
}

int zk_timing_reset(void) {
    std::lock_guard<std::mutex> g(zk::g_mu);
    for (auto &r : zk::g_records) {
        (void)hipEventSynchronize(r.stop);
        zk::g_pool.push_back(r.start);
        zk::g_pool.push_back(r.stop);
    }
    zk::g_records.clear();
    return ZK_OK;
}

int zk_timing_query(const char *kernel, int64_t *launches, double *total_ms) {
    if (!kernel) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_timing_query: NULL name");
    std::lock_guard<std::mutex> g(zk::g_mu);
    int64_t n = 0;
    double ms = 0.0;
    for (auto &r : zk::g_records) {
        if (std::strcmp(r.name, kernel) != 0) continue;
        ZK_HIP_CHECK(hipEventSynchronize(r.stop), "zk_timing_query");
        float t = 0.0f;
        ZK_HIP_CHECK(hipEventElapsedTime(&t, r.start, r.stop), "zk_timing_query");
        ms += t;
        ++n;
    }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    return ZK_OK;
}

}  // extern "C"
