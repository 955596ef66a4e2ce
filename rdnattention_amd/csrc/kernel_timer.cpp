// Event-based timing of the main attention kernels (rdna_kernel_timer_*).
//
// A measurement aid with no counterpart in the reference: benchmarks divide a
// kernel's algorithmic FLOPs or bytes by its own duration, which events
// around a whole library call cannot give when the call also launches a RoPE
// pre-rotation or a split-K combine kernel.
#include "fa_internal.hpp"
#include "rdnattention_ext.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

namespace rdna_amd {
namespace {

std::atomic<bool> g_timer_on{false};
std::mutex g_timer_mu;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_timer_pending;  // guarded by g_timer_mu
int g_timer_failed = 0;                                             // guarded by g_timer_mu

void drop_pending() {
    for (auto& ev : g_timer_pending) {
        hipEventDestroy(ev.first);
        hipEventDestroy(ev.second);
    }
    g_timer_pending.clear();
}

} // namespace

KernelTimerGuard::KernelTimerGuard(hipStream_t stream) : stream_(stream) {
    if (!g_timer_on.load(std::memory_order_relaxed)) {
        return;
    }
    // timing only: no system-scope fence (its L2 writeback would land inside
    // the measured interval)
    if (hipEventCreateWithFlags(&start_, hipEventDisableSystemFence) != hipSuccess ||
        hipEventRecord(start_, stream_) != hipSuccess) {
        if (start_ != nullptr) {
            hipEventDestroy(start_);
        }
        start_ = nullptr;
        std::lock_guard<std::mutex> lk(g_timer_mu);
        g_timer_failed++;
    }
}

KernelTimerGuard::~KernelTimerGuard() {
    if (start_ == nullptr) {
        return;
    }
    hipEvent_t stop = nullptr;
    if (hipEventCreateWithFlags(&stop, hipEventDisableSystemFence) != hipSuccess ||
        hipEventRecord(stop, stream_) != hipSuccess) {
        if (stop != nullptr) {
            hipEventDestroy(stop);
        }
        hipEventDestroy(start_);
        std::lock_guard<std::mutex> lk(g_timer_mu);
        g_timer_failed++;
        return;
    }
    std::lock_guard<std::mutex> lk(g_timer_mu);
    g_timer_pending.emplace_back(start_, stop);
}

} // namespace rdna_amd

extern "C" {

RDNA_API int32_t rdna_kernel_timer_enable(int32_t on) {
    std::lock_guard<std::mutex> lk(rdna_amd::g_timer_mu);
    rdna_amd::drop_pending();
    rdna_amd::g_timer_failed = 0;
    rdna_amd::g_timer_on.store(on != 0, std::memory_order_relaxed);
    return 0;
}

RDNA_API int32_t rdna_kernel_timer_read(double* total_ms, int64_t* launches) {
    if (total_ms == nullptr || launches == nullptr) {
        return -3;
    }
    std::lock_guard<std::mutex> lk(rdna_amd::g_timer_mu);
    double ms = 0.0;
    int64_t n = 0;
    int32_t rc = rdna_amd::g_timer_failed ? -3 : 0;
    for (auto& ev : rdna_amd::g_timer_pending) {
        float t = 0.f;
        if (hipEventSynchronize(ev.second) != hipSuccess || hipEventElapsedTime(&t, ev.first, ev.second) != hipSuccess) {
            rc = -3;
            continue;
        }
        ms += t;
        n++;
    }
    rdna_amd::drop_pending();
    rdna_amd::g_timer_failed = 0;
    *total_ms = ms;
    *launches = n;
    return rc;
}

} // extern "C"
