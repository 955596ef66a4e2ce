// Host-side helpers shared by the kernel launchers (not part of the ABI).
#pragma once

#include "fa_host.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace rdna_amd {

// Stream-ordered scratch memory: allocated with hipMallocAsync on the
// caller's stream and released with hipFreeAsync on the same stream when the
// object goes out of scope, i.e. after every kernel that uses it has been
// enqueued.  Safe across concurrent streams and under graph capture.
struct StreamScratch {
    void* ptr = nullptr;
    hipStream_t stream = nullptr;
    int alloc(size_t bytes, hipStream_t s, std::string& err);
    StreamScratch() = default;
    StreamScratch(const StreamScratch&) = delete;
    StreamScratch& operator=(const StreamScratch&) = delete;
    ~StreamScratch();
};

// Rotates K ([B, Hkv, Sk, D] with a.ks strides) into `dst`, contiguous
// [B, Hkv, Sk, D], with the tables a.rot_cos / a.rot_sin.
int rope_rotate_k(const AttnArgs& a, void* dst, hipStream_t stream, std::string& err);

// Kernel timer for measurement.  While enabled (rdna_kernel_timer_enable),
// every launch of a main attention kernel is bracketed by a HIP event pair
// recorded on the launch stream; rdna_kernel_timer_read sums the elapsed
// times.  Disabled, the guard costs one relaxed atomic load.
class KernelTimerGuard {
  public:
    explicit KernelTimerGuard(hipStream_t stream);
    ~KernelTimerGuard();
    KernelTimerGuard(const KernelTimerGuard&) = delete;
    KernelTimerGuard& operator=(const KernelTimerGuard&) = delete;

  private:
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
};

// Workgroups of `kernel` (launched with `threads` threads and no dynamic LDS)
// that the current device holds at once: compute units x workgroups per
// compute unit. Cached per device and kernel; <= 0 with `err` set on failure.
int64_t resident_workgroups(const void* kernel, int threads, std::string& err);

// Launchers.
int fwd_f16_prefill(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err);
int fwd_f16_splitk(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err);

} // namespace rdna_amd
