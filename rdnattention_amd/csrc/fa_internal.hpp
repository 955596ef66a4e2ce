// Host-side helpers shared by the kernel launchers (not part of the ABI).
#pragma once

#include "fa_host.hpp"

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace rdna_amd {

// A fixed device region that scratch buffers are carved from instead of
// being allocated (the no-allocation entry point's static array): `used`
// bytes of `bytes` at `base` are taken, each buffer 256-byte aligned.
struct ScratchRegion {
    char* base = nullptr;
    size_t bytes = 0;
    size_t used = 0;
};

// Bytes a buffer of `bytes` takes from a ScratchRegion (256-byte aligned).
constexpr size_t region_bytes(size_t bytes) {
    return (bytes + 255) / 256 * 256;
}

// What a scratch buffer holds; calls keep one cached buffer per (device,
// stream, purpose), so buffers of one call never alias.
enum class ScratchUse : int { RotatedK = 0, SplitKPartials = 1, QuantPartials = 2 };

// Scratch memory for one call (scratch.cpp).  Without a region: the buffer
// cached for (device, stream, use); a call that finds it large enough makes
// no allocator call, and the call's first use waits on the GPU
// (hipStreamWaitEvent) for the event recorded after the buffer's previous
// use.  Growth replaces the buffer with hipMallocAsync after releasing the
// old one with hipFreeAsync in the stream's order; the cached bytes of a
// device are capped, with idle entries evicted least recently used first;
// buffers above 256 MiB, calls under graph capture and a second host thread
// that finds the buffer in use take a per-call default-pool block
// (hipMallocAsync / hipFreeAsync).  No path here waits on the host.
// With a region: carved from it, nothing allocated or freed (the caller has
// checked that it fits).
struct StreamScratch {
    void* ptr = nullptr;
    hipStream_t stream = nullptr;
    ScratchRegion* region = nullptr;
    ScratchUse use;
    bool cached = false; // ptr is the (device, stream, use) cache entry's buffer
    bool pooled = false; // ptr is a per-call hipMallocAsync block
    int device = 0;
    explicit StreamScratch(ScratchUse u, ScratchRegion* r = nullptr) : region(r), use(u) {}
    int alloc(size_t bytes, hipStream_t s, std::string& err);
    StreamScratch(const StreamScratch&) = delete;
    StreamScratch& operator=(const StreamScratch&) = delete;
    ~StreamScratch();
};

// Size of the no-allocation entry point's static scratch array per device
// (64 MiB): room for a RoPE-rotated K copy of B * Hkv * Sk * D fp16 values
// up to 2^25 (a 4 x 8 x 4096 x 128 K is 2^24) together with split-K partials.
constexpr size_t kNoAllocBytes = size_t(64) << 20;

// Frees the cached scratch buffers that no call is using (after their last
// use has completed) and returns the default memory pools' free blocks to the
// devices; synchronises each device that has cached scratch.  0, or -1 with
// `err`.
int scratch_trim(std::string& err);

// Cached scratch of `device`: bytes held, buffers held, and the allocator
// calls made for it so far (cache growth and per-call blocks).  Always 0.
int scratch_stats(int device, uint64_t& cached_bytes, int64_t& entries, int64_t& allocations);

// The no-allocation entry point's region on the current device: the
// library's static scratch array (fa_noalloc.hip), its device address looked
// up once per device.  0, or -1 with `err`.
int noalloc_region(ScratchRegion& r, std::string& err);

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

// Launchers.  `region`, when given, supplies every scratch buffer.
int fwd_f16_prefill(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err);
int fwd_f16_splitk(const AttnArgs& a, bool rope_q, hipStream_t stream, std::string& err,
                   ScratchRegion* region = nullptr);

// Split-K plan of a decode launch: key splits and keys per split.  0, or -1
// with `err` (occupancy query failed).
int splitk_plan(const AttnArgs& a, int& splits, int& keys_per_split, std::string& err);

// Bytes of the split-K partials (per split and query row: O in fp32 plus m, l).
size_t splitk_partial_bytes(const AttnArgs& a, int splits);

} // namespace rdna_amd
