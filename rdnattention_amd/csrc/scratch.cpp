// Stream-ordered scratch memory for the attention calls (the RoPE-rotated K
// copy, split-K partials, quantiser partials).
//
// The reference allocates nothing (src/c_api.hpp:3-6); its kernels need no
// scratch.  Here a call that needs scratch takes the buffer cached for its
// (device, stream, use) and touches no allocator once that buffer is large
// enough.  Measured on MI355X under ROCm 7: hipFree waits until the whole
// device is idle (~32 ms behind a busy stream, even for a buffer no kernel
// uses), while hipMalloc and the default pool's hipMallocAsync / hipFreeAsync
// return without waiting for the GPU.  So no call ever runs hipFree:
//   * a buffer that must grow is released with hipFreeAsync on the call's
//     stream (after the buffer's last use) and replaced with hipMallocAsync;
//   * the cached bytes of a device, over all streams and uses, are capped
//     (kDeviceCap); growth past the cap first evicts the least recently used
//     idle entries, released the same way in the calling stream's order
//     after their own last use (hipStreamWaitEvent on the event recorded
//     after it), and a call that still does not fit takes a per-call
//     default-pool block instead;
//   * buffers above kEntryMax are never cached, only taken per call.
// rdna_scratch_trim() (the one synchronising path) frees every idle entry and
// returns the default pool's free blocks to the device.
#include "fa_internal.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <utility>

namespace rdna_amd {
namespace {

constexpr size_t kEntryMax = size_t(256) << 20;  // largest cached buffer
constexpr size_t kDeviceCap = size_t(1) << 30;   // cached bytes per device, all streams and uses
constexpr size_t kGranule = size_t(2) << 20;     // cached buffers grow in 2 MiB steps

struct Entry {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t last_use = nullptr; // recorded on the entry's stream after each use
    bool busy = false;             // a call holds the buffer
    uint64_t tick = 0;             // last use, for LRU eviction
};

struct DeviceCache {
    std::map<std::pair<hipStream_t, int>, Entry> entries;
    size_t bytes = 0;      // sum of the entries' buffers
    uint64_t tick = 0;
    int64_t allocations = 0; // allocator calls made for this device (cache growth and per-call blocks)
};

std::mutex g_mu;
std::map<int, DeviceCache> g_devices; // guarded by g_mu

std::string hip_err(const char* what, hipError_t e) {
    return std::string(what) + ": " + hipGetErrorString(e);
}

// Releases e's buffer in the order of stream s: after the work recorded in
// its last_use event (a GPU-side wait), then hipFreeAsync on s.  Nothing here
// waits on the host.
hipError_t release_in_order(Entry& e, hipStream_t s) {
    hipError_t r = hipSuccess;
    if (e.ptr != nullptr) {
        if (e.last_use != nullptr) {
            r = hipStreamWaitEvent(s, e.last_use, 0);
        }
        if (r == hipSuccess) {
            r = hipFreeAsync(e.ptr, s);
        }
    }
    e.ptr = nullptr;
    e.bytes = 0;
    return r;
}

} // namespace

int StreamScratch::alloc(size_t bytes, hipStream_t s, std::string& err) {
    stream = s;
    if (bytes == 0) {
        return 0;
    }
    if (region != nullptr) {
        const size_t take = region_bytes(bytes);
        if (region->used + take > region->bytes) {
            err = "scratch region exhausted (" + std::to_string(region->used + take) + " of " +
                  std::to_string(region->bytes) + " bytes)";
            return -1;
        }
        ptr = region->base + region->used;
        region->used += take;
        return 0;
    }
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) {
        err = hip_err("scratch allocation failed", e);
        return -1;
    }
    // Under graph capture the allocation becomes a memory node the graph owns.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &capture);
    if (e != hipSuccess) {
        err = hip_err("scratch allocation failed", e);
        return -1;
    }
    bool per_call = capture != hipStreamCaptureStatusNone || bytes > kEntryMax;
    if (!per_call) {
        std::lock_guard<std::mutex> lock(g_mu);
        DeviceCache& dc = g_devices[device];
        const auto key = std::make_pair(s, static_cast<int>(use));
        Entry& ent = dc.entries[key];
        if (ent.busy) {
            // another host thread's call on this stream holds the buffer
            per_call = true;
        } else {
            if (ent.bytes < bytes) {
                const size_t want = std::min(kEntryMax, (bytes + kGranule - 1) / kGranule * kGranule);
                size_t total = dc.bytes - ent.bytes + want;
                // over the cap: evict idle entries, least recently used first
                while (total > kDeviceCap) {
                    auto victim = dc.entries.end();
                    for (auto it = dc.entries.begin(); it != dc.entries.end(); ++it) {
                        if (it->first != key && !it->second.busy && it->second.ptr != nullptr &&
                            (victim == dc.entries.end() || it->second.tick < victim->second.tick)) {
                            victim = it;
                        }
                    }
                    if (victim == dc.entries.end()) {
                        break;
                    }
                    const size_t freed = victim->second.bytes;
                    e = release_in_order(victim->second, s);
                    if (victim->second.last_use != nullptr) {
                        (void)hipEventDestroy(victim->second.last_use);
                    }
                    dc.entries.erase(victim);
                    dc.bytes -= freed;
                    total -= freed;
                    if (e != hipSuccess) {
                        err = hip_err("scratch eviction failed", e);
                        return -1;
                    }
                }
                if (total > kDeviceCap) {
                    per_call = true; // every other entry is in use: do not cache this one
                } else {
                    const size_t old = ent.bytes;
                    e = release_in_order(ent, s);
                    dc.bytes -= old;
                    if (e == hipSuccess) {
                        e = hipMallocAsync(&ent.ptr, want, s);
                        dc.allocations++;
                    }
                    if (e != hipSuccess) {
                        ent.ptr = nullptr;
                        err = hip_err("scratch allocation failed", e);
                        return -1;
                    }
                    ent.bytes = want;
                    dc.bytes += want;
                }
            }
            if (!per_call) {
                if (ent.last_use == nullptr) {
                    // device-scope only: the event orders GPU work (stream waits
                    // and the trim's synchronisation before a stream-ordered
                    // free); a system-scope release at each record would write
                    // back the L2 after every attention kernel
                    e = hipEventCreateWithFlags(&ent.last_use, hipEventDisableTiming | hipEventDisableSystemFence);
                } else {
                    // after the buffer's previous use; a no-op when that use was
                    // on this same stream, and it orders a handle that now names
                    // a new stream
                    e = hipStreamWaitEvent(s, ent.last_use, 0);
                }
                if (e != hipSuccess) {
                    err = hip_err("scratch allocation failed", e);
                    return -1;
                }
                ent.busy = true;
                ent.tick = ++dc.tick;
                ptr = ent.ptr;
                cached = true;
                return 0;
            }
        }
    }
    e = hipMallocAsync(&ptr, bytes, s);
    {
        std::lock_guard<std::mutex> lock(g_mu);
        g_devices[device].allocations++;
    }
    if (e != hipSuccess) {
        ptr = nullptr;
        err = hip_err("scratch allocation failed", e);
        return -1;
    }
    pooled = true;
    return 0;
}

StreamScratch::~StreamScratch() {
    if (cached) {
        // every kernel that uses the buffer has been enqueued on `stream`
        std::lock_guard<std::mutex> lock(g_mu);
        Entry& ent = g_devices[device].entries[std::make_pair(stream, static_cast<int>(use))];
        (void)hipEventRecord(ent.last_use, stream);
        ent.busy = false;
    } else if (pooled && ptr != nullptr) {
        (void)hipFreeAsync(ptr, stream);
    }
}

int scratch_trim(std::string& err) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_devices.empty()) {
        return 0; // nothing cached, no HIP call needed
    }
    int cur = 0;
    (void)hipGetDevice(&cur);
    hipError_t first = hipSuccess;
    for (auto& dv : g_devices) {
        DeviceCache& dc = dv.second;
        hipError_t e = hipSetDevice(dv.first);
        for (auto it = dc.entries.begin(); e == hipSuccess && it != dc.entries.end();) {
            Entry& ent = it->second;
            if (ent.busy) {
                ++it;
                continue;
            }
            if (ent.last_use != nullptr) {
                e = hipEventSynchronize(ent.last_use);
            }
            if (e == hipSuccess && ent.ptr != nullptr) {
                e = hipFreeAsync(ent.ptr, nullptr);
            }
            if (e != hipSuccess) {
                break;
            }
            if (ent.last_use != nullptr) {
                (void)hipEventDestroy(ent.last_use);
            }
            dc.bytes -= ent.bytes;
            it = dc.entries.erase(it);
        }
        if (e == hipSuccess) {
            e = hipDeviceSynchronize();
        }
        hipMemPool_t pool = nullptr;
        if (e == hipSuccess) {
            e = hipDeviceGetDefaultMemPool(&pool, dv.first);
        }
        if (e == hipSuccess) {
            e = hipMemPoolTrimTo(pool, 0);
        }
        if (e != hipSuccess && first == hipSuccess) {
            first = e;
        }
    }
    (void)hipSetDevice(cur);
    if (first != hipSuccess) {
        err = hip_err("scratch trim", first);
        return -1;
    }
    return 0;
}

int scratch_stats(int device, uint64_t& cached_bytes, int64_t& entries, int64_t& allocations) {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_devices.find(device);
    cached_bytes = 0;
    entries = 0;
    allocations = 0;
    if (it != g_devices.end()) {
        cached_bytes = it->second.bytes;
        for (const auto& kv : it->second.entries) {
            entries += kv.second.ptr != nullptr ? 1 : 0;
        }
        allocations = it->second.allocations;
    }
    return 0;
}

} // namespace rdna_amd
