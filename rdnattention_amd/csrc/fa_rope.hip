// RoPE pre-rotation of K and stream-ordered scratch memory.
//
// The reference rotates every K tile inside the attention loop
// (src/rdna/fa2_forward_f16.hip:256), i.e. once per query row tile that
// reads it.  Here K is rotated exactly once, by a streaming kernel, into a
// contiguous [B, Hkv, Sk, D] scratch tensor with the same arithmetic (fp32
// rotation of interleaved pairs, rounded to fp16), and the attention kernels
// read the rotated copy: the result is identical and the inner loop carries no
// table loads.
#include "fa_common.hpp"
#include "fa_host.hpp"
#include "fa_internal.hpp"

#include <algorithm>
#include <cstdint>
#include <map>
#include <tuple>
#include <mutex>

namespace rdna_amd {
namespace {

__global__ __launch_bounds__(256) void rope_rotate_rows(const _Float16* __restrict__ src, _Float16* __restrict__ dst,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, int64_t sb, int64_t sh,
                                                        int64_t ss, int32_t H, int32_t S, int32_t D,
                                                        int64_t n_chunks) {
    const int chunks_per_row = D / 8;
    const int half = D / 2;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n_chunks;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / chunks_per_row;
        const int ch = (int)(e - row * chunks_per_row);
        const int64_t bh = row / S;
        const int s = (int)(row - bh * S);
        const int64_t b = bh / H;
        const int h = (int)(bh - b * H);
        h8 x = *reinterpret_cast<const h8*>(src + b * sb + h * sh + s * ss + 8 * ch);
        x = rope8(x, cos_t + (int64_t)s * half, sin_t + (int64_t)s * half, 4 * ch);
        *reinterpret_cast<h8*>(dst + row * D + 8 * ch) = x;
    }
}

} // namespace

namespace {

constexpr uint64_t kScratchRetain = 256ull << 20;

std::mutex g_pool_mu;
std::map<int, hipMemPool_t> g_pools; // device -> its scratch pool; guarded by g_pool_mu

// One memory pool per device, created on first use, for scratch above the
// cache limit and for a call that finds its stream's cached buffer held by
// another host thread.
// Its release threshold keeps up to kScratchRetain bytes (256 MiB) of freed
// blocks instead of returning them to the device at each synchronisation.
// rdna_scratch_trim() releases what the pools and the caches hold.
int scratch_pool(hipMemPool_t& pool, std::string& err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        err = std::string("scratch pool: ") + hipGetErrorString(e);
        return -1;
    }
    std::lock_guard<std::mutex> lock(g_pool_mu);
    auto it = g_pools.find(dev);
    if (it != g_pools.end()) {
        pool = it->second;
        return 0;
    }
    hipMemPoolProps props = {};
    props.allocType = hipMemAllocationTypePinned;
    props.location.type = hipMemLocationTypeDevice;
    props.location.id = dev;
    e = hipMemPoolCreate(&pool, &props);
    if (e == hipSuccess) {
        uint64_t keep = kScratchRetain;
        e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) {
            (void)hipMemPoolDestroy(pool);
        }
    }
    if (e != hipSuccess) {
        err = std::string("scratch pool: ") + hipGetErrorString(e);
        return -1;
    }
    g_pools[dev] = pool;
    return 0;
}

} // namespace

namespace {

// One cached buffer per (device, stream, use); guarded by g_pool_mu.
struct CachedScratch {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t last_use = nullptr; // recorded on the stream after the buffer's last use
    bool busy = false;             // a call holds it
};
std::map<std::tuple<int, hipStream_t, int>, CachedScratch> g_cache;

constexpr size_t kCacheGranule = size_t(2) << 20; // buffers grow in 2 MiB steps

} // namespace

int scratch_trim(std::string& err) {
    std::lock_guard<std::mutex> lock(g_pool_mu);
    for (auto it = g_cache.begin(); it != g_cache.end();) {
        CachedScratch& c = it->second;
        if (c.busy) {
            ++it;
            continue;
        }
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(std::get<0>(it->first));
        hipError_t e = c.ptr != nullptr ? hipFree(c.ptr) : hipSuccess;
        if (e == hipSuccess && c.last_use != nullptr) {
            e = hipEventDestroy(c.last_use);
        }
        (void)hipSetDevice(cur);
        if (e != hipSuccess) {
            err = std::string("scratch trim: ") + hipGetErrorString(e);
            return -1;
        }
        it = g_cache.erase(it);
    }
    for (auto& kv : g_pools) {
        hipError_t e = hipMemPoolTrimTo(kv.second, 0);
        if (e != hipSuccess) {
            err = std::string("scratch pool trim: ") + hipGetErrorString(e);
            return -1;
        }
    }
    return 0;
}

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
    // Under graph capture the allocation becomes a memory node the graph
    // owns: take it with hipMallocAsync (the device's default pool), which
    // graph capture supports.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &capture);
    if (e != hipSuccess) {
        err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
        return -1;
    }
    if (capture != hipStreamCaptureStatusNone) {
        e = hipMallocAsync(&ptr, bytes, s);
        if (e != hipSuccess) {
            ptr = nullptr;
            err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
            return -1;
        }
        pooled = true;
        return 0;
    }
    e = hipGetDevice(&device);
    if (e != hipSuccess) {
        err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
        return -1;
    }
    // Buffers above kScratchRetain are not cached, which bounds what a stream
    // keeps per use; calls that large run long enough that the pool
    // allocation's host wait costs little.
    if (bytes <= kScratchRetain) {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        CachedScratch& c = g_cache[std::make_tuple(device, s, static_cast<int>(use))];
        if (!c.busy) {
            if (c.bytes < bytes) {
                // growing: the old buffer may still be read by queued work,
                // and hipFree waits for the device before releasing it
                if (c.ptr != nullptr) {
                    e = hipFree(c.ptr);
                    c.ptr = nullptr;
                    c.bytes = 0;
                    if (e != hipSuccess) {
                        err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
                        return -1;
                    }
                }
                const size_t want = std::min(kScratchRetain, (bytes + kCacheGranule - 1) / kCacheGranule * kCacheGranule);
                e = hipMalloc(&c.ptr, want);
                if (e != hipSuccess) {
                    c.ptr = nullptr;
                    err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
                    return -1;
                }
                c.bytes = want;
            }
            if (c.last_use == nullptr) {
                e = hipEventCreateWithFlags(&c.last_use, hipEventDisableTiming);
            } else {
                // after the buffer's previous use (a no-op when that use was on
                // this same stream, already ordered)
                e = hipStreamWaitEvent(s, c.last_use, 0);
            }
            if (e != hipSuccess) {
                err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
                return -1;
            }
            c.busy = true;
            ptr = c.ptr;
            cached = true;
            return 0;
        }
    }
    // above the cache limit, or the cached buffer is held by another host
    // thread's call on this stream
    hipMemPool_t pool = nullptr;
    if (scratch_pool(pool, err) != 0) {
        return -1;
    }
    e = hipMallocFromPoolAsync(&ptr, bytes, pool, s);
    if (e != hipSuccess) {
        ptr = nullptr;
        err = std::string("scratch allocation failed: ") + hipGetErrorString(e);
        return -1;
    }
    pooled = true;
    return 0;
}

StreamScratch::~StreamScratch() {
    if (cached) {
        // every kernel that uses the buffer has been enqueued on `stream`
        std::lock_guard<std::mutex> lock(g_pool_mu);
        CachedScratch& c = g_cache[std::make_tuple(device, stream, static_cast<int>(use))];
        (void)hipEventRecord(c.last_use, stream);
        c.busy = false;
    } else if (pooled && ptr != nullptr) {
        (void)hipFreeAsync(ptr, stream);
    }
}

int rope_rotate_k(const AttnArgs& a, void* dst, hipStream_t stream, std::string& err) {
    const int64_t n_chunks = (int64_t)a.B * a.Hkv * a.Sk * (a.D / 8);
    if (n_chunks == 0) {
        return 0;
    }
    const int64_t blocks64 = (n_chunks + 255) / 256;
    const uint32_t blocks = (uint32_t)(blocks64 < 65536 ? blocks64 : 65536);
    hipLaunchKernelGGL(rope_rotate_rows, dim3(blocks), dim3(256), 0, stream, static_cast<const _Float16*>(a.k),
                       static_cast<_Float16*>(dst), a.rot_cos, a.rot_sin, a.ks[0], a.ks[1], a.ks[2], a.Hkv, a.Sk, a.D,
                       n_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    return 0;
}

} // namespace rdna_amd
