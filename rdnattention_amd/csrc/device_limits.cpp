// Device occupancy queries for the persistent kernels.
#include "fa_internal.hpp"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <utility>

namespace rdna_amd {

int64_t resident_workgroups(const void* kernel, int threads, std::string& err) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, int64_t> cache; // guarded by mu
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = cache.find({dev, kernel});
        if (it != cache.end()) {
            return it->second;
        }
    }
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) {
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0);
    }
    if (e != hipSuccess) {
        err = hipGetErrorString(e);
        return -1;
    }
    if (cus <= 0 || per_cu <= 0) {
        err = "kernel does not fit on a compute unit";
        return -1;
    }
    const int64_t n = (int64_t)cus * per_cu;
    std::lock_guard<std::mutex> lock(mu);
    cache[{dev, kernel}] = n;
    return n;
}

} // namespace rdna_amd
