// The scratch region of rdna_attention_forward_noalloc: a file-scope device
// array, so that entry point allocates nothing.
//
// Each GPU the library runs on holds its own copy of `scratch` (kNoAllocBytes)
// from the first use of the library's code on that device until the process
// ends.  In host code the array's name is only a stand-in, never a device
// address: the address is looked up once per device with
// hipGetSymbolAddress, with that device current, and only that pointer is
// handed to kernels.  Every call on a device shares the array (it keeps the
// last call's contents; the kernels that use it overwrite what they read),
// so calls that overlap on one device -- concurrent streams, or a second call
// before the first has finished on another stream -- race.
#include "fa_internal.hpp"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>

namespace rdna_amd {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

} // namespace

int noalloc_region(ScratchRegion& r, std::string& err) {
    static std::mutex mu;
    static std::map<int, char*> addr; // device -> address of its scratch array; guarded by mu
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        err = std::string("no-allocation scratch: ") + hipGetErrorString(e);
        return -1;
    }
    std::lock_guard<std::mutex> lock(mu);
    auto it = addr.find(dev);
    if (it == addr.end()) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            err = std::string("no-allocation scratch: hipGetSymbolAddress failed: ") +
                  (e != hipSuccess ? hipGetErrorString(e) : "null address");
            return -1;
        }
        it = addr.emplace(dev, static_cast<char*>(p)).first;
    }
    r.base = it->second;
    r.bytes = kNoAllocBytes;
    r.used = 0;
    return 0;
}

} // namespace rdna_amd
