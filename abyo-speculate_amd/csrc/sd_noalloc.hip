// Scratch memory of the allocation-free entry points: one file-scope device
// array per GPU (each device that loads the library holds its own copy until
// the process ends).  Host code never passes the array's name to a kernel or
// a copy -- in host code that name is only a stand-in for the symbol -- but
// the device address that hipGetSymbolAddress returns for the current
// device, resolved once per device and kept here.
#include <mutex>
#include <vector>

#include "sd_kernels.hpp"

namespace sd {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

void *noalloc_scratch(int device) {
    static std::mutex mu;
    static std::vector<void *> ptr;  // per device ordinal
    std::lock_guard<std::mutex> lock(mu);
    if ((size_t)device < ptr.size() && ptr[device]) return ptr[device];
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) throw BackendError(std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (cur != device) throw BackendError("noalloc_scratch: the device must be current");
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) throw BackendError(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    if ((size_t)device >= ptr.size()) ptr.resize(device + 1, nullptr);
    ptr[device] = p;
    return p;
}

}  // namespace sd
