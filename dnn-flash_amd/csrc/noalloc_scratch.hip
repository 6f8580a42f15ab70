// Device scratch of the allocation-free entry point (ofh_attention_fwd_noalloc):
// a file-scope device array that every GPU the library runs on holds from the
// code object's load until the process ends. Its device address is looked up
// once per device with hipGetSymbolAddress (with that device current) and kept;
// kernels receive that address, never the array's host-side name.
//
// Every call on one GPU shares the array, which keeps the last call's contents:
// the kernels that use it (block-mask tile lists, key-split partial rows) write
// every value they read in the same call, so nothing needs clearing. Calls that
// overlap on one GPU (other streams, other host threads) race on it.

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "ofh_kernels.h"

namespace ofh {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_mu;
std::map<int, void*> g_addr;  // device -> address of its copy of `scratch`

}  // namespace

hipError_t noalloc_scratch(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_addr.find(dev);
    if (it == g_addr.end()) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        it = g_addr.emplace(dev, p).first;
    }
    *ptr = it->second;
    return hipSuccess;
}

}  // namespace ofh
