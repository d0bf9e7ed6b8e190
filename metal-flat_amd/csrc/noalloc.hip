// SPDX-License-Identifier: Apache-2.0
// noalloc.hip -- device scratch of the allocation-free search entry point.
//
// The array below exists once in every GPU's copy of this library's device
// code. In host code its name is only a host-side stand-in: its device address
// on the current GPU comes from hipGetSymbolAddress, resolved once per device
// and kept, and only that address is ever handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdexcept>
#include <string>

#include "noalloc.hpp"

namespace mflat_amd {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex gMu;
void* gAddr[kNoAllocMaxDevices] = {};
}  // namespace

void* noalloc_scratch(int device) {
    if (device < 0 || device >= kNoAllocMaxDevices)
        throw std::runtime_error("allocation-free search: device " + std::to_string(device) + " out of range");
    std::lock_guard<std::mutex> lk(gMu);
    if (!gAddr[device]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess || cur != device)
            throw std::runtime_error("allocation-free search: the index's device is not current");
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            throw std::runtime_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        gAddr[device] = p;
    }
    return gAddr[device];
}

}  // namespace mflat_amd
