// SPDX-License-Identifier: Apache-2.0
// noalloc.hpp -- the device scratch of the allocation-free search entry point.
//
// mflat_flat_search_device_noalloc serves callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). Its per-search workspace lives in one statically sized
// device array per GPU (noalloc.hip), so the call itself allocates nothing;
// every call on a GPU shares that GPU's array, so calls that overlap on one
// GPU race.
#pragma once

#include <cstddef>

namespace mflat_amd {

constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;   // per GPU, held until the process ends
constexpr int kNoAllocMaxQ = 16;                           // queries per call
constexpr int kNoAllocMaxDim = 2048;                       // dimension of the index (and the tile's LDS)
constexpr int kNoAllocMaxDevices = 64;

// Device address of `device`'s scratch array (kNoAllocScratchBytes). The first
// call for a device resolves it with hipGetSymbolAddress, which needs that
// device current; later calls return the kept address. Throws if the runtime
// cannot resolve it.
void* noalloc_scratch(int device);

}  // namespace mflat_amd
