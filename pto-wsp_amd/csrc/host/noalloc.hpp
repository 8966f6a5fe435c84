// Fixed device scratch for the no-allocation launch (noalloc.hip).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>

namespace ptowsp {

// Size of the per-device scratch array.  Layout used by a no-allocation run:
//   [0, 256)            the kernels' error flag (int at offset 0);
//   [256, 256 + 16 KiB) decode unit counters (kDecodeMaxUnits int32);
//   then the device-resident loop-extent tensors the cycle model reads;
//   then the decode partials.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
constexpr size_t kNoAllocHeaderBytes = 256;

// Set-up, run by every allocating launch (cheap after the first on a
// device): looks up this device's scratch address with hipGetSymbolAddress
// and runs the zeroing kernel once on it, so that the library's code object
// is loaded and the array is resident before any no-allocation run.
void noalloc_prepare(hipStream_t stream);

// Device address of this device's scratch array, as found by
// noalloc_prepare; throws when no allocating launch has prepared it.
void* noalloc_scratch();

// Zeroes `bytes` (a multiple of 4) at dev_ptr with a small kernel on `stream`.
void noalloc_zero(void* dev_ptr, size_t bytes, hipStream_t stream);

}  // namespace ptowsp
