// Device scratch of ptowsp_hip_launch_noalloc: a file-scope device array, so
// that the entry point never allocates device or pinned memory.
//
// Host code never passes the array's name to a kernel or a copy: in host code
// that name stands for a host-side shadow, not a device address.  The device
// address is looked up once per device with hipGetSymbolAddress, and only
// that pointer is used.  Every GPU holds its own copy of the array, at its own
// address, for the life of the process; every no-allocation run on a GPU
// shares it and finds whatever the previous run left there.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <stdexcept>
#include <string>

#include "noalloc.hpp"

namespace {

static __device__ __align__(256) unsigned char scratch[ptowsp::kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};
std::atomic<bool> g_ready[kMaxDevices] = {};

// Sets n 32-bit words to zero (a kernel rather than hipMemsetAsync: it
// allocates nothing and records no memset node if the stream is captured).
__global__ void zero_words(unsigned int* p, unsigned long long n) {
    for (unsigned long long i = blockIdx.x * static_cast<unsigned long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<unsigned long long>(gridDim.x) * blockDim.x)
        p[i] = 0u;
}

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

namespace ptowsp {

namespace {
int current_device() {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("no-allocation scratch: device index out of range");
    return dev;
}
}  // namespace

void noalloc_prepare(hipStream_t stream) {
    const int dev = current_device();
    if (g_ready[dev].load(std::memory_order_acquire)) return;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ready[dev].load(std::memory_order_relaxed)) return;
    void* p = nullptr;
    check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(no-allocation scratch)");
    if (!p) throw std::runtime_error("hipGetSymbolAddress(no-allocation scratch) returned a null address");
    // The zeroing kernel's first launch loads the code object; every
    // no-allocation run clears the words it needs again before use.
    noalloc_zero(p, 256, stream);
    g_ptr[dev] = p;
    g_ready[dev].store(true, std::memory_order_release);
}

void* noalloc_scratch() {
    const int dev = current_device();
    if (!g_ready[dev].load(std::memory_order_acquire))
        throw std::runtime_error(
            "ptowsp_hip_launch_noalloc: no ptowsp_hip_launch has run on this device yet (it resolves the fixed scratch and "
            "loads its kernel, which this entry point does not)");
    return g_ptr[dev];
}

void noalloc_zero(void* dev_ptr, size_t bytes, hipStream_t stream) {
    if (bytes % 4) throw std::runtime_error("noalloc_zero: size must be a multiple of 4 bytes");
    const unsigned long long n = bytes / 4;
    if (n == 0) return;
    const unsigned blocks = static_cast<unsigned>(n < 256ull * 64 ? (n + 255) / 256 : 64);
    hipLaunchKernelGGL(zero_words, dim3(blocks), dim3(256), 0, stream, static_cast<unsigned int*>(dev_ptr), n);
    check(hipGetLastError(), "zero_words launch");
}

}  // namespace ptowsp
