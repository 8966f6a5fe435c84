// hiprtc compilation of emitted kernels for gfx950, with an in-process and
// an on-disk code-object cache keyed by a hash of source + options.
#pragma once

#include <hip/hip_runtime_api.h>

#include <string>
#include <vector>

namespace ptowsp {

struct JitKernel {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
};

// Compiles (or fetches from cache) and loads `source`, returning the kernel
// named `entry`.  Loaded modules live until the process exits.
const JitKernel& jit_kernel(const std::string& source, const std::string& entry);

// The kernel if `source` is already loaded in this process, else null
// (neither compiles nor loads anything).
const JitKernel* jit_loaded(const std::string& source, const std::string& entry);

// Compiles without loading (no GPU needed); returns the code object bytes.
std::vector<char> jit_compile(const std::string& source);

std::string jit_cache_dir();

}  // namespace ptowsp
