#include "jit.hpp"

#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>

#include "module.hpp"

namespace ptowsp {

namespace {

// Device headers embedded at build time (generated from csrc/device/*.h).
#include "device_headers.inc"

const char* kOptions[] = {
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
};

// Headers a cpp_tu_path translation unit includes, as device code: the task
// descriptor and timing context of the reference's
// include/pto/wsp/codegen/abi/kernel_abi.hpp:21-71 (same layouts; the file
// is compiled with every unannotated function as host and device code, so
// PTO_WSP_KERNEL_ATTR stays empty), the
// PTO_WSP_ADVANCE macro and pto::cpu_sim cycle counter of
// include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:33-64 (one counter per
// launcher thread, zeroed when the launch starts; the PTO-ISA tile API that
// header also pulls in is not provided), and the <cstdint> / <cstddef> names.
const char kStdTypes[] = R"(#pragma once
typedef __hip_internal::int8_t int8_t; typedef __hip_internal::int16_t int16_t;
typedef __hip_internal::int32_t int32_t; typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint8_t uint8_t; typedef __hip_internal::uint16_t uint16_t;
typedef __hip_internal::uint32_t uint32_t; typedef __hip_internal::uint64_t uint64_t;
typedef __SIZE_TYPE__ size_t; typedef __PTRDIFF_TYPE__ ptrdiff_t;
namespace std { using ::int8_t; using ::int16_t; using ::int32_t; using ::int64_t; using ::uint8_t; using ::uint16_t;
                using ::uint32_t; using ::uint64_t; using ::size_t; using ::ptrdiff_t; }
)";
const char kKernelAbi[] = R"(#pragma once
#include <cstdint>
#include <cstddef>
#define PTO_WSP_KERNEL_ATTR
extern "C" {
struct KernelTaskDesc {
    const uint64_t* args;
    uint32_t num_args;
    uint32_t num_axis_args;
    void* const* tensor_ptrs;
    const uint64_t* tensor_strides;
    uint32_t num_tensors;
    uint32_t kernel_id;
    uint32_t task_id;
};
struct TimingConfig {
    uint64_t loop_overhead;
    uint64_t dispatch_overhead;
    uint64_t channel_latency;
};
struct CSPTContext {
    void* ctx;
    void (*advance_cycles)(void* ctx, uint64_t cycles);
    uint64_t (*get_time)(void* ctx);
    const TimingConfig* timing;
};
typedef uint64_t (*KernelFn)(const KernelTaskDesc* task, CSPTContext* cspt);
}
)";
const char kPtoisaBridge[] = R"(#pragma once
#include "pto/wsp/codegen/abi/kernel_abi.hpp"
#define PTO_WSP_ADVANCE(cspt_ptr, cycles_expr) \
    do { \
        if ((cspt_ptr) && (cspt_ptr)->advance_cycles && (cycles_expr) != 0) \
            (cspt_ptr)->advance_cycles((cspt_ptr)->ctx, static_cast<uint64_t>(cycles_expr)); \
    } while (0)
namespace pto { namespace cpu_sim {
__device__ inline uint64_t& ptowsp_cycle_counter() {
    __shared__ uint64_t c[64];
    return c[threadIdx.x & 63];
}
__device__ inline void reset_cycles() { ptowsp_cycle_counter() = 0; }
__device__ inline void add_cycles(uint64_t cycles) { ptowsp_cycle_counter() += cycles; }
__device__ inline uint64_t read_cycles() { return ptowsp_cycle_counter(); }
} }
)";
constexpr const char* kTuMarker = "// ptowsp: cpp_tu\n";

std::string options_key() {
    std::string s;
    for (const char* o : kOptions) s += std::string(o) + " ";
    int major = 0, minor = 0;
    hiprtcVersion(&major, &minor);
    return s + std::to_string(major) + "." + std::to_string(minor);
}

std::string hex64(uint64_t v) {
    char buf[17];
    std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(v));
    return buf;
}

std::mutex g_mu;
std::map<std::string, std::unique_ptr<JitKernel>> g_loaded;

bool read_file(const std::string& path, std::vector<char>& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    return !out.empty();
}

void mkdirs(const std::string& dir) {
    std::string cur;
    std::stringstream ss(dir);
    std::string part;
    if (!dir.empty() && dir[0] == '/') cur = "/";
    while (std::getline(ss, part, '/')) {
        if (part.empty()) continue;
        cur += part + "/";
        ::mkdir(cur.c_str(), 0755);
    }
}

}  // namespace

std::string jit_cache_dir() {
    if (const char* p = std::getenv("PTO_WSP_CODEGEN_CACHE_DIR"); p && *p) return std::string(p) + "/hip";
    const char* home = std::getenv("HOME");
    return std::string(home && *home ? home : "/tmp") + "/.cache/pto_wsp/hip";
}

std::vector<char> jit_compile(const std::string& source) {
    hiprtcProgram prog = nullptr;
    const char* headers[] = {kDeviceHeader, kLaunchHeader, kKernelAbi, kPtoisaBridge, kStdTypes, kStdTypes, kStdTypes, kStdTypes};
    const char* names[] = {"ptowsp_device.h", "ptowsp_launch.h", "pto/wsp/codegen/abi/kernel_abi.hpp",
                           "pto/wsp/codegen/abi/ptoisa_bridge.hpp", "cstdint", "cstddef", "stdint.h", "stddef.h"};
    const int nh = source.rfind(kTuMarker, 0) == 0 ? 8 : 2;
    if (hiprtcCreateProgram(&prog, source.c_str(), "ptowsp_kernel.hip", nh, headers, names) != HIPRTC_SUCCESS)
        throw CompileError("hiprtcCreateProgram failed");
    const int nopt = static_cast<int>(sizeof(kOptions) / sizeof(kOptions[0]));
    hiprtcResult rc = hiprtcCompileProgram(prog, nopt, kOptions);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        throw CompileError("hiprtc failed to compile a kernel for gfx950:\n" + log + "\n--- source ---\n" + source);
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    std::vector<char> code(n);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    return code;
}

namespace {
std::string source_key(const std::string& source) {
    std::string h = source + "\n" + options_key() + "\n" + kDeviceHeader + kLaunchHeader;
    if (source.rfind(kTuMarker, 0) == 0) h += std::string(kKernelAbi) + kPtoisaBridge + kStdTypes;
    return hex64(fnv1a_64(h));
}
}  // namespace

const JitKernel* jit_loaded(const std::string& source, const std::string& entry) {
    const std::string key = source_key(source);
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_loaded.find(key + entry);
    return it == g_loaded.end() ? nullptr : it->second.get();
}

const JitKernel& jit_kernel(const std::string& source, const std::string& entry) {
    const std::string key = source_key(source);
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_loaded.find(key + entry);
    if (it != g_loaded.end()) return *it->second;

    const std::string dir = jit_cache_dir();
    const std::string path = dir + "/" + key + ".hsaco";
    std::vector<char> code;
    if (!read_file(path, code)) {
        code = jit_compile(source);
        mkdirs(dir);
        const std::string tmp = path + ".tmp" + std::to_string(::getpid());
        {
            std::ofstream f(tmp, std::ios::binary);
            f.write(code.data(), static_cast<std::streamsize>(code.size()));
        }
        std::rename(tmp.c_str(), path.c_str());
    }
    auto k = std::make_unique<JitKernel>();
    hipError_t e = hipModuleLoadData(&k->module, code.data());
    if (e != hipSuccess) throw std::runtime_error(std::string("hipModuleLoadData: ") + hipGetErrorString(e));
    e = hipModuleGetFunction(&k->function, k->module, entry.c_str());
    if (e != hipSuccess) throw std::runtime_error(std::string("hipModuleGetFunction: ") + hipGetErrorString(e));
    auto& ref = *k;
    g_loaded.emplace(key + entry, std::move(k));
    return ref;
}

}  // namespace ptowsp
