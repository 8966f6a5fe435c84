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
    const char* headers[] = {kDeviceHeader, kLaunchHeader};
    const char* names[] = {"ptowsp_device.h", "ptowsp_launch.h"};
    if (hiprtcCreateProgram(&prog, source.c_str(), "ptowsp_kernel.hip", 2, headers, names) != HIPRTC_SUCCESS)
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
    return hex64(fnv1a_64(source + "\n" + options_key() + "\n" + kDeviceHeader + kLaunchHeader));
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
