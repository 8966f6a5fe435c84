// A foreign loader for hip_gfx950 artifacts, built against the reference's
// artifact ABI (include/pto/wsp/codegen/abi/workload_abi.hpp): it plays the
// reference's CodegenRuntime / CodegenExecutable
// (src/python/pto_codegen.cpp:3453-3576) with RuntimeContext callbacks of its
// own over host buffers, dlopens the artifact and calls
// `uint64_t <module>_main(RuntimeContext*, CSPTContext*)`.
//
//   abi_main_driver <artifact.so> <entrypoint> <manifest>
//
// Manifest lines:
//   tensor <id> <element bytes> <ndim> <dims...> <strides...> <file>
//                                                         the tensor's buffer (element strides of
//                                                         the view into it); written back to <file>.out
//   axis <name> <value>
//   symu <id> <value>
//   symp <id> <count> <file>                              int32 array
// Prints "total_cycles <n>" (0 and the library's message on failure).
#include <dlfcn.h>

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iostream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "pto/wsp/codegen/abi/workload_abi.hpp"

namespace {

struct Tensor {
    std::vector<char> data;
    std::vector<int64_t> dims;
    std::vector<int64_t> strides;
    int esize = 0;
    std::string file;
};

struct Runtime {
    std::map<uint32_t, Tensor> tensors;
    std::map<std::string, int64_t> axis;
    std::map<uint64_t, uint64_t> symu;
    std::map<uint64_t, std::vector<int32_t>> symp;
    uint64_t slots[256] = {};
};

int64_t get_axis_size(void* c, const char* name) {
    auto& r = *static_cast<Runtime*>(c);
    auto it = r.axis.find(name ? name : "");
    return it == r.axis.end() ? 0 : it->second;
}
uint64_t get_symbol_u64(void* c, uint64_t id) {
    auto& r = *static_cast<Runtime*>(c);
    auto it = r.symu.find(id);
    return it == r.symu.end() ? 0 : it->second;
}
void* get_symbol_ptr(void* c, uint64_t id) {
    auto& r = *static_cast<Runtime*>(c);
    auto it = r.symp.find(id);
    return it == r.symp.end() ? nullptr : it->second.data();
}
uint64_t get_slot_u64(void* c, uint32_t i) { return i < 256 ? static_cast<Runtime*>(c)->slots[i] : 0; }
void set_slot_u64(void* c, uint32_t i, uint64_t v) {
    if (i < 256) static_cast<Runtime*>(c)->slots[i] = v;
}
void* get_tensor_ptr(void* c, uint32_t tid) {
    auto& r = *static_cast<Runtime*>(c);
    auto it = r.tensors.find(tid);
    return it == r.tensors.end() ? nullptr : it->second.data.data();
}
// Element strides of the view (as numpy gives them to the reference's CodegenRuntime).
uint64_t get_tensor_stride(void* c, uint32_t tid, uint32_t dim) {
    auto& r = *static_cast<Runtime*>(c);
    auto it = r.tensors.find(tid);
    if (it == r.tensors.end() || dim >= it->second.strides.size()) return 0;
    return static_cast<uint64_t>(it->second.strides[dim]);
}
KernelFn get_kernel(void*, uint32_t) { return nullptr; }

std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    return std::vector<char>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 4) {
        std::cerr << "usage: abi_main_driver <artifact.so> <entrypoint> <manifest>\n";
        return 2;
    }
    try {
        Runtime rt;
        std::ifstream mf(argv[3]);
        std::string line;
        while (std::getline(mf, line)) {
            std::istringstream is(line);
            std::string kind;
            if (!(is >> kind)) continue;
            if (kind == "tensor") {
                uint32_t id;
                Tensor t;
                int nd;
                is >> id >> t.esize >> nd;
                t.dims.resize(nd);
                t.strides.resize(nd);
                for (auto& d : t.dims) is >> d;
                for (auto& st : t.strides) is >> st;
                is >> t.file;
                t.data = read_file(t.file);
                // Every element the view addresses lies in the buffer.
                int64_t last = 0;
                bool empty = false;
                for (int d = 0; d < nd; ++d) {
                    if (t.dims[d] == 0) empty = true;
                    else last += (t.dims[d] - 1) * t.strides[d];
                }
                if (!empty && (last + 1) * t.esize > static_cast<int64_t>(t.data.size()))
                    throw std::runtime_error("buffer too small for the view of " + t.file);
                rt.tensors[id] = std::move(t);
            } else if (kind == "axis") {
                std::string name;
                int64_t v;
                is >> name >> v;
                rt.axis[name] = v;
            } else if (kind == "symu") {
                uint64_t id, v;
                is >> id >> v;
                rt.symu[id] = v;
            } else if (kind == "symp") {
                uint64_t id;
                size_t n;
                std::string file;
                is >> id >> n >> file;
                const auto raw = read_file(file);
                std::vector<int32_t> v(n);
                if (raw.size() != n * 4) throw std::runtime_error("size mismatch for " + file);
                std::copy(raw.begin(), raw.end(), reinterpret_cast<char*>(v.data()));
                rt.symp[id] = std::move(v);
            } else {
                throw std::runtime_error("bad manifest line: " + line);
            }
        }
        void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
        if (!h) throw std::runtime_error(std::string("dlopen: ") + dlerror());
        auto fn = reinterpret_cast<WorkloadFn>(dlsym(h, argv[2]));
        if (!fn) throw std::runtime_error(std::string("dlsym: ") + dlerror());
        RuntimeContext ctx{};
        ctx.get_axis_size = get_axis_size;
        ctx.get_symbol_u64 = get_symbol_u64;
        ctx.get_symbol_ptr = get_symbol_ptr;
        ctx.get_slot_u64 = get_slot_u64;
        ctx.set_slot_u64 = set_slot_u64;
        ctx.get_tensor_ptr = get_tensor_ptr;
        ctx.get_tensor_stride = get_tensor_stride;
        ctx.get_kernel = get_kernel;
        ctx.ctx = &rt;
        const uint64_t cycles = fn(&ctx, nullptr);
        std::cout << "total_cycles " << cycles << std::endl;
        if (cycles == 0) {
            using ErrFn = const char* (*)();
            if (auto err = reinterpret_cast<ErrFn>(dlsym(h, "ptowsp_hip_last_error"))) std::cout << "error " << err() << std::endl;
            return 1;
        }
        for (auto& [id, t] : rt.tensors) {
            std::ofstream o(t.file + ".out", std::ios::binary);
            o.write(t.data.data(), static_cast<std::streamsize>(t.data.size()));
        }
        for (uint32_t i = 0; i < 256; ++i)
            if (rt.slots[i]) std::cout << "slot " << i << " " << rt.slots[i] << std::endl;
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "abi_main_driver: " << e.what() << "\n";
        return 1;
    }
}
