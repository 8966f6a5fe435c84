// Reference-side half of the "hip_gfx950" target: what a maintainer adds to
// the reference's codegen (src/python/pto_codegen.cpp, compile_codegen at
// :3352-3434) so that compile_codegen(module, {target = "hip_gfx950"}) returns
// an artifact that the unchanged CodegenExecutable loader
// (src/python/pto_codegen.cpp:3510-3576) runs on libptowsp_hip.so.
//
// Builds against the reference's IR headers (include/pto/wsp/ir/*.hpp,
// C++20) and this repository's include/ptowsp_hip.h.
#pragma once

#include <cstdint>
#include <string>

#include "pto/wsp/ir/module.hpp"

namespace ptowsp_integration {

// The module in the "PTOWSP-MODULE 1" text that ptowsp_hip_compile reads:
// tensor table, kernels (CodegenKernelDef), module.workloads[0] with its
// codegen bindings and the schedule of that workload, the same content and
// order as pto_wsp/ir_bridge.py writes from Python.  Throws
// std::runtime_error for nodes the target does not run (Call, CSP pipelines,
// a Sparse axis outside select, C++ include lists on cpp_src kernels).
std::string write_ptowsp_module_text(const pto::wsp::ir::Module& module);

// Where the artifact of one module lives and what CodegenExecutable calls.
struct HipArtifact {
    std::string so_path;     // shared object exporting `entrypoint`
    std::string entrypoint;  // uint64_t <name>_main(RuntimeContext*, CSPTContext*)
    std::string cache_key;   // hex FNV-1a-64 of the module text and the library path
};

// Writes the entry shim of one module (its text embedded, forwarding to
// ptowsp_hip_compile + ptowsp_hip_workload_main) under
// <cache_root>/<name>_hip_<key>/ and compiles it with the host C compiler
// ($PTO_WSP_CODEGEN_CC, default "cc"), linked to libptowsp_hip.so in
// `lib_dir`.  An existing artifact with the same key is reused.  Throws
// std::runtime_error with the compiler output on failure.
HipArtifact build_hip_artifact(const std::string& module_text, const std::string& module_name,
                               const std::string& cache_root, const std::string& include_dir, const std::string& lib_dir);

// A C string literal (with escapes) holding `s`.
std::string c_string_literal(const std::string& s);

// FNV-1a-64 of `s` (the reference's symbol-id hash, src/python/pto_codegen.cpp:118-125).
uint64_t fnv1a_64(const std::string& s);

}  // namespace ptowsp_integration
