// Workload tree -> ordered launches, plus the cpu_sim cycle model.
//
// Device mapping (MI355X-first):
//   * P() loops that enclose a task map to the launch grid (their product is
//     the task count of the launch);
//   * a P.seq chain that ends in a single task runs inside the kernel, in
//     order, so InOut accumulators stay on chip;
//   * any other P.seq loop is a host loop around the launches of its body;
//   * combine / sequential children become consecutive launches on one
//     stream (program order, as the reference artifact executes them).
// P() iterations are independent by contract (a parallel grid,
// python/pto_wsp/p_namespace.py:230-233 of the reference), which is what
// makes grid mapping and loop fission valid.
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "analysis.hpp"
#include "module.hpp"

namespace ptowsp {

struct LoopSpec {
    std::string var;
    const Axis* axis = nullptr;
};

struct LaunchSpec {
    int kernel = -1;
    const Node* task = nullptr;
    std::vector<LoopSpec> grid;    // outer -> inner
    std::vector<LoopSpec> inner;   // in-kernel sequential loops, outer -> inner
    std::vector<const TensorArg*> targs;  // by tensor ordinal
};

struct PlanItem {
    bool is_loop = false;
    int launch = -1;
    LoopSpec loop;
    std::vector<PlanItem> body;
};

struct Plan {
    std::vector<LaunchSpec> launches;
    std::vector<PlanItem> items;
};

Plan build_plan(const Module& m, const std::vector<KernelAnalysis>& ka);

// Resolves run-time quantities for the cycle model: DenseDyn sizes, symbols
// and int32 elements of index tensors.
struct CycleEnv {
    std::function<int64_t(const std::string&)> axis_size;
    std::function<uint64_t(uint64_t)> symbol_u64;
    std::function<const int32_t*(uint64_t)> symbol_ptr;
    std::function<int64_t(const IndexExpr&, const std::vector<std::pair<std::string, int64_t>>&)> index_value;
};

struct CycleResult {
    uint64_t total_cycles = 0;
    uint64_t tasks = 0;
};

// In-order, window-stall makespan over dispatch lanes
// (src/python/pto_codegen.cpp:1561-1607, 2305-2700).
CycleResult run_cycle_model(const Module& m, const std::vector<KernelAnalysis>& ka, const CycleEnv& env);

}  // namespace ptowsp
