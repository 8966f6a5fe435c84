// Workload tree -> ordered launches, plus the cpu_sim cycle model.
//
// Device mapping (MI355X-first):
//   * P() loops that enclose a task map to the launch grid (their product is
//     the task count of the launch);
//   * a P.seq chain that ends in a single task runs inside the kernel, in
//     order, so InOut accumulators stay on chip;
//   * any other P.seq loop is a host loop around the launches of its body;
//   * combine / sequential children become consecutive launches on one
//     stream (program order, as the reference artifact executes them);
//   * a cond whose predicate reads a grid loop variable becomes a task mask
//     on the launches of both branches (the host evaluates it per task and
//     launches only the tasks it keeps); any other cond, slot set and slot
//     load is a host step between launches;
//   * a P() loop whose body sets or loads a slot is a host loop, so that
//     every iteration sees the slot values its predecessors left.
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

// A task runs only where `pred` evaluates to `want`.
struct Mask {
    const SExpr* pred = nullptr;
    bool want = true;
};

struct LaunchSpec {
    int kernel = -1;
    const Node* task = nullptr;
    std::vector<LoopSpec> grid;    // outer -> inner
    std::vector<LoopSpec> inner;   // in-kernel sequential loops, outer -> inner
    std::vector<const TensorArg*> targs;  // by tensor ordinal
    std::vector<Mask> masks;              // conjunction; empty: every task of the grid
};

struct PlanItem {
    bool is_loop = false;
    int launch = -1;
    LoopSpec loop;
    std::vector<PlanItem> body;
    // A host step: a cond evaluated on the host (body = then, alt = else), a
    // slot set or a slot load.
    const Node* ctl = nullptr;
    std::vector<PlanItem> alt;
};

struct Plan {
    std::vector<LaunchSpec> launches;
    std::vector<PlanItem> items;
};

Plan build_plan(const Module& m, const std::vector<KernelAnalysis>& ka);

using VarList = std::vector<std::pair<std::string, int64_t>>;

// Resolves run-time quantities for the cycle model: DenseDyn sizes, symbols,
// int32 elements of index tensors, the slots at the start of the run and the
// value each slot load reads (in program order).
struct CycleEnv {
    std::function<int64_t(const std::string&)> axis_size;
    std::function<uint64_t(uint64_t)> symbol_u64;
    std::function<const int32_t*(uint64_t)> symbol_ptr;
    std::function<int64_t(const IndexExpr&, const VarList&)> index_value;
    std::function<uint64_t(uint32_t)> slot_init;
    std::function<uint64_t(const Node&, const VarList&)> slot_load;
    // Cycles a cpp_src kernel's task reported when it ran on the device.
    std::function<uint64_t(const Node&, const VarList&)> custom_cycles;
};

// The scalar-expression environment over loop variables `vars` (innermost
// last) and the given symbol and slot readers.
SEnv scalar_env(const VarList& vars, std::function<uint64_t(uint64_t)> symbol, std::function<uint64_t(uint32_t)> slot);

// True when the module needs the slot machinery or run-time predicates
// (cond, slot set / load, a dispatch key): their cycle counts are not cached.
bool module_is_dynamic(const Module& m);
bool module_loads_slots(const Module& m);

struct CycleResult {
    uint64_t total_cycles = 0;
    uint64_t tasks = 0;
};

// In-order, window-stall makespan over dispatch lanes
// (src/python/pto_codegen.cpp:1561-1607, 2305-2700).
CycleResult run_cycle_model(const Module& m, const std::vector<KernelAnalysis>& ka, const CycleEnv& env);

}  // namespace ptowsp
