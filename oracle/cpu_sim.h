/* CPU oracle for the PTO-WSP data-parallel tile path.  TEST INFRASTRUCTURE:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, as the checker.  It is never part of the product path.
 *
 * pto_cpusim_run() executes a serialized workload module (the text that the
 * Python bridge pto_wsp.ir_bridge writes, format "PTOWSP-MODULE 1") the way
 * the reference's generated cpu_sim artifact does:
 *   - loop nest, task argument packing and tile view addressing:
 *       src/python/pto_codegen.cpp:2222-2709
 *   - per-op tile semantics of the generated kernels:
 *       src/python/pto_codegen.cpp:471-1241
 *   - cpu_sim cycle counting (valid_rows*valid_cols per tile op, m*k*n per
 *     TMATMUL): include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:54-303
 *   - in-order, window-stall scheduler giving total_cycles (the makespan):
 *       src/python/pto_codegen.cpp:1561-1607
 *   - ragged / sparse-select loops, cond nodes with ScalarExpr predicates,
 *     slot set / load, keyed dispatch (key % lanes):
 *       src/python/pto_codegen.cpp:220-300, 2248-2478, 2679-2690
 *   - cpp_src kernels: called through ctx->get_kernel with the reference's
 *     task descriptor; the caller compiles the bodies (oracle/runner.py)
 * The pto-isa submodule that implements the tile instructions is absent
 * from the reference checkout, so reductions are restated as sequential
 * fp32 sums, TEXP as expf, TRSQRT as 1/sqrtf and TMATMUL as a sequential
 * fp32 dot product; their exact rounding order is "parity unpinned" beyond
 * the tolerances of the reference's own examples.
 */
#ifndef PTOWSP_CPU_SIM_H
#define PTOWSP_CPU_SIM_H

#include <stdint.h>

#include "ptowsp_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Runs the module.  Returns 0 on success and stores the model makespan in
 * *total_cycles; returns -1 on error (message in pto_cpusim_last_error()). */
int pto_cpusim_run(const char* module_text, RuntimeContext* ctx, uint64_t* total_cycles);

/* Number of tasks executed by the last successful run. */
uint64_t pto_cpusim_last_task_count(void);

const char* pto_cpusim_last_error(void);

/* Evaluates one scalar expression in the module's token form (a cond
 * predicate or dispatch key) with symbols and slots read through ctx and no
 * loop variable or task in scope.  Returns 0 and stores the value's bits and
 * its C type ('b' bool, 'i' int64_t, 'u' uint64_t); -1 on error. */
int pto_cpusim_eval_scalar(const char* expr_text, RuntimeContext* ctx, uint64_t* value, char* type);

#ifdef __cplusplus
}
#endif

#endif
