/* C ABI of the PTO-WSP HIP backend (libptowsp_hip.so) for one MI355X GPU.
 *
 * It is the drop-in for the reference's codegen plugin boundary: a loader
 * that today calls compile_codegen() and then dlopens the artifact and
 * calls `<module>_main(RuntimeContext*, CSPTContext*)` calls these entry
 * points instead.  Plain pointers and sizes only; the structures come from
 * ptowsp_abi.h (layouts identical to the reference artifact ABI).
 *
 * Threading: one program may be used by one thread at a time; different
 * programs are independent.  Errors: functions returning int give 0 on
 * success and -1 on failure, with the message in ptowsp_hip_last_error().
 */
#ifndef PTOWSP_HIP_H
#define PTOWSP_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "ptowsp_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ptowsp_program ptowsp_program;
typedef struct ptowsp_runtime ptowsp_runtime;

typedef struct ptowsp_run_info {
    uint64_t total_cycles; /* cpu_sim cycle-model makespan (ProgramStats.total_cycles) */
    uint64_t task_count;   /* tasks executed */
    uint32_t launches;     /* kernel launches enqueued */
    uint32_t reserved;
} ptowsp_run_info;

typedef struct ptowsp_timing {
    double device_ms; /* first launch start .. last launch end (HIP events on the stream) */
    double h2d_ms;    /* staging of host-resident tensors into HBM */
    double d2h_ms;    /* copy-back of written host-resident tensors */
} ptowsp_timing;

/* Replaces compile_codegen(module, CompileOptions{target}) for the target
 * "hip_gfx950" (reference src/python/pto_codegen.cpp:3352-3434; called from
 * python/pto_wsp/program.py:437-454).  `module_text` is the serialized
 * module written by pto_wsp.ir_bridge.workload_to_codegen_ir (the reference
 * passes the pybind ir::Module built by python/pto_wsp/ir_bridge.py:112-139).
 * Parses, validates and plans the workload; kernels are emitted and built
 * with hiprtc for gfx950 on first use (cached on disk). */
int ptowsp_hip_compile(const char* module_text, ptowsp_program** out);

/* Replaces the artifact entry `uint64_t <module>_main(RuntimeContext*, CSPTContext*)`
 * (reference include/pto/wsp/codegen/abi/workload_abi.hpp:71, driven by
 * CodegenExecutable::run_with_symbols, src/python/pto_codegen.cpp:3542-3566).
 * Synchronous: runs every launch on the null stream and returns after all
 * outputs (including host-resident ones) are written.  Returns the cycle-model
 * makespan, or 0 on failure (see ptowsp_hip_last_error).  `cspt` is unused,
 * as in the reference's cpu_sim path. */
uint64_t ptowsp_hip_workload_main(ptowsp_program* prog, RuntimeContext* ctx, CSPTContext* cspt);

/* Non-blocking run behind Program.execute() (reference python/pto_wsp/program.py:670-733):
 * stages host-resident tensors, enqueues every launch on `hip_stream`
 * (a hipStream_t, may be NULL) and returns.  When a loop extent is read from
 * a device-resident tensor, that tensor is copied asynchronously and the
 * cycle model runs in ptowsp_hip_synchronize: info->total_cycles is then
 * UINT64_MAX and ptowsp_hip_run_result gives it after the synchronize (the
 * reference also fills ProgramStats.total_cycles only when the run thread
 * ends, python/pto_wsp/program.py:721-733).  `ctx` must stay valid until
 * the synchronize. */
int ptowsp_hip_launch(ptowsp_program* prog, RuntimeContext* ctx, void* hip_stream, ptowsp_run_info* info);

/* No counterpart in the reference.  For callers that cannot allocate memory
 * (tight serving loops, harnesses that forbid hipMalloc): the same run as
 * ptowsp_hip_launch, allocating no device or pinned memory and loading no
 * code objects.  The decode kernels' unit counters and partials, the
 * kernels' error flag and the copy of device-resident loop-extent tensors
 * use a fixed device scratch of 16 MiB per GPU (held until the process
 * ends); a run that needs more is refused with an error before its decode
 * launch.  Requirements: every tensor is device memory; each launch's
 * kernel was already built and loaded by an earlier ptowsp_hip_launch of
 * the same program (same bindings), which also resolves the device's
 * scratch and loads the kernel that clears it (without one on this device
 * the call is refused); no cpp_src kernels, slot loads, masked
 * (cond-on-grid) launches or tile programs whose tiles exceed LDS (those
 * keep tiles in an allocated global scratch).  It is not made for HIP stream capture: it
 * records timing events and may read index tensors with synchronous
 * copies.  All no-allocation runs on one GPU share its scratch: runs that
 * overlap in time on one GPU race and must not be issued.  Finish with
 * ptowsp_hip_synchronize as usual; device time is reported only when an
 * earlier ptowsp_hip_launch created the program's timing events. */
int ptowsp_hip_launch_noalloc(ptowsp_program* prog, RuntimeContext* ctx, void* hip_stream, ptowsp_run_info* info);

/* Cycle model result of the last synchronized run (new: pairs with the
 * deferred total_cycles of ptowsp_hip_launch).  -1 while a run is pending. */
int ptowsp_hip_run_result(const ptowsp_program* prog, ptowsp_run_info* info);

/* Program.synchronize() (reference python/pto_wsp/program.py:735-743): waits
 * for the last launch, copies written host-resident tensors back, and
 * reports device errors (which the reference has no channel for). */
int ptowsp_hip_synchronize(ptowsp_program* prog, ptowsp_timing* timing);

/* Error message of the last failing call on this thread (new: the
 * reference's run path has no error channel). */
const char* ptowsp_hip_last_error(void);

/* Frees the program and its staging buffers. */
void ptowsp_hip_release(ptowsp_program* prog);

/* Introspection. */
int ptowsp_hip_num_launches(const ptowsp_program* prog);
/* cpu_sim cycles of one task of `kernel` (reference
 * include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:54-303), or UINT64_MAX. */
uint64_t ptowsp_hip_kernel_cycles(const ptowsp_program* prog, const char* kernel);
/* Family chosen for `kernel`: 0 row program, 1 tile program, 2 gemm, 3 decode (online
 * softmax over pages); -1 unknown. */
int ptowsp_hip_kernel_family(const ptowsp_program* prog, const char* kernel);
/* Emits and builds every launch for contiguous row-major tensors without
 * touching a GPU (hiprtc only); returns the source of launch `index` through
 * `source`, valid until the next call.  flags bit 0: build the variant that
 * runs all tasks of a launch in program order (used when grid tasks write
 * overlapping memory), with bits 8-15 the grid variables (bit 8 + v) looped in
 * program order inside each workgroup while the others are decoded from the
 * group index (0: all of them, one workgroup); bit 1: build GEMM launches with 2x2 neighbouring tasks
 * of the last two grid loops merged into one workgroup block; bit 2 (with bit
 * 1): build merged 128x128 tasks with K step 32 or 64 as the two-group
 * ping-pong GEMM block; bit 4: build row-program launches with in-kernel
 * loops as row programs that run the loops inside each row's lane team;
 * bit 5: build decode launches with the following `out = o / l` launch
 * folded into them (the form a run uses when that launch follows). */
int ptowsp_hip_precompile(ptowsp_program* prog, int index, int flags, const char** source);

/* Evaluates only the cpu_sim cycle model (total_cycles, task_count) for the
 * bindings in `ctx`, on the host, without launching anything. */
int ptowsp_hip_cycle_model(ptowsp_program* prog, RuntimeContext* ctx, ptowsp_run_info* info);

/* Runtime tables that back a RuntimeContext, the equivalent of the
 * reference's CodegenRuntime (src/python/pto_codegen.cpp:3453-3508):
 * tensors (pointer + element strides), DenseDyn axis sizes by name, u64 and
 * pointer symbols by FNV-1a-64 id, and 256 zeroed u64 slots. */
ptowsp_runtime* ptowsp_rt_create(void);
void ptowsp_rt_destroy(ptowsp_runtime* rt);
int ptowsp_rt_set_tensor(ptowsp_runtime* rt, uint32_t tensor_id, void* ptr, uint32_t ndim, const int64_t* strides);
int ptowsp_rt_set_axis_size(ptowsp_runtime* rt, const char* name, int64_t size);
int ptowsp_rt_set_symbol_u64(ptowsp_runtime* rt, uint64_t symbol_id, uint64_t value);
int ptowsp_rt_set_symbol_ptr(ptowsp_runtime* rt, uint64_t symbol_id, void* ptr);
void ptowsp_rt_clear(ptowsp_runtime* rt);
/* Zeroes the 256 slots: the reference's CodegenRuntime starts every run with
 * fresh zeroed slots (src/python/pto_codegen.cpp:3546-3550); call it before
 * each ptowsp_hip_launch to get the same. */
int ptowsp_rt_reset_slots(ptowsp_runtime* rt);
RuntimeContext* ptowsp_rt_context(ptowsp_runtime* rt);

#ifdef __cplusplus
}
#endif

#endif /* PTOWSP_HIP_H */
