/* Artifact C ABI shared by the HIP backend (libptowsp_hip.so) and the CPU
 * oracle: the structures a workload entry point receives.
 *
 * The layouts are kept identical to the reference's artifact ABI so that a
 * loader written for it (src/python/pto_codegen.cpp:3453-3576) can drive this
 * backend unchanged:
 *   KernelTaskDesc  include/pto/wsp/codegen/abi/kernel_abi.hpp:21-41
 *   TimingConfig /
 *   CSPTContext     include/pto/wsp/codegen/abi/kernel_abi.hpp:47-60
 *   RuntimeContext  include/pto/wsp/codegen/abi/workload_abi.hpp:17-41
 *   WorkloadFn      include/pto/wsp/codegen/abi/workload_abi.hpp:71
 *
 * Pointer semantics on this backend: get_tensor_ptr may return host memory
 * (staged through HBM by the backend) or device memory (used in place);
 * get_tensor_stride returns element strides; get_symbol_ptr returns host
 * memory (int32 arrays for ragged lengths).
 */
#ifndef PTOWSP_ABI_H
#define PTOWSP_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct KernelTaskDesc {
    const uint64_t* args;
    uint32_t num_args;
    uint32_t num_axis_args;
    void* const* tensor_ptrs;
    const uint64_t* tensor_strides;
    uint32_t num_tensors;
    uint32_t kernel_id;
    uint32_t task_id;
} KernelTaskDesc;

typedef struct TimingConfig {
    uint64_t loop_overhead;
    uint64_t dispatch_overhead;
    uint64_t channel_latency;
} TimingConfig;

typedef struct CSPTContext {
    void* ctx;
    void (*advance_cycles)(void* ctx, uint64_t cycles);
    uint64_t (*get_time)(void* ctx);
    const TimingConfig* timing;
} CSPTContext;

typedef uint64_t (*KernelFn)(const KernelTaskDesc* task, CSPTContext* cspt);

typedef struct RuntimeContext {
    int64_t (*get_axis_size)(void* ctx, const char* name);
    uint64_t (*get_symbol_u64)(void* ctx, uint64_t symbol_id);
    void* (*get_symbol_ptr)(void* ctx, uint64_t symbol_id);
    uint64_t (*get_slot_u64)(void* ctx, uint32_t slot);
    void (*set_slot_u64)(void* ctx, uint32_t slot, uint64_t value);
    void* (*get_tensor_ptr)(void* ctx, uint32_t tensor_id);
    uint64_t (*get_tensor_stride)(void* ctx, uint32_t tensor_id, uint32_t dim);
    KernelFn (*get_kernel)(void* ctx, uint32_t kernel_id);
    void* ctx;
} RuntimeContext;

typedef uint64_t (*WorkloadFn)(RuntimeContext* ctx, CSPTContext* cspt);

#ifdef __cplusplus
}
#endif

#endif /* PTOWSP_ABI_H */
