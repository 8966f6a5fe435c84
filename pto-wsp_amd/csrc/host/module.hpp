// Codegen IR consumed by the HIP backend: tensors, kernel definitions and
// the workload tree, parsed from the "PTOWSP-MODULE 1" text written by
// pto_wsp/ir_bridge.py.
//
// Mirrors the reference's codegen attachments (include/pto/wsp/ir/codegen.hpp:22-77)
// and the workload/axis/schedule nodes the cpu_sim emitter walks
// (include/pto/wsp/ir/workload.hpp:15-54,92,119; axis.hpp:12-50;
// schedule.hpp:13-36,211-231).  Extensions: affine and indirect index
// expressions, and loop extents read from an int32 tensor element.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "scalar.hpp"

namespace ptowsp {

enum class DType : int { F16, BF16, F32, F64, I8, I16, I32, I64, U8, U16, U32, U64, Bool };

const char* dtype_name(DType d);
int dtype_size(DType d);
bool dtype_is_float(DType d);

struct CompileError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

struct TensorInfo {
    DType dtype = DType::F32;
    std::vector<int64_t> shape;
};

struct ValueInfo {
    int id = 0;
    DType dtype = DType::F32;
    bool tile = false;
    int rows = 0, cols = 0;
};

struct ParamInfo {
    std::string name;
    int id = 0;
    std::string direction;
};

enum class OpKind {
    Load, Store, Add, Sub, Mul, Div, Max, Min, Exp, Rsqrt, RowSum, RowMax, RowMean, Matmul, Constant,
    // Top-k helpers of the tracer (python/pto_wsp/kernel.py:689-724) and the
    // PTO-ISA kernel surface (python/pto_wsp/ptoisa_jit.py:187-258): IOTA_U32,
    // TSORT32, the index extraction, TMOV, store_topk_indices_i32 and
    // cpu_sim_add_cycles.
    IotaU32, TSort32, ExtractTopkIndices, TMov, StoreTopkIndices, CpuSimAddCycles,
    Other
};

struct OpInfo {
    OpKind kind = OpKind::Other;
    std::string kind_name;
    int result = -1;  // -1: no result
    std::vector<int> operands;
    bool has_value = false;
    double value = 0.0;
    std::map<std::string, int64_t> ints;  // integer attrs (cols, k, cycles)
    std::shared_ptr<const SExpr> cycles_expr;  // CpuSimAddCycles: cycles as an expression of the kernel's scalars
};

struct KernelDef {
    std::string name;
    std::vector<ValueInfo> values;
    std::vector<ParamInfo> params;
    std::vector<OpInfo> ops;
    bool custom = false;
    std::string custom_src;  // cpp_src: a C++ body over the task descriptor; cpp_tu_path: a whole file
    bool custom_tu = false;  // custom_src is a translation unit defining extern "C" <name>(task, cspt)
};

struct IndexExpr {
    char kind = 'c';  // v: loop var, c: constant, a: affine, t: element of an int32 tensor
    std::string var;
    int64_t c = 0;
    std::vector<std::pair<std::string, int64_t>> terms;  // affine
    int tid = -1, base_rank = 0;                          // indirect
    std::vector<IndexExpr> idx;                           // indirect
};

struct ArgRef {
    char kind = 'c';  // v: loop var, c: literal u64, s: runtime symbol
    std::string var;
    uint64_t u64 = 0;
};

struct TensorArg {
    std::string param;
    int tid = 0, base_rank = 0, view_rank = 0;
    std::vector<IndexExpr> idx;
};

enum class AxisKind { Dense, Dyn, Ragged, DynTensor, Select };

struct Axis {
    AxisKind kind = AxisKind::Dense;
    int64_t size = 0;
    // Dyn: runtime key (a); Ragged: outer / lengths symbol names (a, b);
    // Select: CSR outer-size / indptr / indices symbol names (a, b, c).
    std::string a, b, c;
    IndexExpr expr;    // DynTensor: the i32 element holding the extent
    int64_t max = 0;   // DynTensor: declared upper bound of the extent
};

enum class NodeKind { Empty, ParallelFor, ForEach, Combine, Sequential, Task, Select, Cond, SlotSet, SlotLoad };

struct Node {
    NodeKind kind = NodeKind::Empty;
    std::string var;
    Axis axis;
    std::unique_ptr<Node> body;
    std::vector<std::unique_ptr<Node>> kids;
    // task
    std::string kernel;
    int kernel_index = -1;
    std::vector<ArgRef> axis_args, scalar_args;
    std::vector<TensorArg> tensor_args;
    // cond: the predicate; kids[0] / kids[1] are the then / else branches
    std::unique_ptr<SExpr> pred;
    // slot set / slot load: slot index, value to set, or the tile view and
    // the (row, col) element of it to load
    uint32_t slot = 0;
    uint64_t value = 0;
    TensorArg view;
    int64_t row = 0, col = 0;
};

struct Schedule {
    bool has_dispatch = false;
    std::string dispatch_policy;
    std::unique_ptr<SExpr> dispatch_key;  // affinity / hash / dispatch_by: worker = key % workers
    int64_t num_targets = 0;
    bool has_window = false;
    int64_t window_size = 0;
    std::string window_unit, window_overflow;
    bool has_streams = false;
    int64_t num_streams = 0;
    bool stream_keyed = false;
};

struct Module {
    std::string name;
    std::vector<TensorInfo> tensors;
    std::vector<KernelDef> kernels;
    std::string workload_name;
    std::unique_ptr<Node> root;
    Schedule schedule;
};

Module parse_module(const std::string& text);

uint64_t fnv1a_64(const std::string& s);

}  // namespace ptowsp
