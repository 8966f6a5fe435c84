// Test tool for the reference-side writer (pto-wsp_amd/integration/hip_target.cpp),
// built against the reference's IR headers:
//   ir_cases write <case>                       module text of a case built as a reference ir::Module
//   ir_cases build <text> <name> <cache_root> <include_dir> <lib_dir>
//                                               the case's hip_gfx950 artifact (prints so_path and entrypoint)
// The cases are ir::Modules built with the reference's IRFactory as its Python
// bridge would build them (python/pto_wsp/ir_bridge.py:112-139) for the
// workloads of tests/workloads.py: "quickstart" (the README rmsnorm),
// "bgemm_f16" (examples/bgemm) and "slot_branch"
// (tests/test_codegen_slots_tensor_predicate.py with compute kernels).
#include <fstream>
#include <iostream>
#include <sstream>

#include "hip_target.hpp"

namespace ir = pto::wsp::ir;
using ptowsp_integration::fnv1a_64;

namespace {

ir::IRFactory F;

ir::CodegenIndexExpr var(const std::string& v) {
    ir::CodegenIndexExpr e;
    e.is_var = true;
    e.var = v;
    return e;
}
ir::CodegenIndexExpr cst(int64_t c) {
    ir::CodegenIndexExpr e;
    e.constant = c;
    return e;
}
ir::CodegenAxisArg avar(const std::string& v) {
    ir::CodegenAxisArg a;
    a.is_var = true;
    a.var = v;
    return a;
}
ir::CodegenAxisArg acst(uint64_t u) {
    ir::CodegenAxisArg a;
    a.u64 = u;
    return a;
}
ir::CodegenTensorArg targ(const std::string& p, uint32_t tid, int base_rank, std::vector<ir::CodegenIndexExpr> idx) {
    ir::CodegenTensorArg t;
    t.param = p;
    t.tensor_id = tid;
    t.base_rank = base_rank;
    t.view_rank = 2;
    t.index_exprs = std::move(idx);
    return t;
}
ir::CodegenTensorInfo tensor(ir::DType d, std::vector<int64_t> shape) {
    ir::CodegenTensorInfo t;
    t.dtype = d;
    t.shape = std::move(shape);
    return t;
}
void val(ir::CodegenKernelDef& k, int id, ir::DType d, int r = 0, int c = 0) {
    ir::CodegenKernelValueInfo v;
    v.dtype = d;
    v.has_shape = r > 0;
    v.rows = r;
    v.cols = c;
    k.values[id] = v;
}
void param(ir::CodegenKernelDef& k, const std::string& n, int id) { k.params.push_back({n, id}); }
void op(ir::CodegenKernelDef& k, const std::string& kind, int res, std::vector<int> opnds, ir::AttrMap attrs = {}) {
    ir::CodegenKernelOpInfo o;
    o.kind = kind;
    o.has_result = res > 0;
    o.result = res > 0 ? res : 0;
    o.operands = std::move(opnds);
    o.attrs = std::move(attrs);
    k.ops.push_back(o);
}
ir::AttrMap store_attrs() { return {{"offset", std::vector<int64_t>{0, 0}}}; }

ir::ScheduleDef rr4(const std::string& wl) {
    ir::ScheduleDef s;
    s.name = wl + "_schedule";
    s.workload_name = wl;
    s.level = ir::WorkloadLevel::CPU;
    s.directives.push_back(F.create<ir::DispatchNode>(ir::DispatchPolicy::RoundRobin, 4));
    s.directives.push_back(F.create<ir::TaskWindowNode>(8192, "tasks", ir::TaskWindowOverflowPolicy::Stall));
    return s;
}

ir::IRPtr<ir::WorkloadNode> pfor(const std::string& v, int64_t n, ir::IRPtr<ir::WorkloadNode> body) {
    return F.create<ir::ParallelForNode>(F.create<ir::DenseAxisNode>(n), v, std::move(body));
}

ir::Module quickstart() {
    ir::Module m;
    m.name = "quickstart";
    m.tensors = {tensor(ir::DType::F32, {1, 2, 16, 128}), tensor(ir::DType::F32, {1, 2, 16, 128})};
    ir::CodegenKernelDef k;
    k.name = "rmsnorm_tile";
    val(k, 1, ir::DType::F32, 16, 128);
    val(k, 2, ir::DType::F32, 16, 128);
    val(k, 3, ir::DType::F32, 16, 128);
    val(k, 4, ir::DType::F32, 16, 1);
    val(k, 5, ir::DType::F32, 16, 1);
    val(k, 6, ir::DType::F32, 16, 128);
    param(k, "x", 1);
    param(k, "out", 2);
    op(k, "Mul", 3, {1, 1});
    op(k, "RowMean", 4, {3});
    op(k, "Rsqrt", 5, {4});
    op(k, "Mul", 6, {1, 5});
    op(k, "Store", 0, {2, 6}, store_attrs());
    m.kernels = {k};
    auto task = F.create<ir::TaskNode>("rmsnorm_tile", std::vector<std::string>{"b", "h"}, std::vector<std::string>{"x", "out"},
                                       std::vector<ir::CodegenAxisArg>{avar("b"), avar("h")}, std::vector<ir::CodegenAxisArg>{},
                                       std::vector<ir::CodegenTensorArg>{targ("x", 0, 4, {var("b"), var("h")}),
                                                                          targ("out", 1, 4, {var("b"), var("h")})});
    ir::WorkloadDef w;
    w.name = "unnamed";
    w.level = ir::WorkloadLevel::CPU;
    w.body = pfor("b", 1, pfor("h", 2, task));
    m.workloads = {w};
    m.schedules = {rr4(w.name)};
    return m;
}

ir::Module bgemm_f16() {
    ir::Module m;
    m.name = "bgemm_f16";
    m.tensors = {tensor(ir::DType::F16, {1, 4, 4, 16, 16}), tensor(ir::DType::F16, {1, 4, 4, 16, 16}),
                 tensor(ir::DType::F32, {1, 4, 4, 16, 16})};
    ir::CodegenKernelDef k;
    k.name = "gemm_tile";
    val(k, 1, ir::DType::F16, 16, 16);
    val(k, 2, ir::DType::F16, 16, 16);
    val(k, 3, ir::DType::F32, 16, 16);
    val(k, 4, ir::DType::F32, 16, 16);
    val(k, 5, ir::DType::F32, 16, 16);
    param(k, "a_tile", 1);
    param(k, "b_tile", 2);
    param(k, "c_tile", 3);
    op(k, "Matmul", 4, {1, 2});
    op(k, "Add", 5, {3, 4});
    op(k, "Store", 0, {3, 5}, store_attrs());
    m.kernels = {k};
    auto task = F.create<ir::TaskNode>(
        "gemm_tile", std::vector<std::string>{"b", "h", "s", "i"}, std::vector<std::string>{"a_tile", "b_tile", "c_tile"},
        std::vector<ir::CodegenAxisArg>{avar("b"), avar("h"), avar("s"), avar("i")}, std::vector<ir::CodegenAxisArg>{},
        std::vector<ir::CodegenTensorArg>{
            [] { auto t = targ("a_tile", 0, 5, {var("b"), var("h"), var("i")}); return t; }(),
            [] { auto t = targ("b_tile", 1, 5, {var("b"), var("s"), var("i")}); return t; }(),
            [] { auto t = targ("c_tile", 2, 5, {var("b"), var("h"), var("s")}); return t; }()});
    auto kloop = F.create<ir::ForEachNode>(F.create<ir::DenseAxisNode>(4), "i", task);
    ir::WorkloadDef w;
    w.name = "unnamed";
    w.level = ir::WorkloadLevel::CPU;
    w.body = pfor("b", 1, pfor("h", 4, pfor("s", 4, kloop)));
    m.workloads = {w};
    m.schedules = {rr4(w.name)};
    return m;
}

ir::CodegenKernelDef fill(const std::string& name, double value) {
    ir::CodegenKernelDef k;
    k.name = name;
    val(k, 1, ir::DType::I32, 1, 1);
    val(k, 2, ir::DType::I32, 1, 1);
    val(k, 3, ir::DType::I32);
    val(k, 4, ir::DType::I32, 1, 1);
    val(k, 5, ir::DType::I32);
    val(k, 6, ir::DType::I32, 1, 1);
    param(k, "y_out", 1);
    op(k, "Load", 2, {1}, store_attrs());
    op(k, "Constant", 3, {}, {{"value", 0.0}});
    op(k, "Mul", 4, {2, 3});
    op(k, "Constant", 5, {}, {{"value", value}});
    op(k, "Add", 6, {4, 5});
    op(k, "Store", 0, {1, 6}, store_attrs());
    return k;
}

ir::Module slot_branch() {
    ir::Module m;
    m.name = "slot_branch";
    m.tensors = {tensor(ir::DType::I32, {1, 1, 1, 1}), tensor(ir::DType::I32, {1, 1, 1, 1}), tensor(ir::DType::I32, {1, 1, 1, 1})};
    ir::CodegenKernelDef wf;
    wf.name = "write_flag";
    val(wf, 1, ir::DType::I32, 1, 1);
    val(wf, 2, ir::DType::I32, 1, 1);
    val(wf, 3, ir::DType::I32, 1, 1);
    param(wf, "x_in", 1);
    param(wf, "flag_out", 2);
    op(wf, "Load", 3, {1}, store_attrs());
    op(wf, "Store", 0, {2, 3}, store_attrs());
    m.kernels = {fill("fill_false", 3.0), fill("fill_true", 7.0), wf};
    using Args = std::vector<ir::CodegenAxisArg>;
    using Strs = std::vector<std::string>;
    auto write = F.create<ir::TaskNode>("write_flag", Strs{"0"}, Strs{"x_in", "flag_out"}, Args{acst(0)}, Args{},
                                        std::vector<ir::CodegenTensorArg>{targ("x_in", 0, 4, {cst(0), cst(0)}),
                                                                           targ("flag_out", 1, 4, {cst(0), cst(0)})});
    auto load = F.create<ir::SlotLoadU64Node>(0, targ("", 1, 4, {cst(0), cst(0)}), 0, 0);
    auto t = F.create<ir::TaskNode>("fill_true", Strs{"0"}, Strs{"y_out"}, Args{acst(0)}, Args{},
                                    std::vector<ir::CodegenTensorArg>{targ("y_out", 2, 4, {cst(0), cst(0)})});
    auto f = F.create<ir::TaskNode>("fill_false", Strs{"0"}, Strs{"y_out"}, Args{acst(0)}, Args{},
                                    std::vector<ir::CodegenTensorArg>{targ("y_out", 2, 4, {cst(0), cst(0)})});
    // slot_u64(0) != 0
    ir::ScalarExpr pred = std::make_shared<ir::BinaryExpr>(ir::ScalarBinaryOp::Ne, std::make_shared<ir::SlotExpr>(0, ir::ScalarType::U64),
                                                           std::make_shared<ir::LiteralI64Expr>(0), ir::ScalarType::Bool);
    auto c = F.create<ir::CondNode>("slot_u64(0) != 0", pred, t, f);
    ir::WorkloadDef w;
    w.name = "slot_tensor_predicate";
    w.level = ir::WorkloadLevel::CPU;
    w.body = F.create<ir::SequentialNode>(std::vector<ir::IRPtr<ir::WorkloadNode>>{write, load, c});
    m.workloads = {w};
    return m;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const std::string mode = argc > 1 ? argv[1] : "";
        if (mode == "write" && argc == 3) {
            const std::string c = argv[2];
            ir::Module m = c == "quickstart" ? quickstart() : c == "bgemm_f16" ? bgemm_f16() : c == "slot_branch" ? slot_branch() : ir::Module{};
            if (m.name.empty()) throw std::runtime_error("unknown case " + c);
            std::cout << ptowsp_integration::write_ptowsp_module_text(m);
            return 0;
        }
        if (mode == "build" && argc == 7) {
            std::ifstream f(argv[2], std::ios::binary);
            std::stringstream ss;
            ss << f.rdbuf();
            const auto a = ptowsp_integration::build_hip_artifact(ss.str(), argv[3], argv[4], argv[5], argv[6]);
            std::cout << a.so_path << "\n" << a.entrypoint << "\n" << a.cache_key << "\n";
            return 0;
        }
        std::cerr << "usage: ir_cases write <case> | build <text> <name> <cache_root> <include_dir> <lib_dir>\n";
        return 2;
    } catch (const std::exception& e) {
        std::cerr << "ir_cases: " << e.what() << "\n";
        return 1;
    }
}
