// Emits the HIP source of one launch.  The op-by-op lowering restates the
// reference kernel emitter's semantics (src/python/pto_codegen.cpp:471-1241):
// preloaded param tiles, TLOAD/TSTORE through strides s3/s4, the same
// broadcast rules, RowMean as a sum divided by the column count, Rsqrt as
// 1/sqrt, Matmul as an fp32 accumulation that ignores a third operand.
#include "emit.hpp"

#include <algorithm>
#include <cstdio>
#include <map>
#include <set>
#include <sstream>

#include "../device/ptowsp_launch.h"

namespace ptowsp {

namespace {

// Row pitch (floats) of tile_mma's per-wave operand scratch
// (kTileMmaPitch in ptowsp_device.h).
constexpr int kTileMmaPitchHost = 33;

std::string flt(double v) {
    char buf[64];
    std::snprintf(buf, sizeof buf, "%.17g", v);
    return std::string("((float)(") + buf + "))";
}

const char* op_functor(OpKind k) {
    switch (k) {
        case OpKind::Add: return "OpAdd";
        case OpKind::Sub: return "OpSub";
        case OpKind::Mul: return "OpMul";
        case OpKind::Div: return "OpDiv";
        case OpKind::Max: return "OpMax";
        case OpKind::Min: return "OpMin";
        default: return "OpAdd";
    }
}

int dt_code(DType d) { return static_cast<int>(d); }

// Kernel symbol of a launch: family and traced kernel name, so that profiler
// traces tell launches apart (kernel names are Python identifiers).
std::string entry_name(const char* family, const KernelDef& k) { return std::string("ptowsp_") + family + "_" + k.name; }

// Declarations of scalar params and Constant() values (:607-655).
void emit_scalars(std::ostringstream& o, const KernelAnalysis& a, bool int_ok) {
    const KernelDef& k = *a.def;
    for (size_t i = 0; i < k.params.size(); ++i) {
        const ValueInfo* v = a.by_id[k.params[i].id];
        if (v->tile) continue;
        const int so = a.scalar_ordinal[i];
        if (so >= kMaxScalars) throw CompileError("kernel " + k.name + ": too many scalar params");
        if (v->dtype == DType::F32)
            o << "  const float s" << v->id << " = bits_f32(A.scal[" << so << "]);\n";
        else if (!int_ok)
            throw CompileError("kernel " + k.name + ": integer scalars need the tile-program lowering");
        else if (v->dtype == DType::I32)
            o << "  const i64 s" << v->id << " = (i64)(int)(u32)A.scal[" << so << "];\n";
        else if (v->dtype == DType::I64)
            o << "  const i64 s" << v->id << " = (i64)A.scal[" << so << "];\n";
        else
            o << "  const i64 s" << v->id << " = A.scal[" << so << "] != 0ull ? 1 : 0;\n";
    }
    for (const auto& op : k.ops) {
        if (op.kind != OpKind::Constant || op.result <= 0) continue;
        const ValueInfo* v = a.by_id[op.result];
        if (v->tile || !op.has_value) continue;
        if (v->dtype == DType::F32) {
            o << "  const float s" << v->id << " = " << flt(op.value) << ";\n";
        } else {
            if (!int_ok) throw CompileError("kernel " + k.name + ": integer constants need the tile-program lowering");
            o << "  const i64 s" << v->id << " = (i64)(" << static_cast<long long>(op.value) << "LL);\n";
        }
    }
}

// vars[0..ng) from the task index t (mixed radix, innermost grid loop fastest).
void emit_decode(std::ostringstream& o, const std::string& ind, int ng, const std::string& t) {
    if (ng == 0) return;
    o << ind << "{ i64 q_ = " << t << ";\n";
    for (int v = ng - 1; v >= 1; --v)
        o << ind << "  vars[" << v << "] = q_ % A.ext[" << v << "]; q_ /= A.ext[" << v << "];\n";
    o << ind << "  vars[0] = q_; }\n";
}

// True when an index expression reads loop variable `var`.
bool reads_var(const IndexExpr& e, const std::string& var) {
    switch (e.kind) {
        case 'v': return e.var == var;
        case 'a':
            for (const auto& [n, c] : e.terms)
                if (n == var && c != 0) return true;
            return false;
        case 't':
            for (const auto& x : e.idx)
                if (reads_var(x, var)) return true;
            return false;
        default: return false;
    }
}

// Element offset expression of tensor ordinal p: affine part + indirect terms.
std::string offset_expr(int p, int nvars, int first_term, int nterms) {
    std::ostringstream e;
    e << "(i64)0";
    for (int v = 0; v < nvars; ++v) e << " + A.coef[" << p << "][" << v << "] * vars[" << v << "]";
    for (int k = 0; k < nterms; ++k) e << " + indirect_index(A, " << (first_term + k) << ", vars, " << nvars << ")";
    return e.str();
}

}  // namespace

RowLayout row_layout(int cols, int vw, int up_cap) {
    RowLayout l;
    l.vw = vw;
    const int n = cols / vw;
    int g = 1;
    while (g < 64 && n % (g * 2) == 0) g *= 2;
    l.g = g;
    l.nv = n / g;
    int up = 32 / (l.nv * vw);
    if (up_cap < 1) up_cap = 1;
    l.up = up < 1 ? 1 : (up > up_cap ? up_cap : up);
    return l;
}

namespace {

// ---------------------------------------------------------------------------
// Row programs
// ---------------------------------------------------------------------------
EmittedKernel emit_row(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    (void)m;
    const KernelDef& k = *a.def;
    const RowLayout lay = row_layout(a.cols, spec.vec_width, spec.row_up);
    const char* nt = spec.nontemporal ? ", true" : "";
    const int R = a.rows, C = a.cols, ng = static_cast<int>(L.grid.size());
    const int rpw = 64 / lay.g, ch = rpw * lay.up;
    const bool chunk_in_task = R % ch == 0;
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    auto cls = [&](int id) { return a.row_class[id]; };
    auto vname = [&](int id) { return (a.by_id[id]->tile ? "v" : "s") + std::to_string(id); };
    auto tord = [&](int id) { return a.tensor_ordinal[a.param_of[id]]; };
    // Row loops: the in-kernel loops run inside each row's lane team; params
    // they do not move are read once / accumulated in registers.
    const int ni = spec.row_loops ? static_cast<int>(L.inner.size()) : 0;
    const int nvars = ng + ni;
    std::vector<bool> moving(ntens, false);
    for (int p = 0; p < ntens; ++p)
        for (int i = 0; i < ni; ++i)
            for (const auto& e : L.targs[p]->idx) moving[p] = moving[p] || reads_var(e, L.inner[i].var);
    auto base = [&](int p) {
        return moving[p] ? "(tb" + std::to_string(p) + "[u] + io" + std::to_string(p) + ")" : "tb" + std::to_string(p) + "[u]";
    };

    // Accumulators under row loops (params that the loops do not move and
    // that are stored) live in the register ld<param id> across the
    // iterations.  A Load op of such a param reads that register: its result
    // is a copy taken at the start of each iteration (before the iteration's
    // store, which the admission check guarantees), not a load from memory.
    auto is_acc = [&](int p) { return ni > 0 && !moving[p] && a.stored[p]; };
    std::vector<std::pair<int, int>> acc_loads;  // Load result id, param id
    std::vector<bool> acc_read(ntens, false);
    for (const auto& op : k.ops)
        if (op.kind == OpKind::Load && is_acc(tord(op.operands[0]))) {
            acc_loads.emplace_back(op.result, op.operands[0]);
            acc_read[tord(op.operands[0])] = true;
        }

    // Values loaded up front: preloaded params, accumulators read through a
    // Load op, and the other Load results.
    std::vector<std::pair<int, int>> loads;  // value id, tensor ordinal
    for (size_t i = 0; i < k.params.size(); ++i) {
        const ValueInfo* v = a.by_id[k.params[i].id];
        if (v->tile && (a.preload[v->id] || acc_read[a.tensor_ordinal[i]])) loads.emplace_back(v->id, a.tensor_ordinal[i]);
    }
    for (const auto& op : k.ops)
        if (op.kind == OpKind::Load && !is_acc(tord(op.operands[0]))) loads.emplace_back(op.result, tord(op.operands[0]));

    // A stored tensor that is also read: wait for outstanding loads before stores.
    std::set<int> read_t, stored_t;
    for (const auto& [id, p] : loads)
        if (!ni || moving[p]) read_t.insert(L.targs[p]->tid);
    for (int p = 0; p < ntens; ++p)
        if (a.stored[p] && (!ni || moving[p])) stored_t.insert(L.targs[p]->tid);
    bool rw_alias = false;
    for (int t : stored_t)
        if (read_t.count(t)) rw_alias = true;

    EmittedKernel ek;
    ek.row_program = true;
    ek.threads = 256;
    ek.waves_per_block = 4;
    ek.rows_per_chunk = ch;
    std::ostringstream o;
    o << "#include \"ptowsp_device.h\"\nusing namespace ptowsp;\n";
    o << "// row program: kernel " << k.name << ", rows " << R << " x cols " << C << ", vw " << lay.vw << "\n";
    ek.entry = entry_name("row", k);
    o << "extern \"C\" __global__ void __launch_bounds__(256) " << ek.entry << "(const LaunchArgs A) {\n";
    o << "  constexpr int R = " << R << ", NV = " << lay.nv << ", VW = " << lay.vw << ", G = " << lay.g
      << ", UP = " << lay.up << ";\n";
    o << "  constexpr int RPW = 64 / G, CH = RPW * UP, WPB = 4;\n";
    o << "  typedef RowSlice<NV, VW> RS;\n";
    o << "  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, team = lane / G, j = lane % G;\n";
    o << "  (void)team; (void)j;\n";
    emit_scalars(o, a, false);
    o << "  const i64 total = A.ntasks * R;\n";
    o << "  const i64 nch = (total + CH - 1) / CH;\n";
    o << "  i64 vars[" << (nvars > 0 ? nvars : 1) << "];\n  (void)vars;\n";
    o << "  for (i64 ch = (i64)blockIdx.x * WPB + wave; ch < nch; ch += (i64)gridDim.x * WPB) {\n";
    o << "    int rr[UP]; bool ok[UP];\n";
    for (int p = 0; p < ntens; ++p) o << "    char* tb" << p << "[UP];\n";
    if (chunk_in_task) {
        o << "    const i64 t = (ch * CH) / R;\n    const int r0 = (int)(ch * CH - t * R);\n";
        emit_decode(o, "    ", ng, spec.task_list ? "A.tlist[t]" : "t");
        for (int p = 0; p < ntens; ++p) {
            const int es = dtype_size(a.by_id[k.params[a.tensor_param_index[p]].id]->dtype);
            o << "    char* b" << p << " = A.base[" << p << "] + (" << offset_expr(p, ng, 0, 0) << ") * " << es << ";\n";
        }
        o << "#pragma unroll\n    for (int u = 0; u < UP; ++u) {\n      rr[u] = r0 + u * RPW + team; ok[u] = true;\n";
        for (int p = 0; p < ntens; ++p) o << "      tb" << p << "[u] = b" << p << ";\n";
        o << "    }\n";
    } else {
        o << "#pragma unroll\n    for (int u = 0; u < UP; ++u) {\n";
        o << "      i64 g = ch * CH + u * RPW + team; ok[u] = g < total; if (!ok[u]) g = 0;\n";
        o << "      const i64 t = g / R; rr[u] = (int)(g - t * R);\n";
        emit_decode(o, "      ", ng, spec.task_list ? "A.tlist[t]" : "t");
        for (int p = 0; p < ntens; ++p) {
            const int es = dtype_size(a.by_id[k.params[a.tensor_param_index[p]].id]->dtype);
            o << "      tb" << p << "[u] = A.base[" << p << "] + (" << offset_expr(p, ng, 0, 0) << ") * " << es << ";\n";
        }
        o << "    }\n";
    }
    // Store of value `val` (f32) into param `dparam` (tensor ordinal p) at
    // base pointer `basep`, with the f16 / bf16 store cast for a 16-bit param.
    auto store_row = [&](const std::string& ind, int p, int dparam, const std::string& basep, const std::string& val, bool full) {
        const DType dt = a.by_id[dparam]->dtype;
        const std::string ps = std::to_string(p);
        if (full && dt == DType::F32)
            o << ind << "if (ok[u]) row_store<NV, VW, G" << nt << ">((float*)" << basep << " + (i64)rr[u] * A.s3[" << ps << "], " << val
              << ", A.s4[" << ps << "], j);\n";
        else if (full)
            o << ind << "if (ok[u]) row_store_h<NV, VW, G, " << dt_code(dt) << ">((u16*)" << basep << " + (i64)rr[u] * A.s3[" << ps
              << "], " << val << ", A.s4[" << ps << "], j);\n";
        else if (dt == DType::F32)
            o << ind << "if (ok[u] && j == 0) ((float*)" << basep << ")[(i64)rr[u] * A.s3[" << ps << "]] = " << val << ";\n";
        else
            o << ind << "if (ok[u] && j == 0) ((u16*)" << basep << ")[(i64)rr[u] * A.s3[" << ps << "]] = f32_to_h16_bits<" << dt_code(dt)
              << ">(" << val << ");\n";
    };
    // Phase 1: every load of the chunk, so UP*NV vector loads per value are in flight.
    std::string ind1 = "    ";
    auto phase1 = [&](bool want_moving) {
    for (const auto& [id, p] : loads) {
        if (ni && moving[p] != want_moving) continue;
        const std::string tbp = base(p);
        switch (cls(id)) {
            case RowClass::Full:
                o << ind1 << "RS ld" << id << "[UP];\n#pragma unroll\n" << ind1 << "for (int u = 0; u < UP; ++u) row_load<NV, VW, G" << nt << ">(ld" << id
                  << "[u], (const float*)" << tbp << " + (i64)rr[u] * A.s3[" << p << "], A.s4[" << p << "], j);\n";
                break;
            case RowClass::RowVec:
                o << ind1 << "float ld" << id << "[UP];\n#pragma unroll\n" << ind1 << "for (int u = 0; u < UP; ++u) ld" << id
                  << "[u] = ((const float*)" << tbp << ")[(i64)rr[u] * A.s3[" << p << "]];\n";
                break;
            case RowClass::RowVecT:
                o << ind1 << "float ld" << id << "[UP];\n#pragma unroll\n" << ind1 << "for (int u = 0; u < UP; ++u) ld" << id
                  << "[u] = ((const float*)" << tbp << ")[(i64)rr[u] * A.s4[" << p << "]];\n";
                break;
            case RowClass::ColVec:
                o << ind1 << "RS ld" << id << "[UP];\n#pragma unroll\n" << ind1 << "for (int u = 0; u < UP; ++u) row_load<NV, VW, G>(ld" << id
                  << "[u], (const float*)" << tbp << ", A.s4[" << p << "], j);\n";
                break;
            case RowClass::ColVecT:
                o << ind1 << "RS ld" << id << "[UP];\n#pragma unroll\n" << ind1 << "for (int u = 0; u < UP; ++u) row_load_strided<NV, VW, G>(ld"
                  << id << "[u], (const float*)" << tbp << ", A.s3[" << p << "], j);\n";
                break;
            default: throw CompileError("row program: bad load class");
        }
    }
    };
    phase1(false);
    if (ni) {
        // Accumulators that are stored but never read: their registers.
        for (int p = 0; p < ntens; ++p) {
            const int pid = k.params[a.tensor_param_index[p]].id;
            if (moving[p] || !a.stored[p] || a.preload[pid] || acc_read[p]) continue;
            o << "    " << (cls(pid) == RowClass::Full ? "RS" : "float") << " ld" << pid << "[UP];\n";
        }
        o << "    i64 iters_ = 1;\n";
        for (int i = 0; i < ni; ++i) o << "    iters_ *= A.ext[" << ng + i << "];\n";
        o << "    for (i64 it_ = 0; it_ < iters_; ++it_) {\n";
        o << "    { i64 q_ = it_;\n";
        for (int i = ni - 1; i >= 0; --i)
            o << "      vars[" << ng + i << "] = q_ % A.ext[" << ng + i << "]; q_ /= A.ext[" << ng + i << "];\n";
        o << "    }\n";
        for (int p = 0; p < ntens; ++p) {
            if (!moving[p]) continue;
            const int es = dtype_size(a.by_id[k.params[a.tensor_param_index[p]].id]->dtype);
            o << "    const i64 io" << p << " = ((i64)0";
            for (int i = 0; i < ni; ++i) o << " + A.coef[" << p << "][" << ng + i << "] * vars[" << ng + i << "]";
            o << ") * " << es << ";\n";
        }
        phase1(true);
    }
    // Phase 2: compute and store each pass.
    o << "#pragma unroll\n    for (int u = 0; u < UP; ++u) {\n";
    for (const auto& [id, p] : loads) {
        const RowClass c = cls(id);
        if (c == RowClass::RowVec || c == RowClass::RowVecT) o << "      const float v" << id << " = ld" << id << "[u];\n";
        else o << "      const RS& v" << id << " = ld" << id << "[u];\n";
    }
    for (const auto& [id, pid] : acc_loads)
        o << "      const " << (cls(pid) == RowClass::Full ? "RS" : "float") << " v" << id << " = ld" << pid << "[u];\n";
    bool waited = false;
    for (size_t oi = 0; oi < k.ops.size(); ++oi) {
        const auto& op = k.ops[oi];
        switch (op.kind) {
            case OpKind::Constant:
            case OpKind::Load:
                break;
            case OpKind::Store: {
                const int d = op.operands[0], s = op.operands[1];
                const int p = tord(d);
                if (rw_alias && !waited) {
                    o << "      __builtin_amdgcn_s_waitcnt(0);\n";
                    waited = true;
                }
                if (ni && !moving[p]) {
                    // An accumulator: the register copy, written back after the loops.
                    if (s != d) o << "      ld" << d << "[u] = " << vname(s) << ";\n";
                    break;
                }
                store_row("      ", p, d, base(p), vname(s), cls(s) == RowClass::Full);
                break;
            }
            case OpKind::Add: case OpKind::Sub: case OpKind::Mul: case OpKind::Div: case OpKind::Max: case OpKind::Min: {
                const int r = op.result, x = op.operands[0], y = op.operands[1];
                const char* F = op_functor(op.kind);
                const bool full = cls(r) == RowClass::Full;
                const std::string ty = full ? "RS" : "float";
                o << "      const " << ty << " v" << r << " = ";
                switch (a.bin_mode[oi]) {
                    case BinMode::Same:
                        o << (full ? std::string("ew<") + F + ">(" : std::string(F) + "::f(") << vname(x) << ", " << vname(y) << ");\n";
                        break;
                    case BinMode::RowExpand:
                        o << (full ? std::string("ew_rs<") + F + ">(" : std::string(F) + "::f(") << vname(x) << ", " << vname(y) << ");\n";
                        break;
                    case BinMode::ColExpand:
                        o << "ew<" << F << ">(" << vname(x) << ", " << vname(y) << ");\n";
                        break;
                    case BinMode::ScalarRight:
                        o << (full ? std::string("ew_rs<") + F + ">(" : std::string(F) + "::f(") << vname(x) << ", " << vname(y) << ");\n";
                        break;
                    case BinMode::ScalarLeft:
                        if (op.kind == OpKind::Div)
                            o << (full ? std::string("ew_sr<OpDiv>(") : std::string("OpDiv::f(")) << vname(x) << ", " << vname(y)
                              << ");\n";
                        else
                            o << (full ? std::string("ew_rs<") + F + ">(" : std::string(F) + "::f(") << vname(y) << ", " << vname(x)
                              << ");\n";
                        break;
                }
                break;
            }
            case OpKind::CpuSimAddCycles:
                break;
            case OpKind::TMov: {
                const int r = op.result, x = op.operands[0];
                o << "      const " << (cls(r) == RowClass::Full ? "RS" : "float") << " v" << r << " = " << vname(x) << ";\n";
                break;
            }
            case OpKind::Exp:
            case OpKind::Rsqrt: {
                const int r = op.result, x = op.operands[0];
                const bool full = cls(r) == RowClass::Full;
                if (full) o << "      const RS v" << r << " = " << (op.kind == OpKind::Exp ? "ew_exp(" : "ew_rsqrt(") << vname(x) << ");\n";
                else o << "      const float v" << r << " = " << (op.kind == OpKind::Exp ? "expf(" : "rsqrt_cr(") << vname(x) << ");\n";
                break;
            }
            case OpKind::RowSum:
            case OpKind::RowMax:
            case OpKind::RowMean: {
                const int r = op.result, x = op.operands[0];
                const int src_cols = a.by_id[x]->cols;
                o << "      const float v" << r << " = ";
                if (cls(x) == RowClass::Full) {
                    if (op.kind == OpKind::RowMax) o << "team_max<G>(lane_max<NV * VW>(" << vname(x) << ".v))";
                    else o << "team_sum<G>(lane_sum<NV * VW>(" << vname(x) << ".v))";
                } else {
                    o << vname(x);
                }
                if (op.kind == OpKind::RowMean) o << " / " << flt(static_cast<double>(src_cols));
                o << ";\n";
                break;
            }
            default: throw CompileError("row program: unexpected op " + op.kind_name);
        }
    }
    o << "    }\n";
    if (ni) {
        o << "    }\n";  // in-kernel loops
        // Accumulators back to memory, only when the loops ran: with an empty
        // in-kernel extent no store executes, as in the reference, and the
        // registers of an accumulator that is never read hold nothing.
        o << "    if (iters_ > 0) {\n";
        for (int p = 0; p < ntens; ++p) {
            const int pid = k.params[a.tensor_param_index[p]].id;
            if (moving[p] || !a.stored[p]) continue;
            o << "#pragma unroll\n    for (int u = 0; u < UP; ++u) {\n";
            store_row("      ", p, pid, "tb" + std::to_string(p) + "[u]", "ld" + std::to_string(pid) + "[u]", cls(pid) == RowClass::Full);
            o << "    }\n";
        }
        o << "    }\n";
    }
    o << "  }\n}\n";
    ek.source = o.str();
    return ek;
}

// ---------------------------------------------------------------------------
// Tile programs
// ---------------------------------------------------------------------------
EmittedKernel emit_tile(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    (void)m;
    const KernelDef& k = *a.def;
    const int ng = static_cast<int>(L.grid.size()), ni = static_cast<int>(L.inner.size());
    const int nvars = ng + ni;
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    auto is_int_v = [&](int id) { return !dtype_is_float(a.by_id[id]->dtype); };
    auto tord = [&](int id) { return a.param_of[id] >= 0 ? a.tensor_ordinal[a.param_of[id]] : -1; };

    // Params resident in LDS across the in-kernel loops of a task: views that
    // no in-kernel loop moves, on a tensor that no other param of the launch
    // names, read (preloaded or loaded) and / or stored without a cast, and
    // not read from global by a matmul.  They are loaded once before the
    // in-kernel loops and stored once after them, instead of every iteration
    // (the in-order iterations of one task see the same values either way).
    std::vector<bool> resident(ntens, false);
    if (ni > 0) {
        for (int p = 0; p < ntens; ++p) {
            const int pid = k.params[a.tensor_param_index[p]].id;
            const ValueInfo* v = a.by_id[pid];
            bool ok = v->dtype == DType::F32 || v->dtype == DType::I32 || v->dtype == DType::I64;
            for (int q = 0; q < ntens && ok; ++q)
                if (q != p && L.targs[q]->tid == L.targs[p]->tid) ok = false;
            for (const auto& li : L.inner)
                for (const auto& e : L.targs[p]->idx)
                    if (ok && reads_var(e, li.var)) ok = false;
            if (ok && spec.indirect_count.size() > static_cast<size_t>(p) && spec.indirect_count[p] > 0) ok = false;
            bool used = a.preload[pid], stored = false;
            for (const auto& op : k.ops) {
                if (!ok) break;
                for (size_t j = 0; j < op.operands.size(); ++j) {
                    if (op.operands[j] != pid) continue;
                    if (op.kind == OpKind::Matmul || op.kind == OpKind::StoreTopkIndices) ok = false;
                    const bool is_store = op.kind == OpKind::Store && j == 0;
                    // A read after a store in the same iteration sees the preloaded value,
                    // which the resident tile no longer holds.
                    if (!is_store && stored) ok = false;
                    if (op.kind == OpKind::Load) used = true;
                    if (is_store) {
                        used = stored = true;
                        if (a.by_id[op.operands[1]]->dtype != v->dtype) ok = false;
                    }
                }
            }
            resident[p] = ok && used;
        }
    }
    auto resident_id = [&](int id) { const int p = tord(id); return p >= 0 && resident[p]; };

    // Params staged ahead through the (single) in-kernel loop: views that the
    // loop moves, read (preloaded, loaded or a matmul operand), with no
    // indirect terms, on tensors that no param of the launch stores (so that
    // reading later iterations early sees the same data).  Chunks of SB
    // iterations are loaded into SB LDS slots at once, then the chunk's
    // iterations run from LDS: one memory latency per chunk instead of one per
    // iteration.
    std::vector<bool> staged(ntens, false);
    int SB = 0;
    if (ni == 1) {
        size_t stage_bytes = 0;
        for (int p = 0; p < ntens; ++p) {
            const int pid = k.params[a.tensor_param_index[p]].id;
            const ValueInfo* v = a.by_id[pid];
            bool moves = false;
            for (const auto& e : L.targs[p]->idx) moves = moves || reads_var(e, L.inner[0].var);
            if (!moves || resident[p] || a.stored[p]) continue;
            if (spec.indirect_count.size() > static_cast<size_t>(p) && spec.indirect_count[p] > 0) continue;
            bool written = false;
            for (int q = 0; q < ntens; ++q) written = written || (a.stored[q] && L.targs[q]->tid == L.targs[p]->tid);
            if (written) continue;
            bool read = a.preload[pid];
            for (const auto& op : k.ops)
                if ((op.kind == OpKind::Load || op.kind == OpKind::Matmul) && !op.operands.empty() &&
                    (op.operands[0] == pid || (op.kind == OpKind::Matmul && op.operands.size() > 1 && op.operands[1] == pid)))
                    read = true;
            if (!read) continue;
            staged[p] = true;
            stage_bytes += static_cast<size_t>(v->rows) * v->cols * (is_int_v(pid) ? 8 : 4);
        }
        if (stage_bytes > 0) {
            SB = static_cast<int>(std::min<size_t>(8, (48 * 1024) / stage_bytes));
            if (SB < 2) {
                SB = 0;
                staged.assign(ntens, false);
            }
        }
    }
    auto staged_id = [&](int id) { const int p = tord(id); return p >= 0 && staged[p]; };

    // LDS tiles: op results, preloaded and resident params, placed in one pool
    // by lifetime.  Every op ends with a workgroup barrier, so a tile whose
    // last reader is op i can share bytes with a tile first written by an op
    // after i; a tile written or read by op i does not share with another
    // tile live at op i.  Preloaded params are live from before op 0,
    // resident params for the whole task (prologue to epilogue).
    std::set<int> lds_vals;
    for (const auto& op : k.ops)
        if (op.result > 0 && a.by_id[op.result]->tile) lds_vals.insert(op.result);
    for (const auto& p : k.params)
        if (a.by_id[p.id]->tile && (a.preload[p.id] || resident_id(p.id)) && !staged_id(p.id)) lds_vals.insert(p.id);
    const int nops = static_cast<int>(k.ops.size());
    std::map<int, std::pair<int, int>> life;  // tile -> [first op, last op] (-1: before op 0)
    for (int id : lds_vals) life[id] = resident_id(id) ? std::make_pair(-1, nops) : std::make_pair(a.param_of[id] >= 0 ? -1 : nops, -1);
    for (int oi = 0; oi < nops; ++oi) {
        const auto& op = k.ops[oi];
        if (op.result > 0 && life.count(op.result)) {
            auto& l = life[op.result];
            l.first = std::min(l.first, oi);
            l.second = std::max(l.second, oi);
        }
        for (int id : op.operands)
            if (life.count(id)) {
                auto& l = life[id];
                l.first = std::min(l.first, oi);
                l.second = std::max(l.second, oi);
            }
    }
    auto tile_bytes = [&](int id) { return static_cast<size_t>(a.by_id[id]->rows) * a.by_id[id]->cols * (is_int_v(id) ? 8 : 4); };
    // First-fit placement of a set of tiles by lifetime (largest first).
    auto place = [&](const std::vector<int>& ids, std::map<int, size_t>& offs) {
        std::vector<int> order(ids);
        std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return tile_bytes(x) > tile_bytes(y); });
        size_t top = 0;
        for (int id : order) {
            const size_t sz = (tile_bytes(id) + 15) & ~static_cast<size_t>(15);
            std::vector<std::pair<size_t, size_t>> busy;
            for (const auto& [q, off] : offs)
                if (life[q].first <= life[id].second && life[id].first <= life[q].second)
                    busy.push_back({off, off + ((tile_bytes(q) + 15) & ~static_cast<size_t>(15))});
            std::sort(busy.begin(), busy.end());
            size_t off = 0;
            for (const auto& [lo, hi] : busy)
                if (off + sz > lo && off < hi) off = hi;
            offs[id] = off;
            top = std::max(top, off + sz);
        }
        return top;
    };
    size_t staged_bytes = 0;
    for (const auto& p : k.params)
        if (staged_id(p.id)) staged_bytes += static_cast<size_t>(SB) * a.by_id[p.id]->rows * a.by_id[p.id]->cols * (is_int_v(p.id) ? 8 : 4);
    // 32: 32x32 blocks (M, N multiples of 32, K even); 16: 16x16 blocks (M, N
    // multiples of 16, K a multiple of 4, at least 32^3 products); K at most
    // 32 or a multiple of 32.
    auto mma_kind = [&](const OpInfo& op) {
        if (op.kind != OpKind::Matmul || op.result <= 0) return 0;
        const ValueInfo* av = a.by_id[op.operands[0]];
        const ValueInfo* bv = a.by_id[op.operands[1]];
        const int M = av->rows, K = av->cols, N = bv->cols;
        if (is_int_v(op.result) || is_int_v(op.operands[0]) || is_int_v(op.operands[1]) || spec.threads % 64 != 0) return 0;
        if (K > 32 && K % 32 != 0) return 0;
        if (M % 32 == 0 && N % 32 == 0 && K % 2 == 0) return 32;
        // (smaller products keep the scalar loop, bit for bit the oracle's)
        if (M % 16 == 0 && N % 16 == 0 && K % 4 == 0 && M * N * K >= 32 * 32 * 32) return 16;
        return 0;
    };
    auto mma_shape = [&](const OpInfo& op) { return mma_kind(op) != 0; };
    const size_t mma_scratch = static_cast<size_t>(spec.threads / 64) * 32 * kTileMmaPitchHost * 4;
    bool want_mma = false;
    if (spec.tile_mma)
        for (const auto& op : k.ops) want_mma = want_mma || mma_shape(op);
    // Tiles that do not fit in LDS go to a per-workgroup global scratch
    // (largest first, until the rest fits beside the staged params and the
    // matmul scratch).
    std::vector<int> in_lds(lds_vals.begin(), lds_vals.end()), in_glob;
    std::map<int, size_t> lds_off, glob_off;
    size_t pool = place(in_lds, lds_off);
    const size_t lds_budget = 160 * 1024 - (want_mma ? mma_scratch : 0);
    while (pool + staged_bytes > lds_budget && !in_lds.empty()) {
        auto big = std::max_element(in_lds.begin(), in_lds.end(), [&](int x, int y) { return tile_bytes(x) < tile_bytes(y); });
        in_glob.push_back(*big);
        in_lds.erase(big);
        lds_off.clear();
        pool = place(in_lds, lds_off);
    }
    const size_t gpool = in_glob.empty() ? 0 : place(in_glob, glob_off);
    const bool glob_tiles = gpool > 0 && ntens < kMaxParams;
    if (gpool > 0 && !glob_tiles)
        throw CompileError("kernel " + k.name + ": tiles exceed the 160 KiB of LDS and the launch has no argument slot left for global tiles");
    size_t lds = pool + staged_bytes;
    // Matmul ops of MFMA shape run on the matrix cores (tile_mma), with a
    // 32-row operand scratch per wave, when that scratch fits beside the tiles.
    bool use_mma = want_mma;
    if (use_mma && lds + mma_scratch > 160 * 1024) use_mma = false;
    if (use_mma) lds += mma_scratch;
    if (lds > 160 * 1024)
        throw CompileError("kernel " + k.name + ": tiles need " + std::to_string(lds) +
                           " bytes of LDS, more than the 160 KiB of a gfx950 workgroup");

    EmittedKernel ek;
    ek.row_program = false;
    ek.threads = spec.threads;
    ek.lds_bytes = lds;
    ek.gtile_bytes = glob_tiles ? gpool : 0;
    std::ostringstream o;
    o << "#include \"ptowsp_device.h\"\nusing namespace ptowsp;\n";
    o << "// tile program: kernel " << k.name;
    if (!a.not_row_reason.empty()) o << " (not a row program: " << a.not_row_reason << ")";
    o << "\n";
    ek.entry = entry_name("tile", k);
    o << "extern \"C\" __global__ void __launch_bounds__(" << spec.threads << ") " << ek.entry << "(const LaunchArgs A) {\n";
    o << "  constexpr int NT = " << spec.threads << ";\n";
    if (pool > 0) o << "  __shared__ __attribute__((aligned(16))) char pool_[" << pool << "];\n";
    if (use_mma) o << "  __shared__ __attribute__((aligned(16))) float mma_scratch_[" << mma_scratch / 4 << "];\n";
    // Global tiles: workgroup blockIdx.x's region of base[ntens]; the
    // workgroup barriers between ops order these accesses as they do LDS.
    if (glob_tiles) o << "  char* const gtile_ = A.base[" << ntens << "] + (i64)blockIdx.x * " << gpool << ";\n";
    for (int id : lds_vals) {
        const char* ty = is_int_v(id) ? "i64" : "float";
        if (glob_off.count(id))
            o << "  " << ty << "* const L" << id << " = reinterpret_cast<" << ty << "*>(gtile_ + " << glob_off[id] << ");\n";
        else
            o << "  " << ty << "* const L" << id << " = reinterpret_cast<" << ty << "*>(pool_ + " << lds_off[id] << ");\n";
    }
    for (const auto& p : k.params)
        if (staged_id(p.id)) {
            const ValueInfo* v = a.by_id[p.id];
            o << "  __shared__ __attribute__((aligned(16))) " << (is_int_v(p.id) ? "i64" : "float") << " LP" << p.id << "["
              << SB * v->rows * v->cols << "];\n";
        }
    emit_scalars(o, a, true);
    o << "  i64 vars[" << (nvars > 0 ? nvars : 1) << "];\n  (void)vars;\n";
    // Grid loops are decoded from the task index.  A serial launch without a
    // task list runs one group of tasks per workgroup: the grid variables
    // outside seq_mask are decoded from the group index, those inside are
    // looped in program order.  A serial task-list launch decodes each listed
    // task in one workgroup, in list (program) order.
    const bool grid_loops = spec.serial && !spec.task_list;
    const uint32_t all_grid = ng >= 32 ? 0xFFFFFFFFu : ((1u << ng) - 1u);
    const uint32_t seq = grid_loops ? (spec.seq_mask ? spec.seq_mask : all_grid) : 0u;
    std::vector<int> par, loops;
    for (int v = 0; v < ng; ++v) (((seq >> v) & 1u) ? loops : par).push_back(v);
    for (int v = ng; v < nvars; ++v) loops.push_back(v);
    const int looped = static_cast<int>(loops.size());
    if (grid_loops) {
        o << "  i64 ngroups_ = 1;\n";
        for (int v : par) o << "  ngroups_ *= A.ext[" << v << "];\n";
        o << "  for (i64 t = blockIdx.x; t < ngroups_; t += gridDim.x) {\n";
        if (!par.empty()) {
            o << "    { i64 q_ = t;\n";
            for (size_t i = par.size() - 1; i >= 1; --i)
                o << "      vars[" << par[i] << "] = q_ % A.ext[" << par[i] << "]; q_ /= A.ext[" << par[i] << "];\n";
            o << "      vars[" << par[0] << "] = q_; }\n";
        }
    } else {
        o << "  for (i64 t = blockIdx.x; t < A.ntasks; t += gridDim.x) {\n";
        emit_decode(o, "    ", ng, spec.task_list ? "A.tlist[t]" : "t");
    }
    std::string ind = "    ";
    bool any_resident = false;
    for (int p = 0; p < ntens; ++p) any_resident = any_resident || resident[p];
    // Tile pointer of tensor ordinal p with a per-task bounds check (indirect
    // and run-time extents cannot all be checked on the host).
    std::vector<int> first_term(ntens, 0);
    for (int p = 1; p < ntens; ++p)
        first_term[p] = first_term[p - 1] + (spec.indirect_count.size() > static_cast<size_t>(p - 1) ? spec.indirect_count[p - 1] : 0);
    auto pointer = [&](int p) {
        const ValueInfo* v = a.by_id[k.params[a.tensor_param_index[p]].id];
        const int nt = spec.indirect_count.size() > static_cast<size_t>(p) ? spec.indirect_count[p] : 0;
        o << ind << "const i64 o" << p << " = " << offset_expr(p, nvars, first_term[p], nt) << ";\n";
        o << ind << "if (o" << p << " < 0 || o" << p << " + (i64)" << (v->rows - 1) << " * A.s3[" << p << "] + (i64)" << (v->cols - 1)
          << " * A.s4[" << p << "] >= A.span[" << p << "]) { if (threadIdx.x == 0) *A.err = 2; continue; }\n";
        o << ind << "char* p" << p << " = A.base[" << p << "] + o" << p << " * " << dtype_size(v->dtype) << ";\n";
    };
    auto load_tile = [&](int id, int dst, int p) {
        const ValueInfo* v = a.by_id[id];
        o << ind << "tile_load_" << (is_int_v(id) ? "i" : "f") << "<" << dt_code(v->dtype) << ", " << v->rows << ", " << v->cols
          << ", NT>(L" << dst << ", p" << p << ", A.s3[" << p << "], A.s4[" << p << "]);\n";
    };
    for (int i = 0; i < looped; ++i) {
        const int v = loops[i];
        const int inner_i = v - ng;
        if (inner_i == 0 && any_resident) {
            // Task prologue: the resident params' pointers and first loads (the
            // in-kernel variables do not move them).
            for (int j = 0; j < ni; ++j) o << ind << "vars[" << ng + j << "] = 0;\n";
            for (int p = 0; p < ntens; ++p) {
                if (!resident[p]) continue;
                pointer(p);
                const int pid = k.params[a.tensor_param_index[p]].id;
                bool read = a.preload[pid];
                for (const auto& op : k.ops)
                    if (op.kind == OpKind::Load && op.operands[0] == pid) read = true;
                if (read) load_tile(pid, pid, p);
            }
            o << ind << "bool ran_ = false;\n";
            o << ind << "__syncthreads();\n";
        }
        const int term = inner_i >= 0 && spec.inner_dyn_term.size() > static_cast<size_t>(inner_i) ? spec.inner_dyn_term[inner_i] : -1;
        if (term >= 0) o << ind << "const i64 e" << i << " = indirect_index(A, " << term << ", vars, " << v << ");\n";
        else o << ind << "const i64 e" << i << " = A.ext[" << v << "];\n";
        if (inner_i == 0 && SB > 0) {
            // Chunks of SB iterations: the staged params' tiles of the whole
            // chunk are loaded first, then the iterations run.
            o << ind << "for (i64 c0_ = 0; c0_ < e" << i << "; c0_ += " << SB << ") {\n";
            o << ind << "  const i64 nb_ = e" << i << " - c0_ < " << SB << " ? e" << i << " - c0_ : " << SB << ";\n";
            o << ind << "  for (i64 j_ = 0; j_ < nb_; ++j_) {\n";
            o << ind << "    vars[" << v << "] = c0_ + j_;\n";
            for (int p = 0; p < ntens; ++p) {
                if (!staged[p]) continue;
                const int pid = k.params[a.tensor_param_index[p]].id;
                const ValueInfo* pv = a.by_id[pid];
                o << ind << "    { const i64 o_ = " << offset_expr(p, nvars, first_term[p], 0) << ";\n";
                o << ind << "      if (o_ >= 0 && o_ + (i64)" << (pv->rows - 1) << " * A.s3[" << p << "] + (i64)" << (pv->cols - 1)
                  << " * A.s4[" << p << "] < A.span[" << p << "])\n";
                o << ind << "        tile_load_" << (is_int_v(pid) ? "i" : "f") << "<" << dt_code(pv->dtype) << ", " << pv->rows << ", "
                  << pv->cols << ", NT>(LP" << pid << " + j_ * " << pv->rows * pv->cols << ", A.base[" << p << "] + o_ * "
                  << dtype_size(pv->dtype) << ", A.s3[" << p << "], A.s4[" << p << "]); }\n";
            }
            o << ind << "  }\n";
            o << ind << "  __syncthreads();\n";
            o << ind << "  for (i64 j_ = 0; j_ < nb_; ++j_) {\n";
            ind += "    ";
            o << ind << "vars[" << v << "] = c0_ + j_;\n";
            for (int p = 0; p < ntens; ++p) {
                if (!staged[p]) continue;
                const int pid = k.params[a.tensor_param_index[p]].id;
                const ValueInfo* pv = a.by_id[pid];
                o << ind << (is_int_v(pid) ? "i64" : "float") << "* const L" << pid << " = LP" << pid << " + j_ * "
                  << pv->rows * pv->cols << ";\n";
            }
            continue;
        }
        o << ind << "for (vars[" << v << "] = 0; vars[" << v << "] < e" << i << "; ++vars[" << v << "]) {\n";
        ind += "  ";
    }
    for (int p = 0; p < ntens; ++p)
        if (!resident[p]) pointer(p);
    if (any_resident) o << ind << "ran_ = true;\n";
    // Preloads (:764-779).
    for (size_t i = 0; i < k.params.size(); ++i) {
        const ValueInfo* v = a.by_id[k.params[i].id];
        if (!v->tile || !a.preload[v->id] || resident_id(v->id) || staged_id(v->id)) continue;
        const int p = a.tensor_ordinal[i];
        o << ind << "tile_load_" << (is_int_v(v->id) ? "i" : "f") << "<" << dt_code(v->dtype) << ", " << v->rows << ", " << v->cols
          << ", NT>(L" << v->id << ", p" << p << ", A.s3[" << p << "], A.s4[" << p << "]);\n";
    }
    o << ind << "__syncthreads();\n";
    auto src = [&](int id, const std::string& e) {
        return a.by_id[id]->tile ? "L" + std::to_string(id) + "[" + e + "]" : "s" + std::to_string(id);
    };
    for (size_t oi = 0; oi < k.ops.size(); ++oi) {
        const auto& op = k.ops[oi];
        const ValueInfo* res = op.result > 0 ? a.by_id[op.result] : nullptr;
        switch (op.kind) {
            case OpKind::Constant: continue;
            case OpKind::Load: {
                const ValueInfo* s = a.by_id[op.operands[0]];
                const int p = tord(s->id);
                if (resident[p] || staged[p])
                    o << ind << "for (int e = threadIdx.x; e < " << s->rows * s->cols << "; e += NT) L" << res->id << "[e] = L" << s->id
                      << "[e];\n";
                else
                    o << ind << "tile_load_" << (is_int_v(s->id) ? "i" : "f") << "<" << dt_code(s->dtype) << ", " << s->rows << ", "
                      << s->cols << ", NT>(L" << res->id << ", p" << p << ", A.s3[" << p << "], A.s4[" << p << "]);\n";
                break;
            }
            case OpKind::Store: {
                const ValueInfo* d = a.by_id[op.operands[0]];
                const ValueInfo* s = a.by_id[op.operands[1]];
                const int p = tord(d->id);
                if (resident[p]) {
                    // The param's LDS tile holds its value until the loops end (same dtype: no cast).
                    if (s->id != d->id)
                        o << ind << "for (int e = threadIdx.x; e < " << d->rows * d->cols << "; e += NT) L" << d->id << "[e] = L"
                          << s->id << "[e];\n";
                } else {
                    o << ind << "tile_store_" << (is_int_v(s->id) ? "i" : "f") << "<" << dt_code(d->dtype) << ", " << d->rows << ", "
                      << d->cols << ", NT>(p" << p << ", L" << s->id << ", A.s3[" << p << "], A.s4[" << p << "]);\n";
                }
                break;
            }
            case OpKind::Matmul: {
                const ValueInfo* av = a.by_id[op.operands[0]];
                const ValueInfo* bv = a.by_id[op.operands[1]];
                const int M = av->rows, K = av->cols, N = bv->cols;
                auto elem = [&](const ValueInfo* v, const std::string& r, const std::string& c, int ld) {
                    const int p = tord(v->id);
                    if (p >= 0 && !staged[p])
                        return "gload_f<" + std::to_string(dt_code(v->dtype)) + ">(p" + std::to_string(p) + ", (i64)(" + r + ") * A.s3[" +
                               std::to_string(p) + "] + (i64)(" + c + ") * A.s4[" + std::to_string(p) + "])";
                    return "L" + std::to_string(v->id) + "[(" + r + ") * " + std::to_string(ld) + " + (" + c + ")]";
                };
                if (use_mma && mma_shape(op)) {
                    o << ind << "{\n";
                    o << ind << "  auto fa_ = [&](int i, int q) -> float { return " << elem(av, "i", "q", K) << "; };\n";
                    o << ind << "  auto fb_ = [&](int q, int jj) -> float { return " << elem(bv, "q", "jj", N) << "; };\n";
                    o << ind << "  tile_mma" << (mma_kind(op) == 16 ? "16" : "") << "<" << M << ", " << K << ", " << N
                      << ", NT>(fa_, fb_, L" << res->id << ", mma_scratch_);\n";
                    o << ind << "}\n";
                    break;
                }
                o << ind << "for (int e = threadIdx.x; e < " << M * N << "; e += NT) {\n";
                o << ind << "  const int i = e / " << N << ", jj = e % " << N << ";\n";
                o << ind << "  float acc = 0.0f;\n";
                o << ind << "  for (int q = 0; q < " << K << "; ++q) acc = acc + " << elem(av, "i", "q", K) << " * "
                  << elem(bv, "q", "jj", N) << ";\n";
                o << ind << "  L" << res->id << "[e] = acc;\n" << ind << "}\n";
                break;
            }
            case OpKind::Add: case OpKind::Sub: case OpKind::Mul: case OpKind::Div: case OpKind::Max: case OpKind::Min: {
                const int x = op.operands[0], y = op.operands[1];
                const int C = res->cols;
                const char* F = op_functor(op.kind);
                o << ind << "for (int e = threadIdx.x; e < " << res->rows * C << "; e += NT) L" << res->id << "[e] = ";
                switch (a.bin_mode[oi]) {
                    case BinMode::Same: o << F << "::f(" << src(x, "e") << ", " << src(y, "e") << ");\n"; break;
                    case BinMode::RowExpand: o << F << "::f(" << src(x, "e") << ", " << src(y, "e / " + std::to_string(C)) << ");\n"; break;
                    case BinMode::ColExpand: o << F << "::f(" << src(x, "e") << ", " << src(y, "e % " + std::to_string(C)) << ");\n"; break;
                    case BinMode::ScalarRight: o << F << "::f(" << src(x, "e") << ", " << src(y, "e") << ");\n"; break;
                    case BinMode::ScalarLeft:
                        if (op.kind == OpKind::Div) o << "OpDiv::f(" << src(x, "e") << ", " << src(y, "e") << ");\n";
                        else o << F << "::f(" << src(y, "e") << ", " << src(x, "e") << ");\n";
                        break;
                }
                break;
            }
            case OpKind::Exp:
            case OpKind::Rsqrt:
                o << ind << "for (int e = threadIdx.x; e < " << res->rows * res->cols << "; e += NT) L" << res->id << "[e] = "
                  << (op.kind == OpKind::Exp ? "expf(" : "rsqrt_cr(") << src(op.operands[0], "e") << ");\n";
                break;
            case OpKind::RowSum:
            case OpKind::RowMax:
            case OpKind::RowMean: {
                const ValueInfo* s = a.by_id[op.operands[0]];
                const std::string ty = is_int_v(s->id) ? "i64" : "float";
                const char* fold = op.kind == OpKind::RowMax ? "acc = x > acc ? x : acc;" : "acc = acc + x;";
                o << ind << "for (int r = threadIdx.x; r < " << s->rows << "; r += NT) {\n";
                if (ty == "float" && s->cols % 4 == 0 && s->cols >= 8) {
                    // The oracle's left-to-right order, read 16 bytes at a time and
                    // unrolled so that the loads do not wait on the fold chain.
                    o << ind << "  const float4* row_ = reinterpret_cast<const float4*>(L" << s->id << " + r * " << s->cols << ");\n";
                    o << ind << "  float acc = row_[0].x;\n";
                    o << ind << "  { float x = row_[0].y; " << fold << " x = row_[0].z; " << fold << " x = row_[0].w; " << fold
                      << " }\n";
                    o << ind << "#pragma unroll 8\n";
                    o << ind << "  for (int c4 = 1; c4 < " << s->cols / 4 << "; ++c4) { const float4 v4 = row_[c4]; float x = v4.x; "
                      << fold << " x = v4.y; " << fold << " x = v4.z; " << fold << " x = v4.w; " << fold << " }\n";
                } else {
                    o << ind << "  " << ty << " acc = L" << s->id << "[r * " << s->cols << "];\n";
                    o << ind << "  for (int c = 1; c < " << s->cols << "; ++c) { const " << ty << " x = L" << s->id << "[r * "
                      << s->cols << " + c]; " << fold << " }\n";
                }
                if (op.kind == OpKind::RowMean) {
                    if (ty == "float") o << ind << "  acc = acc / " << flt(static_cast<double>(s->cols)) << ";\n";
                    else o << ind << "  acc = acc / " << s->cols << ";\n";
                }
                o << ind << "  L" << res->id << "[r] = acc;\n" << ind << "}\n";
                break;
            }
            case OpKind::CpuSimAddCycles: continue;
            case OpKind::TMov:
                o << ind << "for (int e = threadIdx.x; e < " << res->rows * res->cols << "; e += NT) L" << res->id << "[e] = "
                  << src(op.operands[0], "e") << ";\n";
                break;
            case OpKind::IotaU32:
                o << ind << "for (int e = threadIdx.x; e < " << res->cols << "; e += NT) L" << res->id << "[e] = e;\n";
                break;
            case OpKind::TSort32:
                // Descending by score, NaN last, ties in source order: each of the 32
                // elements finds its rank and writes its (score, index) pair.
                o << ind << "tsort32_rank<NT>(L" << res->id << ", L" << op.operands[0] << ", L" << op.operands[1] << ");\n";
                break;
            case OpKind::ExtractTopkIndices:
                o << ind << "for (int e = threadIdx.x; e < " << res->cols << "; e += NT) L" << res->id << "[e] = (i64)(int)L"
                  << op.operands[0] << "[2 * e + 1];\n";
                break;
            case OpKind::StoreTopkIndices: {
                const ValueInfo* d = a.by_id[op.operands[0]];
                const int p = tord(d->id);
                o << ind << "for (int e = threadIdx.x; e < " << op.ints.at("k") << "; e += NT) reinterpret_cast<"
                  << (d->dtype == DType::I32 ? "int" : "i64") << "*>(p" << p << ")[(i64)e * A.s4[" << p << "]] = (int)L"
                  << op.operands[1] << "[2 * e + 1];\n";
                break;
            }
            default: throw CompileError("tile program: unexpected op " + op.kind_name);
        }
        o << ind << "__syncthreads();\n";
    }
    for (int i = looped - 1; i >= 0; --i) {
        if (loops[i] == ng && SB > 0) {
            ind.resize(ind.size() - 4);
            o << ind << "  }\n" << ind << "}\n";
        } else {
            ind.resize(ind.size() - 2);
            o << ind << "}\n";
        }
        if (loops[i] == ng && any_resident) {
            // Task epilogue: the stored resident params go back to global
            // memory (when the in-kernel loops ran at least once).
            o << ind << "if (ran_) {\n";
            for (int p = 0; p < ntens; ++p) {
                if (!resident[p] || !a.stored[p]) continue;
                const int pid = k.params[a.tensor_param_index[p]].id;
                const ValueInfo* v = a.by_id[pid];
                o << ind << "  tile_store_" << (is_int_v(pid) ? "i" : "f") << "<" << dt_code(v->dtype) << ", " << v->rows << ", "
                  << v->cols << ", NT>(p" << p << ", L" << pid << ", A.s3[" << p << "], A.s4[" << p << "]);\n";
            }
            o << ind << "}\n";
        }
    }
    o << "  }\n}\n";
    ek.source = o.str();
    return ek;
}

// ---------------------------------------------------------------------------
// GEMM (MFMA) programs
// ---------------------------------------------------------------------------
EmittedKernel emit_gemm(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    (void)m;
    const KernelDef& k = *a.def;
    const GemmInfo& g = a.gemm;
    const int ng = static_cast<int>(L.grid.size()), ni = static_cast<int>(L.inner.size());
    const int nvars = ng + ni;
    const int fm = spec.gemm_vm >= 0 ? spec.gemm_fm : 1, fn = spec.gemm_vn >= 0 ? spec.gemm_fn : 1;
    // Task tiles above 256 rows / columns run as sm x sn blocks of 256.
    const int sm = g.m > 256 ? g.m / 256 : 1, sn = g.n > 256 ? g.n / 256 : 1;
    const int bm = gemm_block_dim(g.m) * fm, bn = gemm_block_dim(g.n) * fn;
    // One LDS stage per kf task K steps (kf consecutive steps are adjacent
    // columns of A and rows of B), two stages (a 4-stage ring of 32-wide
    // stages measured slower on 256x256 blocks: twice the barriers).
    const int wm = gemm_waves_m(), wn = gemm_waves_n(bn);
    const int kf = ni == 1 ? spec.gemm_kf : 1, kstep = g.k * kf;
    // f32 A / B: stages of at most 32 K columns (GemmF32), a K step split
    // over ksplit stages; element size es bytes.
    const int bk = gemm_stage_k(kstep, g.f32), ns = 2, es = g.f32 ? 4 : 2;
    // Stages per K step: GemmF32 takes them as its KSPLIT; the bf16 / f16
    // blocks see each stage as one step of a stage-level offset function
    // (sks stages per task step).
    const int ksplit = g.f32 ? kstep / bk : 1, sks = g.f32 ? 1 : kstep / bk;
    // Ping-pong block: 256x256, K step 32 / 64, row pitches checked on the host.
    const bool pp = !g.f32 && spec.gemm_pingpong && bm == 256 && bn == 256 && (bk == 64 || bk == 32);
    EmittedKernel ek;
    ek.threads = 64 * wm * wn;
    ek.row_program = false;
    ek.tasks_per_block = fm * fn;
    ek.blocks_per_task = sm * sn;
    std::ostringstream o;
    o << "#include \"ptowsp_device.h\"\nusing namespace ptowsp;\n";
    o << "// gemm program: kernel " << k.name << ", task tile " << g.m << "x" << g.n << "x" << g.k
      << (g.f32 ? " f32" : g.f16 ? " f16" : " bf16")
      << (g.accumulate ? ", accumulate" : "") << "; block " << bm << "x" << bn << " (" << fm * fn << " tasks)"
      << (kf > 1 ? "; " + std::to_string(kf) + " K steps per stage" : "")
      << (pp ? ", ping-pong" : "") << "\n";
    ek.entry = entry_name("gemm", k);
    o << "extern \"C\" __global__ void __launch_bounds__(" << ek.threads << ") "
      << ek.entry << "(const LaunchArgs A) {\n";
    if (pp)
        o << "  typedef GemmPingPong<" << bk << ", " << (g.f16 ? "true" : "false") << "> GB;\n";
    else if (g.f32)
        o << "  typedef GemmF32<" << bm << ", " << bn << ", " << bk << ", " << wm << ", " << wn << ", " << ns << ", " << ksplit
          << "> GB;\n";
    else
        o << "  typedef GemmBlock<" << bm << ", " << bn << ", " << bk << ", " << wm << ", " << wn << ", "
          << (g.f16 ? "true" : "false") << ", " << ns << ", " << ksplit << "> GB;\n";
    o << "  __shared__ __attribute__((aligned(1024))) u16 lds[GB::kLdsElems];\n";
    o << "  i64 vars[" << (nvars > 0 ? nvars : 1) << "];\n  (void)vars;\n";
    // One workgroup per block (the host launches every block): nothing of
    // the launch arguments stays live through the K loop.
    o << "  const i64 nblk = A.ntasks / " << fm * fn << " * " << sm * sn << ";\n";
    o << "  {\n    const i64 w = blockIdx.x;\n    if (w >= nblk) return;\n";
    o << "    i64 q_ = xcd_order(w, nblk);\n";
    if (sm * sn > 1) {
        // The block's 256 x 256 sub-tile of its task.
        o << "    const i64 sn_ = q_ % " << sn << "; q_ /= " << sn << ";\n";
        o << "    const i64 sm_ = q_ % " << sm << "; q_ /= " << sm << ";\n";
    }
    // Decode the block index over the grid with the merged extents divided.
    for (int v = ng - 1; v >= 0; --v) {
        const int f = v == spec.gemm_vm ? fm : (v == spec.gemm_vn ? fn : 1);
        const std::string ext = f > 1 ? "(A.ext[" + std::to_string(v) + "] / " + std::to_string(f) + ")" : "A.ext[" + std::to_string(v) + "]";
        if (v > 0) o << "    vars[" << v << "] = q_ % " << ext << "; q_ /= " << ext << ";\n";
        else o << "    vars[0] = q_;\n";
        if (f > 1) o << "    vars[" << v << "] *= " << f << ";\n";
    }
    o << "    i64 iters = 1;\n";
    for (int i = 0; i < ni; ++i) o << "    iters *= A.ext[" << ng + i << "];\n";
    // Merged K steps: iterations count stages of kf task steps (the host has
    // checked that kf divides the loop).
    if (kf > 1) o << "    iters /= " << kf << ";\n";
    o << "    if (iters <= 0) return;\n";
    for (int i = 0; i < ni; ++i) o << "    vars[" << ng + i << "] = 0;\n";
    o << "    const u16* pa = reinterpret_cast<const u16*>(A.base[" << g.a << "] + (" << offset_expr(g.a, nvars, 0, 0) << ") * " << es
      << ");\n";
    o << "    const u16* pb = reinterpret_cast<const u16*>(A.base[" << g.b << "] + (" << offset_expr(g.b, nvars, 0, 0) << ") * " << es
      << ");\n";
    // The output view does not move with the in-kernel loops (checked on the host).
    o << "    float* pc = reinterpret_cast<float*>(A.base[" << g.c << "] + (" << offset_expr(g.c, nvars, 0, 0) << ") * 4);\n";
    if (sm * sn > 1) {
        o << "    pa = reinterpret_cast<const u16*>(reinterpret_cast<const char*>(pa) + sm_ * 256 * A.s3[" << g.a << "] * " << es << ");\n";
        o << "    pb = reinterpret_cast<const u16*>(reinterpret_cast<const char*>(pb) + sn_ * 256 * " << es << ");\n";
        o << "    pc += sm_ * 256 * A.s3[" << g.c << "] + sn_ * 256;\n";
    }
    // Byte offsets of in-kernel iteration `it` from iteration 0 (mixed radix over the inner loops).
    if (ni == 1) {
        // One in-kernel loop: 32-bit byte steps (the host bounds every
        // offset below 2^31).
        o << "    const int da_ = static_cast<int>(A.coef[" << g.a << "][" << ng << "] * " << es * kf << "), db_ = static_cast<int>(A.coef["
          << g.b << "][" << ng << "] * " << es * kf << ");\n";
        o << "    auto off = [=](i64 it, int& soa, int& sob) { soa = static_cast<int>(it) * da_; sob = static_cast<int>(it) * db_; };\n";
    } else {
        o << "    auto off = [&](i64 it, int& soa, int& sob) {\n";
        o << "      i64 oa = 0, ob = 0;\n";
        for (int i = ni - 1; i >= 0; --i) {
            const int v = ng + i;
            o << "      { const i64 x = it % A.ext[" << v << "]; it /= A.ext[" << v << "]; oa += A.coef[" << g.a << "][" << v
              << "] * x; ob += A.coef[" << g.b << "][" << v << "] * x; }\n";
        }
        o << "      soa = static_cast<int>(oa * " << es << "); sob = static_cast<int>(ob * " << es << ");\n";
        o << "    };\n";
    }
    if (sks > 1) {
        // Stage st: task step st / sks, columns (st % sks) * BK of it.
        o << "    const i64 ldb_ = A.s3[" << g.b << "];\n";
        o << "    auto offs = [=](i64 st, int& soa, int& sob) {\n";
        o << "      off(st / " << sks << ", soa, sob);\n";
        o << "      const int h_ = static_cast<int>(st % " << sks << ");\n";
        o << "      soa += h_ * " << bk * es << "; sob += h_ * static_cast<int>(ldb_) * " << bk * es << ";\n";
        o << "    };\n";
    }
    if (pp) {
        // L2 touches: the blocks that share an A panel (same m block) split its
        // rows by their n block (8 x 32 rows); those that share a B panel
        // split the stage's K rows by their m block (BK/16 x 16 rows).
        if (spec.gemm_vm >= 0 && spec.gemm_vn >= 0)
            o << "    const int pfa_row = static_cast<int>((vars[" << spec.gemm_vn << "] / " << fn << ") % 8) * 32;\n"
              << "    const int pfb_row = static_cast<int>((vars[" << spec.gemm_vm << "] / " << fm << ") % " << bk / 16
              << ") * 16;\n";
        else
            o << "    const int pfa_row = -1, pfb_row = -1;\n";
    }
    const std::string its = sks > 1 ? "iters * " + std::to_string(sks) : "iters";
    const std::string it0 = g.accumulate ? "0" : (sks > 1 ? "(iters - 1) * " + std::to_string(sks) : "iters - 1");
    o << "    GB::template run<" << (g.accumulate ? "true" : "false") << ">(lds, pa, static_cast<int>(A.s3[" << g.a
      << "]), pb, static_cast<int>(A.s3[" << g.b << "]), pc, static_cast<int>(A.s3[" << g.c << "]), "
      << it0 << ", " << its << ", " << (sks > 1 ? "offs" : "off") << (pp ? ", pfa_row, pfb_row" : "") << ");\n";
    o << "  }\n}\n";
    ek.source = o.str();
    ek.lds_bytes = pp ? static_cast<size_t>((bk == 64 ? 2 : 4) * 512 * bk * 2 + 256) : static_cast<size_t>(ns * (bm + bn) * bk * es);
    return ek;
}

// ---------------------------------------------------------------------------
// Decode programs (online softmax over pages, balanced over resident waves)
// ---------------------------------------------------------------------------
// One kernel, launched with one block per resident slot.  Every block first
// scans the units' page counts into LDS; then wave w of W = min(resident
// waves, T) folds global pages [w*T/W, (w+1)*T/W) (DecodeSplit) and writes
// one partial per unit it touches.  The wave that completes a unit (the only one, or the last to
// arrive on the unit's counter) folds the unit's partials in page order into
// the accumulators and resets the counter.  Launch arguments beyond the
// kernel's tensors: base[ntens] is the scratch (int32 counters, one per unit,
// zero between launches, then the partials);
// scal[kMaxScalars-1] is the declared maximum page count (larger extents
// raise error 3 and are cut to it).

EmittedKernel emit_decode(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    (void)m;
    const KernelDef& k = *a.def;
    const DecodeInfo& d = a.decode;
    const int ng = static_cast<int>(L.grid.size());
    const int nvars = ng + 1;
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    std::vector<int> first_term(ntens, 0);
    for (int p = 1; p < ntens; ++p) first_term[p] = first_term[p - 1] + spec.indirect_count[p - 1];
    auto nterms = [&](int p) { return spec.indirect_count[p]; };
    const std::string tmpl = "DecodeWave<" + std::to_string(d.g) + ", " + std::to_string(d.d) + ", " +
                             (d.f16 ? "true" : "false") + ", " + (d.mask >= 0 ? "true" : "false") + ", " +
                             (d.pg == 8 ? "true" : "false") + (d.f32 || d.row_mask ? (d.f32 ? ", true" : ", false") : "") +
                             (d.row_mask ? ", true" : "") + ">";
    const int es = d.f32 ? 4 : 2;  // bytes per q / K / V element
    std::ostringstream scale;
    scale.precision(9);
    scale << std::scientific << d.scale << "f";

    const int nw = spec.decode_waves, nt = 64 * nw;
    EmittedKernel ek;
    ek.threads = nt;
    ek.row_program = false;
    ek.part_floats = d.g * d.d + ((2 * d.g + 3) & ~3);  // DecodeWave::kPartFloats
    std::ostringstream o;
    o << "#include \"ptowsp_device.h\"\nusing namespace ptowsp;\n";
    o << "// decode program: kernel " << k.name << ", " << d.g << " query rows, head dim " << d.d
      << (d.f32 ? " f32" : d.f16 ? " f16" : " bf16")
      << (d.mask >= 0 ? ", masked" : "") << ", pages balanced over the resident waves\n";
    // Grid variables of a unit.  Units number at most kDecodeMaxUnits, so
    // every grid extent and unit index fits 32-bit unsigned arithmetic.
    auto decode_vars = [&](const std::string& unit, const std::string& ind) {
        if (ng == 0) return;
        o << ind << "{ u32 q_ = static_cast<u32>(" << unit << ");\n";
        for (int v = ng - 1; v >= 1; --v)
            o << ind << "  { const u32 e_ = static_cast<u32>(A.ext[" << v << "]); vars[" << v << "] = (i64)(q_ % e_); q_ /= e_; }\n";
        o << ind << "  vars[0] = (i64)q_; }\n";
    };
    auto ptr = [&](int p, const std::string& type, int esize) {
        return "reinterpret_cast<" + type + ">(A.base[" + std::to_string(p) + "] + (" +
               offset_expr(p, nvars, first_term[p], nterms(p)) + ") * " + std::to_string(esize) + ")";
    };
    // Bounds check of a unit's fixed tile (q, m, l, o): sets `flag` and the
    // error code 2 when it falls outside its tensor.
    auto unit_check = [&](int p, int rows, int cols, const std::string& flag) {
        o << "      { const i64 o_ = " << offset_expr(p, nvars, first_term[p], nterms(p)) << ";\n";
        o << "        if (o_ < 0 || o_ + (i64)" << rows - 1 << " * A.s3[" << p << "] + (i64)" << cols - 1 << " * A.s4[" << p
          << "] >= A.span[" << p << "]) { " << flag << " = true; if (lane == 0) *A.err = 2; } }\n";
    };
    // One wave per SIMD (the host reserves LDS so that one block runs per
    // CU): waves sharing a SIMD are served oldest first under memory
    // back-pressure, which would leave equal page shares finishing far
    // apart; alone on its SIMD a wave has the register file for its ring.
    ek.entry = entry_name("decode", k);
    o << "extern \"C\" __global__ void __launch_bounds__(" << nt << ") __attribute__((amdgpu_waves_per_eu(" << nw / 4 << ", "
      << nw / 4 << "))) " << ek.entry << "(const LaunchArgs A) {\n";
    o << "  typedef " << tmpl << " DW;\n";
    o << "  static_assert(DecodeSplit::kMaxUnits == " << kDecodeMaxUnits << ", \"unit limit\");\n";
    o << "  static_assert(DecodeSplit::kUnitCost == " << kDecodeUnitCost << ", \"unit cost\");\n";
    o << "  static_assert(DW::kPartFloats == " << ek.part_floats << ", \"partial size\");\n";
    o << "  __shared__ int pre[DecodeSplit::kMaxUnits + 1], cpre[DecodeSplit::kMaxUnits + 1];\n";
    o << "  __shared__ int wsum[" << nw << "], cwsum[" << nw << "];\n";
    o << "  const int tid = threadIdx.x, lane = tid & 63;\n";
    o << "  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);\n";
    o << "  const int U = static_cast<int>(A.ntasks);\n";
    o << "  const i64 maxp = (i64)A.scal[" << kMaxScalars - 1 << "];\n";
    o << "  i64 vars[" << nvars << "];\n";
    // Prefixes of the page counts (pre) and of the units' scheduling costs
    // (cpre, DecodeSplit::cost): thread t owns units t*per .. t*per+per-1.
    o << "  {\n";
    o << "    const int per = (U + " << nt - 1 << ") / " << nt << ", u0 = tid * per;\n";
    o << "    int n_[DecodeSplit::kMaxUnits / " << nt << "];\n";
    o << "    int run = 0, crun = 0;\n";
    o << "#pragma unroll\n";
    o << "    for (int i = 0; i < DecodeSplit::kMaxUnits / " << nt << "; ++i) {\n";
    o << "      n_[i] = 0;\n";
    o << "      if (i < per && u0 + i < U) {\n";
    decode_vars("u0 + i", "        ");
    o << "        vars[" << ng << "] = 0;\n";
    // The unit's page count (vars of the unit set, vars[ng] = 0).
    auto npg_expr = [&](const std::string& ind) {
        const int term = spec.inner_dyn_term.empty() ? -1 : spec.inner_dyn_term[0];
        if (term >= 0) o << ind << "i64 npg = indirect_index(A, " << term << ", vars, " << ng << ");\n";
        else o << ind << "i64 npg = A.ext[" << ng << "];\n";
        o << ind << "if (npg < 0) npg = 0;\n";
    };
    npg_expr("        ");
    o << "        if (npg > maxp) { npg = maxp; if (blockIdx.x == 0) *A.err = 3; }\n";
    // Pages of more than 16 tokens are folded as 16-token sub-pages, pages of
    // 8 tokens two to a 16-token step: the prefixes, the split and the
    // stream count steps.
    if (d.pg == 8) o << "        n_[i] = static_cast<int>((npg + 1) / 2);\n";
    else o << "        n_[i] = static_cast<int>(npg) * " << std::max(1, d.pg / 16) << ";\n";
    o << "        run += n_[i];\n";
    o << "        crun += DecodeSplit::cost(n_[i]);\n";
    o << "      }\n";
    o << "    }\n";
    o << "    int x = run, cx = crun;\n";
    o << "#pragma unroll\n";
    o << "    for (int d_ = 1; d_ < 64; d_ <<= 1) {\n";
    o << "      const int y = __shfl_up(x, d_), cy = __shfl_up(cx, d_);\n";
    o << "      if (lane >= d_) { x += y; cx += cy; }\n";
    o << "    }\n";
    o << "    if (lane == 63) { wsum[wave] = x; cwsum[wave] = cx; }\n";
    o << "    __syncthreads();\n";
    o << "    int base = x - run, cbase = cx - crun;\n";
    o << "    for (int j = 0; j < wave; ++j) { base += wsum[j]; cbase += cwsum[j]; }\n";
    o << "#pragma unroll\n";
    o << "    for (int i = 0; i < DecodeSplit::kMaxUnits / " << nt << "; ++i)\n";
    o << "      if (i < per && u0 + i < U) {\n";
    o << "        pre[u0 + i] = base; base += n_[i];\n";
    o << "        cpre[u0 + i] = cbase; cbase += DecodeSplit::cost(n_[i]);\n";
    o << "      }\n";
    o << "    if (tid == 0) {\n";
    o << "      int t_ = 0, c_ = 0;\n";
    o << "      for (int j = 0; j < " << nw << "; ++j) { t_ += wsum[j]; c_ += cwsum[j]; }\n";
    o << "      pre[U] = t_;\n";
    o << "      cpre[U] = c_;\n";
    o << "    }\n";
    o << "    __syncthreads();\n";
    o << "  }\n";
    if (spec.decode_norm) {
        // The folded normalisation's output tile of a unit (slot ntens + 1,
        // affine over the grid variables), with its bounds check.
        const int q = ntens + 1;
        std::ostringstream e;
        e << "(i64)0";
        for (int v = 0; v < ng; ++v) e << " + A.coef[" << q << "][" << v << "] * vars[" << v << "]";
        o << "  auto norm_check = [&](const i64* vars) {\n";
        o << "    const i64 o_ = " << e.str() << ";\n";
        o << "    if (o_ < 0 || o_ + (i64)" << d.g - 1 << " * A.s3[" << q << "] + (i64)" << d.d - 1 << " * A.s4[" << q
          << "] >= A.span[" << q << "]) { if (lane == 0) *A.err = 2; return false; }\n";
        o << "    return true;\n";
        o << "  };\n";
        o << "  auto norm_ptr = [&](const i64* vars) { return reinterpret_cast<float*>(A.base[" << q << "] + (" << e.str()
          << ") * 4); };\n";
    }
    // Values read from LDS are wave-uniform: readfirstlane keeps the page
    // loop's control and addresses in scalar registers.
    o << "  const i64 TC = __builtin_amdgcn_readfirstlane(cpre[U]);\n";
    // Active waves: at most one per cost position, so that no wave's cost
    // range is empty and a unit's partials fill consecutive slots (a wave
    // whose range holds only cost positions, and no page, returns here).
    o << "  const i64 W = (i64)gridDim.x * " << nw << " < TC ? (i64)gridDim.x * " << nw << " : TC, w = (i64)blockIdx.x * " << nw
      << " + wave;\n";
    o << "  if (w < W) {\n";
    o << "  const i64 s = DecodeSplit::page_at(pre, cpre, U, w * TC / W);\n";
    o << "  const i64 b = DecodeSplit::page_at(pre, cpre, U, (w + 1) * TC / W);\n";
    o << "  if (s < b) {\n";
    o << "  int* cnt = reinterpret_cast<int*>(A.base[" << ntens << "]);\n";
    o << "  float* partials = reinterpret_cast<float*>(A.base[" << ntens << "] + DecodeSplit::kMaxUnits * 4);\n";
    // Offsets of global (sub-)page g (per lane): its unit, the page index
    // within the unit, the affine and page-table terms, and for pages of
    // more than 16 tokens the sub-page's first token (its token stride: s4
    // of the K^T and mask tiles, s3 of the V tile).  With 8-token pages the
    // argument is a half-step index (two pages per step).  The 16-token
    // (8-token) tile that is loaded is bounds-checked; an out-of-range one
    // raises the error flag and reads the tensor's first tile instead.
    const int sub = std::max(1, d.pg / 16), tok = std::min(16, d.pg);
    o << "  auto f_page = [&](i64 h, PageOffs& po) {\n";
    if (d.pg == 8) o << "    const i64 g = h >> 1;\n";
    else o << "    const i64 g = h;\n";
    o << "    const int uu = DecodeSplit::unit_of(pre, U, g);\n";
    o << "    i64 vars[" << nvars << "];\n";
    decode_vars("uu", "    ");
    if (d.pg == 8) {
        // Half h&1 of step g is page 2*(g - pre[uu]) + (h&1) of the unit; a
        // unit with an odd page count has no second page in its last step.
        o << "    vars[" << ng << "] = 0;\n";
        o << "    {\n";
        npg_expr("      ");
        o << "      if (npg > maxp) npg = maxp;\n";
        o << "      vars[" << ng << "] = 2 * (g - pre[uu]) + (h & 1);\n";
        o << "      if (vars[" << ng << "] >= npg) { po.k = -1; po.v = 0; po.m = 0; return; }\n";
        o << "    }\n";
        o << "    const i64 t0_ = 0;\n";
    } else if (sub == 1) {
        o << "    vars[" << ng << "] = g - pre[uu];\n";
        o << "    const i64 t0_ = 0;\n";
    } else {
        o << "    const i64 vp_ = g - pre[uu];\n";
        o << "    vars[" << ng << "] = vp_ / " << sub << ";\n";
        o << "    const i64 t0_ = (vp_ % " << sub << ") * 16;\n";
    }
    auto checked = [&](int p, int rows, int cols, const std::string& field, const std::string& tstride) {
        o << "    { i64 o_ = " << offset_expr(p, nvars, first_term[p], nterms(p)) << " + t0_ * " << tstride << ";\n";
        o << "      if (o_ < 0 || o_ + (i64)" << rows - 1 << " * A.s3[" << p << "] + (i64)" << cols - 1 << " * A.s4[" << p
          << "] >= A.span[" << p << "]) { *A.err = 2; o_ = 0; }\n";
        o << "      po." << field << " = o_; }\n";
    };
    checked(d.kt, d.d, tok, "k", "A.s4[" + std::to_string(d.kt) + "]");
    checked(d.v, tok, d.d, "v", "A.s3[" + std::to_string(d.v) + "]");
    if (d.mask >= 0) checked(d.mask, 1, tok, "m", "A.s4[" + std::to_string(d.mask) + "]");
    else o << "    po.m = 0;\n";
    o << "  };\n";
    o << "  auto f_bases = [&](const PageOffs& po, const u16*& kp, const u16*& vp, const float*& mp) {\n";
    o << "    kp = reinterpret_cast<const u16*>(A.base[" << d.kt << "] + po.k * " << es << ");\n";
    o << "    vp = reinterpret_cast<const u16*>(A.base[" << d.v << "] + po.v * " << es << ");\n";
    if (d.mask >= 0) o << "    mp = reinterpret_cast<const float*>(A.base[" << d.mask << "] + po.m * 4);\n";
    else o << "    mp = nullptr;\n";
    o << "  };\n";
    // q tile of unit u (null, with error 2, when it falls outside q).
    o << "  auto f_q = [&](int u) -> const u16* {\n";
    o << "    i64 vars[" << nvars << "];\n";
    decode_vars("u", "    ");
    o << "    vars[" << ng << "] = 0;\n";
    o << "    bool bad = false;\n";
    unit_check(d.q, d.g, d.d, "bad");
    o << "    return bad ? nullptr : " << ptr(d.q, "const u16*", es) << ";\n";
    o << "  };\n";
    o << "  auto f_slot = [&](int u) { return partials + ((i64)u + w) * DW::kPartFloats; };\n";
    // Folds unit u's partials (slots first .. first+parts-1, in page order)
    // into its accumulators.
    o << "  auto f_combine = [&](int u, int parts, i64 first) {\n";
    o << "    i64 vars[" << nvars << "];\n";
    decode_vars("u", "    ");
    o << "    vars[" << ng << "] = 0;\n";
    o << "    bool bad_acc = false;\n";
    unit_check(d.m, d.g, 1, "bad_acc");
    unit_check(d.l, d.g, 1, "bad_acc");
    unit_check(d.o, d.g, d.d, "bad_acc");
    if (spec.decode_norm) {
        o << "    float* out_ = nullptr;\n";
        o << "    if (!bad_acc) { if (!norm_check(vars)) bad_acc = true; else out_ = norm_ptr(vars); }\n";
    }
    o << "    if (!bad_acc)\n";
    // Accumulators per lane of one combine pass: half as many with two waves
    // per SIMD (half the registers per wave).
    o << "      DecodeCombine<" << d.g << ", " << d.d << ", " << (nw == 8 ? 8 : 16) << ">::run(parts, partials + first * DW::kPartFloats, DW::kPartFloats, "
      << ptr(d.m, "float*", 4) << ", A.s3[" << d.m << "], " << ptr(d.l, "float*", 4) << ", A.s3[" << d.l << "], "
      << ptr(d.o, "float*", 4) << ", A.s3[" << d.o << "], A.s4[" << d.o << "], "
      << (spec.decode_norm ? "out_, A.s3[" + std::to_string(ntens + 1) + "], A.s4[" + std::to_string(ntens + 1) + "]"
                           : std::string("nullptr, 0, 0"))
      << ");\n";
    o << "  };\n";
    o << "  auto fns = decode_fns(f_page, f_bases, f_q, f_slot, f_combine);\n";
    o << "  DecodeStream<DW, " << spec.decode_ring << ", " << (spec.decode_ordered ? "true" : "false") << ">::run(fns, pre, cpre, U, TC, W, w, s, b, cnt, " << scale.str() << ", A.s4[" << d.kt
      << "], A.s3[" << d.v << "], A.s3[" << d.q << "]);\n";
    o << "  }\n";
    o << "  }\n";
    if (spec.decode_norm) {
        const int q = ntens + 1;
        // Units without pages are never completed by a wave: their output is
        // the normalisation of the accumulators as they are.
        o << "  for (int u = blockIdx.x * " << nw << " + wave; u < U; u += gridDim.x * " << nw << ") {\n";
        o << "    if (__builtin_amdgcn_readfirstlane(pre[u + 1]) != __builtin_amdgcn_readfirstlane(pre[u])) continue;\n";
        o << "    i64 vars[" << nvars << "];\n";
        decode_vars("u", "    ");
        o << "    vars[" << ng << "] = 0;\n";
        o << "    bool bad_acc = false;\n";
        unit_check(d.l, d.g, 1, "bad_acc");
        unit_check(d.o, d.g, d.d, "bad_acc");
        o << "    if (bad_acc || !norm_check(vars)) continue;\n";
        o << "    DecodeCombine<" << d.g << ", " << d.d << ", " << (nw == 8 ? 8 : 16) << ">::normalize(" << ptr(d.o, "const float*", 4) << ", A.s3[" << d.o
          << "], A.s4[" << d.o << "], " << ptr(d.l, "const float*", 4) << ", A.s3[" << d.l << "], norm_ptr(vars), A.s3["
          << q << "], A.s4[" << q << "]);\n";
        o << "  }\n";
    }
    o << "}\n";
    ek.source = o.str();
    ek.lds_bytes = static_cast<size_t>((2 * (kDecodeMaxUnits + 1) + 2 * nw) * 4);
    return ek;
}

}  // namespace

// ---------------------------------------------------------------------------
// cpp_src kernels
// ---------------------------------------------------------------------------
// One thread per task runs the body against the reference's task descriptor
// (include/pto/wsp/codegen/abi/kernel_abi.hpp:21-41): args = axis args, the
// (rows, cols) of every tile param, scalar args
// (src/python/pto_codegen.cpp:2503-2545); tensor_ptrs / tensor_strides
// (s3, s4 pairs) in tile-param order.  The body is wrapped as the reference
// wraps it (src/python/pto_codegen.cpp:3294-3324): a `cycles` variable, and
// pto::cpu_sim::reset_cycles / add_cycles / read_cycles with __CPU_SIM set,
// counting per thread.  Each task's cycles go to A.cyc[grid task index].
EmittedKernel emit_custom(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    (void)m;
    const KernelDef& k = *a.def;
    const Node& task = *L.task;
    const int ng = static_cast<int>(L.grid.size());
    if (!L.inner.empty()) throw CompileError("internal: in-kernel loops around a cpp_src kernel");
    const int na = static_cast<int>(task.axis_args.size());
    if (na > kMaxAxisArgs) throw CompileError("kernel " + k.name + ": more than 8 axis arguments");
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    const int nscal = static_cast<int>(task.scalar_args.size());
    EmittedKernel ek;
    ek.entry = entry_name("custom", k);
    ek.threads = 64;
    std::ostringstream o;
    if (k.custom_tu) {
        // cpp_tu_path: the file itself, compiled as device code against the
        // ABI headers (kernel_abi.hpp, ptoisa_bridge.hpp: layouts and cycle
        // counters; no PTO-ISA tile API), defines extern "C" <name>(task,
        // cspt); the launcher below calls it once per task.
        o << "// ptowsp: cpp_tu\n#include \"ptowsp_device.h\"\n#define __CPU_SIM 1\n"
             "#include \"pto/wsp/codegen/abi/kernel_abi.hpp\"\n#include \"pto/wsp/codegen/abi/ptoisa_bridge.hpp\"\n";
        // Every function of the file without an execution space becomes host
        // and device code, so its helpers need no annotation.
        o << "#pragma clang force_cuda_host_device begin\n";
        o << "#line 1 \"cpp_tu of " << k.name << "\"\n" << k.custom_src << "\n";
        o << "#pragma clang force_cuda_host_device end\n";
        o << "using namespace ptowsp;\n";
    } else {
    o << "#include \"ptowsp_device.h\"\nusing namespace ptowsp;\n";
    o << "#define __CPU_SIM 1\n#define PTO_WSP_KERNEL_ATTR __device__\n";
    // The <cstdint> names a body uses (hiprtc provides them in __hip_internal).
    for (const char* t : {"int8_t", "int16_t", "int32_t", "int64_t", "uint8_t", "uint16_t", "uint32_t", "uint64_t"})
        o << "using " << t << " = __hip_internal::" << t << ";\n";
    o << "struct KernelTaskDesc { const uint64_t* args; uint32_t num_args; uint32_t num_axis_args; void* const* tensor_ptrs;\n"
         "  const uint64_t* tensor_strides; uint32_t num_tensors; uint32_t kernel_id; uint32_t task_id; };\n";
    o << "struct CSPTContext;\n";
    o << "namespace pto { namespace cpu_sim {\n"
         "__device__ inline void ptowsp_add_cycles(uint64_t& c, uint64_t n) { c += n; }\n"
         "__device__ inline void ptowsp_reset_cycles(uint64_t& c) { c = 0; }\n"
         "__device__ inline uint64_t ptowsp_read_cycles(const uint64_t& c) { return c; }\n"
         "} }\n";
    o << "#define add_cycles(n) ptowsp_add_cycles(ptowsp_cyc_, (n))\n#define reset_cycles() ptowsp_reset_cycles(ptowsp_cyc_)\n"
         "#define read_cycles() ptowsp_read_cycles(ptowsp_cyc_)\n";
    o << "__device__ __noinline__ uint64_t ptowsp_body(const KernelTaskDesc* task, CSPTContext* cspt) {\n"
         "  uint64_t ptowsp_cyc_ = 0;\n  (void)ptowsp_cyc_;\n  (void)task;\n  (void)cspt;\n  uint64_t cycles = 0;\n"
         "#if defined(__CPU_SIM)\n  pto::cpu_sim::reset_cycles();\n#endif\n";
    o << "#line 1 \"cpp_src of " << k.name << "\"\n" << k.custom_src << "\n";
    o << "#if defined(__CPU_SIM)\n  if (cycles == 0) cycles = pto::cpu_sim::read_cycles();\n#endif\n  return cycles;\n}\n";
    o << "#undef add_cycles\n#undef reset_cycles\n#undef read_cycles\n";
    }
    o << "extern \"C\" __global__ void __launch_bounds__(64) " << ek.entry << "(const LaunchArgs A) {\n";
    o << "  i64 vars[" << (ng > 0 ? ng : 1) << "];\n  (void)vars;\n";
    if (k.custom_tu) o << "  pto::cpu_sim::reset_cycles();\n";
    if (spec.serial) o << "  if (blockIdx.x != 0 || threadIdx.x != 0) return;\n  for (i64 t = 0; t < A.ntasks; ++t) {\n";
    else o << "  for (i64 t = (i64)blockIdx.x * 64 + threadIdx.x; t < A.ntasks; t += (i64)gridDim.x * 64) {\n";
    o << "    const i64 g = " << (spec.task_list ? "A.tlist[t]" : "t") << ";\n";
    emit_decode(o, "    ", ng, "g");
    const int nargs = na + 2 * ntens + nscal;
    o << "    uint64_t args[" << (nargs > 0 ? nargs : 1) << "];\n";
    for (int i = 0; i < na; ++i) {
        const ArgRef& r = task.axis_args[i];
        int gv = -1;
        if (r.kind == 'v')
            for (int v = ng - 1; v >= 0 && gv < 0; --v)
                if (L.grid[v].var == r.var) gv = v;
        if (gv >= 0) o << "    args[" << i << "] = (uint64_t)vars[" << gv << "];\n";
        else o << "    args[" << i << "] = A.aarg[" << i << "];\n";
    }
    for (int p = 0; p < ntens; ++p) {
        const ValueInfo* v = a.by_id[k.params[a.tensor_param_index[p]].id];
        o << "    args[" << (na + 2 * p) << "] = " << v->rows << "ull; args[" << (na + 2 * p + 1) << "] = " << v->cols << "ull;\n";
    }
    for (int i = 0; i < nscal; ++i) o << "    args[" << (na + 2 * ntens + i) << "] = A.scal[" << i << "];\n";
    o << "    void* ptrs[" << (ntens > 0 ? ntens : 1) << "];\n    uint64_t strides[" << (ntens > 0 ? 2 * ntens : 1) << "];\n";
    int term = 0;
    for (int p = 0; p < ntens; ++p) {
        const ValueInfo* v = a.by_id[k.params[a.tensor_param_index[p]].id];
        const int nt = spec.indirect_count.size() > static_cast<size_t>(p) ? spec.indirect_count[p] : 0;
        o << "    { const i64 o_ = " << offset_expr(p, ng, term, nt) << ";\n";
        o << "      if (o_ < 0 || o_ + (i64)" << (v->rows - 1) << " * A.s3[" << p << "] + (i64)" << (v->cols - 1) << " * A.s4[" << p
          << "] >= A.span[" << p << "]) { *A.err = 2; continue; }\n";
        o << "      ptrs[" << p << "] = A.base[" << p << "] + o_ * " << dtype_size(v->dtype) << "; }\n";
        o << "    strides[" << 2 * p << "] = (uint64_t)A.s3[" << p << "]; strides[" << 2 * p + 1 << "] = (uint64_t)A.s4[" << p << "];\n";
        term += nt;
    }
    // kernel_id and task_id are 0, as the reference's cpu_sim artifact passes
    // them (src/python/pto_codegen.cpp:2645-2649); cspt is null.
    o << "    const KernelTaskDesc d = {args, " << nargs << "u, " << (na + 2 * ntens) << "u, ptrs, strides, " << ntens << "u, 0u, 0u};\n";
    o << "    A.cyc[g] = " << (k.custom_tu ? k.name : std::string("ptowsp_body")) << "(&d, nullptr);\n  }\n}\n";
    ek.source = o.str();
    return ek;
}

EmittedKernel emit_launch(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec) {
    if (a.family == Family::Custom) return emit_custom(m, a, L, spec);
    if (spec.gemm && a.family == Family::Gemm && !spec.serial) return emit_gemm(m, a, L, spec);
    if (spec.decode && a.family == Family::Decode && !spec.serial) return emit_decode(m, a, L, spec);
    bool indirect = false;
    for (int c : spec.indirect_count) indirect = indirect || c > 0;
    if (a.family == Family::RowProgram && (L.inner.empty() || spec.row_loops) && !indirect && !spec.serial)
        return emit_row(m, a, L, spec);
    return emit_tile(m, a, L, spec);
}

}  // namespace ptowsp
