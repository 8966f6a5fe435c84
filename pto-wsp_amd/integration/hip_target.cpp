// Reference-side half of the "hip_gfx950" target (see hip_target.hpp).
#include "hip_target.hpp"

#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <array>
#include <charconv>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <variant>
#include <vector>

namespace ir = pto::wsp::ir;

namespace ptowsp_integration {

namespace {

// Token-safe string: bytes outside [A-Za-z0-9_.:-] become %XX; "" becomes "%".
std::string enc(const std::string& s) {
    if (s.empty()) return "%";
    static const char kHex[] = "0123456789ABCDEF";
    std::string out;
    for (unsigned char c : s) {
        const bool safe = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' ||
                          c == '.' || c == ':' || c == '-';
        if (safe) {
            out += static_cast<char>(c);
        } else {
            out += '%';
            out += kHex[c >> 4];
            out += kHex[c & 15];
        }
    }
    return out;
}

const char* dtype_name(ir::DType d) {
    switch (d) {
        case ir::DType::F16: return "f16";
        case ir::DType::BF16: return "bf16";
        case ir::DType::F32: return "f32";
        case ir::DType::F64: return "f64";
        case ir::DType::I8: return "i8";
        case ir::DType::I16: return "i16";
        case ir::DType::I32: return "i32";
        case ir::DType::I64: return "i64";
        case ir::DType::U8: return "u8";
        case ir::DType::U16: return "u16";
        case ir::DType::U32: return "u32";
        case ir::DType::U64: return "u64";
        case ir::DType::Bool: return "bool";
    }
    throw std::runtime_error("write_ptowsp_module_text: unknown dtype");
}

// Shortest decimal form that reads back as the same double.
std::string double_text(double v) {
    std::array<char, 64> buf{};
    const auto r = std::to_chars(buf.data(), buf.data() + buf.size(), v);
    if (r.ec != std::errc()) throw std::runtime_error("write_ptowsp_module_text: bad double attribute");
    std::string s(buf.data(), r.ptr);
    // A value with an integral text form keeps a fraction so it stays a float token.
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
    return s;
}

char type_code(ir::ScalarType t) {
    switch (t) {
        case ir::ScalarType::Bool: return 'b';
        case ir::ScalarType::I64: return 'i';
        case ir::ScalarType::U64: return 'u';
    }
    throw std::runtime_error("write_ptowsp_module_text: unknown scalar type");
}

// ScalarExpr in the module's prefix token form:
//   Lb 0|1 | Li v | Lu v | P ty i | G id | A ty id | Y id | S ty i |
//   U op e | B op e e | T e e e | C ty e
void write_expr(const ir::ScalarExpr& e, std::ostringstream& o) {
    if (!e) throw std::runtime_error("write_ptowsp_module_text: null ScalarExpr");
    switch (e->kind) {
        case ir::ScalarExprKind::LiteralBool:
            o << " Lb " << (static_cast<const ir::LiteralBoolExpr&>(*e).value ? 1 : 0);
            return;
        case ir::ScalarExprKind::LiteralI64: o << " Li " << static_cast<const ir::LiteralI64Expr&>(*e).value; return;
        case ir::ScalarExprKind::LiteralU64: o << " Lu " << static_cast<const ir::LiteralU64Expr&>(*e).value; return;
        case ir::ScalarExprKind::TaskParam:
            o << " P " << type_code(e->type) << ' ' << static_cast<const ir::TaskParamExpr&>(*e).index;
            return;
        case ir::ScalarExprKind::TaskTagU64: o << " G " << static_cast<const ir::TaskTagU64Expr&>(*e).tag_id; return;
        case ir::ScalarExprKind::AxisVar:
            o << " A " << type_code(e->type) << ' ' << static_cast<const ir::AxisVarExpr&>(*e).axis_id;
            return;
        case ir::ScalarExprKind::SymbolU64: o << " Y " << static_cast<const ir::SymbolU64Expr&>(*e).symbol_id; return;
        case ir::ScalarExprKind::Slot:
            o << " S " << type_code(e->type) << ' ' << static_cast<const ir::SlotExpr&>(*e).index;
            return;
        case ir::ScalarExprKind::Unary: {
            const auto& u = static_cast<const ir::UnaryExpr&>(*e);
            const char* op = u.op == ir::ScalarUnaryOp::Not ? "!" : u.op == ir::ScalarUnaryOp::Neg ? "-" : "~";
            o << " U " << op;
            write_expr(u.expr, o);
            return;
        }
        case ir::ScalarExprKind::Binary: {
            const auto& b = static_cast<const ir::BinaryExpr&>(*e);
            o << " B " << ir::binaryOpToString(b.op);
            write_expr(b.lhs, o);
            write_expr(b.rhs, o);
            return;
        }
        case ir::ScalarExprKind::Ternary: {
            const auto& t = static_cast<const ir::TernaryExpr&>(*e);
            o << " T";
            write_expr(t.cond, o);
            write_expr(t.then_expr, o);
            write_expr(t.else_expr, o);
            return;
        }
        case ir::ScalarExprKind::Cast: {
            const auto& c = static_cast<const ir::CastExpr&>(*e);
            o << " C " << type_code(c.to);
            write_expr(c.expr, o);
            return;
        }
    }
    throw std::runtime_error("write_ptowsp_module_text: unknown ScalarExpr kind");
}

std::string expr_text(const ir::ScalarExpr& e) {
    std::ostringstream o;
    write_expr(e, o);
    return o.str().substr(1);
}

std::string index_text(const ir::CodegenIndexExpr& e) {
    return e.is_var ? "v " + enc(e.var) : "c " + std::to_string(e.constant);
}

std::string axis_arg_text(const ir::CodegenAxisArg& a) {
    return a.is_var ? "v " + enc(a.var) : "c " + std::to_string(a.u64);
}

// A scalar argument: loop variable, runtime symbol (name + FNV-1a-64 id, as
// python/pto_wsp/ir_bridge.py:915-919 encodes a Symbol) or constant bits.
std::string scalar_arg_text(const ir::CodegenAxisArg& a) {
    if (a.is_var) return "v " + enc(a.var);
    if (!a.var.empty()) return "s " + enc(a.var) + " " + std::to_string(a.u64);
    return "c " + std::to_string(a.u64);
}

std::string tensor_arg_text(const ir::CodegenTensorArg& t, bool with_param) {
    std::ostringstream o;
    if (with_param) o << enc(t.param) << ' ';
    o << t.tensor_id << ' ' << t.base_rank << ' ' << t.view_rank << ' ' << t.index_exprs.size();
    for (const auto& e : t.index_exprs) o << ' ' << index_text(e);
    return o.str();
}

std::string attr_text(const std::string& key, const ir::AttrValue& v) {
    std::ostringstream o;
    o << enc(key) << ' ';
    if (const auto* x = std::get_if<int64_t>(&v)) o << "i " << *x;
    else if (const auto* d = std::get_if<double>(&v)) o << "d " << double_text(*d);
    else if (const auto* b = std::get_if<bool>(&v)) o << "b " << (*b ? 1 : 0);
    else if (const auto* s = std::get_if<std::string>(&v)) o << "s " << enc(*s);
    else if (const auto* vi = std::get_if<std::vector<int64_t>>(&v)) {
        o << "I " << vi->size();
        for (int64_t x : *vi) o << ' ' << x;
    } else if (const auto* vs = std::get_if<std::vector<std::string>>(&v)) {
        o << "S " << vs->size();
        for (const auto& x : *vs) o << ' ' << enc(x);
    }
    return o.str();
}

class Writer {
public:
    std::ostringstream out;

    void line(const std::string& s) { out << s << '\n'; }

    void kernel(const ir::CodegenKernelDef& kd) {
        int custom = 0;
        std::string src;
        if (auto it = kd.attrs.find("cpp_src"); it != kd.attrs.end()) {
            custom = 1;
            src = std::get<std::string>(it->second);
        } else if (auto jt = kd.attrs.find("cpp_file_src"); jt != kd.attrs.end()) {
            custom = 2;
            src = std::get<std::string>(jt->second);
        }
        if (custom && kd.attrs.count("cpp_includes"))
            throw std::runtime_error("kernel " + kd.name + ": cpp_includes name host headers; device bodies cannot include them");
        std::ostringstream h;
        h << "K " << enc(kd.name) << ' ' << kd.values.size() << ' ' << kd.params.size() << ' ' << kd.ops.size() << ' ' << custom;
        if (custom) h << ' ' << enc(src);
        line(h.str());
        for (const auto& [id, v] : kd.values) {
            std::ostringstream l;
            l << "V " << id << ' ' << dtype_name(v.dtype);
            if (v.has_shape) l << " T " << v.rows << ' ' << v.cols;
            else l << " S";
            line(l.str());
        }
        // The IR carries no param direction; the target derives reads and
        // writes from the ops.
        for (const auto& p : kd.params) line("P " + enc(p.name) + " " + std::to_string(p.id) + " in");
        for (const auto& op : kd.ops) {
            std::ostringstream l;
            l << "O " << op.kind << ' ' << (op.has_result ? op.result : -1) << ' ' << op.operands.size();
            for (int x : op.operands) l << ' ' << x;
            std::vector<std::string> keys;
            for (const auto& kv : op.attrs) keys.push_back(kv.first);
            std::sort(keys.begin(), keys.end());
            l << ' ' << keys.size();
            for (const auto& k : keys) l << ' ' << attr_text(k, op.attrs.at(k));
            line(l.str());
        }
    }

    std::string axis(const ir::IRPtr<ir::AxisNode>& a) {
        if (!a) throw std::runtime_error("write_ptowsp_module_text: loop without an axis");
        switch (a->kind) {
            case ir::NodeKind::DenseAxis:
                return "dense " + std::to_string(static_cast<const ir::DenseAxisNode&>(*a).size);
            case ir::NodeKind::DenseDynAxis:
                return "dyn " + enc(static_cast<const ir::DenseDynAxisNode&>(*a).size_var);
            case ir::NodeKind::RaggedAxis: {
                const auto& r = static_cast<const ir::RaggedAxisNode&>(*a);
                return "ragged " + enc(r.outer_size_var) + " " + enc(r.lengths_var);
            }
            default: throw std::runtime_error("write_ptowsp_module_text: a sparse axis is only valid under select");
        }
    }

    void node(const ir::IRPtr<ir::WorkloadNode>& n) {
        if (!n) {
            line("empty");
            return;
        }
        switch (n->kind) {
            case ir::NodeKind::Task: {
                const auto& t = static_cast<const ir::TaskNode&>(*n);
                std::ostringstream l;
                l << "task " << enc(t.kernel_name) << ' ' << t.axis_args.size();
                for (const auto& a : t.axis_args) l << ' ' << axis_arg_text(a);
                l << ' ' << t.scalar_args.size();
                for (const auto& a : t.scalar_args) l << ' ' << scalar_arg_text(a);
                l << ' ' << t.tensor_args.size();
                line(l.str());
                for (const auto& ta : t.tensor_args) line("  " + tensor_arg_text(ta, true));
                return;
            }
            case ir::NodeKind::ParallelFor: {
                const auto& p = static_cast<const ir::ParallelForNode&>(*n);
                line("pfor " + enc(p.index_var) + " " + axis(p.axis));
                node(p.body);
                return;
            }
            case ir::NodeKind::ForEach: {
                const auto& p = static_cast<const ir::ForEachNode&>(*n);
                line("each " + enc(p.index_var) + " " + axis(p.axis));
                node(p.body);
                return;
            }
            case ir::NodeKind::Select: {
                const auto& s = static_cast<const ir::SelectNode&>(*n);
                if (!s.sparse) throw std::runtime_error("write_ptowsp_module_text: select without a sparse axis");
                line("sel " + enc(s.index_var) + " " + enc(s.sparse->outer_size_var) + " " + enc(s.sparse->indptr_var) + " " +
                     enc(s.sparse->indices_var));
                node(s.body);
                return;
            }
            case ir::NodeKind::Cond: {
                const auto& c = static_cast<const ir::CondNode&>(*n);
                line("cond " + expr_text(c.predicate));
                node(c.then_branch);
                node(c.else_branch);
                return;
            }
            case ir::NodeKind::Combine:
            case ir::NodeKind::Sequential: {
                const auto& kids = n->kind == ir::NodeKind::Combine ? static_cast<const ir::CombineNode&>(*n).workloads
                                                                    : static_cast<const ir::SequentialNode&>(*n).workloads;
                line(std::string(n->kind == ir::NodeKind::Combine ? "comb " : "seqn ") + std::to_string(kids.size()));
                for (const auto& k : kids) node(k);
                return;
            }
            case ir::NodeKind::SlotSetU64: {
                const auto& s = static_cast<const ir::SlotSetU64Node&>(*n);
                line("slotset " + std::to_string(s.slot) + " " + std::to_string(s.value));
                return;
            }
            case ir::NodeKind::SlotLoadU64: {
                const auto& s = static_cast<const ir::SlotLoadU64Node&>(*n);
                line("slotld " + std::to_string(s.slot) + " " + tensor_arg_text(s.tensor, false) + " " + std::to_string(s.row) +
                     " " + std::to_string(s.col));
                return;
            }
            default:
                throw std::runtime_error("write_ptowsp_module_text: workload node kind " +
                                         std::to_string(static_cast<int>(n->kind)) + " (Call or a CSP node) is not supported by the hip_gfx950 target");
        }
    }

    void schedule(const ir::ScheduleDef* s) {
        std::vector<std::string> d;
        if (s) {
            // Same order as pto_wsp/ir_bridge.py: dispatch, window, streams, timing.
            if (auto dn = s->dispatch()) {
                const char* pol = "round_robin";
                switch (dn->policy) {
                    case ir::DispatchPolicy::RoundRobin: pol = "round_robin"; break;
                    case ir::DispatchPolicy::Affinity: pol = "affinity"; break;
                    case ir::DispatchPolicy::Hash: pol = "hash"; break;
                    case ir::DispatchPolicy::WorkSteal: pol = "work_steal"; break;
                    case ir::DispatchPolicy::Custom: pol = "dispatch_by"; break;
                }
                std::string l = std::string("D ") + pol + " " + std::to_string(dn->num_targets) + " ";
                l += dn->key ? "1 " + expr_text(dn->key) : "0";
                d.push_back(l);
            }
            for (const auto& x : s->directives) {
                if (x->kind != ir::NodeKind::TaskWindow) continue;
                const auto& w = static_cast<const ir::TaskWindowNode&>(*x);
                const char* ov = w.overflow == ir::TaskWindowOverflowPolicy::Abort       ? "abort"
                                 : w.overflow == ir::TaskWindowOverflowPolicy::Benchmark ? "benchmark"
                                                                                         : "stall";
                d.push_back("W " + std::to_string(w.size) + " " + enc(w.unit) + " " + ov);
            }
            if (auto sn = s->stream(); sn && sn->num_streams != 1)
                d.push_back("S " + std::to_string(sn->num_streams) + " " + ((sn->key || !sn->key_expr.empty()) ? "1" : "0"));
            if (auto tn = s->timing()) {
                const char* k = "immediate";
                switch (tn->policy) {
                    case ir::TimingPolicy::Immediate: k = "immediate"; break;
                    case ir::TimingPolicy::Batched: k = "batched"; break;
                    case ir::TimingPolicy::Interleaved: k = "interleaved"; break;
                    case ir::TimingPolicy::RateLimited: k = "rate_limit"; break;
                }
                d.push_back(std::string("M ") + k);
            }
        }
        line("schedule " + std::to_string(d.size()));
        for (const auto& x : d) line(x);
    }
};

bool file_exists(const std::string& p) {
    struct stat st;
    return ::stat(p.c_str(), &st) == 0;
}

void make_dirs(const std::string& dir) {
    std::string cur;
    std::stringstream ss(dir);
    std::string part;
    if (!dir.empty() && dir[0] == '/') cur = "/";
    while (std::getline(ss, part, '/')) {
        if (part.empty()) continue;
        cur += part + "/";
        ::mkdir(cur.c_str(), 0755);
    }
}

std::string hex16(uint64_t v) {
    char buf[17];
    std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(v));
    return buf;
}

// Runs `cmd` through the shell; throws with its output when it fails.
void run_or_throw(const std::string& cmd) {
    std::unique_ptr<FILE, int (*)(FILE*)> p(::popen((cmd + " 2>&1").c_str(), "r"), ::pclose);
    if (!p) throw std::runtime_error("cannot run: " + cmd);
    std::string log;
    std::array<char, 4096> buf{};
    while (std::fgets(buf.data(), static_cast<int>(buf.size()), p.get())) log += buf.data();
    const int rc = ::pclose(p.release());
    if (rc != 0) throw std::runtime_error("command failed (" + std::to_string(rc) + "): " + cmd + "\n" + log);
}

std::string shell_quote(const std::string& s) {
    std::string out = "'";
    for (char c : s) out += c == '\'' ? std::string("'\\''") : std::string(1, c);
    return out + "'";
}

}  // namespace

uint64_t fnv1a_64(const std::string& s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) h = (h ^ c) * 0x100000001b3ull;
    return h;
}

std::string c_string_literal(const std::string& s) {
    std::string out = "\"";
    for (unsigned char c : s) {
        if (c == '\\' || c == '"') {
            out += '\\';
            out += static_cast<char>(c);
        } else if (c == '\n') {
            out += "\\n\"\n\"";
        } else if (c < 0x20 || c >= 0x7f) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\%03o", c);
            out += buf;
        } else {
            out += static_cast<char>(c);
        }
    }
    return out + "\"";
}

std::string write_ptowsp_module_text(const ir::Module& m) {
    if (m.workloads.empty()) throw std::runtime_error("Module has no workloads");
    if (!m.pipelines.empty()) throw std::runtime_error("write_ptowsp_module_text: CSP pipelines are not supported by the hip_gfx950 target");
    const ir::WorkloadDef& wl = m.workloads[0];  // the workload the reference's codegen emits
    Writer w;
    w.line("PTOWSP-MODULE 1");
    w.line("name " + enc(m.name.empty() ? std::string("main") : m.name));
    w.line("tensors " + std::to_string(m.tensors.size()));
    for (const auto& t : m.tensors) {
        std::ostringstream l;
        l << "T " << dtype_name(t.dtype) << ' ' << t.shape.size();
        for (int64_t d : t.shape) l << ' ' << d;
        w.line(l.str());
    }
    w.line("kernels " + std::to_string(m.kernels.size()));
    for (const auto& kd : m.kernels) w.kernel(kd);
    w.line("workload " + enc(wl.name.empty() ? std::string("unnamed") : wl.name));
    w.node(wl.body);
    w.schedule(m.findScheduleForWorkload(wl.name));
    w.line("end");
    return w.out.str();
}

HipArtifact build_hip_artifact(const std::string& module_text, const std::string& module_name,
                               const std::string& cache_root, const std::string& include_dir, const std::string& lib_dir) {
    const std::string name = module_name.empty() ? std::string("main") : module_name;
    for (char c : name)
        if (!((c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_'))
            throw std::runtime_error("build_hip_artifact: module name '" + name + "' is not a C identifier");
    HipArtifact a;
    a.entrypoint = name + "_main";
    a.cache_key = hex16(fnv1a_64(module_text + "\n" + lib_dir + "/libptowsp_hip.so"));
    const std::string dir = cache_root + "/" + name + "_hip_" + a.cache_key;
    a.so_path = dir + "/libhip_entry.so";
    if (file_exists(a.so_path)) return a;
    make_dirs(dir);
    {
        std::ofstream c(dir + "/hip_entry.c", std::ios::binary);
        c << "/* Entry of module " << name << " on the hip_gfx950 target (generated). */\n"
          << "#include <stdint.h>\n#include \"ptowsp_hip.h\"\n"
          << "static const char kText[] =\n" << c_string_literal(module_text) << ";\n"
          << "static ptowsp_program* g_prog;\n"
          << "uint64_t " << a.entrypoint << "(RuntimeContext* ctx, CSPTContext* cspt) {\n"
          << "    if (!g_prog && ptowsp_hip_compile(kText, &g_prog) != 0) return 0;\n"
          << "    return ptowsp_hip_workload_main(g_prog, ctx, cspt);\n}\n";
        if (!c) throw std::runtime_error("build_hip_artifact: cannot write " + dir + "/hip_entry.c");
    }
    const char* cc_env = std::getenv("PTO_WSP_CODEGEN_CC");
    const std::string cc = cc_env && *cc_env ? cc_env : "cc";
    const std::string tmp = a.so_path + ".tmp" + std::to_string(::getpid());
    run_or_throw(cc + " -O2 -std=c99 -shared -fPIC -I" + shell_quote(include_dir) + " " + shell_quote(dir + "/hip_entry.c") + " -o " +
                 shell_quote(tmp) + " -L" + shell_quote(lib_dir) + " -lptowsp_hip -Wl,-rpath," + shell_quote(lib_dir));
    if (std::rename(tmp.c_str(), a.so_path.c_str()) != 0) throw std::runtime_error("build_hip_artifact: cannot move " + tmp);
    return a;
}

}  // namespace ptowsp_integration
