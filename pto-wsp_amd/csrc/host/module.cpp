// Parser for the "PTOWSP-MODULE 1" text (token stream; see module.hpp).
#include "module.hpp"

#include <cstdlib>
#include <cstring>

namespace ptowsp {

namespace {

const char* kDTypeNames[] = {"f16", "bf16", "f32", "f64", "i8", "i16", "i32", "i64", "u8", "u16", "u32", "u64", "bool"};
const int kDTypeSizes[] = {2, 2, 4, 8, 1, 2, 4, 8, 1, 2, 4, 8, 1};

class Lexer {
public:
    explicit Lexer(const std::string& s) : s_(s) {}

    std::string tok() {
        while (pos_ < s_.size() && is_space(s_[pos_])) ++pos_;
        if (pos_ >= s_.size()) throw CompileError("module text: unexpected end of input");
        size_t start = pos_;
        while (pos_ < s_.size() && !is_space(s_[pos_])) ++pos_;
        return s_.substr(start, pos_ - start);
    }

    void expect(const char* want) {
        std::string t = tok();
        if (t != want) throw CompileError(std::string("module text: expected '") + want + "', got '" + t + "'");
    }

    int64_t i64() {
        std::string t = tok();
        char* e = nullptr;
        long long v = std::strtoll(t.c_str(), &e, 10);
        if (*e) throw CompileError("module text: bad integer '" + t + "'");
        return v;
    }

    uint64_t u64() {
        std::string t = tok();
        char* e = nullptr;
        unsigned long long v = std::strtoull(t.c_str(), &e, 10);
        if (*e) throw CompileError("module text: bad unsigned '" + t + "'");
        return v;
    }

    double f64() {
        std::string t = tok();
        char* e = nullptr;
        double v = std::strtod(t.c_str(), &e);
        if (*e) throw CompileError("module text: bad float '" + t + "'");
        return v;
    }

    std::string str() {
        std::string t = tok();
        if (t == "%") return "";
        std::string out;
        for (size_t i = 0; i < t.size();) {
            const bool room = i + 2 < t.size();
            int h1 = room ? hex(t[i + 1]) : -1;
            int h2 = room ? hex(t[i + 2]) : -1;
            if (t[i] == '%' && h1 >= 0 && h2 >= 0) {
                out.push_back(static_cast<char>(h1 * 16 + h2));
                i += 3;
            } else {
                out.push_back(t[i++]);
            }
        }
        return out;
    }

    DType dtype() {
        std::string t = tok();
        for (int i = 0; i < 13; ++i)
            if (t == kDTypeNames[i]) return static_cast<DType>(i);
        throw CompileError("module text: unknown dtype '" + t + "'");
    }

private:
    static bool is_space(char c) { return c == ' ' || c == '\n' || c == '\t' || c == '\r'; }
    static int hex(char c) {
        if (c >= '0' && c <= '9') return c - '0';
        if (c >= 'A' && c <= 'F') return c - 'A' + 10;
        if (c >= 'a' && c <= 'f') return c - 'a' + 10;
        return -1;
    }
    const std::string& s_;
    size_t pos_ = 0;
};

OpKind op_kind(const std::string& s) {
    static const std::pair<const char*, OpKind> table[] = {
        {"Load", OpKind::Load},     {"Store", OpKind::Store},     {"Add", OpKind::Add},
        {"Sub", OpKind::Sub},       {"Mul", OpKind::Mul},         {"Div", OpKind::Div},
        {"Max", OpKind::Max},       {"Min", OpKind::Min},         {"Exp", OpKind::Exp},
        {"Rsqrt", OpKind::Rsqrt},   {"RowSum", OpKind::RowSum},   {"RowMax", OpKind::RowMax},
        {"RowMean", OpKind::RowMean}, {"Matmul", OpKind::Matmul}, {"Constant", OpKind::Constant},
        {"IotaU32", OpKind::IotaU32}, {"TSort32", OpKind::TSort32}, {"ExtractTopkIndices", OpKind::ExtractTopkIndices},
        {"TMov", OpKind::TMov}, {"StoreTopkIndices", OpKind::StoreTopkIndices},
        {"CpuSimAddCycles", OpKind::CpuSimAddCycles}};
    for (const auto& [n, k] : table)
        if (s == n) return k;
    return OpKind::Other;
}

void parse_attr(Lexer& L, OpInfo& op) {
    std::string key = L.str();
    std::string ty = L.tok();
    bool is_value = key == "value";
    if (ty == "i" || ty == "b") {
        int64_t v = L.i64();
        if (is_value) { op.has_value = true; op.value = static_cast<double>(v); }
        else if (ty == "i") op.ints[key] = v;
    } else if (ty == "d") {
        double v = L.f64();
        if (is_value) { op.has_value = true; op.value = v; }
    } else if (ty == "s") {
        const std::string v = L.str();
        if (key == "cycles_expr") {
            // A scalar expression in the prefix token form, as one string.
            size_t pos = 0;
            auto next = [&]() -> std::string {
                while (pos < v.size() && v[pos] == ' ') ++pos;
                const size_t b = pos;
                while (pos < v.size() && v[pos] != ' ') ++pos;
                return v.substr(b, pos - b);
            };
            op.cycles_expr = std::shared_ptr<const SExpr>(parse_scalar(next));
            if (!next().empty()) throw CompileError("module text: trailing tokens in a cycles expression");
        }
    } else if (ty == "I") {
        int64_t n = L.i64();
        for (int64_t i = 0; i < n; ++i) (void)L.i64();
    } else if (ty == "S") {
        int64_t n = L.i64();
        for (int64_t i = 0; i < n; ++i) (void)L.str();
    } else {
        throw CompileError("module text: bad attr type '" + ty + "'");
    }
}

KernelDef parse_kernel(Lexer& L) {
    KernelDef k;
    L.expect("K");
    k.name = L.str();
    int64_t nv = L.i64(), np = L.i64(), no = L.i64();
    const int64_t custom = L.i64();
    if (custom < 0 || custom > 2) throw CompileError("kernel " + k.name + ": unknown custom-kernel kind " + std::to_string(custom));
    k.custom = custom != 0;
    k.custom_tu = custom == 2;
    if (k.custom) k.custom_src = L.str();
    for (int64_t i = 0; i < nv; ++i) {
        L.expect("V");
        ValueInfo v;
        v.id = static_cast<int>(L.i64());
        v.dtype = L.dtype();
        std::string kind = L.tok();
        v.tile = kind == "T";
        if (v.tile) {
            v.rows = static_cast<int>(L.i64());
            v.cols = static_cast<int>(L.i64());
            if (v.rows <= 0 || v.cols <= 0)
                throw CompileError("kernel " + k.name + ": tile value " + std::to_string(v.id) + " has an empty shape");
        }
        k.values.push_back(v);
    }
    for (int64_t i = 0; i < np; ++i) {
        L.expect("P");
        ParamInfo p;
        p.name = L.str();
        p.id = static_cast<int>(L.i64());
        p.direction = L.tok();
        k.params.push_back(p);
    }
    for (int64_t i = 0; i < no; ++i) {
        L.expect("O");
        OpInfo op;
        op.kind_name = L.tok();
        op.kind = op_kind(op.kind_name);
        op.result = static_cast<int>(L.i64());
        int64_t n = L.i64();
        for (int64_t j = 0; j < n; ++j) op.operands.push_back(static_cast<int>(L.i64()));
        int64_t na = L.i64();
        for (int64_t j = 0; j < na; ++j) parse_attr(L, op);
        k.ops.push_back(op);
    }
    return k;
}

IndexExpr parse_index(Lexer& L) {
    IndexExpr e;
    std::string k = L.tok();
    e.kind = k.empty() ? '?' : k[0];
    switch (e.kind) {
        case 'v': e.var = L.str(); break;
        case 'c': e.c = L.i64(); break;
        case 'a': {
            e.c = L.i64();
            int64_t n = L.i64();
            for (int64_t i = 0; i < n; ++i) {
                std::string v = L.str();
                int64_t coef = L.i64();
                e.terms.emplace_back(v, coef);
            }
            break;
        }
        case 't': {
            e.tid = static_cast<int>(L.i64());
            e.base_rank = static_cast<int>(L.i64());
            int64_t n = L.i64();
            for (int64_t i = 0; i < n; ++i) e.idx.push_back(parse_index(L));
            break;
        }
        default: throw CompileError("module text: bad index expression '" + k + "'");
    }
    return e;
}

ArgRef parse_arg(Lexer& L) {
    ArgRef a;
    std::string k = L.tok();
    a.kind = k.empty() ? '?' : k[0];
    if (a.kind == 'v') a.var = L.str();
    else if (a.kind == 'c') a.u64 = L.u64();
    else if (a.kind == 's') { a.var = L.str(); a.u64 = L.u64(); }
    else throw CompileError("module text: bad argument kind '" + k + "'");
    return a;
}

Axis parse_axis(Lexer& L) {
    Axis a;
    std::string k = L.tok();
    if (k == "dense") { a.kind = AxisKind::Dense; a.size = L.i64(); }
    else if (k == "dyn") { a.kind = AxisKind::Dyn; a.a = L.str(); }
    else if (k == "ragged") { a.kind = AxisKind::Ragged; a.a = L.str(); a.b = L.str(); }
    else if (k == "dynt") {
        a.kind = AxisKind::DynTensor;
        a.max = L.i64();
        a.expr = parse_index(L);
    }
    else throw CompileError("module text: bad axis kind '" + k + "'");
    return a;
}

std::unique_ptr<SExpr> parse_expr(Lexer& L) {
    try {
        return parse_scalar([&] { return L.tok(); });
    } catch (const std::runtime_error& e) {
        throw CompileError(e.what());
    }
}

std::unique_ptr<Node> parse_node(Lexer& L, const Module& m) {
    auto n = std::make_unique<Node>();
    std::string k = L.tok();
    if (k == "empty") {
        n->kind = NodeKind::Empty;
    } else if (k == "pfor" || k == "each") {
        n->kind = k == "pfor" ? NodeKind::ParallelFor : NodeKind::ForEach;
        n->var = L.str();
        n->axis = parse_axis(L);
        n->body = parse_node(L, m);
    } else if (k == "comb" || k == "seqn") {
        n->kind = k == "comb" ? NodeKind::Combine : NodeKind::Sequential;
        int64_t c = L.i64();
        for (int64_t i = 0; i < c; ++i) n->kids.push_back(parse_node(L, m));
    } else if (k == "task") {
        n->kind = NodeKind::Task;
        n->kernel = L.str();
        for (size_t i = 0; i < m.kernels.size(); ++i)
            if (m.kernels[i].name == n->kernel) n->kernel_index = static_cast<int>(i);
        if (n->kernel_index < 0) throw CompileError("Missing kernel def for task: " + n->kernel);
        int64_t na = L.i64();
        for (int64_t i = 0; i < na; ++i) n->axis_args.push_back(parse_arg(L));
        int64_t ns = L.i64();
        for (int64_t i = 0; i < ns; ++i) n->scalar_args.push_back(parse_arg(L));
        int64_t nt = L.i64();
        for (int64_t i = 0; i < nt; ++i) {
            TensorArg t;
            t.param = L.str();
            t.tid = static_cast<int>(L.i64());
            t.base_rank = static_cast<int>(L.i64());
            t.view_rank = static_cast<int>(L.i64());
            int64_t ni = L.i64();
            for (int64_t j = 0; j < ni; ++j) t.idx.push_back(parse_index(L));
            if (t.tid < 0 || t.tid >= static_cast<int>(m.tensors.size()))
                throw CompileError("task " + n->kernel + ": bad tensor id");
            n->tensor_args.push_back(std::move(t));
        }
    } else if (k == "sel") {
        n->kind = NodeKind::Select;
        n->var = L.str();
        n->axis.kind = AxisKind::Select;
        n->axis.a = L.str();
        n->axis.b = L.str();
        n->axis.c = L.str();
        n->body = parse_node(L, m);
    } else if (k == "cond") {
        n->kind = NodeKind::Cond;
        n->pred = parse_expr(L);
        n->kids.push_back(parse_node(L, m));
        n->kids.push_back(parse_node(L, m));
    } else if (k == "slotset") {
        n->kind = NodeKind::SlotSet;
        n->slot = static_cast<uint32_t>(L.u64());
        n->value = L.u64();
    } else if (k == "slotld") {
        n->kind = NodeKind::SlotLoad;
        n->slot = static_cast<uint32_t>(L.u64());
        TensorArg& t = n->view;
        t.param = "tensor";
        t.tid = static_cast<int>(L.i64());
        t.base_rank = static_cast<int>(L.i64());
        t.view_rank = static_cast<int>(L.i64());
        const int64_t ni = L.i64();
        for (int64_t j = 0; j < ni; ++j) t.idx.push_back(parse_index(L));
        n->row = L.i64();
        n->col = L.i64();
        if (t.tid < 0 || t.tid >= static_cast<int>(m.tensors.size())) throw CompileError("slot_load_u64: bad tensor id");
        if (t.view_rank < 2) throw CompileError("slot_load_u64 tensor view must be rank>=2");
        if (static_cast<size_t>(ni) > m.tensors[t.tid].shape.size()) throw CompileError("slot_load_u64: too many indices");
        switch (m.tensors[t.tid].dtype) {
            case DType::F32: case DType::F16: case DType::I32: case DType::I64: case DType::U32: case DType::U64:
            case DType::Bool: break;
            default:
                throw CompileError(std::string("Unsupported dtype for workload codegen: ") + dtype_name(m.tensors[t.tid].dtype));
        }
    } else {
        throw CompileError("module text: bad node kind '" + k + "'");
    }
    return n;
}

}  // namespace

const char* dtype_name(DType d) { return kDTypeNames[static_cast<int>(d)]; }
int dtype_size(DType d) { return kDTypeSizes[static_cast<int>(d)]; }
bool dtype_is_float(DType d) { return d == DType::F16 || d == DType::BF16 || d == DType::F32 || d == DType::F64; }

uint64_t fnv1a_64(const std::string& s) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001B3ULL;
    }
    return h;
}

Module parse_module(const std::string& text) {
    Lexer L(text);
    Module m;
    L.expect("PTOWSP-MODULE");
    L.expect("1");
    L.expect("name");
    m.name = L.str();
    L.expect("tensors");
    int64_t nt = L.i64();
    for (int64_t i = 0; i < nt; ++i) {
        L.expect("T");
        TensorInfo t;
        t.dtype = L.dtype();
        int64_t rank = L.i64();
        if (rank < 0 || rank > 8) throw CompileError("tensor rank must be in [0, 8]");
        for (int64_t d = 0; d < rank; ++d) t.shape.push_back(L.i64());
        m.tensors.push_back(std::move(t));
    }
    L.expect("kernels");
    int64_t nk = L.i64();
    for (int64_t i = 0; i < nk; ++i) m.kernels.push_back(parse_kernel(L));
    L.expect("workload");
    m.workload_name = L.str();
    m.root = parse_node(L, m);
    L.expect("schedule");
    int64_t nd = L.i64();
    for (int64_t i = 0; i < nd; ++i) {
        std::string d = L.tok();
        if (d == "D") {
            m.schedule.has_dispatch = true;
            m.schedule.dispatch_policy = L.tok();
            m.schedule.num_targets = L.i64();
            if (L.i64() != 0) m.schedule.dispatch_key = parse_expr(L);
            // src/python/pto_codegen.cpp:1547-1556: keyed policies need a ScalarExpr key.
            const std::string& pol = m.schedule.dispatch_policy;
            if (pol != "round_robin" && pol != "work_steal" && !m.schedule.dispatch_key)
                throw CompileError("dispatch policy requires ScalarExpr key (string-eval is not supported in v9 codegen-first)");
        } else if (d == "W") {
            m.schedule.has_window = true;
            m.schedule.window_size = L.i64();
            m.schedule.window_unit = L.str();
            m.schedule.window_overflow = L.tok();
        } else if (d == "S") {
            m.schedule.has_streams = true;
            m.schedule.num_streams = L.i64();
            m.schedule.stream_keyed = L.i64() != 0;
        } else if (d == "M") {
            (void)L.str();
        } else {
            throw CompileError("module text: bad schedule directive '" + d + "'");
        }
    }
    L.expect("end");
    return m;
}

}  // namespace ptowsp
