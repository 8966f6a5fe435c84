#include "scalar.hpp"

#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace ptowsp {

namespace {

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error("scalar expression: " + msg); }

int64_t as_signed(uint64_t v) {
    int64_t r;
    std::memcpy(&r, &v, sizeof r);
    return r;
}

// Integral promotion: bool becomes a signed integer (int, whose values int64_t holds).
SType promoted(SType t) { return t == SType::Bool ? SType::I64 : t; }
SValue promote(SValue x) { return {promoted(x.t), x.v}; }
// Usual arithmetic conversions of two promoted operands.
SType common(SType a, SType b) { return (a == SType::U64 || b == SType::U64) ? SType::U64 : SType::I64; }

bool is_compare(const std::string& op) {
    return op == "<" || op == "<=" || op == ">" || op == ">=" || op == "==" || op == "!=";
}
bool is_logical(const std::string& op) { return op == "&&" || op == "||"; }
bool is_shift(const std::string& op) { return op == "<<" || op == ">>"; }

// The static type of an expression: what the emitted C++ expression has.
SType static_type(const SExpr& e) {
    using K = SExpr::Kind;
    switch (e.kind) {
        case K::LitBool: return SType::Bool;
        case K::LitI64: return SType::I64;
        case K::LitU64:
        case K::TaskTag:
        case K::Symbol: return SType::U64;
        case K::TaskParam:
        case K::KernelScalar:
        case K::AxisVar:
        case K::Slot:
        case K::Cast: return e.type;
        case K::Unary: return e.op == "!" ? SType::Bool : promoted(static_type(*e.a));
        case K::Binary:
            if (is_compare(e.op) || is_logical(e.op)) return SType::Bool;
            if (is_shift(e.op)) return promoted(static_type(*e.a));
            return common(promoted(static_type(*e.a)), promoted(static_type(*e.b)));
        case K::Ternary: {
            const SType t = static_type(*e.b), f = static_type(*e.c);
            if (t == SType::Bool && f == SType::Bool) return SType::Bool;
            return common(promoted(t), promoted(f));
        }
    }
    return SType::I64;
}

// A u64 read with a declared type, as `(int64_t)x`, `(uint64_t)x` or `(bool)(x != 0)`.
SValue typed_read(uint64_t raw, SType t) { return t == SType::Bool ? SValue{SType::Bool, raw != 0} : SValue{t, raw}; }

SValue convert(SValue x, SType to) {
    if (to == SType::Bool) return {SType::Bool, x.v != 0};
    return {to, x.v};  // bool is 0 / 1; i64 <-> u64 keeps the bits
}

SValue binary(const SExpr& e, const SEnv& env) {
    const std::string& op = e.op;
    if (op == "&&") {
        if (eval_scalar(*e.a, env).v == 0) return {SType::Bool, 0};
        return {SType::Bool, eval_scalar(*e.b, env).v != 0};
    }
    if (op == "||") {
        if (eval_scalar(*e.a, env).v != 0) return {SType::Bool, 1};
        return {SType::Bool, eval_scalar(*e.b, env).v != 0};
    }
    const SValue a = promote(eval_scalar(*e.a, env));
    const SValue b = promote(eval_scalar(*e.b, env));
    if (is_shift(op)) {
        if ((b.t == SType::I64 && as_signed(b.v) < 0) || b.v >= 64) fail("shift count out of range");
        const unsigned n = static_cast<unsigned>(b.v);
        if (op == "<<") return {a.t, a.v << n};
        if (a.t == SType::I64) return {SType::I64, static_cast<uint64_t>(as_signed(a.v) >> n)};
        return {SType::U64, a.v >> n};
    }
    const SType t = common(a.t, b.t);
    if (is_compare(op)) {
        bool r;
        if (t == SType::U64) {
            r = op == "<" ? a.v < b.v : op == "<=" ? a.v <= b.v : op == ">" ? a.v > b.v : op == ">=" ? a.v >= b.v
              : op == "==" ? a.v == b.v : a.v != b.v;
        } else {
            const int64_t x = as_signed(a.v), y = as_signed(b.v);
            r = op == "<" ? x < y : op == "<=" ? x <= y : op == ">" ? x > y : op == ">=" ? x >= y
              : op == "==" ? x == y : x != y;
        }
        return {SType::Bool, r};
    }
    if (op == "+") return {t, a.v + b.v};
    if (op == "-") return {t, a.v - b.v};
    if (op == "*") return {t, a.v * b.v};
    if (op == "&") return {t, a.v & b.v};
    if (op == "|") return {t, a.v | b.v};
    if (op == "^") return {t, a.v ^ b.v};
    if (op == "/" || op == "%") {
        if (b.v == 0) fail("division by zero");
        if (t == SType::U64) return {t, op == "/" ? a.v / b.v : a.v % b.v};
        const int64_t x = as_signed(a.v), y = as_signed(b.v);
        if (x == INT64_MIN && y == -1) fail("signed division overflow");
        return {t, static_cast<uint64_t>(op == "/" ? x / y : x % y)};
    }
    fail("unknown binary operator '" + op + "'");
}

}  // namespace

SValue eval_scalar(const SExpr& e, const SEnv& env) {
    using K = SExpr::Kind;
    switch (e.kind) {
        case K::LitBool: return {SType::Bool, e.u != 0};
        case K::LitI64: return {SType::I64, e.u};
        case K::LitU64: return {SType::U64, e.u};
        case K::TaskParam: {
            if (!env.task_param) fail("task_param() outside a task");
            return typed_read(env.task_param(static_cast<uint32_t>(e.u)), e.type);
        }
        case K::KernelScalar: {
            if (!env.kernel_scalar) fail("kernel scalar parameter read outside a task");
            return typed_read(env.kernel_scalar(static_cast<uint32_t>(e.u)), e.type);
        }
        case K::TaskTag: return {SType::U64, env.symbol(e.u)};
        case K::AxisVar: {
            int64_t v = 0;
            if (!env.axis || !env.axis(e.u, v)) fail("axis_var not in scope");
            if (e.type == SType::Bool) fail("axis_var invalid type");
            return {e.type, static_cast<uint64_t>(v)};
        }
        case K::Symbol: return {SType::U64, env.symbol(e.u)};
        case K::Slot: return typed_read(env.slot ? env.slot(static_cast<uint32_t>(e.u)) : 0, e.type);
        case K::Unary: {
            const SValue x = eval_scalar(*e.a, env);
            if (e.op == "!") return {SType::Bool, x.v == 0};
            const SValue p = promote(x);
            if (e.op == "-") return {p.t, 0 - p.v};
            if (e.op == "~") return {p.t, ~p.v};
            fail("unknown unary operator '" + e.op + "'");
        }
        case K::Binary: return binary(e, env);
        case K::Ternary: {
            const SType t = static_type(e);
            const SValue v = eval_scalar(eval_scalar(*e.a, env).v != 0 ? *e.b : *e.c, env);
            return t == SType::Bool ? v : convert(promote(v), t);
        }
        case K::Cast: return convert(promote(eval_scalar(*e.a, env)), e.type);
    }
    fail("unknown expression kind");
}

bool eval_truth(const SExpr& e, const SEnv& env) { return eval_scalar(e, env).v != 0; }

uint64_t eval_u64(const SExpr& e, const SEnv& env) { return eval_scalar(e, env).v; }

void scalar_refs(const SExpr& e, SRefs& out) {
    using K = SExpr::Kind;
    if (e.kind == K::AxisVar) out.axes.push_back(e.u);
    if (e.kind == K::Slot) out.slots = true;
    if (e.kind == K::TaskParam) out.task_params = true;
    if (e.kind == K::KernelScalar) out.kernel_scalars = true;
    if (e.kind == K::Symbol || e.kind == K::TaskTag) out.symbols = true;
    for (const SExpr* k : {e.a.get(), e.b.get(), e.c.get()})
        if (k) scalar_refs(*k, out);
}

std::unique_ptr<SExpr> parse_scalar(const std::function<std::string()>& next) {
    using K = SExpr::Kind;
    auto num_u = [&](const char* what) {
        const std::string t = next();
        char* end = nullptr;
        const unsigned long long v = std::strtoull(t.c_str(), &end, 10);
        if (t.empty() || *end || t[0] == '-') fail(std::string("bad ") + what + " '" + t + "'");
        return static_cast<uint64_t>(v);
    };
    auto type = [&]() {
        const std::string t = next();
        if (t == "b") return SType::Bool;
        if (t == "i") return SType::I64;
        if (t == "u") return SType::U64;
        fail("bad type code '" + t + "'");
    };
    auto e = std::make_unique<SExpr>();
    const std::string k = next();
    if (k == "Lb") {
        e->kind = K::LitBool;
        e->type = SType::Bool;
        e->u = num_u("bool") != 0;
    } else if (k == "Li") {
        const std::string t = next();
        char* end = nullptr;
        const long long v = std::strtoll(t.c_str(), &end, 10);
        if (t.empty() || *end) fail("bad i64 literal '" + t + "'");
        e->kind = K::LitI64;
        e->u = static_cast<uint64_t>(v);
    } else if (k == "Lu") {
        e->kind = K::LitU64;
        e->type = SType::U64;
        e->u = num_u("u64 literal");
    } else if (k == "P" || k == "S" || k == "K") {
        e->kind = k == "P" ? K::TaskParam : k == "S" ? K::Slot : K::KernelScalar;
        e->type = type();
        e->u = num_u("index");
    } else if (k == "A") {
        e->kind = K::AxisVar;
        e->type = type();
        e->u = num_u("axis id");
    } else if (k == "G" || k == "Y") {
        e->kind = k == "G" ? K::TaskTag : K::Symbol;
        e->type = SType::U64;
        e->u = num_u("id");
    } else if (k == "U") {
        e->kind = K::Unary;
        e->op = next();
        if (e->op != "!" && e->op != "-" && e->op != "~") fail("unknown unary operator '" + e->op + "'");
        e->a = parse_scalar(next);
    } else if (k == "B") {
        e->kind = K::Binary;
        e->op = next();
        static const char* ops[] = {"+", "-", "*", "/", "%", "&", "|", "^", "<<", ">>", "<", "<=", ">", ">=", "==", "!=", "&&", "||"};
        bool known = false;
        for (const char* o : ops) known |= e->op == o;
        if (!known) fail("unknown binary operator '" + e->op + "'");
        e->a = parse_scalar(next);
        e->b = parse_scalar(next);
    } else if (k == "T") {
        e->kind = K::Ternary;
        e->a = parse_scalar(next);
        e->b = parse_scalar(next);
        e->c = parse_scalar(next);
    } else if (k == "C") {
        e->kind = K::Cast;
        e->type = type();
        e->a = parse_scalar(next);
    } else {
        fail("bad node '" + k + "'");
    }
    return e;
}

}  // namespace ptowsp
