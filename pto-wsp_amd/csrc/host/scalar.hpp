// Scalar expressions (ScalarExpr): run-time predicates of cond nodes and
// dispatch keys, evaluated on the host with the semantics of the C++
// expression the reference emits for them (src/python/pto_codegen.cpp:220-300):
// bool / int64_t / uint64_t operands under the usual arithmetic conversions
// (bool promotes to a signed integer; a u64 operand makes the operation
// unsigned), comparisons and `!`, `&&`, `||` giving bool, `&&` / `||` / `?:`
// evaluating only the operand they need.
//
// Where the emitted C++ has undefined behaviour this evaluator defines it:
// signed + - * wrap (two's complement); division or remainder by zero, the
// signed INT64_MIN / -1 overflow, and shift counts outside [0, 64) raise.
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

namespace ptowsp {

enum class SType { Bool, I64, U64 };

struct SExpr {
    // KernelScalar: the task's value of the kernel's scalar parameter with
    // that ordinal (cycle expressions of PTO-ISA kernels).
    enum class Kind { LitBool, LitI64, LitU64, TaskParam, TaskTag, AxisVar, Symbol, Slot, Unary, Binary, Ternary, Cast, KernelScalar };
    Kind kind = Kind::LitI64;
    SType type = SType::I64;   // declared type (reads of params/axes/slots, casts)
    uint64_t u = 0;            // literal bits, id, slot or parameter index
    std::string op;            // unary / binary operator
    std::unique_ptr<SExpr> a, b, c;
};

struct SValue {
    SType t = SType::I64;
    uint64_t v = 0;  // bool: 0 / 1; i64: two's complement bits
};

// Values an expression reads.  `axis` returns false for a variable that is
// not in scope; `task_param` may be empty where no task is current.
struct SEnv {
    std::function<bool(uint64_t id, int64_t& value)> axis;
    std::function<uint64_t(uint64_t id)> symbol;
    std::function<uint64_t(uint32_t slot)> slot;
    std::function<uint64_t(uint32_t index)> task_param;
    std::function<uint64_t(uint32_t ordinal)> kernel_scalar;
};

SValue eval_scalar(const SExpr& e, const SEnv& env);
// Truth value (non-zero) of an expression, as `if (e)`.
bool eval_truth(const SExpr& e, const SEnv& env);
// The expression converted to uint64_t, as `(uint64_t)(e)`.
uint64_t eval_u64(const SExpr& e, const SEnv& env);

// What an expression reads.
struct SRefs {
    std::vector<uint64_t> axes;
    bool slots = false, task_params = false, symbols = false, kernel_scalars = false;
};
void scalar_refs(const SExpr& e, SRefs& out);

// Parses the prefix token form written by pto_wsp/scalar_expr.py (Expr.to_text):
// the caller supplies the next token.
std::unique_ptr<SExpr> parse_scalar(const std::function<std::string()>& next_token);

}  // namespace ptowsp
