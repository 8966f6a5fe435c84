"""Scalar expressions (cond predicates, dispatch keys): the DSL and both evaluators.

The reference compiles every ScalarExpr into a C++ expression inside its
artifact (src/python/pto_codegen.cpp:220-300), so C++ itself is the ground
truth here: random expressions are rendered the way that emitter renders them,
compiled with g++ (-fwrapv: signed + - * wrap, the behaviour both evaluators
define), and their values and C types compared with

* the oracle's evaluator (oracle/cpu_sim.c, pto_cpusim_eval_scalar), and
* the product's evaluator (pto-wsp_amd/csrc/host/scalar.cpp, through
  tests/scalar_eval_driver.cpp built with g++).

Division and remainder use non-zero divisors other than -1 and shift counts
stay in [0, 64), the cases where the C++ expression is defined.
"""

import os
import random
import subprocess

import pytest

from oracle.runner import eval_scalar
from pto_wsp.scalar_expr import (Expr, TaskExpr, as_expr, axis, fnv1a_64, slot_bool, slot_i64, slot_u64, symbol_u64,
                                 task_param, trace_task_fn)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
M64 = (1 << 64) - 1
SYMBOL_IDS = [fnv1a_64(n) for n in ("cut", "mask", "special", "n")]


def sym_value(sid: int) -> int:
    return (sid * 0x9E3779B97F4A7C15 + 0x1234567) & M64


def slot_value(i: int) -> int:
    return (i * 0x0123456789ABCDEF + 7) & M64 if i < 256 else 0


# ---------------------------------------------------------------- the DSL
def test_dsl_types_follow_the_reference():
    b = axis("b")
    assert b.kind == "axis_var" and b.type == "i64" and b.a == fnv1a_64("b")
    assert (b < 2).type == "bool"
    assert (symbol_u64("m") & symbol_u64("k")).type == "u64"
    assert ((b < 2) & (b > 0)).a == "&&"
    assert ((b < 2) | (b > 0)).a == "||"
    assert (~(b < 2)).a == "!" and (~symbol_u64("m")).a == "~"
    assert (b << 3).type == "u64" and (b << 3).b.kind == "cast"
    assert (b + 1).type == "i64" and (symbol_u64("m") + 1).type == "u64"
    assert (b == 1).where(0, 1).type == "i64"
    assert b.cast_u64().type == "u64" and slot_bool(3).type == "bool" and slot_i64(2).type == "i64"
    t = TaskExpr()
    assert t.params[0].kind == "task_param" and t.tags["mask"].a == fnv1a_64("mask")
    assert trace_task_fn(lambda t: t.get("b") % 2).kind == "binary"
    assert task_param(1).type == "i64" and slot_u64(0).type == "u64"
    assert as_expr(True).kind == "lit_bool" and as_expr(5).kind == "lit_i64"


@pytest.mark.parametrize("bad", [
    lambda: bool(axis("b") < 1),
    lambda: axis("b") & axis("c"),
    lambda: axis("b") ^ 1,
    lambda: ~axis("b"),
    lambda: -(axis("b") < 1),
    lambda: axis("b").where(1, 2),
    lambda: (axis("b") < 1).where(1, True),
    lambda: as_expr(1.5),
])
def test_dsl_refuses_what_the_reference_refuses(bad):
    with pytest.raises(TypeError):
        bad()


def test_token_form():
    e = (axis("b") < symbol_u64("cut").cast_i64()).where(slot_u64(3), symbol_u64("x") >> 2)
    text = e.to_text()
    assert text.startswith("T B < A i ")
    assert f"Y {fnv1a_64('cut')}" in text and "S u 3" in text and "B >> C u Y" in text
    assert as_expr(-5).to_text() == "Li -5" and as_expr(False).to_text() == "Lb 0"


# ---------------------------------------------------------------- evaluators vs C++
_I64 = [0, 1, -1, 2, 7, -9, 1000, -123456789, (1 << 62) + 3, -(1 << 62), (1 << 63) - 1, -(1 << 63) + 1]
_U64 = [0, 1, 2, 5, 255, 1 << 32, (1 << 63), M64, M64 - 6, 0x9E3779B97F4A7C15]
_CT = {"b": "bool", "i": "int64_t", "u": "uint64_t"}


def _promo(t):
    return "i" if t == "b" else t


def _usual(a, b):
    return "u" if "u" in (a, b) else "i"


def _leaf(rng):
    k = rng.randrange(6)
    if k == 0:
        v = rng.random() < 0.5
        return f"Lb {int(v)}", "true" if v else "false", "b"
    if k == 1:
        v = rng.choice(_I64 + [rng.randrange(-50, 50)])
        return f"Li {v}", f"(int64_t){v}", "i"
    if k == 2:
        v = rng.choice(_U64 + [rng.randrange(0, 100)])
        return f"Lu {v}", f"(uint64_t)0x{v:x}ULL", "u"
    if k == 3:
        sid = rng.choice(SYMBOL_IDS)
        return f"Y {sid}", f"sym(0x{sid:x}ULL)", "u"
    i, t = rng.randrange(0, 300), rng.choice("biu")
    base = f"slot({i}u)"
    cpp = {"i": f"(int64_t){base}", "u": f"(uint64_t){base}", "b": f"((bool)({base} != 0ULL))"}[t]
    return f"S {t} {i}", cpp, t


def _gen(rng, depth):
    if depth == 0 or rng.random() < 0.2:
        return _leaf(rng)
    k = rng.randrange(8)
    a = _gen(rng, depth - 1)
    if k == 0:
        op = rng.choice("!-~")
        t = "b" if op == "!" else _promo(a[2])
        return f"U {op} {a[0]}", f"({op}{a[1]})", t
    if k in (1, 2):
        b = _gen(rng, depth - 1)
        op = rng.choice(["+", "-", "*", "&", "|", "^"])
        return f"B {op} {a[0]} {b[0]}", f"({a[1]} {op} {b[1]})", _usual(_promo(a[2]), _promo(b[2]))
    if k == 3:
        b = _gen(rng, depth - 1)
        op = rng.choice(["<", "<=", ">", ">=", "==", "!=", "&&", "||"])
        return f"B {op} {a[0]} {b[0]}", f"({a[1]} {op} {b[1]})", "b"
    if k == 4:
        op = rng.choice("/%")
        if rng.random() < 0.5:
            d = rng.choice([2, 3, 7, -2, -5, 1 << 33, -(1 << 40) + 1])
            return (f"B {op} {a[0]} Li {d}", f"({a[1]} {op} (int64_t){d})", _usual(_promo(a[2]), "i"))
        d = rng.choice([1, 3, 10, 1 << 35, M64])
        return f"B {op} {a[0]} Lu {d}", f"({a[1]} {op} (uint64_t)0x{d:x}ULL)", "u"
    if k == 5:
        op, n = rng.choice(["<<", ">>"]), rng.randrange(64)
        return (f"B {op} C u {a[0]} C u Lu {n}", f"((uint64_t)({a[1]}) {op} (uint64_t)((uint64_t)0x{n:x}ULL))", "u")
    if k == 6:
        c, f = _gen(rng, depth - 1), _gen(rng, depth - 1)
        t = "b" if a[2] == "b" and f[2] == "b" else _usual(_promo(a[2]), _promo(f[2]))
        return f"T {c[0]} {a[0]} {f[0]}", f"({c[1]} ? {a[1]} : {f[1]})", t
    ty = rng.choice("biu")
    return f"C {ty} {a[0]}", f"({_CT[ty]})({a[1]})", ty


def _cpp_truth(exprs, tmp):
    lines = [
        "#include <cstdint>", "#include <cstdio>",
        "static uint64_t sym(uint64_t id) { return id * 0x9E3779B97F4A7C15ull + 0x1234567ull; }",
        "static uint64_t slot(uint32_t i) { return i < 256 ? i * 0x0123456789ABCDEFull + 7 : 0; }",
        "static char tc(bool) { return 'b'; }", "static char tc(int) { return 'i'; }",
        "static char tc(long) { return 'i'; }", "static char tc(long long) { return 'i'; }",
        "static char tc(unsigned long) { return 'u'; }", "static char tc(unsigned long long) { return 'u'; }",
        "template <class T> static void out(T x) { std::printf(\"%c %llu\\n\", tc(x), (unsigned long long)(uint64_t)x); }",
        "int main() {",
    ]
    lines += [f"  out({cpp});" for _, cpp, _ in exprs]
    lines.append("  return 0;\n}")
    src, exe = os.path.join(tmp, "truth.cpp"), os.path.join(tmp, "truth")
    open(src, "w").write("\n".join(lines))
    subprocess.run(["g++", "-std=c++17", "-O1", "-fwrapv", "-w", src, "-o", exe], check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split("\n")
    return [(ln.split()[0], int(ln.split()[1])) for ln in out if ln]


@pytest.fixture(scope="module")
def random_exprs(tmp_path_factory):
    rng = random.Random(2024)
    exprs = [_gen(rng, rng.randrange(1, 6)) for _ in range(600)]
    truth = _cpp_truth(exprs, str(tmp_path_factory.mktemp("cpp")))
    assert len(truth) == len(exprs)
    return exprs, truth


def test_generator_types_match_cpp(random_exprs):
    exprs, truth = random_exprs
    for (_, cpp, t), (ct, _) in zip(exprs, truth):
        assert t == ct, cpp


def test_oracle_evaluator_matches_cpp(random_exprs):
    exprs, truth = random_exprs
    symbols = {sid: sym_value(sid) for sid in SYMBOL_IDS}
    slots = [slot_value(i) for i in range(256)]
    for (text, cpp, _), want in zip(exprs, truth):
        assert eval_scalar(text, symbols, slots) == want, cpp


def test_product_evaluator_matches_cpp(random_exprs, tmp_path):
    exprs, truth = random_exprs
    exe = str(tmp_path / "driver")
    subprocess.run(["g++", "-std=c++17", "-O1", os.path.join(ROOT, "tests", "scalar_eval_driver.cpp"),
                    os.path.join(ROOT, "pto-wsp_amd", "csrc", "host", "scalar.cpp"), "-o", exe], check=True)
    res = subprocess.run([exe], input="\n".join(t for t, _, _ in exprs) + "\n", capture_output=True, text=True, check=True)
    got = [ln.split() for ln in res.stdout.splitlines()]
    assert len(got) == len(exprs)
    for (_, cpp, _), g, want in zip(exprs, got, truth):
        assert (g[0], int(g[1])) == want, cpp


@pytest.mark.parametrize("text,msg", [
    ("B / Li 5 Li 0", "division by zero"),
    ("B % Lu 5 Lu 0", "division by zero"),
    (f"B / Li {-(1 << 63) + 1} Li 1", None),
    ("B << Lu 1 Lu 64", "shift count"),
])
def test_undefined_cases_are_refused(text, msg):
    if msg is None:
        assert eval_scalar(text)[1] == (-(1 << 63) + 1) & M64
        return
    with pytest.raises(RuntimeError, match=msg):
        eval_scalar(text)
