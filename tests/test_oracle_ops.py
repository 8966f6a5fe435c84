"""Pins the oracle's store cast and the op variants of the arithmetic contract (CPU only).

The reference lowers each of these to one PTO-ISA call whose body is absent
(src/python/pto_codegen.cpp:955-976 TCVT CAST_RINT, :1008-1051 TADDS / TSUBS /
TMULS / TDIVS / TMAXS / TMINS, :1078-1107 TADD..TMIN, TROWEXPAND*, TCOLEXPAND*).
Their fp32 results are fixed by IEEE arithmetic: one correctly rounded
operation per element, so float64 arithmetic rounded once to float32 gives
the exact bits (float64 holds every sum, difference and product of two
floats exactly and rounds a quotient well enough that the second rounding
is innocuous).  Every check is bit-exact and paired with a plausible mistake
(swapped operands, wrong broadcast axis, min for max, truncating cast) that
it rejects.

The store casts are pinned against numpy's float16 conversion (round to
nearest even) and, for bf16, against a distance-based restatement of round
to nearest even on exact halfway values of both parities.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

F32, F16, BF16 = W.F32, W.F16, W.BF16

F64_OPS = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide,
           "max": lambda a, b: np.where(a > b, a, b), "min": lambda a, b: np.where(a < b, a, b)}


def _inputs(shape, yshape, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(np.float32)
    y = rng.standard_normal(shape[:2] + yshape).astype(np.float32)
    y[np.abs(y) < 1e-3] = 0.5  # keep quotients finite
    return x, y


def _expected(op, x, y, mode):
    """float64 op on the broadcast operand, rounded once to float32."""
    x64, y64 = x.astype(np.float64), y.astype(np.float64)
    if mode == "row":
        yb = y64                                  # [.., R, 1] against rows
    elif mode == "row_t":
        yb = np.swapaxes(y64, -1, -2)             # [.., 1, R] -> one value per row
    elif mode == "col":
        yb = y64                                  # [.., 1, C] against columns
    elif mode == "col_t":
        yb = np.swapaxes(y64, -1, -2)             # [.., C, 1] -> one value per column
    else:
        yb = y64
    return F64_OPS[op](x64, yb).astype(np.float32)


def _run_binary(op, mode, R=8, C=32, seed=0, out_dtype=F32):
    x, y = _inputs((2, 3, R, C), W.BIN_SHAPES[mode](R, C), seed)
    out = np.zeros((2, 3, R, C), np.float32 if out_dtype == F32 else (np.float16 if out_dtype == F16 else np.uint16))
    arrs = {"x": x, "y": y, "out": out}
    run_workload(W.rr4(W.binary(arrs, op, out_dtype)))
    return x, y, arrs["out"]


CASES = [(op, "same") for op in F64_OPS] + [(op, m) for op in F64_OPS for m in ("row", "row_t")] + \
        [(op, m) for op in ("sub", "mul", "div") for m in ("col", "col_t")]


@pytest.mark.parametrize("op,mode", CASES)
def test_binary_variant_bit_exact(op, mode):
    x, y, got = _run_binary(op, mode)
    want = _expected(op, x, y, mode)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    # plausible mistakes: swapped operands (for the non-commutative ops) and min / max exchanged
    if op in ("sub", "div"):
        x64 = x.astype(np.float64)
        yb = _expected("add", np.zeros_like(x), y, mode).astype(np.float64)
        swapped = F64_OPS[op](yb, x64).astype(np.float32)
        assert not np.array_equal(got, swapped)
    if op in ("max", "min"):
        other = _expected("min" if op == "max" else "max", x, y, mode)
        assert not np.array_equal(got, other)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "max", "min"])
def test_row_broadcast_on_a_square_tile_is_per_row(op):
    """On a square tile a [1, R] rhs is a row broadcast (the reference checks the row-expand
    shapes first, :1094-1105), never a column broadcast."""
    x, y, got = _run_binary(op, "row_t", R=16, C=16, seed=2)
    np.testing.assert_array_equal(got, _expected(op, x, y, "row_t"))
    as_columns = F64_OPS[op](x.astype(np.float64), y.astype(np.float64)).astype(np.float32)
    assert not np.array_equal(got, as_columns)


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "max", "min"])
@pytest.mark.parametrize("value", [0.75, -2.5])
def test_scalar_right_variant_bit_exact(op, value):
    x = np.random.default_rng(1).standard_normal((2, 2, 8, 64)).astype(np.float32)
    arrs = {"x": x, "out": np.zeros_like(x)}
    run_workload(W.rr4(W.scalar_binary(arrs, op, value)))
    s = np.float64(np.float32(value))
    want = F64_OPS[op](x.astype(np.float64), s).astype(np.float32)
    np.testing.assert_array_equal(arrs["out"].view(np.uint32), want.view(np.uint32))
    if op in ("sub", "div"):
        assert not np.array_equal(arrs["out"], F64_OPS[op](s, x.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("op", ["add", "mul", "div", "max", "min"])
def test_scalar_left_variant_bit_exact(op):
    """op(s, x): TDIVS(dst, s, tile) for Div (s / x, :1031-1036); the other kinds commute."""
    x = np.random.default_rng(4).standard_normal((1, 3, 8, 32)).astype(np.float32)
    x[np.abs(x) < 1e-3] = 0.25
    arrs = {"x": x, "out": np.zeros_like(x)}
    run_workload(W.rr4(W.scalar_binary(arrs, op, 1.5, left=True)))
    want = F64_OPS[op](np.float64(1.5), x.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(arrs["out"].view(np.uint32), want.view(np.uint32))
    if op == "div":
        assert not np.array_equal(arrs["out"], (x.astype(np.float64) / 1.5).astype(np.float32))


def test_scalar_left_sub_is_refused():
    """scalar - tile has no lowering in the reference (:1043-1047)."""
    x = np.zeros((1, 1, 4, 8), np.float32)
    with pytest.raises(RuntimeError, match="scalar - tile"):
        run_workload(W.scalar_binary({"x": x, "out": np.zeros_like(x)}, "sub", 1.0, left=True))


def _probe_tiles(vals, R=16, C=32):
    n = R * C
    reps = -(-len(vals) // n)
    v = np.resize(vals, reps * n).astype(np.float32)
    return v.reshape(1, reps, R, C)


def test_store_cast_f32_to_f16_is_round_to_nearest_even():
    x = _probe_tiles(W.rounding_probe_f32(4000, seed=7))
    arrs = {"x": x, "out": np.zeros(x.shape, np.float16)}
    run_workload(W.rr4(W.store_cast(arrs, F16)))
    want = x.astype(np.float16)  # numpy: round to nearest, ties to even
    np.testing.assert_array_equal(arrs["out"].view(np.uint16), want.view(np.uint16))
    # a truncating cast (toward zero) differs on the halfway and near-halfway probes
    trunc = np.where(np.abs(want.astype(np.float32)) > np.abs(x),
                     np.nextafter(want, np.float16(0)), want).astype(np.float16)
    assert not np.array_equal(arrs["out"].view(np.uint16), trunc.view(np.uint16))
    # the exact halfway probes (every 6th value of the probe's head, both parities of the
    # lower neighbour) all went to the even neighbour
    n_half = len(range(0, 1024, 37))
    got_half = arrs["out"].reshape(-1)[0:6 * n_half:6].view(np.uint16)
    assert np.all((got_half & 1) == 0)
    lower = (x.reshape(-1)[0:6 * n_half:6].view(np.uint32) >> 13) & 1
    assert lower.min() == 0 and lower.max() == 1


def test_store_cast_f32_to_bf16_is_round_to_nearest_even():
    x = _probe_tiles(W.rounding_probe_f32(4000, seed=9, for_bf16=True))
    arrs = {"x": x, "out": np.zeros(x.shape, np.uint16)}
    run_workload(W.rr4(W.store_cast(arrs, BF16)))
    want = W.bf16_rne_by_distance(x.reshape(-1)).reshape(x.shape)
    np.testing.assert_array_equal(arrs["out"], want)
    # exact halfway values of both parities: 1 + 2^-8 rounds down to 1.0 (even) and
    # 1 + 3*2^-8 rounds up to 1 + 2^-6 (even); truncation keeps 1 + 2^-7 for the second,
    # and rounding half away from zero gives 1 + 2^-7 for the first.
    probe = np.zeros((1, 1, 16, 32), np.float32)
    probe[0, 0, 0, :2] = [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8]
    arrs = {"x": probe, "out": np.zeros(probe.shape, np.uint16)}
    run_workload(W.rr4(W.store_cast(arrs, BF16)))
    got = W.bf16_to_f32(arrs["out"][0, 0, 0, :2])
    np.testing.assert_array_equal(got, np.asarray([1.0, 1.0 + 2.0 ** -6], np.float32))
    truncated = (probe[0, 0, 0, :2].view(np.uint32) >> 16).astype(np.uint16)
    assert not np.array_equal(arrs["out"][0, 0, 0, :2], truncated)


@pytest.mark.parametrize("out_dtype", [F16, BF16])
def test_computed_tile_store_cast(out_dtype):
    """A computed f32 tile (x * s) stored through the cast: fp16/bf16(fp32(x*s))."""
    x = np.random.default_rng(11).standard_normal((1, 2, 8, 64)).astype(np.float32)
    out = np.zeros(x.shape, np.float16 if out_dtype == F16 else np.uint16)
    arrs = {"x": x, "out": out}
    run_workload(W.rr4(W.scalar_binary(arrs, "mul", 3.1, out_dtype=out_dtype)))
    prod = (x.astype(np.float64) * np.float64(np.float32(3.1))).astype(np.float32)
    if out_dtype == F16:
        np.testing.assert_array_equal(arrs["out"].view(np.uint16), prod.astype(np.float16).view(np.uint16))
    else:
        np.testing.assert_array_equal(arrs["out"], W.bf16_rne_by_distance(prod.reshape(-1)).reshape(x.shape))


def test_paged_decode_oracle_against_float64():
    """The oracle's paged decode (indirect page-table index, tensor-bound page counts,
    bf16 x f32 matmul, online softmax over pages) against float64 attention over each
    sequence's valid tokens; a page table read as the identity is far outside the bound."""
    lengths = [37, 16, 1, 100, 64, 5]
    arrs = W.paged_decode_arrays(lengths, hkv=2, group=4, d=64, seed=3)
    run_workload(W.rr4(W.paged_decode(arrs)))
    ref = W.paged_decode_ref(arrs)
    rel = np.linalg.norm(arrs["out"].astype(np.float64) - ref) / np.linalg.norm(ref)
    assert rel <= 1e-6, rel
    ident = dict(arrs)
    pt = np.zeros_like(arrs["page_table"])
    off = 0
    for b, n in enumerate(arrs["npages"]):
        pt[b, :n] = np.arange(off, off + n)
        off += n
    ident["page_table"] = pt
    wrong = W.paged_decode_ref(ident)
    assert np.linalg.norm(arrs["out"] - wrong) / np.linalg.norm(wrong) > 1e-2
    # the 1/sqrt(d) scale: attention at scale 1/d is also rejected
    assert np.linalg.norm(arrs["out"] - ref) < 1e-2 * np.linalg.norm(ref)
    arrs2 = W.paged_decode_arrays(lengths, hkv=2, group=4, d=64, seed=3)
    run_workload(W.rr4(W.paged_decode(arrs2, scale=1.0 / 64)))
    assert np.linalg.norm(arrs2["out"] - ref) / np.linalg.norm(ref) > 1e-2
