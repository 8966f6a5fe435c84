"""@ptoisa_kernel: tracing, the oracle's execution of the PTO-ISA ops, and the cycle model (CPU only).

The two cases of the reference's tests/test_ptoisa_kernel_jit.py:22-95 are
pinned against numpy (x*x is one correctly rounded float32 product; the
top-k indices are numpy's argsort of -scores), and so are ties, signed zeros
and NaN in TSORT32 (numpy's stable argsort of -scores: equal keys in source
order, NaN last).  The cycle totals are the wrapper costs of
include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:54-303 summed by hand: rows x
cols per TLOAD / TSTORE / TMOV / elementwise op, 5 per TSORT32 source
element, nothing for the iota and index-store loops, and the makespan over
the round-robin workers.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from pto_wsp import DType, In, Out, Scalar, Tile, ptoisa, ptoisa_kernel

F32, I32 = DType.F32, DType.I32


def test_square_tile_matches_numpy_and_cycles():
    x = np.random.default_rng(0).standard_normal((4, 1, 32, 32), dtype=np.float32)
    y = np.zeros_like(x)
    ref = run_workload(W.rr2(W.ptoisa_square({"x": x, "y": y}), 2048))
    np.testing.assert_array_equal(y, x * x)
    # 4 tasks over 2 workers, TLOAD + TMUL + TSTORE of 32x32 each.
    assert ref.total_cycles == 2 * 3 * 32 * 32


def test_topk8_matches_argsort_and_cycles():
    scores = np.random.default_rng(0).standard_normal((2, 3, 1, 32), dtype=np.float32)
    out = np.zeros((2, 3, 1, 8), np.int32)
    ref = run_workload(W.rr2(W.ptoisa_topk({"scores": scores, "out": out}), 4096))
    want = np.argsort(-scores.reshape(2, 3, 32), axis=-1)[:, :, :8].astype(np.int32)
    np.testing.assert_array_equal(out.reshape(2, 3, 8), want)
    # 6 tasks over 2 workers: TLOAD 1x32 + TSORT32 5*32 each.
    assert ref.total_cycles == 3 * (32 + 5 * 32)


def tie_scores(n_tiles: int, seed: int) -> np.ndarray:
    """[n_tiles, 1, 1, 32] scores with repeated values, +0 / -0, +-inf and NaN."""
    rng = np.random.default_rng(seed)
    s = rng.integers(-3, 4, size=(n_tiles, 1, 1, 32)).astype(np.float32) * np.float32(0.5)
    flat = s.reshape(n_tiles, 32)
    for i in range(n_tiles):
        pos = rng.permutation(32)
        flat[i, pos[0]] = np.float32(-0.0)
        flat[i, pos[1]] = np.float32(0.0)
        if i % 2:
            flat[i, pos[2]] = np.nan
            flat[i, pos[3]] = np.inf
            flat[i, pos[4]] = np.nan
            flat[i, pos[5]] = -np.inf
    return s


def test_tsort32_ties_zero_signs_and_nan_follow_stable_argsort():
    s = tie_scores(6, 1)
    out = np.zeros((6, 1, 1, 32), np.int32)
    run_workload(W.rr2(W.ptoisa_topk({"scores": s, "out": out}, k=32), 4096))
    want = np.argsort(-s.reshape(6, 32), axis=-1, kind="stable").astype(np.int32)
    np.testing.assert_array_equal(out.reshape(6, 32), want)
    # A sort that breaks ties by descending index, or puts NaN first, differs.
    assert not np.array_equal(want, np.argsort(-s.reshape(6, 32)[:, ::-1], axis=-1, kind="stable")[:, ::-1])


def test_topk_store_writes_only_k_columns():
    scores = np.random.default_rng(3).standard_normal((1, 2, 1, 32), dtype=np.float32)
    out = np.full((1, 2, 1, 12), -7, np.int32)
    run_workload(W.rr2(W.ptoisa_topk({"scores": scores, "out": out}, k=5), 64))
    want = np.argsort(-scores.reshape(2, 32), axis=-1)[:, :5]
    np.testing.assert_array_equal(out.reshape(2, 12)[:, :5], want)
    assert (out.reshape(2, 12)[:, 5:] == -7).all()


def test_pto_tracer_topk_matches_ptoisa():
    scores = np.random.default_rng(4).standard_normal((2, 3, 1, 32), dtype=np.float32)
    a, b = np.zeros((2, 3, 1, 8), np.int32), np.zeros((2, 3, 1, 8), np.int32)
    run_workload(W.rr2(W.ptoisa_topk({"scores": scores, "out": a}), 4096))
    ref = run_workload(W.rr2(W.pto_topk({"scores": scores, "out": b}), 4096))
    np.testing.assert_array_equal(a, b)
    # preloaded scores 32 + TSORT32 160 + TSTORE of the [1,8] result.
    assert ref.total_cycles == 3 * (32 + 160 + 8)


def mix_arrays(B=3, R=8, C=32, seed=2):
    rng = np.random.default_rng(seed)
    return {"x": rng.standard_normal((B, R, C), dtype=np.float32),
            "m": rng.standard_normal((B, R, 1), dtype=np.float32),
            "g": rng.standard_normal((B, 1, C), dtype=np.float32),
            "s": np.float32(-1.75), "out": np.zeros((B, R, C), np.float32)}


def mix_expected(a):
    x, m, g, s = a["x"], a["m"], a["g"], np.float32(a["s"])
    y = ((x - m) * g) / s                      # float32 numpy: one rounding per op
    return np.maximum(y, np.maximum(x, np.float32(-0.5))) + (x + np.float32(2))


def test_mix_instructions_and_cycles():
    a = mix_arrays()
    ref = run_workload(W.rr2(W.ptoisa_mix(a, extra_cycles=7), 64))
    want = mix_expected(a)
    np.testing.assert_array_equal(a["out"], want)
    # Swapped TROWEXPANDSUB operands or a missing TADDS give other values.
    y_swapped = ((a["m"] - a["x"]) * a["g"]) / np.float32(a["s"])
    assert not np.array_equal(want, np.maximum(y_swapped, np.maximum(a["x"], np.float32(-0.5))) + (a["x"] + np.float32(2)))
    assert not np.array_equal(want, np.maximum(((a["x"] - a["m"]) * a["g"]) / np.float32(a["s"]),
                                               np.maximum(a["x"], np.float32(-0.5))) + a["x"])
    R, C = 8, 32
    per_task = 10 * R * C + R + C + 7
    assert ref.total_cycles == 2 * per_task  # 3 tasks over 2 workers


def test_unary_exp_rsqrt_close_to_float64():
    x = np.random.default_rng(5).uniform(-4, 4, (2, 4, 32)).astype(np.float32)
    out = np.zeros_like(x)
    run_workload(W.rr2(W.ptoisa_unary({"x": x, "out": out}), 64))
    want = 1.0 / np.sqrt(np.exp(x.astype(np.float64)))
    np.testing.assert_allclose(out, want, rtol=3e-7, atol=0)


# ------------------------------------------------------------------ tracer
def test_tracer_refusals_match_reference_messages():
    with pytest.raises(RuntimeError, match="inside @ptoisa_kernel"):
        ptoisa.tload(None)

    with pytest.raises(ValueError, match="shape/dtype mismatch"):
        @ptoisa_kernel
        def bad_shape(a: In[Tile[4, 8, F32]], b: In[Tile[8, 8, F32]], o: Out[Tile[4, 8, F32]]):
            ptoisa.tstore(o, ptoisa.TADD(ptoisa.tload(a), ptoisa.tload(b)))

    with pytest.raises(TypeError, match="expects a tile value"):
        @ptoisa_kernel
        def param_operand(a: In[Tile[4, 8, F32]], o: Out[Tile[4, 8, F32]]):
            ptoisa.tstore(o, ptoisa.TMUL(a, a))

    with pytest.raises(ValueError, match=r"TSORT32 v9: requires src tile shape \[1,32\]"):
        @ptoisa_kernel
        def bad_sort(a: In[Tile[1, 16, F32]], o: Out[Tile[1, 8, I32]]):
            ptoisa.store_topk_indices_i32(o, ptoisa.TSORT32(ptoisa.tload(a), ptoisa.iota_u32(16)), 8)

    with pytest.raises(ValueError, match="requires idx tile shape"):
        @ptoisa_kernel
        def bad_idx(a: In[Tile[1, 32, F32]], o: Out[Tile[1, 8, I32]]):
            ptoisa.store_topk_indices_i32(o, ptoisa.TSORT32(ptoisa.tload(a), ptoisa.iota_u32(16)), 8)

    with pytest.raises(TypeError, match="only supports Tile"):
        @ptoisa_kernel
        def bad_param(a, o: Out[Tile[1, 8, I32]]):
            pass

    with pytest.raises(ValueError, match="cpp_includes"):
        @ptoisa_kernel(cpp_includes=["<cmath>"])
        def with_includes(a: In[Tile[1, 32, F32]], o: Out[Tile[1, 32, F32]]):
            ptoisa.tstore(o, ptoisa.tload(a))

    with pytest.raises(ValueError, match="is not a scalar parameter"):
        @ptoisa_kernel
        def string_cycles(a: In[Tile[1, 32, F32]], o: Out[Tile[1, 32, F32]]):
            ptoisa.cpu_sim_add_cycles("n * 3")
            ptoisa.tstore(o, ptoisa.tload(a))

    with pytest.raises(TypeError, match="an int, a Scalar parameter or a C expression"):
        @ptoisa_kernel
        def float_cycles(a: In[Tile[1, 32, F32]], o: Out[Tile[1, 32, F32]]):
            ptoisa.cpu_sim_add_cycles(1.5)
            ptoisa.tstore(o, ptoisa.tload(a))

    with pytest.raises(ValueError, match="broadcast operand"):
        @ptoisa_kernel
        def bad_expand(a: In[Tile[4, 8, F32]], m: In[Tile[1, 8, F32]], o: Out[Tile[4, 8, F32]]):
            ptoisa.tstore(o, ptoisa.TROWEXPANDSUB(ptoisa.tload(a), ptoisa.tload(m)))

    with pytest.raises(AttributeError):
        ptoisa.TNOSUCH  # noqa: B018


def test_scalar_param_and_module_text():
    @ptoisa_kernel
    def k(a: In[Tile[1, 32, F32]], s: Scalar[F32], o: Out[Tile[1, 8, I32]]):
        pairs = ptoisa.TSORT32(ptoisa.TMULS(ptoisa.tload(a), s), ptoisa.iota_u32(32))
        ptoisa.store_topk_indices_i32(o, pairs, 8)
        ptoisa.cpu_sim_add_cycles(11)

    ir = k.trace()
    kinds = [op.kind.name for op in ir.ops]
    assert kinds == ["Load", "Mul", "IotaU32", "TSort32", "StoreTopkIndices", "CpuSimAddCycles"]
    assert ir.ops[4].attrs == {"k": 8} and ir.ops[5].attrs == {"cycles": 11}


def test_native_compile_selects_families():
    """The HIP backend accepts every case and emits the expected program family (no GPU needed)."""
    from pto_wsp._hip import NativeProgram
    from pto_wsp.ir_bridge import workload_to_codegen_ir

    x = np.zeros((4, 1, 32, 32), np.float32)
    sc = np.zeros((2, 3, 1, 32), np.float32)
    oi = np.zeros((2, 3, 1, 8), np.int32)
    cases = {
        "row program": W.ptoisa_square({"x": x, "y": x.copy()}),
        "tsort32_rank": W.ptoisa_topk({"scores": sc, "out": oi}),
    }
    for marker, w in cases.items():
        prog = NativeProgram(workload_to_codegen_ir(w, "ptoisa_family").module)
        assert marker in prog.precompile(0)
    mix = NativeProgram(workload_to_codegen_ir(W.ptoisa_mix(mix_arrays()), "ptoisa_mix").module)
    assert "row program" in mix.precompile(0)
    topk = NativeProgram(workload_to_codegen_ir(W.pto_topk({"scores": sc, "out": oi}), "pto_topk").module)
    assert "tsort32_rank" in topk.precompile(0)


# ------------------------------------------------------------------ the reference's PTO-ISA example
@pytest.mark.parametrize("impl,cycles", [("pto", 800), ("ptoisa", 1319680)])
def test_lightning_indexer_example(impl, cycles):
    """examples/deepseek_lightning_indexer: the top-8 indices equal the example's golden
    (descending score, lower index first) and the cycles equal the values the example records
    for its "pto" and "ptoisa" kernels (deepseek_lightning_indexer_example.py:41-45).  The
    ptoisa kernel charges each tier ((pad_to > 32) ? pad_to / 32 * 128 : 0) cycles through
    cpu_sim_add_cycles of a C expression; by hand, worker 0 (b = 0, tiers 65536, 131072,
    131072, 2048) runs 4 x (32 + 160) + 262144 + 2 x 524288 + 8192 = 1319680."""
    scores, eff = W.lightning_inputs()
    out = np.zeros((2, 4, 1, 8), np.int32)
    r = run_workload(W.lightning_indexer(scores, eff, out, impl))
    np.testing.assert_array_equal(out.reshape(2, 4, 8), W.stable_topk_desc(scores, 8))
    assert r.total_cycles == cycles
    assert 4 * (32 + 160) + 262144 + 2 * 524288 + 8192 == 1319680


def test_cycle_expression_parser():
    from pto_wsp.ptoisa_jit import parse_c_expr
    from pto_wsp.scalar_expr import Expr

    env = {"n": Expr("kernel_scalar", "i64", 0), "m": Expr("kernel_scalar", "u64", 1)}
    e = parse_c_expr("((n > 32) ? ((uint64_t)(n / 32) * 128ull) : 0ull)", env)
    assert e.to_text() == "T B > K i 0 Li 32 B * C u B / K i 0 Li 32 Lu 128 Lu 0"
    # precedence: * before +, << below +, && below ==
    assert parse_c_expr("1 + 2 * n", env).to_text() == "B + Li 1 B * Li 2 K i 0"
    assert parse_c_expr("m << 1 + 1", env).to_text() == "B << K u 1 B + Li 1 Li 1"
    assert parse_c_expr("n == 1 && m != 2u", env).to_text() == "B && B == K i 0 Li 1 B != K u 1 Lu 2"
    assert parse_c_expr("-(int64_t)m", env).to_text() == "U - C i K u 1"
    for bad in ["n +", "x + 1", "(uint32_t)n", "n ? 1", "1.5 * n"]:
        with pytest.raises(ValueError):
            parse_c_expr(bad, env)
