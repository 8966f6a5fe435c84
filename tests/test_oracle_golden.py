"""Pins the CPU oracle (oracle/cpu_sim.c) before it is trusted as the parity checker.

The reference's cpu_sim artifact cannot be built here (its tile library, the
pto-isa submodule, is absent), so the oracle is a restatement.  Each check below
ties it to something it cannot simply echo:

* the total_cycles and tolerances the reference's own examples assert
  (tests/golden/reference_examples.json, with file:line sources);
* the exact known answers of the reference's tests (2x2 matmul, copy, x*s,
  dispatch / window and DenseDyn cycle rules);
* closed forms in float64 numpy, each paired with a plausible mistake (wrong
  reduction axis or divisor, transposed operand, missing term, wrong scale)
  that the same tolerance rejects, so the check has teeth.

CPU only: nothing here touches a GPU.
"""

import json
import math
import os

import numpy as np
import pytest

import workloads as W
from oracle.runner import f32_symbol, run_workload
from pto_wsp import Ragged
from pto_wsp.ir_bridge import fnv1a_64

GOLDEN = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_examples.json")))
CYC = GOLDEN["example_cycles"]


def _close(got, ref, rtol, atol):
    return np.allclose(got, ref, rtol=rtol, atol=atol)


def _rel_fro(got, ref):
    return float(np.linalg.norm((np.asarray(got, np.float64) - ref).ravel()) / np.linalg.norm(ref.ravel()))


def test_e2e_rmsnorm_example():
    g = CYC["e2e_rmsnorm"]
    x = np.random.default_rng(0).standard_normal((1, 32, 16), dtype=np.float32)
    arrs = {"x": x.reshape(1, 2, 16, 16).copy(), "y": np.zeros((1, 2, 16, 16), np.float32)}
    r = run_workload(W.rr4(W.rmsnorm(arrs)))
    assert r.total_cycles == g["total_cycles"]
    x64 = arrs["x"].astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).mean(axis=-1, keepdims=True))
    assert _close(arrs["y"], ref, g["rtol"], g["atol"])
    wrong_axis = x64 / np.sqrt((x64 * x64).mean(axis=-2, keepdims=True))
    assert not _close(arrs["y"], wrong_axis, g["rtol"], g["atol"])


def test_quickstart_rmsnorm_divides_by_columns():
    """Config 1 (Tile[16,128]): rowmean divides the row sum by the 128 columns."""
    x = np.random.default_rng(3).standard_normal((1, 2, 16, 128), dtype=np.float32)
    arrs = {"x": x.copy(), "y": np.zeros_like(x)}
    r = run_workload(W.rr4(W.rmsnorm(arrs)))
    assert r.total_cycles == 8240 and r.task_count == 2
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).sum(-1, keepdims=True) / 128)
    np.testing.assert_allclose(arrs["y"], ref, rtol=1e-5, atol=0)
    by_rows = x64 / np.sqrt((x64 * x64).sum(-1, keepdims=True) / 16)
    assert not _close(arrs["y"], by_rows, 1e-5, 0)


def _softmax3_view_semantics(lg):
    """float64 restatement of examples/softmax's three phases with its views as written.

    L[b][s][v] indexes dims (b, s, row-block) of logits.reshape(B, S/8, 8, V/64, 64),
    so each [8, 64] tile starts at row-block v and spans 8 rows of 64 with row
    stride 64: tiles of neighbouring v overlap, and the rescale phase divides the
    shared rows again.  Program order decides the result.
    """
    B, S, V = lg.shape
    tr, tc = 8, 64
    st, vt = S // tr, V // tc
    flat = lg.astype(np.float64).ravel()
    probs = np.zeros(B * S * V)
    rmax = np.full((B, st, tr), -np.inf)
    rsum = np.zeros((B, st, tr))

    def idx(b, s, v):
        return ((b * st + s) * tr + v) * vt * tc + np.arange(tr)[:, None] * tc + np.arange(tc)[None, :]

    for b in range(B):
        for s in range(st):
            for v in range(vt):
                rmax[b, s] = np.maximum(rmax[b, s], flat[idx(b, s, v)].max(1))
    for b in range(B):
        for s in range(st):
            for v in range(vt):
                e = np.exp(flat[idx(b, s, v)] - rmax[b, s][:, None])
                rsum[b, s] += e.sum(1)
                probs[idx(b, s, v)] = e
    for b in range(B):
        for s in range(st):
            for v in range(vt):
                probs[idx(b, s, v)] = probs[idx(b, s, v)] / rsum[b, s][:, None]
    return probs.reshape(lg.shape), rmax[..., None], rsum[..., None]


def test_softmax_three_phase_example():
    g = CYC["softmax_three_phase"]
    lg = (0.1 * np.random.default_rng(0).standard_normal((1, 32, 256), dtype=np.float32)).astype(np.float32)
    arrs = W.softmax3_arrays(lg)
    r = run_workload(W.rr4(W.softmax3(arrs)))
    assert r.total_cycles == g["total_cycles"]
    probs, rmax, rsum = _softmax3_view_semantics(lg)
    np.testing.assert_allclose(arrs["probs"], probs, rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(arrs["rmax"], rmax, rtol=0, atol=0)
    np.testing.assert_allclose(arrs["rsum"], rsum, rtol=1e-5, atol=0)
    # the example's own check (examples/softmax/softmax_example.py:30-31) against a true row softmax
    l64 = lg.astype(np.float64)
    e = np.exp(l64 - l64.max(-1, keepdims=True))
    true_softmax = e / e.sum(-1, keepdims=True)
    assert _close(arrs["probs"], true_softmax, g["rtol"], g["atol"])
    # ... which is loose: the overlapping views are far from a row softmax at rtol 1e-5
    assert not _close(arrs["probs"], true_softmax, 1e-5, 1e-9)


def test_row_softmax_closed_form():
    x = (3.0 * np.random.default_rng(4).standard_normal((2, 3, 32, 512), dtype=np.float32)).astype(np.float32)
    arrs = {"x": x.copy(), "y": np.zeros_like(x)}
    run_workload(W.rr4(W.softmax(arrs)))
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(-1, keepdims=True))
    np.testing.assert_allclose(arrs["y"], e / e.sum(-1, keepdims=True), rtol=1e-5, atol=1e-12)


def test_bgemm_f16_example():
    g = CYC["bgemm_f16"]
    rng = np.random.default_rng(0)
    a = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    b = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    arrs = {"a": a, "b": b, "c": np.zeros((1, 64, 64), np.float32)}
    r = run_workload(W.rr4(W.bgemm(arrs)))
    assert r.total_cycles == g["total_cycles"]
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert _rel_fro(arrs["c"], ref) <= 1e-6
    assert _rel_fro(arrs["c"], a.astype(np.float64) @ b.astype(np.float64).transpose(0, 2, 1)) > 1e-2


def test_bf16_matmul_is_fp32_math_on_exact_bf16_inputs():
    """The oracle's bf16 extension: RNE-rounded bf16 inputs, exact upcast, fp32 accumulate."""
    rng = np.random.default_rng(5)
    a = W.bf16_round(rng.uniform(-1, 1, (2, 128, 256)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (2, 256, 128)).astype(np.float32))
    c0 = rng.standard_normal((2, 128, 128)).astype(np.float32)
    arrs = {"a": a, "b": b, "c": c0.copy()}
    run_workload(W.bgemm(arrs, 64, 64, 64, W.BF16))
    exact = c0.astype(np.float64) + W.bf16_to_f32(a).astype(np.float64) @ W.bf16_to_f32(b).astype(np.float64)
    assert _rel_fro(arrs["c"], exact) <= 1e-6
    # dropping the InOut term (c = a@b) or the first K step is far outside the bound
    assert _rel_fro(arrs["c"], exact - c0) > 1e-2
    first = W.bf16_to_f32(a)[:, :, :64].astype(np.float64) @ W.bf16_to_f32(b)[:, :64, :].astype(np.float64)
    assert _rel_fro(arrs["c"], exact - first) > 1e-2


def test_flashinfer_decode_example():
    g = CYC["flashinfer_decode"]
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 16), dtype=np.float32)
    k = rng.standard_normal((64, 16), dtype=np.float32)
    v = rng.standard_normal((64, 16), dtype=np.float32)
    arrs = {"q": q.copy(), "k_t": k.T.copy(), "v": v.copy(), "o": np.zeros((1, 16), np.float32)}
    r = run_workload(W.rr4(W.decode_attention(arrs), 1024))
    assert r.total_cycles == g["total_cycles"]

    def attend(scale):
        s = (q.astype(np.float64) @ k.T.astype(np.float64)) * scale
        w = np.exp(s - s.max())
        return (w / w.sum()) @ v.astype(np.float64)

    assert _close(arrs["o"], attend(1 / math.sqrt(16)), g["rtol"], g["atol"])
    assert not _close(arrs["o"], attend(1 / 16), g["rtol"], g["atol"])


def test_attention_example():
    g = CYC["attention"]
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    k = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    v = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    arrs = W.attention_arrays(q, k, v, 8)
    r = run_workload(W.rr4(W.tiled_attention(arrs, 8)))
    assert r.total_cycles == g["total_cycles"]
    ref = np.zeros((1, 2, 16, 8))
    for h in range(2):
        for s in range(2):
            sl = slice(8 * s, 8 * s + 8)
            sc = q[0, h, sl].astype(np.float64) @ k[0, h, sl].astype(np.float64).T / math.sqrt(8)
            w = np.exp(sc - sc.max(-1, keepdims=True))
            ref[0, h, sl] = (w / w.sum(-1, keepdims=True)) @ v[0, h, sl].astype(np.float64)
    np.testing.assert_allclose(arrs["o"], ref, rtol=1e-5, atol=1e-6)


def test_validated_matmul_example_and_exact_2x2():
    g = CYC["validated_matmul"]
    rng = np.random.default_rng(0)
    a = rng.standard_normal((1, 1, 16, 16), dtype=np.float32)
    b = rng.standard_normal((1, 1, 16, 16), dtype=np.float32)
    arrs = {"a": a, "b": b, "c": np.zeros((1, 1, 16, 16), np.float32)}
    r = run_workload(W.rr4(W.matmul_tile(arrs, 16, 16, 16), 1024))
    assert r.total_cycles == g["total_cycles"]
    np.testing.assert_allclose(arrs["c"][0, 0], a[0, 0].astype(np.float64) @ b[0, 0], rtol=g["rtol"], atol=g["atol"])
    k = GOLDEN["matmul_2x2"]
    arrs = {"a": np.array([[k["a"]]], np.float32), "b": np.array([[k["b"]]], np.float32),
            "c": np.zeros((1, 1, 2, 2), np.float32)}
    run_workload(W.matmul_tile(arrs, 2, 2, 2))
    np.testing.assert_array_equal(arrs["c"][0, 0], np.array(k["c"], np.float32))


def test_copy_dispatch_and_window_rules():
    from pto_wsp import DispatchPolicy, TaskWindow, WindowMode

    a = np.arange(64, dtype=np.float32).reshape(4, 4, 4)
    arrs = {"a": a, "b": np.zeros_like(a)}
    serial = run_workload(W.copy_tiles(arrs)).total_cycles
    np.testing.assert_array_equal(arrs["b"], a)
    rr2 = run_workload(W.copy_tiles(arrs).dispatch(DispatchPolicy.round_robin(2))).total_cycles
    win1 = run_workload(W.copy_tiles(arrs).dispatch(DispatchPolicy.round_robin(2))
                        .task_graph(window=TaskWindow(1, "tasks", WindowMode.STALL))).total_cycles
    assert serial == 4 * 2 * 16 and rr2 * 2 == serial and win1 == serial


def test_dense_dyn_binding():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((4, 4, 4), dtype=np.float32)
    b = rng.standard_normal((4, 4, 4), dtype=np.float32)
    c = np.zeros((4, 4, 4), np.float32)
    r2 = run_workload(W.dense_dyn_mm({"a": a, "b": b, "c": c}), axis_sizes={"b": 2})
    np.testing.assert_allclose(c[:2], np.matmul(a[:2], b[:2]), rtol=0, atol=1e-5)
    np.testing.assert_array_equal(c[2:], 0)
    r4 = run_workload(W.dense_dyn_mm({"a": a, "b": b, "c": c}), axis_sizes={"b": 4})
    np.testing.assert_allclose(c, np.matmul(a, b), rtol=0, atol=1e-5)
    assert r4.total_cycles / 4 == r2.total_cycles / 2


def test_scalar_symbol_is_exact():
    x = np.arange(16, dtype=np.float32).reshape(4, 4)
    sid = fnv1a_64("scale_s")
    cycles = []
    for s in (2.0, 3.0):
        y = np.zeros((4, 4), np.float32)
        cycles.append(run_workload(W.scale_symbol({"x": x, "y": y}), symbols_u64={sid: f32_symbol(s)}).total_cycles)
        np.testing.assert_array_equal(y, x * s)
    assert cycles[0] == cycles[1]


def test_ragged_axis_flattens_lengths():
    for lengths, want in (([1, 1], [1, 1, 0]), ([1, 2], [1, 1, 1])):
        y = np.zeros((3, 1, 1), np.int32)
        r = Ragged(outer_size=2, lengths=[1, 1])
        run_workload(W.ragged_mark({"y": y}, r), symbols_u64={fnv1a_64(f"outer_{id(r)}"): 2},
                     symbols_ptr={fnv1a_64(f"lengths_{id(r)}"): np.asarray(lengths, np.int32)})
        np.testing.assert_array_equal(y.reshape(3), want)


def _llama_inputs():
    rng = np.random.default_rng(0)  # examples/llama/llama_example.py:19-28
    x = rng.standard_normal((16, 8), dtype=np.float32)
    w1 = rng.standard_normal((8, 16), dtype=np.float32)
    w2 = rng.standard_normal((16, 8), dtype=np.float32)
    return x, w1, w2


def test_llama_example():
    g = CYC["llama"]
    x, w1, w2 = _llama_inputs()
    out = np.zeros_like(x)
    r = run_workload(W.llama_block(x, w1, w2, out, 8, 1e-6))
    assert r.total_cycles == g["total_cycles"]
    ref = W.llama_block_ref(x, w1, w2, 8, 1e-6)
    assert _close(out, ref, g["rtol"], g["atol"])
    # attention over the whole sequence instead of per 8-row tile is another result
    assert not _close(out, W.llama_block_ref(x, w1, w2, 16, 1e-6), g["rtol"], g["atol"])


def _moe_inputs():
    rng = np.random.default_rng(0)  # examples/deepseek_v3/deepseek_v3_example.py:19-28
    x = rng.standard_normal((16, 8), dtype=np.float32)
    w0 = rng.standard_normal((8, 8), dtype=np.float32)
    w1 = rng.standard_normal((8, 8), dtype=np.float32)
    g = rng.random((16, 1), dtype=np.float32)
    return x, w0, w1, g


def test_deepseek_v3_example():
    gold = CYC["deepseek_v3"]
    x, w0, w1, g = _moe_inputs()
    y = np.zeros_like(x)
    r = run_workload(W.moe_block(x, w0, w1, g, y))
    assert r.total_cycles == gold["total_cycles"]
    x64, g64 = x.astype(np.float64), g.astype(np.float64)
    ref = g64 * (x64 @ w0) + (1.0 - g64) * (x64 @ w1)  # examples/deepseek_v3/golden.py:6-9
    assert _close(y, ref, gold["rtol"], gold["atol"])
    assert not _close(y, (1.0 - g64) * (x64 @ w0) + g64 * (x64 @ w1), gold["rtol"], gold["atol"])


def test_tensor_data_examples():
    rng = np.random.default_rng(0)  # examples/tensor_data/tensor_data_example.py:19-29
    a = rng.standard_normal((2, 2, 2, 32, 32), dtype=np.float32)
    b = rng.standard_normal((2, 2, 2, 32, 32), dtype=np.float32)
    x = rng.standard_normal((2, 4, 32, 32), dtype=np.float32)
    c, y = np.zeros_like(a), np.zeros_like(x)
    assert run_workload(W.add_tiles5(a, b, c)).total_cycles == CYC["tensor_data_add"]["total_cycles"]
    assert run_workload(W.square_tiles4(x, y)).total_cycles == CYC["tensor_data_square"]["total_cycles"]
    np.testing.assert_array_equal(c, a + b)
    np.testing.assert_array_equal(y, x * x)
