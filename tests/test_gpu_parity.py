"""GPU parity: the HIP target against the CPU oracle on identical inputs.

Tolerances: fp32 elementwise/reduction work
rtol 1e-5 (atol 1e-6 as in the reference's rmsnorm/decode examples); the
tile-program family reproduces the oracle's operation order, so its results
are compared bit-exactly where no exp() is involved.  Cycle counts must equal
the oracle's (and the reference examples' recorded values).
"""

import math

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu


def run_hip(w, axis_sizes=None, symbols=None):
    prog = w.compile(target="hip_gfx950")
    if axis_sizes:
        prog.set_axis_sizes(axis_sizes)
    for k, v in (symbols or {}).items():
        prog.set_symbol_f32(k, v)
    prog.execute()
    prog.synchronize()
    return prog


def test_rmsnorm_quickstart_host_arrays(gpu):
    x = np.random.default_rng(0).standard_normal((1, 2, 16, 128), dtype=np.float32)
    ga = {"x": x.copy(), "y": np.zeros_like(x)}
    ca = {"x": x.copy(), "y": np.zeros_like(x)}
    prog = run_hip(W.rr4(W.rmsnorm(ga)))
    ref = run_workload(W.rr4(W.rmsnorm(ca)))
    np.testing.assert_allclose(ga["y"], ca["y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(ga["y"], W.rmsnorm_ref(x), rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == ref.total_cycles == 8240
    assert prog.stats.task_count == 2
    np.testing.assert_array_equal(ga["x"], x)


def test_rmsnorm_device_tensors(gpu):
    import torch

    x = np.random.default_rng(3).standard_normal((4, 64, 16, 128), dtype=np.float32)
    xd = torch.from_numpy(x).to(gpu)
    yd = torch.zeros_like(xd)
    prog = run_hip(W.rr4(W.rmsnorm({"x": xd, "y": yd})))
    ca = {"x": x.copy(), "y": np.zeros_like(x)}
    ref = run_workload(W.rr4(W.rmsnorm(ca)))
    np.testing.assert_allclose(yd.cpu().numpy(), ca["y"], rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == ref.total_cycles
    assert prog.stats.device_time_ms > 0


@pytest.mark.parametrize("shape", [(2, 5, 32, 512), (1, 3, 8, 64), (3, 2, 4, 16), (1, 1, 1, 8)])
def test_softmax_tiles(gpu, shape):
    x = (3.0 * np.random.default_rng(1).standard_normal(shape, dtype=np.float32)).astype(np.float32)
    ga = {"x": x.copy(), "y": np.zeros_like(x)}
    ca = {"x": x.copy(), "y": np.zeros_like(x)}
    prog = run_hip(W.rr4(W.softmax(ga)))
    ref = run_workload(W.rr4(W.softmax(ca)))
    np.testing.assert_allclose(ga["y"], ca["y"], rtol=1e-5, atol=0)
    assert prog.stats.total_cycles == ref.total_cycles


def test_example_e2e_rmsnorm(gpu):
    x = np.random.default_rng(0).standard_normal((1, 32, 16), dtype=np.float32)
    ga = {"x": x.reshape(1, 2, 16, 16).copy(), "y": np.zeros((1, 2, 16, 16), np.float32)}
    ca = {"x": x.reshape(1, 2, 16, 16).copy(), "y": np.zeros((1, 2, 16, 16), np.float32)}
    prog = run_hip(W.rr4(W.rmsnorm(ga)))
    run_workload(W.rr4(W.rmsnorm(ca)))
    np.testing.assert_allclose(ga["y"], ca["y"], rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == 1072


def test_example_softmax_three_phase(gpu):
    lg = (0.1 * np.random.default_rng(0).standard_normal((1, 32, 256), dtype=np.float32)).astype(np.float32)
    ga, ca = W.softmax3_arrays(lg), W.softmax3_arrays(lg)
    prog = run_hip(W.rr4(W.softmax3(ga)))
    run_workload(W.rr4(W.softmax3(ca)))
    for k in ("probs", "rmax", "rsum"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=1e-5, atol=1e-7)
    assert prog.stats.total_cycles == 39848


def test_example_bgemm_f16(gpu):
    """examples/bgemm at its own size (16x16x16 f16 tiles, one 64x64 batch): the 4x4 tasks
    of C merge into one 64x64 MFMA block and the four K steps into one 64-column stage.
    The MFMA sums the same exact f16 products as the oracle in another order."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    b = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    ga = {"a": a.copy(), "b": b.copy(), "c": np.zeros((1, 64, 64), np.float32)}
    ca = {"a": a.copy(), "b": b.copy(), "c": np.zeros((1, 64, 64), np.float32)}
    prog = run_hip(W.rr4(W.bgemm(ga)))
    run_workload(W.rr4(W.bgemm(ca)))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    assert _rel_fro(ga["c"], a[0].astype(np.float64) @ b[0].astype(np.float64)) <= 1e-5
    assert prog.stats.total_cycles == 275968


@pytest.mark.parametrize("shape,tile,dt", [
    ((2, 512, 512, 512), 16, "f16"),    # the bgemm example's tiles at scale: 16x16 tasks, 4 K steps per stage
    ((1, 256, 384, 256), 32, "bf16"),   # 32-wide tasks: 8 x 4 per 256 x 128 block (12 along N)
    ((2, 512, 256, 256), 16, "f32"),    # f32 16x16 tiles: stages of two K steps
    ((1, 96, 160, 64), 16, "f16"),      # extents that do not merge to 64: the tile program
])
def test_bgemm_small_tiles_merged(gpu, shape, tile, dt):
    """Task tiles below the MFMA block (the reference's bgemm pattern) merged into
    64..256 blocks and K-merged stages, against the oracle and float64."""
    nb, m, n, k = shape
    rng = np.random.default_rng(m + n + k)
    a32 = rng.uniform(-1, 1, (nb, m, k)).astype(np.float32)
    b32 = rng.uniform(-1, 1, (nb, k, n)).astype(np.float32)
    if dt == "f16":
        a, b, wdt, up = a32.astype(np.float16), b32.astype(np.float16), W.F16, lambda x: x.astype(np.float64)
    elif dt == "bf16":
        a, b, wdt, up = W.bf16_round(a32), W.bf16_round(b32), W.BF16, lambda x: W.bf16_to_f32(x).astype(np.float64)
    else:
        a, b, wdt, up = a32, b32, W.F32, lambda x: x.astype(np.float64)
    c0 = rng.standard_normal((nb, m, n)).astype(np.float32)
    ga = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.rr4(W.bgemm(ga, tile, tile, tile, wdt)))
    ref = run_workload(W.rr4(W.bgemm(ca, tile, tile, tile, wdt)))
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    assert _rel_fro(ga["c"], c0.astype(np.float64) + up(a) @ up(b)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_example_decode_attention(gpu):
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 16), dtype=np.float32)
    k = rng.standard_normal((64, 16), dtype=np.float32)
    v = rng.standard_normal((64, 16), dtype=np.float32)

    def arrs():
        return {"q": q.copy(), "k_t": k.T.copy(), "v": v.copy(), "o": np.zeros((1, 16), np.float32)}

    ga, ca = arrs(), arrs()
    prog = run_hip(W.rr4(W.decode_attention(ga), 1024))
    run_workload(W.rr4(W.decode_attention(ca), 1024))
    np.testing.assert_allclose(ga["o"], ca["o"], rtol=1e-5, atol=1e-6)
    s = (q @ k.T) / math.sqrt(16)
    w = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    np.testing.assert_allclose(ga["o"], w @ v, rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == 4514


def test_example_tiled_attention(gpu):
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    k = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    v = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    ga, ca = W.attention_arrays(q, k, v, 8), W.attention_arrays(q, k, v, 8)
    prog = run_hip(W.rr4(W.tiled_attention(ga, 8)))
    ref = run_workload(W.rr4(W.tiled_attention(ca, 8)))
    np.testing.assert_allclose(ga["o"], ca["o"], rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == ref.total_cycles == 1680


def _has_tile_mma(prog):
    src = prog._native.precompile(0)
    return "tile_mma<" in src or "tile_mma16<" in src


def test_tiled_attention_mfma_tiles(gpu):
    """examples/attention with 64-token tiles and head dim 64: both matmuls of the fused
    tile (q @ k_t and softmax(s) @ v) run on the matrix cores inside the tile program."""
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 2, 128, 64), dtype=np.float32) for _ in range(3))
    ga, ca = W.attention_arrays(q, k, v, 64), W.attention_arrays(q, k, v, 64)
    prog = run_hip(W.rr4(W.tiled_attention(ga, 64)))
    ref = run_workload(W.rr4(W.tiled_attention(ca, 64)))
    assert prog._native.kernel_family("attention_tile") == "tile_program" and _has_tile_mma(prog)
    assert _rel_fro(ga["o"], ca["o"]) <= 1e-5
    q64, k64, v64 = (x.astype(np.float64).reshape(1, 2, 2, 64, 64) for x in (q, k, v))
    s = q64 @ k64.transpose(0, 1, 2, 4, 3) / 8.0
    w = np.exp(s - s.max(-1, keepdims=True))
    exact = ((w / w.sum(-1, keepdims=True)) @ v64).reshape(1, 2, 128, 64)
    assert _rel_fro(ga["o"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_tiled_attention_tiles_beyond_lds(gpu):
    """256-token attention tiles (scores 256 x 256 f32 = 256 KiB): the tiles that do not
    fit in LDS live in a per-workgroup global scratch; results as the oracle's."""
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((1, 2, 512, 64), dtype=np.float32) for _ in range(3))
    ga, ca = W.attention_arrays(q, k, v, 256), W.attention_arrays(q, k, v, 256)
    prog = run_hip(W.rr4(W.tiled_attention(ga, 256)))
    ref = run_workload(W.rr4(W.tiled_attention(ca, 256)))
    assert "gtile_" in prog._native.precompile(0)
    assert _rel_fro(ga["o"], ca["o"]) <= 1e-5
    q64, k64, v64 = (x.astype(np.float64).reshape(1, 2, 2, 256, 64) for x in (q, k, v))
    s = q64 @ k64.transpose(0, 1, 2, 4, 3) / 8.0
    w = np.exp(s - s.max(-1, keepdims=True))
    exact = ((w / w.sum(-1, keepdims=True)) @ v64).reshape(1, 2, 512, 64)
    assert _rel_fro(ga["o"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_llama_block_mfma_tiles(gpu):
    """examples/llama with 64-token tiles, d = 64 and a 128-wide MLP: the attention and
    ReLU-MLP tiles' four matmuls (K = 64 and 128) run on the matrix cores."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((256, 64), dtype=np.float32)
    w1 = (rng.standard_normal((64, 128)) / 8).astype(np.float32)
    w2 = (rng.standard_normal((128, 64)) / 11).astype(np.float32)
    out, ref_out = np.zeros_like(x), np.zeros_like(x)
    prog = run_hip(W.llama_block(x, w1, w2, out, 64, 1e-6))
    ref = run_workload(W.llama_block(x, w1, w2, ref_out, 64, 1e-6))
    assert _has_tile_mma(prog)
    assert _rel_fro(out, ref_out) <= 1e-5
    assert _rel_fro(out, W.llama_block_ref(x, w1, w2, 64, 1e-6)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


@pytest.mark.parametrize("m,k,n", [(32, 16, 32), (32, 64, 96), (96, 32, 32), (32, 48, 32), (16, 64, 48), (48, 32, 80)])
def test_tile_program_matmul_shapes(gpu, m, k, n):
    """Matmul tiles below the GEMM family's blocks on the tile program: M, N multiples of
    32 (or of 16, with at least 32^3 products) with K <= 32 or a multiple of 32 take the
    matrix cores (32x32 or 16x16 MFMA blocks), K = 48 the scalar loop (bit for bit the
    oracle's)."""
    rng = np.random.default_rng(m + k + n)
    a = rng.uniform(-1, 1, (3, 1, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (3, 1, k, n)).astype(np.float32)
    ga = {"a": a, "b": b, "c": np.zeros((3, 1, m, n), np.float32)}
    ca = {k_: v.copy() for k_, v in ga.items()}
    prog = run_hip(W.rr4(W.matmul_tile(ga, m, k, n), 1024))
    ref = run_workload(W.rr4(W.matmul_tile(ca, m, k, n), 1024))
    assert "tile program" in prog._native.precompile(0)  # no merge candidates: below the MFMA block
    mma = k % 2 == 0 and (k <= 32 or k % 32 == 0)
    assert _has_tile_mma(prog) == mma
    if mma and (m % 32 or n % 32):
        assert "tile_mma16<" in prog._native.precompile(0)
    if mma:
        assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    else:
        np.testing.assert_array_equal(ga["c"], ca["c"])
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_validated_matmul_and_exact_2x2(gpu):
    a = np.array([[[[1.0, 2.0], [3.0, 4.0]]]], np.float32)
    b = np.array([[[[5.0, 6.0], [7.0, 8.0]]]], np.float32)
    ga = {"a": a, "b": b, "c": np.zeros((1, 1, 2, 2), np.float32)}
    run_hip(W.matmul_tile(ga, 2, 2, 2))
    np.testing.assert_array_equal(ga["c"][0, 0], np.array([[19.0, 22.0], [43.0, 50.0]], np.float32))
    rng = np.random.default_rng(0)
    a = rng.standard_normal((2, 1, 16, 16), dtype=np.float32)
    b = rng.standard_normal((2, 1, 16, 16), dtype=np.float32)
    ga = {"a": a.copy(), "b": b.copy(), "c": np.zeros((2, 1, 16, 16), np.float32)}
    ca = {"a": a.copy(), "b": b.copy(), "c": np.zeros((2, 1, 16, 16), np.float32)}
    prog = run_hip(W.rr4(W.matmul_tile(ga, 16, 16, 16), 1024))
    ref = run_workload(W.rr4(W.matmul_tile(ca, 16, 16, 16), 1024))
    np.testing.assert_array_equal(ga["c"], ca["c"])
    assert prog.stats.total_cycles == ref.total_cycles


def test_dispatch_and_window_cycle_semantics(gpu):
    from pto_wsp import DispatchPolicy, TaskWindow, WindowMode

    a = np.arange(64, dtype=np.float32).reshape(4, 4, 4)
    arrs = {"a": a, "b": np.zeros_like(a)}
    p0 = run_hip(W.copy_tiles(arrs))
    np.testing.assert_array_equal(arrs["b"], a)
    serial = p0.stats.total_cycles
    arrs["b"][:] = 0
    p1 = run_hip(W.copy_tiles(arrs).dispatch(DispatchPolicy.round_robin(2)))
    np.testing.assert_array_equal(arrs["b"], a)
    assert p1.stats.total_cycles * 2 == serial
    p2 = run_hip(W.copy_tiles(arrs).dispatch(DispatchPolicy.round_robin(2))
                 .task_graph(window=TaskWindow(1, "tasks", WindowMode.STALL)))
    assert p2.stats.total_cycles == serial


def test_dense_dyn_rebinding_without_recompile(gpu):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((4, 4, 4), dtype=np.float32)
    b = rng.standard_normal((4, 4, 4), dtype=np.float32)
    c = np.zeros((4, 4, 4), np.float32)
    prog = W.dense_dyn_mm({"a": a, "b": b, "c": c}).named("dyn_axes").compile(target="hip_gfx950")
    prog.set_axis_sizes({"b": 2})
    prog.execute()
    prog.synchronize()
    np.testing.assert_allclose(c[:2], np.matmul(a[:2], b[:2]), rtol=0, atol=1e-5)
    np.testing.assert_array_equal(c[2:], 0)
    c2 = prog.stats.total_cycles
    c[:] = 0
    prog.set_axis_sizes({"b": 4})
    prog.execute()
    prog.synchronize()
    np.testing.assert_allclose(c, np.matmul(a, b), rtol=0, atol=1e-5)
    assert prog.stats.total_cycles / 4 == c2 / 2


def test_scalar_symbol_rebinding(gpu):
    x = np.arange(16, dtype=np.float32).reshape(4, 4)
    y = np.zeros((4, 4), np.float32)
    prog = W.scale_symbol({"x": x, "y": y}).named("dyn_scalar_symbol").compile(target="hip_gfx950")
    prog.set_symbol_f32("scale_s", 2.0)
    prog.execute()
    prog.synchronize()
    np.testing.assert_array_equal(y, x * 2.0)
    c2 = prog.stats.total_cycles
    prog.set_symbol_f32("scale_s", 3.0)
    prog.execute()
    prog.synchronize()
    np.testing.assert_array_equal(y, x * 3.0)
    assert prog.stats.total_cycles == c2


def test_ragged_axis_rebinding(gpu):
    from pto_wsp import Ragged

    y = np.zeros((3, 1, 1), np.int32)
    r = Ragged(outer_size=2, lengths=[1, 1])
    prog = W.ragged_mark({"y": y}, r).named("dyn_ragged").compile(target="hip_gfx950")
    prog.set_symbol_u64(f"outer_{id(r)}", 2)
    prog.set_symbol_ptr(f"lengths_{id(r)}", np.asarray([1, 1], np.int32))
    prog.execute()
    prog.synchronize()
    np.testing.assert_array_equal(y.reshape(3), [1, 1, 0])
    y[:] = 0
    prog.set_symbol_ptr(f"lengths_{id(r)}", np.asarray([1, 2], np.int32))
    prog.execute()
    prog.synchronize()
    np.testing.assert_array_equal(y.reshape(3), [1, 1, 1])


def test_sparse_select_indices_can_change_without_recompile(gpu):
    """tests/test_codegen_select_sparse.py on the HIP target, plus repeated indices (every
    occurrence applies, in order) and an empty selection; cycles and tasks as the oracle's."""
    from pto_wsp import Sparse

    y = np.zeros((4, 1, 1), np.int32)
    sp = Sparse(outer_size=2, indptr=[0, 2, 3], indices=[0, 2, 1])
    prog = W.sparse_mark({"y": y}, sp).named("dyn_sparse_select").compile(target="hip_gfx950")
    sid = id(sp)
    for outer, indptr, indices, want in [(2, [0, 2, 3], [0, 2, 1], [1, 1, 1, 0]),
                                         (1, [0, 1], [3], [0, 0, 0, 1]),
                                         (3, [0, 3, 3, 6], [1, 1, 0, 3, 1, 2], [1, 3, 1, 1]),
                                         (2, [0, 0, 0], [], [0, 0, 0, 0])]:
        y[:] = 0
        prog.set_symbol_u64(f"outer_{sid}", outer)
        prog.set_symbol_ptr(f"indptr_{sid}", np.asarray(indptr, dtype=np.int32))
        prog.set_symbol_ptr(f"indices_{sid}", np.asarray(indices, dtype=np.int32))
        prog.execute()
        prog.synchronize()
        np.testing.assert_array_equal(y.reshape(4), np.asarray(want, np.int32))
        su, sptr = W.sparse_symbols(sp, outer, indptr, indices)
        ref = run_workload(W.sparse_mark({"y": np.zeros((4, 1, 1), np.int32)}, sp), symbols_u64=su,
                           symbols_ptr=sptr, module_name="dyn_sparse_select")
        assert (int(prog.stats.total_cycles), int(prog.stats.task_count)) == (ref.total_cycles, ref.task_count)
        assert int(prog.stats.task_count) == len(indices)
    # A selected index past the tensor is refused on the host, before any launch; the program
    # stays usable.
    prog.set_symbol_u64(f"outer_{sid}", 1)
    prog.set_symbol_ptr(f"indptr_{sid}", np.asarray([0, 1], np.int32))
    prog.set_symbol_ptr(f"indices_{sid}", np.asarray([4], np.int32))
    with pytest.raises(RuntimeError, match="addressable elements"):
        prog.execute()
    y[:] = 0
    prog.set_symbol_ptr(f"indices_{sid}", np.asarray([2], np.int32))
    prog.execute()
    prog.synchronize()
    np.testing.assert_array_equal(y.reshape(4), [0, 0, 1, 0])


def test_sparse_select_on_device_rows(gpu):
    """Selected tiles of device-resident tensors: each selected tile of y is the rmsnorm of x's,
    the others keep their contents; fp32 rtol 1e-5 against the oracle on the same symbols."""
    import torch
    from pto_wsp import Sparse

    x = np.random.default_rng(7).standard_normal((64, 16, 512), dtype=np.float32)
    y0 = np.full_like(x, -3.0)
    sp = Sparse(outer_size=1, indptr=[0, 3], indices=[5, 40, 63])
    xd, yd = torch.from_numpy(x).to(gpu), torch.from_numpy(y0).to(gpu)
    prog = W.rmsnorm_select({"x": xd, "y": yd}, sp).compile(target="hip_gfx950")
    outer, indptr, sel = 2, [0, 3, 5], [5, 40, 63, 0, 17]
    prog.set_symbol_u64(f"outer_{id(sp)}", outer)
    prog.set_symbol_ptr(f"indptr_{id(sp)}", np.asarray(indptr, np.int32))
    prog.set_symbol_ptr(f"indices_{id(sp)}", np.asarray(sel, np.int32))
    prog.execute()
    prog.synchronize()
    ca = {"x": x.copy(), "y": y0.copy()}
    su, sptr = W.sparse_symbols(sp, outer, indptr, sel)
    ref = run_workload(W.rmsnorm_select(ca, sp), symbols_u64=su, symbols_ptr=sptr)
    got = yd.cpu().numpy()
    np.testing.assert_allclose(got, ca["y"], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(np.delete(got, sel, axis=0), np.delete(y0, sel, axis=0))
    assert (int(prog.stats.total_cycles), int(prog.stats.task_count)) == (ref.total_cycles, ref.task_count)


def _rel_fro(got, ref):
    return float(np.linalg.norm((got - ref).ravel()) / np.linalg.norm(ref.ravel()))


@pytest.mark.parametrize("tiles", [(128, 128, 64), (64, 64, 16), (128, 64, 32)])
def test_bgemm_bf16_mfma_accumulate(gpu, tiles):
    """bf16 x bf16 -> fp32 on MFMA with the InOut accumulator kept on chip (nonzero initial C)."""
    tm, tn, tk = tiles
    rng = np.random.default_rng(5)
    a = W.bf16_round(rng.uniform(-1, 1, (2, 256, 512)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (2, 512, 256)).astype(np.float32))
    c0 = rng.standard_normal((2, 256, 256)).astype(np.float32)
    ga = {"a": a, "b": b, "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.rr4(W.bgemm(ga, tm, tn, tk, W.BF16)))
    ref = run_workload(W.rr4(W.bgemm(ca, tm, tn, tk, W.BF16)))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    rel = _rel_fro(ga["c"], ca["c"])
    assert rel <= 1e-2, rel      # north_star tolerance for bf16 matmul
    assert rel <= 1e-5, rel      # observed: only fp32 summation order differs
    exact = c0.astype(np.float64) + W.bf16_to_f32(a).astype(np.float64) @ W.bf16_to_f32(b).astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


@pytest.mark.parametrize("shape,tiles", [
    ((1, 384, 384, 256), (128, 128, 128)),   # odd tile counts: no merge, K step 128
    ((1, 256, 192, 128), (64, 64, 32)),      # rows merged only (block 128x64)
    ((3, 512, 512, 128), (128, 128, 64)),    # 12 merged blocks: XCD order with a remainder
    ((1, 128, 256, 64), (128, 64, 16)),      # columns merged only (block 128x128, K step 16)
])
def test_bgemm_bf16_mfma_block_shapes(gpu, shape, tiles):
    """GEMM blocks with and without task merging against float64 and the oracle."""
    nb, m, n, k = shape
    tm, tn, tk = tiles
    rng = np.random.default_rng(11)
    a = W.bf16_round(rng.uniform(-1, 1, (nb, m, k)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (nb, k, n)).astype(np.float32))
    c0 = rng.standard_normal((nb, m, n)).astype(np.float32)
    ga = {"a": a, "b": b, "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.bgemm(ga, tm, tn, tk, W.BF16))
    ref = run_workload(W.bgemm(ca, tm, tn, tk, W.BF16))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    exact = c0.astype(np.float64) + W.bf16_to_f32(a).astype(np.float64) @ W.bf16_to_f32(b).astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


@pytest.mark.parametrize("shape,tiles,f16,plain,split", [
    ((2, 256, 256, 64), (128, 128, 64), False, False, 1),     # one K step
    ((1, 512, 256, 128), (128, 128, 64), False, False, 1),    # two K steps, two blocks
    ((1, 256, 512, 192), (128, 128, 64), True, False, 1),     # three K steps, f16
    ((2, 256, 256, 320), (128, 128, 64), False, False, 1),    # five K steps: touches run ahead
    ((2, 256, 256, 256), (128, 128, 32), False, False, 1),    # K step 32: four-stage ring
    ((1, 256, 256, 256), (128, 128, 64), False, True, 1),     # plain store: last K step only
    ((1, 256, 256, 512), (128, 128, 64), False, False, 2),    # K over two P.seq loops
    ((1, 256, 256, 96), (128, 128, 32), False, False, 1),     # A pitch 96: GemmBlock path
])
def test_bgemm_pingpong_block(gpu, shape, tiles, f16, plain, split):
    """256x256 blocks (2x2 merged 128x128 tasks) on the two-group ping-pong template."""
    nb, m, n, k = shape
    tm, tn, tk = tiles
    rng = np.random.default_rng(13)
    a = rng.uniform(-1, 1, (nb, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (nb, k, n)).astype(np.float32)
    if f16:
        a, b = a.astype(np.float16), b.astype(np.float16)
        af, bf = a.astype(np.float64), b.astype(np.float64)
    else:
        a, b = W.bf16_round(a), W.bf16_round(b)
        af, bf = W.bf16_to_f32(a).astype(np.float64), W.bf16_to_f32(b).astype(np.float64)
    c0 = rng.standard_normal((nb, m, n)).astype(np.float32)
    ga = {"a": a, "b": b, "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    dt = W.F16 if f16 else W.BF16
    if split > 1:
        prog = run_hip(W.bgemm_split_k(ga, tm, tn, tk, split, dt))
        ref = run_workload(W.bgemm_split_k(ca, tm, tn, tk, split, dt))
    else:
        prog = run_hip(W.bgemm(ga, tm, tn, tk, dt, plain=plain))
        ref = run_workload(W.bgemm(ca, tm, tn, tk, dt, plain=plain))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    if plain:
        exact = af[:, :, k - tk:] @ bf[:, k - tk:, :]
    else:
        exact = c0.astype(np.float64) + af @ bf
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_bgemm_two_inner_loops(gpu):
    """K split over two P.seq loops: in-kernel iterations decode a mixed radix."""
    rng = np.random.default_rng(12)
    a = W.bf16_round(rng.uniform(-1, 1, (2, 128, 512)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (2, 512, 128)).astype(np.float32))
    c0 = rng.standard_normal((2, 128, 128)).astype(np.float32)
    ga = {"a": a, "b": b, "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.bgemm_split_k(ga, 64, 64, 64, 2))
    ref = run_workload(W.bgemm_split_k(ca, 64, 64, 64, 2))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    exact = c0.astype(np.float64) + W.bf16_to_f32(a).astype(np.float64) @ W.bf16_to_f32(b).astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_bgemm_plain_store_keeps_last_k_step(gpu):
    """store(c, matmul(a, b)) inside P.seq(k): each step overwrites C, so C = A[:, k_last] @ B[k_last]."""
    rng = np.random.default_rng(6)
    a = W.bf16_round(rng.uniform(-1, 1, (1, 128, 256)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (1, 256, 128)).astype(np.float32))
    ga = {"a": a, "b": b, "c": np.zeros((1, 128, 128), np.float32)}
    ca = {"a": a.copy(), "b": b.copy(), "c": np.zeros((1, 128, 128), np.float32)}
    run_hip(W.bgemm(ga, 64, 64, 64, W.BF16, plain=True))
    run_workload(W.bgemm(ca, 64, 64, 64, W.BF16, plain=True))
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    last = W.bf16_to_f32(a)[0, :, 192:].astype(np.float64) @ W.bf16_to_f32(b)[0, 192:, :].astype(np.float64)
    assert _rel_fro(ga["c"][0], last) <= 1e-5


@pytest.mark.parametrize("shape,tiles,plain", [
    ((2, 256, 256, 512), (128, 128, 64), False),   # merged 256x256 blocks, K step 64 as two 32-column stages
    ((1, 384, 384, 256), (128, 128, 128), False),  # odd tile counts (no merge), K step 128 as four stages
    ((3, 256, 192, 96), (64, 64, 32), False),      # rows and columns merged into 128x128 blocks
    ((1, 128, 256, 64), (128, 64, 16), True),      # plain store (last K step), K step 16
    ((1, 128, 128, 64), (64, 64, 8), False),       # K step 8: below the MFMA block, tile program
])
def test_bgemm_f32_mfma(gpu, shape, tiles, plain):
    """f32 x f32 -> f32 tiles (the reference's validated_matmul form) on the f32 MFMA
    block, against the oracle and float64 (MFMA sums the same exact products in
    another order: relative Frobenius 1e-5, the examples' rtol)."""
    nb, m, n, k = shape
    tm, tn, tk = tiles
    rng = np.random.default_rng(13)
    a = rng.uniform(-1, 1, (nb, m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (nb, k, n)).astype(np.float32)
    c0 = rng.standard_normal((nb, m, n)).astype(np.float32)
    ga = {"a": a, "b": b, "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.bgemm(ga, tm, tn, tk, W.F32, plain=plain))
    ref = run_workload(W.bgemm(ca, tm, tn, tk, W.F32, plain=plain))
    assert prog._native.kernel_family("gemm_tile") == ("tile_program" if tk < 16 else "gemm")
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    if plain:
        exact = a[:, :, k - tk:].astype(np.float64) @ b[:, k - tk:, :].astype(np.float64)
    else:
        exact = c0.astype(np.float64) + a.astype(np.float64) @ b.astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


@pytest.mark.parametrize("m,k,n,dt", [
    (512, 512, 512, "f32"),     # 2 x 2 blocks of 256, 16 stages of 32 columns
    (512, 1024, 256, "bf16"),   # 2 x 1 blocks, 16 stages of 64 (ping-pong)
    (768, 192, 512, "f16"),     # 3 x 2 blocks, 3 stages of 64
])
def test_matmul_large_tiles(gpu, m, k, n, dt):
    """The validated_matmul form (one task per batch, C[b] = A[b] @ B[b]) with tiles above
    256 rows / columns and K above 128: each task runs as 256 x 256 blocks whose K loop
    takes the task's K in LDS stages."""
    rng = np.random.default_rng(m + k + n)
    a32 = rng.uniform(-1, 1, (2, 1, m, k)).astype(np.float32)
    b32 = rng.uniform(-1, 1, (2, 1, k, n)).astype(np.float32)
    if dt == "f16":
        a, b, wdt, up = a32.astype(np.float16), b32.astype(np.float16), W.F16, lambda x: x.astype(np.float64)
    elif dt == "bf16":
        a, b, wdt, up = W.bf16_round(a32), W.bf16_round(b32), W.BF16, lambda x: W.bf16_to_f32(x).astype(np.float64)
    else:
        a, b, wdt, up = a32, b32, W.F32, lambda x: x.astype(np.float64)
    ga = {"a": a.copy(), "b": b.copy(), "c": np.zeros((2, 1, m, n), np.float32)}
    ca = {k_: v.copy() for k_, v in ga.items()}
    prog = run_hip(W.rr4(W.matmul_tile(ga, m, k, n, wdt), 1024))
    ref = run_workload(W.rr4(W.matmul_tile(ca, m, k, n, wdt), 1024))
    assert prog._native.kernel_family("mm") == "gemm" and "gemm program" in prog._native.precompile(0)
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    assert _rel_fro(ga["c"], up(a) @ up(b)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_bgemm_large_tiles_accumulate(gpu):
    """512 x 512 task tiles with a K step of 256 over a P.seq loop of 3 steps (accumulate
    form): 2 x 2 blocks per task, 4 stages per step, against the oracle and float64."""
    rng = np.random.default_rng(21)
    a = W.bf16_round(rng.uniform(-1, 1, (1, 1024, 768)).astype(np.float32))
    b = W.bf16_round(rng.uniform(-1, 1, (1, 768, 512)).astype(np.float32))
    c0 = rng.standard_normal((1, 1024, 512)).astype(np.float32)
    ga = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    ca = {"a": a.copy(), "b": b.copy(), "c": c0.copy()}
    prog = run_hip(W.bgemm(ga, 512, 512, 256, W.BF16))
    ref = run_workload(W.bgemm(ca, 512, 512, 256, W.BF16))
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    assert _rel_fro(ga["c"], ca["c"]) <= 1e-5
    exact = c0.astype(np.float64) + W.bf16_to_f32(a).astype(np.float64) @ W.bf16_to_f32(b).astype(np.float64)
    assert _rel_fro(ga["c"], exact) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


def test_bgemm_f16_mfma_device_tensors(gpu):
    import torch

    rng = np.random.default_rng(7)
    a = rng.uniform(-1, 1, (3, 128, 192)).astype(np.float16)
    b = rng.uniform(-1, 1, (3, 192, 128)).astype(np.float16)
    ad, bd = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    cd = torch.zeros((3, 128, 128), device=gpu, dtype=torch.float32)
    from pto_wsp import DType

    prog = run_hip(W.rr4(W.bgemm({"a": ad, "b": bd, "c": cd}, 64, 64, 64, DType.F16)))
    ca = {"a": a.copy(), "b": b.copy(), "c": np.zeros((3, 128, 128), np.float32)}
    ref = run_workload(W.rr4(W.bgemm(ca, 64, 64, 64, DType.F16)))
    assert _rel_fro(cd.cpu().numpy(), ca["c"]) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles


# ---------------------------------------------------------------- paged GQA decode
def _decode_case(lengths, hkv, group, d, page=16, seed=0, masked=True, f16=False, f32=False):
    ga = W.paged_decode_arrays(lengths, hkv, group, d, page=page, seed=seed, f16=f16, f32=f32)
    ca = {k: v.copy() for k, v in ga.items()}
    dt = W.F32 if f32 else W.F16 if f16 else W.BF16
    prog = run_hip(W.paged_decode(ga, masked=masked, dtype=dt))
    ref = run_workload(W.paged_decode(ca, masked=masked, dtype=dt))
    return prog, ref, ga, ca


@pytest.mark.parametrize("lengths,hkv,group,d", [
    ([37, 16, 200, 1, 256, 513], 2, 4, 128),    # partial, exact, single-token and multi-chunk sequences
    ([300, 77], 1, 8, 64),                       # head dim 64 (one column per lane), 8 query rows
    ([129, 40], 2, 1, 256),                      # head dim 256, one query row
])
def test_paged_decode_family(gpu, lengths, hkv, group, d):
    prog, ref, ga, ca = _decode_case(lengths, hkv, group, d, seed=len(lengths))
    assert prog._native.kernel_family("decode_page") == "decode"
    # chunked folding reassociates fp32 sums: per element rtol 2e-5 with an atol
    # of 2e-5 of the tensor's largest magnitude (entries near zero cancel)
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k]).max()), err_msg=k)
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


@pytest.mark.parametrize("lengths,hkv,group,d,page", [
    ([300, 77, 1, 33], 2, 16, 128, 32),          # 16 query rows at head dim 128 (a 2-pass combine)
    ([129, 40, 700], 2, 8, 256, 16),              # 8 rows at head dim 256 (2-step page ring)
    ([513, 64, 5], 1, 16, 256, 64),               # 16 rows at head dim 256 (4 passes of 4 rows)
    ([300, 77, 1, 33], 1, 32, 128, 16),           # two 16-row blocks per step
    ([129, 40, 700], 2, 48, 128, 8),              # three row blocks, 8-token pages, 2-step ring
    ([513, 64, 5], 2, 24, 64, 16),                # a half-filled second row block at head dim 64
    ([200, 17, 1000], 1, 48, 64, 32),             # three row blocks at head dim 64
])
def test_paged_decode_wide_units(gpu, lengths, hkv, group, d, page):
    """Units of more than 1024 accumulators (query rows x head dim) on the decode
    family: the completing wave folds the partials a few rows per pass; more than
    16 query rows fold as 16-row blocks that share each step's page registers."""
    prog, ref, ga, ca = _decode_case(lengths, hkv, group, d, page=page, seed=len(lengths) + group)
    assert prog._native.kernel_family("decode_page") == "decode"
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k]).max()), err_msg=k)
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


@pytest.mark.parametrize("lengths,hkv,group,d,page,masked", [
    ([37, 16, 200, 1, 256, 513], 2, 4, 128, 16, True),   # partial, exact, single-token and multi-page sequences
    ([300, 77, 0], 1, 8, 64, 32, True),                   # head dim 64, sub-pages, an empty sequence
    ([129, 40, 700], 2, 16, 128, 8, True),                # 16 rows, 8-token pages two to a step
    ([64, 160, 32], 2, 1, 128, 16, False),                # unmasked, one query row
    ([400, 33, 1000], 1, 32, 128, 16, True),              # 32 rows: two row blocks, 2-step rings
    ([250, 0, 1300, 16], 2, 48, 64, 32, True),            # 48 rows at head dim 64
    ([90, 700], 1, 20, 128, 8, True),                     # 20 rows, 8-token pages
    ([333, 64, 1], 2, 8, 256, 32, True),                  # head dim 256
    ([500, 17], 1, 16, 256, 16, False),                   # 16 rows at head dim 256, unmasked
])
def test_paged_decode_f32(gpu, lengths, hkv, group, d, page, masked):
    """f32 q / K / V (the reference's own dtype) on the decode family: scores and p @ v on
    v_mfma_f32_16x16x4_f32, against the oracle and float64 attention."""
    prog, ref, ga, ca = _decode_case(lengths, hkv, group, d, page=page, seed=len(lengths) + d, masked=masked, f32=True)
    assert prog._native.kernel_family("decode_page") == "decode"
    for k in ("m", "l", "o", "out"):
        fin = np.isfinite(ca[k])
        assert np.array_equal(fin, np.isfinite(ga[k])), k
        np.testing.assert_allclose(ga[k][fin], ca[k][fin], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k][fin]).max()), err_msg=k)
    live = np.asarray(lengths) > 0
    if masked or all(n % page == 0 for n in lengths):
        assert _rel_fro(ga["out"][live], W.paged_decode_ref(ga)[live]) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


def test_paged_decode_long_streams(gpu):
    """Thousands of pages: every wave folds a long stream of pages that crosses
    unit and page-table-run boundaries, mixing long units (split over several
    waves, completed by the last arriver), units shorter than the page ring,
    and an empty sequence (its accumulators stay untouched)."""
    lengths = [8192, 1, 0, 17, 5000, 40, 16, 3000, 7777, 2, 600, 4096, 33, 2500]
    prog, ref, ga, ca = _decode_case(lengths, 8, 4, 128, seed=11)
    assert prog._native.kernel_family("decode_page") == "decode"
    assert ref.task_count > 8 * 1024
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k][np.isfinite(ca[k])]).max()),
                                   err_msg=k)
    assert np.all(ga["m"][2] == -np.inf) and np.all(ga["l"][2] == 0) and np.all(ga["o"][2] == 0)
    live = np.asarray(lengths) > 0
    assert _rel_fro(ga["out"][live], W.paged_decode_ref(ga)[live]) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


def test_paged_decode_folds_the_normalisation(gpu):
    """The out = o / l launch that follows the page loop runs inside the decode
    kernel (one launch) with the same bits as the separate launch; written in
    place (out is o) it overlaps the decode's own tensors and stays a launch."""
    lengths = [300, 0, 77, 1]
    prog, ref, ga, ca = _decode_case(lengths, 2, 4, 128, seed=4)
    assert prog.stats.launches == 1
    live = np.asarray(lengths) > 0
    np.testing.assert_array_equal(ga["out"][live], ga["o"][live] / ga["l"][live])
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k][np.isfinite(ca[k])]).max()),
                                   err_msg=k)
    assert np.isnan(ga["out"][1]).all() and np.isnan(ca["out"][1]).all()  # 0 / 0 for the empty sequence

    ga = W.paged_decode_arrays(lengths, 2, 4, 128, seed=4)
    ca = {k: v.copy() for k, v in ga.items()}
    prog = run_hip(W.paged_decode(ga, out_key="o"))
    run_workload(W.paged_decode(ca, out_key="o"))
    assert prog.stats.launches == 2
    np.testing.assert_allclose(ga["o"], ca["o"], rtol=2e-5, atol=2e-5 * float(np.abs(ca["o"][np.isfinite(ca["o"])]).max()))


def test_paged_decode_sixteen_rows(gpu):
    """16 query rows fill every MFMA column.  Unmasked it is the decode family; with
    the [1,16] mask on a square [16,16] score tile the reference's broadcast rule
    subtracts mask[row] (a row broadcast, src/python/pto_codegen.cpp:1094-1105),
    which the decode template's row-mask form applies (each lane subtracts its
    query row's value): the launch matches the oracle, not a token mask.  Rows
    whose value is 1e30 end with uniform weights, as in the oracle."""
    prog, ref, ga, ca = _decode_case([96, 512, 16], 1, 16, 64, seed=3, masked=False)
    assert prog._native.kernel_family("decode_page") == "decode"
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k]).max()), err_msg=k)
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5
    for lengths, hkv, d in (([90, 40], 1, 64), ([700, 5, 0, 260], 2, 128), ([33, 1500], 1, 256)):
        prog, ref, ga, ca = _decode_case(lengths, hkv, 16, d, seed=3, masked=True)
        assert prog._native.kernel_family("decode_page") == "decode"
        assert "true, false, false, true>" in prog._native.precompile(0)  # the row-mask form
        for k in ("m", "l", "o", "out"):
            fin = np.isfinite(ca[k])
            assert np.array_equal(fin, np.isfinite(ga[k])), k
            np.testing.assert_allclose(ga[k][fin], ca[k][fin], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k][fin]).max()),
                                       err_msg=k)
        assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


def test_paged_decode_f16_and_unmasked(gpu):
    lengths = [64, 160, 32]                      # multiples of the page: no mask needed
    prog, ref, ga, ca = _decode_case(lengths, 2, 4, 128, seed=5, masked=False, f16=True)
    assert prog._native.kernel_family("decode_page") == "decode"
    np.testing.assert_allclose(ga["out"], ca["out"], rtol=2e-5, atol=2e-5 * float(np.abs(ca["out"]).max()))
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5


def test_paged_decode_8_token_pages(gpu):
    """8-token pages run on the decode family two to a 16-token step (tokens 8-15
    from the step's second page); a unit with an odd page count ends on a step
    without a second page, whose tokens 8-15 get -inf scores.  The lengths give
    5, 1, 8, 1, 38 and 2 pages."""
    prog, ref, ga, ca = _decode_case([37, 8, 61, 1, 300, 16], 2, 4, 64, page=8, seed=3)
    assert prog._native.kernel_family("decode_page") == "decode"
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=2e-5, atol=2e-5 * float(np.abs(ca[k]).max()), err_msg=k)
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count


def test_paged_decode_tile_program_path(gpu):
    """A [1, page] mask with as many query rows as page tokens also fits the scores as a
    row broadcast, which the decode template does not take: the tile program runs the
    page loop in order.  The lengths are whole pages, so the mask is zero and both
    readings of it agree with attention over the valid tokens."""
    prog, ref, ga, ca = _decode_case([40, 8, 64], 2, 8, 64, page=8, seed=3)
    assert prog._native.kernel_family("decode_page") == "tile_program"
    for k in ("m", "l", "o", "out"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=1e-5, atol=1e-6, err_msg=k)
    assert _rel_fro(ga["out"], W.paged_decode_ref(ga)) <= 1e-5


def test_paged_decode_extent_above_declared_maximum_raises(gpu):
    """A page count above DenseDyn's declared maximum is reported by synchronize()
    (forced from the host; every device access stays bounds-checked)."""
    from pto_wsp import ExecutionError

    ga = W.paged_decode_arrays([40, 20], 1, 4, 128, seed=2)
    ga["npages"][1] = ga["page_table"].shape[1] + 1
    prog = W.paged_decode(ga).compile(target="hip_gfx950")
    prog.execute()
    with pytest.raises(ExecutionError, match="declared maximum"):
        prog.synchronize()


# ---------------------------------------------------------------- host path
def test_device_extent_cycles_follow_the_page_counts(gpu):
    """Page counts in a device tensor: total_cycles comes from the cycle model at
    synchronize() and follows the tensor's contents from run to run (the oracle on
    host copies gives the expected values)."""
    import torch

    ga = W.paged_decode_arrays([37, 200, 16, 90], 2, 4, 128, seed=21)
    dev = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in ga.items() if k != "lengths"}
    for k in ("q", "k_cache", "v_cache"):  # bf16 bits held as uint16
        dev[k] = torch.from_numpy(ga[k].view(np.int16)).to(gpu).view(torch.bfloat16)
    prog = W.paged_decode(dev).compile(target="hip_gfx950")
    for npg in ([3, 13, 1, 6], [1, 2, 1, 1], [3, 13, 1, 6]):
        dev["npages"].copy_(torch.tensor(npg, dtype=torch.int32))
        for k, v in (("m", -np.inf), ("l", 0.0), ("o", 0.0)):
            dev[k].fill_(v)
        prog.execute()
        prog.synchronize()
        ca = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in ga.items()}
        ca["npages"] = np.asarray(npg, np.int32)
        ref = run_workload(W.paged_decode(ca))
        assert prog.stats.total_cycles == ref.total_cycles, npg
        assert prog.stats.task_count == ref.task_count, npg
        np.testing.assert_allclose(dev["out"].cpu().numpy(), ca["out"], rtol=2e-5,
                                   atol=2e-5 * float(np.abs(ca["out"]).max()))


def test_rebinding_follows_a_swapped_tensor(gpu):
    """Device tensors are rebound only when their storage changes: swapping the
    data of the input Tensor between runs is seen by the next run."""
    import torch

    from pto_wsp import Dense, In, Out, P, Tensor, Tile, kernel, pto, workload

    x1 = torch.randn((2, 4, 16, 128), device=gpu)
    x2 = torch.randn((2, 4, 16, 128), device=gpu)
    y = torch.zeros_like(x1)
    X = Tensor(data=x1, shape=tuple(x1.shape), dtype=W.F32)
    Y = Tensor(data=y, shape=tuple(y.shape), dtype=W.F32)

    @kernel
    def scale_tile(x: In[Tile[16, 128, W.F32]], out: Out[Tile[16, 128, W.F32]]):
        pto.store(out, pto.mul(x, x))

    @workload
    def wl():
        for b in P(Dense[2]()):
            for t in P(Dense[4]()):
                scale_tile[b, t](x=X[b][t], out=Y[b][t])

    prog = wl().compile(target="hip_gfx950")
    for x in (x1, x1, x2, x1):
        X.data = x
        prog.execute()
        prog.synchronize()
        torch.testing.assert_close(y, x * x, rtol=0, atol=0)


# ---------------------------------------------------------------- cond, slots, keyed dispatch
def _cond_arrays():
    return {"a0": np.full((4, 1, 2, 2), 1.0, np.float32), "a1": np.full((4, 1, 2, 2), 2.0, np.float32),
            "c": np.zeros((4, 1, 2, 2), np.float32)}


def test_cond_runtime_predicate_by_axis_var(gpu):
    """tests/test_codegen_cond.py (predicate on the grid variable: a task mask per branch)."""
    from pto_wsp.scalar_expr import axis

    a = _cond_arrays()
    prog = run_hip(W.cond_copy(a, axis("b") < 2))
    np.testing.assert_array_equal(a["c"][:2], a["a0"][:2])
    np.testing.assert_array_equal(a["c"][2:], a["a1"][2:])
    ref = run_workload(W.cond_copy(_cond_arrays(), axis("b") < 2))
    assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


def test_cond_runtime_predicate_by_symbol_without_rebuild(gpu):
    from pto_wsp.scalar_expr import axis, fnv1a_64, symbol_u64

    pred = axis("b") < symbol_u64("cut").cast_i64()
    a = _cond_arrays()
    prog = W.cond_copy(a, pred).compile(target="hip_gfx950")
    for cut, split in [(2, 2), (1, 1), (0, 0), (7, 4), (3, 3)]:
        a["c"].fill(0)
        prog.set_symbol_u64("cut", cut)
        prog.execute()
        prog.synchronize()
        np.testing.assert_array_equal(a["c"][:split], a["a0"][:split])
        np.testing.assert_array_equal(a["c"][split:], a["a1"][split:])
        ref = run_workload(W.cond_copy(_cond_arrays(), pred), symbols_u64={fnv1a_64("cut"): cut})
        assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


def test_scalar_expr_dispatch_reads_task_params_tags_and_symbols(gpu):
    """tests/test_codegen_scalar_expr_eval.py: results and the makespans 6, 3, 5, 6 x per task."""
    from pto_wsp import DispatchPolicy
    from pto_wsp.scalar_expr import symbol_u64

    a = np.arange(6 * 4 * 4, dtype=np.float32).reshape(6, 4, 4)
    arrs = {"a": a, "b": np.zeros_like(a)}
    p0 = run_hip(W.copy_tiles(arrs, 6).named("scalar_expr_serial"))
    np.testing.assert_array_equal(arrs["b"], a)
    per = int(p0.stats.total_cycles) // 6
    assert int(p0.stats.total_cycles) == 6 * per > 0
    by_tags = DispatchPolicy.affinity(lambda t: (t.tags["mask"] & t.params[0].cast_u64()), num_aicpus=2)
    ternary = DispatchPolicy.affinity(
        lambda t: (t.params[0] == symbol_u64("special").cast_i64()).where(0, 1).cast_u64(), num_aicpus=2)
    for policy, sym, runs in [(by_tags, "mask", [(0, 6), (1, 3)]), (ternary, "special", [(0, 5), (7, 6)])]:
        prog = W.copy_tiles(arrs, 6).dispatch(policy).compile(target="hip_gfx950")
        for value, lanes in runs:
            arrs["b"][:] = 0
            prog.set_symbol_u64(sym, value)
            prog.execute()
            prog.synchronize()
            np.testing.assert_array_equal(arrs["b"], a)
            assert int(prog.stats.total_cycles) == lanes * per


@pytest.mark.parametrize("device", [False, True])
def test_slot_load_from_tensor_drives_cond_without_rebuild(gpu, device):
    """tests/test_codegen_slots_tensor_predicate.py: a kernel writes the flag, the slot load reads
    it back from the device in the same run, and the branch follows it."""
    import torch

    host = {"src": np.zeros((1, 1, 1, 1), np.int32), "flag": np.zeros((1, 1, 1, 1), np.int32),
            "y": np.zeros((1, 1, 1, 1), np.int32)}
    arrs = {k: torch.from_numpy(v).to(gpu) for k, v in host.items()} if device else host
    prog = W.slot_branch(arrs).compile(target="hip_gfx950")
    for src, want in [(-1, 7), (0, 3), (1, 7), (0, 3)]:
        for k in ("src", "flag", "y"):
            if device:
                arrs[k].fill_(src if k == "src" else 5)
            else:
                arrs[k].fill(src if k == "src" else 5)
        prog.execute()
        prog.synchronize()
        flag = int(arrs["flag"].reshape(-1)[0])
        y = int(arrs["y"].reshape(-1)[0])
        assert (flag, y) == (src, want)
        ref_arrs = {"src": np.full((1, 1, 1, 1), src, np.int32), "flag": np.full((1, 1, 1, 1), 5, np.int32),
                    "y": np.full((1, 1, 1, 1), 5, np.int32)}
        ref = run_workload(W.slot_branch(ref_arrs))
        assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


def test_slot_loads_inside_a_parallel_loop(gpu):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 4, 8)).astype(np.float32)
    src = np.array([3, 0, 8, 5, 1, 2], np.int32).reshape(6, 1, 1)
    arrs = {"x": x, "y": np.zeros_like(x), "src": src.copy(), "sel": np.zeros_like(src)}
    prog = run_hip(W.slot_chain(arrs))
    odd = (src.reshape(6) & 1) == 1
    np.testing.assert_array_equal(arrs["sel"], src)
    np.testing.assert_allclose(arrs["y"][odd], x[odd] * 2, rtol=1e-6)
    np.testing.assert_allclose(arrs["y"][~odd], x[~odd] + 1, rtol=1e-6)
    ref = run_workload(W.slot_chain({"x": x.copy(), "y": np.zeros_like(x), "src": src.copy(), "sel": np.zeros_like(src)}))
    assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


@pytest.mark.parametrize("case", ["mod3", "corner", "none", "all", "symbol"])
def test_masked_grid_row_program(gpu, case):
    """A predicate on both grid variables: only the kept tiles are written (task list on the row
    program); fp32 rtol 1e-5 against the oracle, untouched tiles unchanged, and the symbol case
    rebinds without a rebuild."""
    import torch
    from pto_wsp.scalar_expr import axis, fnv1a_64, symbol_u64

    preds = {"mod3": ((axis("b") + axis("t")) % 3) != 0, "corner": (axis("t") >= 5) & (axis("b") == 1),
             "none": axis("b") < 0, "all": axis("b") >= 0, "symbol": axis("t") < symbol_u64("n").cast_i64()}
    x = np.random.default_rng(2).standard_normal((3, 7, 16, 128)).astype(np.float32)
    y0 = np.full_like(x, -4.0)
    xd, yd = torch.from_numpy(x).to(gpu), torch.from_numpy(y0).to(gpu)
    prog = W.masked_rmsnorm({"x": xd, "y": yd}, preds[case]).compile(target="hip_gfx950")
    for n in ([2, 6, 0] if case == "symbol" else [0]):
        yd.copy_(torch.from_numpy(y0))
        prog.set_symbol_u64("n", n)
        prog.execute()
        prog.synchronize()
        ca = {"x": x.copy(), "y": y0.copy()}
        ref = run_workload(W.masked_rmsnorm(ca, preds[case]), symbols_u64={fnv1a_64("n"): n})
        np.testing.assert_allclose(yd.cpu().numpy(), ca["y"], rtol=1e-5, atol=1e-6)
        assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


def test_masked_grid_tile_program_with_accumulator(gpu):
    """A mask over bgemm output tiles with the K loop inside the kernel (tile program with a task
    list): kept tiles get C += A @ B, the others keep C."""
    from pto_wsp.scalar_expr import axis

    rng = np.random.default_rng(3)
    a = rng.standard_normal((2, 64, 48)).astype(np.float16)
    b = rng.standard_normal((2, 48, 32)).astype(np.float16)
    c = rng.standard_normal((2, 64, 32)).astype(np.float32)
    pred = ((axis("m") * 2 + axis("n") + axis("b")) % 3) == 1
    arrs = {"a": a, "b": b, "c": c.copy()}
    prog = run_hip(W.masked_bgemm(arrs, pred))
    ca = {"a": a, "b": b, "c": c.copy()}
    ref = run_workload(W.masked_bgemm(ca, pred))
    np.testing.assert_allclose(arrs["c"], ca["c"], rtol=1e-5, atol=1e-5)
    assert not np.array_equal(ca["c"], c) and np.any(ca["c"] == c)
    assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


# ---------------------------------------------------------------- cpp_src kernels
@pytest.mark.parametrize("device", [False, True])
def test_cpp_src_slot_predicate_without_rebuild(gpu, device):
    """tests/test_codegen_slots_tensor_predicate.py with cpp_src bodies run on the device: the
    flag a body writes drives the branch through a slot; two cycles per run (one per body)."""
    import torch

    host = {"x": np.zeros((1, 1, 1, 1), np.float32), "flag": np.zeros((1, 1, 1, 1), np.int32),
            "y": np.zeros((1, 1, 1, 1), np.int32)}
    arrs = {k: torch.from_numpy(v).to(gpu) for k, v in host.items()} if device else host
    prog = W.cpp_slot_branch(arrs).compile(target="hip_gfx950")
    for x, flag, y in [(-1.0, 0, 3), (1.0, 1, 7), (0.5, 1, 7), (0.0, 0, 3)]:
        if device:
            arrs["x"].fill_(x), arrs["flag"].fill_(9), arrs["y"].fill_(0)
        else:
            arrs["x"].fill(x), arrs["flag"].fill(9), arrs["y"].fill(0)
        prog.execute()
        prog.synchronize()
        assert (int(arrs["flag"].reshape(-1)[0]), int(arrs["y"].reshape(-1)[0])) == (flag, y)
        assert (int(prog.stats.total_cycles), int(prog.stats.task_count)) == (2, 2)


@pytest.mark.parametrize("tu", [False, True], ids=["cpp_src", "cpp_tu_path"])
@pytest.mark.parametrize("masked", [False, True])
def test_cpp_src_task_descriptor_matches_oracle(gpu, masked, tu, tmp_path):
    """A body that copies its task descriptor (args, counts, strides, two x elements) into its
    output and reports per-task cycles: bit-identical to the oracle's g++ build of the same body.
    tu: the same probe as a whole translation unit (a helper function, pto::cpu_sim's counter)."""
    from pto_wsp.scalar_expr import axis

    path = None
    if tu:
        path = str(tmp_path / "probe.cpp")
        with open(path, "w") as f:
            f.write(W.PROBE_TU)
    pred = (axis("b") != 1) if masked else None
    x = np.arange(3 * 2 * 8, dtype=np.float32).reshape(3, 2, 2, 4)
    ga = {"x": x.copy(), "o": np.full((2, 3, 2, 2, 16), -1.0, np.float32)}
    ca = {"x": x.copy(), "o": np.full((2, 3, 2, 2, 16), -1.0, np.float32)}
    prog = run_hip(W.cpp_probe(ga, pred, tu_path=path))
    ref = run_workload(W.cpp_probe(ca, pred, tu_path=path))
    np.testing.assert_array_equal(ga["o"], ca["o"])
    assert (int(prog.stats.total_cycles), int(prog.stats.task_count)) == (ref.total_cycles, ref.task_count)


def test_cpp_tu_path_copy_like_the_reference(gpu, tmp_path):
    """The reference's tu_copy translation unit (tests/test_npu_codegen_emit.py:155-206) on the
    device: an exact 4x4 copy, 0 cycles, also through a transposed output view."""
    from test_custom_kernels import TU_COPY, tu_copy_workload

    p = tmp_path / "tu_copy.cpp"
    p.write_text(TU_COPY)
    x = np.arange(16, dtype=np.float32).reshape(4, 4)
    y = np.zeros((4, 4), np.float32)
    prog = run_hip(tu_copy_workload(x, y, p))
    np.testing.assert_array_equal(y, x)
    assert (int(prog.stats.total_cycles), int(prog.stats.task_count)) == (0, 1)
    yt = np.zeros((4, 4), np.float32)
    run_hip(tu_copy_workload(x, yt.T, p))
    np.testing.assert_array_equal(yt.T, x)


def test_cond_on_a_symbol_inside_a_grid(gpu):
    """A predicate that reads no grid variable is evaluated once on the host and picks the
    branch launched over the whole grid; nested under it, a grid-variable predicate masks."""
    from pto_wsp.scalar_expr import axis, fnv1a_64, symbol_u64

    pred = (symbol_u64("flag") != 0) & (axis("b") >= 0)
    host_only = symbol_u64("flag") != 0
    for p in (host_only, pred):
        a = _cond_arrays()
        prog = W.cond_copy(a, p).compile(target="hip_gfx950")
        for flag in (0, 1, 0):
            a["c"].fill(0)
            prog.set_symbol_u64("flag", flag)
            prog.execute()
            prog.synchronize()
            np.testing.assert_array_equal(a["c"], a["a0"] if flag else a["a1"])
            ref = run_workload(W.cond_copy(_cond_arrays(), p), symbols_u64={fnv1a_64("flag"): flag})
            assert (prog.stats.total_cycles, prog.stats.task_count) == (ref.total_cycles, ref.task_count)


def test_example_llama(gpu):
    """examples/llama: five kernels per seq tile (attention, residual, rmsnorm, MLP, residual)."""
    from test_oracle_golden import CYC, _llama_inputs

    x, w1, w2 = _llama_inputs()
    out, ref_out = np.zeros_like(x), np.zeros_like(x)
    prog = run_hip(W.llama_block(x, w1, w2, out, 8, 1e-6))
    ref = run_workload(W.llama_block(x, w1, w2, ref_out, 8, 1e-6))
    np.testing.assert_allclose(out, ref_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, W.llama_block_ref(x, w1, w2, 8, 1e-6), rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == ref.total_cycles == CYC["llama"]["total_cycles"]


def test_example_deepseek_v3(gpu):
    """examples/deepseek_v3: two expert matmuls and the gated mix per 8-row tile."""
    from test_oracle_golden import CYC, _moe_inputs

    x, w0, w1, g = _moe_inputs()
    y, ref_y = np.zeros_like(x), np.zeros_like(x)
    prog = run_hip(W.moe_block(x, w0, w1, g, y))
    ref = run_workload(W.moe_block(x, w0, w1, g, ref_y))
    np.testing.assert_allclose(y, ref_y, rtol=1e-5, atol=1e-6)
    assert prog.stats.total_cycles == ref.total_cycles == CYC["deepseek_v3"]["total_cycles"]


def test_example_tensor_data(gpu):
    from test_oracle_golden import CYC

    rng = np.random.default_rng(0)
    a = rng.standard_normal((2, 2, 2, 32, 32), dtype=np.float32)
    b = rng.standard_normal((2, 2, 2, 32, 32), dtype=np.float32)
    x = rng.standard_normal((2, 4, 32, 32), dtype=np.float32)
    c, y = np.zeros_like(a), np.zeros_like(x)
    p1 = run_hip(W.add_tiles5(a, b, c))
    p2 = run_hip(W.square_tiles4(x, y))
    np.testing.assert_array_equal(c, a + b)
    np.testing.assert_array_equal(y, x * x)
    assert p1.stats.total_cycles == CYC["tensor_data_add"]["total_cycles"]
    assert p2.stats.total_cycles == CYC["tensor_data_square"]["total_cycles"]


def test_row_program_store_into_a_transposed_view(gpu):
    """The row program's vector width must follow the strides of the params that are only
    stored: out is a transposed view (column stride R), so its rows are written element by
    element while x's are read 16 bytes at a time."""
    from pto_wsp import In, Out, P, Dense, Tensor, Tile, kernel, pto, workload

    x = np.random.default_rng(8).standard_normal((2, 3, 16, 64)).astype(np.float32)
    y_base = np.zeros((2, 3, 64, 16), np.float32)
    y_view = y_base.transpose(0, 1, 3, 2)
    X = Tensor(data=x, shape=x.shape, dtype=W.F32)
    Y = Tensor(data=y_view, shape=y_view.shape, dtype=W.F32)

    @kernel
    def scale_tile(x_t: In[Tile[16, 64, W.F32]], out: Out[Tile[16, 64, W.F32]]):
        pto.store(out, pto.mul(x_t, pto.constant(2.0, W.F32)))

    @workload
    def wl():
        for b in P(Dense[2]()):
            for t in P(Dense[3]()):
                scale_tile[b, t](x_t=X[b][t], out=Y[b][t])

    run_hip(W.rr4(wl()))
    np.testing.assert_array_equal(y_base.transpose(0, 1, 3, 2), x * np.float32(2.0))


def test_softmax_three_phase_row_loops(gpu):
    """examples/softmax with 8 vocab tiles (disjoint views): the two launches with P.seq
    accumulators run as row programs over their in-kernel loop (accumulators in registers,
    butterfly reductions), within rtol 1e-5 of the oracle's sequential order."""
    lg = (0.1 * np.random.default_rng(2).standard_normal((2, 64, 512), dtype=np.float32)).astype(np.float32)
    ga, ca = W.softmax3_arrays(lg), W.softmax3_arrays(lg)
    prog = run_hip(W.rr4(W.softmax3(ga)))
    ref = run_workload(W.rr4(W.softmax3(ca)))
    for k in ("probs", "rmax", "rsum"):
        np.testing.assert_allclose(ga[k], ca[k], rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(ga["rmax"], ca["rmax"])  # max is exact in any order
    assert prog.stats.total_cycles == ref.total_cycles
