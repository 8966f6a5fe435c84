"""CPU-side checks of the native HIP backend (no GPU needed).

* libptowsp_hip.so loads and exports every function include/*.h declares;
* every test workload is accepted, and each of its launches is emitted and
  built for gfx950 by hiprtc;
* the product's cycle model (C++) gives the same total_cycles and task
  count as the oracle (C) on every workload;
* a CSR select (P.sel) follows its runtime symbols in the cycle model exactly
  as the oracle does.
"""

import ctypes
import os
import re

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from pto_wsp import CompileError, DType, Dense, In, Out, P, Ragged, Sparse, Tensor, Tile, kernel, pto, workload
from pto_wsp.ir_bridge import workload_to_codegen_ir
from pto_wsp.program import Program

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(header: str) -> list[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ptowsp_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    from pto_wsp import _hip

    lib = _hip.library()
    names = declared_functions("ptowsp_hip.h")
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_oracle_exports_its_header():
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "_build", "libptowsp_cpusim.so"))
    text = open(os.path.join(ROOT, "oracle", "cpu_sim.h")).read()
    for n in re.findall(r"\b(pto_cpusim_\w+)\s*\(", text):
        assert hasattr(lib, n), n


def _cases():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 16, 128), dtype=np.float32)
    xs = rng.standard_normal((1, 3, 32, 512), dtype=np.float32)
    lg = (0.1 * rng.standard_normal((1, 32, 256), dtype=np.float32)).astype(np.float32)
    a16 = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    b16 = rng.standard_normal((1, 64, 64), dtype=np.float32).astype(np.float16)
    q = rng.standard_normal((1, 16), dtype=np.float32)
    k = rng.standard_normal((64, 16), dtype=np.float32)
    v = rng.standard_normal((64, 16), dtype=np.float32)
    qa = rng.standard_normal((1, 2, 16, 8), dtype=np.float32)
    return {
        "rmsnorm": (lambda: W.rr4(W.rmsnorm({"x": x, "y": np.zeros_like(x)})), {}),
        "softmax": (lambda: W.rr4(W.softmax({"x": xs, "y": np.zeros_like(xs)})), {}),
        "softmax3": (lambda: W.rr4(W.softmax3(W.softmax3_arrays(lg))), {}),
        "bgemm_f16": (lambda: W.rr4(W.bgemm({"a": a16, "b": b16, "c": np.zeros((1, 64, 64), np.float32)})), {}),
        "bgemm_bf16": (lambda: W.rr4(W.bgemm({"a": W.bf16_round(np.ones((1, 256, 256), np.float32)),
                                               "b": W.bf16_round(np.ones((1, 256, 256), np.float32)),
                                               "c": np.zeros((1, 256, 256), np.float32)}, 128, 128, 64, W.BF16)), {}),
        "decode": (lambda: W.rr4(W.decode_attention({"q": q, "k_t": k.T.copy(), "v": v, "o": np.zeros((1, 16), np.float32)}), 1024), {}),
        "attention": (lambda: W.rr4(W.tiled_attention(W.attention_arrays(qa, qa, qa, 8), 8)), {}),
        "copy": (lambda: W.copy_tiles({"a": np.arange(64, dtype=np.float32).reshape(4, 4, 4),
                                       "b": np.zeros((4, 4, 4), np.float32)}), {}),
        "dense_dyn": (lambda: W.dense_dyn_mm({"a": np.ones((4, 4, 4), np.float32), "b": np.ones((4, 4, 4), np.float32),
                                              "c": np.zeros((4, 4, 4), np.float32)}), {"b": 3}),
        "paged_decode": (lambda: W.paged_decode(W.paged_decode_arrays([37, 16, 200], 2, 4, 128, seed=1)), {}),
        "paged_decode_p8": (lambda: W.paged_decode(W.paged_decode_arrays([37, 9], 1, 4, 64, page=8, seed=1)), {}),
        "lightning_pto": (lambda: W.lightning_indexer(*W.lightning_inputs(), np.zeros((2, 4, 1, 8), np.int32), "pto"), {}),
        "lightning_ptoisa": (lambda: W.lightning_indexer(*W.lightning_inputs(), np.zeros((2, 4, 1, 8), np.int32),
                                                         "ptoisa"), {}),
    }


@pytest.mark.parametrize("name", list(_cases()))
def test_emitted_kernels_build_for_gfx950(name):
    from pto_wsp._hip import NativeProgram

    make, _ = _cases()[name]
    prog = NativeProgram(workload_to_codegen_ir(make(), name).module)
    assert prog.num_launches() >= 1
    src = prog.precompile(0)
    assert re.search(r"__global__ void __launch_bounds__\(\d+\) (__attribute__\(\(\w+\(\d+(, \d+)?\)\)\) )?"
                     r"ptowsp_(row|tile|gemm|decode)_\w+\(", src)


@pytest.mark.parametrize("name", ["rmsnorm", "softmax3", "bgemm_f16"])
def test_serial_variants_build_for_gfx950(name):
    from pto_wsp._hip import NativeProgram

    make, _ = _cases()[name]
    prog = NativeProgram(workload_to_codegen_ir(make(), name).module)
    src = prog.precompile(0, serial=True)
    # one workgroup: no grid variable is decoded from the group index
    assert "t < ngroups_;" in src and "ngroups_ *=" not in src


def test_grouped_serial_variant_builds_for_gfx950():
    """The rescale launch of the three-phase softmax with v (grid variable 2) looped in program
    order inside each workgroup and (b, s) decoded from the group index."""
    from pto_wsp._hip import NativeProgram

    make, _ = _cases()["softmax3"]
    prog = NativeProgram(workload_to_codegen_ir(make(), "softmax3").module)
    src = prog.precompile(2, serial=True, seq_mask=0b100)
    assert "ngroups_ *= A.ext[0];" in src and "ngroups_ *= A.ext[1];" in src and "ngroups_ *= A.ext[2]" not in src
    assert "vars[1] = q_ % A.ext[1]" in src and "vars[0] = q_;" in src
    assert "for (vars[2] = 0; vars[2] < e0; ++vars[2])" in src


@pytest.mark.parametrize("name", list(_cases()))
def test_cycle_model_matches_oracle(name):
    from pto_wsp._hip import NativeProgram

    make, sizes = _cases()[name]
    w = make()
    build = workload_to_codegen_ir(w, name)
    prog = NativeProgram(build.module)
    axis = Program._infer_axis_sizes(w)
    axis.update(sizes)
    got = prog.cycle_model(build.tensors, axis, {}, {})
    ref = run_workload(make(), axis_sizes=sizes)
    assert (got.total_cycles, got.task_count) == (ref.total_cycles, ref.task_count)


def test_family_selection():
    from pto_wsp._hip import NativeProgram

    x = np.zeros((1, 1, 16, 128), np.float32)
    prog = NativeProgram(workload_to_codegen_ir(W.rmsnorm({"x": x, "y": x.copy()}), "r").module)
    assert prog.kernel_family("rmsnorm_tile") == "row_program"
    assert prog.kernel_cycles("rmsnorm_tile") == 4 * 2048 + 3 * 16
    a = np.zeros((1, 64, 64), np.float16)
    prog = NativeProgram(workload_to_codegen_ir(W.bgemm({"a": a, "b": a, "c": np.zeros((1, 64, 64), np.float32)}), "g").module)
    # 16x16 tiles (the reference's bgemm example): GEMM family; the host merges neighbouring
    # tasks into MFMA blocks, and without merge candidates the launch is a tile program
    assert prog.kernel_family("gemm_tile") == "gemm"
    src = prog.precompile(0)
    assert "tile program" in src and "gemm program" not in src
    src = prog.precompile(0, merged=True)   # 2x2 tasks: 32x32, still below the MFMA block
    assert "tile program" in src
    a = np.zeros((1, 256, 256), np.uint16)
    prog = NativeProgram(workload_to_codegen_ir(
        W.bgemm({"a": a, "b": a, "c": np.zeros((1, 256, 256), np.float32)}, 128, 128, 64, W.BF16), "g").module)
    assert prog.kernel_family("gemm_tile") == "gemm"
    assert "gemm program" in prog.precompile(0)
    prog = NativeProgram(workload_to_codegen_ir(W.paged_decode(W.paged_decode_arrays([20, 5], 2, 4, 128)), "d").module)
    assert prog.kernel_family("decode_page") == "decode"
    assert prog.kernel_family("normalize") == "row_program"
    assert "decode program" in prog.precompile(0)
    # the same body with one op changed (rowsum -> rowmax) is no longer the decode pattern
    src = workload_to_codegen_ir(W.paged_decode(W.paged_decode_arrays([20, 5], 2, 4, 128)), "d").module
    assert "O RowSum" in src
    prog = NativeProgram(src.replace("O RowSum", "O RowMax"))
    assert prog.kernel_family("decode_page") == "tile_program"


@pytest.mark.parametrize("page, family", [(16, "decode"), (32, "decode"), (64, "decode"), (128, "decode"),
                                          (8, "decode"), (48, "tile_program"), (4, "tile_program")])
def test_decode_family_page_sizes(page, family):
    """Pages of 8, 16, 32, 64 or 128 tokens take the decode family (pages of more than
    16 tokens are folded as 16-token sub-pages: each sub-page's offset is the page's plus
    16 tokens times the token stride; 8-token pages two to a 16-token step, with a
    per-unit step count of ceil(pages / 2)); other sizes stay on the tile program."""
    from pto_wsp._hip import NativeProgram

    arrs = W.paged_decode_arrays([40, 300, 0, 17], 2, 4, 128, page=page)
    prog = NativeProgram(workload_to_codegen_ir(W.rr4(W.paged_decode(arrs)), "d").module)
    assert prog.kernel_family("decode_page") == family
    if family == "decode":
        src = prog.precompile(0)
        assert "decode program" in src
        if page == 8:
            assert "n_[i] = static_cast<int>((npg + 1) / 2);" in src  # step counts in the prefixes
            assert "DecodeWave<4, 128, false, true, true>" in src      # the paired-page template
        else:
            assert f"n_[i] = static_cast<int>(npg) * {page // 16};" in src  # sub-page counts in the prefixes
            assert "DecodeWave<4, 128, false, true, false>" in src
        assert ("vp_ %" in src) == (page > 16)


@pytest.mark.parametrize("group, d, family", [(48, 128, "decode"), (49, 128, "tile_program"), (48, 64, "decode"),
                                           (16, 256, "decode"), (17, 256, "tile_program"), (32, 128, "decode")])
def test_decode_family_query_rows(group, d, family):
    """Up to 48 query rows per KV head at head dims 64 and 128 (blocks of 16 rows that
    share each step's pages), 16 at head dim 256; wider units stay on the tile program."""
    from pto_wsp._hip import NativeProgram

    arrs = W.paged_decode_arrays([40, 300], 1, group, d, page=64)
    prog = NativeProgram(workload_to_codegen_ir(W.rr4(W.paged_decode(arrs)), "d").module)
    assert prog.kernel_family("decode_page") == family
    if family == "decode":
        assert f"DecodeWave<{group}, {d}, false, true, false>" in prog.precompile(0)


@pytest.mark.parametrize("group, d, family, ring", [(4, 128, "decode", 2), (16, 64, "decode", 4), (32, 128, "decode", 2),
                                                 (48, 64, "decode", 2), (49, 64, "tile_program", 0),
                                                 (4, 256, "decode", 2), (17, 256, "tile_program", 0)])
def test_decode_family_f32(group, d, family, ring):
    """f32 q / K / V take the decode family at the bf16 shapes (48 query rows at head dims
    64 and 128, 16 at 256), with 2-step page rings from head dim 128 or beyond 16 rows."""
    from pto_wsp._hip import NativeProgram

    arrs = W.paged_decode_arrays([40, 300], 1, group, d, page=64, f32=True)
    prog = NativeProgram(workload_to_codegen_ir(W.rr4(W.paged_decode(arrs, dtype=W.F32)), "d").module)
    assert prog.kernel_family("decode_page") == family
    if family == "decode":
        src = prog.precompile(0)
        assert f"DecodeWave<{group}, {d}, false, true, false, true>" in src
        assert f"DecodeStream<DW, {ring}, false>" in src


def test_tile_program_matmul_on_matrix_cores():
    """A fused tile with matmuls of MFMA shape (the attention example at 64-token tiles)
    stays a tile program whose matmuls call tile_mma; 8-token tiles keep the scalar loop."""
    from pto_wsp._hip import NativeProgram

    for ts, want in ((64, 2), (8, 0)):
        q = np.zeros((1, 2, 128, 64), np.float32)
        arrs = W.attention_arrays(q, q, q, ts)
        prog = NativeProgram(workload_to_codegen_ir(W.tiled_attention(arrs, ts), "a").module)
        src = prog.precompile(0)
        assert prog.kernel_family("attention_tile") == "tile_program"
        assert src.count("tile_mma<") == want
        if want:
            assert "tile_mma<64, 64, 64, NT>" in src and "mma_scratch_[" in src


def test_tile_program_tiles_beyond_lds_go_to_global_scratch():
    """A fused tile whose tiles exceed the 160 KiB of LDS (256-token attention: 256 x 256
    f32 scores) keeps the largest ones in a per-workgroup global scratch instead of
    failing to compile; 64-token tiles stay in LDS."""
    from pto_wsp._hip import NativeProgram

    for ts, glob in ((256, True), (64, False)):
        q = np.zeros((1, 2, 512, 64), np.float32)
        arrs = W.attention_arrays(q, q, q, ts)
        src = NativeProgram(workload_to_codegen_ir(W.tiled_attention(arrs, ts), "a").module).precompile(0)
        assert ("gtile_" in src) == glob


def test_decode_precompile_folded_normalisation():
    """precompile(decode_norm=True) emits the form a run uses when `out = o / l`
    follows the decode launch: the completion writes out, and units without pages
    are normalised from their accumulators."""
    from pto_wsp._hip import NativeProgram

    arrs = W.paged_decode_arrays([40, 300, 0, 17], 2, 4, 128)
    prog = NativeProgram(workload_to_codegen_ir(W.rr4(W.paged_decode(arrs)), "d").module)
    plain, folded = prog.precompile(0), prog.precompile(0, decode_norm=True)
    assert "norm_ptr" not in plain and "::normalize(" not in plain
    assert "norm_ptr" in folded and "::normalize(" in folded


def _compile_err(w, match):
    with pytest.raises(CompileError, match=match):
        Program(w, "hip_gfx950", {})


def test_unknown_target_is_refused_like_the_reference():
    x = np.zeros((1, 1, 16, 128), np.float32)
    with pytest.raises(CompileError, match="unsupported target: cpu_sim"):
        W.rmsnorm({"x": x, "y": x.copy()}).compile(target="cpu_sim")


def test_ops_without_reference_compute_are_refused():
    X = Tensor(data=None, shape=(2, 4, 4), dtype=DType.F32)
    Y = Tensor(data=None, shape=(2, 4, 4), dtype=DType.F32)

    @kernel
    def k(x: In[Tile[4, 4, DType.F32]], y: Out[Tile[4, 4, DType.F32]]):
        pto.store(y, pto.tanh(x))

    @workload
    def wl():
        for i in P(Dense[2]()):
            k[i](x=X[i], y=Y[i])

    _compile_err(wl(), "no compute")


@pytest.mark.parametrize("op", ["slice_even", "slice_odd", "interleave", "broadcast"])
def test_rope_helpers_trace_then_refuse(op):
    """The reference traces these as tile-shaped Constant ops carrying their operands
    (python/pto_wsp/kernel.py:631-685), which its lowering gives no compute; the trace
    succeeds here with the same shapes and markers, and compiling refuses it."""
    from pto_wsp.kernel import OpKind

    X = Tensor(data=None, shape=(2, 8, 16), dtype=DType.F32)
    Y = Tensor(data=None, shape=(2, 8, 16), dtype=DType.F32)

    @kernel
    def k(x: In[Tile[8, 16, DType.F32]], y: Out[Tile[8, 16, DType.F32]]):
        if op == "slice_even":
            r = pto.interleave(pto.slice_even(x), pto.slice_even(x))
        elif op == "slice_odd":
            r = pto.interleave(pto.slice_odd(x), pto.slice_odd(x))
        elif op == "interleave":
            r = pto.interleave(pto.slice_even(x), pto.slice_odd(x))
        else:
            r = pto.broadcast(pto.rowsum(x), (8, 16))
        pto.store(y, r)

    ir = k.trace()
    consts = [o for o in ir.ops if o.kind == OpKind.Constant]
    assert consts and all(o.result.shape is not None for o in consts)
    if op == "broadcast":
        assert consts[0].result.shape == (8, 16) and consts[0].attrs["broadcast_shape"] == (8, 16)
    else:
        halves = [o for o in consts if "slice_type" in o.attrs]
        assert {o.result.shape for o in halves} == {(8, 8)}
        assert consts[-1].attrs["op_type"] == "interleave" and consts[-1].result.shape == (8, 16)
        assert len(consts[-1].operands) == 2

    @workload
    def wl():
        for i in P(Dense[2]()):
            k[i](x=X[i], y=Y[i])

    _compile_err(wl(), "no compute")


def test_ragged_axis_compiles():
    y = np.zeros((3, 1, 1), np.int32)
    r = Ragged(2, [1, 1])
    Program(W.ragged_mark({"y": y}, r), "hip_gfx950", {})


# (outer, indptr, indices): the reference test's two bindings, repeated and unordered indices,
# an empty row, an empty selection.
_SELECTIONS = [
    (2, [0, 2, 3], [0, 2, 1]),
    (1, [0, 1], [3]),
    (3, [0, 3, 3, 6], [1, 1, 0, 3, 1, 2]),
    (2, [0, 0, 0], []),
]


def test_select_compiles():
    y = np.zeros((4, 1, 1), np.int32)
    sp = Sparse(outer_size=2, indptr=[0, 2, 3], indices=[0, 2, 1])
    src = workload_to_codegen_ir(W.sparse_mark({"y": y}, sp), "s").module
    assert f"outer_{id(sp)}" in src and f"indices_{id(sp)}" in src
    Program(W.sparse_mark({"y": y}, sp), "hip_gfx950", {})


@pytest.mark.parametrize("sel", range(len(_SELECTIONS)))
def test_select_cycle_model_matches_oracle(sel):
    from pto_wsp._hip import NativeProgram

    outer, indptr, indices = _SELECTIONS[sel]
    y = np.zeros((4, 1, 1), np.int32)
    sp = Sparse(outer_size=2, indptr=[0, 2, 3], indices=[0, 2, 1])
    w = W.sparse_mark({"y": y}, sp)
    build = workload_to_codegen_ir(w, "s")
    su, sptr = W.sparse_symbols(sp, outer, indptr, indices)
    got = NativeProgram(build.module).cycle_model(build.tensors, Program._infer_axis_sizes(w), su, sptr)
    ref = run_workload(W.sparse_mark({"y": y}, sp), symbols_u64=su, symbols_ptr=sptr, module_name="s")
    assert (got.total_cycles, got.task_count) == (ref.total_cycles, ref.task_count)
    assert got.task_count == len(indices)
    # the oracle applied the selection: one increment per occurrence of each index
    np.testing.assert_array_equal(y.reshape(4), np.bincount(np.asarray(indices, int), minlength=4))


def test_select_without_bound_symbols_runs_nothing():
    """Unbound symbols read as 0 / null: an empty selection, as in the reference's artifact."""
    from pto_wsp._hip import NativeProgram

    y = np.zeros((4, 1, 1), np.int32)
    sp = Sparse(outer_size=2, indptr=[0, 2, 3], indices=[0, 2, 1])
    w = W.sparse_mark({"y": y}, sp)
    build = workload_to_codegen_ir(w, "s")
    got = NativeProgram(build.module).cycle_model(build.tensors, {}, {}, {})
    assert got.task_count == 0


def test_row_loop_variant_builds_for_gfx950():
    """exp_and_accumulate (launch 1 of the three-phase softmax) as a row program over its
    in-kernel loop: the fixed running max and running sum stay in registers, the x tile is
    loaded and the y tile stored every iteration, the sum is written back after the loop."""
    from pto_wsp._hip import NativeProgram

    lg = np.zeros((1, 32, 512), np.float32)
    prog = NativeProgram(workload_to_codegen_ir(W.rr4(W.softmax3(W.softmax3_arrays(lg))), "s3").module)
    src = prog.precompile(1, row_loops=True)
    assert "row program" in src and "for (i64 it_ = 0; it_ < iters_; ++it_)" in src
    assert "(tb0[u] + io0)" in src and "(tb2[u] + io2)" in src and "io1" not in src and "io3" not in src
    assert "ld4[u] = v8;" in src
