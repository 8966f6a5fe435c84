"""Row programs over in-kernel (P.seq) loops: accumulators read through a Load op
(``pto.load`` / ``ptoisa.tload``) and empty in-kernel extents.

The reference runs every task of a P.seq loop in order, so an InOut tile that a
task loads, updates and stores carries its value from one iteration to the next
(``src/python/pto_codegen.cpp:764-815`` loads the param, ``:931-988`` stores it),
and a loop with no iterations stores nothing (``:2222-2340``, the generated
``for`` runs zero times).  The row program keeps such an accumulator in
registers across the loop; these tests pin that a Load of it sees the value
of the previous iteration and that an empty loop leaves memory untouched.
"""

import numpy as np
import pytest

from oracle.runner import run_workload
from pto_wsp import DType, Dense, DenseDyn, In, InOut, Out, P, Tensor, Tile, kernel, pto, ptoisa, ptoisa_kernel, workload

F32 = DType.F32
R, C = 8, 64


def _accumulate(x, acc, via="pto", nk=None):
    """acc[b] <- acc[b] + x[b, t] for t in P.seq, the accumulator read through a Load op."""
    X = Tensor(data=x, shape=x.shape, dtype=F32)
    A = Tensor(data=acc, shape=acc.shape, dtype=F32)
    nb, nt = x.shape[0], x.shape[1]
    seq = Dense[nt]() if nk is None else DenseDyn(nk)

    if via == "pto":
        @kernel
        def accum(x_t: In[Tile[R, C, F32]], a_t: InOut[Tile[R, C, F32]]):
            pto.store(a_t, pto.add(pto.load(a_t), x_t))
    else:
        @ptoisa_kernel
        def accum(x_t: In[Tile[R, C, F32]], a_t: InOut[Tile[R, C, F32]]):
            ptoisa.tstore(a_t, ptoisa.TADD(ptoisa.tload(a_t), ptoisa.tload(x_t)))

    @workload
    def wl():
        for b in P(Dense[nb]()):
            for t in P.seq(seq, name="t"):
                accum[b, t](x_t=X[b][t], a_t=A[b])

    return wl()


def _overwrite(x, out, nk):
    """out[b] <- 2 * x[b, t] for t in P.seq over a run-time extent: out is stored every
    iteration and never read, so after the loop it holds the last iteration's value."""
    X = Tensor(data=x, shape=x.shape, dtype=F32)
    O = Tensor(data=out, shape=out.shape, dtype=F32)
    nb = x.shape[0]

    @kernel
    def twice(x_t: In[Tile[R, C, F32]], o_t: Out[Tile[R, C, F32]]):
        pto.store(o_t, pto.mul(x_t, pto.constant(2.0, F32)))

    @workload
    def wl():
        for b in P(Dense[nb]()):
            for t in P.seq(DenseDyn(nk), name="t"):
                twice[b, t](x_t=X[b][t], o_t=O[b])

    return wl()


def _inputs(seed, nb=3, nt=5):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((nb, nt, R, C), dtype=np.float32)
    acc = rng.standard_normal((nb, R, C), dtype=np.float32)
    return x, acc


def _sequential_sum(x, acc):
    """((acc + x0) + x1) + ... in float32, the reference's per-iteration rounding."""
    want = acc.copy()
    for t in range(x.shape[1]):
        want = (want + x[:, t]).astype(np.float32)
    return want


# ---------------------------------------------------------------------------
# CPU: the oracle and the emitted row program
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("via", ["pto", "ptoisa"])
def test_oracle_accumulates_through_load(via):
    """The oracle's result is the in-order float32 sum (a stale read of the accumulator
    would give acc + x[:, -1], a dropped initial value sum(x))."""
    x, acc = _inputs(1)
    a = acc.copy()
    run_workload(_accumulate(x, a, via))
    np.testing.assert_array_equal(a, _sequential_sum(x, acc))
    assert not np.array_equal(a, acc + x[:, -1])


def test_oracle_empty_loop_stores_nothing():
    x, _ = _inputs(2)
    out = np.full((x.shape[0], R, C), 7.0, np.float32)
    w = _overwrite(x, out, 0)
    run_workload(w, axis_sizes={"t": 0})
    assert np.all(out == 7.0)


@pytest.mark.parametrize("via", ["pto", "ptoisa"])
def test_row_program_reads_the_accumulator_register(via):
    """The Load result of an accumulator is a copy of its register taken each iteration,
    not a value loaded once before the loop."""
    from pto_wsp._hip import NativeProgram
    from pto_wsp.ir_bridge import workload_to_codegen_ir

    x, acc = _inputs(3)
    prog = NativeProgram(workload_to_codegen_ir(_accumulate(x, acc, via), "rl").module)
    src = prog.precompile(0, row_loops=True)
    assert "row program" in src and "for (i64 it_ = 0; it_ < iters_; ++it_)" in src
    loop = src[src.index("for (i64 it_ = 0; it_ < iters_; ++it_)"):]
    body, after = loop.split("if (iters_ > 0) {", 1)
    # exactly one register holds the accumulator: the one the store updates and the
    # write-back stores
    stored = [ln.split("=")[0].strip() for ln in body.splitlines() if ln.strip().startswith("ld") and "[u] = v" in ln]
    assert len(stored) == 1, body
    reg = stored[0].split("[")[0]
    assert f"= {reg}[u];" in body      # the Load result reads that register inside the loop
    assert f"{reg}[u], A.s4" in after  # and it is what gets written back


def test_row_program_write_back_needs_an_iteration():
    from pto_wsp._hip import NativeProgram
    from pto_wsp.ir_bridge import workload_to_codegen_ir

    x, _ = _inputs(4)
    out = np.zeros((x.shape[0], R, C), np.float32)
    prog = NativeProgram(workload_to_codegen_ir(_overwrite(x, out, 3), "ow").module)
    src = prog.precompile(0, row_loops=True)
    assert "if (iters_ > 0) {" in src
    tail = src[src.index("if (iters_ > 0) {"):]
    assert "row_store" in tail


# ---------------------------------------------------------------------------
# GPU: parity against the oracle
# ---------------------------------------------------------------------------

def _run_hip(w, axis_sizes=None):
    prog = w.compile(target="hip_gfx950")
    if axis_sizes:
        prog.set_axis_sizes(axis_sizes)
    prog.execute()
    prog.synchronize()
    return prog


@pytest.mark.gpu
@pytest.mark.parametrize("via", ["pto", "ptoisa"])
@pytest.mark.parametrize("nt", [1, 5])
def test_accumulator_load_under_p_seq(gpu, via, nt):
    x, acc = _inputs(10 + nt, nt=nt)
    ga, ca = acc.copy(), acc.copy()
    prog = _run_hip(_accumulate(x, ga, via))
    ref = run_workload(_accumulate(x, ca, via))
    np.testing.assert_array_equal(ga, ca)
    np.testing.assert_array_equal(ga, _sequential_sum(x, acc))
    assert prog.stats.total_cycles == ref.total_cycles


@pytest.mark.gpu
@pytest.mark.parametrize("nk", [0, 2])
def test_run_time_extent_overwrite(gpu, nk):
    """An Out accumulator that is never read: with an empty in-kernel extent the output keeps
    its contents; otherwise it holds the last iteration's value."""
    x, _ = _inputs(20, nt=4)
    g = np.full((x.shape[0], R, C), 7.0, np.float32)
    c = g.copy()
    _run_hip(_overwrite(x, g, nk), {"t": nk})
    run_workload(_overwrite(x, c, nk), axis_sizes={"t": nk})
    np.testing.assert_array_equal(g, c)
    if nk == 0:
        assert np.all(g == 7.0)
    else:
        np.testing.assert_array_equal(g, x[:, nk - 1] * np.float32(2.0))


@pytest.mark.gpu
@pytest.mark.parametrize("nk", [0, 3])
def test_accumulator_load_run_time_extent(gpu, nk):
    x, acc = _inputs(30, nt=4)
    ga, ca = acc.copy(), acc.copy()
    _run_hip(_accumulate(x, ga, "pto", nk=4), {"t": nk})
    run_workload(_accumulate(x, ca, "pto", nk=4), axis_sizes={"t": nk})
    np.testing.assert_array_equal(ga, ca)
    np.testing.assert_array_equal(ga, _sequential_sum(x[:, :nk], acc))
