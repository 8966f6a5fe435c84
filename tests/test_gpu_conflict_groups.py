"""GPU parity for launches whose grid tasks write overlapping memory.

The HIP backend runs them as parallel groups of tasks that write disjoint
memory, each group in program order (one group when nothing finer is
provably disjoint).  Results must equal the oracle's, which runs every task
in program order: bit for bit for the float32 accumulations, and at rtol 1e-5
for the three-phase softmax example (exp).
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from test_conflict_groups import _arrays

pytestmark = pytest.mark.gpu


def _hip(w):
    prog = w.compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    return prog


@pytest.mark.parametrize("shape", [(2, 5, 3, 4, 16), (4, 9, 16, 8, 64)])
def test_groups_sum_in_program_order(gpu, shape):
    ga, ca = _arrays(shape, 3), _arrays(shape, 3)
    want = W.conflict_accumulate_ref(ga["x"], ga["out"])
    prog = _hip(W.rr4(W.conflict_accumulate(ga)))
    ref = run_workload(W.rr4(W.conflict_accumulate(ca)))
    np.testing.assert_array_equal(ga["out"], want)
    np.testing.assert_array_equal(ga["out"], ca["out"])
    assert prog.stats.total_cycles == ref.total_cycles


def test_one_shared_tile_runs_in_order(gpu):
    ga, ca = _arrays((2, 3, 4, 4, 16), 4), _arrays((2, 3, 4, 4, 16), 4)
    want = W.conflict_accumulate_ref(ga["x"], ga["out"], shared_all=True)
    _hip(W.rr4(W.conflict_accumulate(ga, shared_all=True)))
    run_workload(W.rr4(W.conflict_accumulate(ca, shared_all=True)))
    np.testing.assert_array_equal(ga["out"], want)
    np.testing.assert_array_equal(ga["out"], ca["out"])


def test_softmax_three_phase_overlapping_views(gpu):
    """examples/softmax with V = 256: neighbouring v tiles overlap, so the rescale launch
    divides shared rows twice, in program order within each (b, s) group."""
    lg = (0.1 * np.random.default_rng(6).standard_normal((2, 256, 256))).astype(np.float32)
    ga, ca = W.softmax3_arrays(lg), W.softmax3_arrays(lg)
    prog = _hip(W.rr4(W.softmax3(ga)))
    ref = run_workload(W.rr4(W.softmax3(ca)))
    np.testing.assert_allclose(ga["probs"], ca["probs"], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(ga["rsum"], ca["rsum"], rtol=1e-5, atol=0)
    np.testing.assert_array_equal(ga["rmax"], ca["rmax"])
    assert prog.stats.total_cycles == ref.total_cycles
