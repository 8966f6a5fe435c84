"""Random kernels (tests/fuzz_programs.py) on the HIP target against the oracle.

Each seed builds one random program (ops, tile shape, layouts, grid or
P.seq accumulation), runs it on the GPU and on the oracle over the same
seeded host arrays, and requires equal cycle counts and a GPU result as
close to the float64 referee as the oracle's (within 4x and a floor of 1e-5
of the result's scale for f32, one f16 / bf16 rounding step for the cast
outputs).  The programs land on the row program (with and without in-kernel
loops) and on the tile program.
"""

import pytest

import fuzz_programs as FP
import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu

SEEDS = range(0, 80)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_program_matches_oracle(gpu, seed):
    prog = FP.generate(seed)
    print(prog.describe(), flush=True)
    arrs = FP.arrays(prog)
    ga = {k: v.copy() for k, v in arrs.items()}
    ca = {k: v.copy() for k, v in arrs.items()}
    p = W.rr4(FP.make_workload(prog, ga)).compile(target="hip_gfx950")
    p.execute()
    p.synchronize()
    ref = run_workload(W.rr4(FP.make_workload(prog, ca)))
    assert p.stats.total_cycles == ref.total_cycles
    bad = FP.compare(prog, ga, ca, FP.evaluate(prog, arrs))
    assert not bad, "\n".join(bad)
