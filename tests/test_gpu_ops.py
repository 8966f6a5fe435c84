"""GPU parity for the store cast and the op variants of the arithmetic contract.

Each case runs the same seeded workload on the HIP target and on the CPU
oracle (whose results tests/test_oracle_ops.py pins bit for bit against
float64 arithmetic and numpy's float16 cast) and requires identical bits:
every op here is one correctly rounded fp32 operation or an exact min / max,
and the casts round to nearest even.  These kernels run as row programs (the
F16 / BF16 outputs through row_store_h); the rounding probe also runs through
the tile program's cast (tile_store_f).
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu

F32, F16, BF16 = W.F32, W.F16, W.BF16
NP_OUT = {F32: np.float32, F16: np.float16, BF16: np.uint16}


def _hip(w):
    prog = w.compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    return prog


def _pair(make, arrs):
    """Runs make(arrs) on the GPU (host arrays, staged through HBM) and on the oracle."""
    ga = {k: v.copy() for k, v in arrs.items()}
    ca = {k: v.copy() for k, v in arrs.items()}
    prog = _hip(W.rr4(make(ga)))
    ref = run_workload(W.rr4(make(ca)))
    assert prog.stats.total_cycles == ref.total_cycles
    return ga, ca


CASES = [(op, "same") for op in W.BIN_OPS] + [(op, m) for op in W.BIN_OPS for m in ("row", "row_t")] + \
        [(op, m) for op in ("sub", "mul", "div") for m in ("col", "col_t")]


@pytest.mark.parametrize("out_dtype", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("op,mode", CASES)
def test_binary_variant(gpu, op, mode, out_dtype):
    R, C = 16, 64
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, R, C)).astype(np.float32)
    y = rng.standard_normal((2, 3) + W.BIN_SHAPES[mode](R, C)).astype(np.float32)
    y[np.abs(y) < 1e-3] = 0.5
    arrs = {"x": x, "y": y, "out": np.zeros(x.shape, NP_OUT[out_dtype])}
    ga, ca = _pair(lambda a: W.binary(a, op, out_dtype), arrs)
    np.testing.assert_array_equal(ga["out"].view(np.uint8), ca["out"].view(np.uint8))


@pytest.mark.parametrize("out_dtype", [F32, F16, BF16], ids=["f32", "f16", "bf16"])
@pytest.mark.parametrize("op", list(W.BIN_OPS))
def test_scalar_right_variant(gpu, op, out_dtype):
    x = np.random.default_rng(6).standard_normal((2, 2, 8, 64)).astype(np.float32)
    arrs = {"x": x, "out": np.zeros(x.shape, NP_OUT[out_dtype])}
    ga, ca = _pair(lambda a: W.scalar_binary(a, op, -2.5, out_dtype=out_dtype), arrs)
    np.testing.assert_array_equal(ga["out"].view(np.uint8), ca["out"].view(np.uint8))


@pytest.mark.parametrize("out_dtype", [F32, F16], ids=["f32", "f16"])
@pytest.mark.parametrize("op", ["add", "mul", "div", "max", "min"])
def test_scalar_left_variant(gpu, op, out_dtype):
    x = np.random.default_rng(7).standard_normal((1, 3, 8, 32)).astype(np.float32)
    x[np.abs(x) < 1e-3] = 0.25
    arrs = {"x": x, "out": np.zeros(x.shape, NP_OUT[out_dtype])}
    ga, ca = _pair(lambda a: W.scalar_binary(a, op, 1.5, left=True, out_dtype=out_dtype), arrs)
    np.testing.assert_array_equal(ga["out"].view(np.uint8), ca["out"].view(np.uint8))


@pytest.mark.parametrize("family", ["row", "tile"])
@pytest.mark.parametrize("out_dtype", [F16, BF16], ids=["f16", "bf16"])
def test_store_cast_rounding_probe(gpu, out_dtype, family):
    vals = W.rounding_probe_f32(6000, seed=13, for_bf16=out_dtype == BF16)
    R, C = 16, 32
    reps = -(-len(vals) // (R * C))
    x = np.resize(vals, reps * R * C).astype(np.float32).reshape(1, reps, R, C)
    arrs = {"x": x, "out": np.zeros(x.shape, NP_OUT[out_dtype])}
    ga, ca = _pair(lambda a: W.store_cast(a, out_dtype, via_tile=family == "tile"), arrs)
    np.testing.assert_array_equal(ga["out"].view(np.uint16), ca["out"].view(np.uint16))
    if out_dtype == F16:
        with np.errstate(over="ignore"):
            np.testing.assert_array_equal(ga["out"].view(np.uint16), x.astype(np.float16).view(np.uint16))
    else:
        np.testing.assert_array_equal(ga["out"], W.bf16_rne_by_distance(x.reshape(-1)).reshape(x.shape))


def test_store_cast_device_tensors(gpu):
    """The same cast with the output as a ROCm torch tensor (bf16 storage)."""
    import torch

    x = np.random.default_rng(14).standard_normal((2, 4, 16, 128)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)
    od = torch.zeros(x.shape, dtype=torch.bfloat16, device=gpu)
    _hip(W.rr4(W.store_cast({"x": xd, "out": od}, BF16)))
    got = od.view(torch.int16).cpu().numpy().view(np.uint16)
    np.testing.assert_array_equal(got, W.bf16_rne_by_distance(x.reshape(-1)).reshape(x.shape))
