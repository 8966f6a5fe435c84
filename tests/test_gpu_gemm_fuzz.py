"""Random MFMA GEMM launches against the oracle.

Each seed draws a task tile (tm, tn in {64, 128, 256}, tk in {16, 32, 64,
128}, within the LDS budget of the GEMM family), a batch, tile counts along
M, N and K (odd counts leave the 2x2 block merge half used or off), the
input dtype (f16 / bf16, or f32 for about a third of the seeds: the f32
block on v_mfma_f32_32x32x2_f32), the InOut accumulate form or the plain store, the
order of the m and n loops, and seeded inputs with a random initial C (a
second set of seeds draws tiles of 16 / 32, merged into MFMA blocks or run
as tile programs, and of 512, split into 256-wide blocks, with K steps up to
256).  The
GPU result must equal the oracle's within a relative Frobenius error of 1e-5
(both accumulate exact products in fp32, in different orders), with equal
cycle counts.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload
from pto_wsp import Dense, In, InOut, Out, P, Tile, kernel, pto, workload

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(seed)
    while True:
        tm, tn = int(rng.choice([64, 128, 256])), int(rng.choice([64, 128, 256]))
        tk = int(rng.choice([16, 32, 64, 128]))
        if 2 * (tm + tn) * tk * 2 <= 160 * 1024:
            break
    c = dict(tm=tm, tn=tn, tk=tk, B=int(rng.integers(1, 3)), mt=int(rng.integers(1, 5)), nt=int(rng.integers(1, 5)),
             kt=int(rng.integers(1, 6)), f16=bool(rng.random() < 0.5), plain=bool(rng.random() < 0.25),
             n_outer=bool(rng.random() < 0.3))
    c["f32"] = bool(rng.random() < 0.35)
    return c


def _workload(c, arrs):
    tm, tn, tk = c["tm"], c["tn"], c["tk"]
    dt = W.F32 if c["f32"] else W.F16 if c["f16"] else W.BF16
    a, b_, cc = arrs["a"], arrs["b"], arrs["c"]
    B, M, K = a.shape
    N = b_.shape[2]
    A = W.T(a.reshape(B, M // tm, tm, K // tk, tk).transpose(0, 1, 3, 2, 4), dt)
    Bm = W.T(b_.reshape(B, K // tk, tk, N // tn, tn).transpose(0, 3, 1, 2, 4), dt)
    C = W.T(cc.reshape(B, M // tm, tm, N // tn, tn).transpose(0, 1, 3, 2, 4))
    if c["plain"]:
        @kernel
        def gemm_tile(a_tile: In[Tile[tm, tk, dt]], b_tile: In[Tile[tk, tn, dt]], c_tile: Out[Tile[tm, tn, W.F32]]):
            pto.store(c_tile, pto.matmul(a_tile, b_tile))
    else:
        @kernel
        def gemm_tile(a_tile: In[Tile[tm, tk, dt]], b_tile: In[Tile[tk, tn, dt]], c_tile: InOut[Tile[tm, tn, W.F32]]):
            pto.store(c_tile, pto.add(c_tile, pto.matmul(a_tile, b_tile)))

    bb, mm, nn, kk = Dense[B](), Dense[M // tm](), Dense[N // tn](), Dense[K // tk]()

    @workload
    def gemm_wl():
        for b in P(bb):
            for x in P(nn if c["n_outer"] else mm):
                for y in P(mm if c["n_outer"] else nn):
                    m, n = (y, x) if c["n_outer"] else (x, y)
                    for k in P.seq(kk):
                        gemm_tile[b, m, n, k](a_tile=A[b][m][k], b_tile=Bm[b][n][k], c_tile=C[b][m][n])

    return gemm_wl()


@pytest.mark.parametrize("seed", range(24))
def test_random_gemm_matches_oracle(gpu, seed):
    c = _case(seed)
    print(c, flush=True)
    rng = np.random.default_rng(seed + 77)
    M, N, K = c["tm"] * c["mt"], c["tn"] * c["nt"], c["tk"] * c["kt"]
    a = rng.uniform(-1, 1, (c["B"], M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (c["B"], K, N)).astype(np.float32)
    if c["f32"]:
        a16, b16 = a, b
    elif c["f16"]:
        a16, b16 = a.astype(np.float16), b.astype(np.float16)
    else:
        a16, b16 = W.bf16_round(a), W.bf16_round(b)
    c0 = rng.uniform(-1, 1, (c["B"], M, N)).astype(np.float32)
    ga = {"a": a16.copy(), "b": b16.copy(), "c": c0.copy()}
    ca = {"a": a16.copy(), "b": b16.copy(), "c": c0.copy()}
    prog = W.rr4(_workload(c, ga)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    prog.execute()
    prog.synchronize()
    ref = run_workload(W.rr4(_workload(c, ca)))
    assert prog.stats.total_cycles == ref.total_cycles
    err = np.linalg.norm(ga["c"] - ca["c"]) / np.linalg.norm(ca["c"])
    assert err <= 1e-5, err


def _case_tiles(seed):
    """Task tiles below and above the MFMA block: 16 / 32 (merged into blocks, or the
    tile program when the extents do not merge to 64) and 512 (split into 256-wide
    blocks), with K steps up to 256 (taken in LDS stages)."""
    rng = np.random.default_rng(1000 + seed)
    tm, tn = int(rng.choice([16, 32, 64, 512])), int(rng.choice([16, 32, 128, 512]))
    tk = int(rng.choice([16, 32, 64, 256]))
    small = lambda t: int(rng.integers(1, 9)) if t <= 32 else (int(rng.integers(1, 3)) if t == 512 else int(rng.integers(1, 4)))
    c = dict(tm=tm, tn=tn, tk=tk, B=1, mt=small(tm), nt=small(tn), kt=int(rng.integers(1, 4)), f16=bool(rng.random() < 0.5),
             plain=bool(rng.random() < 0.25), n_outer=bool(rng.random() < 0.3))
    c["f32"] = bool(rng.random() < 0.3)
    return c


@pytest.mark.parametrize("seed", range(12))
def test_random_gemm_tile_sizes_match_oracle(gpu, seed):
    c = _case_tiles(seed)
    print(c, flush=True)
    rng = np.random.default_rng(seed + 99)
    M, N, K = c["tm"] * c["mt"], c["tn"] * c["nt"], c["tk"] * c["kt"]
    a = rng.uniform(-1, 1, (c["B"], M, K)).astype(np.float32)
    b = rng.uniform(-1, 1, (c["B"], K, N)).astype(np.float32)
    if c["f32"]:
        a16, b16 = a, b
    elif c["f16"]:
        a16, b16 = a.astype(np.float16), b.astype(np.float16)
    else:
        a16, b16 = W.bf16_round(a), W.bf16_round(b)
    c0 = rng.uniform(-1, 1, (c["B"], M, N)).astype(np.float32)
    ga = {"a": a16.copy(), "b": b16.copy(), "c": c0.copy()}
    ca = {"a": a16.copy(), "b": b16.copy(), "c": c0.copy()}
    prog = W.rr4(_workload(c, ga)).compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    ref = run_workload(W.rr4(_workload(c, ca)))
    assert prog.stats.total_cycles == ref.total_cycles
    err = np.linalg.norm(ga["c"] - ca["c"]) / np.linalg.norm(ca["c"])
    assert err <= 1e-5, err
