"""Random paged-decode launches against the oracle.

Each seed draws the query rows per KV head (1..16, or 17..48 at head dim 64
and 128 for a fifth of the seeds), the head dim (64, 128, 256), the KV
heads, 1..24 sequences whose lengths mix empty, sub-page, exact-page and
multi-thousand-token sequences, the page size (8, 16, 32, 64: the streaming
decode family, which folds pages of more than 16 tokens as 16-token
sub-pages and 8-token pages two to a 16-token step), the mask, and the
input dtype (bf16 / f16, or f32 for a fifth of the seeds).  The GPU
accumulators and output must equal the oracle's within rtol 2e-5 (with an
atol of 2e-5 of each tensor's largest magnitude: both fold the pages in fp32, split differently), sequences with
pages must match float64 attention over their valid tokens when masked (and
the mask is read as a column broadcast), and the cycle counts must be equal.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu


def _case(seed):
    rng = np.random.default_rng(seed)
    group, d = int(rng.integers(1, 17)), int(rng.choice([64, 128, 256]))
    if d < 256 and rng.random() < 0.2:
        group = int(rng.integers(17, 49))  # 2 or 3 blocks of 16 query rows
    page = int(rng.choice([8, 16, 16, 16, 32, 32, 64]))
    n = int(rng.integers(1, 25))
    kinds = rng.integers(0, 4, n)
    lengths = [0 if k == 0 else int(rng.integers(1, page + 1)) if k == 1 else page * int(rng.integers(1, 9)) if k == 2
               else int(rng.integers(page + 1, 3000)) for k in kinds]
    if max(lengths) == 0:
        lengths[0] = 5
    c = dict(lengths=lengths, hkv=int(rng.integers(1, 5)), group=group, d=d, page=page,
             masked=bool(rng.random() < 0.8), f16=bool(rng.random() < 0.3))
    # f32 q / K / V for about a fifth of the seeds
    c["f32"] = bool(rng.random() < 0.2)
    return c


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_matches_oracle(gpu, seed):
    c = _case(seed)
    print(c, flush=True)
    ga = W.paged_decode_arrays(c["lengths"], c["hkv"], c["group"], c["d"], page=c["page"], seed=seed, f16=c["f16"],
                               f32=c["f32"])
    ca = {k: v.copy() for k, v in ga.items()}
    dt = W.F32 if c["f32"] else W.F16 if c["f16"] else W.BF16
    prog = W.paged_decode(ga, masked=c["masked"], dtype=dt).compile(target="hip_gfx950")
    # (a [1, page] mask with as many query rows as page tokens is a row broadcast, see
    # below: the decode template takes it for 16 rows and 16-token pages)
    want_family = "tile_program" if c["masked"] and c["group"] == c["page"] != 16 else "decode"
    assert prog._native.kernel_family("decode_page") == want_family
    prog.execute()
    prog.synchronize()
    ref = run_workload(W.paged_decode(ca, masked=c["masked"], dtype=dt))
    assert prog.stats.total_cycles == ref.total_cycles and prog.stats.task_count == ref.task_count
    for k in ("m", "l", "o", "out"):
        fin = np.isfinite(ca[k])
        assert np.array_equal(fin, np.isfinite(ga[k])), k
        scale = float(np.abs(ca[k][fin]).max()) if fin.any() else 1.0
        np.testing.assert_allclose(ga[k][fin], ca[k][fin], rtol=2e-5, atol=2e-5 * scale, err_msg=k)
    live = np.asarray(c["lengths"]) > 0
    # With as many query rows as page tokens the [1, page] mask tile also fits the
    # [group, page] scores as a row broadcast, which the reference's emitter tries
    # first (src/python/pto_codegen.cpp:1094-1099): the kernel then is no longer
    # token masking, and only the oracle comparison above applies.
    if c["masked"] and c["group"] != c["page"]:
        got, want = ga["out"][live], W.paged_decode_ref(ga)[live]
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-5
