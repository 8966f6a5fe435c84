"""BASELINE.json configurations at full size on the GPU, checked against the
oracle over every element, plus size-independent invariants of the math.

rmsnorm_tile over X[16,8192,16,128] f32 ~ N(0,1)  (1 GiB in)
row softmax over X[8,4096,32,512] f32 ~ N(0,3)    (2 GiB in)
bgemm, A,B[64,2048,2048] bf16 U(-1,1), C fp32, 128x128 tiles, K step 64
paged GQA decode, 64 sequences of 512..8192 tokens, 32/8 heads, d 128

For configs 3 and 4 the oracle runs on a slice (it is single-threaded); the
whole output, every batch and every sequence x KV head, is checked against
float64 references computed on the GPU (the reference's harness compares
whole outputs, examples/_harness/harness.py:19-32), and through invariants
of the math.
"""

import numpy as np
import pytest

import workloads as W
from oracle.runner import run_workload

pytestmark = pytest.mark.gpu


def _close(got, ref, rtol, atol):
    """Elementwise |got-ref| <= atol + rtol*|ref| on the GPU; returns the worst ratio."""
    import torch

    err = (got - ref).abs()
    tol = atol + rtol * ref.abs()
    worst = float((err / tol.clamp_min(1e-38)).max())
    return bool((err <= tol).all()), worst


def _run(kind, shape, sigma, seed):
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * sigma
    y = torch.empty_like(x)
    make = W.rmsnorm if kind == "rmsnorm" else W.softmax
    prog = W.rr4(make({"x": x, "y": y})).compile(target="hip_gfx950")
    prog.execute()
    prog.synchronize()
    xh = x.cpu().numpy()
    yh = np.zeros_like(xh)
    ref = run_workload(W.rr4(make({"x": xh, "y": yh})))
    return x, y, torch.from_numpy(yh).to(dev), prog, ref


def test_config1_rmsnorm_bandwidth_full(gpu):
    import torch

    x, y, yref, prog, ref = _run("rmsnorm", (16, 8192, 16, 128), 1.0, 0)
    ok, worst = _close(y, yref, 1e-5, 1e-6)
    assert ok, f"worst |err|/tol = {worst}"
    assert prog.stats.task_count == ref.task_count == 16 * 8192
    assert prog.stats.total_cycles == ref.total_cycles == 270_008_320
    # Invariant: every output row has mean square 1.
    ms = (y.double() ** 2).mean(dim=-1)
    assert float((ms - 1.0).abs().max()) < 1e-5
    del x, y, yref
    torch.cuda.empty_cache()


def test_config2_softmax_full(gpu):
    import torch

    x, y, yref, prog, ref = _run("softmax", (8, 4096, 32, 512), 3.0, 0)
    ok, worst = _close(y, yref, 1e-5, 0.0)
    assert ok, f"worst |err|/tol = {worst}"
    assert prog.stats.total_cycles == ref.total_cycles
    # Invariants: rows sum to 1; the row maximum maps to 1/rowsum.
    s = y.double().sum(dim=-1)
    assert float((s - 1.0).abs().max()) < 1e-5
    assert float(y.min()) >= 0.0
    del x, y, yref
    torch.cuda.empty_cache()


def test_config3_bgemm_full(gpu):
    import torch

    from test_gpu_parity import _rel_fro  # noqa: F401  (same metric)

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    a = (torch.rand((64, 2048, 2048), generator=g, device=dev) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand((64, 2048, 2048), generator=g, device=dev) * 2 - 1).to(torch.bfloat16)
    c = torch.zeros((64, 2048, 2048), device=dev, dtype=torch.float32)
    prog = W.rr4(W.bgemm({"a": a, "b": b, "c": c}, 128, 128, 64, W.BF16)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    prog.execute()
    prog.synchronize()
    assert prog.stats.task_count == 64 * 16 * 16 * 32
    # Every batch against float64.  Per element, fp32 summation of K = 2048
    # exact bf16 products is within K * 2^-24 * (|A| |B|) of the exact sum in
    # any order; a block skipped, doubled or written to the wrong place misses
    # that bound by orders of magnitude.  Per batch, rel-Frobenius <= 1e-5.
    gamma = 2048 * 2.0 ** -24
    for bi in range(64):
        a64, b64 = a[bi].double(), b[bi].double()
        ref = a64 @ b64
        err = (c[bi].double() - ref).abs()
        bound = gamma * (a64.abs() @ b64.abs())
        assert bool((err <= bound).all()), (bi, float((err / bound.clamp_min(1e-300)).max()))
        rel = float((c[bi].double() - ref).norm() / ref.norm())
        assert rel <= 1e-5, (bi, rel)
        del a64, b64, ref, err, bound
    # Oracle on a slice: batch 0, m-tiles 0-1, all n, all k.
    a0 = a[:1, :256].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    b0 = b[:1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    c0 = np.zeros((1, 256, 2048), np.float32)
    run_workload(W.bgemm({"a": a0, "b": b0, "c": c0}, 128, 128, 64, W.BF16))
    got = c[0, :256].cpu().numpy()
    assert float(np.linalg.norm(got - c0[0]) / np.linalg.norm(c0[0])) <= 1e-5
    del a, b, c
    torch.cuda.empty_cache()


def test_config4_paged_decode_full(gpu):
    import torch

    dev = torch.device("cuda:0")
    t = W.paged_decode_torch(dev, 64, 32, 8, 128, 512, 8192, seed=0)
    prog = W.rr4(W.paged_decode(t)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("decode_page") == "decode"
    prog.execute()
    prog.synchronize()
    lengths = t["lengths"]
    npg = (lengths + 15) // 16
    assert prog.stats.task_count == 8 * int(npg.sum()) + 64 * 8
    out = t["out"]
    # float64 reference on the GPU for every sequence and KV head: rel-Frobenius
    # <= 1e-5 per (sequence, KV head), and every element within 2e-5 of that
    # unit's largest |output| (a page skipped or folded twice moves the unit's
    # softmax weights by far more).
    for b in range(64):
        L, n = int(lengths[b]), int(npg[b])
        pages = t["page_table"][b, :n].long()
        k = t["k_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 16, 128)[:, :L]
        v = t["v_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 16, 128)[:, :L]
        q = t["q"][b].double()                                        # [8, 4, 128]
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) / (128 ** 0.5)
        ref = torch.matmul(torch.softmax(s, dim=-1), v)               # [8, 4, 128]
        got = out[b].double()
        for g in range(8):
            rel = float((got[g] - ref[g]).norm() / ref[g].norm())
            assert rel <= 1e-5, (b, g, rel)
            worst = float((got[g] - ref[g]).abs().max())
            assert worst <= 2e-5 * float(ref[g].abs().max()), (b, g, worst)
        del k, v, s, ref, got
    # Invariants for every sequence: l >= 1 (the max term contributes exp(0)),
    # and each output is a convex combination of that sequence's V rows.
    assert float(t["l"].min()) >= 1.0 - 1e-6
    assert bool(torch.isfinite(out).all())
    assert float(out.abs().max()) <= float(t["v_cache"].float().abs().max()) + 1e-4
    # Oracle on a slice: the first 4 sequences, all KV heads.
    u16 = lambda x: x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    nb = 4
    h = {"q": u16(t["q"][:nb]), "k_cache": u16(t["k_cache"]), "v_cache": u16(t["v_cache"]),
         "page_table": t["page_table"][:nb].cpu().numpy(), "npages": t["npages"][:nb].cpu().numpy(),
         "mask": t["mask"][:nb].cpu().numpy(), "m": np.full((nb, 8, 4, 1), -np.inf, np.float32),
         "l": np.zeros((nb, 8, 4, 1), np.float32), "o": np.zeros((nb, 8, 4, 128), np.float32),
         "out": np.zeros((nb, 8, 4, 128), np.float32)}
    run_workload(W.paged_decode(h))
    got = out[:nb].cpu().numpy()
    np.testing.assert_allclose(got, h["out"], rtol=2e-5, atol=2e-5 * float(np.abs(h["out"]).max()))
    del t
    torch.cuda.empty_cache()


def test_paged_decode_32_token_pages_full(gpu):
    """Config 5's shape with 32-token pages (folded as two 16-token sub-pages by the
    decode family): every sequence and KV head against float64 attention."""
    import torch

    dev = torch.device("cuda:0")
    t = W.paged_decode_torch(dev, 64, 32, 8, 128, 512, 8192, seed=1, page=32)
    prog = W.rr4(W.paged_decode(t)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("decode_page") == "decode"
    prog.execute()
    prog.synchronize()
    lengths = t["lengths"]
    npg = (lengths + 31) // 32
    assert prog.stats.task_count == 8 * int(npg.sum()) + 64 * 8
    out = t["out"]
    for b in range(64):
        L, n = int(lengths[b]), int(npg[b])
        pages = t["page_table"][b, :n].long()
        k = t["k_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 32, 128)[:, :L]
        v = t["v_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 32, 128)[:, :L]
        q = t["q"][b].double()
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) / (128 ** 0.5)
        ref = torch.matmul(torch.softmax(s, dim=-1), v)
        got = out[b].double()
        for g in range(8):
            rel = float((got[g] - ref[g]).norm() / ref[g].norm())
            assert rel <= 1e-5, (b, g, rel)
        del k, v, s, ref, got
    del t
    torch.cuda.empty_cache()


def test_config3_bgemm_f32_full(gpu):
    """The C4 shape with f32 A and B (the f32 MFMA block): every batch against float64,
    per element within K * 2^-24 * (|A| |B|) and per batch at rel-Frobenius 1e-5."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    a = torch.rand((64, 2048, 2048), generator=g, device=dev) * 2 - 1
    b = torch.rand((64, 2048, 2048), generator=g, device=dev) * 2 - 1
    c = torch.zeros((64, 2048, 2048), device=dev, dtype=torch.float32)
    prog = W.rr4(W.bgemm({"a": a, "b": b, "c": c}, 128, 128, 64, W.F32)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("gemm_tile") == "gemm"
    prog.execute()
    prog.synchronize()
    gamma = 2048 * 2.0 ** -24
    for bi in range(64):
        a64, b64 = a[bi].double(), b[bi].double()
        ref = a64 @ b64
        err = (c[bi].double() - ref).abs()
        bound = gamma * (a64.abs() @ b64.abs())
        assert bool((err <= bound).all()), (bi, float((err / bound.clamp_min(1e-300)).max()))
        assert float((c[bi].double() - ref).norm() / ref.norm()) <= 1e-5, bi
        del a64, b64, ref, err, bound
    # Oracle on a slice: batch 0, m-tiles 0-1, all n, all k.
    c0 = np.zeros((1, 256, 2048), np.float32)
    run_workload(W.bgemm({"a": a[:1, :256].cpu().numpy(), "b": b[:1].cpu().numpy(), "c": c0}, 128, 128, 64, W.F32))
    got = c[0, :256].cpu().numpy()
    assert float(np.linalg.norm(got - c0[0]) / np.linalg.norm(c0[0])) <= 1e-5
    del a, b, c
    torch.cuda.empty_cache()


def test_config4_paged_decode_f32_full(gpu):
    """The C5 shape with f32 q / K / V: every sequence and KV head against float64
    attention, rel-Frobenius <= 1e-5 per (sequence, KV head)."""
    import torch

    dev = torch.device("cuda:0")
    t = W.paged_decode_torch(dev, 64, 32, 8, 128, 512, 8192, seed=2, f32=True)
    prog = W.rr4(W.paged_decode(t, dtype=W.F32)).compile(target="hip_gfx950")
    assert prog._native.kernel_family("decode_page") == "decode"
    prog.execute()
    prog.synchronize()
    lengths, out = t["lengths"], t["out"]
    npg = (lengths + 15) // 16
    for b in range(64):
        L, n = int(lengths[b]), int(npg[b])
        pages = t["page_table"][b, :n].long()
        k = t["k_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 16, 128)[:, :L]
        v = t["v_cache"][pages].double().permute(1, 0, 2, 3).reshape(8, n * 16, 128)[:, :L]
        s = torch.matmul(t["q"][b].double(), k.transpose(1, 2).contiguous()) / (128 ** 0.5)
        ref = torch.matmul(torch.softmax(s, dim=-1), v)
        got = out[b].double()
        for g in range(8):
            assert float((got[g] - ref[g]).norm() / ref[g].norm()) <= 1e-5, (b, g)
        del k, v, s, ref, got
    del t
    torch.cuda.empty_cache()
