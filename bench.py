#!/usr/bin/env python3
"""Benchmark of the PTO-WSP data-parallel tile path on one MI355X.

Headline workload: the README rmsnorm tile kernel
over X[16, 8192, 16, 128] fp32 ~ N(0,1) (1 GiB in, 1 GiB out), workload
P(batch=16) x P(tiles=8192), schedule round_robin(4) + TaskWindow(8192,
STALL), compiled with ``compile(target="hip_gfx950")``.  A step is one
``execute()`` + ``synchronize()`` of the compiled program over device-resident
buffers; K steps are timed between ``torch.cuda.synchronize()`` calls.

``configs`` reports every BASELINE config this build runs (GB/s or TFLOP/s
and the fraction of the MI355X peak, from HIP-event kernel time), and
``cpu_baseline`` times this repository's C restatement of the reference
cpu_sim artifact (oracle/, 1 thread) on the same inputs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME|all] [--no-cpu] [--warm-s S]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "pto-wsp_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
F32_PEAK_TFLOPS = 157.3        # MI355X dense fp32 MFMA
METRIC = "GB/s & TFLOP/s as % of MI355X roofline per config, 1 GPU, vs cpu_sim wall"
HEADLINE = "rmsnorm_bw"


def rr4(w):
    from pto_wsp import DispatchPolicy, TaskWindow, WindowMode

    return (w.dispatch(DispatchPolicy.round_robin(num_aicpus=4))
            .task_graph(window=TaskWindow(8192, "tasks", WindowMode.STALL)))


def row_workload(kind, X, Y):
    """rmsnorm / softmax / copy tile kernels over X[B, T, R, C] (rows of R x C tiles)."""
    from pto_wsp import DType, Dense, In, Out, P, Tensor, Tile, kernel, pto, workload

    f32 = DType.F32
    B, NT, R, C = tuple(X.shape)
    Xt = Tensor(data=X, shape=tuple(X.shape), dtype=f32)
    Yt = Tensor(data=Y, shape=tuple(Y.shape), dtype=f32)
    if kind == "rmsnorm":
        @kernel
        def rmsnorm_tile(x: In[Tile[R, C, f32]], out: Out[Tile[R, C, f32]]):
            sq = pto.mul(x, x)
            mean_sq = pto.rowmean(sq)
            inv = pto.rsqrt(mean_sq)
            pto.store(out, pto.mul(x, inv))

        body = rmsnorm_tile
    elif kind == "softmax":
        @kernel
        def softmax_tile(x: In[Tile[R, C, f32]], out: Out[Tile[R, C, f32]]):
            m = pto.rowmax(x)
            e = pto.exp(pto.sub(x, m))
            pto.store(out, pto.div(e, pto.rowsum(e)))

        body = softmax_tile
    else:
        @kernel
        def copy_tile(x: In[Tile[R, C, f32]], out: Out[Tile[R, C, f32]]):
            pto.store(out, x)

        body = copy_tile

    batch, tiles = Dense[B](), Dense[NT]()

    @workload
    def wl():
        for b in P(batch):
            for t in P(tiles):
                body[b, t](x=Xt[b][t], out=Yt[b][t])

    return rr4(wl())


def bgemm_workload(A, Bm, C, tm=128, tn=128, tk=64, f32_inputs=False, f16_inputs=False):
    """examples/bgemm pattern: C[b] += A[b] @ B[b] with a P.seq K loop and an InOut fp32 tile
    (bf16 A / B, or f32 / f16 with f32_inputs / f16_inputs)."""
    from pto_wsp import DType, Dense, In, InOut, P, Tensor, Tile, kernel, pto, workload

    bf16 = DType.F32 if f32_inputs else DType.F16 if f16_inputs else DType.BF16  # A / B dtype
    f32 = DType.F32
    nb, M, K = tuple(A.shape)
    N = Bm.shape[2]

    def tiles(x, r, c, rt, ct):  # x[b, R, Cc] -> [b, R/rt, Cc/ct, rt, ct] view, either library
        v = x.reshape(nb, r // rt, rt, c // ct, ct)
        return v.permute(0, 1, 3, 2, 4) if hasattr(v, "permute") else v.transpose(0, 1, 3, 2, 4)

    at = tiles(A, M, K, tm, tk)
    bt = tiles(Bm, K, N, tk, tn)
    bt = bt.permute(0, 2, 1, 3, 4) if hasattr(bt, "permute") else bt.transpose(0, 2, 1, 3, 4)
    ct = tiles(C, M, N, tm, tn)
    At = Tensor(data=at, shape=tuple(at.shape), dtype=bf16)
    Bt = Tensor(data=bt, shape=tuple(bt.shape), dtype=bf16)
    Ct = Tensor(data=ct, shape=tuple(ct.shape), dtype=f32)

    @kernel
    def gemm_tile(a_tile: In[Tile[tm, tk, bf16]], b_tile: In[Tile[tk, tn, bf16]], c_tile: InOut[Tile[tm, tn, f32]]):
        acc = pto.matmul(a_tile, b_tile)
        pto.store(c_tile, pto.add(c_tile, acc))

    batch, mt, nt, kt = Dense[nb](), Dense[M // tm](), Dense[N // tn](), Dense[K // tk]()

    @workload
    def bgemm():
        for b in P(batch):
            for m in P(mt):
                for n in P(nt):
                    for k in P.seq(kt):
                        gemm_tile[b, m, n, k](a_tile=At[b][m][k], b_tile=Bt[b][n][k], c_tile=Ct[b][m][n])

    return rr4(bgemm())


def decode_workload(t, page=16):
    """flashinfer_decode over a paged KV cache: for each sequence b and
    KV head g, P.seq over the sequence's pages folds one 16-token page into running
    (m, l, o) for the 4 query heads of the group (online softmax); a second launch
    writes out = o / l.  The page count of sequence b is npages[b] (a tensor-bound
    DenseDyn, declared maximum 512 pages), the page comes from the page table, and
    padding tokens of the last page are masked by a 0 / 1e30 penalty row."""
    import math

    from pto_wsp import DType, Dense, DenseDyn, In, InOut, Out, P, Tensor, Tile, kernel, pto, workload

    f32, i32 = DType.F32, DType.I32
    bf16 = DType.F32 if str(t["q"].dtype) in ("torch.float32", "float32") else DType.BF16  # q / K / V dtype
    B, Hkv, G, D = tuple(t["q"].shape)
    max_pages = t["page_table"].shape[1]
    sc = 1.0 / math.sqrt(D)

    def T(x, dt):
        return Tensor(data=x, shape=tuple(x.shape), dtype=dt)

    kt = t["k_cache"].permute(0, 1, 3, 2) if hasattr(t["k_cache"], "permute") else t["k_cache"].transpose(0, 1, 3, 2)
    Q, KT, V = T(t["q"], bf16), T(kt, bf16), T(t["v_cache"], bf16)
    PT, NP, MASK = T(t["page_table"], i32), T(t["npages"], i32), T(t["mask"], f32)
    M, L, O, OUT = T(t["m"], f32), T(t["l"], f32), T(t["o"], f32), T(t["out"], f32)

    @kernel
    def decode_page(q: In[Tile[G, D, bf16]], k_t: In[Tile[D, page, bf16]], v: In[Tile[page, D, bf16]],
                    mask: In[Tile[1, page, f32]], m_acc: InOut[Tile[G, 1, f32]], l_acc: InOut[Tile[G, 1, f32]],
                    o_acc: InOut[Tile[G, D, f32]]):
        s = pto.sub(pto.mul(pto.matmul(q, k_t), pto.constant(sc, f32)), mask)
        m_new = pto.max(m_acc, pto.rowmax(s))
        p = pto.exp(pto.sub(s, m_new))
        alpha = pto.exp(pto.sub(m_acc, m_new))
        pto.store(l_acc, pto.add(pto.mul(l_acc, alpha), pto.rowsum(p)))
        pto.store(o_acc, pto.add(pto.mul(o_acc, alpha), pto.matmul(p, v)))
        pto.store(m_acc, m_new)

    @kernel
    def normalize(o_acc: In[Tile[G, D, f32]], l_acc: In[Tile[G, 1, f32]], out: Out[Tile[G, D, f32]]):
        pto.store(out, pto.div(o_acc, l_acc))

    @workload
    def paged_decode():
        for b in P(Dense[B]()):
            for g in P(Dense[Hkv]()):
                for pg in P.seq(DenseDyn(max_pages, extent=NP[b]), name="pg"):
                    decode_page[b, g, pg](q=Q[b][g], k_t=KT[PT[b][pg]][g], v=V[PT[b][pg]][g], mask=MASK[b][pg],
                                          m_acc=M[b][g], l_acc=L[b][g], o_acc=O[b][g])
        for b in P(Dense[B]()):
            for g in P(Dense[Hkv]()):
                normalize[b, g](o_acc=O[b][g], l_acc=L[b][g], out=OUT[b][g])

    return rr4(paged_decode())


def softmax3_workload(lg, pr, rmax, rsum):
    """examples/softmax/pto_wsp_impl.py:52-105 as written: logits [B,S,V] viewed as
    [B, S/8, 8, V/64, 64], three launches (running max and exp + running sum with P.seq
    accumulators over v, then an in-place rescale over P(v)).  Each [8,64] tile view
    L[b][s][v] starts at row-block v of seq tile s; with V = 512 (8 vocab tiles) the views
    of a launch are disjoint, with V < 512 neighbouring v overlap."""
    from pto_wsp import DType, Dense, In, InOut, Out, P, Tensor, Tile, kernel, pto, workload

    f32 = DType.F32
    B, S, V = tuple(lg.shape)
    tr, tc = 8, 64
    st, vt = S // tr, V // tc

    def T(x, shape):
        v = x.reshape(shape)  # a view of the same memory (numpy or torch, contiguous)
        return Tensor(data=v, shape=shape, dtype=f32)

    L = T(lg, (B, st, tr, vt, tc))
    PR = T(pr, (B, st, tr, vt, tc))
    RM, RS = T(rmax, tuple(rmax.shape)), T(rsum, tuple(rsum.shape))

    @kernel
    def update_rowmax(x_tile: In[Tile[tr, tc, f32]], m_acc: InOut[Tile[tr, 1, f32]]):
        pto.store(m_acc, pto.max(m_acc, pto.rowmax(x_tile)))

    @kernel
    def exp_and_accumulate(x_tile: In[Tile[tr, tc, f32]], m_tile: In[Tile[tr, 1, f32]],
                           y_tile: Out[Tile[tr, tc, f32]], l_acc: InOut[Tile[tr, 1, f32]]):
        e = pto.exp(pto.sub(x_tile, m_tile))
        pto.store(l_acc, pto.add(l_acc, pto.rowsum(e)))
        pto.store(y_tile, e)

    @kernel
    def rescale(y_tile: InOut[Tile[tr, tc, f32]], l_tile: In[Tile[tr, 1, f32]]):
        pto.store(y_tile, pto.div(y_tile, l_tile))

    bb, ss, vv = Dense[B](), Dense[st](), Dense[vt]()

    @workload
    def softmax_workload():
        for b in P(bb):
            for s in P(ss):
                for v in P.seq(vv):
                    update_rowmax[b, s, v](x_tile=L[b][s][v], m_acc=RM[b][s])
        for b in P(bb):
            for s in P(ss):
                for v in P.seq(vv):
                    exp_and_accumulate[b, s, v](x_tile=L[b][s][v], m_tile=RM[b][s], y_tile=PR[b][s][v], l_acc=RS[b][s])
        for b in P(bb):
            for s in P(ss):
                for v in P(vv):
                    rescale[b, s, v](y_tile=PR[b][s][v], l_tile=RS[b][s])

    return rr4(softmax_workload())


class Softmax3Case:
    """The three-phase softmax example on the tile-program family.  Work = the bytes the
    tasks' tiles read and write (each task: one [8,64] f32 tile per tile operand, the [8,1]
    accumulators)."""
    unit, bound, dtype = "GB/s", "hbm", "f32"

    def __init__(self, name, shape, seed):
        self.name, self.shape, self.seed = name, shape, seed
        self.baseline_config = None

    def setup(self, dev):
        import torch

        g = torch.Generator(device=dev)
        g.manual_seed(self.seed)
        B, S, V = self.shape
        self.lg = torch.randn(self.shape, generator=g, device=dev, dtype=torch.float32) * 0.1
        self.pr = torch.zeros_like(self.lg)
        self.rmax = torch.full((B, S // 8, 8, 1), float("-inf"), device=dev)
        self.rsum = torch.zeros((B, S // 8, 8, 1), device=dev)
        self.prog = softmax3_workload(self.lg, self.pr, self.rmax, self.rsum).compile(target="hip_gfx950")
        tasks = B * (S // 8) * (V // 64)
        tile, acc = 8 * 64 * 4, 8 * 4
        # phase 1: x + m read, m written; phase 2: x, m, l read, y, l written; phase 3: y, l read, y written
        self.work = tasks * ((tile + 2 * acc) + (tile + 2 * acc + tile + acc) + (2 * tile + acc))

    def before_step(self):
        self.rmax.fill_(float("-inf"))
        self.rsum.zero_()

    def peak(self):
        return HBM_PEAK_GBS

    def rate(self, seconds):
        return self.work / seconds / 1e9

    def describe(self):
        B, S, V = self.shape
        return (f"{self.name}: examples/softmax three phases over logits [{B},{S},{V}], [8,64] f32 tiles, "
                f"{'disjoint' if V == 512 else 'overlapping'} views, three launches on the tile-program family")

    def cpu(self, budget_s):
        """Oracle on a bounded sample: batch 0, seq rows 0-63 (8 seq tiles: groups of tasks that
        touch no other rows), against the same rows of the GPU result."""
        import numpy as np

        from oracle.runner import run_workload

        del budget_s
        self.before_step()
        self.prog.execute()
        self.prog.synchronize()
        B, S, V = self.shape
        lg = self.lg[:1, :64].cpu().numpy().copy()
        pr = np.zeros_like(lg)
        rmax = np.full((1, 8, 8, 1), -np.inf, np.float32)
        rsum = np.zeros((1, 8, 8, 1), np.float32)
        t0 = time.perf_counter()
        run_workload(softmax3_workload(lg, pr, rmax, rsum))
        sec = time.perf_counter() - t0
        got = self.pr[:1, :64].cpu().numpy()
        same = bool(np.allclose(got, pr, rtol=1e-5, atol=1e-9))
        nbytes = self.work * 64 / (B * S)
        return nbytes / sec / 1e9, f"batch 0, seq rows 0-63 of [{B},{S},{V}], one oracle run", same


class DecodeCase:
    unit, bound, dtype = "GB/s", "hbm", "bf16"

    def __init__(self, name, batch, hq, hkv, d, lmin, lmax, seed, baseline_config, page=16, f32_inputs=False):
        self.name, self.batch, self.hq, self.hkv, self.d = name, batch, hq, hkv, d
        self.lmin, self.lmax, self.seed, self.page = lmin, lmax, seed, page
        self.baseline_config = baseline_config
        self.f32_inputs = f32_inputs
        self.dtype = "f32" if f32_inputs else "bf16"

    def setup(self, dev):
        import numpy as np
        import torch

        rng = np.random.default_rng(self.seed)
        B, page, G = self.batch, self.page, self.hq // self.hkv
        self.lengths = rng.integers(self.lmin, self.lmax + 1, size=B)
        npages = (self.lengths + page - 1) // page
        max_pages = (self.lmax + page - 1) // page
        total = int(npages.sum())
        phys = rng.permutation(total).astype(np.int32)
        pt = np.zeros((B, max_pages), np.int32)
        mask = np.zeros((B, max_pages, 1, page), np.float32)
        tok = np.arange(max_pages * page).reshape(max_pages, page)
        off = 0
        for b in range(B):
            pt[b, :npages[b]] = phys[off:off + npages[b]]
            off += npages[b]
            mask[b, :, 0, :] = np.where(tok < self.lengths[b], 0.0, 1e30)
        g = torch.Generator(device=dev)
        g.manual_seed(self.seed)
        shape_kv = (total, self.hkv, page, self.d)
        dt = torch.float32 if self.f32_inputs else torch.bfloat16
        t = {"q": torch.randn((B, self.hkv, G, self.d), generator=g, device=dev, dtype=dt),
             "k_cache": torch.randn(shape_kv, generator=g, device=dev, dtype=dt),
             "v_cache": torch.randn(shape_kv, generator=g, device=dev, dtype=dt),
             "page_table": torch.from_numpy(pt).to(dev), "npages": torch.from_numpy(npages.astype(np.int32)).to(dev),
             "mask": torch.from_numpy(mask).to(dev),
             "m": torch.full((B, self.hkv, G, 1), float("-inf"), device=dev),
             "l": torch.zeros((B, self.hkv, G, 1), device=dev), "o": torch.zeros((B, self.hkv, G, self.d), device=dev),
             "out": torch.zeros((B, self.hkv, G, self.d), device=dev)}
        self.t = t
        self.prog = decode_workload(t, page).compile(target="hip_gfx950")
        ntok = int(self.lengths.sum())
        # Algorithmic bytes: K and V of the valid tokens, q (bf16 / f32), out (f32), the page table entries used.
        es = 4 if self.f32_inputs else 2
        self.work = ntok * self.hkv * self.d * es * 2 + B * self.hq * self.d * es + B * self.hq * self.d * 4 + 4 * total

    def before_step(self):
        self.t["m"].fill_(float("-inf"))
        self.t["l"].zero_()
        self.t["o"].zero_()

    def peak(self):
        return HBM_PEAK_GBS

    def rate(self, seconds):
        return self.work / seconds / 1e9

    def describe(self):
        return (f"{self.name}: paged GQA decode, batch {self.batch}, {self.hq} query / {self.hkv} KV heads, head dim "
                f"{self.d}, {self.dtype} Q/K/V N(0,1), lengths U[{self.lmin},{self.lmax}] (sum {int(self.lengths.sum())}), "
                f"{self.page}-token pages, permuted page table; P(batch) x P(kv_head) x P.seq(DenseDyn(pages)) "
                "+ normalize")

    def cpu(self, budget_s):
        """Oracle on a bounded sample: the first 16 sequences (all KV heads), same inputs."""
        import numpy as np
        import torch

        from oracle.runner import run_workload

        del budget_s
        nb = 16
        self.before_step()
        self.prog.execute()
        self.prog.synchronize()
        if self.f32_inputs:
            u16 = lambda x: x.contiguous().cpu().numpy()  # f32 inputs pass through as they are
        else:
            u16 = lambda x: x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        h = {"q": u16(self.t["q"][:nb]), "k_cache": u16(self.t["k_cache"]), "v_cache": u16(self.t["v_cache"]),
             "page_table": self.t["page_table"][:nb].cpu().numpy(), "npages": self.t["npages"][:nb].cpu().numpy(),
             "mask": self.t["mask"][:nb].cpu().numpy()}
        G = self.hq // self.hkv
        h["m"] = np.full((nb, self.hkv, G, 1), -np.inf, np.float32)
        h["l"] = np.zeros((nb, self.hkv, G, 1), np.float32)
        h["o"] = np.zeros((nb, self.hkv, G, self.d), np.float32)
        h["out"] = np.zeros((nb, self.hkv, G, self.d), np.float32)
        t0 = time.perf_counter()
        run_workload(decode_workload(h, self.page))
        sec = time.perf_counter() - t0
        ntok = int(self.lengths[:nb].sum())
        nbytes = ntok * self.hkv * self.d * 4 + nb * self.hq * self.d * 6 + 4 * int(h["npages"].sum())
        got = self.t["out"][:nb].cpu().numpy()
        rel = float(np.linalg.norm(got - h["out"]) / np.linalg.norm(h["out"]))
        self.cpu_rel = rel
        sample = f"sequences 0-15 of the batch ({ntok} tokens, all {self.hkv} KV heads), one oracle run"
        return nbytes / sec / 1e9, sample, rel <= 1e-2


class RowCase:
    unit, bound, dtype = "GB/s", "hbm", "f32"

    def __init__(self, name, kind, shape, sigma, seed, baseline_config):
        self.name, self.kind, self.shape, self.sigma, self.seed = name, kind, shape, sigma, seed
        self.baseline_config = baseline_config

    def setup(self, dev):
        import torch

        g = torch.Generator(device=dev)
        g.manual_seed(self.seed)
        self.x = torch.randn(self.shape, generator=g, device=dev, dtype=torch.float32) * self.sigma
        self.y = torch.empty_like(self.x)
        self.prog = row_workload(self.kind, self.x, self.y).compile(target="hip_gfx950")
        self.work = 2 * self.x.numel() * 4  # bytes read + written

    def peak(self):
        return HBM_PEAK_GBS

    def rate(self, seconds):
        return self.work / seconds / 1e9

    def describe(self):
        return (f"{self.name}: {self.kind}_tile Tile[{self.shape[2]},{self.shape[3]},F32] over X{list(self.shape)}, "
                f"P(batch={self.shape[0]}) x P(tiles={self.shape[1]}), round_robin(4), TaskWindow(8192, STALL)")

    def cpu(self, budget_s):
        """Oracle over the whole workload (repeated within the budget) + parity of the GPU output.
        The module is serialized once, as the reference compiles its artifact once; each timed
        run is the oracle's execution of the whole workload (wall clock around the call, like the
        reference's execute() + synchronize()).  Small workloads repeat up to 5000 times."""
        import numpy as np

        from oracle.runner import run_module
        from pto_wsp.ir_bridge import workload_to_codegen_ir
        from pto_wsp.program import Program

        xh = self.x.detach().cpu().numpy()
        yh = np.zeros_like(xh)
        wl = row_workload(self.kind, xh, yh)
        build = workload_to_codegen_ir(wl, module_name="bench_cpu")
        arrays = [t.data for t in build.tensors]
        sizes = Program._infer_axis_sizes(wl)
        times = []
        t_start = time.perf_counter()
        while len(times) < 5000 and (len(times) < 8 or self.x.numel() < (1 << 20)) and (time.perf_counter() - t_start) < budget_s:
            t0 = time.perf_counter()
            res = run_module(build.module, arrays, sizes)
            times.append(time.perf_counter() - t0)
        sec = sum(times) / len(times)
        self.cpu_us_per_run = sec * 1e6
        self.cpu_tasks_per_s = res.task_count / sec
        same = bool(np.allclose(self.y.cpu().numpy(), yh, rtol=1e-5, atol=1e-6 if self.kind != "softmax" else 0.0))
        sample = (f"the full {self.name} workload X{list(self.shape)}, {len(times)} run(s) of {sec * 1e3:.4g} ms each, "
                  f"wall clock around the oracle call")
        return self.work / sec / 1e9, sample, same


class GemmCase:
    unit, bound = "TFLOP/s", "mfma"

    def __init__(self, name, nb, m, n, k, seed, baseline_config, f32_inputs=False, tile=(128, 128, 64), dtype="bf16"):
        self.name, self.nb, self.m, self.n, self.k, self.seed = name, nb, m, n, k, seed
        self.baseline_config = baseline_config
        self.shape = (nb, m, k)
        self.f32_inputs = f32_inputs
        self.tile = tile
        self.in_dtype = "f32" if f32_inputs else dtype
        self.dtype = self.in_dtype

    def setup(self, dev):
        import torch

        g = torch.Generator(device=dev)
        g.manual_seed(self.seed)
        dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[self.in_dtype]
        self.a = (torch.rand((self.nb, self.m, self.k), generator=g, device=dev) * 2 - 1).to(dt)
        self.b = (torch.rand((self.nb, self.k, self.n), generator=g, device=dev) * 2 - 1).to(dt)
        self.c = torch.zeros((self.nb, self.m, self.n), device=dev, dtype=torch.float32)
        tm, tn, tk = self.tile
        self.prog = bgemm_workload(self.a, self.b, self.c, tm, tn, tk, f32_inputs=self.f32_inputs,
                                   f16_inputs=self.in_dtype == "f16").compile(target="hip_gfx950")
        self.work = 2.0 * self.nb * self.m * self.n * self.k  # FLOP per step

    def peak(self):
        return F32_PEAK_TFLOPS if self.f32_inputs else BF16_PEAK_TFLOPS

    def rate(self, seconds):
        return self.work / seconds / 1e12

    def describe(self):
        tm, tn, tk = self.tile
        return (f"{self.name}: C[b] += A[b] @ B[b], A,B[{self.nb},{self.m},{self.k}] {self.dtype} U(-1,1), C fp32, "
                f"tiles {tm}x{tn} K-step {tk}, P(batch) x P(m_tiles) x P(n_tiles) x P.seq(k)")

    def cpu(self, budget_s):
        """Oracle on a bounded sample: batch 0, the first 2 m-tiles (all n, all k), from C = 0."""
        import numpy as np

        from oracle.runner import run_workload

        del budget_s
        import torch

        if self.in_dtype in ("f32", "f16"):
            a0, b0 = self.a[:1, :256].contiguous().cpu().numpy(), self.b[:1].contiguous().cpu().numpy()
        else:
            a0 = self.a[:1, :256].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
            b0 = self.b[:1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        c0 = np.zeros((1, 256, self.n), np.float32)
        tm, tn, tk = self.tile
        t0 = time.perf_counter()
        run_workload(bgemm_workload(a0, b0, c0, tm, tn, tk, f32_inputs=self.f32_inputs, f16_inputs=self.in_dtype == "f16"))
        sec = time.perf_counter() - t0
        flop = 2.0 * 256 * self.n * self.k
        # GPU result for the same tiles, from a fresh C = 0 run.
        self.c.zero_()
        self.prog.execute()
        self.prog.synchronize()
        got = self.c[0, :256].cpu().numpy()
        rel = float(np.linalg.norm(got - c0) / np.linalg.norm(c0))
        sample = f"batch 0, m-tiles 0-1 (256 x {self.n} outputs, K={self.k}), {flop / 1e9:.1f} GFLOP, one oracle run"
        return flop / sec / 1e12, sample, rel <= 1e-2


CASES = {
    "rmsnorm_quickstart": lambda: RowCase("rmsnorm_quickstart", "rmsnorm", (1, 2, 16, 128), 1.0, 0, 0),
    "rmsnorm_bw": lambda: RowCase("rmsnorm_bw", "rmsnorm", (16, 8192, 16, 128), 1.0, 0, 1),
    "softmax": lambda: RowCase("softmax", "softmax", (8, 4096, 32, 512), 3.0, 0, 2),
    "bgemm": lambda: GemmCase("bgemm", 64, 2048, 2048, 2048, 0, 3),
    "paged_decode": lambda: DecodeCase("paged_decode", 64, 32, 8, 128, 512, 8192, 0, 4),
    # Not a BASELINE config: a plain tile copy of known size (1 GiB in, 1 GiB
    # out) through the same backend, used to calibrate rocprofv3 traffic
    # counters and as the achievable-bandwidth reference.
    "copy_calib": lambda: RowCase("copy_calib", "copy", (16, 8192, 16, 128), 1.0, 0, None),
    # Not BASELINE configs: the reference's three-phase softmax example on the
    # tile-program family, with disjoint views (V = 512) and with overlapping
    # views (V = 256), whose rescale launch runs as groups of tasks in program
    # order (PTOWSP_SERIAL_GROUPS=0: the whole launch in one workgroup).
    "softmax3": lambda: Softmax3Case("softmax3", (8, 4096, 512), 0),
    "softmax3_overlap": lambda: Softmax3Case("softmax3_overlap", (8, 4096, 256), 0),
    # Not BASELINE configs: the C5 decode with 32- and 64-token pages (the same
    # lengths and heads; the decode family folds them as 16-token sub-pages)
    # and with 8-token pages (folded two to a 16-token step).
    "paged_decode_page32": lambda: DecodeCase("paged_decode_page32", 64, 32, 8, 128, 512, 8192, 0, None, page=32),
    "paged_decode_page64": lambda: DecodeCase("paged_decode_page64", 64, 32, 8, 128, 512, 8192, 0, None, page=64),
    "paged_decode_page8": lambda: DecodeCase("paged_decode_page8", 64, 32, 8, 128, 512, 8192, 0, None, page=8),
    # Not BASELINE configs: the C5 lengths and KV heads with other query-row
    # counts and head dims (head dim 64 with 8 rows, head dim 256 with 4
    # rows, 16 rows at head dim 128 with 32-token pages, 32 rows at 128).
    "paged_decode_d64": lambda: DecodeCase("paged_decode_d64", 64, 64, 8, 64, 512, 8192, 0, None),
    "paged_decode_d256": lambda: DecodeCase("paged_decode_d256", 64, 32, 8, 256, 512, 8192, 0, None),
    "paged_decode_g16": lambda: DecodeCase("paged_decode_g16", 64, 128, 8, 128, 512, 8192, 0, None, page=32),
    "paged_decode_g32": lambda: DecodeCase("paged_decode_g32", 64, 256, 8, 128, 512, 8192, 0, None),
    # 16 rows with 16-token pages: the [1, 16] mask is a row broadcast there.
    "paged_decode_g16_rowmask": lambda: DecodeCase("paged_decode_g16_rowmask", 64, 128, 8, 128, 512, 8192, 0, None),
    # Not a BASELINE config: the C5 decode with f32 q / K / V.
    "paged_decode_f32": lambda: DecodeCase("paged_decode_f32", 64, 32, 8, 128, 512, 8192, 0, None, f32_inputs=True),
    "paged_decode_f32_g32": lambda: DecodeCase("paged_decode_f32_g32", 64, 256, 8, 128, 512, 8192, 0, None, f32_inputs=True),
    "paged_decode_f32_d64_g48": lambda: DecodeCase("paged_decode_f32_d64_g48", 64, 384, 8, 64, 512, 8192, 0, None,
                                                   f32_inputs=True),
    "paged_decode_f32_d256": lambda: DecodeCase("paged_decode_f32_d256", 64, 32, 8, 256, 512, 8192, 0, None, f32_inputs=True),
    # Not a BASELINE config: the C4 GEMM with f32 A and B (the reference's own
    # matmul dtype), on the f32 MFMA block.
    "bgemm_f32": lambda: GemmCase("bgemm_f32", 64, 2048, 2048, 2048, 0, None, f32_inputs=True),
    # Not a BASELINE config: the reference bgemm example's own pattern (16x16x16
    # f16 tiles) at the C4 shape; the host merges 16 x 16 tasks per block and
    # 4 K steps per LDS stage.
    "bgemm_tile16": lambda: GemmCase("bgemm_tile16", 64, 2048, 2048, 2048, 0, None, tile=(16, 16, 16), dtype="f16"),
}
EXTRA = ("copy_calib", "softmax3", "softmax3_overlap", "paged_decode_page32", "paged_decode_page64", "paged_decode_page8",
         "paged_decode_d64", "paged_decode_d256", "paged_decode_g16", "paged_decode_g32", "paged_decode_g16_rowmask",
         "paged_decode_f32",
         "paged_decode_f32_g32", "paged_decode_f32_d64_g48", "paged_decode_f32_d256", "bgemm_f32", "bgemm_tile16")


def load_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (profiles/<name>_traffic.md, line 'traffic_bytes: N'), or None."""
    path = os.path.join(ROOT, "profiles", f"{name}_traffic.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.strip().startswith("traffic_bytes:"):
                return int(line.split(":", 1)[1].strip())
    return None


def time_case(case, steps, warmup, warm_s=0.0):
    """W untimed warmup steps (continued until warm_s seconds have passed:
    the GPU raises its clocks over the first tens of milliseconds of sustained
    MFMA work), then exactly `steps` timed steps."""
    import torch

    before = getattr(case, "before_step", lambda: None)
    # The first step builds the kernels (hiprtc, on a fresh box); the warmup
    # clock starts after it.
    before()
    case.prog.execute()
    case.prog.synchronize()
    done = 1
    t_warm = time.perf_counter()
    while done < warmup or time.perf_counter() - t_warm < warm_s:
        before()
        case.prog.execute()
        case.prog.synchronize()
        done += 1
    case.warmup_done = done
    torch.cuda.synchronize()
    kernel_ms = []
    t0 = time.perf_counter()
    for _ in range(steps):
        before()
        case.prog.execute()
        case.prog.synchronize()
        kernel_ms.append(case.prog.stats.device_time_ms)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    k_ms = sum(kernel_ms) / len(kernel_ms)
    return wall_s / steps * 1000.0, k_ms


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="all", help=f"one of {list(CASES)} or 'all'")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--warm-s", type=float, default=0.25,
                    help="minimum warmup time (s) of every config line but the headline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if not os.path.exists(os.path.join(ROOT, "pto-wsp_amd", "pto_wsp", "libptowsp_hip.so")):
        import __graft_entry__

        __graft_entry__.build()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")

    if args.config == "all":
        names = [n for n in CASES if n not in EXTRA]
    else:
        names = [args.config]
    head = HEADLINE if HEADLINE in names else names[0]
    per, line_main, cpu = {}, None, None
    for name in names:
        case = CASES[name]()
        case.setup(dev)
        # The headline config (rmsnorm_bw) keeps exactly W warmup steps; every other config
        # line is measured at steady clocks (at least 0.25 s of warmup).
        ms_step, k_ms = time_case(case, args.steps, args.warmup, 0.0 if name == HEADLINE else args.warm_s)
        achieved = case.rate(k_ms * 1e-3)
        entry = {"baseline_config": case.baseline_config, "kernel_ms": round(k_ms, 5), "ms_per_step": round(ms_step, 5),
                 "achieved": round(achieved, 2), "unit": case.unit, "peak": case.peak(),
                 "frac": round(achieved / case.peak(), 4), "warmup": case.warmup_done, "steps": args.steps,
                 "tasks": case.prog.stats.task_count,
                 "total_cycles": case.prog.stats.total_cycles,
                 "kernel_us": round(k_ms * 1e3, 2), "step_us": round(ms_step * 1e3, 2),
                 "tasks_per_s": round(case.prog.stats.task_count / (ms_step * 1e-3), 1)}
        if not args.no_cpu:
            rate, sample, same = case.cpu(12.0 if name == head else (2.0 if name == "rmsnorm_quickstart" else 6.0))
            entry["cpu_sim_port"] = round(rate, 6)
            entry["matches_cpu_sim"] = same
            entry["cpu_sample"] = sample
            entry["cpu_cores"] = f"1 of {len(os.sched_getaffinity(0))}"
            if hasattr(case, "cpu_us_per_run"):
                entry["cpu_us_per_run"] = round(case.cpu_us_per_run, 2)
                entry["cpu_tasks_per_s"] = round(case.cpu_tasks_per_s, 1)
            if name == head:
                cpu = {"value": round(rate, 4), "unit": case.unit, "cores": 1, "kind": "port",
                       "sample": sample + f", 1 of {len(os.sched_getaffinity(0))} cores"}
        per[name] = entry
        if name == head:
            line_main = {"case": case, "ms_step": ms_step, "k_ms": k_ms, "achieved": achieved}
        else:
            del case
            torch.cuda.empty_cache()

    case = line_main["case"]
    line = {
        "metric": METRIC,
        "value": round(case.rate(line_main["ms_step"] * 1e-3), 2),
        "unit": case.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(line_main["ms_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": case.dtype,
        "data": "synthetic (torch RNG on device, seeded)",
        "config": {"workload": case.describe(), "baseline_config": case.baseline_config,
                   "work_per_step": case.work, "target": "hip_gfx950"},
        "roofline": {"bound": case.bound, "achieved": round(line_main["achieved"], 2), "peak": case.peak(),
                     "unit": case.unit, "frac": round(line_main["achieved"] / case.peak(), 4),
                     "traffic": load_traffic(head)},
        "cpu_baseline": cpu,
        "configs": per,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
