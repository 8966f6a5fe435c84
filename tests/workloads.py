"""Workload factories shared by the tests.

Each factory takes a dict of arrays (numpy, or torch tensors on the GPU)
and returns an un-scheduled Workload over them, so the same workload can be
built twice: once over the GPU-side buffers and once over the oracle's
numpy copies.  The kernels restate the reference's README quickstart, its
examples (examples/*/pto_wsp_impl.py) and its codegen tests
(tests/test_codegen_*.py) in this repository's own words.
"""

import math

import numpy as np

from pto_wsp import (DType, Dense, DenseDyn, DispatchPolicy, In, InOut, Out, P, Ragged, Scalar, Symbol,
                     TaskWindow, Tensor, Tile, WindowMode, Workload, kernel, pto, workload)

F32, F16, BF16, I32 = DType.F32, DType.F16, DType.BF16, DType.I32


def T(arr, dtype=F32) -> Tensor:
    return Tensor(data=arr, shape=tuple(arr.shape), dtype=dtype)


def rr4(w, window: int = 8192):
    """The schedule every reference example uses: round_robin(4) + STALL window."""
    return w.dispatch(DispatchPolicy.round_robin(num_aicpus=4)).task_graph(
        window=TaskWindow(window, "tasks", WindowMode.STALL))


# ---------------------------------------------------------------- rmsnorm
def rmsnorm(arrs: dict):
    """README quickstart kernel over X[B, T, R, C]: out = x * rsqrt(rowmean(x*x)), no eps."""
    x = arrs["x"]
    B, NT, R, C = x.shape
    X, Y = T(arrs["x"]), T(arrs["y"])

    @kernel
    def rmsnorm_tile(x: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        sq = pto.mul(x, x)
        mean_sq = pto.rowmean(sq)
        inv = pto.rsqrt(mean_sq)
        pto.store(out, pto.mul(x, inv))

    batch, tiles = Dense[B](), Dense[NT]()

    @workload
    def rmsnorm_wl():
        for b in P(batch):
            for t in P(tiles):
                rmsnorm_tile[b, t](x=X[b][t], out=Y[b][t])

    return rmsnorm_wl()


# ---------------------------------------------------------------- row softmax
def softmax(arrs: dict):
    """Row softmax tile kernel over X[B, T, R, C]: e = exp(x - rowmax(x)); out = e / rowsum(e)."""
    x = arrs["x"]
    B, NT, R, C = x.shape
    X, Y = T(arrs["x"]), T(arrs["y"])

    @kernel
    def softmax_tile(x: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        m = pto.rowmax(x)
        e = pto.exp(pto.sub(x, m))
        s = pto.rowsum(e)
        pto.store(out, pto.div(e, s))

    batch, tiles = Dense[B](), Dense[NT]()

    @workload
    def softmax_wl():
        for b in P(batch):
            for t in P(tiles):
                softmax_tile[b, t](x=X[b][t], out=Y[b][t])

    return softmax_wl()


# ---------------------------------------------------------------- 3-phase softmax (examples/softmax)
def softmax3(arrs: dict):
    """Three launches with P.seq accumulators: running max, exp + running sum, rescale."""
    lg, pr = arrs["logits"], arrs["probs"]
    B, S, V = lg.shape
    tr, tc = 8, 64
    st, vt = S // tr, V // tc
    L = T(lg.reshape(B, st, tr, vt, tc))
    PR = T(pr.reshape(B, st, tr, vt, tc))
    RM, RS = T(arrs["rmax"]), T(arrs["rsum"])

    @kernel
    def update_rowmax(x_tile: In[Tile[tr, tc, F32]], m_acc: InOut[Tile[tr, 1, F32]]):
        pto.store(m_acc, pto.max(m_acc, pto.rowmax(x_tile)))

    @kernel
    def exp_and_accumulate(x_tile: In[Tile[tr, tc, F32]], m_tile: In[Tile[tr, 1, F32]],
                           y_tile: Out[Tile[tr, tc, F32]], l_acc: InOut[Tile[tr, 1, F32]]):
        e = pto.exp(pto.sub(x_tile, m_tile))
        pto.store(l_acc, pto.add(l_acc, pto.rowsum(e)))
        pto.store(y_tile, e)

    @kernel
    def rescale(y_tile: InOut[Tile[tr, tc, F32]], l_tile: In[Tile[tr, 1, F32]]):
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

    return softmax_workload()


def softmax3_arrays(logits: np.ndarray) -> dict:
    B, S, V = logits.shape
    return {"logits": logits.copy(), "probs": np.zeros_like(logits),
            "rmax": np.full((B, S // 8, 8, 1), -np.inf, np.float32), "rsum": np.zeros((B, S // 8, 8, 1), np.float32)}


# ---------------------------------------------------------------- bgemm (examples/bgemm pattern)
def bgemm(arrs: dict, tm: int = 16, tn: int = 16, tk: int = 16, dtype=F16, plain: bool = False):
    """C[b] += A[b] @ B[b] over tiles with a P.seq K loop and an InOut accumulator.
    plain=True stores matmul(a, b) alone (the last K step wins, as in the reference)."""
    a, b_, c = arrs["a"], arrs["b"], arrs["c"]
    B, M, K = a.shape
    N = b_.shape[2]
    def perm(x, axes):  # numpy or torch
        return x.permute(*axes) if hasattr(x, "permute") else x.transpose(*axes)

    at = perm(a.reshape(B, M // tm, tm, K // tk, tk), (0, 1, 3, 2, 4))
    bt = perm(b_.reshape(B, K // tk, tk, N // tn, tn), (0, 3, 1, 2, 4))
    ct = perm(c.reshape(B, M // tm, tm, N // tn, tn), (0, 1, 3, 2, 4))
    A, Bm, C = T(at, dtype), T(bt, dtype), T(ct)

    if plain:
        @kernel
        def gemm_tile(a_tile: In[Tile[tm, tk, dtype]], b_tile: In[Tile[tk, tn, dtype]], c_tile: Out[Tile[tm, tn, F32]]):
            pto.store(c_tile, pto.matmul(a_tile, b_tile))
    else:
        @kernel
        def gemm_tile(a_tile: In[Tile[tm, tk, dtype]], b_tile: In[Tile[tk, tn, dtype]], c_tile: InOut[Tile[tm, tn, F32]]):
            acc = pto.matmul(a_tile, b_tile)
            pto.store(c_tile, pto.add(c_tile, acc))

    batch, mt, nt, kt = Dense[B](), Dense[M // tm](), Dense[N // tn](), Dense[K // tk]()

    @workload
    def bgemm_wl():
        for b in P(batch):
            for m in P(mt):
                for n in P(nt):
                    for k in P.seq(kt):
                        gemm_tile[b, m, n, k](a_tile=A[b][m][k], b_tile=Bm[b][n][k], c_tile=C[b][m][n])

    return bgemm_wl()


def bgemm_split_k(arrs: dict, tm: int, tn: int, tk: int, k_outer: int, dtype=BF16):
    """bgemm with the K loop split into two nested P.seq loops (k = ko * (K/tk/k_outer) + ki)."""
    a, b_, c = arrs["a"], arrs["b"], arrs["c"]
    B, M, K = a.shape
    N = b_.shape[2]
    kin = K // tk // k_outer
    at = a.reshape(B, M // tm, tm, k_outer, kin, tk).transpose(0, 1, 3, 4, 2, 5)
    bt = b_.reshape(B, k_outer, kin, tk, N // tn, tn).transpose(0, 4, 1, 2, 3, 5)
    ct = c.reshape(B, M // tm, tm, N // tn, tn).transpose(0, 1, 3, 2, 4)
    A, Bm, C = T(at, dtype), T(bt, dtype), T(ct)

    @kernel
    def gemm_tile(a_tile: In[Tile[tm, tk, dtype]], b_tile: In[Tile[tk, tn, dtype]], c_tile: InOut[Tile[tm, tn, F32]]):
        pto.store(c_tile, pto.add(c_tile, pto.matmul(a_tile, b_tile)))

    @workload
    def split_wl():
        for b in P(Dense[B]()):
            for m in P(Dense[M // tm]()):
                for n in P(Dense[N // tn]()):
                    # named: P.seq defaults every loop variable to "i", so nested loops would shadow
                    for ko in P.seq(Dense[k_outer](), name="ko"):
                        for ki in P.seq(Dense[kin](), name="ki"):
                            gemm_tile[b, m, n, ko, ki](a_tile=A[b][m][ko][ki], b_tile=Bm[b][n][ko][ki], c_tile=C[b][m][n])

    return split_wl()


# ---------------------------------------------------------------- decode / attention (f32 examples)
def decode_attention(arrs: dict):
    """examples/flashinfer_decode: one task, whole KV in one tile."""
    q, kt, v, o = arrs["q"], arrs["k_t"], arrs["v"], arrs["o"]
    d, kv = q.shape[1], kt.shape[1]
    Q, KT, V, O = T(q), T(kt), T(v), T(o)

    @kernel
    def decode_attention_tile(q_tile: In[Tile[1, d, F32]], k_t_tile: In[Tile[d, kv, F32]],
                              v_tile: In[Tile[kv, d, F32]], out_tile: Out[Tile[1, d, F32]]):
        scores = pto.matmul(q_tile, k_t_tile)
        scores = pto.mul(scores, pto.constant(1.0 / math.sqrt(d), F32))
        scores = pto.sub(scores, pto.rowmax(scores))
        e = pto.exp(scores)
        w = pto.div(e, pto.rowsum(e))
        pto.store(out_tile, pto.matmul(w, v_tile))

    @workload
    def decode():
        decode_attention_tile[0](q_tile=Q, k_t_tile=KT, v_tile=V, out_tile=O)

    return decode()


def tiled_attention(arrs: dict, tile_seq: int):
    """examples/attention: per (b, h, s-tile) softmax(q k^T / sqrt(d)) v."""
    q, kt, v, o = arrs["q"], arrs["k_t"], arrs["v"], arrs["o"]
    B, H, S, D = q.shape
    st = S // tile_seq
    Q = T(q.reshape(B, H, st, tile_seq, D))
    KT = T(kt)
    V = T(v.reshape(B, H, st, tile_seq, D))
    O = T(o.reshape(B, H, st, tile_seq, D))

    @kernel
    def attention_tile(q: In[Tile[tile_seq, D, F32]], k_t: In[Tile[D, tile_seq, F32]],
                       v: In[Tile[tile_seq, D, F32]], out: Out[Tile[tile_seq, D, F32]]):
        s = pto.mul(pto.matmul(q, k_t), pto.constant(1.0 / math.sqrt(D), F32))
        s = pto.sub(s, pto.rowmax(s))
        e = pto.exp(s)
        pto.store(out, pto.matmul(pto.div(e, pto.rowsum(e)), v))

    bb, hh, ss = Dense[B](), Dense[H](), Dense[st]()

    @workload
    def attention():
        for b, h in P(bb, hh):
            for s in P(ss):
                attention_tile[b, h, s](q=Q[b][h][s], k_t=KT[b][h][s], v=V[b][h][s], out=O[b][h][s])

    return attention()


def attention_arrays(q, k, v, tile_seq):
    B, H, S, D = q.shape
    kt = np.ascontiguousarray(k.reshape(B, H, S // tile_seq, tile_seq, D).transpose(0, 1, 2, 4, 3))
    return {"q": q.copy(), "k_t": kt, "v": v.copy(), "o": np.zeros_like(q)}


# ---------------------------------------------------------------- paged GQA decode (config 5)
def paged_decode(arrs: dict, scale: float | None = None, masked: bool = True, dtype=BF16, out_key: str = "out"):
    """flashinfer_decode over a paged KV cache: P(batch) x P(kv_head) x P.seq(pages).

    Per (b, g) the kernel folds one 16-token page into running (m, l, o) with
    online softmax for the G query heads of KV group g; the page comes from the
    page table (indirect index) and the page count of sequence b from npages[b]
    (a tensor-bound DenseDyn).  The last page's padding tokens are masked with a
    [1, page] penalty (0 or 1e30) subtracted from the scores.  A second launch
    writes out = o / l.

    arrs: q [B, Hkv, G, D] bf16 bits; k_cache, v_cache [P, Hkv, page, D] bf16 bits;
    page_table [B, max_pages] i32; npages [B] i32; mask [B, max_pages, 1, page] f32;
    m [B, Hkv, G, 1] f32 (-inf); l [B, Hkv, G, 1] f32 (0); o [B, Hkv, G, D] f32 (0);
    out [B, Hkv, G, D] f32.  out_key names the array the second launch writes
    (out_key="o" normalises in place).
    """
    q, kc, vc = arrs["q"], arrs["k_cache"], arrs["v_cache"]
    B, Hkv, G, D = q.shape
    page = kc.shape[2]
    max_pages = arrs["page_table"].shape[1]
    sc = float(scale if scale is not None else 1.0 / math.sqrt(D))

    def perm(x, axes):  # numpy or torch
        return x.permute(*axes) if hasattr(x, "permute") else x.transpose(*axes)

    Q, KT, V = T(q, dtype), T(perm(kc, (0, 1, 3, 2)), dtype), T(vc, dtype)
    PT, NP = T(arrs["page_table"], I32), T(arrs["npages"], I32)
    MASK, M, L, O = T(arrs["mask"]), T(arrs["m"]), T(arrs["l"]), T(arrs["o"])
    OUT = O if out_key == "o" else T(arrs[out_key])

    @kernel
    def decode_page(q: In[Tile[G, D, dtype]], k_t: In[Tile[D, page, dtype]], v: In[Tile[page, D, dtype]],
                    mask: In[Tile[1, page, F32]], m_acc: InOut[Tile[G, 1, F32]], l_acc: InOut[Tile[G, 1, F32]],
                    o_acc: InOut[Tile[G, D, F32]]):
        s = pto.mul(pto.matmul(q, k_t), pto.constant(sc, F32))
        if masked:
            s = pto.sub(s, mask)
        m_new = pto.max(m_acc, pto.rowmax(s))
        p = pto.exp(pto.sub(s, m_new))
        alpha = pto.exp(pto.sub(m_acc, m_new))
        pto.store(l_acc, pto.add(pto.mul(l_acc, alpha), pto.rowsum(p)))
        pto.store(o_acc, pto.add(pto.mul(o_acc, alpha), pto.matmul(p, v)))
        pto.store(m_acc, m_new)

    @kernel
    def normalize(o_acc: In[Tile[G, D, F32]], l_acc: In[Tile[G, 1, F32]], out: Out[Tile[G, D, F32]]):
        pto.store(out, pto.div(o_acc, l_acc))

    @workload
    def paged_decode_wl():
        for b in P(Dense[B]()):
            for g in P(Dense[Hkv]()):
                for pg in P.seq(DenseDyn(max_pages, extent=NP[b]), name="pg"):
                    decode_page[b, g, pg](q=Q[b][g], k_t=KT[PT[b][pg]][g], v=V[PT[b][pg]][g], mask=MASK[b][pg],
                                          m_acc=M[b][g], l_acc=L[b][g], o_acc=O[b][g])
        for b in P(Dense[B]()):
            for g in P(Dense[Hkv]()):
                normalize[b, g](o_acc=O[b][g], l_acc=L[b][g], out=OUT[b][g])

    return paged_decode_wl()


def paged_decode_arrays(lengths, hkv: int, group: int, d: int, page: int = 16, seed: int = 0,
                        spare_pages: int = 3, f16: bool = False, f32: bool = False) -> dict:
    """Seeded numpy inputs: bf16 (f16, f32) q / K / V ~ N(0,1); page table = a random permutation
    of the physical pages (plus a few never-referenced spares)."""
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, np.int64)
    B = len(lengths)
    npages = (lengths + page - 1) // page
    max_pages = int(npages.max())
    total = int(npages.sum()) + spare_pages
    phys = rng.permutation(total).astype(np.int32)
    pt = np.zeros((B, max_pages), np.int32)
    mask = np.zeros((B, max_pages, 1, page), np.float32)
    off = 0
    for b in range(B):
        n = int(npages[b])
        pt[b, :n] = phys[off:off + n]
        off += n
        t = np.arange(max_pages * page).reshape(max_pages, page)
        mask[b, :, 0, :] = np.where(t < lengths[b], 0.0, 1e30)
    if f32:
        bf = lambda shape: rng.standard_normal(shape).astype(np.float32)
    elif f16:
        bf = lambda shape: rng.standard_normal(shape).astype(np.float16)
    else:
        bf = lambda shape: bf16_round(rng.standard_normal(shape).astype(np.float32))
    return {"q": bf((B, hkv, group, d)), "k_cache": bf((total, hkv, page, d)), "v_cache": bf((total, hkv, page, d)),
            "page_table": pt, "npages": npages.astype(np.int32), "mask": mask,
            "m": np.full((B, hkv, group, 1), -np.inf, np.float32), "l": np.zeros((B, hkv, group, 1), np.float32),
            "o": np.zeros((B, hkv, group, d), np.float32), "out": np.zeros((B, hkv, group, d), np.float32),
            "lengths": lengths}


def paged_decode_torch(dev, batch: int, hq: int, hkv: int, d: int, lmin: int, lmax: int, seed: int = 0,
                       page: int = 16, f32: bool = False) -> dict:
    """Config-5 sized inputs on the device: lengths ~ U[lmin, lmax] and a permuted page
    table from numpy (seeded), bf16 (f32) q / K / V ~ N(0,1) from torch's device RNG."""
    import torch

    rng = np.random.default_rng(seed)
    G = hq // hkv
    lengths = rng.integers(lmin, lmax + 1, size=batch)
    npages = (lengths + page - 1) // page
    max_pages = (lmax + page - 1) // page
    total = int(npages.sum())
    phys = rng.permutation(total).astype(np.int32)
    pt = np.zeros((batch, max_pages), np.int32)
    mask = np.zeros((batch, max_pages, 1, page), np.float32)
    tok = np.arange(max_pages * page).reshape(max_pages, page)
    off = 0
    for b in range(batch):
        pt[b, :npages[b]] = phys[off:off + npages[b]]
        off += npages[b]
        mask[b, :, 0, :] = np.where(tok < lengths[b], 0.0, 1e30)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    kv = (total, hkv, page, d)
    dt = torch.float32 if f32 else torch.bfloat16
    return {"q": torch.randn((batch, hkv, G, d), generator=g, device=dev, dtype=dt),
            "k_cache": torch.randn(kv, generator=g, device=dev, dtype=dt),
            "v_cache": torch.randn(kv, generator=g, device=dev, dtype=dt),
            "page_table": torch.from_numpy(pt).to(dev), "npages": torch.from_numpy(npages.astype(np.int32)).to(dev),
            "mask": torch.from_numpy(mask).to(dev),
            "m": torch.full((batch, hkv, G, 1), float("-inf"), device=dev),
            "l": torch.zeros((batch, hkv, G, 1), device=dev), "o": torch.zeros((batch, hkv, G, d), device=dev),
            "out": torch.zeros((batch, hkv, G, d), device=dev), "lengths": lengths}


def paged_decode_ref(arrs: dict) -> np.ndarray:
    """float64 softmax(q k^T / sqrt(d)) v over each sequence's valid tokens."""
    up = ((lambda x: x.astype(np.float64)) if arrs["q"].dtype in (np.float16, np.float32)
          else (lambda x: bf16_to_f32(x).astype(np.float64)))
    q, kc, vc = up(arrs["q"]), up(arrs["k_cache"]), up(arrs["v_cache"])
    B, Hkv, G, D = q.shape
    page = kc.shape[2]
    out = np.zeros((B, Hkv, G, D))
    for b in range(B):
        L = int(arrs["lengths"][b])
        if L == 0:
            continue  # no tokens: no softmax (left at zero)
        n = (L + page - 1) // page
        pages = arrs["page_table"][b, :n]
        k = kc[pages].transpose(1, 0, 2, 3).reshape(Hkv, n * page, D)[:, :L]
        v = vc[pages].transpose(1, 0, 2, 3).reshape(Hkv, n * page, D)[:, :L]
        s = np.einsum("hgd,htd->hgt", q[b], k) / math.sqrt(D)
        w = np.exp(s - s.max(-1, keepdims=True))
        out[b] = np.einsum("hgt,htd->hgd", w / w.sum(-1, keepdims=True), v)
    return out


# ---------------------------------------------------------------- small reference tests
def matmul_tile(arrs: dict, m: int, k: int, n: int, dtype=F32):
    """tests/test_codegen_execute_basic.py / examples/validated_matmul: C[b][0] = A[b][0] @ B[b][0]."""
    A, B, C = T(arrs["a"], dtype), T(arrs["b"], dtype), T(arrs["c"])
    nb = arrs["a"].shape[0]

    @kernel
    def mm(a: In[Tile[m, k, dtype]], b: In[Tile[k, n, dtype]], out: Out[Tile[m, n, F32]]):
        pto.store(out, pto.matmul(a, b))

    batch = Dense[nb]()

    @workload
    def wl():
        for b in P(batch):
            mm[b](a=A[b][0], b=B[b][0], out=C[b][0])

    return wl()


def copy_tiles(arrs: dict, n: int = 4):
    """tests/test_codegen_schedule_dispatch_window.py: copy 4x4 tiles."""
    A, B = T(arrs["a"]), T(arrs["b"])
    tiles = Dense[n]()

    @kernel
    def copy_tile(src: In[Tile[4, 4, F32]], dst: Out[Tile[4, 4, F32]]):
        pto.store(dst, src)

    @workload
    def wl():
        for t in P(tiles):
            copy_tile[t](src=A[t], dst=B[t])

    return wl()


def scale_symbol(arrs: dict):
    """tests/test_codegen_dynamic_symbols.py: y = x * s with s a runtime symbol."""
    X, Y = T(arrs["x"]), T(arrs["y"])

    @kernel
    def scale(x_tile: In[Tile[4, 4, F32]], y_tile: Out[Tile[4, 4, F32]], s: Scalar[F32]):
        pto.store(y_tile, pto.mul(x_tile, s))

    @workload
    def wl():
        scale(x_tile=X, y_tile=Y, s=Symbol("scale_s"))

    return wl()


def dense_dyn_mm(arrs: dict):
    """tests/test_codegen_dynamic_axes.py: DenseDyn batch bound at run time ("b")."""
    a, b, c = T(arrs["a"]), T(arrs["b"]), T(arrs["c"])
    batch = DenseDyn(0)

    @kernel
    def mm(a_tile: In[Tile[4, 4, F32]], b_tile: In[Tile[4, 4, F32]], c_tile: Out[Tile[4, 4, F32]]):
        pto.store(c_tile, pto.matmul(a_tile, b_tile))

    @workload
    def wl():
        for bidx in P(batch):
            mm[bidx](a_tile=a[bidx], b_tile=b[bidx], c_tile=c[bidx])

    return wl()


def ragged_mark(arrs: dict, ragged: Ragged):
    """tests/test_codegen_ragged_axis.py: y[t] += 1 over a flattened ragged axis."""
    Y = T(arrs["y"], I32)

    @kernel
    def mark(y_tile: InOut[Tile[1, 1, I32]]):
        v = pto.load(y_tile)
        one = pto.constant(1.0, I32)
        pto.store(y_tile, pto.add(v, one))

    @workload
    def wl():
        for t in P.seq(ragged, name="t"):
            mark[t](y_tile=Y[t])

    return wl()


def sparse_mark(arrs: dict, sparse):
    """tests/test_codegen_select_sparse.py: y[e] += 1 for every selected index e of a CSR axis."""
    Y = T(arrs["y"], I32)

    @kernel
    def mark(y_tile: InOut[Tile[1, 1, I32]]):
        v = pto.load(y_tile)
        one = pto.constant(1.0, I32)
        pto.store(y_tile, pto.add(v, one))

    @workload
    def wl():
        for e in P.sel(sparse, name="e"):
            mark[e](y_tile=Y[e])

    return wl()


def rmsnorm_select(arrs: dict, sparse):
    """The quickstart rmsnorm tile over the selected rows e of X[rows, R, C] only."""
    x = arrs["x"]
    _, R, C = x.shape
    X, Y = T(arrs["x"]), T(arrs["y"])

    @kernel
    def rmsnorm_tile(x: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        inv = pto.rsqrt(pto.rowmean(pto.mul(x, x)))
        pto.store(out, pto.mul(x, inv))

    @workload
    def wl():
        for e in P.sel(sparse, name="e"):
            rmsnorm_tile[e](x=X[e], out=Y[e])

    return wl()


def sparse_symbols(sparse, outer: int, indptr, indices):
    """(symbols_u64, symbols_ptr) binding a CSR selection to ``sparse``'s runtime symbols,
    keyed by the FNV-1a-64 ids of ``outer_<id>`` / ``indptr_<id>`` / ``indices_<id>``."""
    from pto_wsp.program import Program

    sid = id(sparse)
    fnv = Program._fnv1a_64
    return ({fnv(f"outer_{sid}"): int(outer)},
            {fnv(f"indptr_{sid}"): np.asarray(indptr, np.int32), fnv(f"indices_{sid}"): np.asarray(indices, np.int32)})


# ---------------------------------------------------------------- numpy references (float64)
def rmsnorm_ref(x):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True))


def softmax_ref(x):
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- cond / slots / keyed dispatch
def cond_copy(arrs: dict, pred):
    """tests/test_codegen_cond.py: C[b] = A0[b] where pred, A1[b] otherwise, over P(Dense[B])."""
    B = arrs["c"].shape[0]
    R, C = arrs["c"].shape[2:]
    A0, A1, Cc = T(arrs["a0"]), T(arrs["a1"]), T(arrs["c"])

    @kernel
    def copy(src: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        pto.store(out, pto.load(src))

    @workload
    def wl():
        for b in P(Dense[B]()):
            with P.when(pred):
                copy[b](src=A0[b][0], out=Cc[b][0])
            with P.otherwise():
                copy[b](src=A1[b][0], out=Cc[b][0])

    return wl()


def slot_branch(arrs: dict):
    """tests/test_codegen_slots_tensor_predicate.py with compute kernels in place of its cpp_src
    bodies: flag <- src (a device kernel), slot 0 <- flag[0,0], then y = 7 if slot 0 != 0 else 3."""
    from pto_wsp.primitives import cond, sequential, slot_load_u64
    from pto_wsp.scalar_expr import slot_u64

    src, flag, y = T(arrs["src"], I32), T(arrs["flag"], I32), T(arrs["y"], I32)

    @kernel
    def write_flag(x_in: In[Tile[1, 1, I32]], flag_out: Out[Tile[1, 1, I32]]):
        pto.store(flag_out, pto.load(x_in))

    @kernel
    def fill_true(y_out: InOut[Tile[1, 1, I32]]):
        v = pto.load(y_out)
        pto.store(y_out, pto.add(pto.mul(v, pto.constant(0.0, I32)), pto.constant(7.0, I32)))

    @kernel
    def fill_false(y_out: InOut[Tile[1, 1, I32]]):
        v = pto.load(y_out)
        pto.store(y_out, pto.add(pto.mul(v, pto.constant(0.0, I32)), pto.constant(3.0, I32)))

    write = Workload("task", kernel=write_flag, params=[0], resources={"x_in": src[0][0], "flag_out": flag[0][0]})
    load = slot_load_u64(0, flag[0][0], row=0, col=0)
    t = Workload("task", kernel=fill_true, params=[0], resources={"y_out": y[0][0]})
    f = Workload("task", kernel=fill_false, params=[0], resources={"y_out": y[0][0]})
    return sequential(write, load, cond(slot_u64(0) != 0, t, f)).named("slot_tensor_predicate")


def masked_rmsnorm(arrs: dict, pred):
    """Quickstart rmsnorm over X[B, T, R, C] where pred(b, t) holds; other tiles of y are left
    as they are.  The predicate reads both grid loop variables."""
    x = arrs["x"]
    B, NT, R, C = x.shape
    X, Y = T(arrs["x"]), T(arrs["y"])

    @kernel
    def rmsnorm_tile(x: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        inv = pto.rsqrt(pto.rowmean(pto.mul(x, x)))
        pto.store(out, pto.mul(x, inv))

    @workload
    def wl():
        for b in P(Dense[B](), names=["b"]):
            for t in P(Dense[NT](), names=["t"]):
                with P.when(pred):
                    rmsnorm_tile[b, t](x=X[b][t], out=Y[b][t])

    return wl()


def slot_chain(arrs: dict):
    """Slot loads inside P(): for each b, slot 1 <- sel[b] (written by a kernel in the same run
    from src), then y[b] = x[b] * 2 if slot 1 is odd, else y[b] = x[b] + 1.  The P() loop
    must run as a host loop so each iteration sees its own slot value."""
    from pto_wsp.primitives import slot_load_u64
    from pto_wsp.scalar_expr import slot_i64

    n = arrs["x"].shape[0]
    X, Y, S, SEL = T(arrs["x"]), T(arrs["y"]), T(arrs["src"], I32), T(arrs["sel"], I32)

    @kernel
    def copy_sel(a: In[Tile[1, 1, I32]], o: Out[Tile[1, 1, I32]]):
        pto.store(o, pto.load(a))

    @kernel
    def twice(x: In[Tile[4, 8, F32]], y: Out[Tile[4, 8, F32]]):
        pto.store(y, pto.mul(x, pto.constant(2.0, F32)))

    @kernel
    def plus_one(x: In[Tile[4, 8, F32]], y: Out[Tile[4, 8, F32]]):
        pto.store(y, pto.add(x, pto.constant(1.0, F32)))

    @workload
    def wl():
        for b in P(Dense[n]()):
            copy_sel[b](a=S[b], o=SEL[b])
            slot_load_u64(1, SEL[b], 0, 0)
            with P.when((slot_i64(1) % 2) == 1):
                twice[b](x=X[b], y=Y[b])
            with P.otherwise():
                plus_one[b](x=X[b], y=Y[b])

    return wl()


def masked_bgemm(arrs: dict, pred, tm: int = 16, tn: int = 16, tk: int = 16, dtype=F16):
    """bgemm (InOut C, P.seq K loop) on the output tiles (b, m, n) where pred holds."""
    a, b_, c = arrs["a"], arrs["b"], arrs["c"]
    B, M, K = a.shape
    N = b_.shape[2]

    def perm(x, axes):
        return x.permute(*axes) if hasattr(x, "permute") else x.transpose(*axes)

    A = T(perm(a.reshape(B, M // tm, tm, K // tk, tk), (0, 1, 3, 2, 4)), dtype)
    Bm = T(perm(b_.reshape(B, K // tk, tk, N // tn, tn), (0, 3, 1, 2, 4)), dtype)
    C = T(perm(c.reshape(B, M // tm, tm, N // tn, tn), (0, 1, 3, 2, 4)))

    @kernel
    def gemm_tile(a_tile: In[Tile[tm, tk, dtype]], b_tile: In[Tile[tk, tn, dtype]], c_tile: InOut[Tile[tm, tn, F32]]):
        pto.store(c_tile, pto.add(c_tile, pto.matmul(a_tile, b_tile)))

    @workload
    def wl():
        for b, m, n in P(Dense[B](), Dense[M // tm](), Dense[N // tn](), names=["b", "m", "n"]):
            with P.when(pred):
                for k in P.seq(Dense[K // tk](), name="k"):
                    gemm_tile[b, m, n, k](a_tile=A[b][m][k], b_tile=Bm[b][n][k], c_tile=C[b][m][n])

    return wl()


# ---------------------------------------------------------------- cpp_src kernels
_FLAG_BODY = r"""
  // flag = 1 when x > 0, else 0 (one element each; strides from the descriptor)
  const float* xv = (const float*)task->tensor_ptrs[0];
  int32_t* fv = (int32_t*)task->tensor_ptrs[1];
  fv[0] = xv[0] > 0.0f ? 1 : 0;
#if defined(__CPU_SIM)
  pto::cpu_sim::add_cycles(1);
#endif
"""


def _fill_body(value: int) -> str:
    return f"""
  int32_t* yv = (int32_t*)task->tensor_ptrs[0];
  yv[0 * (int64_t)task->tensor_strides[0] + 0 * (int64_t)task->tensor_strides[1]] = {value};
#if defined(__CPU_SIM)
  pto::cpu_sim::add_cycles(1);
#endif
"""


def cpp_slot_branch(arrs: dict):
    """tests/test_codegen_slots_tensor_predicate.py with cpp_src bodies of this repository's own:
    flag <- (x > 0), slot 0 <- flag, y = 7 if slot 0 != 0 else 3; each body adds 1 cycle."""
    from pto_wsp.primitives import cond, sequential, slot_load_u64
    from pto_wsp.scalar_expr import slot_u64

    x, flag, y = T(arrs["x"]), T(arrs["flag"], I32), T(arrs["y"], I32)

    @kernel(cpp_src=_FLAG_BODY)
    def write_flag(x_in: In[Tile[1, 1, F32]], flag_out: Out[Tile[1, 1, I32]]):
        pass

    @kernel(cpp_src=_fill_body(7))
    def fill_true(y_out: Out[Tile[1, 1, I32]]):
        pass

    @kernel(cpp_src=_fill_body(3))
    def fill_false(y_out: Out[Tile[1, 1, I32]]):
        pass

    write = Workload("task", kernel=write_flag, params=[0], resources={"x_in": x[0][0], "flag_out": flag[0][0]})
    load = slot_load_u64(0, flag[0][0], row=0, col=0)
    t = Workload("task", kernel=fill_true, params=[0], resources={"y_out": y[0][0]})
    f = Workload("task", kernel=fill_false, params=[0], resources={"y_out": y[0][0]})
    return sequential(write, load, cond(slot_u64(0) != 0, t, f)).named("slot_tensor_predicate")


_PROBE_BODY = r"""
  // Writes what the task descriptor holds into its output tile (row 0: args;
  // row 1: num_axis_args, num_tensors, x's strides, x[0,0] + x[1,0]).
  const float* xv = (const float*)task->tensor_ptrs[0];
  float* ov = (float*)task->tensor_ptrs[1];
  const uint64_t os3 = task->tensor_strides[2], os4 = task->tensor_strides[3];
  for (uint32_t j = 0; j < task->num_args && j < 16; ++j) ov[j * os4] = (float)task->args[j];
  ov[os3 + 0 * os4] = (float)task->num_axis_args;
  ov[os3 + 1 * os4] = (float)task->num_tensors;
  ov[os3 + 2 * os4] = (float)task->tensor_strides[0];
  ov[os3 + 3 * os4] = (float)task->tensor_strides[1];
  ov[os3 + 4 * os4] = xv[0] + xv[task->tensor_strides[0]];
  cycles = 5 + task->args[0] * 3 + task->args[1] + 100 * task->args[2];
"""


# The same probe as a whole translation unit (@kernel(cpp_tu_path=...)): the entry has the
# kernel's name, a helper function without annotations computes the sum, and the cycles go
# through pto::cpu_sim's counter.
PROBE_TU = r"""
#include "pto/wsp/codegen/abi/kernel_abi.hpp"
#include "pto/wsp/codegen/abi/ptoisa_bridge.hpp"
#include <cstdint>
#include <cstddef>

static float column_pair(const float* x, uint64_t s3) { return x[0] + x[s3]; }

extern "C" PTO_WSP_KERNEL_ATTR uint64_t probe(const KernelTaskDesc* task, CSPTContext* cspt) {
  (void)cspt;
  const float* xv = (const float*)task->tensor_ptrs[0];
  float* ov = (float*)task->tensor_ptrs[1];
  const uint64_t os3 = task->tensor_strides[2], os4 = task->tensor_strides[3];
  for (uint32_t j = 0; j < task->num_args && j < 16; ++j) ov[j * os4] = (float)task->args[j];
  ov[os3 + 0 * os4] = (float)task->num_axis_args;
  ov[os3 + 1 * os4] = (float)task->num_tensors;
  ov[os3 + 2 * os4] = (float)task->tensor_strides[0];
  ov[os3 + 3 * os4] = (float)task->tensor_strides[1];
  ov[os3 + 4 * os4] = column_pair(xv, task->tensor_strides[0]);
  pto::cpu_sim::reset_cycles();
  pto::cpu_sim::add_cycles(5 + task->args[0] * 3);
  pto::cpu_sim::add_cycles(task->args[1] + 100 * task->args[2]);
  return pto::cpu_sim::read_cycles();
}
"""


def cpp_probe(arrs: dict, pred=None, tu_path: str | None = None):
    """A cpp_src kernel over a host P.seq loop (i) around a P() grid (b, h), with a scalar arg;
    with `pred`, only the grid tasks where it holds run; with `tu_path` (a file holding
    PROBE_TU) the kernel is that translation unit instead."""
    from pto_wsp import Scalar

    X, O = T(arrs["x"]), T(arrs["o"])
    nb, nh = arrs["x"].shape[:2]
    ni = arrs["o"].shape[0]
    opts = {"cpp_tu_path": tu_path} if tu_path else {"cpp_src": _PROBE_BODY}

    @kernel(**opts)
    def probe(x: In[Tile[2, 4, F32]], out: Out[Tile[2, 16, F32]], s: Scalar[F32] = 1.5):
        pass

    @workload
    def wl():
        for i in P.seq(Dense[ni](), name="i"):
            for b, h in P(Dense[nb](), Dense[nh](), names=["b", "h"]):
                if pred is None:
                    probe[b, h, i](x=X[b][h], out=O[i][b][h], s=2.5)
                else:
                    with P.when(pred):
                        probe[b, h, i](x=X[b][h], out=O[i][b][h], s=2.5)

    return wl()


# ---------------------------------------------------------------- op variants of the arithmetic contract
# Broadcast operand shapes for binary(): the rhs tile of out = op(x, y) with x [R, C].
BIN_SHAPES = {"same": lambda R, C: (R, C), "row": lambda R, C: (R, 1), "row_t": lambda R, C: (1, R),
              "col": lambda R, C: (1, C), "col_t": lambda R, C: (C, 1)}
BIN_OPS = {"add": "add", "sub": "sub", "mul": "mul", "div": "div", "max": "max", "min": "min"}


def binary(arrs: dict, op: str, out_dtype=F32):
    """out[b][t] = op(x[b][t], y[b][t]) over X[B, T, R, C] and Y[B, T, yr, yc]: TADD..TMIN on equal
    shapes, TROWEXPAND* for a [R,1] / [1,R] rhs, TCOLEXPAND{SUB,MUL,DIV} for [1,C] / [C,1]
    (src/python/pto_codegen.cpp:1078-1107).  out_dtype F16 / BF16 adds the TCVT store cast
    (:955-976) and moves the kernel onto the tile program."""
    x, y = arrs["x"], arrs["y"]
    B, NT, R, C = x.shape
    yr, yc = y.shape[2:]
    X, Y, O = T(x), T(y), T(arrs["out"], out_dtype)
    fn = getattr(pto, BIN_OPS[op])

    @kernel
    def bin_tile(x_t: In[Tile[R, C, F32]], y_t: In[Tile[yr, yc, F32]], out: Out[Tile[R, C, out_dtype]]):
        pto.store(out, fn(x_t, y_t))

    @workload
    def wl():
        for b in P(Dense[B]()):
            for t in P(Dense[NT]()):
                bin_tile[b, t](x_t=X[b][t], y_t=Y[b][t], out=O[b][t])

    return wl()


def scalar_binary(arrs: dict, op: str, value: float, left: bool = False, out_dtype=F32):
    """out = op(x, s) with s = pto.constant(value): TADDS / TSUBS / TMULS / TDIVS / TMAXS / TMINS
    (src/python/pto_codegen.cpp:1008-1051).  left=True builds op(s, x) with a tile result; the
    tracer types a binary op by its first operand, so that form is written against the kernel IR
    directly (the reference's emitter lowers it to TDIVS(dst, s, tile) for Div)."""
    from pto_wsp.kernel import OpKind, Value, ValueId

    x = arrs["x"]
    B, NT, R, C = x.shape
    X, O = T(x), T(arrs["out"], out_dtype)
    kind = {"add": OpKind.Add, "sub": OpKind.Sub, "mul": OpKind.Mul, "div": OpKind.Div, "max": OpKind.Max,
            "min": OpKind.Min}[op]

    @kernel
    def scal_tile(x_t: In[Tile[R, C, F32]], out: Out[Tile[R, C, out_dtype]]):
        s = pto.constant(value, F32)
        if left:
            r = Value(ValueId.next(), F32, (R, C))
            pto._ir().add_op(kind, [s, x_t], r)
        else:
            r = getattr(pto, BIN_OPS[op])(x_t, s)
        pto.store(out, r)

    @workload
    def wl():
        for b in P(Dense[B]()):
            for t in P(Dense[NT]()):
                scal_tile[b, t](x_t=X[b][t], out=O[b][t])

    return wl()


def store_cast(arrs: dict, out_dtype, via_tile: bool = False):
    """out (F16 / BF16 tile) = x (f32 tile): the TCVT CAST_RINT store (src/python/pto_codegen.cpp:955-976).
    via_tile=True adds a [R, 2C] input and an op on it whose result nothing reads: the kernel's
    tiles then share no row shape, so the cast runs on the tile program instead of a row program."""
    x = arrs["x"]
    B, NT, R, C = x.shape
    X, O = T(x), T(arrs["out"], out_dtype)

    if via_tile:
        WD = T(np.zeros((B, NT, R, 2 * C), np.float32) if isinstance(x, np.ndarray) else
               __import__("torch").zeros((B, NT, R, 2 * C), device=x.device))

        @kernel
        def cast_tile(x_t: In[Tile[R, C, F32]], wide: In[Tile[R, 2 * C, F32]], out: Out[Tile[R, C, out_dtype]]):
            pto.max(wide, wide)
            pto.store(out, x_t)

        @workload
        def wl():
            for b in P(Dense[B]()):
                for t in P(Dense[NT]()):
                    cast_tile[b, t](x_t=X[b][t], wide=WD[b][t], out=O[b][t])

        return wl()

    @kernel
    def cast_tile(x_t: In[Tile[R, C, F32]], out: Out[Tile[R, C, out_dtype]]):
        pto.store(out, x_t)

    @workload
    def wl():
        for b in P(Dense[B]()):
            for t in P(Dense[NT]()):
                cast_tile[b, t](x_t=X[b][t], out=O[b][t])

    return wl()


def f16_from_bits(h: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(h).view(np.float16)


def bf16_rne_by_distance(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits by comparing distances to the two neighbouring bf16 values in float64
    (exact for finite f32 inputs); ties go to the even mantissa.  A restatement independent of
    the add-and-shift bit trick, for finite inputs whose rounding stays finite."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32)
    lo = (u >> 16).astype(np.uint32)           # truncation toward zero (same sign)
    hi = lo + 1                                # next bf16 away from zero
    vlo = (lo << 16).view(np.float32).astype(np.float64)
    vhi = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    dlo, dhi = ax - np.abs(vlo), np.abs(vhi) - ax
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (lo & 1 == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def rounding_probe_f32(n_random: int, seed: int = 0, for_bf16: bool = False) -> np.ndarray:
    """f32 values that separate rounding rules: exact halfway cases between neighbours of both
    parities and both signs, values just either side of a halfway point, signed zeros, f16
    subnormals and the f16 overflow boundary, then random values over a wide exponent range."""
    vals = []
    if for_bf16:
        for m in range(0, 128, 7):            # bf16 mantissas of both parities
            base = np.float32(1.0 + m / 128.0)
            ulp = np.float32(2.0 ** -7)
            half = np.float32(base + ulp / 2)  # exactly between base and base + ulp
            vals += [half, -half, np.nextafter(half, np.float32(0)), np.nextafter(half, np.float32(9))]
            vals += [np.float32(half * 2.0 ** 20), np.float32(half * 2.0 ** -30)]
    else:
        for m in range(0, 1024, 37):          # f16 mantissas of both parities
            base = np.float32(1.0 + m / 1024.0)
            ulp = np.float32(2.0 ** -10)
            half = np.float32(base + ulp / 2)
            vals += [half, -half, np.nextafter(half, np.float32(0)), np.nextafter(half, np.float32(9))]
            vals += [np.float32(half * 2.0 ** 10), np.float32(half * 2.0 ** -12)]
        vals += [np.float32(2.0 ** -24), np.float32(2.0 ** -25), np.float32(1.5 * 2.0 ** -25), np.float32(3 * 2.0 ** -26),
                 np.float32(2.0 ** -14), np.float32(2.0 ** -14 - 2.0 ** -25), np.float32(65504.0), np.float32(65519.0),
                 np.float32(65520.0), np.float32(-65520.0), np.float32(1e6), np.float32(2.0 ** -30)]
    vals += [np.float32(0.0), np.float32(-0.0), np.float32(1.0), np.float32(-1.0)]
    rng = np.random.default_rng(seed)
    lim = 12 if not for_bf16 else 60
    rand = (rng.standard_normal(n_random) * np.exp2(rng.integers(-lim, lim, n_random))).astype(np.float32)
    return np.concatenate([np.asarray(vals, np.float32), rand])


# ---------------------------------------------------------------- @ptoisa_kernel
def rr2(w, window: int):
    """round_robin(2) + a STALL window: the schedule of tests/test_ptoisa_kernel_jit.py:45-48, 85-88."""
    return w.dispatch(DispatchPolicy.round_robin(num_aicpus=2)).task_graph(
        window=TaskWindow(window, "tasks", WindowMode.STALL))


def ptoisa_square(arrs: dict):
    """Y[t][0] = X[t][0] * X[t][0] over X[NT, 1, R, C] with tload / TMUL / tstore
    (tests/test_ptoisa_kernel_jit.py:22-54)."""
    from pto_wsp import ptoisa, ptoisa_kernel

    x = arrs["x"]
    NT, _, R, C = x.shape
    X, Y = T(x), T(arrs["y"])

    @ptoisa_kernel
    def square(src: In[Tile[R, C, F32]], dst: Out[Tile[R, C, F32]]):
        a = ptoisa.tload(src)
        b = ptoisa.TMUL(a, a)
        ptoisa.tstore(dst, b)

    @workload
    def wl():
        for t in P(Dense[NT]()):
            square[t](src=X[t][0], dst=Y[t][0])

    return wl()


def ptoisa_topk(arrs: dict, k: int = 8):
    """out[b][t][0, :k] = the indices of the k largest of scores[b][t] ([1,32] f32) with
    iota_u32 / TSORT32 / store_topk_indices_i32 (tests/test_ptoisa_kernel_jit.py:57-95)."""
    from pto_wsp import ptoisa, ptoisa_kernel

    s, o = arrs["scores"], arrs["out"]
    B, NT = s.shape[:2]
    S, O = T(s), T(o, I32)
    oc = o.shape[-1]

    @ptoisa_kernel
    def topk(scores: In[Tile[1, 32, F32]], out_idx: Out[Tile[1, oc, I32]]):
        sv = ptoisa.tload(scores)
        idx = ptoisa.iota_u32(32)
        pairs = ptoisa.TSORT32(sv, idx)
        ptoisa.store_topk_indices_i32(out_idx, pairs, k)

    @workload
    def wl():
        for b in P(Dense[B]()):
            for t in P(Dense[NT]()):
                topk[b, t](scores=S[b][t], out_idx=O[b][t])

    return wl()


def pto_topk(arrs: dict, k: int = 8):
    """The same top-k through the pto.* tracer: pto.iota_u32 / pto.tsort32 /
    pto.extract_topk_indices and a store of the [1,k] i32 tile."""
    s, o = arrs["scores"], arrs["out"]
    B, NT = s.shape[:2]
    S, O = T(s), T(o, I32)

    @kernel
    def topk_tile(scores: In[Tile[1, 32, F32]], out_idx: Out[Tile[1, k, I32]]):
        pairs = pto.tsort32(scores, pto.iota_u32(32))
        pto.store(out_idx, pto.extract_topk_indices(pairs, k))

    @workload
    def wl():
        for b in P(Dense[B]()):
            for t in P(Dense[NT]()):
                topk_tile[b, t](scores=S[b][t], out_idx=O[b][t])

    return wl()


def ptoisa_mix(arrs: dict, extra_cycles: int = 7):
    """A chain of the other PTO-ISA instructions over X[B, R, C] (f32) with a
    per-row m[B, R, 1], a per-column g[B, 1, C] and a Scalar[F32] divisor:
    out = TMAX(TMOV(TDIVS(TCOLEXPANDMUL(TROWEXPANDSUB(x, m), g), s)), TMAXS(x, -0.5)) + TADDS(x, 2)
    plus cpu_sim_add_cycles(extra_cycles)."""
    from pto_wsp import ptoisa, ptoisa_kernel

    x = arrs["x"]
    B, R, C = x.shape
    X, M, G, O = T(x), T(arrs["m"]), T(arrs["g"]), T(arrs["out"])
    s_val = float(arrs["s"])

    @ptoisa_kernel
    def mix(x_t: In[Tile[R, C, F32]], m_t: In[Tile[R, 1, F32]], g_t: In[Tile[1, C, F32]], s: Scalar[F32],
            out: Out[Tile[R, C, F32]]):
        a = ptoisa.tload(x_t)
        m = ptoisa.tload(m_t)
        g = ptoisa.tload(g_t)
        y = ptoisa.TMOV(ptoisa.TDIVS(ptoisa.TCOLEXPANDMUL(ptoisa.TROWEXPANDSUB(a, m), g), s))
        z = ptoisa.TADD(ptoisa.TMAX(y, ptoisa.TMAXS(a, -0.5)), ptoisa.TADDS(a, 2))
        ptoisa.cpu_sim_add_cycles(extra_cycles)
        ptoisa.tstore(out, z)

    @workload
    def wl():
        for b in P(Dense[B]()):
            mix[b](x_t=X[b], m_t=M[b], g_t=G[b], s=s_val, out=O[b])

    return wl()


def ptoisa_unary(arrs: dict):
    """out = TRSQRT(TEXP(x)) over X[B, R, C] (f32)."""
    from pto_wsp import ptoisa, ptoisa_kernel

    x = arrs["x"]
    B, R, C = x.shape
    X, O = T(x), T(arrs["out"])

    @ptoisa_kernel
    def unary(x_t: In[Tile[R, C, F32]], out: Out[Tile[R, C, F32]]):
        ptoisa.tstore(out, ptoisa.TRSQRT(ptoisa.TEXP(ptoisa.tload(x_t))))

    @workload
    def wl():
        for b in P(Dense[B]()):
            unary[b](x_t=X[b], out=O[b])

    return wl()


# ---------------------------------------------------------------- overlapping output views
def conflict_accumulate(arrs: dict, shared_all: bool = False):
    """out[b][v] += x[b][s][v] over P(b) x P(s) x P(v) (X[B, S, V, R, C], O[B, V, R, C]):
    tasks that differ only in s write the same out tile, so the result depends on the
    program order; the launch runs the groups (b, v) in parallel, s in order within
    each.  shared_all: every task writes out[0][0] (one group)."""
    x = arrs["x"]
    B, S, V, R, C = x.shape
    X, O = T(x), T(arrs["out"])

    @kernel
    def acc_tile(x_t: In[Tile[R, C, F32]], o_t: InOut[Tile[R, C, F32]]):
        pto.store(o_t, pto.add(o_t, x_t))

    @workload
    def wl():
        for b in P(Dense[B]()):
            for s in P(Dense[S]()):
                for v in P(Dense[V]()):
                    if shared_all:
                        acc_tile[b, s, v](x_t=X[b][s][v], o_t=O[0][0])
                    else:
                        acc_tile[b, s, v](x_t=X[b][s][v], o_t=O[b][v])

    return wl()


def conflict_accumulate_ref(x: np.ndarray, out: np.ndarray, shared_all: bool = False) -> np.ndarray:
    """The same sums in program order, one float32 add at a time."""
    r = out.copy()
    B, S, V = x.shape[:3]
    for b in range(B):
        for s in range(S):
            for v in range(V):
                if shared_all:
                    r[0, 0] = r[0, 0] + x[b, s, v]
                else:
                    r[b, v] = r[b, v] + x[b, s, v]
    return r


# ---------------------------------------------------------------- deepseek lightning indexer
def lightning_inputs(seed: int = 0, bsz: int = 2, tiles: int = 4, cand: int = 32):
    """examples/deepseek_lightning_indexer/golden.py:28-38: N(0,1) scores and one effective
    sequence length per (b, s) drawn from the four tiers."""
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((bsz, tiles, cand), dtype=np.float32)
    eff_seq = rng.choice(np.array([512, 4096, 16384, 131072], dtype=np.uint64), size=(bsz, tiles, 1, 1), replace=True)
    return scores, eff_seq


def stable_topk_desc(scores: np.ndarray, k: int) -> np.ndarray:
    """examples/deepseek_lightning_indexer/golden.py:6-25: per row, descending score with the
    lower index first on ties."""
    B, S, C = scores.shape
    out = np.empty((B, S, k), np.int32)
    idx = np.arange(C)
    for b in range(B):
        for s in range(S):
            out[b, s] = np.lexsort((idx, -scores[b, s].astype(np.float64)))[:k]
    return out


def lightning_indexer(scores: np.ndarray, eff_seq: np.ndarray, out_idx: np.ndarray, impl: str):
    """examples/deepseek_lightning_indexer/pto_wsp_impl.py:30-150: a slot loaded from EffSeq[b][s]
    picks one of four tiers (pad_to 2048 / 8192 / 65536 / 131072) and the top-8 of the 32
    candidates is taken with TSORT32; impl "pto" traces pto.* ops, "ptoisa" the PTO-ISA calls
    with the tier cost as cpu_sim_add_cycles of a C expression of pad_to."""
    from pto_wsp import ptoisa, ptoisa_kernel
    from pto_wsp.primitives import slot_load_u64
    from pto_wsp.scalar_expr import slot_u64

    bsz, tiles, cand = scores.shape
    Scores = Tensor(data=scores.reshape(bsz, tiles, 1, cand), shape=(bsz, tiles, 1, cand), dtype=F32)
    EffSeq = Tensor(data=eff_seq, shape=eff_seq.shape, dtype=DType.U64)
    OutIdx = Tensor(data=out_idx, shape=out_idx.shape, dtype=I32)

    @kernel
    def topk8_sort32_pto(scores_tile: In[Tile[1, 32, F32]], out_idx_tile: Out[Tile[1, 8, I32]], pad_to: Scalar[I32]):
        idx = pto.iota_u32(32)
        pairs = pto.tsort32(scores_tile, idx)
        pto.store(out_idx_tile, pto.extract_topk_indices(pairs, 8))

    @ptoisa_kernel
    def topk8_sort32(scores_tile: In[Tile[1, 32, F32]], out_idx_tile: Out[Tile[1, 8, I32]], pad_to: Scalar[I32]):
        s = ptoisa.tload(scores_tile)
        pairs = ptoisa.TSORT32(s, ptoisa.iota_u32(32))
        ptoisa.store_topk_indices_i32(out_idx_tile, pairs, 8)
        ptoisa.cpu_sim_add_cycles(f"(({pad_to.debug_name} > 32) ? ((uint64_t)({pad_to.debug_name} / 32) * 128ull) : 0ull)")

    topk = topk8_sort32_pto if impl == "pto" else topk8_sort32

    @workload
    def wl():
        for b in P(Dense[bsz]()):
            for s in P(Dense[tiles]()):
                slot_load_u64(0, EffSeq[b][s], row=0, col=0)
                with P.when(slot_u64(0) <= 2048):
                    topk[b, s](scores_tile=Scores[b][s], out_idx_tile=OutIdx[b][s], pad_to=2048)
                with P.otherwise():
                    with P.when(slot_u64(0) <= 8192):
                        topk[b, s](scores_tile=Scores[b][s], out_idx_tile=OutIdx[b][s], pad_to=8192)
                    with P.otherwise():
                        with P.when(slot_u64(0) <= 65536):
                            topk[b, s](scores_tile=Scores[b][s], out_idx_tile=OutIdx[b][s], pad_to=65536)
                        with P.otherwise():
                            topk[b, s](scores_tile=Scores[b][s], out_idx_tile=OutIdx[b][s], pad_to=131072)

    return (wl().dispatch(DispatchPolicy.affinity(lambda t: t.get("b"), num_aicpus=4))
            .task_graph(window=TaskWindow(1024, "tasks", WindowMode.STALL)))


# ---------------------------------------------------------------- llama / deepseek_v3 / tensor_data examples
def llama_block(x: np.ndarray, w1: np.ndarray, w2: np.ndarray, out: np.ndarray, tile_seq: int, eps: float):
    """examples/llama/pto_wsp_impl.py:21-118: per seq tile, attention (q = k = v = x), residual
    add, rmsnorm (eps), ReLU MLP, residual add, as five kernels in one P() body."""
    seq, d = x.shape
    st = seq // tile_seq
    mlp = w1.shape[1]
    xt = x.reshape(st, tile_seq, d).astype(np.float32)
    X, KT = T(xt), T(xt.transpose(0, 2, 1))
    W1, W2 = T(w1.astype(np.float32)), T(w2.astype(np.float32))
    O = T(out.reshape(st, tile_seq, d))
    Xn, Attn, Res1, Mlp = (T(np.zeros_like(xt)) for _ in range(4))

    @kernel
    def rmsnorm_tile(x: In[Tile[tile_seq, d, F32]], out: Out[Tile[tile_seq, d, F32]]):
        inv = pto.rsqrt(pto.add(pto.rowmean(pto.mul(x, x)), pto.constant(eps, F32)))
        pto.store(out, pto.mul(x, inv))

    @kernel
    def attn_tile(q: In[Tile[tile_seq, d, F32]], k_t: In[Tile[d, tile_seq, F32]], v: In[Tile[tile_seq, d, F32]],
                  out: Out[Tile[tile_seq, d, F32]]):
        s = pto.mul(pto.matmul(q, k_t), pto.constant(1.0 / math.sqrt(d), F32))
        e = pto.exp(pto.sub(s, pto.rowmax(s)))
        pto.store(out, pto.matmul(pto.div(e, pto.rowsum(e)), v))

    @kernel
    def add_tile(a: In[Tile[tile_seq, d, F32]], b: In[Tile[tile_seq, d, F32]], out: Out[Tile[tile_seq, d, F32]]):
        pto.store(out, pto.add(a, b))

    @kernel
    def mlp_tile(x: In[Tile[tile_seq, d, F32]], w1: In[Tile[d, mlp, F32]], w2: In[Tile[mlp, d, F32]],
                 out: Out[Tile[tile_seq, d, F32]]):
        h = pto.matmul(x, w1)
        pto.store(out, pto.matmul(pto.max(h, pto.constant(0.0, F32)), w2))

    @workload
    def wl():
        for s in P(Dense[st]()):
            attn_tile[s](q=X[s], k_t=KT[s], v=X[s], out=Attn[s])
            add_tile[s](a=X[s], b=Attn[s], out=Res1[s])
            rmsnorm_tile[s](x=Res1[s], out=Xn[s])
            mlp_tile[s](x=Xn[s], w1=W1, w2=W2, out=Mlp[s])
            add_tile[s](a=Res1[s], b=Mlp[s], out=O[s])

    return rr4(wl())


def llama_block_ref(x, w1, w2, tile_seq, eps):
    """examples/llama/golden.py:7-35 in float64."""
    out = np.zeros(x.shape, np.float64)
    d = x.shape[1]
    for t in range(x.shape[0] // tile_seq):
        xt = x[t * tile_seq:(t + 1) * tile_seq].astype(np.float64)
        s = (xt @ xt.T) / math.sqrt(d)
        e = np.exp(s - s.max(-1, keepdims=True))
        res1 = xt + (e / e.sum(-1, keepdims=True)) @ xt
        xn = res1 / np.sqrt((res1 * res1).mean(-1, keepdims=True) + eps)
        out[t * tile_seq:(t + 1) * tile_seq] = res1 + np.maximum(xn @ w1, 0.0) @ w2
    return out


def moe_block(x: np.ndarray, w0: np.ndarray, w1: np.ndarray, g: np.ndarray, y: np.ndarray):
    """examples/deepseek_v3/pto_wsp_impl.py:20-95: two expert matmuls and a gated mix
    y = g * (x @ w0) + (1 - g) * (x @ w1) per 8-row seq tile."""
    seq, d = x.shape
    ts = 8
    st = seq // ts
    xt = x.reshape(st, ts, d).astype(np.float32)
    X, G = T(xt), T(g.reshape(st, ts, 1).astype(np.float32))
    W0, W1, Y = T(w0.astype(np.float32)), T(w1.astype(np.float32)), T(y.reshape(st, ts, d))
    E0, E1 = T(np.zeros_like(xt)), T(np.zeros_like(xt))

    @kernel
    def expert_linear(x: In[Tile[ts, d, F32]], w: In[Tile[d, d, F32]], out: Out[Tile[ts, d, F32]]):
        pto.store(out, pto.matmul(x, w))

    @kernel
    def moe_mix(e0: In[Tile[ts, d, F32]], e1: In[Tile[ts, d, F32]], g: In[Tile[ts, 1, F32]], out: Out[Tile[ts, d, F32]]):
        g1 = pto.add(pto.mul(g, pto.constant(-1.0, F32)), pto.constant(1.0, F32))
        pto.store(out, pto.add(pto.mul(e0, g), pto.mul(e1, g1)))

    @workload
    def wl():
        for s in P(Dense[st]()):
            expert_linear[s](x=X[s], w=W0, out=E0[s])
            expert_linear[s](x=X[s], w=W1, out=E1[s])
            moe_mix[s](e0=E0[s], e1=E1[s], g=G[s], out=Y[s])

    return rr4(wl())


def add_tiles5(a: np.ndarray, b: np.ndarray, c: np.ndarray):
    """examples/tensor_data/pto_wsp_impl.py:20-66: C = A + B over [B, TM, TN, R, C] tiles."""
    nb, tm, tn, r, cc = a.shape
    A, B, C = T(a), T(b), T(c)

    @kernel
    def add_tiles(a_tile: In[Tile[r, cc, F32]], b_tile: In[Tile[r, cc, F32]], c_tile: Out[Tile[r, cc, F32]]):
        pto.store(c_tile, pto.add(a_tile, b_tile))

    @workload
    def wl():
        for bb in P(Dense[nb]()):
            for i in P(Dense[tm]()):
                for j in P(Dense[tn]()):
                    add_tiles[bb, i, j](a_tile=A[bb][i][j], b_tile=B[bb][i][j], c_tile=C[bb][i][j])

    return rr4(wl())


def square_tiles4(x: np.ndarray, y: np.ndarray):
    """examples/tensor_data/pto_wsp_impl.py:69-107: Y = X * X over [B, T, R, C] tiles."""
    nb, nt, r, cc = x.shape
    X, Y = T(x), T(y)

    @kernel
    def square_tile(in_tile: In[Tile[r, cc, F32]], out_tile: Out[Tile[r, cc, F32]]):
        pto.store(out_tile, pto.mul(in_tile, in_tile))

    @workload
    def wl():
        for bb in P(Dense[nb]()):
            for t in P(Dense[nt]()):
                square_tile[bb, t](in_tile=X[bb][t], out_tile=Y[bb][t])

    return rr4(wl())
