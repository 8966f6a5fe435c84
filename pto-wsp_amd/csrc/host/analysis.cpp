// Kernel analysis.  The validation rules and the cycle cost restate the
// reference's kernel emitter (src/python/pto_codegen.cpp:350-1241) and the
// cpu_sim cycle wrappers (include/pto/wsp/codegen/abi/ptoisa_bridge.hpp:54-303):
// every tile op costs valid_rows*valid_cols of its destination, TMATMUL costs
// m*k*n, TROWSUM/TROWMAX cost the rows of the [rows,1] result and RowMean adds
// a TDIVS of the same size.  Valid dims always equal the static tile shapes,
// because the workload emitter passes the static shapes as tail arguments
// (src/python/pto_codegen.cpp:2507-2545).
#include "analysis.hpp"

#include <functional>
#include <map>
#include <set>

#include <algorithm>

namespace ptowsp {

namespace {

[[noreturn]] void refuse(const KernelDef& k, const std::string& msg) {
    throw CompileError("kernel " + k.name + ": " + msg);
}

uint64_t rc(const ValueInfo* v) { return static_cast<uint64_t>(v->rows) * static_cast<uint64_t>(v->cols); }

bool is_binary(OpKind k) {
    return k == OpKind::Add || k == OpKind::Sub || k == OpKind::Mul || k == OpKind::Div || k == OpKind::Max ||
           k == OpKind::Min;
}

bool is_int(DType d) { return !dtype_is_float(d); }

// Row-program classification (see analysis.hpp).  Returns false with a
// reason when the kernel does not decompose into independent rows.
bool classify_rows(const KernelDef& k, KernelAnalysis& a) {
    auto no = [&](const std::string& why) {
        a.not_row_reason = why;
        return false;
    };
    for (const auto& op : k.ops) {
        if (op.kind == OpKind::Matmul) return no("matmul");
        if (op.kind == OpKind::IotaU32 || op.kind == OpKind::TSort32 || op.kind == OpKind::ExtractTopkIndices ||
            op.kind == OpKind::StoreTopkIndices)
            return no("top-k ops");
    }
    // A 16-bit float param that is only ever a Store destination receives
    // the store cast; every value of the program stays f32.
    auto cast_out = [&](const ValueInfo& v) {
        if ((v.dtype != DType::F16 && v.dtype != DType::BF16) || a.param_of[v.id] < 0 || a.preload[v.id]) return false;
        for (const auto& op : k.ops)
            for (size_t j = 0; j < op.operands.size(); ++j)
                if (op.operands[j] == v.id && !(op.kind == OpKind::Store && j == 0)) return false;
        return true;
    };
    int R = 0, C = 0;
    for (const auto& v : k.values) {
        if (!v.tile) continue;
        if (v.dtype != DType::F32 && !cast_out(v)) return no("non-f32 tile");
        if (v.cols > C || (v.cols == C && v.rows > R)) {
            C = v.cols;
            R = v.rows;
        }
    }
    if (C == 0) return no("no tiles");
    a.rows = R;
    a.cols = C;
    a.row_class.assign(a.max_id + 1, RowClass::None);
    auto shape_is = [](const ValueInfo* v, int r, int c) { return v->rows == r && v->cols == c; };

    // Uses of each value as a broadcast operand, to tell [1,C] col vectors
    // from other [1,*] tiles.
    std::vector<int> bcast_row(a.max_id + 1, 0), bcast_col(a.max_id + 1, 0), other_use(a.max_id + 1, 0);
    for (size_t i = 0; i < k.ops.size(); ++i) {
        const auto& op = k.ops[i];
        for (size_t j = 0; j < op.operands.size(); ++j) {
            int id = op.operands[j];
            if (is_binary(op.kind) && j == 1 && a.bin_mode[i] == BinMode::RowExpand) bcast_row[id]++;
            else if (is_binary(op.kind) && j == 1 && a.bin_mode[i] == BinMode::ColExpand) bcast_col[id]++;
            else if (!(op.kind == OpKind::Store && j == 0) && op.kind != OpKind::TMov && op.kind != OpKind::Load)
                other_use[id]++;
        }
    }
    auto base_class = [&](const ValueInfo* v) -> RowClass {
        if (C > 1 && shape_is(v, R, C)) return RowClass::Full;
        if (shape_is(v, R, 1)) return RowClass::RowVec;
        if (R > 1 && v->rows == 1 && v->cols == R && bcast_row[v->id] && !other_use[v->id]) return RowClass::RowVecT;
        if (R > 1 && v->rows == 1 && v->cols == C && bcast_col[v->id] && !other_use[v->id] && !bcast_row[v->id])
            return RowClass::ColVec;
        if (C > 1 && v->rows == C && v->cols == 1 && bcast_col[v->id] && !other_use[v->id] && !bcast_row[v->id])
            return RowClass::ColVecT;
        return RowClass::None;
    };
    for (const auto& v : k.values) {
        if (!v.tile) {
            a.row_class[v.id] = RowClass::Scalar;
            continue;
        }
        RowClass c = base_class(&v);
        // A param tile read only through Load ops (or only stored to) is no
        // value of the program (its Load results are): its class only
        // records its shape, and one that fits no class is no obstacle.
        if (a.param_of[v.id] >= 0 && !a.preload[v.id]) {
            a.row_class[v.id] = c;
            continue;
        }
        if (c == RowClass::None)
            return no("tile " + std::to_string(v.id) + " of shape " + std::to_string(v.rows) + "x" +
                      std::to_string(v.cols) + " does not fit rows of " + std::to_string(R) + "x" + std::to_string(C));
        bool from_param = a.param_of[v.id] >= 0;
        bool from_load = false;
        for (const auto& op : k.ops)
            if (op.kind == OpKind::Load && op.result == v.id) from_load = true;
        if ((c == RowClass::RowVecT || c == RowClass::ColVec || c == RowClass::ColVecT) && !from_param && !from_load)
            return no("computed broadcast vector");
        a.row_class[v.id] = c;
    }
    for (size_t i = 0; i < k.ops.size(); ++i) {
        const auto& op = k.ops[i];
        if (op.kind == OpKind::Store) {
            RowClass s = a.row_class[op.operands[1]];
            if (s != RowClass::Full && s != RowClass::RowVec) return no("store of a broadcast vector");
        }
        if (op.kind == OpKind::RowSum || op.kind == OpKind::RowMax || op.kind == OpKind::RowMean) {
            RowClass s = a.row_class[op.operands[0]];
            if (s != RowClass::Full && !(s == RowClass::RowVec && C == 1)) return no("row reduction of a vector");
        }
    }
    return true;
}

// MFMA GEMM pattern: Matmul(a, b) -> r1; optional Add(c, r1) -> r2; Store(c, r2|r1).
GemmInfo classify_gemm(const KernelDef& k, const KernelAnalysis& a) {
    GemmInfo g;
    std::vector<const OpInfo*> ops;
    for (const auto& op : k.ops)
        if (op.kind != OpKind::Constant && op.kind != OpKind::CpuSimAddCycles) ops.push_back(&op);
    if (ops.size() != 2 && ops.size() != 3) return g;
    const OpInfo& mm = *ops[0];
    if (mm.kind != OpKind::Matmul || mm.result <= 0) return g;
    const int pa = a.param_of[mm.operands[0]], pb = a.param_of[mm.operands[1]];
    if (pa < 0 || pb < 0) return g;
    int stored_val = mm.result;
    int pc = -1;
    if (ops.size() == 3) {
        const OpInfo& add = *ops[1];
        if (add.kind != OpKind::Add || add.operands.size() != 2) return g;
        const int x = add.operands[0], y = add.operands[1];
        const int other = x == mm.result ? y : (y == mm.result ? x : -1);
        if (other < 0 || a.param_of[other] < 0) return g;
        pc = a.param_of[other];
        stored_val = add.result;
        g.accumulate = true;
    }
    const OpInfo& st = *ops.back();
    if (st.kind != OpKind::Store || st.operands[1] != stored_val) return g;
    if (pc >= 0 && a.param_of[st.operands[0]] != pc) return g;
    pc = a.param_of[st.operands[0]];
    if (pc < 0 || pa == pb || pa == pc || pb == pc) return g;
    const ValueInfo* va = a.by_id[k.params[pa].id];
    const ValueInfo* vb = a.by_id[k.params[pb].id];
    const ValueInfo* vc = a.by_id[k.params[pc].id];
    if (va->dtype != vb->dtype || (va->dtype != DType::BF16 && va->dtype != DType::F16 && va->dtype != DType::F32)) return g;
    if (vc->dtype != DType::F32) return g;
    const int M = va->rows, K = va->cols, N = vb->cols;
    const bool f32 = va->dtype == DType::F32;
    // Task tiles of 16..256 rows / columns (multiples of 16; the host merges
    // neighbouring tasks into blocks of 64..256, or runs the tile program when
    // it cannot), or multiples of 256 up to 16384 (split into 256-wide
    // blocks); K step a power of two in 16..128 or a multiple of 64 (f32: 32)
    // up to 16384, taken in stages (gemm_stage_k); two LDS stages of A and B
    // within 160 KiB.
    auto dim_ok = [](int t) { return (t % 16 == 0 && t >= 16 && t <= 256) || (t % 256 == 0 && t <= 16384); };
    if (!dim_ok(M) || !dim_ok(N)) return g;
    const bool k_small = K == 16 || K == 32 || K == 64 || K == 128;
    if (!k_small && (K % (f32 ? 32 : 64) || K > 16384)) return g;
    if (2 * (gemm_block_dim(M) + gemm_block_dim(N)) * gemm_stage_k(K, f32) * (f32 ? 4 : 2) > 160 * 1024) return g;
    g.ok = true;
    g.a = a.tensor_ordinal[pa];
    g.b = a.tensor_ordinal[pb];
    g.c = a.tensor_ordinal[pc];
    g.m = M;
    g.n = N;
    g.k = K;
    g.f16 = va->dtype == DType::F16;
    g.f32 = f32;
    return g;
}

// Recognizes store(out, div(o, l)) over params (see NormInfo).
NormInfo classify_norm(const KernelDef& k, const KernelAnalysis& a) {
    NormInfo info;
    const OpInfo *div = nullptr, *store = nullptr;
    size_t div_index = 0;
    for (size_t i = 0; i < k.ops.size(); ++i) {
        const OpInfo& op = k.ops[i];
        if (op.kind == OpKind::CpuSimAddCycles) continue;
        if (op.kind == OpKind::Div && !div) {
            div = &op;
            div_index = i;
        } else if (op.kind == OpKind::Store && !store) {
            store = &op;
        } else {
            return info;
        }
    }
    if (!div || !store || div->operands.size() != 2 || store->operands.size() != 2) return info;
    if (store->operands[1] != div->result || div_index >= a.bin_mode.size() || a.bin_mode[div_index] != BinMode::RowExpand)
        return info;
    auto param = [&](int id) { return id >= 0 && id < static_cast<int>(a.param_of.size()) ? a.param_of[id] : -1; };
    const int po = param(div->operands[0]), pl = param(div->operands[1]), pout = param(store->operands[0]);
    if (po < 0 || pl < 0 || pout < 0 || po == pout || pl == pout) return info;
    const ValueInfo *o = a.by_id[k.params[po].id], *l = a.by_id[k.params[pl].id], *out = a.by_id[k.params[pout].id];
    if (o->dtype != DType::F32 || l->dtype != DType::F32 || out->dtype != DType::F32) return info;
    if (l->rows != o->rows || l->cols != 1 || out->rows != o->rows || out->cols != o->cols) return info;
    info.ok = true;
    info.o = a.tensor_ordinal[po];
    info.l = a.tensor_ordinal[pl];
    info.out = a.tensor_ordinal[pout];
    info.g = o->rows;
    info.d = o->cols;
    return info;
}

// Recognizes the online-softmax decode step (see DecodeInfo) by its dataflow,
// starting from the three accumulator stores.  Binary ops may take their
// operands in either order; every non-constant op must belong to the pattern.
DecodeInfo classify_decode(const KernelDef& k, const KernelAnalysis& a) {
    DecodeInfo info;
    std::map<int, const OpInfo*> def;
    int n_ops = 0;
    std::vector<const OpInfo*> stores;
    for (const auto& op : k.ops) {
        if (op.result > 0) def[op.result] = &op;
        if (op.kind == OpKind::Constant || op.kind == OpKind::CpuSimAddCycles) continue;
        ++n_ops;
        if (op.kind == OpKind::Store) stores.push_back(&op);
    }
    if (stores.size() != 3) return info;
    auto producer = [&](int id, OpKind kind) -> const OpInfo* {
        auto it = def.find(id);
        return it != def.end() && it->second->kind == kind && it->second->operands.size() == 2 ? it->second : nullptr;
    };
    auto unary = [&](int id, OpKind kind) -> const OpInfo* {
        auto it = def.find(id);
        return it != def.end() && it->second->kind == kind && it->second->operands.size() == 1 ? it->second : nullptr;
    };
    auto param = [&](int id) { return id >= 0 && id < static_cast<int>(a.param_of.size()) ? a.param_of[id] : -1; };
    std::set<const OpInfo*> used;
    // Each store: target param and the stored value.
    int pm = -1, pl = -1, po = -1, xm = -1, xl = -1, xo = -1;
    for (const OpInfo* st : stores) {
        const int tp = param(st->operands[0]);
        if (tp < 0) return info;
        const int x = st->operands[1];
        if (producer(x, OpKind::Max)) { pm = tp; xm = x; }
        else if (const OpInfo* add = producer(x, OpKind::Add)) {
            bool is_o = false;
            for (int w : add->operands) is_o = is_o || producer(w, OpKind::Matmul) != nullptr;
            if (is_o) { po = tp; xo = x; } else { pl = tp; xl = x; }
        } else {
            return info;
        }
        used.insert(st);
    }
    if (pm < 0 || pl < 0 || po < 0) return info;
    const int m_id = k.params[pm].id, l_id = k.params[pl].id, o_id = k.params[po].id;
    // m' = max(m, rowmax(s))
    const OpInfo* mx = producer(xm, OpKind::Max);
    int rm = -1;
    if (mx->operands[0] == m_id) rm = mx->operands[1];
    else if (mx->operands[1] == m_id) rm = mx->operands[0];
    const OpInfo* rowmax = rm > 0 ? unary(rm, OpKind::RowMax) : nullptr;
    if (!rowmax) return info;
    used.insert(mx);
    used.insert(rowmax);
    const int s_id = rowmax->operands[0];
    // s = mul(matmul(q, k_t), c) [- mask]
    int s2 = s_id, mask_p = -1;
    bool row_mask = false;
    if (const OpInfo* sub = producer(s_id, OpKind::Sub)) {
        mask_p = param(sub->operands[1]);
        if (mask_p < 0) return info;
        // The mask applies one value per token (a column broadcast, or the same
        // [1, PG] shape when there is one query row).  When the score tile is
        // square the reference's rule makes a [1,R] operand a row broadcast
        // (src/python/pto_codegen.cpp:1094-1105): one value per query row,
        // taken by the template for 16 rows and 16-token pages.
        const size_t oi = static_cast<size_t>(sub - k.ops.data());
        if (oi >= a.bin_mode.size()) return info;
        row_mask = a.bin_mode[oi] == BinMode::RowExpand;
        if (a.bin_mode[oi] != BinMode::ColExpand && a.bin_mode[oi] != BinMode::Same && !row_mask) return info;
        s2 = sub->operands[0];
        used.insert(sub);
    }
    const OpInfo* mul = producer(s2, OpKind::Mul);
    if (!mul) return info;
    int s1 = -1;
    double scale = 0.0;
    for (int w = 0; w < 2; ++w) {
        auto it = def.find(mul->operands[w]);
        if (it != def.end() && it->second->kind == OpKind::Constant && it->second->has_value) {
            scale = it->second->value;
            s1 = mul->operands[1 - w];
        }
    }
    const OpInfo* qk = s1 > 0 ? producer(s1, OpKind::Matmul) : nullptr;
    if (!qk) return info;
    used.insert(mul);
    used.insert(qk);
    const int pq = param(qk->operands[0]), pkt = param(qk->operands[1]);
    if (pq < 0 || pkt < 0) return info;
    // p = exp(s - m'), a = exp(m - m')
    auto is_exp_sub = [&](int id, int x, int y) -> bool {
        const OpInfo* e = unary(id, OpKind::Exp);
        const OpInfo* sb = e ? producer(e->operands[0], OpKind::Sub) : nullptr;
        if (!sb || sb->operands[0] != x || sb->operands[1] != y) return false;
        used.insert(e);
        used.insert(sb);
        return true;
    };
    // l' = l*a + rowsum(p), o' = o*a + p @ v (operands of add / mul in any order)
    auto split_update = [&](int x, int acc_id, OpKind other_kind, const OpInfo*& other, int& alpha) -> bool {
        const OpInfo* add = producer(x, OpKind::Add);
        if (!add) return false;
        for (int w = 0; w < 2; ++w) {
            const OpInfo* ml = producer(add->operands[w], OpKind::Mul);
            const OpInfo* ot = other_kind == OpKind::RowSum ? unary(add->operands[1 - w], other_kind)
                                                            : producer(add->operands[1 - w], other_kind);
            if (!ml || !ot) continue;
            if (ml->operands[0] == acc_id) alpha = ml->operands[1];
            else if (ml->operands[1] == acc_id) alpha = ml->operands[0];
            else continue;
            other = ot;
            used.insert(add);
            used.insert(ml);
            used.insert(ot);
            return true;
        }
        return false;
    };
    const OpInfo *rowsum = nullptr, *pv = nullptr;
    int alpha_l = -1, alpha_o = -1;
    if (!split_update(xl, l_id, OpKind::RowSum, rowsum, alpha_l)) return info;
    if (!split_update(xo, o_id, OpKind::Matmul, pv, alpha_o)) return info;
    const int p_id = rowsum->operands[0];
    if (pv->operands[0] != p_id) return info;
    const int pv_p = param(pv->operands[1]);
    if (pv_p < 0) return info;
    if (!is_exp_sub(p_id, s_id, xm)) return info;
    if (!is_exp_sub(alpha_l, m_id, xm)) return info;
    if (alpha_o != alpha_l && !is_exp_sub(alpha_o, m_id, xm)) return info;
    if (static_cast<int>(used.size()) != n_ops) return info;
    // Shapes and dtypes.
    auto vi = [&](int pidx) { return a.by_id[k.params[pidx].id]; };
    const ValueInfo *q = vi(pq), *kt = vi(pkt), *v = vi(pv_p), *m = vi(pm), *l = vi(pl), *o = vi(po);
    const int G = q->rows, D = q->cols, PG = kt->cols;
    if (q->dtype != kt->dtype || q->dtype != v->dtype ||
        (q->dtype != DType::BF16 && q->dtype != DType::F16 && q->dtype != DType::F32))
        return info;
    const bool f32 = q->dtype == DType::F32;
    if (m->dtype != DType::F32 || l->dtype != DType::F32 || o->dtype != DType::F32) return info;
    if (kt->rows != D || v->rows != PG || v->cols != D || m->rows != G || m->cols != 1 || l->rows != G || l->cols != 1 ||
        o->rows != G || o->cols != D)
        return info;
    if (mask_p >= 0) {
        const ValueInfo* mk = vi(mask_p);
        if (mk->dtype != DType::F32 || mk->rows != 1 || mk->cols != PG) return info;
        if (row_mask && (G != 16 || PG != 16)) return info;
    }
    // Device template shapes: pages of 8, 16, 32, 64 or 128 tokens (folded as 16-token
    // steps: larger pages as 16-token sub-pages, 8-token pages two to a step),
    // head dim 64 / 128 / 256, query rows in blocks of 16 (one MFMA row block
    // each) up to what the wave's registers hold beside its page ring: 48
    // rows at head dim 64 or 128, 16 at 256, in every dtype (f32 pages are
    // twice the registers and take 2-step rings from head dim 128).
    const int max_rows = D == 256 ? 16 : 48;
    if ((PG != 8 && PG != 16 && PG != 32 && PG != 64 && PG != 128) || G < 1 || G > max_rows ||
        (D != 64 && D != 128 && D != 256))
        return info;
    info.ok = true;
    info.f32 = f32;
    info.row_mask = row_mask;
    info.q = a.tensor_ordinal[pq];
    info.kt = a.tensor_ordinal[pkt];
    info.v = a.tensor_ordinal[pv_p];
    info.mask = mask_p >= 0 ? a.tensor_ordinal[mask_p] : -1;
    info.m = a.tensor_ordinal[pm];
    info.l = a.tensor_ordinal[pl];
    info.o = a.tensor_ordinal[po];
    info.g = G;
    info.d = D;
    info.pg = PG;
    info.f16 = q->dtype == DType::F16;
    info.scale = static_cast<float>(scale);
    return info;
}

}  // namespace

KernelAnalysis analyze_kernel(const KernelDef& k) {
    KernelAnalysis a;
    a.def = &k;
    for (const auto& v : k.values) a.max_id = std::max(a.max_id, v.id);
    for (const auto& op : k.ops) a.max_id = std::max(a.max_id, op.result);
    const int n = a.max_id + 1;
    a.by_id.assign(n, nullptr);
    a.param_of.assign(n, -1);
    a.preload.assign(n, false);
    a.acc_vec.assign(n, false);
    for (const auto& v : k.values) {
        if (v.id <= 0) refuse(k, "bad value id");
        a.by_id[v.id] = &v;
    }
    a.tensor_ordinal.assign(k.params.size(), -1);
    a.scalar_ordinal.assign(k.params.size(), -1);
    int nt = 0, ns = 0;
    for (size_t i = 0; i < k.params.size(); ++i) {
        int id = k.params[i].id;
        if (id <= 0 || id >= n || !a.by_id[id]) refuse(k, "param " + k.params[i].name + " has no value");
        a.param_of[id] = static_cast<int>(i);
        if (a.by_id[id]->tile) {
            a.tensor_ordinal[i] = nt++;
            a.tensor_param_index.push_back(static_cast<int>(i));
        } else {
            a.scalar_ordinal[i] = ns++;
        }
    }
    a.stored.assign(nt, false);
    a.read.assign(nt, false);
    a.bin_mode.assign(k.ops.size(), BinMode::Same);
    if (k.custom) {
        // A cpp_src body: it may read and write every tile param; its cycles
        // are what the body reports when it runs.
        a.family = Family::Custom;
        a.stored.assign(nt, true);
        a.read.assign(nt, true);
        a.cycles = 0;
        return a;
    }

    auto val = [&](int id) -> const ValueInfo* {
        if (id <= 0 || id >= n || !a.by_id[id]) refuse(k, "op references undefined value " + std::to_string(id));
        return a.by_id[id];
    };
    // Scalars that have a value: scalar params and Constant() results (:605-655).
    std::vector<bool> scalar_known(n, false);
    for (size_t i = 0; i < k.params.size(); ++i)
        if (!a.by_id[k.params[i].id]->tile) {
            DType d = a.by_id[k.params[i].id]->dtype;
            if (d != DType::F32 && d != DType::I32 && d != DType::I64 && d != DType::Bool)
                refuse(k, "unsupported scalar param dtype " + std::string(dtype_name(d)));
            scalar_known[k.params[i].id] = true;
        }
    for (const auto& op : k.ops) {
        if (op.kind != OpKind::Constant || op.result <= 0) continue;
        const ValueInfo* r = val(op.result);
        if (r->tile) refuse(k, "tile-shaped Constant ops have no compute in the reference lowering");
        if (!op.has_value) continue;
        if (dtype_is_float(r->dtype) && r->dtype != DType::F32) refuse(k, "unsupported constant dtype");
        scalar_known[op.result] = true;
    }

    // Param tiles TLOADed at entry: used by any op except Matmul and Load,
    // excluding a Store destination (:453-469).
    for (const auto& op : k.ops) {
        if (op.kind == OpKind::Matmul || op.kind == OpKind::Load) continue;
        for (size_t j = 0; j < op.operands.size(); ++j) {
            const ValueInfo* v = val(op.operands[j]);
            if (!v->tile || a.param_of[v->id] < 0) continue;
            if ((op.kind == OpKind::Store || op.kind == OpKind::StoreTopkIndices) && j == 0) continue;
            a.preload[v->id] = true;
        }
    }
    // Matmul results read by vector ops get a TMOV into a vector tile (:700-710).
    for (const auto& op : k.ops) {
        if (op.kind == OpKind::Matmul || op.kind == OpKind::Store) continue;
        for (int id : op.operands) {
            if (a.param_of[id] >= 0) continue;
            for (const auto& q : k.ops)
                if (q.kind == OpKind::Matmul && q.result == id) a.acc_vec[id] = true;
        }
    }

    // u32 tiles carry sort indices only: produced by IotaU32 (or a TMov of
    // one) and read by TSort32 as its index operand.
    for (const auto& op : k.ops)
        for (size_t j = 0; j < op.operands.size(); ++j) {
            const ValueInfo* v = val(op.operands[j]);
            if (v->tile && v->dtype == DType::U32 && !(op.kind == OpKind::TSort32 && j == 1) && op.kind != OpKind::TMov)
                refuse(k, "u32 tiles may only feed TSort32 (as its index operand) or TMov");
        }

    uint64_t cycles = 0;
    for (size_t i = 0; i < k.params.size(); ++i) {
        const ValueInfo* v = a.by_id[k.params[i].id];
        if (v->tile && a.preload[v->id]) {
            cycles += rc(v);
            a.read[a.tensor_ordinal[i]] = true;
        }
    }
    for (size_t oi = 0; oi < k.ops.size(); ++oi) {
        const auto& op = k.ops[oi];
        const ValueInfo* res = op.result > 0 ? val(op.result) : nullptr;
        switch (op.kind) {
            case OpKind::Constant: break;
            case OpKind::Load: {
                if (op.operands.empty()) refuse(k, "Load missing operand");
                const ValueInfo* s = val(op.operands[0]);
                if (a.param_of[s->id] < 0 || !s->tile) refuse(k, "Load src must be a kernel param tile");
                if (!res || !res->tile) refuse(k, "Load without a tile result");
                if (res->rows != s->rows || res->cols != s->cols || res->dtype != s->dtype) refuse(k, "Load shape mismatch");
                a.read[a.tensor_ordinal[a.param_of[s->id]]] = true;
                cycles += rc(s);
                break;
            }
            case OpKind::Store: {
                if (op.operands.size() < 2) refuse(k, "Store expects dst, src");
                const ValueInfo* d = val(op.operands[0]);
                const ValueInfo* s = val(op.operands[1]);
                if (a.param_of[d->id] < 0 || !d->tile) refuse(k, "Store dst must be a kernel param tile");
                if (!s->tile) refuse(k, "Store src must be a tile");
                if (s->rows != d->rows || s->cols != d->cols)
                    refuse(k, "Store of a " + std::to_string(s->rows) + "x" + std::to_string(s->cols) + " tile into a " +
                                  std::to_string(d->rows) + "x" + std::to_string(d->cols) + " param");
                const bool same = s->dtype == d->dtype;
                const bool cast_ok = s->dtype == DType::F32 && (d->dtype == DType::F16 || d->dtype == DType::BF16);
                if (!same && !cast_ok)
                    refuse(k, std::string("Store dtype mismatch (unsupported cast ") + dtype_name(s->dtype) + " -> " +
                                  dtype_name(d->dtype) + ")");
                if (same && (d->dtype == DType::F64 || d->dtype == DType::Bool || d->dtype == DType::I8 ||
                             d->dtype == DType::U8 || d->dtype == DType::I16 || d->dtype == DType::U16 ||
                             d->dtype == DType::U32 || d->dtype == DType::U64))
                    refuse(k, std::string("tiles of dtype ") + dtype_name(d->dtype) + " are not supported");
                a.stored[a.tensor_ordinal[a.param_of[d->id]]] = true;
                if (!same) cycles += rc(d);  // TCVT
                cycles += rc(d);             // TSTORE
                break;
            }
            case OpKind::Matmul: {
                if (op.operands.size() < 2 || !res || !res->tile) refuse(k, "malformed Matmul");
                const ValueInfo* av = val(op.operands[0]);
                const ValueInfo* bv = val(op.operands[1]);
                if (!av->tile || !bv->tile) refuse(k, "Matmul expects tile operands");
                if (av->cols != bv->rows) refuse(k, "Matmul K mismatch");
                // f32 x f32, f16 x f16 (reference :863-873); bf16 x bf16 and a 16-bit float
                // operand with an f32 one (exact upcast, f32 math) are extensions.
                auto h16 = [](DType d) { return d == DType::F16 || d == DType::BF16; };
                const bool ok = (av->dtype == DType::F32 && bv->dtype == DType::F32) ||
                                (av->dtype == DType::F16 && bv->dtype == DType::F16) ||
                                (av->dtype == DType::BF16 && bv->dtype == DType::BF16) ||
                                (av->dtype == DType::F32 && h16(bv->dtype)) || (h16(av->dtype) && bv->dtype == DType::F32);
                if (!ok || res->dtype != DType::F32)
                    refuse(k, std::string("Matmul: unsupported dtype combination ") + dtype_name(av->dtype) + " x " +
                                  dtype_name(bv->dtype) + " -> " + dtype_name(res->dtype));
                if (res->rows != av->rows || res->cols != bv->cols) refuse(k, "Matmul result shape mismatch");
                for (int id : {av->id, bv->id})
                    if (a.param_of[id] >= 0) a.read[a.tensor_ordinal[a.param_of[id]]] = true;
                const uint64_t M = av->rows, K = av->cols, N = bv->cols;
                cycles += M * K + K * N + M * K * N;
                if (a.acc_vec[res->id]) cycles += M * N;
                break;
            }
            case OpKind::Add: case OpKind::Sub: case OpKind::Mul: case OpKind::Div: case OpKind::Max: case OpKind::Min: {
                if (op.operands.size() != 2 || !res) refuse(k, "binary op missing result/operands");
                if (!res->tile) refuse(k, "binary op with a scalar result has no tile lowering");
                const ValueInfo* av = val(op.operands[0]);
                const ValueInfo* bv = val(op.operands[1]);
                if (!av->tile && !scalar_known[av->id]) refuse(k, "scalar operand has no value");
                if (!bv->tile && !scalar_known[bv->id]) refuse(k, "scalar operand has no value");
                if (!av->tile && !bv->tile) refuse(k, "binary op on two scalars has no tile lowering");
                if (dtype_is_float(res->dtype) && res->dtype != DType::F32)
                    refuse(k, std::string("vector ops on ") + dtype_name(res->dtype) + " tiles are not supported");
                if (!av->tile || !bv->tile) {
                    const ValueInfo* tv = av->tile ? av : bv;
                    const ValueInfo* sv = av->tile ? bv : av;
                    if (!av->tile && op.kind == OpKind::Sub) refuse(k, "Sub: scalar - tile not supported");
                    if (tv->rows != res->rows || tv->cols != res->cols) refuse(k, "scalar op shape mismatch");
                    if (is_int(tv->dtype) != is_int(sv->dtype) || tv->dtype != res->dtype)
                        refuse(k, "mixed int/float scalar op");
                    a.bin_mode[oi] = av->tile ? BinMode::ScalarRight : BinMode::ScalarLeft;
                } else {
                    const int R = res->rows, C = res->cols;
                    if (av->rows != R || av->cols != C) refuse(k, "Binary op broadcast pattern unsupported");
                    if (av->dtype != res->dtype || bv->dtype != res->dtype) refuse(k, "mixed dtype tile op");
                    if (bv->rows == R && bv->cols == C) a.bin_mode[oi] = BinMode::Same;
                    else if ((bv->rows == R && bv->cols == 1) || (bv->rows == 1 && bv->cols == R))
                        a.bin_mode[oi] = BinMode::RowExpand;
                    else if ((op.kind == OpKind::Sub || op.kind == OpKind::Mul || op.kind == OpKind::Div) &&
                             ((bv->rows == 1 && bv->cols == C) || (bv->rows == C && bv->cols == 1)))
                        a.bin_mode[oi] = BinMode::ColExpand;
                    else refuse(k, "Binary op broadcast pattern unsupported");
                }
                cycles += rc(res);
                break;
            }
            case OpKind::Exp: case OpKind::Rsqrt: {
                if (op.operands.size() != 1 || !res || !res->tile) refuse(k, "unary op expects a tile");
                const ValueInfo* s = val(op.operands[0]);
                if (!s->tile || s->dtype != DType::F32 || res->dtype != DType::F32) refuse(k, "Exp/Rsqrt need f32 tiles");
                if (s->rows != res->rows || s->cols != res->cols) refuse(k, "unary op shape mismatch");
                cycles += rc(res);
                break;
            }
            case OpKind::RowSum: case OpKind::RowMax: case OpKind::RowMean: {
                if (op.operands.size() != 1 || !res || !res->tile) refuse(k, "row reduce expects a tile");
                const ValueInfo* s = val(op.operands[0]);
                if (!s->tile) refuse(k, "row reduce expects a tile operand");
                if (res->rows != s->rows || res->cols != 1) refuse(k, "row reduce result shape");
                if (is_int(s->dtype) != is_int(res->dtype)) refuse(k, "row reduce dtype mismatch");
                if (dtype_is_float(s->dtype) && s->dtype != DType::F32) refuse(k, "row reduce of non-f32 tiles");
                cycles += static_cast<uint64_t>(res->rows) * (op.kind == OpKind::RowMean ? 2u : 1u);
                break;
            }
            case OpKind::TMov: {
                // TMOV: a tile copy; rows x cols of the destination
                // (ptoisa_bridge.hpp:104-109).
                if (op.operands.size() != 1 || !res || !res->tile) refuse(k, "TMov expects one tile operand and a tile result");
                const ValueInfo* s = val(op.operands[0]);
                if (!s->tile || s->rows != res->rows || s->cols != res->cols || s->dtype != res->dtype)
                    refuse(k, "TMov shape/dtype mismatch");
                if (dtype_is_float(res->dtype) && res->dtype != DType::F32)
                    refuse(k, std::string("TMov of ") + dtype_name(res->dtype) + " tiles is not supported");
                cycles += rc(res);
                break;
            }
            case OpKind::IotaU32: {
                // A [1,C] u32 tile holding 0..C-1: a scalar loop in the reference
                // emitter (src/python/pto_codegen.cpp:1132-1150), no cycles.
                if (!op.operands.empty() || !res || !res->tile || res->rows != 1 || res->dtype != DType::U32)
                    refuse(k, "IotaU32 expects a [1,C] u32 result");
                auto it = op.ints.find("cols");
                if (it != op.ints.end() && it->second != res->cols) refuse(k, "IotaU32 cols attr does not match its result");
                break;
            }
            case OpKind::TSort32: {
                // TSORT32 of a [1,32] f32 score tile with a [1,32] u32 index tile into
                // [1,64] (score, index) pairs; 5 cycles per source element
                // (ptoisa_bridge.hpp:280-292, ptoisa_jit.py:247-258).
                if (op.operands.size() != 2 || !res || !res->tile) refuse(k, "TSort32 expects (scores, idx) and a tile result");
                const ValueInfo* sc = val(op.operands[0]);
                const ValueInfo* ix = val(op.operands[1]);
                if (!sc->tile || sc->rows != 1 || sc->cols != 32 || sc->dtype != DType::F32)
                    refuse(k, "TSort32 requires a [1,32] f32 score tile");
                if (!ix->tile || ix->rows != 1 || ix->cols != 32 || ix->dtype != DType::U32)
                    refuse(k, "TSort32 requires a [1,32] u32 index tile");
                if (res->rows != 1 || res->cols != 64 || res->dtype != DType::F32) refuse(k, "TSort32 result must be [1,64] f32");
                cycles += 5 * rc(sc);
                break;
            }
            case OpKind::ExtractTopkIndices: {
                // The first k pair indices as i32 (src/python/pto_codegen.cpp:1170-1193); no cycles.
                if (op.operands.size() != 1 || !res || !res->tile) refuse(k, "ExtractTopkIndices expects one operand");
                const ValueInfo* pr = val(op.operands[0]);
                if (!pr->tile || pr->rows != 1 || pr->cols != 64 || pr->dtype != DType::F32)
                    refuse(k, "ExtractTopkIndices expects the [1,64] f32 pairs of TSort32");
                auto it = op.ints.find("k");
                const int64_t kk = it != op.ints.end() && it->second > 0 ? it->second : res->cols;
                if (res->rows != 1 || res->dtype != DType::I32 || kk != res->cols || kk > 32)
                    refuse(k, "ExtractTopkIndices result must be a [1,k] i32 tile with 1 <= k <= 32");
                break;
            }
            case OpKind::StoreTopkIndices: {
                // dst[i * col_stride] = (int)pairs[2i+1] for i < k, along row 0 of an
                // output param (ptoisa_jit.py:197-204, 445-456); no cycles.
                if (op.operands.size() != 2 || res) refuse(k, "StoreTopkIndices expects (dst, pairs)");
                const ValueInfo* d = val(op.operands[0]);
                const ValueInfo* pr = val(op.operands[1]);
                if (a.param_of[d->id] < 0 || !d->tile) refuse(k, "StoreTopkIndices dst must be a kernel param tile");
                if (d->dtype != DType::I32 && d->dtype != DType::I64) refuse(k, "StoreTopkIndices dst must be i32 or i64");
                if (!pr->tile || pr->rows != 1 || pr->cols != 64 || pr->dtype != DType::F32)
                    refuse(k, "StoreTopkIndices expects the [1,64] f32 pairs of TSort32");
                auto it = op.ints.find("k");
                const int64_t kk = it != op.ints.end() ? it->second : 0;
                if (kk < 1 || kk > 32 || kk > d->cols) refuse(k, "StoreTopkIndices k must be in [1, min(32, dst cols)]");
                a.stored[a.tensor_ordinal[a.param_of[d->id]]] = true;
                break;
            }
            case OpKind::CpuSimAddCycles: {
                // pto::cpu_sim::add_cycles(n) in the kernel body (ptoisa_jit.py:206-208, 458-463):
                // an integer, or an expression of the kernel's scalar parameters.
                if (!op.operands.empty() || res) refuse(k, "CpuSimAddCycles takes no operands");
                if (op.cycles_expr) {
                    SRefs refs;
                    scalar_refs(*op.cycles_expr, refs);
                    if (!refs.axes.empty() || refs.slots || refs.task_params || refs.symbols)
                        refuse(k, "a cycles expression may read only the kernel's scalar parameters");
                    std::function<void(const SExpr&)> check = [&](const SExpr& e) {
                        if (e.kind == SExpr::Kind::KernelScalar && static_cast<int>(e.u) >= ns)
                            refuse(k, "a cycles expression reads scalar parameter " + std::to_string(e.u) + " of " +
                                          std::to_string(ns));
                        for (const SExpr* c : {e.a.get(), e.b.get(), e.c.get()})
                            if (c) check(*c);
                    };
                    check(*op.cycles_expr);
                    a.cycle_exprs.push_back(op.cycles_expr);
                    break;
                }
                auto it = op.ints.find("cycles");
                if (it == op.ints.end() || it->second < 0)
                    refuse(k, "CpuSimAddCycles expects a non-negative integer 'cycles' attr or a cycles expression");
                cycles += static_cast<uint64_t>(it->second);
                break;
            }
            default:
                // The reference emitter adds r*c cycles and computes nothing
                // for these (:1223-1231); this backend refuses them.
                refuse(k, "op '" + op.kind_name + "' has no compute in the reference cpu_sim lowering");
        }
    }
    a.cycles = cycles;
    for (size_t i = 0; i < a.tensor_param_index.size(); ++i) {
        const ValueInfo* v = a.by_id[k.params[a.tensor_param_index[i]].id];
        if (!dtype_is_float(v->dtype) && v->dtype != DType::I32 && v->dtype != DType::I64)
            refuse(k, std::string("tensor params of dtype ") + dtype_name(v->dtype) + " are not supported");
        if (v->dtype == DType::F64) refuse(k, "f64 tensor params are not supported");
    }
    if (classify_rows(k, a)) {
        a.family = Family::RowProgram;
        a.norm = classify_norm(k, a);
    } else {
        a.gemm = classify_gemm(k, a);
        a.decode = a.gemm.ok ? DecodeInfo{} : classify_decode(k, a);
        a.family = a.gemm.ok ? Family::Gemm : (a.decode.ok ? Family::Decode : Family::TileProgram);
    }
    return a;
}

}  // namespace ptowsp
