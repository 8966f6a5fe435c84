#include "plan.hpp"

#include <algorithm>
#include <functional>
#include <queue>
#include <stdexcept>

namespace ptowsp {

namespace {

// True when `n` is a chain of ForEach loops ending in one task.
bool is_seq_chain(const Node* n) {
    while (n && n->kind == NodeKind::ForEach) n = n->body.get();
    return n && n->kind == NodeKind::Task;
}

struct Ctx {
    std::vector<LoopSpec> grid, inner;
    std::vector<std::string> host;  // host-loop variables in scope
    std::vector<Mask> masks;
};

// A P.seq chain whose task runs a cpp_src body: its loops run on the host
// (the body is one thread's code for one task).
bool chain_is_custom(const Module& m, const Node* n) {
    while (n && n->kind == NodeKind::ForEach) n = n->body.get();
    return n && n->kind == NodeKind::Task && m.kernels[n->kernel_index].custom;
}

bool has_slot_ops(const Node* n) {
    if (!n) return false;
    if (n->kind == NodeKind::SlotSet || n->kind == NodeKind::SlotLoad) return true;
    if (has_slot_ops(n->body.get())) return true;
    for (const auto& k : n->kids)
        if (has_slot_ops(k.get())) return true;
    return false;
}

// Where a variable an expression reads is bound: 2 grid loop, 1 host or
// in-kernel loop; the reference's emitter refuses one out of scope
// (src/python/pto_codegen.cpp:257-263).
int scope_of(const Ctx& ctx, uint64_t id) {
    for (auto it = ctx.inner.rbegin(); it != ctx.inner.rend(); ++it)
        if (fnv1a_64(it->var) == id) return 1;
    for (auto it = ctx.host.rbegin(); it != ctx.host.rend(); ++it)
        if (fnv1a_64(*it) == id) return 1;
    for (auto it = ctx.grid.rbegin(); it != ctx.grid.rend(); ++it)
        if (fnv1a_64(it->var) == id) return 2;
    throw CompileError("emit_scalar_expr_cpp: axis_var not in scope");
}

// True when the expression reads a grid loop variable (checking scope).
bool reads_grid(const Ctx& ctx, const SExpr& e) {
    SRefs r;
    scalar_refs(e, r);
    bool grid = false;
    for (uint64_t id : r.axes) grid |= scope_of(ctx, id) == 2;
    if (r.task_params) throw CompileError("emit_scalar_expr_cpp: task_param() requires task_param_expr callback");
    return grid;
}

void lower(const Module& m, const std::vector<KernelAnalysis>& ka, const Node* n, Ctx ctx, Plan& plan,
           std::vector<PlanItem>& out) {
    switch (n->kind) {
        case NodeKind::Empty: return;
        case NodeKind::Task: {
            LaunchSpec L;
            L.kernel = n->kernel_index;
            L.task = n;
            L.grid = ctx.grid;
            L.inner = ctx.inner;
            const KernelAnalysis& a = ka[n->kernel_index];
            const KernelDef& k = m.kernels[n->kernel_index];
            for (int pi : a.tensor_param_index) {
                const TensorArg* found = nullptr;
                for (const auto& t : n->tensor_args)
                    if (t.param == k.params[pi].name) found = &t;
                if (!found) throw CompileError("Missing tensor arg for param: " + k.params[pi].name);
                const ValueInfo* v = a.by_id[k.params[pi].id];
                if (m.tensors[found->tid].dtype != v->dtype)
                    throw CompileError("task " + k.name + ": param " + k.params[pi].name + " is " + dtype_name(v->dtype) +
                                       " but its tensor is " + dtype_name(m.tensors[found->tid].dtype));
                if (found->idx.size() > m.tensors[found->tid].shape.size())
                    throw CompileError("task " + k.name + ": too many indices into tensor for param " + k.params[pi].name);
                L.targs.push_back(found);
            }
            int nscal = 0;
            for (int so : a.scalar_ordinal)
                if (so >= 0) ++nscal;
            if (static_cast<int>(n->scalar_args.size()) != nscal)
                throw CompileError("task " + k.name + ": scalar argument count mismatch");
            if (L.grid.size() + L.inner.size() > 8) throw CompileError("loop nests deeper than 8 are not supported");
            L.masks = ctx.masks;
            if (m.schedule.dispatch_key) {
                SRefs r;
                scalar_refs(*m.schedule.dispatch_key, r);
                for (uint64_t id : r.axes) (void)scope_of(ctx, id);
            }
            plan.launches.push_back(L);
            PlanItem it;
            it.launch = static_cast<int>(plan.launches.size()) - 1;
            out.push_back(std::move(it));
            return;
        }
        case NodeKind::ParallelFor: {
            if (!ctx.inner.empty()) throw CompileError("internal: P() inside an in-kernel loop");
            if (n->axis.kind == AxisKind::DynTensor)
                throw CompileError("P() over a tensor-bound extent is not supported (use P.seq)");
            if (has_slot_ops(n->body.get())) {
                PlanItem loop;
                loop.is_loop = true;
                loop.loop = LoopSpec{n->var, &n->axis};
                ctx.host.push_back(n->var);
                lower(m, ka, n->body.get(), ctx, plan, loop.body);
                out.push_back(std::move(loop));
                return;
            }
            ctx.grid.push_back(LoopSpec{n->var, &n->axis});
            lower(m, ka, n->body.get(), ctx, plan, out);
            return;
        }
        case NodeKind::ForEach: {
            if (is_seq_chain(n->body.get()) && !chain_is_custom(m, n)) {
                ctx.inner.push_back(LoopSpec{n->var, &n->axis});
                lower(m, ka, n->body.get(), ctx, plan, out);
                return;
            }
            if (n->axis.kind == AxisKind::DynTensor)
                throw CompileError("P.seq over a tensor-bound extent must directly enclose its task");
            PlanItem loop;
            loop.is_loop = true;
            loop.loop = LoopSpec{n->var, &n->axis};
            ctx.host.push_back(n->var);
            lower(m, ka, n->body.get(), ctx, plan, loop.body);
            out.push_back(std::move(loop));
            return;
        }
        case NodeKind::Combine:
        case NodeKind::Sequential:
            for (const auto& c : n->kids) lower(m, ka, c.get(), ctx, plan, out);
            return;
        case NodeKind::Select: {
            // The selected indices are host symbols that may change between
            // runs: a host loop over them, each iteration launching its body
            // (iterations run in order, as in the reference's artifact loop,
            // src/python/pto_codegen.cpp:2417-2452, so repeated indices stay
            // exact).
            PlanItem loop;
            loop.is_loop = true;
            loop.loop = LoopSpec{n->var, &n->axis};
            ctx.host.push_back(n->var);
            lower(m, ka, n->body.get(), ctx, plan, loop.body);
            out.push_back(std::move(loop));
            return;
        }
        case NodeKind::Cond: {
            // src/python/pto_codegen.cpp:2458-2478: the branch the predicate picks.
            if (reads_grid(ctx, *n->pred)) {
                Ctx t = ctx, f = ctx;
                t.masks.push_back(Mask{n->pred.get(), true});
                f.masks.push_back(Mask{n->pred.get(), false});
                lower(m, ka, n->kids[0].get(), t, plan, out);
                lower(m, ka, n->kids[1].get(), f, plan, out);
                return;
            }
            PlanItem c;
            c.ctl = n;
            lower(m, ka, n->kids[0].get(), ctx, plan, c.body);
            lower(m, ka, n->kids[1].get(), ctx, plan, c.alt);
            out.push_back(std::move(c));
            return;
        }
        case NodeKind::SlotSet:
        case NodeKind::SlotLoad: {
            if (!ctx.grid.empty()) throw CompileError("internal: a slot step inside a launch grid");
            PlanItem c;
            c.ctl = n;
            out.push_back(std::move(c));
            return;
        }
    }
}

}  // namespace

Plan build_plan(const Module& m, const std::vector<KernelAnalysis>& ka) {
    Plan p;
    if (!m.root) throw CompileError("Workload body is null");
    lower(m, ka, m.root.get(), Ctx{}, p, p.items);
    return p;
}

namespace {

struct Scheduler {
    uint32_t workers = 1;
    uint64_t window = 0, issue_time = 0, rr = 0;
    std::vector<uint64_t> avail;
    std::priority_queue<uint64_t, std::vector<uint64_t>, std::greater<uint64_t>> in_flight;

    void advance_to(uint64_t t) {
        issue_time = std::max(issue_time, t);
        while (!in_flight.empty() && in_flight.top() <= issue_time) in_flight.pop();
    }

    uint64_t issue(uint64_t dur, uint32_t w, uint64_t ready) {
        if (w >= workers) w = 0;
        advance_to(ready);
        if (window > 0)
            while (in_flight.size() >= window) advance_to(in_flight.top());
        const uint64_t start = std::max(avail[w], issue_time);
        const uint64_t end = start + dur;
        avail[w] = end;
        in_flight.push(end);
        return end;
    }
};

struct Walker {
    const Module& m;
    const std::vector<KernelAnalysis>& ka;
    const CycleEnv& env;
    Scheduler s;
    uint64_t tasks = 0;
    VarList vars;
    std::vector<uint64_t> slots;

    SEnv senv() {
        return scalar_env(vars, env.symbol_u64, [this](uint32_t i) { return i < slots.size() ? slots[i] : 0; });
    }

    uint64_t arg_value(const ArgRef& a) {
        if (a.kind == 'c') return a.u64;
        if (a.kind == 's') return env.symbol_u64(a.u64);
        for (auto it = vars.rbegin(); it != vars.rend(); ++it)
            if (it->first == a.var) return static_cast<uint64_t>(it->second);
        throw std::runtime_error("unbound loop variable '" + a.var + "'");
    }

    // The task's argument vector as the reference packs it
    // (src/python/pto_codegen.cpp:2503-2545): axis args, (rows, cols) of each
    // tile param in kernel order, scalar args.
    std::vector<uint64_t> task_args(const Node* n) {
        std::vector<uint64_t> args;
        for (const auto& a : n->axis_args) args.push_back(arg_value(a));
        const KernelAnalysis& a = ka[n->kernel_index];
        for (const auto& p : a.def->params) {
            const ValueInfo* v = a.by_id[p.id];
            if (!v->tile) continue;
            args.push_back(static_cast<uint64_t>(v->rows));
            args.push_back(static_cast<uint64_t>(v->cols));
        }
        for (const auto& sa : n->scalar_args) args.push_back(arg_value(sa));
        return args;
    }

    uint32_t worker_of(const Node* n) {
        if (!m.schedule.has_dispatch) return 0;
        if (!m.schedule.dispatch_key) return static_cast<uint32_t>(s.rr++ % s.workers);
        // src/python/pto_codegen.cpp:2679-2690: key % workers.
        SEnv e = senv();
        std::vector<uint64_t> args;
        bool have = false;
        e.task_param = [&](uint32_t i) -> uint64_t {
            if (!have) args = task_args(n), have = true;
            return i < args.size() ? args[i] : 0;
        };
        return static_cast<uint32_t>(eval_u64(*m.schedule.dispatch_key, e) % s.workers);
    }

    int64_t extent(const Axis& a) {
        switch (a.kind) {
            case AxisKind::Dense: return a.size;
            case AxisKind::Dyn: return env.axis_size(a.a);
            case AxisKind::Ragged: {
                const int64_t outer = static_cast<int64_t>(env.symbol_u64(fnv1a_64(a.a)));
                const int32_t* len = env.symbol_ptr(fnv1a_64(a.b));
                int64_t ub = 0;
                if (len)
                    for (int64_t i = 0; i < outer; ++i) ub += len[i];
                return ub;
            }
            case AxisKind::DynTensor: return env.index_value(a.expr, vars);
            case AxisKind::Select: break;
        }
        return 0;
    }

    uint64_t eval(const Node* n, uint64_t ready) {
        switch (n->kind) {
            case NodeKind::Empty: return ready;
            case NodeKind::ParallelFor: {
                uint64_t done = ready;
                const int64_t ub = extent(n->axis);
                vars.emplace_back(n->var, 0);
                for (int64_t i = 0; i < ub; ++i) {
                    vars.back().second = i;
                    done = std::max(done, eval(n->body.get(), ready));
                }
                vars.pop_back();
                return done;
            }
            case NodeKind::ForEach: {
                uint64_t cur = ready;
                const int64_t ub = extent(n->axis);
                vars.emplace_back(n->var, 0);
                for (int64_t i = 0; i < ub; ++i) {
                    vars.back().second = i;
                    cur = eval(n->body.get(), cur);
                }
                vars.pop_back();
                return cur;
            }
            case NodeKind::Combine: {
                uint64_t done = ready;
                for (const auto& c : n->kids) done = std::max(done, eval(c.get(), ready));
                return done;
            }
            case NodeKind::Sequential: {
                uint64_t cur = ready;
                for (const auto& c : n->kids) cur = eval(c.get(), cur);
                return cur;
            }
            case NodeKind::Select: {
                // CSR select (src/python/pto_codegen.cpp:2417-2452): every
                // selected index starts at `ready`.
                const int64_t outer = static_cast<int64_t>(env.symbol_u64(fnv1a_64(n->axis.a)));
                const int32_t* indptr = env.symbol_ptr(fnv1a_64(n->axis.b));
                const int32_t* indices = env.symbol_ptr(fnv1a_64(n->axis.c));
                if (outer < 0) throw std::runtime_error("P.sel: negative outer size");
                const int64_t nnz = indptr ? indptr[outer] : 0;
                uint64_t done = ready;
                vars.emplace_back(n->var, 0);
                for (int64_t p = 0; p < nnz; ++p) {
                    vars.back().second = indices ? indices[p] : 0;
                    done = std::max(done, eval(n->body.get(), ready));
                }
                vars.pop_back();
                return done;
            }
            case NodeKind::Task: {
                ++tasks;
                const uint32_t w = worker_of(n);
                const KernelAnalysis& kn = ka[n->kernel_index];
                uint64_t dur = kn.cycles;
                if (kn.family == Family::Custom) {
                    if (!env.custom_cycles) throw std::runtime_error("the cycles of a cpp_src kernel are known only after it runs");
                    dur = env.custom_cycles(*n, vars);
                }
                if (!kn.cycle_exprs.empty()) {
                    // add_cycles((uint64_t)(expr)) with the task's scalar arguments.
                    SEnv e = senv();
                    e.kernel_scalar = [&](uint32_t i) -> uint64_t {
                        return i < n->scalar_args.size() ? arg_value(n->scalar_args[i]) : 0;
                    };
                    for (const auto& x : kn.cycle_exprs) dur += eval_u64(*x, e);
                }
                return s.issue(dur, w, ready);
            }
            case NodeKind::Cond:
                // src/python/pto_codegen.cpp:2458-2478.
                return eval(n->kids[eval_truth(*n->pred, senv()) ? 0 : 1].get(), ready);
            case NodeKind::SlotSet:
                // src/python/pto_codegen.cpp:2248-2253.
                if (n->slot < slots.size()) slots[n->slot] = n->value;
                return ready;
            case NodeKind::SlotLoad: {
                // src/python/pto_codegen.cpp:2254-2303.
                const uint64_t v = env.slot_load(*n, vars);
                if (n->slot < slots.size()) slots[n->slot] = v;
                return ready;
            }
            default: throw CompileError("cycle model: unsupported node");
        }
    }
};

}  // namespace

SEnv scalar_env(const VarList& vars, std::function<uint64_t(uint64_t)> symbol, std::function<uint64_t(uint32_t)> slot) {
    SEnv e;
    e.axis = [&vars](uint64_t id, int64_t& v) {
        for (auto it = vars.rbegin(); it != vars.rend(); ++it)
            if (fnv1a_64(it->first) == id) {
                v = it->second;
                return true;
            }
        return false;
    };
    e.symbol = std::move(symbol);
    e.slot = std::move(slot);
    return e;
}

namespace {
bool any_node(const Node* n, const std::function<bool(const Node*)>& f) {
    if (!n) return false;
    if (f(n) || any_node(n->body.get(), f)) return true;
    for (const auto& k : n->kids)
        if (any_node(k.get(), f)) return true;
    return false;
}
}  // namespace

bool module_is_dynamic(const Module& m) {
    if (m.schedule.dispatch_key) return true;
    for (const auto& k : m.kernels) {
        if (k.custom) return true;
        for (const auto& op : k.ops)
            if (op.cycles_expr) return true;  // per-task cycles read the scalar arguments
    }
    return any_node(m.root.get(), [](const Node* n) {
        return n->kind == NodeKind::Cond || n->kind == NodeKind::SlotSet || n->kind == NodeKind::SlotLoad;
    });
}

bool module_loads_slots(const Module& m) {
    return any_node(m.root.get(), [](const Node* n) { return n->kind == NodeKind::SlotLoad; });
}

CycleResult run_cycle_model(const Module& m, const std::vector<KernelAnalysis>& ka, const CycleEnv& env) {
    const Schedule& sc = m.schedule;
    Walker w{m, ka, env, {}, 0, {}, std::vector<uint64_t>(256, 0)};
    if (env.slot_init)
        for (uint32_t i = 0; i < 256; ++i) w.slots[i] = env.slot_init(i);
    int64_t W = 1;
    if (sc.has_dispatch && sc.num_targets > 0) W = sc.num_targets;
    else if (sc.has_streams && sc.num_streams > 0) W = sc.num_streams;
    w.s.workers = static_cast<uint32_t>(W > 0 ? W : 1);
    w.s.avail.assign(w.s.workers, 0);
    const bool window_ok = sc.has_window && sc.window_unit == "tasks" && sc.window_overflow == "stall";
    w.s.window = window_ok && sc.window_size > 0 ? static_cast<uint64_t>(sc.window_size) : 0;
    CycleResult r;
    r.total_cycles = w.eval(m.root.get(), 0);
    r.tasks = w.tasks;
    return r;
}

}  // namespace ptowsp
