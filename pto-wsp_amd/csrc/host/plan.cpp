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
};

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
            ctx.grid.push_back(LoopSpec{n->var, &n->axis});
            lower(m, ka, n->body.get(), ctx, plan, out);
            return;
        }
        case NodeKind::ForEach: {
            if (is_seq_chain(n->body.get())) {
                ctx.inner.push_back(LoopSpec{n->var, &n->axis});
                lower(m, ka, n->body.get(), ctx, plan, out);
                return;
            }
            if (n->axis.kind == AxisKind::DynTensor)
                throw CompileError("P.seq over a tensor-bound extent must directly enclose its task");
            PlanItem loop;
            loop.is_loop = true;
            loop.loop = LoopSpec{n->var, &n->axis};
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
            lower(m, ka, n->body.get(), ctx, plan, loop.body);
            out.push_back(std::move(loop));
            return;
        }
        case NodeKind::Cond:
            throw CompileError("P.when / cond is not supported by the HIP target");
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
    std::vector<std::pair<std::string, int64_t>> vars;

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
                const uint32_t w = m.schedule.has_dispatch ? static_cast<uint32_t>(s.rr++ % s.workers) : 0u;
                return s.issue(ka[n->kernel_index].cycles, w, ready);
            }
            default: throw CompileError("cycle model: unsupported node");
        }
    }
};

}  // namespace

CycleResult run_cycle_model(const Module& m, const std::vector<KernelAnalysis>& ka, const CycleEnv& env) {
    const Schedule& sc = m.schedule;
    if (sc.has_dispatch && sc.dispatch_policy != "round_robin" && sc.dispatch_policy != "work_steal")
        throw CompileError("dispatch policy requires ScalarExpr key (not supported by this module format)");
    Walker w{m, ka, env, {}, 0, {}};
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
