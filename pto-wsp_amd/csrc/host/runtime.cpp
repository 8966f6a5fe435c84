// C ABI entry points of libptowsp_hip.so: compile, launch, synchronize and
// the RuntimeContext tables.  See include/ptowsp_hip.h.
#include <hip/hip_ext.h>
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <set>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "../device/ptowsp_launch.h"
#include "analysis.hpp"
#include "emit.hpp"
#include "jit.hpp"
#include "module.hpp"
#include "noalloc.hpp"
#include "plan.hpp"
#include "ptowsp_hip.h"

using namespace ptowsp;

namespace {

thread_local std::string g_last_error;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

bool is_device_pointer(const void* p) {
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof attr);
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

struct TensorState {
    char* host = nullptr;      // caller pointer when host-resident
    char* dev = nullptr;       // device address used by kernels
    std::vector<int64_t> stride;
    int64_t span = 0;          // elements addressable from element 0
    size_t bytes = 0;
    bool staged = false;
    bool written = false;
};

struct LaunchCache {
    std::map<std::string, const JitKernel*> by_spec;
    std::map<std::string, EmittedKernel> emitted;
};

}  // namespace

struct ptowsp_program {
    Module m;
    std::vector<KernelAnalysis> ka;
    Plan plan;
    std::vector<LaunchCache> cache;
    std::vector<bool> tensor_written;
    std::vector<void*> stage_buf;
    std::vector<size_t> stage_bytes;
    struct CopyBack {
        void* host;
        const void* dev;
        size_t bytes;
    };
    std::vector<CopyBack> copy_back;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    bool have_events = false;
    bool pending = false;
    // Error flag written by the kernels: pinned host memory mapped into the
    // device address space, so synchronize() reads it without a copy.
    int* h_err = nullptr;
    int* d_err = nullptr;
    double h2d_ms = 0.0;
    std::string cycle_key;
    CycleResult cycles;
    bool cycles_valid = false;
    // A run whose cycle model reads device-resident extent tensors: they are
    // copied into pinned memory ahead of the kernels and the model runs at
    // synchronize() from these tensor states and that copy.
    bool cycles_deferred = false;
    RuntimeContext* deferred_ctx = nullptr;
    std::vector<TensorState> deferred_ts;
    std::vector<std::pair<int, size_t>> deferred_tids;  // tensor id, int32 offset in key_stage
    int32_t* key_stage = nullptr;
    size_t key_stage_elems = 0;
    ptowsp_run_info last_run{};  // cycle model result of the last synchronized run
    std::string precompiled_source;
    void* scratch = nullptr;  // decode: unit counters and partials
    size_t scratch_bytes = 0;
    void* gtile = nullptr;    // tile programs: tiles beyond LDS, one region per workgroup
    size_t gtile_bytes = 0;
    // Task lists of masked launches: pinned host chunks copied into device
    // chunks on the launch stream; reused from the start at every run (the
    // previous run has been synchronized by then).
    struct ListChunk {
        int64_t* host = nullptr;
        int64_t* dev = nullptr;
        size_t cap = 0;
    };
    std::vector<ListChunk> lists;
    size_t list_chunk = 0, list_used = 0;
    // Per-task cycles of cpp_src kernels: one region of the list arena per
    // launch (by grid task index), copied back after the run; keyed by task
    // node and the host loop variables of the launch.
    struct CustomRun {
        size_t chunk = 0, off = 0;
        VarList host;
        std::vector<std::string> grid;
        std::vector<int64_t> ext;
    };
    std::map<const Node*, std::vector<CustomRun>> custom_runs;
    std::vector<std::array<size_t, 3>> readback;  // chunk, offset, count
    // Run started by ptowsp_hip_launch_noalloc: its error flag and deferred
    // extent copies live in the device scratch of noalloc.hip.
    bool noalloc_run = false;
    int* noalloc_err = nullptr;
    const int32_t* deferred_dev = nullptr;  // device copy of the deferred extent tensors
    bool timed = false;                     // the run recorded ev0 / ev1
    uint64_t* slot_stage = nullptr;     // pinned: one element read by a slot load
    std::vector<uint64_t> slot_log;     // values of the run's slot loads, in order
    std::vector<uint64_t> slot_start;   // slots when the run started

    ~ptowsp_program() {
        for (auto& c : lists) {
            if (c.host) (void)hipHostFree(c.host);
            if (c.dev) (void)hipFree(c.dev);
        }
        if (slot_stage) (void)hipHostFree(slot_stage);
        if (scratch) (void)hipFree(scratch);
        if (gtile) (void)hipFree(gtile);
        for (void* b : stage_buf)
            if (b) (void)hipFree(b);
        if (h_err) (void)hipHostFree(h_err);
        if (key_stage) (void)hipHostFree(key_stage);
        if (ev0) (void)hipEventDestroy(ev0);
        if (ev1) (void)hipEventDestroy(ev1);
    }
};

struct ptowsp_runtime {
    struct T {
        void* ptr = nullptr;
        std::vector<int64_t> strides;
    };
    std::map<uint32_t, T> tensors;
    std::map<std::string, int64_t> axis;
    std::map<uint64_t, uint64_t> sym;
    std::map<uint64_t, void*> symp;
    std::vector<uint64_t> slots = std::vector<uint64_t>(256, 0);
    RuntimeContext ctx{};
};

namespace {

int64_t rt_axis(void* c, const char* name) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    auto it = rt->axis.find(name ? name : "");
    return it == rt->axis.end() ? 0 : it->second;
}
uint64_t rt_sym(void* c, uint64_t id) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    auto it = rt->sym.find(id);
    return it == rt->sym.end() ? 0 : it->second;
}
void* rt_symp(void* c, uint64_t id) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    auto it = rt->symp.find(id);
    return it == rt->symp.end() ? nullptr : it->second;
}
uint64_t rt_slot(void* c, uint32_t i) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    return i < rt->slots.size() ? rt->slots[i] : 0;
}
void rt_set_slot(void* c, uint32_t i, uint64_t v) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    if (i < rt->slots.size()) rt->slots[i] = v;
}
void* rt_tptr(void* c, uint32_t tid) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    auto it = rt->tensors.find(tid);
    return it == rt->tensors.end() ? nullptr : it->second.ptr;
}
uint64_t rt_tstride(void* c, uint32_t tid, uint32_t dim) {
    auto* rt = static_cast<ptowsp_runtime*>(c);
    auto it = rt->tensors.find(tid);
    if (it == rt->tensors.end() || dim >= it->second.strides.size()) return 0;
    return static_cast<uint64_t>(it->second.strides[dim]);
}
KernelFn rt_kernel(void*, uint32_t) { return nullptr; }

// ---------------------------------------------------------------------------
// launch construction
// ---------------------------------------------------------------------------

struct RunEnv {
    ptowsp_program* P;
    RuntimeContext* ctx;
    std::vector<TensorState> ts;
    std::vector<std::pair<std::string, int64_t>> host_vars;
    std::map<int, std::vector<int32_t>> idx_host;  // device index tensors read on the host, copied once per run
    bool timing_started = false;                   // ev0 recorded (just before the first kernel)
    bool replay_slots = false;                     // cycle model: slot loads replay P->slot_log
    bool timing = true;                            // record ev0 / ev1 (the program's events exist)
    // No-allocation run: the kernels' error flag, and the device scratch that
    // replaces the program's hipMalloc'd decode scratch (counters at
    // nscratch + kNoAllocHeaderBytes, partials after them, nscratch_limit
    // bytes usable from nscratch).
    int* err = nullptr;
    char* nscratch = nullptr;
    size_t nscratch_limit = 0;
};

// Workgroups of a tile-program launch whose tiles exceed LDS (each has its
// own region of global tile scratch).
constexpr int64_t kGlobalTileBlocks = 1024;

// Device time starts at the program's first kernel: host work that precedes
// it (building launch arguments, compiling) is not counted.
void start_timing(RunEnv& E, hipStream_t stream) {
    if (E.timing_started || !E.timing) return;
    check(hipEventRecord(E.P->ev0, stream), "hipEventRecord");
    E.timing_started = true;
}

// Launches one kernel.  Device time runs from the start event, recorded on
// the stream just before the run's first kernel, to the end event recorded
// after its last one.  Events attached to the dispatch itself
// (hipExtModuleLaunchKernel's start / stop events) would leave out the
// command processor's latency before the first dispatch (about 1 us), but
// measured 15 us more host time per launch on the MI355X box; the separate
// records cost about 2.5 us each.
void launch_kernel(RunEnv& E, hipFunction_t f, int64_t blocks, int threads, size_t lds, hipStream_t stream, void** params,
                   const char* what) {
    start_timing(E, stream);
    check(hipModuleLaunchKernel(f, static_cast<unsigned>(blocks), 1, 1, static_cast<unsigned>(threads), 1, 1,
                                static_cast<unsigned>(lds), stream, params, nullptr),
          what);
}

int64_t axis_extent(RunEnv& E, const Axis& a) {
    switch (a.kind) {
        case AxisKind::Dense: return a.size;
        case AxisKind::Dyn: return E.ctx->get_axis_size(E.ctx->ctx, a.a.c_str());
        case AxisKind::Ragged: {
            const int64_t outer = static_cast<int64_t>(E.ctx->get_symbol_u64(E.ctx->ctx, fnv1a_64(a.a)));
            const auto* len = static_cast<const int32_t*>(E.ctx->get_symbol_ptr(E.ctx->ctx, fnv1a_64(a.b)));
            int64_t ub = 0;
            if (len)
                for (int64_t i = 0; i < outer; ++i) ub += len[i];
            return ub;
        }
        case AxisKind::DynTensor: throw CompileError("internal: tensor-bound extent evaluated on the host");
        case AxisKind::Select: throw CompileError("internal: a select axis used as a loop extent");
    }
    return 0;
}

// Reads one int32 element of an index tensor (host or device resident).
// Host view of a device-resident i32 index tensor, copied on first use in a run.
const std::vector<int32_t>& index_host_copy(RunEnv& E, int tid) {
    auto it = E.idx_host.find(tid);
    if (it != E.idx_host.end()) return it->second;
    const TensorState& t = E.ts[tid];
    std::vector<int32_t> v(static_cast<size_t>(std::max<int64_t>(t.span, 0)));
    if (!v.empty()) check(hipMemcpy(v.data(), t.dev, v.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy(index tensor)");
    return E.idx_host.emplace(tid, std::move(v)).first->second;
}

int64_t read_index_elem(RunEnv& E, int tid, int64_t off) {
    const TensorState& t = E.ts[tid];
    if (off < 0 || off >= t.span) throw std::runtime_error("index tensor element out of range");
    int32_t v = 0;
    if (t.host) std::memcpy(&v, t.host + off * 4, 4);
    else v = index_host_copy(E, tid)[static_cast<size_t>(off)];
    return v;
}

int64_t eval_index_host(RunEnv& E, const IndexExpr& e, const std::vector<std::pair<std::string, int64_t>>& vars) {
    auto lookup = [&](const std::string& n) -> int64_t {
        for (auto it = vars.rbegin(); it != vars.rend(); ++it)
            if (it->first == n) return it->second;
        for (auto it = E.host_vars.rbegin(); it != E.host_vars.rend(); ++it)
            if (it->first == n) return it->second;
        throw std::runtime_error("unbound loop variable '" + n + "'");
    };
    switch (e.kind) {
        case 'v': return lookup(e.var);
        case 'c': return e.c;
        case 'a': {
            int64_t v = e.c;
            for (const auto& [n, c] : e.terms) v += c * lookup(n);
            return v;
        }
        case 't': {
            if (E.P->m.tensors[e.tid].dtype != DType::I32) throw std::runtime_error("index tensors must be i32");
            int64_t off = 0;
            for (size_t d = 0; d < e.idx.size(); ++d) off += eval_index_host(E, e.idx[d], vars) * E.ts[e.tid].stride[d];
            return read_index_elem(E, e.tid, off);
        }
    }
    return 0;
}

// The element a slot load reads: the view's indices, then (row, col) within
// its tile (src/python/pto_codegen.cpp:2254-2303).
struct SlotElem {
    int64_t off;  // elements from the tensor's base
    size_t size;  // bytes
};

SlotElem slot_elem(RunEnv& E, const Node& n, const std::vector<std::pair<std::string, int64_t>>& vars) {
    const TensorArg& ta = n.view;
    const TensorState& T = E.ts[ta.tid];
    int64_t off = 0;
    for (size_t d = 0; d < ta.idx.size(); ++d) off += eval_index_host(E, ta.idx[d], vars) * T.stride[d];
    int64_t s3 = 0, s4 = 1;
    if (ta.view_rank >= 2) {
        const int d3 = ta.base_rank - ta.view_rank;
        s3 = T.stride[d3];
        s4 = T.stride[d3 + 1];
    } else if (ta.view_rank == 1) {
        s4 = T.stride[ta.base_rank - 1];
    }
    off += n.row * s3 + n.col * s4;
    if (off < 0 || off >= T.span) throw std::runtime_error("slot_load_u64: element outside its tensor");
    return {off, static_cast<size_t>(dtype_size(E.P->m.tensors[ta.tid].dtype))};
}

float half_bits_to_float(uint16_t h) {
    const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
    const float sign = (h & 0x8000) ? -1.0f : 1.0f;
    if (e == 0) return sign * std::ldexp(static_cast<float>(m), -24);
    if (e == 31) return m ? std::numeric_limits<float>::quiet_NaN() : sign * std::numeric_limits<float>::infinity();
    return sign * std::ldexp(static_cast<float>(m + 1024), e - 25);
}

// `(uint64_t)element` as C++ converts it; a float outside (-1, 2^64) has no
// defined conversion and is refused.
uint64_t slot_value(DType dt, const void* p) {
    auto from_float = [](float f) {
        if (!(f > -1.0f) || !(f < 18446744073709551616.0f))
            throw std::runtime_error("slot_load_u64: the element is not representable as u64");
        return static_cast<uint64_t>(f);
    };
    switch (dt) {
        case DType::F32: {
            float f;
            std::memcpy(&f, p, 4);
            return from_float(f);
        }
        case DType::F16: {
            uint16_t h;
            std::memcpy(&h, p, 2);
            return from_float(half_bits_to_float(h));
        }
        case DType::I32: {
            int32_t x;
            std::memcpy(&x, p, 4);
            return static_cast<uint64_t>(static_cast<int64_t>(x));
        }
        case DType::U32: {
            uint32_t x;
            std::memcpy(&x, p, 4);
            return x;
        }
        case DType::I64:
        case DType::U64: {
            uint64_t x;
            std::memcpy(&x, p, 8);
            return x;
        }
        case DType::Bool: return *static_cast<const unsigned char*>(p) != 0;
        default: throw std::runtime_error("slot_load_u64: unsupported dtype");
    }
}

// Affine decomposition: `scale * e` added into (constant, coef per loop var).
struct Affine {
    int64_t c = 0;
    std::vector<int64_t> coef;
};

void add_affine(RunEnv& E, const IndexExpr& e, int64_t scale, const std::map<std::string, int>& loop_index, Affine& out) {
    auto add_var = [&](const std::string& n, int64_t k) {
        auto it = loop_index.find(n);
        if (it != loop_index.end()) {
            out.coef[it->second] += k;
            return;
        }
        for (auto h = E.host_vars.rbegin(); h != E.host_vars.rend(); ++h)
            if (h->first == n) {
                out.c += k * h->second;
                return;
            }
        throw std::runtime_error("unbound loop variable '" + n + "' in a tensor index");
    };
    switch (e.kind) {
        case 'c': out.c += scale * e.c; break;
        case 'v': add_var(e.var, scale); break;
        case 'a':
            out.c += scale * e.c;
            for (const auto& [n, k] : e.terms) add_var(n, scale * k);
            break;
        default: throw std::runtime_error("internal: indirect index in an affine context");
    }
}

struct BuiltLaunch {
    LaunchArgs args{};
    EmitSpec spec;
    int64_t ntasks = 0;
    bool host_checked = false;
    std::vector<int64_t> tasks;  // task-list launches: the grid tasks kept by the masks
};

// Row-program vector width allowed by the actual strides and alignment.
int pick_vec_width(const KernelAnalysis& a, const LaunchArgs& A, int nvars) {
    for (int vw : {4, 2}) {
        if (a.cols % vw) continue;
        bool ok = true;
        for (size_t p = 0; p < a.tensor_param_index.size() && ok; ++p) {
            const int id = a.def->params[a.tensor_param_index[p]].id;
            // The param's own class, or that of a Load of it, decides how it is accessed.
            RowClass c = a.row_class[id];
            for (const auto& op : a.def->ops)
                if (op.kind == OpKind::Load && op.operands[0] == id && op.result > 0 &&
                    (a.row_class[op.result] == RowClass::Full || a.row_class[op.result] == RowClass::ColVec))
                    c = a.row_class[op.result];
            if (c != RowClass::Full && c != RowClass::ColVec) continue;
            if (A.s4[p] != 1) ok = false;
            if (reinterpret_cast<uintptr_t>(A.base[p]) % (vw * 4)) ok = false;
            if (c == RowClass::Full && A.s3[p] % vw) ok = false;
            for (int v = 0; v < nvars; ++v)
                if (A.coef[p][v] % vw) ok = false;
        }
        if (ok) return vw;
    }
    return 1;
}

// Launch-shape defaults of the row-program family, from a sweep on MI355X
// (2 passes per wave iteration with non-temporal loads/stores was fastest
// for both the rmsnorm and the softmax configurations);
// PTOWSP_ROW_UNROLL / PTOWSP_NONTEMPORAL override them.
struct Tuning {
    int row_up = 2;
    bool nontemporal = true;
    bool gemm_pingpong = true;
    int decode_ring = 0;  // 0: decode_ring_for(head dim)
    int decode_waves = 0;  // 0: decode_waves_for(head dim)
    bool decode_ordered = false;
    bool serial_groups = true;  // overlapping grids run as parallel groups of in-order tasks
    int tile_threads = 256;     // threads of a tile-program workgroup
    bool row_loops = true;      // row programs over in-kernel loops
    bool tile_mma = true;       // tile-program matmuls of MFMA shape on the matrix cores
};

// Page ring depth of the decode family: 32 KiB of K and V in flight per
// wave at head dim 128 (4 steps of 16 tokens).  At head dim 256 a step is
// twice the registers, and a 4-step ring spills to scratch (0.75 ms against
// 0.41 ms with 2 steps on the C5 shape with head dim 256); 2 steps keep the
// same bytes in flight.
// More than 16 query rows add a block of accumulators and q registers per
// 16 rows, and the fold, not the page latency, bounds them: 2 steps (C5
// lengths, one box: 32 rows at head dim 128 0.282 against 0.295 ms with 4,
// 48 rows at head dim 64 0.289 against 0.299 ms).  f32 pages are twice the
// registers of bf16 ones: 2 steps at head dim 128 (0.406 against 0.409 ms
// with 3 on the C5 shape in f32); 4 at head dim 64 up to 16 rows.  bf16 /
// f16 at head dim 128 (C5 lengths, rings of 2 / 3 / 4 steps, one box): 4
// rows 0.204 / 0.205 / 0.202 ms, 8 rows 0.210 / 0.208 / 0.209, 12 rows
// 0.218 / 0.218 / 0.219, 16 rows (32-token pages) 0.222 / 0.224 / 0.227.
int decode_ring_for(int head_dim, int rows, bool f32) {
    if (rows > 16) return 2;
    if (f32) return head_dim >= 128 ? 2 : 4;
    if (head_dim >= 256) return 2;
    if (head_dim <= 64) return 3;
    return rows <= 4 ? 4 : rows <= 12 ? 3 : 2;
}
// Waves per decode block (per CU).  At head dim 64 a step is 4 KiB of K and
// V, and one wave per SIMD cannot cover the fold's latency chain with it;
// two waves per SIMD (3-step rings, half the registers each) can, up to 16
// query rows.
int decode_waves_for(int head_dim, int rows, bool f32) { return !f32 && head_dim <= 64 && rows <= 16 ? 8 : 4; }

const Tuning& tuning() {
    static const Tuning t = [] {
        Tuning v;
        if (const char* s = std::getenv("PTOWSP_ROW_UNROLL")) v.row_up = std::max(1, std::atoi(s));
        if (const char* s = std::getenv("PTOWSP_NONTEMPORAL")) v.nontemporal = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_GEMM_PINGPONG")) v.gemm_pingpong = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_DECODE_RING")) v.decode_ring = std::min(8, std::max(2, std::atoi(s)));
        if (const char* s = std::getenv("PTOWSP_DECODE_WAVES")) v.decode_waves = std::atoi(s) == 8 ? 8 : 4;
        if (const char* s = std::getenv("PTOWSP_DECODE_ORDERED")) v.decode_ordered = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_SERIAL_GROUPS")) v.serial_groups = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_ROW_LOOPS")) v.row_loops = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_TILE_MMA")) v.tile_mma = std::atoi(s) != 0;
        if (const char* s = std::getenv("PTOWSP_TILE_THREADS")) {
            const int t = std::atoi(s);
            v.tile_threads = t == 64 || t == 128 || t == 256 || t == 512 ? t : 256;
        }
        return v;
    }();
    return t;
}

// Grid variables whose tasks must run in program order (bit v for grid
// variable v; 0: none).  P() promises independent iterations; a workload
// that breaks the promise (overlapping output views) still gets the
// reference's result: the launch is split into groups, one workgroup each,
// that write disjoint memory, and each group runs its tasks in program order.
// A group is the set of tasks that agree on the grid variables outside the
// mask.  The mask is the smallest (most groups) that the footprint analysis
// below proves safe for every written tensor; all grid variables (one
// group) when the analysis cannot tell.
uint32_t grid_write_hazard(const KernelAnalysis& a, const LaunchSpec& L, const LaunchArgs& A, const EmitSpec& spec, int ng,
                           int nvars) {
    const uint32_t all = ng >= 32 ? 0xFFFFFFFFu : ((1u << ng) - 1u);
    if (A.ntasks <= 1) return 0;
    const KernelDef& k = *a.def;
    const size_t np = a.tensor_param_index.size();
    // Per written tensor: the dims that move one task's footprint (tile rows /
    // cols, in-kernel loops) and the grid dims, as (|stride|, extent).
    struct Written {
        std::vector<std::pair<int64_t, int64_t>> tile_dims, grid_dims;
    };
    std::vector<Written> ws;
    for (size_t p = 0; p < np; ++p) {
        if (!a.stored[p]) continue;
        const int tid = L.targs[p]->tid;
        if (spec.indirect_count[p] > 0) return all;
        const ValueInfo* vp = a.by_id[k.params[a.tensor_param_index[p]].id];
        // Every other access to the written tensor must be the very same view.
        for (size_t q = 0; q < np; ++q) {
            if (q == p || L.targs[q]->tid != tid) continue;
            const ValueInfo* vq = a.by_id[k.params[a.tensor_param_index[q]].id];
            if (spec.indirect_count[q] > 0 || A.base[q] != A.base[p] || A.s3[q] != A.s3[p] || A.s4[q] != A.s4[p] ||
                vq->rows != vp->rows || vq->cols != vp->cols)
                return all;
            for (int v = 0; v < nvars; ++v)
                if (A.coef[q][v] != A.coef[p][v]) return all;
        }
        Written w;
        w.tile_dims.emplace_back(std::llabs(A.s3[p]), vp->rows);
        w.tile_dims.emplace_back(std::llabs(A.s4[p]), vp->cols);
        for (size_t i = 0; i < L.inner.size(); ++i) {
            const int v = ng + static_cast<int>(i);
            if (A.coef[p][v] == 0) continue;
            if (spec.inner_dyn_term[i] >= 0) return all;
            w.tile_dims.emplace_back(std::llabs(A.coef[p][v]), A.ext[v]);
        }
        for (int v = 0; v < ng; ++v) w.grid_dims.emplace_back(std::llabs(A.coef[p][v]), A.ext[v]);
        ws.push_back(std::move(w));
    }
    // True when (stride, extent) dims with offsets from `start` never revisit
    // an element: every index nests like the strides of an array.
    auto nests = [](std::vector<std::pair<int64_t, int64_t>> dims, int64_t start) {
        std::sort(dims.begin(), dims.end());
        int64_t span = start;
        for (const auto& [c, e] : dims) {
            if (e <= 1) continue;
            if (c < span) return false;
            span += c * (e - 1);
        }
        return true;
    };
    // Groups of mask m write disjoint memory when, for every written tensor,
    // either the whole map (grid x task) is injective or one group's
    // footprint fits in an interval and the other grid dims step over whole
    // intervals.
    auto safe = [&](uint32_t m) {
        for (const Written& w : ws) {
            std::vector<std::pair<int64_t, int64_t>> inside = w.tile_dims, across;
            for (int v = 0; v < ng; ++v) (((m >> v) & 1u) ? inside : across).push_back(w.grid_dims[v]);
            std::vector<std::pair<int64_t, int64_t>> every = inside;
            every.insert(every.end(), across.begin(), across.end());
            if (m == 0 && nests(every, 1)) continue;
            int64_t width = 1;
            for (const auto& [c, e] : inside) width += c * std::max<int64_t>(0, e - 1);
            if (!nests(across, width)) return false;
        }
        return true;
    };
    if (safe(0)) return 0;
    if (ng > 16) return all;
    uint32_t best = all;
    int64_t best_groups = 1;
    for (uint32_t m = 1; m < all; ++m) {
        int64_t groups = 1;
        for (int v = 0; v < ng; ++v)
            if (!((m >> v) & 1u)) groups *= std::max<int64_t>(1, A.ext[v]);
        if (groups > best_groups && safe(m)) {
            best = m;
            best_groups = groups;
        }
    }
    return best;
}

// The MFMA GEMM template needs unit column strides, 16-byte aligned operand
// rows at every task and K step, an output tile that stays put across the
// in-kernel loops, and operands that the launch does not write.
// Chooses the MFMA GEMM path for a launch of a GEMM-family kernel and, where
// neighbouring tasks' tiles are contiguous in A, B and C, the grid variables
// whose task pairs are merged into one workgroup block.  Returns false (tile
// program fallback) when strides, alignment or offset ranges do not allow the
// direct buffer->LDS loads of the GEMM block.
bool gemm_allowed(const KernelAnalysis& a, const LaunchSpec& L, const LaunchArgs& A, EmitSpec& spec, int ng, int nvars) {
    spec.gemm_vm = spec.gemm_vn = -1;
    spec.gemm_fm = spec.gemm_fn = spec.gemm_kf = 1;
    spec.gemm_pingpong = false;
    if (a.family != Family::Gemm || spec.serial) return false;
    for (int c : spec.indirect_count)
        if (c) return false;
    for (int t : spec.inner_dyn_term)
        if (t >= 0) return false;
    const GemmInfo& g = a.gemm;
    // Element size of A / B, and elements per 16-byte chunk of the direct loads.
    const int64_t es = g.f32 ? 4 : 2, epc = 16 / es;
    if (A.s4[g.a] != 1 || A.s4[g.b] != 1 || A.s4[g.c] != 1) return false;
    if (reinterpret_cast<uintptr_t>(A.base[g.a]) % 16 || reinterpret_cast<uintptr_t>(A.base[g.b]) % 16) return false;
    if (reinterpret_cast<uintptr_t>(A.base[g.c]) % 4) return false;
    if (A.s3[g.a] % epc || A.s3[g.b] % epc) return false;
    for (int v = 0; v < nvars; ++v) {
        if (A.coef[g.a][v] % epc || A.coef[g.b][v] % epc) return false;
        if (v >= ng && A.coef[g.c][v] != 0) return false;
        if (v >= ng && (A.coef[g.a][v] < 0 || A.coef[g.b][v] < 0)) return false;
    }
    const int tc = L.targs[g.c]->tid;
    if (L.targs[g.a]->tid == tc || L.targs[g.b]->tid == tc) return false;
    // Merge candidates: rows of C move with A's rows, columns with B's.
    const int64_t M = g.m, N = g.n;
    int vm = -1, vn = -1;
    for (int v = 0; v < ng; ++v) {
        if (A.ext[v] <= 0 || A.ext[v] % 2) continue;
        if (vm < 0 && A.coef[g.a][v] == M * A.s3[g.a] && A.coef[g.c][v] == M * A.s3[g.c] && A.coef[g.b][v] == 0)
            vm = v;
        else if (vn < 0 && A.coef[g.b][v] == N && A.coef[g.c][v] == N && A.coef[g.a][v] == 0)
            vn = v;
    }
    // Task K steps per LDS stage: in the accumulate form with one in-kernel
    // loop whose consecutive steps are adjacent A columns and B rows, steps
    // are merged up to 64 columns per stage (32 for f32), dividing the loop.
    int64_t kf = 1;
    if (g.accumulate && nvars == ng + 1) {
        const int v = ng;
        const int64_t kmax = g.f32 ? 32 : 64;
        if (A.coef[g.a][v] == g.k && A.coef[g.b][v] == g.k * A.s3[g.b])
            while (g.k * kf * 2 <= kmax && A.ext[v] % (kf * 2) == 0) kf *= 2;
    }
    const int64_t bk = g.k * kf;
    auto lds_fits = [&](int64_t bm, int64_t bn) {
        return bm <= 256 && bn <= 256 && 2 * (bm + bn) * gemm_stage_k(static_cast<int>(bk), g.f32) * es <= 160 * 1024;
    };
    // Tasks per block: powers of two along the merge variables (dividing
    // their extents), growing the smaller side first, up to 256 x 256.
    // Tiles above 256 are split into 256-wide blocks instead.
    const int64_t M0 = gemm_block_dim(static_cast<int>(M)), N0 = gemm_block_dim(static_cast<int>(N));
    int64_t fm = 1, fn = 1;
    for (;;) {
        const bool gm = vm >= 0 && M0 * fm * 2 <= 256 && A.ext[vm] % (fm * 2) == 0 && lds_fits(M0 * fm * 2, N0 * fn);
        const bool gn = vn >= 0 && N0 * fn * 2 <= 256 && A.ext[vn] % (fn * 2) == 0 && lds_fits(M0 * fm, N0 * fn * 2);
        if (gm && (M0 * fm <= N0 * fn || !gn)) fm *= 2;
        else if (gn) fn *= 2;
        else break;
    }
    const int64_t bm = M0 * fm, bn = N0 * fn;
    // Blocks below the MFMA block shape (64 rows / columns) stay on the tile program.
    if (bm % 64 || bn % 64 || !lds_fits(bm, bn)) return false;
    spec.gemm_vm = fm > 1 ? vm : -1;
    spec.gemm_vn = fn > 1 ? vn : -1;
    spec.gemm_fm = static_cast<int>(fm);
    spec.gemm_fn = static_cast<int>(fn);
    spec.gemm_kf = static_cast<int>(kf);
    // Buffer offsets (32-bit) from a block's step-0 origins.
    int64_t ka = 0, kb = 0;
    for (int v = ng; v < nvars; ++v) {
        ka += A.coef[g.a][v] * std::max<int64_t>(0, A.ext[v] - 1);
        kb += A.coef[g.b][v] * std::max<int64_t>(0, A.ext[v] - 1);
    }
    const int64_t lim = int64_t(1) << 31;
    if (A.s3[g.a] >= lim || A.s3[g.b] >= lim || A.s3[g.c] >= lim) return false;
    if (((bm - 1) * A.s3[g.a] + g.k) * es + ka * es >= lim) return false;
    if (((bk - 1) * A.s3[g.b] + bn) * es + kb * es >= lim) return false;
    if (((bm - 1) * A.s3[g.c] + bn) * 4 >= lim) return false;
    spec.gemm_pingpong = tuning().gemm_pingpong && !g.f32 && bm == 256 && bn == 256 && (bk == 64 || bk == 32) &&
                         A.s3[g.a] % 64 == 0 && A.s3[g.b] % 64 == 0;
    return true;
}

// Row programs over in-kernel (P.seq) loops: every row of a task runs the
// whole loop in one lane team, params that the loop does not move stay in
// registers (read once; stored ones are accumulators written back after the
// loop), and the others are loaded / stored every iteration.  Rows of one
// task then run concurrently, so the launch must have no memory dependence
// between two (row, iteration) pairs except through those accumulators:
// - an accumulator's tensor is named by no other param, and no op reads it
//   after its store in an iteration;
// - a param read every iteration is on a tensor that no param stores;
// - a param stored every iteration is on a tensor no other param names, and
//   its elements over (row, column, in-kernel iterations, grid) never repeat.
// Static in-kernel extents, no indirect indices, not serial.
bool row_loops_allowed(const KernelAnalysis& a, const LaunchSpec& L, const LaunchArgs& A, const EmitSpec& spec, int ng,
                       int nvars) {
    if (a.family != Family::RowProgram || L.inner.empty() || spec.serial || spec.task_list) return false;
    for (int c : spec.indirect_count)
        if (c > 0) return false;
    for (int t : spec.inner_dyn_term)
        if (t >= 0) return false;
    const KernelDef& k = *a.def;
    const size_t np = a.tensor_param_index.size();
    auto nests = [](std::vector<std::pair<int64_t, int64_t>> dims) {
        std::sort(dims.begin(), dims.end());
        int64_t span = 1;
        for (const auto& [c, e] : dims) {
            if (e <= 1) continue;
            if (c < span) return false;
            span += c * (e - 1);
        }
        return true;
    };
    for (size_t p = 0; p < np; ++p) {
        const int pid = k.params[a.tensor_param_index[p]].id;
        const ValueInfo* vp = a.by_id[pid];
        bool moves = false;
        for (int v = ng; v < nvars; ++v) moves = moves || A.coef[p][v] != 0;
        bool alone = true, stored_elsewhere = false;
        for (size_t q = 0; q < np; ++q) {
            if (q == p || L.targs[q]->tid != L.targs[p]->tid) continue;
            alone = false;
            if (a.stored[q]) stored_elsewhere = true;
        }
        if (!a.stored[p]) {
            if (stored_elsewhere) return false;  // read while another param writes the tensor
            continue;
        }
        if (!alone) return false;
        // No read after a store (a 16-bit param is never read: it only takes
        // the store cast, at every store or when written back).
        bool stored = false;
        for (const auto& op : k.ops)
            for (size_t j = 0; j < op.operands.size(); ++j) {
                if (op.operands[j] != pid) continue;
                const bool is_store = op.kind == OpKind::Store && j == 0;
                if (!is_store && stored) return false;
                stored = stored || is_store;
            }
        if (moves) {
            std::vector<std::pair<int64_t, int64_t>> dims;
            dims.emplace_back(std::llabs(A.s3[p]), vp->rows);
            dims.emplace_back(std::llabs(A.s4[p]), vp->cols);
            for (int v = 0; v < nvars; ++v) dims.emplace_back(std::llabs(A.coef[p][v]), A.ext[v]);
            if (!nests(dims)) return false;
        }
    }
    return true;
}

// Chooses the balanced decode path for a Decode-family kernel: one in-kernel
// (page) loop; q and the accumulators fixed along it; at most
// kDecodeMaxUnits units and fewer than 2^31 pages in all; strides and
// alignment that the 128-bit / 32-bit loads of DecodeWave need.  Otherwise
// the launch stays a tile program.
bool decode_allowed(const KernelAnalysis& a, const LaunchSpec& L, const LaunchArgs& A, const EmitSpec& spec, int ng) {
    if (a.family != Family::Decode || spec.serial || L.inner.size() != 1) return false;
    // The last scalar slot carries the declared page maximum.
    if (L.task->scalar_args.size() + 1 > static_cast<size_t>(kMaxScalars)) return false;
    const Axis& ax = *L.inner[0].axis;
    if (ax.kind == AxisKind::DynTensor && ax.max <= 0) return false;
    const int64_t maxp = ax.kind == AxisKind::DynTensor ? ax.max : A.ext[ng];
    int64_t units = 1;
    for (int v = 0; v < ng; ++v) units *= A.ext[v];
    // Page and cost prefixes (16-token sub-pages + kDecodeUnitCost per unit) stay below 2^31.
    const DecodeInfo& d = a.decode;
    const int64_t sub = d.pg >= 16 ? d.pg / 16 : 1;
    if (units < 1 || units > kDecodeMaxUnits || maxp < 0 || maxp > (int64_t(1) << 31) / sub ||
        maxp * sub + kDecodeUnitCost >= (int64_t(1) << 31) / units)
        return false;
    const int nvars = ng + 1;
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    if (ntens + 1 > kMaxParams) return false;  // one extra slot: counters and partials
    std::vector<int> first(ntens, 0);
    for (int p = 1; p < ntens; ++p) first[p] = first[p - 1] + spec.indirect_count[p - 1];
    auto aligned = [&](int p, int64_t elems, int esize) {
        if (reinterpret_cast<uintptr_t>(A.base[p]) % (elems * esize)) return false;
        for (int v = 0; v < nvars; ++v)
            if (A.coef[p][v] % elems) return false;
        for (int t = 0; t < spec.indirect_count[p]; ++t)
            if (A.ind[first[p] + t].stride % elems) return false;
        return true;
    };
    for (int p : {d.q, d.m, d.l, d.o}) {
        if (spec.indirect_count[p] != 0 || A.coef[p][ng] != 0) return false;
    }
    // 16-byte q and K loads; V loads of 8 (bf16 / f16 at d 64) or 16 bytes
    // per lane and token.
    const int es = d.f32 ? 4 : 2, e16 = 16 / es;
    const int dv = std::min(d.d / 16, e16);
    if (A.s4[d.q] != 1 || A.s3[d.q] % e16 || !aligned(d.q, e16, es)) return false;
    if (A.s3[d.kt] != 1 || A.s4[d.kt] % e16 || !aligned(d.kt, e16, es)) return false;
    if (A.s4[d.v] != 1 || A.s3[d.v] % dv || !aligned(d.v, dv, es)) return false;
    if (d.mask >= 0 && (A.s4[d.mask] != 1 || !aligned(d.mask, 1, 4))) return false;
    // Page loads use 32-bit byte offsets from the page base.
    const int64_t lim = int64_t(1) << 30;
    if (A.s4[d.kt] >= lim / (8 * es) || A.s3[d.v] >= lim / (8 * es)) return false;
    std::set<int> tids;
    for (int p : {d.q, d.kt, d.v, d.m, d.l, d.o}) tids.insert(L.targs[p]->tid);
    if (d.mask >= 0) tids.insert(L.targs[d.mask]->tid);
    if (static_cast<int>(tids.size()) != (d.mask >= 0 ? 7 : 6)) return false;
    return true;
}

uint64_t ctx_slot(RunEnv& E, uint32_t i) { return E.ctx->get_slot_u64 ? E.ctx->get_slot_u64(E.ctx->ctx, i) : 0; }

SEnv host_env(RunEnv& E, const VarList& vars) {
    return scalar_env(vars, [&E](uint64_t id) { return E.ctx->get_symbol_u64(E.ctx->ctx, id); },
                      [&E](uint32_t i) { return ctx_slot(E, i); });
}

// Evaluates the launch's masks for every grid task (mixed radix, innermost
// grid loop fastest, as the kernels decode it) and keeps those that pass.
void apply_masks(RunEnv& E, const LaunchSpec& L, BuiltLaunch& B) {
    const int ng = static_cast<int>(L.grid.size());
    VarList vars = E.host_vars;
    const size_t g0 = vars.size();
    for (int v = 0; v < ng; ++v) vars.emplace_back(L.grid[v].var, 0);
    const SEnv env = host_env(E, vars);
    std::vector<int64_t> keep;
    for (int64_t t = 0; t < B.ntasks; ++t) {
        int64_t q = t;
        for (int v = ng - 1; v >= 0; --v) {
            vars[g0 + v].second = q % B.args.ext[v];
            q /= B.args.ext[v];
        }
        bool ok = true;
        for (const Mask& mk : L.masks) ok = ok && eval_truth(*mk.pred, env) == mk.want;
        if (ok) keep.push_back(t);
    }
    if (static_cast<int64_t>(keep.size()) == B.ntasks) return;
    B.ntasks = B.args.ntasks = static_cast<int64_t>(keep.size());
    if (keep.empty()) return;
    B.tasks = std::move(keep);
    B.spec.task_list = true;
    // The GEMM and decode programs map several tasks or a cost-balanced
    // split onto a workgroup; a task list runs on the row or tile program.
    B.spec.gemm = false;
    B.spec.gemm_pingpong = false;
    B.spec.gemm_vm = B.spec.gemm_vn = -1;
    B.spec.gemm_fm = B.spec.gemm_fn = B.spec.gemm_kf = 1;
    B.spec.decode = false;
}

// A region of n u64 / i64 words in the per-run arena: (chunk, offset).
std::pair<size_t, size_t> arena_region(ptowsp_program* P, size_t n) {
    while (P->list_chunk < P->lists.size() && P->lists[P->list_chunk].cap - P->list_used < n) {
        ++P->list_chunk;
        P->list_used = 0;
    }
    if (P->list_chunk == P->lists.size()) {
        ptowsp_program::ListChunk c;
        c.cap = std::max<size_t>(n, size_t(1) << 16);
        check(hipHostMalloc(reinterpret_cast<void**>(&c.host), c.cap * 8, hipHostMallocDefault), "hipHostMalloc(arena)");
        if (hipMalloc(reinterpret_cast<void**>(&c.dev), c.cap * 8) != hipSuccess) {
            (void)hipHostFree(c.host);
            throw std::runtime_error("hipMalloc(arena) failed");
        }
        P->lists.push_back(c);
        P->list_used = 0;
    }
    const std::pair<size_t, size_t> r{P->list_chunk, P->list_used};
    P->list_used += n;
    return r;
}

// Device copy of a launch's task list (valid until the next run starts).
const int64_t* upload_task_list(RunEnv& E, const std::vector<int64_t>& tasks, hipStream_t stream) {
    ptowsp_program* P = E.P;
    const size_t n = tasks.size();
    const auto [ci, off] = arena_region(P, n);
    ptowsp_program::ListChunk& c = P->lists[ci];
    std::memcpy(c.host + off, tasks.data(), n * 8);
    check(hipMemcpyAsync(c.dev + off, c.host + off, n * 8, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(task list)");
    return c.dev + off;
}

// Host-known axis arguments of a cpp_src task (constants, symbols, host loop
// variables); grid variables are decoded in the kernel.
void custom_axis_args(RunEnv& E, const LaunchSpec& L, LaunchArgs& A) {
    const auto& args = L.task->axis_args;
    for (size_t i = 0; i < args.size() && i < static_cast<size_t>(kMaxAxisArgs); ++i) {
        const ArgRef& r = args[i];
        if (r.kind == 'c') A.aarg[i] = r.u64;
        else if (r.kind == 's') A.aarg[i] = E.ctx->get_symbol_u64(E.ctx->ctx, r.u64);
        else {
            bool grid = false;
            for (const auto& g : L.grid) grid |= g.var == r.var;
            if (grid) continue;
            bool found = false;
            for (auto h = E.host_vars.rbegin(); h != E.host_vars.rend() && !found; ++h)
                if (h->first == r.var) A.aarg[i] = static_cast<uint64_t>(h->second), found = true;
            if (!found) throw std::runtime_error("unbound loop variable '" + r.var + "'");
        }
    }
}

BuiltLaunch build_launch(RunEnv& E, const LaunchSpec& L) {
    ptowsp_program* P = E.P;
    const KernelAnalysis& a = P->ka[L.kernel];
    const KernelDef& k = P->m.kernels[L.kernel];
    BuiltLaunch B;
    LaunchArgs& A = B.args;
    const int ng = static_cast<int>(L.grid.size()), ni = static_cast<int>(L.inner.size());
    const int nvars = ng + ni;
    std::map<std::string, int> loop_index;
    for (int v = 0; v < nvars; ++v) loop_index[v < ng ? L.grid[v].var : L.inner[v - ng].var] = v;

    B.ntasks = 1;
    for (int v = 0; v < ng; ++v) {
        A.ext[v] = axis_extent(E, *L.grid[v].axis);
        if (A.ext[v] < 0) throw std::runtime_error("negative axis extent");
        B.ntasks *= A.ext[v];
    }
    A.ntasks = B.ntasks;
    int nterm = 0;
    bool dyn_inner = false;
    B.spec.inner_dyn_term.assign(ni, -1);
    auto new_term = [&]() -> IndirectTerm& {
        if (nterm >= kMaxIndirect) throw CompileError("kernel " + k.name + ": too many indirect index terms");
        return A.ind[nterm++];
    };
    // Indirect terms for tensor params first (emitted in tensor order), then extents.
    std::vector<Affine> aff(a.tensor_param_index.size());
    B.spec.indirect_count.assign(a.tensor_param_index.size(), 0);
    for (size_t p = 0; p < a.tensor_param_index.size(); ++p) {
        const TensorArg& ta = *L.targs[p];
        const TensorState& T = E.ts[ta.tid];
        const TensorInfo& ti = P->m.tensors[ta.tid];
        Affine& af = aff[p];
        af.coef.assign(nvars, 0);
        for (size_t d = 0; d < ta.idx.size(); ++d) {
            const IndexExpr& e = ta.idx[d];
            if (e.kind != 't') {
                add_affine(E, e, T.stride[d], loop_index, af);
                continue;
            }
            // Indirect: stride_d * index_tensor[affine(vars)].
            IndirectTerm& it = new_term();
            const TensorState& I = E.ts[e.tid];
            if (P->m.tensors[e.tid].dtype != DType::I32) throw std::runtime_error("index tensors must be i32");
            Affine ia;
            ia.coef.assign(nvars, 0);
            for (size_t q = 0; q < e.idx.size(); ++q) add_affine(E, e.idx[q], I.stride[q], loop_index, ia);
            it.base = reinterpret_cast<const int*>(I.dev);
            for (int v = 0; v < nvars; ++v) it.coef[v] = ia.coef[v];
            it.c = ia.c;
            it.span = I.span;
            it.bound = ti.shape[d];
            it.stride = T.stride[d];
            B.spec.indirect_count[p]++;
        }
    }
    for (int i = 0; i < ni; ++i) {
        const Axis& ax = *L.inner[i].axis;
        if (ax.kind != AxisKind::DynTensor) {
            A.ext[ng + i] = axis_extent(E, ax);
            continue;
        }
        dyn_inner = true;
        if (ax.expr.kind != 't') throw CompileError("tensor-bound extent must be an element of an i32 tensor");
        IndirectTerm& it = new_term();
        const TensorState& I = E.ts[ax.expr.tid];
        Affine ia;
        ia.coef.assign(nvars, 0);
        for (size_t q = 0; q < ax.expr.idx.size(); ++q) add_affine(E, ax.expr.idx[q], I.stride[q], loop_index, ia);
        for (int v = ng + i; v < nvars; ++v)
            if (ia.coef[v] != 0) throw CompileError("a loop extent may only depend on enclosing loops");
        it.base = reinterpret_cast<const int*>(I.dev);
        for (int v = 0; v < nvars; ++v) it.coef[v] = ia.coef[v];
        it.c = ia.c;
        it.span = I.span;
        it.bound = int64_t(1) << 40;
        it.stride = 1;
        B.spec.inner_dyn_term[i] = nterm - 1;
    }
    bool any_indirect = nterm > 0;
    for (size_t p = 0; p < a.tensor_param_index.size(); ++p) {
        const TensorArg& ta = *L.targs[p];
        const TensorState& T = E.ts[ta.tid];
        const ValueInfo* v = a.by_id[k.params[a.tensor_param_index[p]].id];
        const int es = dtype_size(v->dtype);
        int64_t s3 = 0, s4 = 1;
        if (ta.view_rank >= 2) {
            const int d3 = ta.base_rank - ta.view_rank;
            s3 = T.stride[d3];
            s4 = T.stride[d3 + 1];
        } else if (ta.view_rank == 1) {
            s4 = T.stride[ta.base_rank - 1];
        }
        A.s3[p] = s3;
        A.s4[p] = s4;
        for (int q = 0; q < nvars; ++q) A.coef[p][q] = aff[p].coef[q];
        A.base[p] = T.dev + aff[p].c * es;
        A.span[p] = T.span - aff[p].c;
        if (T.span == 0 && B.ntasks > 0)
            throw std::runtime_error("kernel " + k.name + ": param " + k.params[a.tensor_param_index[p]].name +
                                     " is bound to an empty tensor");
        // Host-side bounds check over the whole launch box (affine part only).
        if (!any_indirect && !dyn_inner && B.ntasks > 0) {
            int64_t lo = aff[p].c, hi = aff[p].c + (v->rows - 1) * s3 + (v->cols - 1) * s4;
            bool empty = false;
            for (int q = 0; q < nvars; ++q) {
                if (A.ext[q] <= 0) empty = true;
                const int64_t span = A.coef[p][q] * (A.ext[q] - 1);
                lo += std::min<int64_t>(0, span);
                hi += std::max<int64_t>(0, span);
            }
            if (!empty && (lo < 0 || hi >= T.span)) {
                std::ostringstream msg;
                msg << "kernel " << k.name << ": tiles of param " << k.params[a.tensor_param_index[p]].name << " reach elements ["
                    << lo << ", " << hi << "] of tensor " << ta.tid << ", which has " << T.span << " addressable elements";
                throw std::runtime_error(msg.str());
            }
        }
    }
    B.host_checked = !any_indirect && !dyn_inner;
    // Scalars.
    const auto& sargs = L.task->scalar_args;
    if (sargs.size() > static_cast<size_t>(kMaxScalars)) throw CompileError("too many scalar args");
    for (size_t i = 0; i < sargs.size(); ++i) {
        const ArgRef& s = sargs[i];
        if (s.kind == 'c') A.scal[i] = s.u64;
        else if (s.kind == 's') A.scal[i] = E.ctx->get_symbol_u64(E.ctx->ctx, s.u64);
        else {
            bool found = false;
            for (auto h = E.host_vars.rbegin(); h != E.host_vars.rend(); ++h)
                if (h->first == s.var) {
                    A.scal[i] = static_cast<uint64_t>(h->second);
                    found = true;
                    break;
                }
            if (!found) throw CompileError("a scalar argument bound to a grid or in-kernel loop variable is not supported");
        }
    }
    A.err = E.err ? E.err : P->d_err;
    B.spec.seq_mask = grid_write_hazard(a, L, A, B.spec, ng, nvars);
    B.spec.serial = B.spec.seq_mask != 0;
    if (B.spec.serial && !tuning().serial_groups) B.spec.seq_mask = 0;  // 0: every grid variable, one workgroup
    B.spec.row_up = tuning().row_up;
    B.spec.nontemporal = tuning().nontemporal;
    B.spec.gemm = gemm_allowed(a, L, A, B.spec, ng, nvars);
    if (!B.spec.gemm) {
        B.spec.gemm_vm = B.spec.gemm_vn = -1;
        B.spec.gemm_fm = B.spec.gemm_fn = B.spec.gemm_kf = 1;
        B.spec.gemm_pingpong = false;
    }
    B.spec.decode = decode_allowed(a, L, A, B.spec, ng);
    B.spec.row_loops = tuning().row_loops && row_loops_allowed(a, L, A, B.spec, ng, nvars);
    B.spec.decode_ring = tuning().decode_ring ? tuning().decode_ring : decode_ring_for(a.decode.d, a.decode.g, a.decode.f32);
    B.spec.decode_waves = tuning().decode_waves ? tuning().decode_waves : decode_waves_for(a.decode.d, a.decode.g, a.decode.f32);
    B.spec.decode_ordered = tuning().decode_ordered;
    B.spec.vec_width = a.family == Family::RowProgram ? pick_vec_width(a, A, nvars) : 1;
    B.spec.threads = tuning().tile_threads;
    B.spec.tile_mma = tuning().tile_mma;
    if (P->ka[L.kernel].family == Family::Custom) {
        custom_axis_args(E, L, A);
        B.spec.gemm = B.spec.decode = B.spec.gemm_pingpong = false;
    }
    if (!L.masks.empty() && B.ntasks > 0) apply_masks(E, L, B);
    return B;
}

std::string spec_key(const EmitSpec& s) {
    std::ostringstream o;
    o << "vw" << s.vec_width << (s.serial ? ";serial" + std::to_string(s.seq_mask) : "") << (s.task_list ? ";tl" : "") << ";up" << s.row_up << (s.nontemporal ? ";nt" : "")
      << (s.row_loops ? ";rl" : "") << (s.gemm ? ";gemm" : "") << ";m" << s.gemm_vm << ";n" << s.gemm_vn << ";f" << s.gemm_fm << "x" << s.gemm_fn << "x" << s.gemm_kf
      << (s.gemm_pingpong ? ";pp" : "")
      << (s.decode ? ";dec" : "")
      << (s.decode_norm ? ";norm" : "") << (s.tile_mma ? ";mma" : "") << ";t" << s.threads << ";r" << s.decode_ring << ";w" << s.decode_waves << (s.decode_ordered ? ";ord" : "")
      << ";i";
    for (int c : s.indirect_count) o << c << ",";
    o << ";d";
    for (int c : s.inner_dyn_term) o << c << ",";
    return o.str();
}

const EmittedKernel& emitted_for(ptowsp_program* P, int li, const EmitSpec& spec) {
    LaunchCache& c = P->cache[li];
    const std::string key = spec_key(spec);
    auto it = c.emitted.find(key);
    if (it != c.emitted.end()) return it->second;
    const LaunchSpec& L = P->plan.launches[li];
    EmittedKernel ek = emit_launch(P->m, P->ka[L.kernel], L, spec);
    return c.emitted.emplace(key, std::move(ek)).first->second;
}

// Launch shape of a decode kernel: one 256-thread block per CU.  The
// dynamic LDS reserved per block is just over half a CU's LDS beyond the
// kernel's own, so that no second block fits on a CU.
struct DecodeShape {
    int64_t blocks = 1;
    unsigned dyn_lds = 0;
};
DecodeShape decode_shape(hipFunction_t f, int threads) {
    static std::mutex mu;
    static std::map<std::pair<int, hipFunction_t>, DecodeShape> memo;
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    auto it = memo.find({dev, f});
    if (it != memo.end()) return it->second;
    int cus = 0, lds_cu = 0, lds_static = 0;
    check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    check(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev), "hipDeviceGetAttribute");
    check(hipFuncGetAttribute(&lds_static, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f), "hipFuncGetAttribute");
    DecodeShape r;
    const int half = lds_cu / 2 + 1024;
    r.dyn_lds = static_cast<unsigned>(std::max(0, half - lds_static));
    int per_cu = 0;
    check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, threads, r.dyn_lds),
          "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
    if (per_cu != 1)
        throw std::runtime_error("decode launch: expected one resident block per CU, occupancy reports " + std::to_string(per_cu));
    r.blocks = std::max<int64_t>(1, cus);
    memo[{dev, f}] = r;
    return r;
}

// One launch of the balanced decode kernel (emit_decode): one block per
// CU.  The program's scratch starts with kDecodeMaxUnits int32
// counters, zeroed when the scratch is allocated and left at zero by every
// launch; the partials follow, one slot per (unit, wave) pair: units + waves
// slots.
void enqueue_decode(RunEnv& E, int li, BuiltLaunch& B, const EmittedKernel& ek, const JitKernel& jk, hipStream_t stream,
                    uint64_t& launches) {
    ptowsp_program* P = E.P;
    const LaunchSpec& L = P->plan.launches[li];
    const KernelAnalysis& a = P->ka[L.kernel];
    const int ng = static_cast<int>(L.grid.size());
    const Axis& ax = *L.inner[0].axis;
    const int64_t maxp = std::max<int64_t>(0, ax.kind == AxisKind::DynTensor ? ax.max : B.args.ext[ng]);
    const DecodeShape shape = decode_shape(jk.function, ek.threads);
    const int64_t grid = shape.blocks;
    const int64_t waves = static_cast<int64_t>(ek.threads / 64) * grid;
    const size_t count_bytes = static_cast<size_t>(kDecodeMaxUnits) * sizeof(int32_t);
    const size_t part_bytes = static_cast<size_t>(B.ntasks + waves) * static_cast<size_t>(ek.part_floats) * sizeof(float);
    const size_t need = count_bytes + part_bytes;
    const int ntens = static_cast<int>(a.tensor_param_index.size());
    if (ntens >= kMaxParams) throw std::runtime_error("decode launch: no argument slot for its scratch");
    if (E.nscratch) {
        // No-allocation run: counters (zeroed at the start of the run) and
        // partials in the fixed device scratch.
        char* base = E.nscratch + kNoAllocHeaderBytes;
        if (kNoAllocHeaderBytes + need > E.nscratch_limit)
            throw std::runtime_error("ptowsp_hip_launch_noalloc: the decode launch needs " +
                                     std::to_string(kNoAllocHeaderBytes + need) + " bytes of scratch, more than the " +
                                     std::to_string(E.nscratch_limit) + " bytes available (the fixed scratch holds " +
                                     std::to_string(kNoAllocScratchBytes) + " bytes)");
        B.args.base[ntens] = base;
    } else if (need > P->scratch_bytes) {
        if (P->scratch) check(hipFree(P->scratch), "hipFree(scratch)");
        P->scratch = nullptr;
        P->scratch_bytes = 0;
        check(hipMalloc(&P->scratch, need), "hipMalloc(decode scratch)");
        check(hipMemset(P->scratch, 0, count_bytes), "hipMemset(decode counters)");
        check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        P->scratch_bytes = need;
    }
    if (!E.nscratch) B.args.base[ntens] = static_cast<char*>(P->scratch);
    B.args.span[ntens] = static_cast<int64_t>(need / sizeof(float));
    B.args.scal[kMaxScalars - 1] = static_cast<uint64_t>(maxp);
    void* params[] = {&B.args};
    launch_kernel(E, jk.function, grid, ek.threads, shape.dyn_lds, stream, params, "hipModuleLaunchKernel(decode)");
    launches += 1;
}

void enqueue_built(RunEnv& E, int li, BuiltLaunch& B, hipStream_t stream, uint64_t& launches) {
    ptowsp_program* P = E.P;
    const EmittedKernel& ek = emitted_for(P, li, B.spec);
    LaunchCache& c = P->cache[li];
    const std::string key = spec_key(B.spec);
    const JitKernel* jk;
    auto it = c.by_spec.find(key);
    if (it == c.by_spec.end()) {
        if (E.nscratch) {
            // A no-allocation run loads no code objects (loading allocates).
            jk = jit_loaded(ek.source, ek.entry);
            if (!jk)
                throw std::runtime_error("ptowsp_hip_launch_noalloc: the kernel of launch " + std::to_string(li) +
                                         " is not loaded yet; run the program once through ptowsp_hip_launch, "
                                         "which builds and loads its kernels");
        } else {
            jk = &jit_kernel(ek.source, ek.entry);
        }
        c.by_spec[key] = jk;
    } else {
        jk = it->second;
    }
    if (B.spec.decode) {
        enqueue_decode(E, li, B, ek, *jk, stream, launches);
        return;
    }
    if (B.spec.task_list) B.args.tlist = reinterpret_cast<const i64*>(upload_task_list(E, B.tasks, stream));
    const LaunchSpec& L = P->plan.launches[li];
    if (P->ka[L.kernel].family == Family::Custom) {
        ptowsp_program::CustomRun run;
        size_t grid = 1;
        for (size_t v = 0; v < L.grid.size(); ++v) {
            run.grid.push_back(L.grid[v].var);
            run.ext.push_back(B.args.ext[v]);
            grid *= static_cast<size_t>(B.args.ext[v]);
        }
        std::tie(run.chunk, run.off) = arena_region(P, grid);
        run.host = E.host_vars;
        B.args.cyc = reinterpret_cast<u64*>(P->lists[run.chunk].dev + run.off);
        P->readback.push_back({run.chunk, run.off, grid});
        P->custom_runs[L.task].push_back(std::move(run));
    }
    int64_t blocks;
    if (P->ka[L.kernel].family == Family::Custom) {
        blocks = B.spec.serial ? 1 : (B.ntasks + 63) / 64;
    } else if (ek.row_program) {
        const KernelAnalysis& a = P->ka[P->plan.launches[li].kernel];
        const int64_t rows = B.ntasks * a.rows;
        const int64_t chunks = (rows + ek.rows_per_chunk - 1) / ek.rows_per_chunk;
        blocks = (chunks + ek.waves_per_block - 1) / ek.waves_per_block;
    } else if (B.spec.serial) {
        // One workgroup per group of tasks (the grid variables outside the
        // mask); a task list runs in one workgroup.
        blocks = 1;
        const uint32_t seq = B.spec.seq_mask ? B.spec.seq_mask : 0xFFFFFFFFu;  // 0: every grid variable
        if (!B.spec.task_list)
            for (size_t v = 0; v < L.grid.size(); ++v)
                if (!((seq >> v) & 1u)) blocks *= std::max<int64_t>(1, B.args.ext[v]);
    } else {
        blocks = B.ntasks / ek.tasks_per_block * ek.blocks_per_task;
    }
    if (B.spec.gemm && !B.spec.serial) {
        // GEMM kernels run exactly one block per workgroup.
        if (blocks > 0x7FFFFFFF) throw std::runtime_error("GEMM launch: more than 2^31-1 blocks");
    } else {
        blocks = std::min<int64_t>(blocks, int64_t(1) << 20);
    }
    blocks = std::max<int64_t>(1, blocks);
    if (ek.gtile_bytes > 0) {
        // Tiles beyond LDS live in global scratch, one region per workgroup;
        // the kernel walks its tasks grid-stride, so the grid is capped (four
        // workgroups per CU of the MI355X).
        blocks = std::min<int64_t>(blocks, kGlobalTileBlocks);
        const int ntens = static_cast<int>(P->ka[L.kernel].tensor_param_index.size());
        const size_t need = static_cast<size_t>(blocks) * ek.gtile_bytes;
        if (E.nscratch)
            throw std::runtime_error("ptowsp_hip_launch_noalloc: launch " + std::to_string(li) +
                                     " keeps tiles beyond LDS in global scratch, which this entry point does not provide");
        if (need > P->gtile_bytes) {
            // Earlier launches of this run may still use the smaller region.
            if (P->gtile) {
                check(hipDeviceSynchronize(), "hipDeviceSynchronize");
                check(hipFree(P->gtile), "hipFree(tile scratch)");
            }
            P->gtile = nullptr;
            P->gtile_bytes = 0;
            check(hipMalloc(&P->gtile, need), "hipMalloc(tile scratch)");
            P->gtile_bytes = need;
        }
        B.args.base[ntens] = static_cast<char*>(P->gtile);
        B.args.span[ntens] = static_cast<int64_t>(need / sizeof(float));
    }
    void* params[] = {&B.args};
    launch_kernel(E, jk->function, blocks, ek.threads, 0, stream, params, "hipModuleLaunchKernel");
    ++launches;
}

void enqueue_launch(RunEnv& E, int li, hipStream_t stream, uint64_t& launches) {
    BuiltLaunch B = build_launch(E, E.P->plan.launches[li]);
    if (B.ntasks <= 0) return;
    enqueue_built(E, li, B, stream, launches);
}

// Launch li on the decode path with launch lj, the next one in program
// order, folded in when lj is a NormInfo kernel over the same grid, whose
// o / l tiles are the decode accumulators' and whose output overlaps no
// tensor of li.  Returns false (nothing launched) otherwise.
bool enqueue_decode_folded(RunEnv& E, int li, int lj, hipStream_t stream, uint64_t& launches) {
    ptowsp_program* P = E.P;
    const LaunchSpec &Li = P->plan.launches[li], &Lj = P->plan.launches[lj];
    const KernelAnalysis &ai = P->ka[Li.kernel], &aj = P->ka[Lj.kernel];
    if (ai.family != Family::Decode || !aj.norm.ok || !Lj.inner.empty() || Lj.grid.size() != Li.grid.size()) return false;
    if (!Li.masks.empty() || !Lj.masks.empty()) return false;
    if (aj.norm.g != ai.decode.g || aj.norm.d != ai.decode.d) return false;
    const int ntens = static_cast<int>(ai.tensor_param_index.size());
    if (ntens + 2 > kMaxParams) return false;
    BuiltLaunch Bi = build_launch(E, Li);
    if (!Bi.spec.decode || Bi.ntasks <= 0) return false;
    BuiltLaunch Bj = build_launch(E, Lj);
    if (Bj.ntasks != Bi.ntasks || Bj.spec.serial) return false;
    for (int c : Bj.spec.indirect_count)
        if (c != 0) return false;
    const int ng = static_cast<int>(Li.grid.size());
    for (int v = 0; v < ng; ++v)
        if (Bi.args.ext[v] != Bj.args.ext[v]) return false;
    auto same_view = [&](int pi, int pj) {
        if (Bi.args.base[pi] != Bj.args.base[pj] || Bi.args.s3[pi] != Bj.args.s3[pj] || Bi.args.s4[pi] != Bj.args.s4[pj])
            return false;
        for (int v = 0; v < ng; ++v)
            if (Bi.args.coef[pi][v] != Bj.args.coef[pj][v]) return false;
        return true;
    };
    if (!same_view(ai.decode.o, aj.norm.o) || !same_view(ai.decode.l, aj.norm.l)) return false;
    const int tout = Lj.targs[aj.norm.out]->tid;
    const TensorState& To = E.ts[tout];
    const char* out_lo = To.dev;
    const char* out_hi = To.dev + To.span * 4;
    for (int p = 0; p < ntens; ++p) {
        const int t = Li.targs[p]->tid;
        const TensorState& T = E.ts[t];
        const size_t es = dtype_size(P->m.tensors[t].dtype);
        if (t == tout || (T.dev < out_hi && out_lo < T.dev + T.span * static_cast<int64_t>(es))) return false;
    }
    const int q = ntens + 1, pj = aj.norm.out;
    Bi.args.base[q] = Bj.args.base[pj];
    Bi.args.span[q] = Bj.args.span[pj];
    Bi.args.s3[q] = Bj.args.s3[pj];
    Bi.args.s4[q] = Bj.args.s4[pj];
    for (int v = 0; v < kMaxVars; ++v) Bi.args.coef[q][v] = v < ng ? Bj.args.coef[pj][v] : 0;
    Bi.spec.decode_norm = true;
    enqueue_built(E, li, Bi, stream, launches);
    return true;
}

void run_host_step(RunEnv& E, const PlanItem& it, hipStream_t stream, uint64_t& launches);

void run_items(RunEnv& E, const std::vector<PlanItem>& items, hipStream_t stream, uint64_t& launches) {
    for (size_t i = 0; i < items.size(); ++i) {
        const PlanItem& it = items[i];
        if (it.ctl) {
            run_host_step(E, it, stream, launches);
            continue;
        }
        if (!it.is_loop) {
            if (i + 1 < items.size() && !items[i + 1].is_loop && !items[i + 1].ctl &&
                enqueue_decode_folded(E, it.launch, items[i + 1].launch, stream, launches)) {
                ++i;
                continue;
            }
            enqueue_launch(E, it.launch, stream, launches);
            continue;
        }
        const Axis& ax = *it.loop.axis;
        if (ax.kind == AxisKind::Select) {
            // CSR select: indices[0 .. indptr[outer]) from host symbols, in order.
            const int64_t outer = static_cast<int64_t>(E.ctx->get_symbol_u64(E.ctx->ctx, fnv1a_64(ax.a)));
            const int32_t* indptr = static_cast<const int32_t*>(E.ctx->get_symbol_ptr(E.ctx->ctx, fnv1a_64(ax.b)));
            const int32_t* indices = static_cast<const int32_t*>(E.ctx->get_symbol_ptr(E.ctx->ctx, fnv1a_64(ax.c)));
            if (outer < 0) throw std::runtime_error("P.sel: negative outer size");
            const int64_t nnz = indptr ? indptr[outer] : 0;
            E.host_vars.emplace_back(it.loop.var, 0);
            for (int64_t p = 0; p < nnz; ++p) {
                E.host_vars.back().second = indices ? indices[p] : 0;
                run_items(E, it.body, stream, launches);
            }
            E.host_vars.pop_back();
            continue;
        }
        const int64_t ub = axis_extent(E, ax);
        E.host_vars.emplace_back(it.loop.var, 0);
        for (int64_t i = 0; i < ub; ++i) {
            E.host_vars.back().second = i;
            run_items(E, it.body, stream, launches);
        }
        E.host_vars.pop_back();
    }
}

// A cond evaluated on the host, a slot set or a slot load
// (src/python/pto_codegen.cpp:2248-2303, 2458-2478).
void run_host_step(RunEnv& E, const PlanItem& it, hipStream_t stream, uint64_t& launches) {
    const Node& n = *it.ctl;
    if (n.kind == NodeKind::Cond) {
        run_items(E, eval_truth(*n.pred, host_env(E, E.host_vars)) ? it.body : it.alt, stream, launches);
        return;
    }
    uint64_t v = n.value;
    if (n.kind == NodeKind::SlotLoad) {
        // The element as the kernels enqueued so far leave it: read back
        // after the stream drains.
        const SlotElem el = slot_elem(E, n, E.host_vars);
        const TensorState& T = E.ts[n.view.tid];
        if (!E.P->slot_stage)
            check(hipHostMalloc(reinterpret_cast<void**>(&E.P->slot_stage), 64, hipHostMallocDefault), "hipHostMalloc(slot)");
        check(hipMemcpyAsync(E.P->slot_stage, T.dev + el.off * el.size, el.size, hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync(slot load)");
        check(hipStreamSynchronize(stream), "hipStreamSynchronize(slot load)");
        v = slot_value(E.P->m.tensors[n.view.tid].dtype, E.P->slot_stage);
        E.P->slot_log.push_back(v);
    }
    if (E.ctx->set_slot_u64) E.ctx->set_slot_u64(E.ctx->ctx, n.slot, v);
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// Resolves every tensor, staging host-resident ones into HBM.
void resolve_tensors(RunEnv& E, hipStream_t stream) {
    ptowsp_program* P = E.P;
    const size_t nt = P->m.tensors.size();
    E.ts.assign(nt, TensorState{});
    if (P->stage_buf.size() < nt) {
        P->stage_buf.resize(nt, nullptr);
        P->stage_bytes.resize(nt, 0);
    }
    P->copy_back.clear();
    P->h2d_ms = 0.0;
    for (size_t t = 0; t < nt; ++t) {
        const TensorInfo& ti = P->m.tensors[t];
        TensorState& T = E.ts[t];
        char* ptr = static_cast<char*>(E.ctx->get_tensor_ptr(E.ctx->ctx, static_cast<uint32_t>(t)));
        T.stride.resize(ti.shape.size());
        int64_t span = 1;
        for (size_t d = 0; d < ti.shape.size(); ++d) {
            T.stride[d] = static_cast<int64_t>(E.ctx->get_tensor_stride(E.ctx->ctx, static_cast<uint32_t>(t), static_cast<uint32_t>(d)));
            if (ti.shape[d] == 0) span = 0;
        }
        if (span) {
            int64_t mx = 0;
            for (size_t d = 0; d < ti.shape.size(); ++d) {
                if (T.stride[d] < 0) throw std::runtime_error("tensor " + std::to_string(t) + ": negative strides are not supported");
                mx += (ti.shape[d] - 1) * T.stride[d];
            }
            span = mx + 1;
        }
        T.span = span;
        T.bytes = static_cast<size_t>(span) * dtype_size(ti.dtype);
        T.written = P->tensor_written[t];
        if (span == 0) continue;
        if (!ptr) throw std::runtime_error("tensor " + std::to_string(t) + " has no data");
        if (is_device_pointer(ptr)) {
            T.dev = ptr;
            continue;
        }
        T.host = ptr;
        T.staged = true;
        if (P->stage_bytes[t] < T.bytes) {
            if (P->stage_buf[t]) check(hipFree(P->stage_buf[t]), "hipFree");
            P->stage_buf[t] = nullptr;
            check(hipMalloc(&P->stage_buf[t], T.bytes), "hipMalloc(staging)");
            P->stage_bytes[t] = T.bytes;
        }
        T.dev = static_cast<char*>(P->stage_buf[t]);
        const auto t0 = std::chrono::steady_clock::now();
        check(hipMemcpyAsync(T.dev, T.host, T.bytes, hipMemcpyHostToDevice, stream), "hipMemcpyAsync(H2D)");
        check(hipStreamSynchronize(stream), "hipStreamSynchronize(H2D)");
        P->h2d_ms += ms_since(t0);
        if (T.written) P->copy_back.push_back({T.host, T.dev, T.bytes});
    }
}

CycleResult cycles_for(RunEnv& E) {
    ptowsp_program* P = E.P;
    CycleEnv env;
    env.axis_size = [&](const std::string& n) { return E.ctx->get_axis_size(E.ctx->ctx, n.c_str()); };
    env.symbol_u64 = [&](uint64_t id) { return E.ctx->get_symbol_u64(E.ctx->ctx, id); };
    env.symbol_ptr = [&](uint64_t id) { return static_cast<const int32_t*>(E.ctx->get_symbol_ptr(E.ctx->ctx, id)); };
    std::ostringstream key;
    std::function<void(const Node*)> walk = [&](const Node* n) {
        if (!n) return;
        if (n->kind == NodeKind::Select) {
            // The selected index list (its contents decide the tasks).
            const Axis& a = n->axis;
            const int64_t outer = static_cast<int64_t>(env.symbol_u64(fnv1a_64(a.a)));
            const int32_t* indptr = env.symbol_ptr(fnv1a_64(a.b));
            const int32_t* indices = env.symbol_ptr(fnv1a_64(a.c));
            key << "s" << outer << ":";
            if (indptr && outer >= 0) {
                for (int64_t i = 0; i <= outer; ++i) key << indptr[i] << ",";
                key << "|";
                if (indices)
                    for (int64_t i = 0; i < indptr[outer]; ++i) key << indices[i] << ",";
            }
            key << ";";
        }
        if (n->kind == NodeKind::ParallelFor || n->kind == NodeKind::ForEach) {
            const Axis& a = n->axis;
            if (a.kind == AxisKind::Dyn) key << "d" << a.a << "=" << env.axis_size(a.a) << ";";
            if (a.kind == AxisKind::Ragged) {
                const int64_t outer = static_cast<int64_t>(env.symbol_u64(fnv1a_64(a.a)));
                key << "r" << outer << ":";
                if (const int32_t* len = env.symbol_ptr(fnv1a_64(a.b)))
                    for (int64_t i = 0; i < outer; ++i) key << len[i] << ",";
                key << ";";
            }
            if (a.kind == AxisKind::DynTensor) {
                // Key on the whole extent tensor's contents (small: one count per outer index).
                const int tid = a.expr.tid;
                const TensorState& t = E.ts[tid];
                uint64_t h = 0xcbf29ce484222325ull;
                auto mix = [&](int32_t x) {
                    for (int b = 0; b < 4; ++b) h = (h ^ ((static_cast<uint32_t>(x) >> (8 * b)) & 0xFF)) * 0x100000001b3ull;
                };
                if (t.host)
                    for (int64_t i = 0; i < t.span; ++i) mix(reinterpret_cast<const int32_t*>(t.host)[i]);
                else
                    for (int32_t x : index_host_copy(E, tid)) mix(x);
                key << "t" << tid << ":" << t.span << ":" << h << ";";
            }
        }
        walk(n->body.get());
        for (const auto& c : n->kids) walk(c.get());
    };
    walk(P->m.root.get());
    const bool dynamic = module_is_dynamic(P->m);
    if (!dynamic && P->cycles_valid && P->cycle_key == key.str()) return P->cycles;
    env.index_value = [&](const IndexExpr& e, const std::vector<std::pair<std::string, int64_t>>& vars) {
        return eval_index_host(E, e, vars);
    };
    env.slot_init = [&](uint32_t i) { return i < P->slot_start.size() ? P->slot_start[i] : ctx_slot(E, i); };
    size_t replayed = 0;
    env.slot_load = [&](const Node& n, const VarList& vars) -> uint64_t {
        if (E.replay_slots) {
            if (replayed >= P->slot_log.size()) throw std::runtime_error("internal: more slot loads than the run made");
            return P->slot_log[replayed++];
        }
        const SlotElem el = slot_elem(E, n, vars);
        const TensorState& T = E.ts[n.view.tid];
        unsigned char buf[8] = {};
        if (T.host) std::memcpy(buf, T.host + el.off * el.size, el.size);
        else check(hipMemcpy(buf, T.dev + el.off * el.size, el.size, hipMemcpyDeviceToHost), "hipMemcpy(slot load)");
        return slot_value(P->m.tensors[n.view.tid].dtype, buf);
    };
    if (!P->custom_runs.empty())
        env.custom_cycles = [&](const Node& n, const VarList& vars) -> uint64_t {
            auto value = [&](const std::string& name) -> int64_t {
                for (auto it = vars.rbegin(); it != vars.rend(); ++it)
                    if (it->first == name) return it->second;
                throw std::runtime_error("internal: loop variable '" + name + "' of a cpp_src task not bound");
            };
            auto it = P->custom_runs.find(&n);
            if (it != P->custom_runs.end())
                for (const auto& run : it->second) {
                    bool same = true;
                    for (const auto& [name, v] : run.host) same = same && value(name) == v;
                    if (!same) continue;
                    size_t g = 0;
                    for (size_t d = 0; d < run.grid.size(); ++d) g = g * static_cast<size_t>(run.ext[d]) + static_cast<size_t>(value(run.grid[d]));
                    return static_cast<uint64_t>(P->lists[run.chunk].host[run.off + g]);
                }
            throw std::runtime_error("internal: no run of cpp_src kernel task");
        };
    CycleResult r = run_cycle_model(P->m, P->ka, env);
    if (dynamic) return r;
    P->cycle_key = key.str();
    P->cycles = r;
    P->cycles_valid = true;
    return r;
}

// Tensors holding loop extents (DenseDyn bound to a tensor) that live on the
// device: the cycle-model key reads their contents.
std::vector<int> device_extent_tensors(RunEnv& E) {
    std::vector<int> out;
    std::function<void(const Node*)> walk = [&](const Node* n) {
        if (!n) return;
        if ((n->kind == NodeKind::ParallelFor || n->kind == NodeKind::ForEach) && n->axis.kind == AxisKind::DynTensor) {
            const int tid = n->axis.expr.tid;
            if (!E.ts[tid].host && std::find(out.begin(), out.end(), tid) == out.end()) out.push_back(tid);
        }
        walk(n->body.get());
        for (const auto& c : n->kids) walk(c.get());
    };
    walk(E.P->m.root.get());
    return out;
}

// Copies the device extent tensors into pinned memory on `stream` and keeps
// what the cycle model needs at synchronize().  The copy must see the values
// the launches start from: it is enqueued ahead of the kernels when a launch
// writes one of the tensors (`before`), and after them otherwise, so that it
// does not delay the first kernel.
void defer_cycles(RunEnv& E, const std::vector<int>& tids, hipStream_t stream) {
    ptowsp_program* P = E.P;
    size_t total = 0;
    P->deferred_tids.clear();
    for (int tid : tids) {
        P->deferred_tids.push_back({tid, total});
        total += static_cast<size_t>(std::max<int64_t>(E.ts[tid].span, 0));
    }
    P->deferred_ts = E.ts;
    P->deferred_ctx = E.ctx;
    P->cycles_deferred = true;
    if (E.nscratch) {
        // No-allocation run: device-to-device copies into the tail of the
        // fixed scratch (reserved by the entry point), read back at synchronize.
        int32_t* dst = reinterpret_cast<int32_t*>(E.nscratch + E.nscratch_limit);
        for (const auto& [tid, off] : P->deferred_tids) {
            const size_t n = static_cast<size_t>(std::max<int64_t>(E.ts[tid].span, 0));
            if (n)
                check(hipMemcpyAsync(dst + off, E.ts[tid].dev, n * 4, hipMemcpyDeviceToDevice, stream),
                      "hipMemcpyAsync(extent tensor)");
        }
        P->deferred_dev = dst;
        return;
    }
    P->deferred_dev = nullptr;
    if (total > P->key_stage_elems) {
        if (P->key_stage) check(hipHostFree(P->key_stage), "hipHostFree(key stage)");
        P->key_stage = nullptr;
        P->key_stage_elems = 0;
        check(hipHostMalloc(reinterpret_cast<void**>(&P->key_stage), total * 4, hipHostMallocDefault), "hipHostMalloc(key stage)");
        P->key_stage_elems = total;
    }
    for (const auto& [tid, off] : P->deferred_tids) {
        const size_t n = static_cast<size_t>(std::max<int64_t>(E.ts[tid].span, 0));
        if (n)
            check(hipMemcpyAsync(P->key_stage + off, E.ts[tid].dev, n * 4, hipMemcpyDeviceToHost, stream),
                  "hipMemcpyAsync(extent tensor)");
    }
}

// Both launch entry points.  noalloc: the run allocates no device or pinned
// memory: every tensor must already be in device memory, the kernels' error
// flag and the decode scratch live in the fixed device scratch of
// noalloc.hip, the deferred cycle-model input is copied there too, and
// features whose host steps need staging buffers are refused.
int launch_impl(ptowsp_program* P, RuntimeContext* ctx, void* hip_stream, ptowsp_run_info* info, bool noalloc) {
    if (!P || !ctx) throw std::runtime_error("null argument");
    if (P->pending) throw std::runtime_error("Program already started");
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    bool custom = false;
    for (const auto& k : P->m.kernels) custom |= k.custom;
    RunEnv E{P, ctx, {}, {}, {}};
    if (noalloc) {
        const char* who = "ptowsp_hip_launch_noalloc: ";
        if (custom) throw std::runtime_error(std::string(who) + "cpp_src kernels read their per-task cycles back through staging memory");
        if (module_loads_slots(P->m)) throw std::runtime_error(std::string(who) + "slot loads read tensors back through staging memory");
        for (const auto& L : P->plan.launches)
            if (!L.masks.empty())
                throw std::runtime_error(std::string(who) + "masked launches upload task lists through staging memory");
        // Every tensor must be device memory: host tensors would need staging buffers.
        const size_t nt = P->m.tensors.size();
        for (size_t t = 0; t < nt; ++t) {
            bool empty = false;
            for (int64_t d : P->m.tensors[t].shape) empty |= d == 0;
            if (empty) continue;
            const void* ptr = ctx->get_tensor_ptr(ctx->ctx, static_cast<uint32_t>(t));
            if (ptr && !is_device_pointer(ptr))
                throw std::runtime_error(std::string(who) + "tensor " + std::to_string(t) +
                                         " is host memory; this entry point needs device-resident tensors");
        }
        E.nscratch = static_cast<char*>(noalloc_scratch());
        E.err = reinterpret_cast<int*>(E.nscratch);
        E.timing = P->have_events;
    } else {
        noalloc_prepare(stream);
        if (!P->h_err) {
            check(hipHostMalloc(reinterpret_cast<void**>(&P->h_err), sizeof(int), hipHostMallocMapped | hipHostMallocCoherent),
                  "hipHostMalloc(err)");
            __atomic_store_n(P->h_err, 0, __ATOMIC_RELAXED);
            check(hipHostGetDevicePointer(reinterpret_cast<void**>(&P->d_err), P->h_err, 0), "hipHostGetDevicePointer(err)");
        }
        if (!P->have_events) {
            // Timing-only events: no system-scope fence (cache writeback) of
            // their own, which would otherwise be counted as device time.
            check(hipEventCreateWithFlags(&P->ev0, hipEventDisableSystemFence), "hipEventCreate");
            check(hipEventCreateWithFlags(&P->ev1, hipEventDisableSystemFence), "hipEventCreate");
            P->have_events = true;
        }
    }
    resolve_tensors(E, stream);
    P->cycles_deferred = false;
    P->deferred_dev = nullptr;
    P->list_chunk = P->list_used = 0;
    P->custom_runs.clear();
    P->readback.clear();
    P->slot_log.clear();
    P->slot_start.assign(256, 0);
    for (uint32_t i = 0; i < 256; ++i) P->slot_start[i] = ctx_slot(E, i);
    // A slot load reads what the kernels before it wrote: the cycle model
    // replays the values the run read, after the run.
    const bool slot_loads = module_loads_slots(P->m) || custom;
    const std::vector<int> dev_ext = device_extent_tensors(E);
    if (noalloc) {
        // The extent copies sit at the tail of the scratch; the decode
        // launches may use everything before them.
        size_t ext_bytes = 0;
        for (int tid : dev_ext) ext_bytes += static_cast<size_t>(std::max<int64_t>(E.ts[tid].span, 0)) * 4;
        ext_bytes = (ext_bytes + 255) / 256 * 256;
        if (ext_bytes + kNoAllocHeaderBytes + kDecodeMaxUnits * sizeof(int32_t) > kNoAllocScratchBytes)
            throw std::runtime_error("ptowsp_hip_launch_noalloc: the loop-extent tensors (" + std::to_string(ext_bytes) +
                                     " bytes) do not fit in the fixed scratch of " + std::to_string(kNoAllocScratchBytes) +
                                     " bytes");
        E.nscratch_limit = kNoAllocScratchBytes - ext_bytes;
        // The error flag and the decode unit counters start at zero.
        noalloc_zero(E.nscratch, kNoAllocHeaderBytes + kDecodeMaxUnits * sizeof(int32_t), stream);
    }
    CycleResult cyc{};
    bool ext_written = false;
    for (int tid : dev_ext) ext_written |= E.ts[tid].written;
    if (dev_ext.empty() && !slot_loads) cyc = cycles_for(E);
    else if (!dev_ext.empty() && ext_written) defer_cycles(E, dev_ext, stream);
    uint64_t launches = 0;
    run_items(E, P->plan.items, stream, launches);
    if (custom) {
        // The cpp_src tasks' cycles: copied back after the kernels, the
        // model runs at synchronize().
        if (dev_ext.empty()) P->deferred_tids.clear();
        for (const auto& r : P->readback) {
            ptowsp_program::ListChunk& c = P->lists[r[0]];
            if (r[2])
                check(hipMemcpyAsync(c.host + r[1], c.dev + r[1], r[2] * 8, hipMemcpyDeviceToHost, stream),
                      "hipMemcpyAsync(task cycles)");
        }
        P->deferred_ts = E.ts;
        P->deferred_ctx = E.ctx;
        P->cycles_deferred = true;
    } else if (dev_ext.empty() && slot_loads) {
        E.replay_slots = true;
        cyc = cycles_for(E);
    }
    start_timing(E, stream);
    if (E.timing) check(hipEventRecord(P->ev1, stream), "hipEventRecord");
    // After the end event: the copy is not device time of the program.
    if (!dev_ext.empty() && !ext_written) defer_cycles(E, dev_ext, stream);
    check(hipGetLastError(), "kernel launch");
    P->stream = stream;
    P->pending = true;
    P->timed = E.timing;
    P->noalloc_run = noalloc;
    P->noalloc_err = E.err;
    P->last_run = ptowsp_run_info{cyc.total_cycles, cyc.tasks, static_cast<uint32_t>(launches), 0};
    if (P->cycles_deferred) P->last_run.total_cycles = P->last_run.task_count = UINT64_MAX;
    if (info) *info = P->last_run;
    return 0;
}

int fail(const std::exception& e) {
    g_last_error = e.what();
    return -1;
}

}  // namespace

extern "C" {

const char* ptowsp_hip_last_error(void) { return g_last_error.c_str(); }

int ptowsp_hip_compile(const char* module_text, ptowsp_program** out) {
    try {
        if (!module_text || !out) throw std::runtime_error("null argument");
        auto P = std::make_unique<ptowsp_program>();
        P->m = parse_module(module_text);
        for (const auto& k : P->m.kernels) P->ka.push_back(analyze_kernel(k));
        P->plan = build_plan(P->m, P->ka);
        P->cache.resize(P->plan.launches.size());
        P->tensor_written.assign(P->m.tensors.size(), false);
        for (const auto& L : P->plan.launches) {
            const KernelAnalysis& a = P->ka[L.kernel];
            for (size_t p = 0; p < L.targs.size(); ++p)
                if (a.stored[p]) P->tensor_written[L.targs[p]->tid] = true;
        }
        *out = P.release();
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

void ptowsp_hip_release(ptowsp_program* prog) { delete prog; }

int ptowsp_hip_num_launches(const ptowsp_program* prog) { return prog ? static_cast<int>(prog->plan.launches.size()) : -1; }

uint64_t ptowsp_hip_kernel_cycles(const ptowsp_program* prog, const char* kernel) {
    if (!prog || !kernel) return UINT64_MAX;
    for (size_t i = 0; i < prog->m.kernels.size(); ++i)
        if (prog->m.kernels[i].name == kernel) return prog->ka[i].cycles;
    return UINT64_MAX;
}

int ptowsp_hip_kernel_family(const ptowsp_program* prog, const char* kernel) {
    if (!prog || !kernel) return -1;
    for (size_t i = 0; i < prog->m.kernels.size(); ++i)
        if (prog->m.kernels[i].name == kernel) return static_cast<int>(prog->ka[i].family);
    return -1;
}

int ptowsp_hip_precompile(ptowsp_program* P, int index, int flags, const char** source) {
    try {
        if (!P) throw std::runtime_error("null program");
        for (size_t li = 0; li < P->plan.launches.size(); ++li) {
            const LaunchSpec& L = P->plan.launches[li];
            const KernelAnalysis& a = P->ka[L.kernel];
            EmitSpec spec;
            spec.serial = (flags & 1) != 0;
            spec.seq_mask = spec.serial ? static_cast<uint32_t>((flags >> 8) & 0xFF) : 0u;
            spec.row_loops = (flags & 16) && !spec.serial && a.family == Family::RowProgram && !L.inner.empty();
            spec.row_up = tuning().row_up;
            spec.nontemporal = tuning().nontemporal;
            spec.gemm = a.family == Family::Gemm && !spec.serial;
            spec.decode = a.family == Family::Decode && !spec.serial && L.inner.size() == 1;
            spec.decode_ring = tuning().decode_ring ? tuning().decode_ring : decode_ring_for(a.decode.d, a.decode.g, a.decode.f32);
            spec.decode_waves = tuning().decode_waves ? tuning().decode_waves : decode_waves_for(a.decode.d, a.decode.g, a.decode.f32);
            spec.decode_ordered = tuning().decode_ordered;
            spec.decode_norm = spec.decode && (flags & 32) != 0;
            spec.indirect_count.assign(L.targs.size(), 0);
            for (size_t p = 0; p < L.targs.size(); ++p)
                for (const auto& e : L.targs[p]->idx)
                    if (e.kind == 't') spec.indirect_count[p]++;
            spec.inner_dyn_term.assign(L.inner.size(), -1);
            int term = 0;
            for (int c : spec.indirect_count) term += c;
            for (size_t i = 0; i < L.inner.size(); ++i)
                if (L.inner[i].axis->kind == AxisKind::DynTensor) spec.inner_dyn_term[i] = term++;
            if (a.family == Family::RowProgram) {
                // Contiguous row-major views: vector width limited by the row length and row strides.
                int vw = 4;
                while (vw > 1 && a.cols % vw) vw /= 2;
                for (size_t p = 0; p < L.targs.size(); ++p) {
                    const auto& shape = P->m.tensors[L.targs[p]->tid].shape;
                    if (L.targs[p]->view_rank >= 2 && !shape.empty())
                        while (vw > 1 && shape.back() % vw) vw /= 2;
                }
                spec.vec_width = vw;
            }
            const int ng = static_cast<int>(L.grid.size());
            if ((flags & 2) && spec.gemm && ng >= 2 && a.gemm.m <= 128 && a.gemm.n <= 128 &&
                2 * (2 * a.gemm.m + 2 * a.gemm.n) * a.gemm.k * 2 <= 160 * 1024) {
                spec.gemm_vm = ng - 2;
                spec.gemm_vn = ng - 1;
                spec.gemm_fm = spec.gemm_fn = 2;
                spec.gemm_pingpong = (flags & 4) && a.gemm.m == 128 && a.gemm.n == 128 && (a.gemm.k == 64 || a.gemm.k == 32);
            }
            // Blocks below the MFMA block shape: the tile program.
            if (spec.gemm && ((a.gemm.m * spec.gemm_fm) % 64 || (a.gemm.n * spec.gemm_fn) % 64)) {
                spec.gemm = spec.gemm_pingpong = false;
                spec.gemm_vm = spec.gemm_vn = -1;
                spec.gemm_fm = spec.gemm_fn = 1;
            }
            const EmittedKernel& ek = emitted_for(P, static_cast<int>(li), spec);
            (void)jit_compile(ek.source);
            if (static_cast<int>(li) == index) P->precompiled_source = ek.source;
        }
        if (source) *source = P->precompiled_source.c_str();
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int ptowsp_hip_cycle_model(ptowsp_program* P, RuntimeContext* ctx, ptowsp_run_info* info) {
    try {
        if (!P || !ctx) throw std::runtime_error("null argument");
        RunEnv E{P, ctx, {}, {}, {}};
        P->slot_start.clear();  // the model starts from the context's slots
        const size_t nt = P->m.tensors.size();
        E.ts.assign(nt, TensorState{});
        for (size_t t = 0; t < nt; ++t) {
            const TensorInfo& ti = P->m.tensors[t];
            TensorState& T = E.ts[t];
            T.stride.resize(ti.shape.size());
            int64_t span = 1;
            bool empty = false;
            for (size_t d = 0; d < ti.shape.size(); ++d) {
                T.stride[d] = static_cast<int64_t>(ctx->get_tensor_stride(ctx->ctx, static_cast<uint32_t>(t), static_cast<uint32_t>(d)));
                if (ti.shape[d] == 0) empty = true;
                else span += (ti.shape[d] - 1) * T.stride[d];
            }
            T.span = empty ? 0 : span;
            char* ptr = static_cast<char*>(ctx->get_tensor_ptr(ctx->ctx, static_cast<uint32_t>(t)));
            if (ptr && is_device_pointer(ptr)) T.dev = ptr;
            else T.host = ptr;
        }
        const CycleResult cyc = cycles_for(E);
        if (info) {
            info->total_cycles = cyc.total_cycles;
            info->task_count = cyc.tasks;
            info->launches = 0;
            info->reserved = 0;
        }
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int ptowsp_hip_launch(ptowsp_program* P, RuntimeContext* ctx, void* hip_stream, ptowsp_run_info* info) {
    try {
        return launch_impl(P, ctx, hip_stream, info, false);
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int ptowsp_hip_launch_noalloc(ptowsp_program* P, RuntimeContext* ctx, void* hip_stream, ptowsp_run_info* info) {
    try {
        return launch_impl(P, ctx, hip_stream, info, true);
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int ptowsp_hip_synchronize(ptowsp_program* P, ptowsp_timing* timing) {
    try {
        if (!P) throw std::runtime_error("null program");
        if (!P->pending) {
            if (timing) *timing = ptowsp_timing{0.0, 0.0, 0.0};
            return 0;
        }
        P->pending = false;
        check(hipStreamSynchronize(P->stream), "hipStreamSynchronize");
        if (P->cycles_deferred) {
            P->cycles_deferred = false;
            RunEnv E{P, P->deferred_ctx, P->deferred_ts, {}, {}};
            E.replay_slots = module_loads_slots(P->m);
            for (const auto& [tid, off] : P->deferred_tids) {
                const size_t n = static_cast<size_t>(std::max<int64_t>(E.ts[tid].span, 0));
                if (P->deferred_dev) {
                    std::vector<int32_t> v(n);
                    if (n) check(hipMemcpy(v.data(), P->deferred_dev + off, n * 4, hipMemcpyDeviceToHost), "hipMemcpy(extent tensor)");
                    E.idx_host[tid] = std::move(v);
                } else {
                    E.idx_host[tid] = std::vector<int32_t>(P->key_stage + off, P->key_stage + off + n);
                }
            }
            const CycleResult cyc = cycles_for(E);
            P->last_run.total_cycles = cyc.total_cycles;
            P->last_run.task_count = cyc.tasks;
        }
        float dev_ms = 0.0f;
        if (P->timed) check(hipEventElapsedTime(&dev_ms, P->ev0, P->ev1), "hipEventElapsedTime");
        const auto t0 = std::chrono::steady_clock::now();
        for (const auto& cb : P->copy_back) check(hipMemcpy(cb.host, cb.dev, cb.bytes, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
        const double d2h = ms_since(t0);
        P->copy_back.clear();
        int err = 0;
        if (P->noalloc_run) check(hipMemcpy(&err, P->noalloc_err, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(error flag)");
        else err = __atomic_load_n(P->h_err, __ATOMIC_ACQUIRE);
        if (err) {
            if (!P->noalloc_run) __atomic_store_n(P->h_err, 0, __ATOMIC_RELAXED);
            throw std::runtime_error(err == 1   ? "an indirect tensor index was out of range (tasks skipped)"
                                     : err == 3 ? "a loop extent read from a tensor exceeded its declared maximum"
                                                : "a task's tile fell outside its tensor (tasks skipped)");
        }
        if (timing) *timing = ptowsp_timing{static_cast<double>(dev_ms), P->h2d_ms, d2h};
        return 0;
    } catch (const std::exception& e) {
        return fail(e);
    }
}

int ptowsp_hip_run_result(const ptowsp_program* P, ptowsp_run_info* info) {
    if (!P || !info) {
        g_last_error = "null argument";
        return -1;
    }
    if (P->pending) {
        g_last_error = "the run has not been synchronized";
        return -1;
    }
    *info = P->last_run;
    return 0;
}

uint64_t ptowsp_hip_workload_main(ptowsp_program* prog, RuntimeContext* ctx, CSPTContext* cspt) {
    (void)cspt;
    if (ptowsp_hip_launch(prog, ctx, nullptr, nullptr) != 0) return 0;
    if (ptowsp_hip_synchronize(prog, nullptr) != 0) return 0;
    return prog->last_run.total_cycles;
}

ptowsp_runtime* ptowsp_rt_create(void) {
    auto* rt = new ptowsp_runtime();
    rt->ctx.get_axis_size = rt_axis;
    rt->ctx.get_symbol_u64 = rt_sym;
    rt->ctx.get_symbol_ptr = rt_symp;
    rt->ctx.get_slot_u64 = rt_slot;
    rt->ctx.set_slot_u64 = rt_set_slot;
    rt->ctx.get_tensor_ptr = rt_tptr;
    rt->ctx.get_tensor_stride = rt_tstride;
    rt->ctx.get_kernel = rt_kernel;
    rt->ctx.ctx = rt;
    return rt;
}

void ptowsp_rt_destroy(ptowsp_runtime* rt) { delete rt; }

int ptowsp_rt_set_tensor(ptowsp_runtime* rt, uint32_t tid, void* ptr, uint32_t ndim, const int64_t* strides) {
    if (!rt || (ndim && !strides)) return -1;
    auto& t = rt->tensors[tid];
    t.ptr = ptr;
    t.strides.assign(strides, strides + ndim);
    return 0;
}

int ptowsp_rt_set_axis_size(ptowsp_runtime* rt, const char* name, int64_t size) {
    if (!rt || !name) return -1;
    rt->axis[name] = size;
    return 0;
}

int ptowsp_rt_set_symbol_u64(ptowsp_runtime* rt, uint64_t id, uint64_t value) {
    if (!rt) return -1;
    rt->sym[id] = value;
    return 0;
}

int ptowsp_rt_set_symbol_ptr(ptowsp_runtime* rt, uint64_t id, void* ptr) {
    if (!rt) return -1;
    rt->symp[id] = ptr;
    return 0;
}

int ptowsp_rt_reset_slots(ptowsp_runtime* rt) {
    if (!rt) return -1;
    std::fill(rt->slots.begin(), rt->slots.end(), 0);
    return 0;
}

void ptowsp_rt_clear(ptowsp_runtime* rt) {
    if (!rt) return;
    rt->tensors.clear();
    rt->axis.clear();
    rt->sym.clear();
    rt->symp.clear();
    std::fill(rt->slots.begin(), rt->slots.end(), 0);
}

RuntimeContext* ptowsp_rt_context(ptowsp_runtime* rt) { return rt ? &rt->ctx : nullptr; }

}  // extern "C"
