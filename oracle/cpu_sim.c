/* CPU oracle: a plain-C restatement of the reference's cpu_sim artifact.
 * TEST INFRASTRUCTURE ONLY (see cpu_sim.h).  Every semantic choice below
 * cites the reference line it restates.  Single-threaded, -O2, no
 * fast-math and no FMA contraction (the reference builds its artifacts
 * -O3 without fast-math, src/pto/wsp/codegen/cmake_compiler.cpp:235-236).
 */
#include "cpu_sim.h"

#include <math.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* errors + arena                                                       */
/* ------------------------------------------------------------------ */

static __thread char g_err[1024];
static __thread jmp_buf* g_jmp;
static __thread uint64_t g_tasks;

static void fail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    longjmp(*g_jmp, 1);
}

typedef struct Block { struct Block* next; size_t used, cap; unsigned char data[]; } Block;
static __thread Block* g_arena;

static void* alloc(size_t n) {
    n = (n + 15) & ~(size_t)15;
    if (!g_arena || g_arena->used + n > g_arena->cap) {
        size_t cap = n > (1u << 20) ? n : (1u << 20);
        Block* b = (Block*)malloc(sizeof(Block) + cap);
        if (!b) fail("out of memory");
        b->next = g_arena;
        b->used = 0;
        b->cap = cap;
        g_arena = b;
    }
    void* p = g_arena->data + g_arena->used;
    g_arena->used += n;
    memset(p, 0, n);
    return p;
}

static void arena_free(void) {
    while (g_arena) {
        Block* n = g_arena->next;
        free(g_arena);
        g_arena = n;
    }
}

/* ------------------------------------------------------------------ */
/* module data model (mirrors include/pto/wsp/ir/codegen.hpp:22-77)     */
/* ------------------------------------------------------------------ */

enum { DT_F16, DT_BF16, DT_F32, DT_F64, DT_I8, DT_I16, DT_I32, DT_I64, DT_U8, DT_U16, DT_U32, DT_U64, DT_BOOL };
static const char* k_dtype_names[] = {"f16", "bf16", "f32", "f64", "i8", "i16", "i32",
                                      "i64", "u8", "u16", "u32", "u64", "bool"};
static const int k_dtype_size[] = {2, 2, 4, 8, 1, 2, 4, 8, 1, 2, 4, 8, 1};

static int is_float_dt(int dt) { return dt == DT_F16 || dt == DT_BF16 || dt == DT_F32 || dt == DT_F64; }

typedef struct { int dtype, rank; int64_t shape[8]; } TensorInfo;
typedef struct { int id, dtype, tile, rows, cols; } Val;
typedef struct { char* name; int id; } Param;
struct SX;
typedef struct {
    int kind; int result; int nopnd; int* opnd; int has_value; double value;
    int has_k, has_cols, has_cycles; int64_t k, cols, cycles; /* integer attrs */
    struct SX* cycles_expr; /* CpuSimAddCycles: cycles as an expression of the kernel's scalars */
} Op;

enum { OP_LOAD, OP_STORE, OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MAX, OP_MIN, OP_EXP, OP_RSQRT,
       OP_ROWSUM, OP_ROWMAX, OP_ROWMEAN, OP_MATMUL, OP_CONSTANT,
       OP_IOTA_U32, OP_TSORT32, OP_EXTRACT_TOPK, OP_TMOV, OP_STORE_TOPK, OP_ADD_CYCLES, OP_OTHER };

typedef struct {
    char* name;
    int nvals, nparams, nops, custom, max_id;
    Val* vals;
    Param* params;
    Op* ops;
    /* derived */
    Val** by_id;          /* value id -> Val */
    int* param_of;        /* value id -> param index or -1 */
    int* tensor_index;    /* param index -> tensor-param ordinal or -1 */
    int ntensor_params;
    unsigned char* preload; /* value id -> 1 if the param tile is TLOADed at entry */
    unsigned char* acc_vec; /* value id -> 1 if a matmul result feeds a vector op */
} Kernel;

typedef struct IExpr {
    char kind; /* v c a t */
    char* var;
    int64_t c;
    int nterms;
    char** tvars;
    int64_t* coefs;
    int tid, base_rank, nidx;
    struct IExpr* idx;
} IExpr;

typedef struct { char kind; char* var; uint64_t u64; } Arg; /* v c s */

/* Scalar expression (the reference's ScalarExpr, include/pto/wsp/ir/ as
 * emitted by src/python/pto_codegen.cpp:220-300). ty: 'b' bool, 'i' int64_t,
 * 'u' uint64_t. kind: L literal, P task param, G task tag, A axis var,
 * Y symbol, S slot, U unary, B binary, T ternary, C cast, K kernel scalar
 * parameter (cycle expressions of PTO-ISA kernels). */
typedef struct SX {
    char kind, ty;
    uint64_t u;
    char op[4];
    struct SX *a, *b, *c;
} SX;
typedef struct { char* param; int tid, base_rank, view_rank, nidx; IExpr* idx; } TArg;

enum { N_EMPTY, N_PFOR, N_EACH, N_COMB, N_SEQN, N_TASK, N_SEL, N_COND, N_SLOTSET, N_SLOTLD };
enum { AX_DENSE, AX_DYN, AX_RAGGED, AX_DYNT };

typedef struct Node {
    int kind;
    char* var;
    int axis_kind;
    int64_t axis_size;
    char *axis_a, *axis_b;
    IExpr* axis_expr;
    struct Node* body;
    int nkids;
    struct Node** kids;
    char* kernel_name;
    Kernel* kernel;
    int naxis, nscal, nten;
    Arg *axis, *scal;
    TArg* ten;
    char *sel_outer, *sel_indptr, *sel_indices;
    SX* pred;                     /* cond */
    uint32_t slot;                /* slot set / load */
    uint64_t slot_value;
    TArg slot_view;
    int64_t slot_row, slot_col;
} Node;

typedef struct {
    int ntensors, nkernels;
    TensorInfo* tensors;
    Kernel* kernels;
    Node* root;
    int has_dispatch, dispatch_rr, dispatch_keyed;
    SX* dispatch_key;
    int64_t num_targets;
    int has_window, window_ok;
    int64_t window_size;
    int has_streams;
    int64_t num_streams;
} Module;

/* ------------------------------------------------------------------ */
/* tokenizer                                                           */
/* ------------------------------------------------------------------ */

typedef struct { const char* p; } Lex;

static char* tok(Lex* L) {
    while (*L->p == ' ' || *L->p == '\n' || *L->p == '\t' || *L->p == '\r') L->p++;
    if (!*L->p) fail("module text: unexpected end of input");
    const char* s = L->p;
    while (*L->p && *L->p != ' ' && *L->p != '\n' && *L->p != '\t' && *L->p != '\r') L->p++;
    size_t n = (size_t)(L->p - s);
    char* out = (char*)alloc(n + 1);
    memcpy(out, s, n);
    return out;
}

static void expect(Lex* L, const char* want) {
    char* t = tok(L);
    if (strcmp(t, want) != 0) fail("module text: expected '%s', got '%s'", want, t);
}

static int64_t tok_i64(Lex* L) {
    char* t = tok(L);
    char* e;
    long long v = strtoll(t, &e, 10);
    if (*e) fail("module text: bad integer '%s'", t);
    return (int64_t)v;
}

static uint64_t tok_u64(Lex* L) {
    char* t = tok(L);
    char* e;
    unsigned long long v = strtoull(t, &e, 10);
    if (*e) fail("module text: bad unsigned '%s'", t);
    return (uint64_t)v;
}

static double tok_f64(Lex* L) {
    char* t = tok(L);
    char* e;
    double v = strtod(t, &e);
    if (*e) fail("module text: bad float '%s'", t);
    return v;
}

static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    return -1;
}

static char* tok_str(Lex* L) {
    char* t = tok(L);
    if (strcmp(t, "%") == 0) { t[0] = 0; return t; }
    char* o = t;
    for (char* s = t; *s;) {
        if (*s == '%' && hexval(s[1]) >= 0 && hexval(s[2]) >= 0) {
            *o++ = (char)(hexval(s[1]) * 16 + hexval(s[2]));
            s += 3;
        } else {
            *o++ = *s++;
        }
    }
    *o = 0;
    return t;
}

static int tok_dtype(Lex* L) {
    char* t = tok(L);
    for (int i = 0; i < 13; ++i)
        if (strcmp(t, k_dtype_names[i]) == 0) return i;
    fail("module text: unknown dtype '%s'", t);
    return -1;
}

/* ------------------------------------------------------------------ */
/* parsing                                                             */
/* ------------------------------------------------------------------ */

static int op_kind(const char* s) {
    static const char* names[] = {"Load", "Store", "Add", "Sub", "Mul", "Div", "Max", "Min", "Exp",
                                  "Rsqrt", "RowSum", "RowMax", "RowMean", "Matmul", "Constant",
                                  "IotaU32", "TSort32", "ExtractTopkIndices", "TMov", "StoreTopkIndices",
                                  "CpuSimAddCycles"};
    for (int i = 0; i < 21; ++i)
        if (strcmp(s, names[i]) == 0) return i;
    return OP_OTHER;
}

static SX* parse_sx(Lex* L);

/* True when the expression reads nothing but literals and kernel scalars. */
static int sx_kernel_only(const SX* e) {
    if (!e) return 1;
    if (e->kind == 'P' || e->kind == 'G' || e->kind == 'A' || e->kind == 'Y' || e->kind == 'S') return 0;
    return sx_kernel_only(e->a) && sx_kernel_only(e->b) && sx_kernel_only(e->c);
}

static void parse_attr_skip(Lex* L, Op* op) {
    char* key = tok_str(L);
    char* ty = tok(L);
    int is_value = strcmp(key, "value") == 0;
    switch (ty[0]) {
        case 'i': {
            int64_t v = tok_i64(L);
            if (is_value) { op->has_value = 1; op->value = (double)v; }
            else if (strcmp(key, "k") == 0) { op->has_k = 1; op->k = v; }
            else if (strcmp(key, "cols") == 0) { op->has_cols = 1; op->cols = v; }
            else if (strcmp(key, "cycles") == 0) { op->has_cycles = 1; op->cycles = v; }
            break;
        }
        case 'd': { double v = tok_f64(L); if (is_value) { op->has_value = 1; op->value = v; } break; }
        case 'b': { int64_t v = tok_i64(L); if (is_value) { op->has_value = 1; op->value = (double)v; } break; }
        case 's': {
            char* v = tok_str(L);
            if (strcmp(key, "cycles_expr") == 0) {
                Lex sub = {v};
                op->cycles_expr = parse_sx(&sub);
                while (*sub.p == ' ') sub.p++;
                if (*sub.p) fail("module text: trailing tokens in a cycles expression");
                if (!sx_kernel_only(op->cycles_expr))
                    fail("a cycles expression may read only the kernel's scalar parameters");
            }
            break;
        }
        case 'I': { int64_t n = tok_i64(L); for (int64_t i = 0; i < n; ++i) (void)tok_i64(L); break; }
        case 'S': { int64_t n = tok_i64(L); for (int64_t i = 0; i < n; ++i) (void)tok_str(L); break; }
        default: fail("module text: bad attr type '%s'", ty);
    }
}

static void parse_kernel(Lex* L, Kernel* k) {
    expect(L, "K");
    k->name = tok_str(L);
    k->nvals = (int)tok_i64(L);
    k->nparams = (int)tok_i64(L);
    k->nops = (int)tok_i64(L);
    k->custom = (int)tok_i64(L);
    if (k->custom) (void)tok_str(L); /* the cpp_src body (1) or cpp_tu_path file (2): compiled by the caller,
                                        reached via get_kernel */
    k->vals = (Val*)alloc(sizeof(Val) * (size_t)(k->nvals + 1));
    k->params = (Param*)alloc(sizeof(Param) * (size_t)(k->nparams + 1));
    k->ops = (Op*)alloc(sizeof(Op) * (size_t)(k->nops + 1));
    k->max_id = 0;
    for (int i = 0; i < k->nvals; ++i) {
        expect(L, "V");
        Val* v = &k->vals[i];
        v->id = (int)tok_i64(L);
        v->dtype = tok_dtype(L);
        char* kind = tok(L);
        v->tile = kind[0] == 'T';
        if (v->tile) {
            v->rows = (int)tok_i64(L);
            v->cols = (int)tok_i64(L);
            if (v->rows <= 0 || v->cols <= 0) fail("kernel %s: tile value %d has empty shape", k->name, v->id);
        }
        if (v->id > k->max_id) k->max_id = v->id;
    }
    for (int i = 0; i < k->nparams; ++i) {
        expect(L, "P");
        k->params[i].name = tok_str(L);
        k->params[i].id = (int)tok_i64(L);
        (void)tok(L); /* direction: informational, the semantics follow the ops */
    }
    for (int i = 0; i < k->nops; ++i) {
        expect(L, "O");
        Op* op = &k->ops[i];
        op->kind = op_kind(tok(L));
        op->result = (int)tok_i64(L);
        op->nopnd = (int)tok_i64(L);
        op->opnd = (int*)alloc(sizeof(int) * (size_t)(op->nopnd + 1));
        for (int j = 0; j < op->nopnd; ++j) op->opnd[j] = (int)tok_i64(L);
        int64_t na = tok_i64(L);
        for (int64_t j = 0; j < na; ++j) parse_attr_skip(L, op);
    }
}

static IExpr* parse_iexpr(Lex* L) {
    IExpr* e = (IExpr*)alloc(sizeof(IExpr));
    char* k = tok(L);
    e->kind = k[0];
    switch (e->kind) {
        case 'v': e->var = tok_str(L); break;
        case 'c': e->c = tok_i64(L); break;
        case 'a':
            e->c = tok_i64(L);
            e->nterms = (int)tok_i64(L);
            e->tvars = (char**)alloc(sizeof(char*) * (size_t)(e->nterms + 1));
            e->coefs = (int64_t*)alloc(sizeof(int64_t) * (size_t)(e->nterms + 1));
            for (int i = 0; i < e->nterms; ++i) {
                e->tvars[i] = tok_str(L);
                e->coefs[i] = tok_i64(L);
            }
            break;
        case 't':
            e->tid = (int)tok_i64(L);
            e->base_rank = (int)tok_i64(L);
            e->nidx = (int)tok_i64(L);
            e->idx = (IExpr*)alloc(sizeof(IExpr) * (size_t)(e->nidx + 1));
            for (int i = 0; i < e->nidx; ++i) e->idx[i] = *parse_iexpr(L);
            break;
        default: fail("module text: bad index expr kind '%s'", k);
    }
    return e;
}

static void parse_arg(Lex* L, Arg* a) {
    char* k = tok(L);
    a->kind = k[0];
    if (a->kind == 'v') a->var = tok_str(L);
    else if (a->kind == 'c') a->u64 = tok_u64(L);
    else if (a->kind == 's') { a->var = tok_str(L); a->u64 = tok_u64(L); }
    else fail("module text: bad arg kind '%s'", k);
}

static void parse_axis(Lex* L, Node* n) {
    char* k = tok(L);
    if (strcmp(k, "dense") == 0) { n->axis_kind = AX_DENSE; n->axis_size = tok_i64(L); }
    else if (strcmp(k, "dyn") == 0) { n->axis_kind = AX_DYN; n->axis_a = tok_str(L); }
    else if (strcmp(k, "ragged") == 0) { n->axis_kind = AX_RAGGED; n->axis_a = tok_str(L); n->axis_b = tok_str(L); }
    else if (strcmp(k, "dynt") == 0) {
        n->axis_kind = AX_DYNT;
        (void)tok_i64(L); /* max extent: a sizing hint for the HIP backend */
        n->axis_expr = parse_iexpr(L);
    }
    else fail("module text: bad axis kind '%s'", k);
}

static SX* parse_sx(Lex* L) {
    SX* e = (SX*)alloc(sizeof(SX));
    char* k = tok(L);
    if (strcmp(k, "Lb") == 0 || strcmp(k, "Li") == 0 || strcmp(k, "Lu") == 0) {
        e->kind = 'L';
        e->ty = k[1] == 'b' ? 'b' : k[1] == 'i' ? 'i' : 'u';
        e->u = e->ty == 'i' ? (uint64_t)tok_i64(L) : tok_u64(L);
        if (e->ty == 'b') e->u = e->u != 0;
    } else if (strcmp(k, "P") == 0 || strcmp(k, "S") == 0 || strcmp(k, "A") == 0 || strcmp(k, "C") == 0 ||
               strcmp(k, "K") == 0) {
        e->kind = k[0];
        char* t = tok(L);
        if (strcmp(t, "b") != 0 && strcmp(t, "i") != 0 && strcmp(t, "u") != 0) fail("scalar expression: bad type '%s'", t);
        e->ty = t[0];
        if (k[0] == 'C') e->a = parse_sx(L);
        else e->u = tok_u64(L);
    } else if (strcmp(k, "G") == 0 || strcmp(k, "Y") == 0) {
        e->kind = k[0];
        e->ty = 'u';
        e->u = tok_u64(L);
    } else if (strcmp(k, "U") == 0 || strcmp(k, "B") == 0) {
        e->kind = k[0];
        char* op = tok(L);
        if (strlen(op) > 2) fail("scalar expression: bad operator '%s'", op);
        strcpy(e->op, op);
        e->a = parse_sx(L);
        if (k[0] == 'B') e->b = parse_sx(L);
    } else if (strcmp(k, "T") == 0) {
        e->kind = 'T';
        e->a = parse_sx(L);
        e->b = parse_sx(L);
        e->c = parse_sx(L);
    } else {
        fail("scalar expression: bad node '%s'", k);
    }
    return e;
}

static Kernel* find_kernel(Module* m, const char* name) {
    for (int i = 0; i < m->nkernels; ++i)
        if (strcmp(m->kernels[i].name, name) == 0) return &m->kernels[i];
    return NULL;
}

static Node* parse_node(Lex* L, Module* m) {
    Node* n = (Node*)alloc(sizeof(Node));
    char* k = tok(L);
    if (strcmp(k, "empty") == 0) {
        n->kind = N_EMPTY;
    } else if (strcmp(k, "pfor") == 0 || strcmp(k, "each") == 0) {
        n->kind = k[0] == 'p' ? N_PFOR : N_EACH;
        n->var = tok_str(L);
        parse_axis(L, n);
        n->body = parse_node(L, m);
    } else if (strcmp(k, "comb") == 0 || strcmp(k, "seqn") == 0) {
        n->kind = k[0] == 'c' ? N_COMB : N_SEQN;
        n->nkids = (int)tok_i64(L);
        n->kids = (Node**)alloc(sizeof(Node*) * (size_t)(n->nkids + 1));
        for (int i = 0; i < n->nkids; ++i) n->kids[i] = parse_node(L, m);
    } else if (strcmp(k, "task") == 0) {
        n->kind = N_TASK;
        n->kernel_name = tok_str(L);
        n->kernel = find_kernel(m, n->kernel_name);
        if (!n->kernel) fail("Missing kernel def for task: %s", n->kernel_name);
        n->naxis = (int)tok_i64(L);
        n->axis = (Arg*)alloc(sizeof(Arg) * (size_t)(n->naxis + 1));
        for (int i = 0; i < n->naxis; ++i) parse_arg(L, &n->axis[i]);
        n->nscal = (int)tok_i64(L);
        n->scal = (Arg*)alloc(sizeof(Arg) * (size_t)(n->nscal + 1));
        for (int i = 0; i < n->nscal; ++i) parse_arg(L, &n->scal[i]);
        n->nten = (int)tok_i64(L);
        n->ten = (TArg*)alloc(sizeof(TArg) * (size_t)(n->nten + 1));
        for (int i = 0; i < n->nten; ++i) {
            TArg* t = &n->ten[i];
            t->param = tok_str(L);
            t->tid = (int)tok_i64(L);
            t->base_rank = (int)tok_i64(L);
            t->view_rank = (int)tok_i64(L);
            t->nidx = (int)tok_i64(L);
            t->idx = (IExpr*)alloc(sizeof(IExpr) * (size_t)(t->nidx + 1));
            for (int j = 0; j < t->nidx; ++j) t->idx[j] = *parse_iexpr(L);
            if (t->tid < 0 || t->tid >= m->ntensors) fail("task %s: bad tensor id %d", n->kernel_name, t->tid);
        }
    } else if (strcmp(k, "sel") == 0) {
        n->kind = N_SEL;
        n->var = tok_str(L);
        n->sel_outer = tok_str(L);
        n->sel_indptr = tok_str(L);
        n->sel_indices = tok_str(L);
        n->body = parse_node(L, m);
    } else if (strcmp(k, "slotset") == 0) {
        n->kind = N_SLOTSET;
        n->slot = (uint32_t)tok_u64(L);
        n->slot_value = tok_u64(L);
    } else if (strcmp(k, "slotld") == 0) {
        n->kind = N_SLOTLD;
        n->slot = (uint32_t)tok_u64(L);
        TArg* t = &n->slot_view;
        t->tid = (int)tok_i64(L);
        t->base_rank = (int)tok_i64(L);
        t->view_rank = (int)tok_i64(L);
        t->nidx = (int)tok_i64(L);
        t->idx = (IExpr*)alloc(sizeof(IExpr) * (size_t)(t->nidx + 1));
        for (int j = 0; j < t->nidx; ++j) t->idx[j] = *parse_iexpr(L);
        n->slot_row = tok_i64(L);
        n->slot_col = tok_i64(L);
        if (t->tid < 0 || t->tid >= m->ntensors) fail("slot_load_u64: bad tensor id %d", t->tid);
    } else if (strcmp(k, "cond") == 0) {
        n->kind = N_COND;
        n->pred = parse_sx(L);
        n->nkids = 2;
        n->kids = (Node**)alloc(sizeof(Node*) * 2);
        n->kids[0] = parse_node(L, m);
        n->kids[1] = parse_node(L, m);
    } else {
        fail("module text: bad node kind '%s'", k);
    }
    return n;
}

/* Derived per-kernel tables: which param tiles are loaded at entry
 * (collect_param_tiles_to_load, src/python/pto_codegen.cpp:453-469) and which
 * matmul results are moved into a vector tile (:700-710). */
static void analyze_kernel(Kernel* k) {
    int n = k->max_id + 1;
    k->by_id = (Val**)alloc(sizeof(Val*) * (size_t)n);
    k->param_of = (int*)alloc(sizeof(int) * (size_t)n);
    k->preload = (unsigned char*)alloc((size_t)n);
    k->acc_vec = (unsigned char*)alloc((size_t)n);
    k->tensor_index = (int*)alloc(sizeof(int) * (size_t)(k->nparams + 1));
    for (int i = 0; i < n; ++i) k->param_of[i] = -1;
    for (int i = 0; i < k->nvals; ++i) k->by_id[k->vals[i].id] = &k->vals[i];
    k->ntensor_params = 0;
    for (int i = 0; i < k->nparams; ++i) {
        int id = k->params[i].id;
        if (id <= 0 || id >= n || !k->by_id[id]) fail("kernel %s: param %s has no value", k->name, k->params[i].name);
        k->param_of[id] = i;
        k->tensor_index[i] = k->by_id[id]->tile ? k->ntensor_params++ : -1;
    }
    for (int i = 0; i < k->nops; ++i) {
        Op* op = &k->ops[i];
        for (int j = 0; j < op->nopnd; ++j) {
            int id = op->opnd[j];
            if (id <= 0 || id >= n || !k->by_id[id]) fail("kernel %s: op operand %d undefined", k->name, id);
        }
        if (op->result > 0 && (op->result >= n || !k->by_id[op->result])) fail("kernel %s: bad op result", k->name);
        if (op->kind == OP_MATMUL || op->kind == OP_LOAD) continue;
        for (int j = 0; j < op->nopnd; ++j) {
            int id = op->opnd[j];
            if (!k->by_id[id]->tile || k->param_of[id] < 0) continue;
            if ((op->kind == OP_STORE || op->kind == OP_STORE_TOPK) && j == 0) continue;
            k->preload[id] = 1;
        }
    }
    for (int i = 0; i < k->nops; ++i) {
        Op* op = &k->ops[i];
        if (op->kind == OP_MATMUL || op->kind == OP_STORE) continue;
        for (int j = 0; j < op->nopnd; ++j) {
            int id = op->opnd[j];
            if (k->param_of[id] >= 0) continue;
            for (int q = 0; q < k->nops; ++q)
                if (k->ops[q].kind == OP_MATMUL && k->ops[q].result == id) k->acc_vec[id] = 1;
        }
    }
}

static void parse_module(const char* text, Module* m) {
    Lex L = {text};
    expect(&L, "PTOWSP-MODULE");
    expect(&L, "1");
    expect(&L, "name");
    (void)tok_str(&L);
    expect(&L, "tensors");
    m->ntensors = (int)tok_i64(&L);
    m->tensors = (TensorInfo*)alloc(sizeof(TensorInfo) * (size_t)(m->ntensors + 1));
    for (int i = 0; i < m->ntensors; ++i) {
        expect(&L, "T");
        m->tensors[i].dtype = tok_dtype(&L);
        m->tensors[i].rank = (int)tok_i64(&L);
        if (m->tensors[i].rank > 8) fail("tensor rank > 8 unsupported");
        for (int d = 0; d < m->tensors[i].rank; ++d) m->tensors[i].shape[d] = tok_i64(&L);
    }
    expect(&L, "kernels");
    m->nkernels = (int)tok_i64(&L);
    m->kernels = (Kernel*)alloc(sizeof(Kernel) * (size_t)(m->nkernels + 1));
    for (int i = 0; i < m->nkernels; ++i) {
        parse_kernel(&L, &m->kernels[i]);
        analyze_kernel(&m->kernels[i]);
    }
    expect(&L, "workload");
    (void)tok_str(&L);
    m->root = parse_node(&L, m);
    expect(&L, "schedule");
    int64_t nd = tok_i64(&L);
    for (int64_t i = 0; i < nd; ++i) {
        char* d = tok(&L);
        if (strcmp(d, "D") == 0) {
            char* pol = tok(&L);
            m->has_dispatch = 1;
            m->num_targets = tok_i64(&L);
            m->dispatch_rr = strcmp(pol, "round_robin") == 0 || strcmp(pol, "work_steal") == 0;
            m->dispatch_keyed = !m->dispatch_rr;
            if (tok_i64(&L) != 0) m->dispatch_key = parse_sx(&L);
        } else if (strcmp(d, "W") == 0) {
            m->has_window = 1;
            m->window_size = tok_i64(&L);
            char* unit = tok_str(&L);
            char* ovf = tok(&L);
            m->window_ok = strcmp(unit, "tasks") == 0 && strcmp(ovf, "stall") == 0;
        } else if (strcmp(d, "S") == 0) {
            m->has_streams = 1;
            m->num_streams = tok_i64(&L);
            (void)tok_i64(&L);
        } else if (strcmp(d, "M") == 0) {
            (void)tok_str(&L);
        } else {
            fail("module text: bad schedule directive '%s'", d);
        }
    }
    expect(&L, "end");
    /* Keyed dispatch needs a ScalarExpr key (src/python/pto_codegen.cpp:1547-1556). */
    if (m->has_dispatch && m->dispatch_keyed && !m->dispatch_key)
        fail("dispatch policy requires ScalarExpr key (string-eval is not supported in v9 codegen-first)");
}

/* ------------------------------------------------------------------ */
/* scalar conversions                                                   */
/* ------------------------------------------------------------------ */

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1F, man = h & 0x3FF;
    if (exp == 0x1F) return f32_from_bits(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return f32_from_bits(sign);
        float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24 */
        return sign ? -v : v;
    }
    return f32_from_bits(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round-to-nearest-even float -> binary16 (the TCVT CAST_RINT of a f32->f16
 * store, src/python/pto_codegen.cpp:955-976). */
static uint16_t float_to_half(float f) {
    uint32_t x = bits_from_f32(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* subnormal or zero in half */
        float a = f32_from_bits(ax) * 16777216.0f;              /* exact scaling to units of 2^-24 */
        float r = nearbyintf(a);                                /* default mode: ties to even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t man = ax & 0x7FFFFFu, e = (ax >> 23) - 112u;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

static float bf16_to_float(uint16_t b) { return f32_from_bits((uint32_t)b << 16); }

static uint16_t float_to_bf16(float f) {
    uint32_t x = bits_from_f32(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

/* ------------------------------------------------------------------ */
/* tiles                                                               */
/* ------------------------------------------------------------------ */

typedef struct { int dtype, rows, cols; float* f; int64_t* i; } Tile;

typedef struct {
    char* ptr;   /* element (0,0) of the view */
    int dtype;
    int64_t s3, s4;
} View;

static double load_elem(const View* v, int64_t r, int64_t c) {
    const char* p = v->ptr + (r * v->s3 + c * v->s4) * k_dtype_size[v->dtype];
    switch (v->dtype) {
        case DT_F32: { float x; memcpy(&x, p, 4); return x; }
        case DT_F16: { uint16_t x; memcpy(&x, p, 2); return half_to_float(x); }
        case DT_BF16: { uint16_t x; memcpy(&x, p, 2); return bf16_to_float(x); }
        case DT_F64: { double x; memcpy(&x, p, 8); return x; }
        case DT_I8: return *(const int8_t*)p;
        case DT_U8: case DT_BOOL: return *(const uint8_t*)p;
        case DT_I16: { int16_t x; memcpy(&x, p, 2); return x; }
        case DT_U16: { uint16_t x; memcpy(&x, p, 2); return x; }
        case DT_I32: { int32_t x; memcpy(&x, p, 4); return x; }
        case DT_U32: { uint32_t x; memcpy(&x, p, 4); return x; }
        case DT_I64: { int64_t x; memcpy(&x, p, 8); return (double)x; }
        case DT_U64: { uint64_t x; memcpy(&x, p, 8); return (double)x; }
    }
    return 0;
}

static int64_t load_int(const View* v, int64_t r, int64_t c) {
    const char* p = v->ptr + (r * v->s3 + c * v->s4) * k_dtype_size[v->dtype];
    switch (v->dtype) {
        case DT_I64: { int64_t x; memcpy(&x, p, 8); return x; }
        case DT_U64: { uint64_t x; memcpy(&x, p, 8); return (int64_t)x; }
        default: return (int64_t)load_elem(v, r, c);
    }
}

static void tile_alloc(Tile* t, int dtype, int rows, int cols) {
    t->dtype = dtype;
    t->rows = rows;
    t->cols = cols;
    size_t n = (size_t)rows * (size_t)cols;
    if (is_float_dt(dtype)) t->f = (float*)alloc(sizeof(float) * n);
    else t->i = (int64_t*)alloc(sizeof(int64_t) * n);
}

/* TLOAD: copy a rows x cols tile through strides s3/s4 (src/python/pto_codegen.cpp:764-815). */
static void tload(Tile* t, const View* v) {
    for (int r = 0; r < t->rows; ++r)
        for (int c = 0; c < t->cols; ++c) {
            size_t k = (size_t)r * t->cols + c;
            if (t->f) t->f[k] = (float)load_elem(v, r, c);
            else t->i[k] = load_int(v, r, c);
        }
}

/* TSTORE, with the f32 -> f16 (and, as an extension, f32 -> bf16) RINT cast
 * inserted when the destination dtype differs (src/python/pto_codegen.cpp:931-988). */
static void tstore(const View* v, const Tile* t, const char* kname) {
    for (int r = 0; r < t->rows; ++r)
        for (int c = 0; c < t->cols; ++c) {
            size_t k = (size_t)r * t->cols + c;
            char* p = v->ptr + (r * v->s3 + c * v->s4) * k_dtype_size[v->dtype];
            if (t->f) {
                float x = t->f[k];
                if (v->dtype == DT_F32) memcpy(p, &x, 4);
                else if (v->dtype == DT_F16 && t->dtype == DT_F32) { uint16_t h = float_to_half(x); memcpy(p, &h, 2); }
                else if (v->dtype == DT_BF16 && t->dtype == DT_F32) { uint16_t h = float_to_bf16(x); memcpy(p, &h, 2); }
                else if (v->dtype == t->dtype && v->dtype == DT_F16) { uint16_t h = float_to_half(x); memcpy(p, &h, 2); }
                else if (v->dtype == t->dtype && v->dtype == DT_BF16) { uint16_t h = float_to_bf16(x); memcpy(p, &h, 2); }
                else fail("kernel %s: Store dtype mismatch (unsupported cast %s -> %s)", kname,
                          k_dtype_names[t->dtype], k_dtype_names[v->dtype]);
            } else {
                if (v->dtype != t->dtype) fail("kernel %s: Store dtype mismatch", kname);
                int64_t x = t->i[k];
                switch (v->dtype) {
                    case DT_I8: case DT_U8: case DT_BOOL: { uint8_t y = (uint8_t)x; memcpy(p, &y, 1); break; }
                    case DT_I16: case DT_U16: { uint16_t y = (uint16_t)x; memcpy(p, &y, 2); break; }
                    case DT_I32: case DT_U32: { uint32_t y = (uint32_t)x; memcpy(p, &y, 4); break; }
                    default: memcpy(p, &x, 8); break;
                }
            }
        }
}

/* ------------------------------------------------------------------ */
/* run-time environment                                                 */
/* ------------------------------------------------------------------ */

typedef struct { const char* name; int64_t value; } Binding;

typedef struct {
    Module* m;
    RuntimeContext* ctx;
    char** tbase;
    int64_t* tstride; /* [tid * 8 + d] */
    int64_t* tspan;   /* max element offset + 1 per tensor (0: empty) */
    Binding env[64];
    int nenv;
    /* scheduler (src/python/pto_codegen.cpp:1561-1607) */
    uint32_t workers;
    uint64_t window, issue_time, rr;
    uint64_t* avail;
    uint64_t* heap;
    size_t hn, hcap;
    struct TaskScratch** scratch; /* per kernel, allocated on first use */
} Run;

static int64_t lookup(Run* R, const char* name) {
    for (int i = R->nenv - 1; i >= 0; --i)
        if (strcmp(R->env[i].name, name) == 0) return R->env[i].value;
    fail("unbound loop variable '%s'", name);
    return 0;
}

static void check_span(Run* R, int tid, int64_t lo, int64_t hi, const char* what) {
    if (lo < 0 || hi >= R->tspan[tid])
        fail("%s: access [%lld, %lld] outside tensor %d (span %lld elements)", what, (long long)lo, (long long)hi,
             tid, (long long)R->tspan[tid]);
}

static int64_t eval_iexpr(Run* R, const IExpr* e) {
    switch (e->kind) {
        case 'v': return lookup(R, e->var);
        case 'c': return e->c;
        case 'a': {
            int64_t v = e->c;
            for (int i = 0; i < e->nterms; ++i) v += e->coefs[i] * lookup(R, e->tvars[i]);
            return v;
        }
        case 't': {
            int tid = e->tid;
            if (R->m->tensors[tid].dtype != DT_I32) fail("indirect index tensor %d must be i32", tid);
            int64_t off = 0;
            for (int i = 0; i < e->nidx; ++i) off += eval_iexpr(R, &e->idx[i]) * R->tstride[tid * 8 + i];
            check_span(R, tid, off, off, "indirect index");
            int32_t x;
            memcpy(&x, R->tbase[tid] + off * 4, 4);
            return x;
        }
    }
    return 0;
}

static void heap_push(Run* R, uint64_t v) {
    if (R->hn == R->hcap) {
        size_t cap = R->hcap ? R->hcap * 2 : 1024;
        uint64_t* h = (uint64_t*)alloc(sizeof(uint64_t) * cap);
        if (R->hn) memcpy(h, R->heap, sizeof(uint64_t) * R->hn);
        R->heap = h;
        R->hcap = cap;
    }
    size_t i = R->hn++;
    R->heap[i] = v;
    while (i > 0) {
        size_t p = (i - 1) / 2;
        if (R->heap[p] <= R->heap[i]) break;
        uint64_t t = R->heap[p]; R->heap[p] = R->heap[i]; R->heap[i] = t;
        i = p;
    }
}

static void heap_pop(Run* R) {
    R->heap[0] = R->heap[--R->hn];
    size_t i = 0;
    for (;;) {
        size_t l = 2 * i + 1, r = l + 1, s = i;
        if (l < R->hn && R->heap[l] < R->heap[s]) s = l;
        if (r < R->hn && R->heap[r] < R->heap[s]) s = r;
        if (s == i) break;
        uint64_t t = R->heap[s]; R->heap[s] = R->heap[i]; R->heap[i] = t;
        i = s;
    }
}

static void advance_to(Run* R, uint64_t t) {
    if (t > R->issue_time) R->issue_time = t;
    while (R->hn && R->heap[0] <= R->issue_time) heap_pop(R);
}

static uint64_t issue(Run* R, uint64_t dur, uint32_t w, uint64_t ready) {
    if (w >= R->workers) w = 0;
    advance_to(R, ready);
    if (R->window > 0)
        while (R->hn >= R->window) advance_to(R, R->heap[0]);
    uint64_t start = R->avail[w] > R->issue_time ? R->avail[w] : R->issue_time;
    uint64_t end = start + dur;
    R->avail[w] = end;
    heap_push(R, end);
    return end;
}

/* ------------------------------------------------------------------ */
/* kernel execution (src/python/pto_codegen.cpp:471-1241)               */
/* ------------------------------------------------------------------ */

typedef struct {
    Tile* tiles;     /* by value id */
    double* scalars; /* by value id */
    unsigned char* is_scalar;
    int64_t* iscal;
} Work;

static Work* kernel_work(Kernel* k) {
    Work* w = (Work*)alloc(sizeof(Work));
    int n = k->max_id + 1;
    w->tiles = (Tile*)alloc(sizeof(Tile) * (size_t)n);
    w->scalars = (double*)alloc(sizeof(double) * (size_t)n);
    w->is_scalar = (unsigned char*)alloc((size_t)n);
    w->iscal = (int64_t*)alloc(sizeof(int64_t) * (size_t)n);
    for (int i = 0; i < k->nvals; ++i) {
        Val* v = &k->vals[i];
        if (v->tile) tile_alloc(&w->tiles[v->id], v->dtype, v->rows, v->cols);
    }
    return w;
}

static uint64_t rc(const Val* v) { return (uint64_t)v->rows * (uint64_t)v->cols; }

static float ew_f(int kind, float a, float b) {
    switch (kind) {
        case OP_ADD: return a + b;
        case OP_SUB: return a - b;
        case OP_MUL: return a * b;
        case OP_DIV: return a / b;
        case OP_MAX: return a > b ? a : b;
        case OP_MIN: return a < b ? a : b;
    }
    return 0;
}

static int64_t ew_i(int kind, int64_t a, int64_t b, const char* kname) {
    switch (kind) {
        case OP_ADD: return a + b;
        case OP_SUB: return a - b;
        case OP_MUL: return a * b;
        case OP_DIV: if (b == 0) fail("kernel %s: integer division by zero", kname); return a / b;
        case OP_MAX: return a > b ? a : b;
        case OP_MIN: return a < b ? a : b;
    }
    return 0;
}

/* TSORT32 of one [1,32] row (ptoisa_jit.py:247-258): (score, (float)index)
 * pairs in descending score order, NaN after every number, equal scores in
 * source order.  Stable insertion sort on the key -score (NaN largest). */
static int tsort_after(float a, float b) { /* a strictly after b */
    if (b != b) return 0;
    if (a != a) return 1;
    return a < b;
}

static void tsort32_pairs(float* dst, const float* sc, const int64_t* ix) {
    float key[32];
    int64_t id[32];
    for (int i = 0; i < 32; ++i) {
        float x = sc[i];
        int64_t xi = ix[i];
        int j = i;
        while (j > 0 && tsort_after(key[j - 1], x)) {
            key[j] = key[j - 1];
            id[j] = id[j - 1];
            --j;
        }
        key[j] = x;
        id[j] = xi;
    }
    for (int i = 0; i < 32; ++i) {
        dst[2 * i] = key[i];
        dst[2 * i + 1] = (float)id[i];
    }
}

static uint64_t cycles_expr_value(const SX* e, const uint64_t* kscal, int nk);

/* Executes one task; returns its cpu_sim cycle count. */
static uint64_t run_kernel(Kernel* k, Work* w, View* views, const uint64_t* scalar_args) {
    uint64_t cycles = 0;
    const char* kn = k->name;
    if (k->custom) fail("kernel %s: custom C++ kernel bodies are not supported", kn);
    /* Scalar params from task->args after the axis args (:607-640). */
    for (int i = 0, si = 0; i < k->nparams; ++i) {
        Val* v = k->by_id[k->params[i].id];
        if (v->tile) continue;
        uint64_t a = scalar_args[si++];
        w->is_scalar[v->id] = 1;
        switch (v->dtype) {
            case DT_F32: w->scalars[v->id] = f32_from_bits((uint32_t)a); w->iscal[v->id] = 0; break;
            case DT_I32: w->iscal[v->id] = (int32_t)(uint32_t)a; w->scalars[v->id] = (double)w->iscal[v->id]; break;
            case DT_I64: w->iscal[v->id] = (int64_t)a; w->scalars[v->id] = (double)w->iscal[v->id]; break;
            case DT_BOOL: w->iscal[v->id] = a != 0; w->scalars[v->id] = (double)(a != 0); break;
            default: fail("kernel %s: unsupported scalar param dtype %s", kn, k_dtype_names[v->dtype]);
        }
    }
    /* Constant() scalars: (elem)value (:642-655). */
    for (int i = 0; i < k->nops; ++i) {
        Op* op = &k->ops[i];
        if (op->kind != OP_CONSTANT || op->result <= 0) continue;
        Val* v = k->by_id[op->result];
        if (v->tile || !op->has_value) continue;
        w->is_scalar[v->id] = 1;
        if (v->dtype == DT_F32) w->scalars[v->id] = (float)op->value;
        else if (is_float_dt(v->dtype)) fail("kernel %s: unsupported constant dtype", kn);
        else { w->iscal[v->id] = (int64_t)op->value; w->scalars[v->id] = (double)w->iscal[v->id]; }
    }
    /* Param tiles used by vector ops are TLOADed at entry (:764-779). */
    for (int i = 0; i < k->nparams; ++i) {
        Val* v = k->by_id[k->params[i].id];
        if (!v->tile || !k->preload[v->id]) continue;
        tload(&w->tiles[v->id], &views[k->tensor_index[i]]);
        cycles += rc(v);
    }
    for (int oi = 0; oi < k->nops; ++oi) {
        Op* op = &k->ops[oi];
        Val* res = op->result > 0 ? k->by_id[op->result] : NULL;
        switch (op->kind) {
            case OP_CONSTANT:
                if (res && res->tile) fail("kernel %s: tile-shaped Constant ops have no compute", kn);
                break;
            case OP_LOAD: {
                int src = op->opnd[0];
                int pi = k->param_of[src];
                if (pi < 0 || !k->by_id[src]->tile) fail("kernel %s: Load src must be a kernel param tile", kn);
                if (!res || !res->tile) fail("kernel %s: Load without a tile result", kn);
                tload(&w->tiles[res->id], &views[k->tensor_index[pi]]);
                cycles += rc(k->by_id[src]);
                break;
            }
            case OP_STORE: {
                int dst = op->opnd[0], src = op->opnd[1];
                int pi = k->param_of[dst];
                if (pi < 0 || !k->by_id[dst]->tile) fail("kernel %s: Store dst must be a kernel param tile", kn);
                Val* sv = k->by_id[src];
                Val* dv = k->by_id[dst];
                if (!sv->tile) fail("kernel %s: Store src must be a tile", kn);
                if (sv->rows != dv->rows || sv->cols != dv->cols)
                    fail("kernel %s: Store of a %dx%d tile into a %dx%d param", kn, sv->rows, sv->cols, dv->rows, dv->cols);
                if (k->param_of[src] >= 0 && !k->preload[src]) fail("kernel %s: Store src not loaded", kn);
                tstore(&views[k->tensor_index[pi]], &w->tiles[src], kn);
                if (dv->dtype != sv->dtype) cycles += rc(dv); /* TCVT */
                cycles += rc(dv);                              /* TSTORE */
                break;
            }
            case OP_MATMUL: {
                if (op->nopnd < 2 || !res || !res->tile) fail("kernel %s: malformed Matmul", kn);
                Val* av = k->by_id[op->opnd[0]];
                Val* bv = k->by_id[op->opnd[1]];
                if (!av->tile || !bv->tile) fail("kernel %s: Matmul expects tile operands", kn);
                int M = av->rows, K = av->cols, N = bv->cols;
                if (bv->rows != K) fail("kernel %s: Matmul K mismatch", kn);
                /* f32 x f32 and f16 x f16 as in the reference (:863-873); extensions:
                 * bf16 x bf16, and a 16-bit float operand with an f32 one (the 16-bit
                 * operand is upcast exactly; f32 math). */
                int f32a = av->dtype == DT_F32, f32b = bv->dtype == DT_F32;
                int h16a = av->dtype == DT_F16 || av->dtype == DT_BF16;
                int h16b = bv->dtype == DT_F16 || bv->dtype == DT_BF16;
                int ok = (f32a && f32b) || (av->dtype == DT_F16 && bv->dtype == DT_F16) ||
                         (av->dtype == DT_BF16 && bv->dtype == DT_BF16) || (f32a && h16b) || (h16a && f32b);
                if (!ok || res->dtype != DT_F32)
                    fail("kernel %s: Matmul: unsupported dtype combination %s x %s -> %s", kn,
                         k_dtype_names[av->dtype], k_dtype_names[bv->dtype], k_dtype_names[res->dtype]);
                if (res->rows != M || res->cols != N) fail("kernel %s: Matmul result shape mismatch", kn);
                /* Operands: TLOAD from the param view, or TMOV of a local tile (:891-923). */
                float* A = (float*)alloc(sizeof(float) * (size_t)M * K);
                float* B = (float*)alloc(sizeof(float) * (size_t)K * N);
                int pa = k->param_of[av->id], pb = k->param_of[bv->id];
                for (int r = 0; r < M; ++r)
                    for (int c = 0; c < K; ++c)
                        A[(size_t)r * K + c] = pa >= 0 ? (float)load_elem(&views[k->tensor_index[pa]], r, c)
                                                       : w->tiles[av->id].f[(size_t)r * K + c];
                for (int r = 0; r < K; ++r)
                    for (int c = 0; c < N; ++c)
                        B[(size_t)r * N + c] = pb >= 0 ? (float)load_elem(&views[k->tensor_index[pb]], r, c)
                                                       : w->tiles[bv->id].f[(size_t)r * N + c];
                cycles += (uint64_t)M * K + (uint64_t)K * N;
                /* TMATMUL into a fresh fp32 accumulator; a third (acc) operand is
                 * ignored exactly as the emitter ignores it (:817-929). */
                float* C = w->tiles[res->id].f;
                for (int i = 0; i < M; ++i)
                    for (int j = 0; j < N; ++j) {
                        float acc = 0.0f;
                        for (int q = 0; q < K; ++q) acc += A[(size_t)i * K + q] * B[(size_t)q * N + j];
                        C[(size_t)i * N + j] = acc;
                    }
                cycles += (uint64_t)M * K * N;
                if (k->acc_vec[res->id]) cycles += (uint64_t)M * N; /* TMOV acc -> vec */
                break;
            }
            case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: case OP_MAX: case OP_MIN: {
                if (op->nopnd != 2 || !res) fail("kernel %s: binary op missing result/operands", kn);
                if (!res->tile) fail("kernel %s: binary op with a scalar result has no tile lowering", kn);
                int a = op->opnd[0], b = op->opnd[1];
                if (!k->by_id[a]->tile && !w->is_scalar[a]) fail("kernel %s: scalar operand %d has no value", kn, a);
                if (!k->by_id[b]->tile && !w->is_scalar[b]) fail("kernel %s: scalar operand %d has no value", kn, b);
                int as = !k->by_id[a]->tile, bs = !k->by_id[b]->tile;
                Tile* d = &w->tiles[res->id];
                size_t n = (size_t)res->rows * res->cols;
                if (as ^ bs) {
                    /* Scalar fast paths TADDS/TMULS/TDIVS/TSUBS/TMAXS/TMINS (:1008-1051). */
                    int tid = as ? b : a, sid = as ? a : b;
                    if (as && op->kind == OP_SUB) fail("kernel %s: Sub: scalar - tile not supported", kn);
                    Val* tv = k->by_id[tid];
                    if (tv->rows != res->rows || tv->cols != res->cols) fail("kernel %s: scalar op shape mismatch", kn);
                    Tile* t = &w->tiles[tid];
                    if (d->f && t->f) {
                        float s = (float)w->scalars[sid];
                        for (size_t q = 0; q < n; ++q)
                            d->f[q] = (op->kind == OP_DIV && as) ? s / t->f[q] : ew_f(op->kind, t->f[q], s);
                    } else if (d->i && t->i) {
                        int64_t s = w->iscal[sid];
                        for (size_t q = 0; q < n; ++q)
                            d->i[q] = (op->kind == OP_DIV && as) ? ew_i(OP_DIV, s, t->i[q], kn) : ew_i(op->kind, t->i[q], s, kn);
                    } else {
                        fail("kernel %s: mixed int/float scalar op", kn);
                    }
                    cycles += rc(res);
                    break;
                }
                if (as && bs) fail("kernel %s: binary op on two scalars has no tile lowering", kn);
                Val* av = k->by_id[a];
                Val* bv = k->by_id[b];
                int R_ = res->rows, C_ = res->cols;
                if (!(av->rows == R_ && av->cols == C_)) fail("kernel %s: Binary op broadcast pattern unsupported", kn);
                if (is_float_dt(res->dtype) && res->dtype != DT_F32)
                    fail("kernel %s: vector ops on %s tiles are not supported", kn, k_dtype_names[res->dtype]);
                Tile* ta = &w->tiles[a];
                Tile* tb = &w->tiles[b];
                if (!!ta->f != !!d->f || !!tb->f != !!d->f) fail("kernel %s: mixed int/float tile op", kn);
                int mode; /* 0 same shape, 1 row-expand, 2 col-expand (:1078-1107) */
                if (bv->rows == R_ && bv->cols == C_) mode = 0;
                else if ((bv->rows == R_ && bv->cols == 1) || (bv->rows == 1 && bv->cols == R_)) mode = 1;
                else if ((op->kind == OP_SUB || op->kind == OP_MUL || op->kind == OP_DIV) &&
                         ((bv->rows == 1 && bv->cols == C_) || (bv->rows == C_ && bv->cols == 1))) mode = 2;
                else { fail("kernel %s: Binary op broadcast pattern unsupported", kn); mode = -1; }
                for (int r = 0; r < R_; ++r)
                    for (int c = 0; c < C_; ++c) {
                        size_t q = (size_t)r * C_ + c;
                        size_t qb = mode == 0 ? q : (mode == 1 ? (size_t)r : (size_t)c);
                        if (d->f) d->f[q] = ew_f(op->kind, ta->f[q], tb->f[qb]);
                        else d->i[q] = ew_i(op->kind, ta->i[q], tb->i[qb], kn);
                    }
                cycles += rc(res);
                break;
            }
            case OP_EXP: case OP_RSQRT: {
                if (op->nopnd != 1 || !res || !res->tile) fail("kernel %s: unary op expects a tile", kn);
                Val* sv = k->by_id[op->opnd[0]];
                if (!sv->tile || sv->dtype != DT_F32 || res->dtype != DT_F32)
                    fail("kernel %s: Exp/Rsqrt need f32 tiles", kn);
                Tile* s = &w->tiles[sv->id];
                Tile* d = &w->tiles[res->id];
                size_t n = (size_t)res->rows * res->cols;
                for (size_t q = 0; q < n; ++q) d->f[q] = op->kind == OP_EXP ? expf(s->f[q]) : 1.0f / sqrtf(s->f[q]);
                cycles += rc(res);
                break;
            }
            case OP_ROWSUM: case OP_ROWMAX: case OP_ROWMEAN: {
                if (op->nopnd != 1 || !res || !res->tile) fail("kernel %s: row reduce expects a tile", kn);
                Val* sv = k->by_id[op->opnd[0]];
                if (!sv->tile) fail("kernel %s: row reduce expects a tile operand", kn);
                if (res->rows != sv->rows || res->cols != 1) fail("kernel %s: row reduce result shape", kn);
                Tile* s = &w->tiles[sv->id];
                Tile* d = &w->tiles[res->id];
                if (!!s->f != !!d->f) fail("kernel %s: row reduce dtype mismatch", kn);
                for (int r = 0; r < sv->rows; ++r) {
                    if (s->f) {
                        float acc = s->f[(size_t)r * sv->cols];
                        for (int c = 1; c < sv->cols; ++c) {
                            float x = s->f[(size_t)r * sv->cols + c];
                            acc = op->kind == OP_ROWMAX ? (x > acc ? x : acc) : acc + x;
                        }
                        /* RowMean = TROWSUM then TDIVS by the column count (:1212-1219). */
                        if (op->kind == OP_ROWMEAN) acc = acc / (float)sv->cols;
                        d->f[r] = acc;
                    } else {
                        int64_t acc = s->i[(size_t)r * sv->cols];
                        for (int c = 1; c < sv->cols; ++c) {
                            int64_t x = s->i[(size_t)r * sv->cols + c];
                            acc = op->kind == OP_ROWMAX ? (x > acc ? x : acc) : acc + x;
                        }
                        if (op->kind == OP_ROWMEAN) acc = acc / sv->cols;
                        d->i[r] = acc;
                    }
                }
                cycles += (uint64_t)res->rows * (op->kind == OP_ROWMEAN ? 2u : 1u);
                break;
            }
            case OP_TMOV: { /* TMOV: copy, rows x cols of the destination (ptoisa_bridge.hpp:104-109) */
                if (op->nopnd != 1 || !res || !res->tile) fail("kernel %s: TMov expects one tile operand", kn);
                Val* sv = k->by_id[op->opnd[0]];
                if (!sv->tile || sv->rows != res->rows || sv->cols != res->cols || sv->dtype != res->dtype)
                    fail("kernel %s: TMov shape/dtype mismatch", kn);
                Tile* s = &w->tiles[sv->id];
                Tile* d = &w->tiles[res->id];
                size_t n = (size_t)res->rows * res->cols;
                if (d->f) memcpy(d->f, s->f, sizeof(float) * n);
                else memcpy(d->i, s->i, sizeof(int64_t) * n);
                cycles += rc(res);
                break;
            }
            case OP_IOTA_U32: { /* 0..C-1 (src/python/pto_codegen.cpp:1132-1150), no cycles */
                if (!res || !res->tile || res->rows != 1 || res->dtype != DT_U32)
                    fail("kernel %s: IotaU32 expects a [1,C] u32 result", kn);
                for (int c = 0; c < res->cols; ++c) w->tiles[res->id].i[c] = c;
                break;
            }
            case OP_TSORT32: { /* (ptoisa_bridge.hpp:280-292): 5 cycles per source element */
                if (op->nopnd != 2 || !res || !res->tile) fail("kernel %s: TSort32 expects (scores, idx)", kn);
                Val* sv = k->by_id[op->opnd[0]];
                Val* iv = k->by_id[op->opnd[1]];
                if (!sv->tile || sv->rows != 1 || sv->cols != 32 || sv->dtype != DT_F32)
                    fail("kernel %s: TSort32 requires a [1,32] f32 score tile", kn);
                if (!iv->tile || iv->rows != 1 || iv->cols != 32 || iv->dtype != DT_U32)
                    fail("kernel %s: TSort32 requires a [1,32] u32 index tile", kn);
                if (res->rows != 1 || res->cols != 64 || res->dtype != DT_F32)
                    fail("kernel %s: TSort32 result must be [1,64] f32", kn);
                tsort32_pairs(w->tiles[res->id].f, w->tiles[sv->id].f, w->tiles[iv->id].i);
                cycles += 5u * rc(sv);
                break;
            }
            case OP_EXTRACT_TOPK: { /* (src/python/pto_codegen.cpp:1170-1193), no cycles */
                if (op->nopnd != 1 || !res || !res->tile) fail("kernel %s: ExtractTopkIndices expects one operand", kn);
                Val* pv = k->by_id[op->opnd[0]];
                if (!pv->tile || pv->rows != 1 || pv->cols != 64 || pv->dtype != DT_F32)
                    fail("kernel %s: ExtractTopkIndices expects [1,64] f32 pairs", kn);
                int64_t kk = op->has_k && op->k > 0 ? op->k : res->cols;
                if (res->rows != 1 || res->dtype != DT_I32 || kk != res->cols || kk > 32)
                    fail("kernel %s: ExtractTopkIndices result must be a [1,k] i32 tile, 1 <= k <= 32", kn);
                for (int64_t q = 0; q < kk; ++q) w->tiles[res->id].i[q] = (int32_t)w->tiles[pv->id].f[2 * q + 1];
                break;
            }
            case OP_STORE_TOPK: { /* dst[i * s4] = (int)pairs[2i+1] (ptoisa_jit.py:445-456), no cycles */
                if (op->nopnd != 2 || res) fail("kernel %s: StoreTopkIndices expects (dst, pairs)", kn);
                int dst = op->opnd[0];
                int pi = k->param_of[dst];
                Val* dv = k->by_id[dst];
                Val* pv = k->by_id[op->opnd[1]];
                if (pi < 0 || !dv->tile) fail("kernel %s: StoreTopkIndices dst must be a kernel param tile", kn);
                if (dv->dtype != DT_I32 && dv->dtype != DT_I64) fail("kernel %s: StoreTopkIndices dst must be i32 or i64", kn);
                if (!pv->tile || pv->rows != 1 || pv->cols != 64 || pv->dtype != DT_F32)
                    fail("kernel %s: StoreTopkIndices expects [1,64] f32 pairs", kn);
                if (!op->has_k || op->k < 1 || op->k > 32 || op->k > dv->cols)
                    fail("kernel %s: StoreTopkIndices k must be in [1, min(32, dst cols)]", kn);
                View* v = &views[k->tensor_index[pi]];
                for (int64_t q = 0; q < op->k; ++q) {
                    int64_t x = (int32_t)w->tiles[pv->id].f[2 * q + 1];
                    char* p = v->ptr + (q * v->s4) * k_dtype_size[v->dtype];
                    if (v->dtype == DT_I32) { int32_t y = (int32_t)x; memcpy(p, &y, 4); }
                    else memcpy(p, &x, 8);
                }
                break;
            }
            case OP_ADD_CYCLES: /* pto::cpu_sim::add_cycles(n) (ptoisa_jit.py:458-463) */
                if (op->cycles_expr) {
                    int nscal = 0;
                    for (int i = 0; i < k->nparams; ++i)
                        if (!k->by_id[k->params[i].id]->tile) ++nscal;
                    cycles += cycles_expr_value(op->cycles_expr, scalar_args, nscal);
                    break;
                }
                if (!op->has_cycles || op->cycles < 0) fail("kernel %s: CpuSimAddCycles needs a cycles attr", kn);
                cycles += (uint64_t)op->cycles;
                break;
            default:
                /* The emitter adds r*c cycles and computes nothing for other op
                 * kinds (:1223-1231); the oracle refuses them instead. */
                fail("kernel %s: op kind has no compute in the reference cpu_sim lowering", kn);
        }
    }
    return cycles;
}

/* ------------------------------------------------------------------ */
/* workload walk (src/python/pto_codegen.cpp:2305-2700)                 */
/* ------------------------------------------------------------------ */

typedef struct TaskScratch { Work* w; View* views; uint64_t* scal; } TaskScratch;

static uint64_t fnv1a_64(const char* s) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (const unsigned char* p = (const unsigned char*)s; *p; ++p) {
        h ^= *p;
        h *= 0x100000001B3ULL;
    }
    return h;
}

static int64_t axis_extent(Run* R, Node* n) {
    switch (n->axis_kind) {
        case AX_DENSE: return n->axis_size;
        case AX_DYN: return R->ctx->get_axis_size(R->ctx->ctx, n->axis_a);
        case AX_RAGGED: {
            /* ub = sum of lengths[0..outer) read through symbols (:2321-2340). */
            int64_t outer = (int64_t)R->ctx->get_symbol_u64(R->ctx->ctx, fnv1a_64(n->axis_a));
            const int32_t* len = (const int32_t*)R->ctx->get_symbol_ptr(R->ctx->ctx, fnv1a_64(n->axis_b));
            int64_t ub = 0;
            if (len)
                for (int64_t i = 0; i < outer; ++i) ub += len[i];
            return ub;
        }
        case AX_DYNT: return eval_iexpr(R, n->axis_expr);
    }
    return 0;
}

static void push_var(Run* R, const char* name, int64_t v) {
    if (R->nenv >= 64) fail("loop nest deeper than 64");
    R->env[R->nenv].name = name;
    R->env[R->nenv].value = v;
    R->nenv++;
}

/* ---- scalar expressions: the C expression the reference emits for each
 * node (src/python/pto_codegen.cpp:220-300, slot / param reads :2232-2238,
 * :2663-2678), evaluated with C's usual arithmetic conversions: _Bool
 * promotes to int, an unsigned 64-bit operand makes the operation unsigned.
 * Undefined cases are refused (division by zero, INT64_MIN / -1, shift
 * counts outside [0, 64)); signed + - * wrap. */
typedef struct { char t; uint64_t v; } SV;

static char sx_promo(char t) { return t == 'b' ? 'i' : t; }
static char sx_usual(char a, char b) { return (a == 'u' || b == 'u') ? 'u' : 'i'; }
static int sx_is_cmp(const char* op) {
    return !strcmp(op, "<") || !strcmp(op, "<=") || !strcmp(op, ">") || !strcmp(op, ">=") || !strcmp(op, "==") ||
           !strcmp(op, "!=");
}

static char sx_type(const SX* e) {
    switch (e->kind) {
        case 'L': case 'P': case 'A': case 'S': case 'C': case 'K': return e->ty;
        case 'G': case 'Y': return 'u';
        case 'U': return e->op[0] == '!' ? 'b' : sx_promo(sx_type(e->a));
        case 'B':
            if (sx_is_cmp(e->op) || !strcmp(e->op, "&&") || !strcmp(e->op, "||")) return 'b';
            if (!strcmp(e->op, "<<") || !strcmp(e->op, ">>")) return sx_promo(sx_type(e->a));
            return sx_usual(sx_promo(sx_type(e->a)), sx_promo(sx_type(e->b)));
        case 'T': {
            char t = sx_type(e->b), f = sx_type(e->c);
            return (t == 'b' && f == 'b') ? 'b' : sx_usual(sx_promo(t), sx_promo(f));
        }
    }
    return 'i';
}

static SV sx_read(uint64_t raw, char ty) {
    SV r = {ty, ty == 'b' ? (uint64_t)(raw != 0) : raw};
    return r;
}

/* The scalar arguments of the task whose cycle expressions are evaluated. */
static const uint64_t* g_kscal = NULL;
static int g_nkscal = 0;

static SV sx_eval(Run* R, const SX* e, const uint64_t* args, int nargs) {
    SV r = {'i', 0};
    switch (e->kind) {
        case 'L': r.t = e->ty; r.v = e->u; return r;
        case 'P':
            if (!args) fail("emit_scalar_expr_cpp: task_param() requires task_param_expr callback");
            return sx_read(e->u < (uint64_t)nargs ? args[e->u] : 0, e->ty);
        case 'K':
            if (!g_kscal) fail("kernel scalar parameter read outside a task");
            return sx_read(e->u < (uint64_t)g_nkscal ? g_kscal[e->u] : 0, e->ty);
        case 'G':
        case 'Y': r.t = 'u'; r.v = R->ctx->get_symbol_u64(R->ctx->ctx, e->u); return r;
        case 'S':
            return sx_read(R->ctx->get_slot_u64 ? R->ctx->get_slot_u64(R->ctx->ctx, (uint32_t)e->u) : 0, e->ty);
        case 'A': {
            for (int i = R->nenv - 1; i >= 0; --i)
                if (fnv1a_64(R->env[i].name) == e->u) {
                    if (e->ty == 'b') fail("emit_scalar_expr_cpp: axis_var invalid type");
                    r.t = e->ty;
                    r.v = (uint64_t)R->env[i].value;
                    return r;
                }
            fail("emit_scalar_expr_cpp: axis_var not in scope");
            return r;
        }
        case 'U': {
            SV x = sx_eval(R, e->a, args, nargs);
            if (e->op[0] == '!') { r.t = 'b'; r.v = x.v == 0; return r; }
            r.t = sx_promo(x.t);
            r.v = e->op[0] == '-' ? (uint64_t)0 - x.v : ~x.v;
            return r;
        }
        case 'T': {
            char t = sx_type(e);
            SV c = sx_eval(R, e->a, args, nargs);
            SV x = sx_eval(R, c.v ? e->b : e->c, args, nargs);
            r.t = t;
            r.v = t == 'b' ? (x.v != 0) : x.v;
            return r;
        }
        case 'C': {
            SV x = sx_eval(R, e->a, args, nargs);
            r.t = e->ty;
            r.v = e->ty == 'b' ? (uint64_t)(x.v != 0) : x.v;
            return r;
        }
        case 'B': {
            const char* op = e->op;
            if (!strcmp(op, "&&") || !strcmp(op, "||")) {
                SV a = sx_eval(R, e->a, args, nargs);
                r.t = 'b';
                if (op[0] == '&' && !a.v) return r;
                if (op[0] == '|' && a.v) { r.v = 1; return r; }
                r.v = sx_eval(R, e->b, args, nargs).v != 0;
                return r;
            }
            SV a = sx_eval(R, e->a, args, nargs), b = sx_eval(R, e->b, args, nargs);
            a.t = sx_promo(a.t);
            b.t = sx_promo(b.t);
            if (!strcmp(op, "<<") || !strcmp(op, ">>")) {
                if ((b.t == 'i' && (int64_t)b.v < 0) || b.v >= 64) fail("scalar expression: shift count out of range");
                r.t = a.t;
                if (op[0] == '<') r.v = a.v << b.v;
                else r.v = a.t == 'i' ? (uint64_t)((int64_t)a.v >> b.v) : a.v >> b.v;
                return r;
            }
            char t = sx_usual(a.t, b.t);
            if (sx_is_cmp(op)) {
                int lt, eq;
                if (t == 'u') { lt = a.v < b.v; eq = a.v == b.v; }
                else { lt = (int64_t)a.v < (int64_t)b.v; eq = a.v == b.v; }
                r.t = 'b';
                if (!strcmp(op, "<")) r.v = lt;
                else if (!strcmp(op, "<=")) r.v = lt || eq;
                else if (!strcmp(op, ">")) r.v = !lt && !eq;
                else if (!strcmp(op, ">=")) r.v = !lt;
                else if (!strcmp(op, "==")) r.v = eq;
                else r.v = !eq;
                return r;
            }
            r.t = t;
            if (!strcmp(op, "+")) r.v = a.v + b.v;
            else if (!strcmp(op, "-")) r.v = a.v - b.v;
            else if (!strcmp(op, "*")) r.v = a.v * b.v;
            else if (!strcmp(op, "&")) r.v = a.v & b.v;
            else if (!strcmp(op, "|")) r.v = a.v | b.v;
            else if (!strcmp(op, "^")) r.v = a.v ^ b.v;
            else if (!strcmp(op, "/") || !strcmp(op, "%")) {
                if (!b.v) fail("scalar expression: division by zero");
                if (t == 'u') r.v = op[0] == '/' ? a.v / b.v : a.v % b.v;
                else {
                    int64_t x = (int64_t)a.v, y = (int64_t)b.v;
                    if (x == INT64_MIN && y == -1) fail("scalar expression: signed division overflow");
                    r.v = (uint64_t)(op[0] == '/' ? x / y : x % y);
                }
            } else {
                fail("scalar expression: bad operator '%s'", op);
            }
            return r;
        }
    }
    fail("scalar expression: bad node");
    return r;
}

/* (uint64_t)(e) with the task's kernel scalar arguments (the expression reads
 * nothing else, checked when it is parsed). */
static uint64_t cycles_expr_value(const SX* e, const uint64_t* kscal, int nk) {
    g_kscal = kscal;
    g_nkscal = nk;
    SV v = sx_eval(NULL, e, NULL, 0);
    g_kscal = NULL;
    g_nkscal = 0;
    return v.v;
}

/* `(uint64_t)element` of a slot load (src/python/pto_codegen.cpp:2254-2303). */
static uint64_t slot_load_value(Run* R, Node* n) {
    TArg* t = &n->slot_view;
    int tid = t->tid;
    int64_t off = 0;
    for (int d = 0; d < t->nidx; ++d) off += eval_iexpr(R, &t->idx[d]) * R->tstride[tid * 8 + d];
    int64_t s3 = 0, s4 = 1;
    if (t->view_rank >= 2) {
        int d3 = t->base_rank - t->view_rank;
        s3 = R->tstride[tid * 8 + d3];
        s4 = R->tstride[tid * 8 + d3 + 1];
    } else if (t->view_rank == 1) {
        s4 = R->tstride[tid * 8 + t->base_rank - 1];
    }
    off += n->slot_row * s3 + n->slot_col * s4;
    check_span(R, tid, off, off, "slot_load_u64");
    int dt = R->m->tensors[tid].dtype;
    const char* p = R->tbase[tid] + off * k_dtype_size[dt];
    float f;
    switch (dt) {
        case DT_F32: memcpy(&f, p, 4); break;
        case DT_F16: { uint16_t h; memcpy(&h, p, 2); f = half_to_float(h); break; }
        case DT_I32: { int32_t x; memcpy(&x, p, 4); return (uint64_t)(int64_t)x; }
        case DT_U32: { uint32_t x; memcpy(&x, p, 4); return x; }
        case DT_I64:
        case DT_U64: { uint64_t x; memcpy(&x, p, 8); return x; }
        case DT_BOOL: return *(const unsigned char*)p != 0;
        default: fail("Unsupported dtype for workload codegen: %s", k_dtype_names[dt]); return 0;
    }
    if (!(f > -1.0f) || !(f < 18446744073709551616.0f)) fail("slot_load_u64: the element is not representable as u64");
    return (uint64_t)f;
}

/* A task's argument vector: axis args, (rows, cols) per tile param, scalar
 * args (src/python/pto_codegen.cpp:2503-2545).  Returns the count. */
static int task_args(Run* R, Node* n, Kernel* k, const uint64_t* scal, uint64_t* args, int cap) {
    int na = 0;
    for (int i = 0; i < n->naxis; ++i) {
        Arg* a = &n->axis[i];
        if (na >= cap) fail("task %s: too many arguments", k->name);
        args[na++] = a->kind == 'v' ? (uint64_t)lookup(R, a->var)
                   : a->kind == 's' ? R->ctx->get_symbol_u64(R->ctx->ctx, a->u64)
                                    : a->u64;
    }
    for (int i = 0; i < k->nparams; ++i) {
        Val* v = k->by_id[k->params[i].id];
        if (!v->tile) continue;
        if (na + 2 > cap) fail("task %s: too many arguments", k->name);
        args[na++] = (uint64_t)v->rows;
        args[na++] = (uint64_t)v->cols;
    }
    for (int i = 0; i < n->nscal; ++i) {
        if (na >= cap) fail("task %s: too many arguments", k->name);
        args[na++] = scal[i];
    }
    return na;
}

static uint64_t eval_node(Run* R, Node* n, uint64_t ready);

static uint64_t run_task(Run* R, Node* n, uint64_t ready) {
    Kernel* k = n->kernel;
    int kidx = (int)(k - R->m->kernels);
    TaskScratch* s = R->scratch[kidx];
    if (!s) {
        s = (TaskScratch*)alloc(sizeof(TaskScratch));
        s->w = kernel_work(k);
        s->views = (View*)alloc(sizeof(View) * (size_t)(k->ntensor_params + 1));
        s->scal = (uint64_t*)alloc(sizeof(uint64_t) * (size_t)(n->nscal + 8));
        R->scratch[kidx] = s;
    }
    /* Scalar args: loop var, symbol lookup, or literal (:193-203). */
    int nscal_params = 0;
    for (int i = 0; i < k->nparams; ++i)
        if (!k->by_id[k->params[i].id]->tile) ++nscal_params;
    if (n->nscal != nscal_params) fail("task %s: %d scalar args for %d scalar params", k->name, n->nscal, nscal_params);
    for (int i = 0; i < n->nscal; ++i) {
        Arg* a = &n->scal[i];
        s->scal[i] = a->kind == 'v' ? (uint64_t)lookup(R, a->var)
                   : a->kind == 's' ? R->ctx->get_symbol_u64(R->ctx->ctx, a->u64)
                                    : a->u64;
    }
    /* Tensor bindings in kernel param order; pointer = base + sum(idx*stride),
     * s3/s4 from the view rank (:2556-2621). */
    for (int i = 0; i < k->nparams; ++i) {
        Val* v = k->by_id[k->params[i].id];
        if (!v->tile) continue;
        TArg* ta = NULL;
        for (int j = 0; j < n->nten; ++j)
            if (strcmp(n->ten[j].param, k->params[i].name) == 0) ta = &n->ten[j];
        if (!ta) fail("Missing tensor arg for param: %s", k->params[i].name);
        int tid = ta->tid;
        int64_t off = 0;
        if (ta->nidx > R->m->tensors[tid].rank) fail("task %s: too many indices for tensor %d", k->name, tid);
        for (int d = 0; d < ta->nidx; ++d) off += eval_iexpr(R, &ta->idx[d]) * R->tstride[tid * 8 + d];
        int64_t s3 = 0, s4 = 1;
        if (ta->view_rank >= 2) {
            int d3 = ta->base_rank - ta->view_rank;
            s3 = R->tstride[tid * 8 + d3];
            s4 = R->tstride[tid * 8 + d3 + 1];
        } else if (ta->view_rank == 1) {
            s4 = R->tstride[tid * 8 + ta->base_rank - 1];
        }
        if (s3 < 0 || s4 < 0) fail("negative strides are not supported");
        if (R->m->tensors[tid].dtype != v->dtype)
            fail("task %s: param %s is %s but tensor %d is %s", k->name, k->params[i].name,
                 k_dtype_names[v->dtype], tid, k_dtype_names[R->m->tensors[tid].dtype]);
        check_span(R, tid, off, off + (int64_t)(v->rows - 1) * s3 + (int64_t)(v->cols - 1) * s4, k->name);
        View* vw = &s->views[k->tensor_index[i]];
        vw->ptr = R->tbase[tid] + off * k_dtype_size[v->dtype];
        vw->dtype = v->dtype;
        vw->s3 = s3;
        vw->s4 = s4;
    }
    uint64_t dur;
    if (k->custom) {
        /* A cpp_src body or cpp_tu_path file, called through the runtime's kernel table with the
         * reference's task descriptor (include/pto/wsp/codegen/abi/kernel_abi.hpp:21-41). */
        KernelFn fn = R->ctx->get_kernel ? R->ctx->get_kernel(R->ctx->ctx, (uint32_t)kidx) : NULL;
        if (!fn) fail("kernel %s: no compiled custom kernel", k->name);
        uint64_t args[64];
        void* ptrs[32];
        uint64_t strides[64];
        int na = task_args(R, n, k, s->scal, args, 64), nt = 0;
        for (int i = 0; i < k->nparams; ++i) {
            if (!k->by_id[k->params[i].id]->tile) continue;
            if (nt >= 32) fail("kernel %s: too many tile params", k->name);
            View* vw = &s->views[k->tensor_index[i]];
            ptrs[nt] = (void*)vw->ptr;
            strides[2 * nt] = (uint64_t)vw->s3;
            strides[2 * nt + 1] = (uint64_t)vw->s4;
            ++nt;
        }
        /* kernel_id and task_id are 0, as the reference's artifact passes them
         * (src/python/pto_codegen.cpp:2645-2649). */
        KernelTaskDesc d = {args, (uint32_t)na, (uint32_t)(n->naxis + 2 * nt), ptrs, strides, (uint32_t)nt, 0u, 0u};
        dur = fn(&d, NULL);
    } else {
        dur = run_kernel(k, s->w, s->views, s->scal);
    }
    ++g_tasks;
    uint32_t wid = 0;
    if (R->m->has_dispatch && !R->m->dispatch_key) wid = (uint32_t)(R->rr++ % R->workers);
    if (R->m->dispatch_key) {
        /* worker = key % workers (src/python/pto_codegen.cpp:2679-2690). */
        uint64_t args[64];
        int na = task_args(R, n, k, s->scal, args, 64);
        wid = (uint32_t)(sx_eval(R, R->m->dispatch_key, args, na).v % R->workers);
    }
    return issue(R, dur, wid, ready);
}

static uint64_t eval_node(Run* R, Node* n, uint64_t ready) {
    switch (n->kind) {
        case N_EMPTY: return ready;
        case N_PFOR: {
            uint64_t done = ready;
            int64_t ub = axis_extent(R, n);
            for (int64_t i = 0; i < ub; ++i) {
                push_var(R, n->var, i);
                uint64_t d = eval_node(R, n->body, ready);
                R->nenv--;
                if (d > done) done = d;
            }
            return done;
        }
        case N_EACH: {
            uint64_t cur = ready;
            int64_t ub = axis_extent(R, n);
            for (int64_t i = 0; i < ub; ++i) {
                push_var(R, n->var, i);
                cur = eval_node(R, n->body, cur);
                R->nenv--;
            }
            return cur;
        }
        case N_COMB: {
            uint64_t done = ready;
            for (int i = 0; i < n->nkids; ++i) {
                uint64_t d = eval_node(R, n->kids[i], ready);
                if (d > done) done = d;
            }
            return done;
        }
        case N_SEQN: {
            uint64_t cur = ready;
            for (int i = 0; i < n->nkids; ++i) cur = eval_node(R, n->kids[i], cur);
            return cur;
        }
        case N_TASK: return run_task(R, n, ready);
        case N_SEL: {
            /* CSR select (:2417-2452). */
            int64_t outer = (int64_t)R->ctx->get_symbol_u64(R->ctx->ctx, fnv1a_64(n->sel_outer));
            const int32_t* indptr = (const int32_t*)R->ctx->get_symbol_ptr(R->ctx->ctx, fnv1a_64(n->sel_indptr));
            const int32_t* indices = (const int32_t*)R->ctx->get_symbol_ptr(R->ctx->ctx, fnv1a_64(n->sel_indices));
            int64_t nnz = indptr ? indptr[outer] : 0;
            uint64_t done = ready;
            for (int64_t p = 0; p < nnz; ++p) {
                push_var(R, n->var, indices ? indices[p] : 0);
                uint64_t d = eval_node(R, n->body, ready);
                R->nenv--;
                if (d > done) done = d;
            }
            return done;
        }
        case N_COND:
            /* src/python/pto_codegen.cpp:2458-2478. */
            return eval_node(R, n->kids[sx_eval(R, n->pred, NULL, 0).v ? 0 : 1], ready);
        case N_SLOTSET:
            if (R->ctx->set_slot_u64) R->ctx->set_slot_u64(R->ctx->ctx, n->slot, n->slot_value);
            return ready;
        case N_SLOTLD: {
            uint64_t v = slot_load_value(R, n);
            if (R->ctx->set_slot_u64) R->ctx->set_slot_u64(R->ctx->ctx, n->slot, v);
            return ready;
        }
    }
    return ready;
}

/* ------------------------------------------------------------------ */
/* entry point                                                          */
/* ------------------------------------------------------------------ */

int pto_cpusim_run(const char* module_text, RuntimeContext* ctx, uint64_t* total_cycles) {
    jmp_buf jb;
    jmp_buf* prev = g_jmp;
    g_jmp = &jb;
    g_err[0] = 0;
    g_tasks = 0;
    volatile int rcode = 0;
    if (setjmp(jb) == 0) {
        Module* m = (Module*)alloc(sizeof(Module));
        parse_module(module_text, m);
        Run* R = (Run*)alloc(sizeof(Run));
        R->m = m;
        R->ctx = ctx;
        R->tbase = (char**)alloc(sizeof(char*) * (size_t)(m->ntensors + 1));
        R->tstride = (int64_t*)alloc(sizeof(int64_t) * 8 * (size_t)(m->ntensors + 1));
        R->tspan = (int64_t*)alloc(sizeof(int64_t) * (size_t)(m->ntensors + 1));
        for (int t = 0; t < m->ntensors; ++t) {
            R->tbase[t] = (char*)ctx->get_tensor_ptr(ctx->ctx, (uint32_t)t);
            int64_t span = 1;
            for (int d = 0; d < m->tensors[t].rank; ++d) {
                int64_t st = (int64_t)ctx->get_tensor_stride(ctx->ctx, (uint32_t)t, (uint32_t)d);
                R->tstride[t * 8 + d] = st;
                if (m->tensors[t].shape[d] == 0) span = 0;
            }
            if (span) {
                int64_t mx = 0;
                for (int d = 0; d < m->tensors[t].rank; ++d) {
                    if (R->tstride[t * 8 + d] < 0) fail("tensor %d: negative strides are not supported", t);
                    mx += (m->tensors[t].shape[d] - 1) * R->tstride[t * 8 + d];
                }
                span = mx + 1;
            }
            R->tspan[t] = span;
            if (span && !R->tbase[t]) fail("tensor %d has no data", t);
        }
        /* Worker lanes and window (src/python/pto_codegen.cpp:1527-1545). */
        int64_t W = 1;
        if (m->has_dispatch && m->num_targets > 0) W = m->num_targets;
        else if (m->has_streams && m->num_streams > 0) W = m->num_streams;
        R->workers = (uint32_t)(W > 0 ? W : 1);
        R->window = (m->has_window && m->window_ok && m->window_size > 0) ? (uint64_t)m->window_size : 0;
        R->avail = (uint64_t*)alloc(sizeof(uint64_t) * R->workers);
        R->scratch = (TaskScratch**)alloc(sizeof(TaskScratch*) * (size_t)(m->nkernels + 1));
        *total_cycles = eval_node(R, m->root, 0);
    } else {
        rcode = -1;
    }
    g_jmp = prev;
    arena_free();
    return rcode;
}

uint64_t pto_cpusim_last_task_count(void) { return g_tasks; }

int pto_cpusim_eval_scalar(const char* expr_text, RuntimeContext* ctx, uint64_t* value, char* type) {
    jmp_buf jb;
    jmp_buf* prev = g_jmp;
    g_jmp = &jb;
    g_err[0] = 0;
    volatile int rcode = 0;
    if (setjmp(jb) == 0) {
        Lex L = {expr_text};
        SX* e = parse_sx(&L);
        while (*L.p == ' ' || *L.p == '\n' || *L.p == '\t') ++L.p;
        if (*L.p) fail("scalar expression: trailing text '%s'", L.p);
        Module m;
        memset(&m, 0, sizeof m);
        Run* R = (Run*)alloc(sizeof(Run));
        R->m = &m;
        R->ctx = ctx;
        SV v = sx_eval(R, e, NULL, 0);
        *value = v.v;
        *type = v.t;
    } else {
        rcode = -1;
    }
    g_jmp = prev;
    arena_free();
    return rcode;
}

const char* pto_cpusim_last_error(void) { return g_err; }
