// Kernel-argument layout shared by the host library and every emitted HIP
// kernel (plain data, no device code).
#pragma once

namespace ptowsp {

typedef long long i64;
typedef unsigned long long u64;
typedef unsigned int u32;
typedef int i32;
typedef unsigned short u16;

constexpr int kMaxParams = 12;
constexpr int kMaxVars = 8;
constexpr int kMaxScalars = 8;
constexpr int kMaxIndirect = 4;
constexpr int kMaxAxisArgs = 8;

// One indirect index term: the element offset of a tensor param gets
// `stride * idx`, where idx is the int32 element base[c + sum(coef*var)].
struct IndirectTerm {
    const int* base;
    i64 coef[kMaxVars];
    i64 c;
    i64 span;   // addressable elements of the index tensor
    i64 bound;  // idx must lie in [0, bound)
    i64 stride;
};

// Arguments of every emitted launch (by value, in the kernarg segment).
// Loop variables are numbered grid loops first (outer->inner), then
// in-kernel loops (outer->inner).  The element offset of tensor param p is
// sum_v coef[p][v]*var_v plus its indirect terms; base[p] already includes
// the constant part and the values of host-level loop variables; span[p] is
// the number of elements addressable from base[p].
struct LaunchArgs {
    char* base[kMaxParams];
    i64 coef[kMaxParams][kMaxVars];
    i64 s3[kMaxParams];
    i64 s4[kMaxParams];
    i64 span[kMaxParams];
    i64 ext[kMaxVars];
    i64 ntasks;
    u64 scal[kMaxScalars];
    IndirectTerm ind[kMaxIndirect];
    int* err;  // 1: indirect index out of range, 2: tile outside its tensor,
               // 3: a tensor-bound loop extent above its declared maximum
    const i64* tlist;  // task-list launches: grid task index of task t (ascending)
    // cpp_src kernels: axis arguments known on the host (constants, symbols,
    // host loop variables), and where each task's reported cycles go (by
    // grid task index).
    u64 aarg[kMaxAxisArgs];
    u64* cyc;
};

}  // namespace ptowsp
