// Per-kernel analysis: validation against the reference lowering rules,
// the static cpu_sim cycle cost of one task, and the choice of device
// template family.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "module.hpp"

namespace ptowsp {

// How a binary op combines its operands (src/python/pto_codegen.cpp:1078-1107).
enum class BinMode { Same, RowExpand, ColExpand, ScalarRight, ScalarLeft };

enum class Family { RowProgram, TileProgram, Gemm, Decode, Custom };

// Role of a value inside a row program.
enum class RowClass { None, Full, RowVec, RowVecT, ColVec, ColVecT, Scalar };

// A kernel of the form  acc = matmul(a, b); [out = add(c, acc);] store(c, out|acc)
// with bf16/f16 a, b and an fp32 c: runs on MFMA with the accumulator on chip.
// K columns per LDS stage of a GEMM block: the task's K step; f32 A / B
// stages hold at most 32 columns (a task step of 64 or 128 is split over 2
// or 4 stages), bf16 / f16 stages 64 once a step exceeds 128 columns.
inline int gemm_stage_k(int k, bool f32) { return f32 ? (k > 32 ? 32 : k) : (k > 128 ? 64 : k); }
// Rows / columns of a GEMM block for a task tile dimension: tiles above 256
// (multiples of 256) are split into blocks of 256.
inline int gemm_block_dim(int t) { return t > 256 ? 256 : t; }

struct GemmInfo {
    bool ok = false;
    int a = -1, b = -1, c = -1;  // tensor ordinals
    int m = 0, n = 0, k = 0;
    bool f16 = false;
    bool f32 = false;            // f32 A and B (v_mfma_f32_32x32x2_f32)
    bool accumulate = false;     // c + a@b (InOut accumulator) instead of a@b
};

// Online-softmax decode step (flashinfer_decode over pages): with s = (q @ k_t)
// * scale [- mask], m' = max(m, rowmax(s)), p = exp(s - m'), a = exp(m - m'):
// l <- l*a + rowsum(p), o <- o*a + p @ v, m <- m'.  Folding the pages of a
// P.seq loop in any grouping gives the same (m, l, o) up to fp32 rounding.
struct DecodeInfo {
    bool ok = false;
    int q = -1, kt = -1, v = -1, mask = -1;  // tensor ordinals (mask -1: none)
    int m = -1, l = -1, o = -1;              // accumulators (InOut)
    int g = 0, d = 0, pg = 0;                // query rows, head dim, tokens per page
    bool f16 = false;                        // q / k / v are f16 (else bf16)
    bool f32 = false;                        // q / k / v are f32
    bool row_mask = false;                   // the [1, PG] mask is a row broadcast (G == PG == 16)
    float scale = 1.0f;                      // score scale (a Constant)
};

// out = o / l with o a [G,D] and l a [G,1] fp32 param (a row-broadcast
// divide) stored to a [G,D] fp32 param: the normalisation that follows the
// page loop of a decode workload.  Launched right after a decode launch
// over the same grid and the same o / l views, it is applied by the decode
// kernel to each unit it completes (bit for bit the same division).
struct NormInfo {
    bool ok = false;
    int o = -1, l = -1, out = -1;  // tensor ordinals
    int g = 0, d = 0;
};

struct KernelAnalysis {
    const KernelDef* def = nullptr;
    int max_id = 0;
    std::vector<const ValueInfo*> by_id;   // value id -> info
    std::vector<int> param_of;             // value id -> param index, -1
    std::vector<int> tensor_ordinal;       // param index -> tensor-param ordinal, -1
    std::vector<int> scalar_ordinal;       // param index -> scalar-param ordinal, -1
    std::vector<int> tensor_param_index;   // tensor ordinal -> param index
    std::vector<bool> preload;             // value id: param tile TLOADed at entry
    std::vector<bool> acc_vec;             // value id: matmul result moved to a vector tile
    std::vector<bool> stored;              // tensor ordinal: written by a Store
    std::vector<bool> read;                // tensor ordinal: read (preload, Load, Matmul operand)
    std::vector<BinMode> bin_mode;         // per op (binary ops only)
    uint64_t cycles = 0;                   // cpu_sim cycles of one task
    // Cycles added per task by expressions of the kernel's scalar parameters
    // (cpu_sim_add_cycles with an expression), evaluated with each task's
    // scalar arguments.
    std::vector<std::shared_ptr<const SExpr>> cycle_exprs;

    Family family = Family::TileProgram;
    // Row-program shape: every Full value is [rows, cols].
    int rows = 0, cols = 0;
    std::vector<RowClass> row_class;       // value id -> class
    std::string not_row_reason;
    GemmInfo gemm;
    DecodeInfo decode;
    NormInfo norm;
};

// Throws CompileError for kernels the reference lowering cannot compute.
KernelAnalysis analyze_kernel(const KernelDef& k);

}  // namespace ptowsp
