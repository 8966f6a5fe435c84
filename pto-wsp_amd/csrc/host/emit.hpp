// HIP source emission for one launch of a traced kernel.
#pragma once

#include <string>
#include <vector>

#include "analysis.hpp"
#include "plan.hpp"

namespace ptowsp {

// Launch-time facts a kernel is specialized on.
struct EmitSpec {
    int vec_width = 1;                 // row programs: 4, 2 or 1 floats per access
    std::vector<int> indirect_count;   // per tensor ordinal: indirect index terms (in dim order)
    std::vector<int> inner_dyn_term;   // per inner loop: indirect term index of its extent, or -1
    int threads = 256;
    // Run every task of the launch in program order in one workgroup: used
    // when tasks of the grid write overlapping memory (the result then
    // depends on the reference's sequential order).
    bool serial = false;
    // Row programs: the kernel's in-kernel (P.seq) loops run inside each row's
    // lane team (the host has checked that rows do not depend on each other).
    bool row_loops = false;
    // Serial launches: the grid variables (bit v) iterated in program order
    // inside a workgroup; the others are decoded from the block index, one
    // group of tasks per workgroup.  0 means all of them.
    uint32_t seq_mask = 0;
    // The launch runs the grid tasks listed in A.tlist (ascending), not all
    // of them: a task mask from a cond on grid variables.
    bool task_list = false;
    // Row programs: cap on passes per wave iteration, and non-temporal
    // (streaming) global accesses for full-row tiles.
    int row_up = 8;
    bool nontemporal = false;
    // Tile programs: matmul ops of MFMA shape (M, N multiples of 32) on the
    // matrix cores (tile_mma) instead of the scalar loop.
    bool tile_mma = true;
    // GEMM family on MFMA (only when strides and alignment allow it).
    bool gemm = false;
    // GEMM: grid variables whose neighbouring tasks are merged into one
    // workgroup block (factor 2 along rows / columns of C), or -1.
    int gemm_vm = -1, gemm_vn = -1;
    // GEMM: tasks per block along those variables (powers of two), and task
    // K steps per LDS stage (consecutive steps whose A columns and B rows
    // are adjacent, in the accumulate form).
    int gemm_fm = 1, gemm_fn = 1, gemm_kf = 1;
    // GEMM: 256x256 blocks with K step 32 or 64 and A / B row pitches that
    // are multiples of 64 elements run as a two-group ping-pong block.
    bool gemm_pingpong = false;
    // Decode family (online softmax over pages): the in-kernel page loop of
    // every unit is split over the resident waves.
    bool decode = false;
    // Decode: the next launch (a NormInfo kernel over the same grid and o / l
    // views) is folded in; its output tensor is argument slot ntens + 1.
    bool decode_norm = false;
    // Decode: pages in each wave's register ring, and waves per block (4:
    // one per SIMD; 8: two per SIMD, 256 VGPRs each).
    int decode_ring = 4;
    int decode_waves = 4;
    bool decode_ordered = false;  // release / acquire fences around the unit completion count
};

// Units (grid tasks) of one decode launch at most: every block holds their
// page-count prefix in LDS (DecodeSplit::kMaxUnits on the device).
constexpr int kDecodeMaxUnits = 4096;
// Scheduling cost of starting a unit, in pages (DecodeSplit::kUnitCost).
constexpr int kDecodeUnitCost = 3;

// Waves of a GEMM block: 2 along M, 4 along N for 256-wide blocks, else 2.
inline int gemm_waves_n(int bn) { return bn >= 256 ? 4 : 2; }
inline int gemm_waves_m() { return 2; }

struct EmittedKernel {
    std::string source;
    std::string entry;          // kernel symbol
    int threads = 256;
    int rows_per_chunk = 0;     // row programs: rows handled per wave iteration
    int waves_per_block = 4;
    bool row_program = false;
    int tasks_per_block = 1;    // GEMM: tasks merged into one workgroup
    int blocks_per_task = 1;    // GEMM: 256-wide blocks of a task tile above 256
    int part_floats = 0;        // decode: floats per partial (m, l, o of one unit)
    size_t lds_bytes = 0;
    // Tile programs: bytes of global scratch per workgroup for the tiles that
    // do not fit in LDS (base[ntens] of the launch; the grid is capped so
    // that blocks x gtile_bytes stays bounded).
    size_t gtile_bytes = 0;
};

EmittedKernel emit_launch(const Module& m, const KernelAnalysis& a, const LaunchSpec& L, const EmitSpec& spec);

// Parameters of the row-program layout for a row of `cols` floats with
// accesses `vw` wide: lanes per row G, chunks per lane NV, unrolled passes UP.
struct RowLayout {
    int vw = 1, g = 1, nv = 1, up = 1;
};
RowLayout row_layout(int cols, int vw, int up_cap = 8);

}  // namespace ptowsp
