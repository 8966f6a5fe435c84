// Hand-written CDNA4 (gfx950) device templates for the PTO-WSP HIP backend.
//
// The host library emits one small kernel per launch of a traced @kernel and
// compiles it with hiprtc; those kernels are written in terms of the
// templates below.  No host code, no CUDA shims: wave64, 128-bit global
// accesses, xor-butterfly reductions inside a wavefront, LDS tiles.
//
// Families:
//   * row programs   - vector-only kernels whose tiles are [R,C] / [R,1] /
//                      broadcast [1,C]; every row is an independent job for a
//                      "team" of G lanes holding the row in registers.
//   * tile programs  - anything else (matmul, in-kernel sequential loops):
//                      one workgroup per task, values in LDS, each op a
//                      cooperative pass separated by barriers.
#pragma once

#include "ptowsp_launch.h"

namespace ptowsp {

__device__ inline float bits_f32(u64 b) { return __uint_as_float(static_cast<u32>(b)); }

// Reads one element of an indirect index; out-of-range indices are clamped
// to 0 after raising the error flag, so the access stays in bounds.
__device__ inline i64 indirect_value(const LaunchArgs& A, int k, const i64* vars, int nvars) {
    const IndirectTerm& t = A.ind[k];
    i64 off = t.c;
    for (int v = 0; v < nvars; ++v) off += t.coef[v] * vars[v];
    i64 idx = 0;
    if (off >= 0 && off < t.span) idx = t.base[off];
    if (off < 0 || off >= t.span || idx < 0 || idx >= t.bound) {
        *A.err = 1;
        idx = 0;
    }
    return idx;
}
__device__ inline i64 indirect_index(const LaunchArgs& A, int k, const i64* vars, int nvars) {
    return indirect_value(A, k, vars, nvars) * A.ind[k].stride;
}

// ---------------------------------------------------------------------------
// Row programs
// ---------------------------------------------------------------------------

// Per-lane share of one row: NV chunks of VW contiguous elements.  Chunk k
// of team lane j covers columns (k*G + j)*VW .. +VW-1, so for each k the G
// lanes of a team read one contiguous run of G*VW elements.
template <int NV, int VW>
struct RowSlice {
    float v[NV * VW];
};

typedef float f32x4v __attribute__((ext_vector_type(4)));

// NT: non-temporal (streaming) accesses, for data touched exactly once.
template <int NV, int VW, int G, bool NT = false>
__device__ inline void row_load(RowSlice<NV, VW>& r, const float* p, i64 s4, int j) {
    if constexpr (VW == 4) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const f32x4v* q = reinterpret_cast<const f32x4v*>(p + (k * G + j) * 4);
            const f32x4v x = NT ? __builtin_nontemporal_load(q) : *q;
            r.v[k * 4 + 0] = x.x;
            r.v[k * 4 + 1] = x.y;
            r.v[k * 4 + 2] = x.z;
            r.v[k * 4 + 3] = x.w;
        }
    } else if constexpr (VW == 2) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const float2 x = *reinterpret_cast<const float2*>(p + (k * G + j) * 2);
            r.v[k * 2 + 0] = x.x;
            r.v[k * 2 + 1] = x.y;
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) r.v[k] = p[static_cast<i64>(k * G + j) * s4];
    }
}

// Same lane layout, element-wise loads through an arbitrary stride.
template <int NV, int VW, int G>
__device__ inline void row_load_strided(RowSlice<NV, VW>& r, const float* p, i64 stride, int j) {
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < VW; ++e) r.v[k * VW + e] = p[static_cast<i64>((k * G + j) * VW + e) * stride];
}

template <int NV, int VW, int G, bool NT = false>
__device__ inline void row_store(float* p, const RowSlice<NV, VW>& r, i64 s4, int j) {
    if constexpr (VW == 4) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            f32x4v* q = reinterpret_cast<f32x4v*>(p + (k * G + j) * 4);
            f32x4v x;
            x.x = r.v[k * 4 + 0];
            x.y = r.v[k * 4 + 1];
            x.z = r.v[k * 4 + 2];
            x.w = r.v[k * 4 + 3];
            if (NT) __builtin_nontemporal_store(x, q);
            else *q = x;
        }
    } else if constexpr (VW == 2) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            *reinterpret_cast<float2*>(p + (k * G + j) * 2) = make_float2(r.v[k * 2 + 0], r.v[k * 2 + 1]);
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) p[static_cast<i64>(k * G + j) * s4] = r.v[k];
    }
}

// Lane-local then team-wide reductions.  The xor butterfly leaves the same
// (bitwise) value in every lane of the team because fp addition commutes.
template <int N>
__device__ inline float lane_sum(const float* v) {
    float a = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) a = a + v[i];
    return a;
}

template <int N>
__device__ inline float lane_max(const float* v) {
    float a = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) a = v[i] > a ? v[i] : a;
    return a;
}

template <int G>
__device__ inline float team_sum(float x) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) x = x + __shfl_xor(x, o, 64);
    return x;
}

template <int G>
__device__ inline float team_max(float x) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) {
        const float y = __shfl_xor(x, o, 64);
        x = y > x ? y : x;
    }
    return x;
}

// Elementwise binary ops with the cpu_sim operator semantics (a>b?a:b for max).
struct OpAdd { template <class T> __device__ static T f(T a, T b) { return a + b; } };
struct OpSub { template <class T> __device__ static T f(T a, T b) { return a - b; } };
struct OpMul { template <class T> __device__ static T f(T a, T b) { return a * b; } };
struct OpDiv { template <class T> __device__ static T f(T a, T b) { return a / b; } };
struct OpMax { template <class T> __device__ static T f(T a, T b) { return a > b ? a : b; } };
struct OpMin { template <class T> __device__ static T f(T a, T b) { return a < b ? a : b; } };

template <class Op, int NV, int VW>
__device__ inline RowSlice<NV, VW> ew(const RowSlice<NV, VW>& a, const RowSlice<NV, VW>& b) {
    RowSlice<NV, VW> r;
#pragma unroll
    for (int i = 0; i < NV * VW; ++i) r.v[i] = Op::f(a.v[i], b.v[i]);
    return r;
}

template <class Op, int NV, int VW>
__device__ inline RowSlice<NV, VW> ew_rs(const RowSlice<NV, VW>& a, float s) {
    RowSlice<NV, VW> r;
#pragma unroll
    for (int i = 0; i < NV * VW; ++i) r.v[i] = Op::f(a.v[i], s);
    return r;
}

template <class Op, int NV, int VW>
__device__ inline RowSlice<NV, VW> ew_sr(float s, const RowSlice<NV, VW>& a) {
    RowSlice<NV, VW> r;
#pragma unroll
    for (int i = 0; i < NV * VW; ++i) r.v[i] = Op::f(s, a.v[i]);
    return r;
}

template <int NV, int VW>
__device__ inline RowSlice<NV, VW> ew_exp(const RowSlice<NV, VW>& a) {
    RowSlice<NV, VW> r;
#pragma unroll
    for (int i = 0; i < NV * VW; ++i) r.v[i] = expf(a.v[i]);
    return r;
}

// TRSQRT restated as two correctly rounded operations, 1/sqrt(x).
__device__ inline float rsqrt_cr(float x) { return 1.0f / sqrtf(x); }

template <int NV, int VW>
__device__ inline RowSlice<NV, VW> ew_rsqrt(const RowSlice<NV, VW>& a) {
    RowSlice<NV, VW> r;
#pragma unroll
    for (int i = 0; i < NV * VW; ++i) r.v[i] = rsqrt_cr(a.v[i]);
    return r;
}

// ---------------------------------------------------------------------------
// Tile programs (one workgroup per task, values in LDS)
// ---------------------------------------------------------------------------

__device__ inline float half_bits_to_f32(u16 h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ inline float bf16_bits_to_f32(u16 b) { return __uint_as_float(static_cast<u32>(b) << 16); }

// f32 -> f16, round to nearest even.  The empty asm makes f an opaque f32
// register value: without it the compiler folds a producing f32 multiply
// into the conversion (v_fma_mixlo_f16: one rounding of the exact product,
// where the oracle rounds the product to f32 and then to f16).
__device__ inline u16 f32_to_half_bits(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(u16, static_cast<_Float16>(f));
}

// Round-to-nearest-even f32 -> bf16 (NaN stays NaN).
__device__ inline u16 f32_to_bf16_bits(float f) {
    const u32 x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<u16>((x >> 16) | 0x40u);
    return static_cast<u16>((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// Row store into a 16-bit float tile (DT 0: f16, 1: bf16), each element
// rounded to nearest even as tile_store_f does; the same lane layout as
// row_store, VW 16-bit values per chunk.
template <int DT>
__device__ inline u16 f32_to_h16_bits(float f) {
    if constexpr (DT == 0) return f32_to_half_bits(f);
    else return f32_to_bf16_bits(f);
}
template <int NV, int VW, int G, int DT>
__device__ inline void row_store_h(u16* p, const RowSlice<NV, VW>& r, i64 s4, int j) {
    if constexpr (VW == 4) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const u32 lo = f32_to_h16_bits<DT>(r.v[k * 4 + 0]) | (static_cast<u32>(f32_to_h16_bits<DT>(r.v[k * 4 + 1])) << 16);
            const u32 hi = f32_to_h16_bits<DT>(r.v[k * 4 + 2]) | (static_cast<u32>(f32_to_h16_bits<DT>(r.v[k * 4 + 3])) << 16);
            *reinterpret_cast<uint2*>(p + (k * G + j) * 4) = make_uint2(lo, hi);
        }
    } else if constexpr (VW == 2) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            *reinterpret_cast<u32*>(p + (k * G + j) * 2) =
                f32_to_h16_bits<DT>(r.v[k * 2 + 0]) | (static_cast<u32>(f32_to_h16_bits<DT>(r.v[k * 2 + 1])) << 16);
    } else {
#pragma unroll
        for (int k = 0; k < NV; ++k) p[static_cast<i64>(k * G + j) * s4] = f32_to_h16_bits<DT>(r.v[k]);
    }
}

// Element loaders from global memory, widened to float (or int).
template <int DT>
__device__ inline float gload_f(const char* p, i64 e);
template <>
__device__ inline float gload_f<2>(const char* p, i64 e) { return reinterpret_cast<const float*>(p)[e]; }
template <>
__device__ inline float gload_f<0>(const char* p, i64 e) { return half_bits_to_f32(reinterpret_cast<const u16*>(p)[e]); }
template <>
__device__ inline float gload_f<1>(const char* p, i64 e) { return bf16_bits_to_f32(reinterpret_cast<const u16*>(p)[e]); }

template <int DT>
__device__ inline i64 gload_i(const char* p, i64 e);
template <>
__device__ inline i64 gload_i<6>(const char* p, i64 e) { return reinterpret_cast<const int*>(p)[e]; }
template <>
__device__ inline i64 gload_i<7>(const char* p, i64 e) { return reinterpret_cast<const i64*>(p)[e]; }

// Cooperative TLOAD of a rows x cols tile into LDS (float or int storage).
template <int DT, int ROWS, int COLS, int NT>
__device__ inline void tile_load_f(float* dst, const char* p, i64 s3, i64 s4) {
    for (int e = threadIdx.x; e < ROWS * COLS; e += NT) {
        const int r = e / COLS, c = e % COLS;
        dst[e] = gload_f<DT>(p, r * s3 + c * s4);
    }
}

template <int DT, int ROWS, int COLS, int NT>
__device__ inline void tile_load_i(i64* dst, const char* p, i64 s3, i64 s4) {
    for (int e = threadIdx.x; e < ROWS * COLS; e += NT) {
        const int r = e / COLS, c = e % COLS;
        dst[e] = gload_i<DT>(p, r * s3 + c * s4);
    }
}

// Cooperative TSTORE from LDS with the destination-dtype cast.
template <int DT, int ROWS, int COLS, int NT>
__device__ inline void tile_store_f(char* p, const float* src, i64 s3, i64 s4) {
    for (int e = threadIdx.x; e < ROWS * COLS; e += NT) {
        const int r = e / COLS, c = e % COLS;
        const i64 o = r * s3 + c * s4;
        if constexpr (DT == 2) reinterpret_cast<float*>(p)[o] = src[e];
        else if constexpr (DT == 0) reinterpret_cast<u16*>(p)[o] = f32_to_half_bits(src[e]);
        else reinterpret_cast<u16*>(p)[o] = f32_to_bf16_bits(src[e]);
    }
}

template <int DT, int ROWS, int COLS, int NT>
__device__ inline void tile_store_i(char* p, const i64* src, i64 s3, i64 s4) {
    for (int e = threadIdx.x; e < ROWS * COLS; e += NT) {
        const int r = e / COLS, c = e % COLS;
        const i64 o = r * s3 + c * s4;
        if constexpr (DT == 6) reinterpret_cast<int*>(p)[o] = static_cast<int>(src[e]);
        else reinterpret_cast<i64*>(p)[o] = src[e];
    }
}

// TSORT32 of one [1,32] row into [1,64] (score, index) pairs: descending by
// score, NaN after every number, equal scores (+0 and -0 included) in source
// order, i.e. a stable ascending sort of -score.  Each lane counts the
// elements ordered before its own and writes its pair at that rank; the
// index is the u32 index tile's element converted to float.
template <int NT>
__device__ inline void tsort32_rank(float* dst, const float* sc, const i64* ix) {
    for (int e = threadIdx.x; e < 32; e += NT) {
        const float x = sc[e];
        const bool xn = x != x;
        int rank = 0;
        for (int j = 0; j < 32; ++j) {
            const float y = sc[j];
            const bool yn = y != y;
            const bool before = xn ? (!yn || j < e) : (!yn && (y > x || (y == x && j < e)));
            rank += before ? 1 : 0;
        }
        dst[2 * rank] = x;
        dst[2 * rank + 1] = static_cast<float>(ix[e]);
    }
}

// ---------------------------------------------------------------------------
// GEMM blocks: C[BM,BN] (fp32) (+)= sum over K steps of A[BM,BK] x B[BK,BN]
// (bf16 or f16) on MFMA v_mfma_f32_32x32x16
// ---------------------------------------------------------------------------
//
// A workgroup of WM x WN waves owns a BM x BN block of C (one task's tile, or
// several neighbouring tasks' tiles merged by the host).  Wave (wm, wn) holds
// its (BM/WM) x (BN/WN) quadrant in registers as 32x32 MFMA blocks for the
// whole K loop; for an accumulating kernel the block starts from C.
//
// K steps go through two LDS stages filled by direct buffer->LDS loads (each
// wave instruction moves 1 KiB, no VGPR staging):
//   A stage [BM][BK]: 16-byte chunk c of row m lives at chunk c ^ swa(m), so
//     the 32 rows of an MFMA operand read hit distinct banks;
//   B stage [BK][BN] (k-major, as in memory): 32-byte segment g of row k lives
//     at g ^ swb(k); the MFMA B operand is read with ds_read_b64_tr_b16,
//     which transposes 16-bit elements across each group of 16 lanes.  A
//     transpose read serves 32 lanes per LDS cycle (256 bytes): lanes 0-15
//     read 4 rows of segment s, lanes 16-31 the same rows of segment s+1.
//     For rows of 256 bytes or more (BN >= 128) the banks repeat every 8
//     segments, and swb(k) = 2*(k & 3) puts the two 16-lane groups on
//     disjoint bank halves (s ^ {0,2,4,6} and (s+1) ^ {0,2,4,6}, s even);
//     with k & 3 the two groups hit the same 32 banks and each read takes
//     twice the cycles.  128-byte rows (BN = 64) alternate bank halves by
//     row parity, and k & 3 is conflict-free there.
// MFMA 32x32x16 lane l holds A row / B column (l % 32) with k = 8*(l/32)..+7;
// accumulator element e sits at row (e/4)*8 + (l/32)*4 + e%4, column l % 32.
// ds_read_b64_tr_b16: in each 16-lane group, lane l receives element (l % 4)
// of the 8-byte chunks addressed by lanes 16*(l/16) + (l%16)/4 + 4e, e = 0..3.

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t buf_rsrc;

template <bool F16>
__device__ inline f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

// Compile-time bool carried as a type (for generic lambdas under C++17).
template <bool B>
struct BoolC {
    static constexpr bool value = B;
};

__device__ inline int wave_index() { return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6)); }

// Raw dword buffer descriptor for p (no range check: offsets are bounded on the host).
__device__ inline u32x4 buffer_words(const void* p) {
    const u64 a = reinterpret_cast<u64>(p);
    u32x4 r;
    r.x = __builtin_amdgcn_readfirstlane(static_cast<u32>(a));
    r.y = __builtin_amdgcn_readfirstlane(static_cast<u32>(a >> 32) & 0xFFFFu);
    r.z = 0xFFFFFFFFu;
    r.w = 0x00020000u;
    return r;
}

__device__ inline u32 lds_address(const void* p) {
    return static_cast<u32>(reinterpret_cast<u64>((const __attribute__((address_space(3))) void*)p));
}

// 16 bytes per lane from global (descriptor + voff + soff) into LDS at
// lds_addr + 16*lane.  Written as inline asm so that the compiler's wait-count
// pass does not serialise later LDS reads behind it; callers wait with
// wait_vmcnt<0>() and a barrier before the stage is read.  M0 is restored.
__device__ inline void dma16(u32x4 rsrc, int voff, int soff, u32 lds_addr) {
    u32 saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %4\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen lds\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soff)), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
        : "memory");
}

// s_waitcnt on vmcnt only (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Position of workgroup w among n workgroups dispatched round-robin over the
// 8 XCDs, so that each XCD (own L2) gets a contiguous run of tiles.
__device__ inline i64 xcd_order(i64 w, i64 n) {
    const i64 q = n / 8, r = n % 8, x = w % 8, l = w / 8;
    return x * q + (x < r ? x : r) + l;
}

// NS: LDS stages in the ring (DMA issued NS-1 stages ahead); KSPLIT: LDS
// stages per task K step (a stage holds BK of the task's BK*KSPLIT columns).
template <int BM, int BN, int BK, int WM, int WN, bool F16, int NS = 2, int KSPLIT = 1>
struct GemmBlock {
    static constexpr int NW = WM * WN, NT = 64 * NW, KS = BK / 16;
    static constexpr int TM = BM / WM, TN = BN / WN, FI = TM / 32, FJ = TN / 32;
    static constexpr int CH = BK / 8;                  // 16-byte chunks per A row
    static constexpr int RPL = CH >= 8 ? 1 : 8 / CH;   // A rows per 128-byte LDS line
    static constexpr int SWM = (CH < 8 ? CH : 8) - 1;
    static constexpr int ARPB = 1024 / (2 * BK);       // A rows per 1 KiB load
    static constexpr int BCPR = BN / 8;                // 16-byte chunks per B row
    static constexpr int BRPB = 1024 / (2 * BN);       // B rows per 1 KiB load
    static constexpr int ABLK = BM * BK * 2 / 1024, BBLK = BK * BN * 2 / 1024;
    static constexpr int AQ = (ABLK + NW - 1) / NW, BQ = (BBLK + NW - 1) / NW;
    static constexpr int ASZ = BM * BK, STAGE = ASZ + BK * BN;
    static constexpr int kLdsElems = NS * STAGE;
    static constexpr int kStageOps = AQ + BQ;  // DMA instructions of one wave per stage
    static_assert(NS == 2 || (NS == 4 && AQ * NW == ABLK && BQ * NW == BBLK), "stage ring: every wave moves the same share");
    static_assert(TM % 32 == 0 && TN % 32 == 0 && BK % 16 == 0 && (BK & (BK - 1)) == 0, "GEMM block shape");
    static_assert(BN >= 64 && BN <= 512 && (BM * BK * 2) % 1024 == 0 && (BK * BN * 2) % 1024 == 0, "GEMM block shape");

    struct Acc {
        f32x16 v[FI][FJ];
    };
    struct Offs {
        int a[AQ];
        int b[BQ];
    };

    __device__ static int swa(int m) { return ((m / RPL) ^ (m >> 3)) & SWM; }
    __device__ static int swb(int k) { return BN >= 128 ? (k & 3) << 1 : k & 3; }

    // Per-lane byte offsets, from the block's A / B origin at the first K step,
    // of the chunks this wave moves (lda / ldb: row pitch in elements).
    __device__ static void offsets(Offs& o, int lda, int ldb) {
        const int lane = threadIdx.x & 63, w = wave_index();
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int m = (w * AQ + q) * ARPB + lane / CH, p = lane % CH;
            o.a[q] = (m * lda + ((p ^ swa(m)) << 3)) * 2;
        }
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int k = (w * BQ + q) * BRPB + lane / BCPR, p = lane % BCPR;
            const int c = (((p >> 1) ^ swb(k)) << 1) | (p & 1);
            o.b[q] = (k * ldb + c * 8) * 2;
        }
    }

    // Issues the direct loads of one K step (soa / sob: its uniform byte offsets).
    __device__ static void load(u16* stage, const Offs& o, u32x4 ra, int soa, u32x4 rb, int sob) {
        const int w = wave_index();
        const u32 base = lds_address(stage);
#pragma unroll
        for (int q = 0; q < AQ; ++q)
            if (AQ * NW == ABLK || w * AQ + q < ABLK) dma16(ra, o.a[q], soa, base + (w * AQ + q) * 1024);
#pragma unroll
        for (int q = 0; q < BQ; ++q)
            if (BQ * NW == BBLK || w * BQ + q < BBLK) dma16(rb, o.b[q], sob, base + ASZ * 2 + (w * BQ + q) * 1024);
    }

    __device__ static void mma(Acc& acc, const u16* stage) {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave / WN, wn = wave % WN;
        const int r = lane & 31, kc = lane >> 5;
        const int g = lane >> 4, a4 = lane & 3, e = (lane >> 2) & 3;
        const u16* as = stage + (wm * TM + r) * BK;
        const u16* bs = stage + ASZ;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            u32x4 af[FI], bf[FJ];
#pragma unroll
            for (int i = 0; i < FI; ++i)
                af[i] = *reinterpret_cast<const u32x4*>(as + i * 32 * BK + ((((kk >> 3) + kc) ^ swa(wm * TM + i * 32 + r)) << 3));
#pragma unroll
            for (int j = 0; j < FJ; ++j) {
                const int n = wn * TN + j * 32 + 16 * (g & 1) + 4 * a4;
                const int pn = (((n >> 4) ^ swb(e)) << 4) | (n & 15);
                const int k = kk + 8 * (g >> 1) + e;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(bs + k * BN + pn));
                const s16x4 hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(bs + (k + 4) * BN + pn));
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                bf[j] = u32x4{l2.x, l2.y, h2.x, h2.y};
            }
#pragma unroll
            for (int i = 0; i < FI; ++i)
#pragma unroll
                for (int j = 0; j < FJ; ++j) acc.v[i][j] = mfma_32x32x16<F16>(af[i], bf[j], acc.v[i][j]);
        }
    }

    // C block I/O in the accumulator layout (ldc: row pitch in elements).
    template <bool STORE>
    __device__ static void c_io(Acc& acc, buf_rsrc rc, int ldc) {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave / WN, wn = wave % WN;
        const int vc = ((lane >> 5) * 4 * ldc + (lane & 31)) * 4;
        const int so = (wm * TM * ldc + wn * TN) * 4;
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int s = so + (i * 32 + (e >> 2) * 8 + (e & 3)) * ldc * 4;
#pragma unroll
                for (int j = 0; j < FJ; ++j) {
                    if constexpr (STORE)
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc.v[i][j][e]), rc, vc + j * 128, s, 2);
                    else
                        acc.v[i][j][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, vc + j * 128, s, 2));
                }
            }
    }

    // Writes the block (plus C when ADD_C) in the accumulator layout, one
    // 32x32 accumulator at a time: the next accumulator's C is read while
    // this one is added and stored, and scheduling barriers keep the
    // accumulators apart so that few values sit in VGPRs at once.
    template <bool ADD_C>
    __device__ static void c_out(Acc& acc, buf_rsrc rc, int ldc) {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave / WN, wn = wave % WN;
        const int vc = ((lane >> 5) * 4 * ldc + (lane & 31)) * 4;
        const int so = (wm * TM * ldc + wn * TN) * 4;
        auto row = [&](int i, int e) { return so + (i * 32 + (e >> 2) * 8 + (e & 3)) * ldc * 4; };
        float t[2][16];
        auto fetch = [&](int n, float (&d)[16]) {
            const int i = n / FJ, j = n % FJ;
#pragma unroll
            for (int e = 0; e < 16; ++e) d[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rc, vc + j * 128, row(i, e), 2));
        };
        if constexpr (ADD_C) fetch(0, t[0]);
#pragma unroll
        for (int n = 0; n < FI * FJ; ++n) {
            const int i = n / FJ, j = n % FJ;
            if constexpr (ADD_C) {
                if (n + 1 < FI * FJ) fetch(n + 1, t[(n + 1) & 1]);
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float x = ADD_C ? t[n & 1][e] + acc.v[i][j][e] : acc.v[i][j][e];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rc, vc + j * 128, row(i, e), 2);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Waits until at most `ahead` stages of this wave's DMA are in flight.
    __device__ static void wait_stages(i64 ahead) {
        if constexpr (NS == 2) {
            wait_vmcnt<0>();
        } else {
            if (ahead >= 2) wait_vmcnt<2 * kStageOps>();
            else if (ahead == 1) wait_vmcnt<kStageOps>();
            else wait_vmcnt<0>();
        }
    }

    // Task K steps it0 .. iters-1, as (iters-it0)*KSPLIT LDS stages; off(it,
    // soa, sob) gives task step it's byte offsets from the step-0 origins pa /
    // pb.  The block sums A x B from zero; ACC: then adds C, as c + sum.
    template <bool ACC, class Off>
    __device__ static void run(u16* lds, const u16* pa, int lda, const u16* pb, int ldb, float* pc, int ldc, i64 it0,
                               i64 iters, Off off) {
        const u32x4 ra = buffer_words(pa), rb = buffer_words(pb);
        const buf_rsrc rc = __builtin_amdgcn_make_buffer_rsrc(pc, 0, -1, 0x00020000);
        Offs o;
        offsets(o, lda, ldb);
        Acc acc;
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int j = 0; j < FJ; ++j) acc.v[i][j] = f32x16{};
        const i64 nst = (iters - it0) * KSPLIT;
        auto issue = [&](i64 st) {
            int soa, sob;
            off(it0 + st / KSPLIT, soa, sob);
            const int h = static_cast<int>(st % KSPLIT);
            load(lds + static_cast<int>(st & (NS - 1)) * STAGE, o, ra, soa + h * BK * 2, rb, sob + h * BK * ldb * 2);
        };
        wait_vmcnt<0>();
        __syncthreads();  // the previous block's last stage reads are done
#pragma unroll
        for (int p = 0; p < NS - 1; ++p)
            if (p < nst) issue(p);
        for (i64 st = 0; st < nst; ++st) {
            const i64 ahead = nst - 1 - st < NS - 2 ? nst - 1 - st : NS - 2;
            wait_stages(ahead);
            __syncthreads();
            if (st + NS - 1 < nst) issue(st + NS - 1);
            mma(acc, lds + static_cast<int>(st & (NS - 1)) * STAGE);
        }
        c_out<ACC>(acc, rc, ldc);
    }
};

// ---------------------------------------------------------------------------
// f32 GEMM block: f32 A and B on v_mfma_f32_32x32x2_f32
// ---------------------------------------------------------------------------
//
// The block structure of GemmBlock (NS-stage LDS ring filled by direct
// buffer->LDS loads, waves WM x WN over the C block, 32x32 accumulators in
// the same layout, so the C epilogue is GemmBlock's) with 4-byte elements.
// A stage holds A as [BM][BK] and B as [BK][BN], row-major, in 16-byte
// chunks: A's chunks XOR-swizzled by row as in GemmBlock (every lane of a
// half-wave reads the same chunk of 32 rows), B's 128-byte halves swapped on
// rows whose bit 2 is set (the two half-waves read rows k and k+4 of the
// same columns).
//
// v_mfma_f32_32x32x2_f32 takes one A and one B value per lane: lane l
// supplies A[i = l%32][k = l/32] and B[k = l/32][j = l%32].  The K order of
// a product is free, so for the 8 columns kk..kk+7 half-wave h reads
// A[m][kk+4h .. +3] as one 16-byte chunk, and MFMA q (0..3) pairs column
// kk+q (half 0) with kk+4+q (half 1).
template <int BM, int BN, int BK, int WM, int WN, int NS = 2, int KSPLIT = 1>
struct GemmF32 {
    static constexpr int NW = WM * WN, NT = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN, FI = TM / 32, FJ = TN / 32;
    static constexpr int CH = BK / 4;                  // 16-byte chunks per A row
    static constexpr int RPL = CH >= 8 ? 1 : 8 / CH;   // A rows per 128-byte LDS line
    static constexpr int SWM = (CH < 8 ? CH : 8) - 1;
    static constexpr int ARPB = 1024 / (4 * BK);       // A rows per 1 KiB load
    static constexpr int BCPR = BN / 4;                // 16-byte chunks per B row
    static constexpr int BRPB = 1024 / (4 * BN);       // B rows per 1 KiB load
    static constexpr int ABLK = BM * BK * 4 / 1024, BBLK = BK * BN * 4 / 1024;
    static constexpr int AQ = (ABLK + NW - 1) / NW, BQ = (BBLK + NW - 1) / NW;
    static constexpr int ASZ = BM * BK, STAGE = ASZ + BK * BN;  // floats
    static constexpr int kLdsElems = NS * STAGE * 2;            // 16-bit units (the kernel's LDS array)
    static_assert(NS == 2, "two-stage ring");
    static_assert(TM % 32 == 0 && TN % 32 == 0 && (BK == 16 || BK == 32), "f32 GEMM block shape");
    static_assert(BN >= 64 && BN <= 256 && (BM * BK * 4) % 1024 == 0 && (BK * BN * 4) % 1024 == 0, "f32 GEMM block shape");
    typedef GemmBlock<BM, BN, 16, WM, WN, false> Out;  // the C epilogue (same accumulator layout)
    typedef typename Out::Acc Acc;

    struct Offs {
        int a[AQ];
        int b[BQ];
    };
    __device__ static int swa(int m) { return ((m / RPL) ^ (m >> 3)) & SWM; }
    __device__ static int swb(int k) { return ((k >> 2) & 1) << 3; }

    // Per-lane byte offsets, from the block's A / B origin at the first K
    // step, of the chunks this wave moves (lda / ldb: row pitch in elements).
    __device__ static void offsets(Offs& o, int lda, int ldb) {
        const int lane = threadIdx.x & 63, w = wave_index();
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int m = (w * AQ + q) * ARPB + lane / CH, p = lane % CH;
            o.a[q] = (m * lda + ((p ^ swa(m)) << 2)) * 4;
        }
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int k = (w * BQ + q) * BRPB + lane / BCPR, p = lane % BCPR;
            o.b[q] = (k * ldb + ((p ^ swb(k)) << 2)) * 4;
        }
    }

    __device__ static void load(float* stage, const Offs& o, u32x4 ra, int soa, u32x4 rb, int sob) {
        const int w = wave_index();
        const u32 base = lds_address(stage);
#pragma unroll
        for (int q = 0; q < AQ; ++q)
            if (AQ * NW == ABLK || w * AQ + q < ABLK) dma16(ra, o.a[q], soa, base + (w * AQ + q) * 1024);
#pragma unroll
        for (int q = 0; q < BQ; ++q)
            if (BQ * NW == BBLK || w * BQ + q < BBLK) dma16(rb, o.b[q], sob, base + ASZ * 4 + (w * BQ + q) * 1024);
    }

    __device__ static void mma(Acc& acc, const float* stage) {
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave / WN, wn = wave % WN;
        const int r = lane & 31, h = lane >> 5;
        const float* as = stage + (wm * TM + r) * BK;
        const float* bs = stage + ASZ;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 8) {
            f32x4v_t af[FI];
#pragma unroll
            for (int i = 0; i < FI; ++i)
                af[i] = *reinterpret_cast<const f32x4v_t*>(as + i * 32 * BK + ((((kk >> 2) + h) ^ swa(wm * TM + i * 32 + r)) << 2));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int k = kk + 4 * h + q;
                float bf[FJ];
#pragma unroll
                for (int j = 0; j < FJ; ++j) {
                    const int n = wn * TN + j * 32 + r;
                    bf[j] = bs[k * BN + ((((n >> 2) ^ swb(k)) << 2) | (n & 3))];
                }
#pragma unroll
                for (int i = 0; i < FI; ++i)
#pragma unroll
                    for (int j = 0; j < FJ; ++j) acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][q], bf[j], acc.v[i][j], 0, 0, 0);
            }
        }
    }

    // Task K steps it0 .. iters-1, as (iters-it0)*KSPLIT LDS stages (see
    // GemmBlock::run); pa / pb point at f32 data.
    template <bool ACC, class Off>
    __device__ static void run(u16* lds, const u16* pa, int lda, const u16* pb, int ldb, float* pc, int ldc, i64 it0,
                               i64 iters, Off off) {
        float* ring = reinterpret_cast<float*>(lds);
        const u32x4 ra = buffer_words(pa), rb = buffer_words(pb);
        const buf_rsrc rc = __builtin_amdgcn_make_buffer_rsrc(pc, 0, -1, 0x00020000);
        Offs o;
        offsets(o, lda, ldb);
        Acc acc;
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int j = 0; j < FJ; ++j) acc.v[i][j] = f32x16{};
        const i64 nst = (iters - it0) * KSPLIT;
        auto issue = [&](i64 st) {
            int soa, sob;
            off(it0 + st / KSPLIT, soa, sob);
            const int hs = static_cast<int>(st % KSPLIT);
            load(ring + static_cast<int>(st & 1) * STAGE, o, ra, soa + hs * BK * 4, rb, sob + hs * BK * ldb * 4);
        };
        wait_vmcnt<0>();
        __syncthreads();  // the previous block's last stage reads are done
        if (nst > 0) issue(0);
        for (i64 st = 0; st < nst; ++st) {
            wait_vmcnt<0>();
            __syncthreads();
            if (st + 1 < nst) issue(st + 1);
            mma(acc, ring + static_cast<int>(st & 1) * STAGE);
        }
        Out::template c_out<ACC>(acc, rc, ldc);
    }
};

// ---------------------------------------------------------------------------
// Matmul op of a tile program on the matrix cores
// ---------------------------------------------------------------------------
//
// c[M][N] = a @ b for fp32 tile values (a(i, q), b(q, j): the operand
// elements, from an LDS tile or a global param), M and N multiples of 32,
// K even and at most 32 or a multiple of 32, on v_mfma_f32_32x32x2_f32.
// Wave w of NT/64 computes the 32x32 output blocks w, w + NW, ...  Lane l
// supplies A[i0 + l%32][q + l/32] and B[q + l/32][j0 + l%32]; an LDS tile
// of A is row-major with a row pitch of K floats, so the 32 rows one MFMA
// reads at one column would share a bank.  Each 32-column slice of the
// block's 32 A rows is therefore copied first into the wave's scratch with
// a row pitch of 33 floats (32 distinct banks per column).  Products are
// exact in the MFMA; the sum runs in its order, not the scalar loop's.
constexpr int kTileMmaPitch = 33;
__device__ inline void wave_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
template <int M, int K, int N, int NT, class FA, class FB>
__device__ inline void tile_mma(FA a, FB b, float* c, float* scratch) {
    static_assert(M % 32 == 0 && N % 32 == 0 && K % 2 == 0 && (K <= 32 || K % 32 == 0) && NT % 64 == 0, "tile_mma shape");
    constexpr int NW = NT / 64, BJ = N / 32, NB = (M / 32) * BJ, KC = K < 32 ? K : 32;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r = lane & 31, h = lane >> 5;
    float* s = scratch + w * 32 * kTileMmaPitch;
    for (int blk = w; blk < NB; blk += NW) {
        const int i0 = (blk / BJ) * 32, j0 = (blk % BJ) * 32;
        f32x16 acc = {};
        for (int k0 = 0; k0 < K; k0 += KC) {
            // Lanes exchange the slice through LDS, whose operations a wave
            // performs in order; the wave barriers (wave-scope fences around
            // the wave barrier) keep the compiler from moving the copy across
            // the previous slice's reads or this slice's.
            wave_lds_barrier();
#pragma unroll
            for (int e = lane; e < 32 * KC; e += 64) s[(e / KC) * kTileMmaPitch + e % KC] = a(i0 + e / KC, k0 + e % KC);
            wave_lds_barrier();
#pragma unroll 8
            for (int q = 0; q < KC; q += 2)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(s[r * kTileMmaPitch + q + h], b(k0 + q + h, j0 + r), acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) c[(i0 + 8 * (e >> 2) + 4 * h + (e & 3)) * N + j0 + r] = acc[e];
    }
}

// The same for M and N multiples of 16 (K a multiple of 4, at most 32 or a
// multiple of 32) on v_mfma_f32_16x16x4_f32: 16x16 output blocks, lane l
// supplying A[i0 + l%16][q + l/16] (from the wave's scratch copy of the
// block's 16 A rows) and B[q + l/16][j0 + l%16].
template <int M, int K, int N, int NT, class FA, class FB>
__device__ inline void tile_mma16(FA a, FB b, float* c, float* scratch) {
    static_assert(M % 16 == 0 && N % 16 == 0 && K % 4 == 0 && (K <= 32 || K % 32 == 0) && NT % 64 == 0, "tile_mma16 shape");
    constexpr int NW = NT / 64, BJ = N / 16, NB = (M / 16) * BJ, KC = K < 32 ? K : 32;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, r = lane & 15, h = lane >> 4;
    float* s = scratch + w * 32 * kTileMmaPitch;
    for (int blk = w; blk < NB; blk += NW) {
        const int i0 = (blk / BJ) * 16, j0 = (blk % BJ) * 16;
        f32x4v_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k0 = 0; k0 < K; k0 += KC) {
            wave_lds_barrier();
#pragma unroll
            for (int e = lane; e < 16 * KC; e += 64) s[(e / KC) * kTileMmaPitch + e % KC] = a(i0 + e / KC, k0 + e % KC);
            wave_lds_barrier();
#pragma unroll 8
            for (int q = 0; q < KC; q += 4)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s[r * kTileMmaPitch + q + h], b(k0 + q + h, j0 + r), acc, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) c[(i0 + 4 * h + e) * N + j0 + r] = acc[e];
    }
}

// ---------------------------------------------------------------------------
// Ping-pong GEMM block: 256x256 C block, 8 waves in two groups of four
// ---------------------------------------------------------------------------
//
// Same LDS layout, operand reads and accumulator layout as
// GemmBlock<256, 256, BK, 2, 4>: wave w owns rows (w/4)*128..+127 and
// columns (w%4)*64..+63; group 0 (waves 0-3) and group 1 (waves 4-7) put one
// wave on each SIMD.  The groups take turns between slots separated by
// workgroup barriers: while one group runs the 32 (BK = 64) MFMAs of a stage
// from registers, the other reads the next stage's fragments from LDS, so
// each SIMD's matrix pipe is fed by one wave while its other wave does the
// memory work.  Group 1 runs one slot behind group 0:
//   slot 2j:   group 0 reads stage j (and issues the DMA of stage j+NS-1),
//              group 1 computes stage j-1;
//   slot 2j+1: group 0 computes stage j, group 1 reads stage j.
// Stage j's buffer is last read in slot 2j+1, so its reuse for stage j+NS is
// issued in slot 2j+2 and has 2*NS-2 slots to land.  Group 0 issues all
// DMA; wave 0 also touches the A / B lines of stage j+PF (its share of the
// lines that the blocks sharing those panels will load) so that they are in
// L2 when their DMA is issued.  Every wave executes the same barriers.

// Workgroup barrier that the compiler schedules nothing across.
__device__ inline void block_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

__device__ inline void wait_lgkm0() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// 4 bytes per lane from global into LDS at lds_addr + 4*lane; used to pull
// lines into L2 ahead of their DMA (the LDS bytes are scratch).
__device__ inline void dma4(u32x4 rsrc, int voff, int soff, u32 lds_addr) {
    u32 saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %4\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %1, %2, %3 offen lds\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soff)), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
        : "memory");
}

template <int BK, bool F16>
struct GemmPingPong {
    typedef GemmBlock<256, 256, BK, 2, 4, F16, 2, 1> GB;
    static constexpr int NS = BK == 64 ? 2 : 4;        // LDS stages (128 KiB)
    static constexpr int PF = 3;                       // L2 touch distance in stages
    static constexpr int WN = 4, TM = 128, TN = 64, FI = 4, FJ = 2, KS = BK / 16;
    static constexpr int CH = BK / 8, ARPB = 1024 / (2 * BK), BCPR = 32, BRPB = 2;
    static constexpr int ABLK = 256 * BK * 2 / 1024, BBLK = BK * 256 * 2 / 1024;
    static constexpr int NL = 4, AQ = ABLK / NL, BQ = BBLK / NL;  // group 0 loads
    static constexpr int ASZ = 256 * BK, STAGE = ASZ + BK * 256;
    static constexpr int kScratch = 128;               // u16 elements after the stages
    static constexpr int kLdsElems = NS * STAGE + kScratch;
    static constexpr int kStageOps = AQ + BQ;
    static_assert(BK == 64 || BK == 32, "ping-pong K step");
    static_assert(AQ * NL == ABLK && BQ * NL == BBLK && (NS - 2) * kStageOps <= 63, "ping-pong loads");

    struct Frag {
        u32x4 a[KS][FI];
        u32x4 b[KS][FJ];
    };
    typedef typename GB::Acc Acc;

    // DMA lane offsets of loader wave w (0..3) for its first A / B chunk.
    // With row pitches that are multiples of 64 elements (checked on the
    // host), chunk q of A sits at va with its 16-byte column bits flipped by
    // q (BK = 64) or by bit 1 of q (BK = 32).  Chunk q of B (K rows 2q, 2q+1
    // after the wave's first) uses vb[q & 1]: the rows' swizzle GB::swb
    // depends on k & 3, which moves by 2 with each chunk.  The row steps
    // q*ARPB / q*BRPB go into the uniform offset.
    __device__ static void offsets(int& va, int (&vb)[2], int w, int lda, int ldb) {
        const int lane = threadIdx.x & 63;
        const int m = w * AQ * ARPB + lane / CH, p = lane % CH;
        va = (m * lda + ((p ^ GB::swa(m)) << 3)) * 2;
        const int k = w * BQ * BRPB + lane / BCPR, pb = lane % BCPR;
#pragma unroll
        for (int h = 0; h < 2; ++h) vb[h] = (k * ldb + (((((pb >> 1) ^ GB::swb(k + 2 * h)) << 1) | (pb & 1)) * 8)) * 2;
    }
    __device__ static int a_voff(int va, int q) { return BK == 64 ? va ^ (q << 4) : va ^ ((q & 1) << 5); }

    __device__ static void load(u16* stage, int w, int va, const int (&vb)[2], u32x4 ra, int soa, u32x4 rb, int sob, int lda, int ldb) {
        const u32 base = lds_address(stage);
#pragma unroll
        for (int q = 0; q < AQ; ++q) dma16(ra, a_voff(va, q), soa + q * ARPB * lda * 2, base + (w * AQ + q) * 1024);
#pragma unroll
        for (int q = 0; q < BQ; ++q) dma16(rb, vb[q & 1], sob + q * BRPB * ldb * 2, base + ASZ * 2 + (w * BQ + q) * 1024);
    }

    struct NoDma {
        __device__ void operator()(int) const {}
    };

    // All fragments of one stage (the address math of GemmBlock::mma); dma(k)
    // is issued after the wave's (4k+4)-th LDS read, k = 0 .. KS*(FI+2*FJ)/4-1.
    template <class Dma = NoDma>
    __device__ static void read(Frag& f, const u16* stage, int wm, int wn, Dma dma = Dma()) {
        const int lane = threadIdx.x & 63;
        const int r = lane & 31, kc = lane >> 5;
        const int g = lane >> 4, a4 = lane & 3, e = (lane >> 2) & 3;
        const u16* as = stage + (wm * TM + r) * BK;
        const u16* bs = stage + ASZ;
        int nl = 0;
        auto tick = [&]() {
            if (++nl % 4 == 0) {
                __builtin_amdgcn_sched_barrier(0);
                dma(nl / 4 - 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int kk = s * 16;
#pragma unroll
            for (int i = 0; i < FI; ++i) {
                f.a[s][i] = *reinterpret_cast<const u32x4*>(as + i * 32 * BK + ((((kk >> 3) + kc) ^ GB::swa(wm * TM + i * 32 + r)) << 3));
                tick();
            }
#pragma unroll
            for (int j = 0; j < FJ; ++j) {
                const int n = wn * TN + j * 32 + 16 * (g & 1) + 4 * a4;
                const int pn = (((n >> 4) ^ GB::swb(e)) << 4) | (n & 15);
                const int k = kk + 8 * (g >> 1) + e;
                const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(bs + k * 256 + pn));
                tick();
                const s16x4 hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(bs + (k + 4) * 256 + pn));
                tick();
                const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                f.b[s][j] = u32x4{l2.x, l2.y, h2.x, h2.y};
            }
        }
    }

    // BK = 64: A chunk c of a stage (rows 8c..8c+7) and B chunk c (K rows 2c,
    // 2c+1), from the lane offsets va0 / vb0 of chunk 0 (offsets(.., 0, ..)):
    // chunk c flips A's 16-byte column bits by c & 7 and takes B's offset
    // for its parity.
    __device__ static void achunk(u32 base, int c, int va0, u32x4 ra, int soa, int lda) {
        dma16(ra, va0 ^ ((c & 7) << 4), soa + c * ARPB * lda * 2, base + c * 1024);
    }
    __device__ static void bchunk(u32 base, int c, const int (&vb0)[2], u32x4 rb, int sob, int ldb) {
        dma16(rb, vb0[c & 1], sob + c * BRPB * ldb * 2, base + ASZ * 2 + c * 1024);
    }

    __device__ static void mma(Acc& acc, const Frag& f) {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int i = 0; i < FI; ++i)
#pragma unroll
                for (int j = 0; j < FJ; ++j) acc.v[i][j] = mfma_32x32x16<F16>(f.a[s][i], f.b[s][j], acc.v[i][j]);
    }

    // Waits until at most `pending` later stages of this wave's DMA are in flight.
    __device__ static void wait_pending(int pending) {
        if constexpr (NS == 2) {
            wait_vmcnt<0>();
        } else {
            if (pending >= 2) wait_vmcnt<2 * kStageOps>();
            else if (pending == 1) wait_vmcnt<kStageOps>();
            else wait_vmcnt<0>();
        }
    }

    // C block (plus C when ACC) through LDS, with 128-bit global accesses.
    // The accumulator layout gives each lane 4 rows of one column, so moving
    // C straight from it takes 32-bit accesses, and the texture path
    // addresses 4 lanes per clock: 16 B/clk per CU against 64 B/clk for
    // 16-byte lanes.  Instead each wave writes one 32-row slab of its
    // quadrant (accumulators (i, 0) and (i, 1)) into a private LDS region in
    // row-major order (32-bit writes; the row pitch of 72 floats puts the two
    // 32-lane halves of a write on disjoint banks), reads it back as 16-byte
    // pieces (lane l: row 4q + l/16, columns 4*(l%16)..+3) and stores them
    // with buffer_store_dwordx4; for ACC the slab's C is read ahead with
    // buffer_load_dwordx4, one slab in advance, and added as c + sum.  A
    // wave's LDS operations complete in order, so one region serves all four
    // slabs.  The stage buffers are free here: group 0 runs this after group
    // 1's last stage read (the barrier before group 0's last compute slot
    // waits for it), group 1 after the barrier that ends group 0's epilogue.
    template <bool ACC>
    __device__ static void c_out(Acc& acc, u16* lds, buf_rsrc rc, int ldc) {
        constexpr int P = 72;
        const int lane = threadIdx.x & 63, wave = wave_index();
        const int wm = wave / WN, wn = wave % WN;
        float* reg = reinterpret_cast<float*>(lds) + (wave & 3) * 32 * P;
        const int so = (wm * TM * ldc + wn * TN) * 4;
        const int vg = ((lane >> 4) * ldc + (lane & 15) * 4) * 4;
        const int wr = (lane >> 5) * 4 * P + (lane & 31), rd = (lane >> 4) * P + (lane & 15) * 4;
        f32x4v c[2][8];
        auto fetch = [&](int i, f32x4v(&d)[8]) {
#pragma unroll
            for (int q = 0; q < 8; ++q)
                d[q] = __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(rc, vg, so + (i * 32 + q * 4) * ldc * 4, 2));
        };
        if constexpr (ACC) fetch(0, c[0]);
#pragma unroll
        for (int i = 0; i < FI; ++i) {
            if constexpr (ACC) {
                if (i + 1 < FI) fetch(i + 1, c[(i + 1) & 1]);
            }
#pragma unroll
            for (int j = 0; j < FJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) reg[wr + ((e >> 2) * 8 + (e & 3)) * P + j * 32] = acc.v[i][j][e];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                f32x4v x = *reinterpret_cast<const f32x4v*>(reg + rd + q * 4 * P);
                if constexpr (ACC) x = c[i & 1][q] + x;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rc, vg, so + (i * 32 + q * 4) * ldc * 4, 2);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }

    // BK = 64 schedule.  A wave's DMA instructions block its issue until the
    // texture path drains them (64 B/clk per CU), so a read slot that also
    // issues a whole 64 KiB stage outlasts the compute slot beside it.  The
    // stage DMA is therefore split by consumer, 32 KiB per read slot, and
    // interleaved with that slot's LDS reads:
    //   group 0 (A rows 0-127), slot 2j: B of stage j+1 (8 chunks per wave);
    //   group 1 (A rows 128-255), slot 2j+1: A rows 128-255 of stage j+1 and
    //     A rows 0-127 of stage j+2 (4 + 4 chunks per wave).
    // Buffer reuse: B of stage j+1 replaces B of stage j-1 (read in slots
    // 2j-2 / 2j-1); A rows 128-255 of stage j+1 replace those of stage j-1
    // (read by group 1 in slot 2j-1); A rows 0-127 of stage j+2 replace those
    // of stage j (read by group 0 in slot 2j).  Waits: group 0 waits for its
    // B of stage j+1 at the end of slot 2j+1; group 1 waits for A rows 0-127
    // of stage j+1 at the end of slot 2j+1 and for rows 128-255 of stage j+1
    // at the end of slot 2j+2, each before the barrier that precedes the read.
    template <bool ACC, class Off>
    __device__ static void run_split(u16* lds, const u16* pa, int lda, const u16* pb, int ldb, float* pc, int ldc, i64 it0,
                                     i64 iters, Off off, int pfa_row, int pfb_row) {
        const int w = wave_index(), grp = w >> 2, wq = w & 3, wm = w / WN, wn = w % WN;
        const int lane = threadIdx.x & 63;
        const u32x4 ra = buffer_words(pa), rb = buffer_words(pb);
        const buf_rsrc rc = __builtin_amdgcn_make_buffer_rsrc(pc, 0, -1, 0x00020000);
        const int nst = static_cast<int>(iters - it0);
        const u32 scratch = lds_address(lds + NS * STAGE);
        int va0, vb0[2];
        offsets(va0, vb0, 0, lda, ldb);
        const int pfa_v = (pfa_row + (lane & 31)) * lda * 2, pfb_v = ((pfb_row + (lane >> 2)) * ldb + (lane & 3) * 64) * 2;
        const bool touch = w == 0 && pfa_row >= 0 && pfb_row >= 0;
        Acc acc;
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int j = 0; j < FJ; ++j) acc.v[i][j] = f32x16{};
        Frag f;
        auto sbase = [&](int st) { return lds_address(lds + (st % NS) * STAGE); };
        // group 0 wave wq: B chunks 8wq..8wq+7 of stage st
        auto issue_b = [&](int st, int k) {
            int soa, sob;
            off(it0 + st, soa, sob);
            bchunk(sbase(st), wq * 8 + k, vb0, rb, sob, ldb);
        };
        // group 1 wave wq: A chunk 16*half + 4wq + k of stage st (half 0: rows 0-127, 1: rows 128-255)
        auto issue_a = [&](int st, int half, int k) {
            int soa, sob;
            off(it0 + st, soa, sob);
            achunk(sbase(st), half * 16 + wq * 4 + k, va0, ra, soa, lda);
        };
        wait_vmcnt<0>();
        block_barrier();  // the previous block's last stage reads are done
        // stage 0, and A rows 0-127 of stage 1
        if (grp == 0) {
            for (int k = 0; k < 8; ++k) issue_b(0, k);
        } else {
            for (int k = 0; k < 4; ++k) issue_a(0, 0, k);
            for (int k = 0; k < 4; ++k) issue_a(0, 1, k);
            if (nst > 1)
                for (int k = 0; k < 4; ++k) issue_a(1, 0, k);
        }
        wait_vmcnt<0>();
        block_barrier();
        if (grp == 1) block_barrier();  // group 1 runs one slot behind
        // One iteration (stage j) of group G.  H1 / H2: stages j+1 / j+2
        // exist (their DMA is issued here); T: wave 0's L2 touches of stage
        // j+PF.  The conditions are compile-time: a branch on them inside
        // the loop delays the computing group's barrier arrival and the
        // reading group's reads (measured without DMA: 36.7 cycles per MFMA
        // with the branches against 34.6 without, 32.4 for the bare
        // alternation).
        auto step = [&](auto g_, auto h1_, auto h2_, auto t_, int j) {
            constexpr bool G1 = decltype(g_)::value, H1 = decltype(h1_)::value, H2 = decltype(h2_)::value;
            constexpr bool T = decltype(t_)::value;
            if constexpr (!G1) {
                read(f, lds + (j % NS) * STAGE, wm, wn, [&](int k) {
                    if constexpr (H1) {
                        if (k < 8) issue_b(j + 1, k);
                    }
                });
                if constexpr (T) {
                    int soa, sob;
                    off(it0 + j + PF, soa, sob);
                    dma4(ra, pfa_v, soa, scratch);
                    dma4(rb, pfb_v, sob, scratch);
                }
            } else {
                read(f, lds + (j % NS) * STAGE, wm, wn, [&](int k) {
                    if (k < 4) {
                        if constexpr (H1) issue_a(j + 1, 1, k);
                    } else if (k < 8) {
                        if constexpr (H2) issue_a(j + 2, 0, k - 4);
                    }
                });
                // A rows 0-127 of stage j+1 (issued in this group's previous read slot) have landed
                if constexpr (H1 && H2) wait_vmcnt<8>();
                else if constexpr (H1 || H2) wait_vmcnt<4>();
                else wait_vmcnt<0>();
            }
            wait_lgkm0();
            block_barrier();
            mma(acc, f);
            if constexpr (!G1) {
                // own B of stage j+1 landed (wave 0's two touches may stay in flight)
                if constexpr (T) wait_vmcnt<2>();
                else wait_vmcnt<0>();
            } else {
                // own A rows 128-255 of stage j+1 landed (rows 0-127 of stage j+2 may stay in flight)
                if constexpr (H2) wait_vmcnt<4>();
                else wait_vmcnt<0>();
            }
            block_barrier();
        };
        // Stages 0 .. nst-PF-1 in the steady loop (every condition holds),
        // then the last three with their own conditions.
        static_assert(PF == 3, "the peeled tail covers the stages without L2 touches");
        auto run_group = [&](auto g_, auto t_) {
            int j = 0;
            for (; j + PF < nst; ++j) step(g_, BoolC<true>{}, BoolC<true>{}, t_, j);
            if (j + 2 < nst) step(g_, BoolC<true>{}, BoolC<true>{}, BoolC<false>{}, j++);
            if (j + 1 < nst) step(g_, BoolC<true>{}, BoolC<false>{}, BoolC<false>{}, j++);
            if (j < nst) step(g_, BoolC<false>{}, BoolC<false>{}, BoolC<false>{}, j);
        };
        if (grp == 0) {
            if (touch) run_group(BoolC<false>{}, BoolC<true>{});
            else run_group(BoolC<false>{}, BoolC<false>{});
        } else {
            run_group(BoolC<true>{}, BoolC<false>{});
        }
        wait_vmcnt<0>();
        c_out<ACC>(acc, lds, rc, ldc);
        if (grp == 0) block_barrier();
    }

    // Task K steps it0 .. iters-1 (off(it, soa, sob): step it's byte offsets
    // from the step-0 origins pa / pb).  The block sums A x B from zero; ACC:
    // then adds C, as c + sum.  pfa_row / pfb_row (< 0: no L2 touches): the
    // A rows pfa_row..+31 and B rows pfb_row..+15 of each stage that wave 0
    // pulls into L2 PF stages ahead.
    template <bool ACC, class Off>
    __device__ static void run(u16* lds, const u16* pa, int lda, const u16* pb, int ldb, float* pc, int ldc, i64 it0, i64 iters,
                               Off off, int pfa_row, int pfb_row) {
        if constexpr (BK == 64) {
            run_split<ACC>(lds, pa, lda, pb, ldb, pc, ldc, it0, iters, off, pfa_row, pfb_row);
            return;
        }
        const int w = wave_index(), grp = w >> 2, wm = w / WN, wn = w % WN;
        const int lane = threadIdx.x & 63;
        const u32x4 ra = buffer_words(pa), rb = buffer_words(pb);
        const buf_rsrc rc = __builtin_amdgcn_make_buffer_rsrc(pc, 0, -1, 0x00020000);
        const int nst = static_cast<int>(iters - it0);
        const u32 scratch = lds_address(lds + NS * STAGE);
        int va, vb[2];
        offsets(va, vb, w & 3, lda, ldb);
        const int pfa_v = (pfa_row + (lane & 31)) * lda * 2, pfb_v = ((pfb_row + (lane >> 2)) * ldb + (lane & 3) * 64) * 2;
        const bool touch = w == 0 && pfa_row >= 0 && pfb_row >= 0;
        Acc acc;
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
            for (int j = 0; j < FJ; ++j) acc.v[i][j] = f32x16{};
        Frag f;
        auto issue = [&](int st) {
            int soa, sob;
            off(it0 + st, soa, sob);
            load(lds + (st % NS) * STAGE, w & 3, va, vb, ra, soa, rb, sob, lda, ldb);
        };
        wait_vmcnt<0>();
        block_barrier();  // the previous block's last stage reads are done
        if (grp == 0) {
            for (int p = 0; p < NS - 1; ++p)
                if (p < nst) issue(p);
            wait_pending(nst - 1 < NS - 2 ? nst - 1 : NS - 2);
        }
        block_barrier();
        if (grp == 1) block_barrier();  // group 1 runs one slot behind
        for (int j = 0; j < nst; ++j) {
            if (grp == 0 && j + NS - 1 < nst) issue(j + NS - 1);
            const bool t = touch && j + PF < nst;
            if (t) {
                int soa, sob;
                off(it0 + j + PF, soa, sob);
                dma4(ra, pfa_v, soa, scratch);
                dma4(rb, pfb_v, sob, scratch);
            }
            read(f, lds + (j % NS) * STAGE, wm, wn);
            wait_lgkm0();
            block_barrier();
            mma(acc, f);
            if (grp == 0 && j + 1 < nst) {
                // wave 0's two touches of this iteration may stay in flight
                if (NS == 2 && t) wait_vmcnt<2>();
                else wait_pending((j + NS - 1 < nst ? j + NS - 1 : nst - 1) - (j + 1));
            }
            block_barrier();
        }
        c_out<ACC>(acc, lds, rc, ldc);
        if (grp == 0) block_barrier();
    }
};

// ---------------------------------------------------------------------------
// Decode: online softmax over 16-token pages (flashinfer_decode pattern)
// ---------------------------------------------------------------------------
//
// The pages of one unit (sequence b, KV group g) are folded by one or more
// waves (DecodeSplit); each wave folds its pages into a partial (m, l, o) for
// the unit's G query rows, starting from (-inf, 0, 0), and DecodeCombine folds
// the unit's partials in page order into the accumulators.  Per page:
//  * scores transposed, S^T = K q^T, on v_mfma_f32_16x16x32 (one per 32-wide
//    head-dim slice): A = the K page (lane l: token l%16, head dims
//    8*(l/16)..+7 of the slice), B = q^T (lane l: query row l%16, zero for
//    rows >= G); lane l then holds tokens 4*(l/16)..+3 of query row l%16,
//    which is the A operand layout of p @ v, so p never leaves the lane;
//  * a query row's max and sum: over the lane's 4 tokens, then over the 4
//    lanes l%16 + 16*i with two lane swaps (v_permlane32_swap,
//    v_permlane16_swap), so every lane of the row ends with the result;
//  * p @ v on the matrix cores (v_mfma_f32_16x16x16, p split into two
//    16-bit parts), lane l supplying tokens 4*(l/16)..+3 of every page for
//    head dims (D/16)*(l%16)+e and accumulating query rows 4*(l/16)..+3.


template <bool F16>
__device__ inline f32x4v_t mfma_16x16x32(u32x4 a, u32x4 b, f32x4v_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

// Reduction over the lanes l%16 + 16*i (i = 0..3), the four lanes that hold
// one query row of the transposed scores: a swap of the wave's halves, then
// of its odd and even 16-lane rows.  Every lane ends with the result, and
// computes it with the same operand order (lower lane's value first).
template <class Op>
__device__ inline float cross4_reduce(float x, Op op) {
    const u32 b = __float_as_uint(x);
    const auto h = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    x = op(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const u32 c = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane16_swap(c, c, false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Partials pass between waves of different XCDs (each XCD has its own L2).
// They are written and read as relaxed agent-scope atomics: global_store /
// global_load with sc1, the agent-coherent form of the LLVM AMDGPU memory
// model for gfx942/gfx950, so no L2 write-back (buffer_wbl2) or invalidate
// (buffer_inv) is needed for them.  What the agent-scope release sequence
// adds beyond that, s_waitcnt vmcnt(0) before the arrival RMW, publish()
// does directly (with compiler barriers on both sides) or the deferred
// arrival of DecodeStream gets from in-order completion: a wave's vector
// memory operations report completion in issue order, so once a load issued
// after the partial stores has returned, the stores are complete.
__device__ inline void coherent_store(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float coherent_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void publish() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    wait_vmcnt<0>();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// The wave that brings a unit's completion count to `parts` folds the unit
// and sets the count back to zero for the next launch.
__device__ inline void reset_count(int* cnt) {
    if ((threadIdx.x & 63) == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// H8: pages of 8 tokens, folded two to a 16-token step: page a supplies
// tokens 0-7, page b tokens 8-15 (see load_pair).
// F32: f32 q, K and V (the reference's own dtype): scores on
// v_mfma_f32_16x16x4_f32 with lane l holding head dims 16*j + 4*(l/16) .. +3
// of its token for j < D/16 (the K order of a product is free), p @ v on the same MFMA
// with p as it is (no hi / lo split); F16 is then unused.
// RM: the [1, 16] mask is a row broadcast (the reference's rule for a square
// score tile): one value per query row, mask[r] for row r, G == 16.
template <int G, int D, bool F16, bool MASK, bool H8 = false, bool F32 = false, bool RM = false>
struct DecodeWave {
    static_assert(G >= 1 && G <= 48 && (D == 64 || D == 128 || D == 256), "decode shape");
    static_assert(!F32 || D <= 128 || G <= 16, "f32 decode shape");
    static_assert(!RM || (G == 16 && MASK && !H8), "row-broadcast mask shape");
    static constexpr int ES = F32 ? 4 : 2;     // element bytes of q, K, V
    static constexpr int NS = D * ES / 64;     // u32x4 of K per lane (bf16 / f16: head-dim slices of the score MFMA)
    static constexpr int DV = D / 16;          // head-dim columns per lane in p @ v
    static constexpr int VW = DV * ES / 4;     // u32 of V per lane and token
    static_assert(VW == 2 || VW % 4 == 0, "V loads");
    static constexpr int KC = 64;              // bytes between a lane's K chunks
    static constexpr int RB = (G + 15) / 16;   // blocks of 16 query rows (one MFMA row block each)
    static constexpr int NQ = RB * NS;         // q registers (u32x4) per lane
    static constexpr int kHalves = H8 ? 2 : 1;  // pages per 16-token step
    // The stream holds the next unit's q in registers ahead of its first
    // page, except with more than 16 query rows at head dim 128 or in f32:
    // there a second q set (16 or 32 registers per 16 rows) costs the fold
    // more than reading q behind a full wait at each unit start.
    static constexpr bool kPrefetchQ = !((RB > 1 && (F32 || D >= 128)) || (F32 && D > 128));
    // Partial layout: o[G][D] (head dims permuted, see store), then m[G] and
    // l[G]; padded to 16 bytes so that every partial's o rows are 16-byte
    // aligned.
    static constexpr int kPartM = G * D;
    static constexpr int kPartFloats = G * D + ((2 * G + 3) & ~3);

    struct Page {
        u32x4 k[NS];           // lane l: token l%16, head dims 32*j + 8*(l/16) .. +7 (F32: 16*j + 4*(l/16) .. +3)
        u32 v[4][VW];          // lane l: tokens 4*(l/16) + i, head dims DV*(l%16) .. +DV-1
        float mask[4];         // lane l: tokens 4*(l/16) .. +3 (RM: query row l%16's value, four times)
        float hneg;            // H8: added to the scores of tokens 8-15 (0, or -inf without page b)
    };

    // Per-lane byte offsets within a page, fixed for a launch: K (token t at
    // t*ks elements, head dims contiguous), V (token t at t*vs), mask (token t
    // at t, four tokens per lane).  With H8 tokens 8-15 are tokens 0-7 of the
    // second page.
    struct Lanes {
        u32 k, v, m;
        u32 vrow;    // bytes between consecutive V tokens
    };
    __device__ static Lanes lanes(i64 ks, i64 vs) {
        const int lane = threadIdx.x & 63, t = lane & 15, grp = lane >> 4;
        const int tk = H8 ? (t & 7) : t, gv = H8 ? (grp & 1) : grp;
        Lanes r;
        r.k = static_cast<u32>((tk * ks + (F32 ? 4 : 8) * grp) * ES);
        r.v = static_cast<u32>((4 * gv * vs + DV * t) * ES);
        r.m = static_cast<u32>(RM ? t * 4 : gv * 16);
        r.vrow = static_cast<u32>(vs * ES);
        return r;
    }

    // H8: one step of two 8-token pages.  Each lane reads from the page its
    // tokens belong to (K: token l%16 < 8 from page a; V and mask: tokens
    // 4*(l/16)..+3 < 8 from page a), through a per-lane address: nontemporal
    // global loads, one instruction per register as for a 16-token page.
    // Without a page b (a unit's odd last page) the b bases are a's again, so
    // the lanes of tokens 8-15 re-read page a (no new lines), and hneg sets
    // those tokens' scores to -inf.  Steps past the stream's end are loaded
    // from the stream's last step in the same way and never folded.
    __device__ static void load_pair(Page& pg, const u16* ka, const u16* va, const float* ma, const u16* kb, const u16* vb,
                                     const float* mb, const Lanes& ln, bool two) {
        const int lane = threadIdx.x & 63, t = lane & 15, grp = lane >> 4;
        const char* kp = reinterpret_cast<const char*>(t < 8 ? ka : kb) + ln.k;
#pragma unroll
        for (int j = 0; j < NS; ++j) pg.k[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + KC * j));
        const char* vp = reinterpret_cast<const char*>(grp < 2 ? va : vb) + ln.v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const char* vi = vp + static_cast<u64>(i * ln.vrow);
            if constexpr (VW % 4 == 0) {
#pragma unroll
                for (int c = 0; c < VW / 4; ++c) {
                    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vi + 16 * c));
                    pg.v[i][4 * c] = a.x; pg.v[i][4 * c + 1] = a.y; pg.v[i][4 * c + 2] = a.z; pg.v[i][4 * c + 3] = a.w;
                }
            } else {
                const u32x2 a = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vi));
                pg.v[i][0] = a.x; pg.v[i][1] = a.y;
            }
        }
        if constexpr (MASK) {
            const u32x4 mk = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(grp < 2 ? ma : mb) + ln.m));
            pg.mask[0] = __uint_as_float(mk.x);
            pg.mask[1] = __uint_as_float(mk.y);
            pg.mask[2] = __uint_as_float(mk.z);
            pg.mask[3] = __uint_as_float(mk.w);
        }
        pg.hneg = two ? 0.0f : -__builtin_inff();
    }

    // kp, vp, mp: wave-uniform page bases (buffer loads, streaming).  With
    // real false every load is out of range of its buffer (no records): it
    // reads no memory and returns zeros, and it still counts as a load.
    __device__ static void load_page(Page& pg, const u16* kp, const u16* vp, const float* mp, const Lanes& ln, bool real) {
        const int nrec = __builtin_amdgcn_readfirstlane(real ? -1 : 0);  // real is wave-uniform
        const buf_rsrc rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<u16*>(kp), 0, nrec, 0x00020000);
        const buf_rsrc rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<u16*>(vp), 0, nrec, 0x00020000);
#pragma unroll
        for (int j = 0; j < NS; ++j)
            pg.k[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, ln.k + KC * j, 0, 2));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32 so = i * ln.vrow;
            if constexpr (VW % 4 == 0) {
#pragma unroll
                for (int c = 0; c < VW / 4; ++c) {
                    const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, ln.v + 16 * c, so, 2));
                    pg.v[i][4 * c] = a.x; pg.v[i][4 * c + 1] = a.y; pg.v[i][4 * c + 2] = a.z; pg.v[i][4 * c + 3] = a.w;
                }
            } else {
                const u32x2 a = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rv, ln.v, so, 2));
                pg.v[i][0] = a.x; pg.v[i][1] = a.y;
            }
        }
        if constexpr (MASK && RM) {
            // The lane's query row's value, for all four of its tokens.
            const buf_rsrc rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(mp), 0, nrec, 0x00020000);
            const float mk = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, ln.m, 0, 2));
            pg.mask[0] = mk;
            pg.mask[1] = mk;
            pg.mask[2] = mk;
            pg.mask[3] = mk;
        } else if constexpr (MASK) {
            const buf_rsrc rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(mp), 0, nrec, 0x00020000);
            const u32x4 mk = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rm, ln.m, 0, 2));
            pg.mask[0] = __uint_as_float(mk.x);
            pg.mask[1] = __uint_as_float(mk.y);
            pg.mask[2] = __uint_as_float(mk.z);
            pg.mask[3] = __uint_as_float(mk.w);
        }
    }

    struct State {
        float m[RB], l[RB];    // query row 16*rb + l%16, replicated over its 4 lanes
        f32x4v_t o[RB][DV];    // o[rb][e][j]: query row 16*rb + 4*(l/16) + j, head dim DV*(l%16) + e
    };

    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    // hi + lo == x for four fp32 values x to about 2^-17 (bf16) / 2^-22 (f16)
    // relative: hi = x rounded to 16 bits, lo = (x - hi) rounded (x - hi is
    // exact in fp32).  Packed two per dword, element 0 in the low half.
    template <bool H, class A, class B> struct Pick { typedef B type; };
    template <class A, class B> struct Pick<true, A, B> { typedef A type; };
    __device__ static void split4(f32x4v_t x, u32x2& hi, u32x2& lo) {
        typedef typename Pick<F16, _Float16, __bf16>::type h_t;
        typedef h_t h2_t __attribute__((ext_vector_type(2)));
        const f32x2_t x0 = {x[0], x[1]}, x1 = {x[2], x[3]};
        const h2_t a = __builtin_convertvector(x0, h2_t), b = __builtin_convertvector(x1, h2_t);
        const f32x2_t r0 = x0 - __builtin_convertvector(a, f32x2_t), r1 = x1 - __builtin_convertvector(b, f32x2_t);
        hi = u32x2{__builtin_bit_cast(u32, a), __builtin_bit_cast(u32, b)};
        lo = u32x2{__builtin_bit_cast(u32, __builtin_convertvector(r0, h2_t)), __builtin_bit_cast(u32, __builtin_convertvector(r1, h2_t))};
    }
    // v_mfma_f32_16x16x16 (bf16 / f16): lane l holds A[l%16][4*(l/16)..+3],
    // B[4*(l/16)..+3][l%16] and D[4*(l/16)..+3][l%16].
    __device__ static f32x4v_t mfma16(u32x2 a, u32x2 b, f32x4v_t c) {
        if constexpr (F16) {
            typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
            return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4_t, a), __builtin_bit_cast(h4_t, b), c, 0, 0, 0);
        } else {
            return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
        }
    }

    __device__ static void step(State& st, const Page& pg, const u32x4* qa, float scale) {
        const int lane = threadIdx.x & 63, t = lane & 15, grp = lane >> 4;
        // Scores S^T: A = the K page, B = q^T; lane l holds tokens 4*(l/16) + i
        // of query row 16*rb + l%16.  The page registers serve every row block.
        f32x4v_t acc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            acc[rb] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (F32) {
                // MFMA (j, x) pairs head dim 16*j + 4*g + x of lane group g of
                // K and q: a K load instruction covers 64 contiguous bytes of
                // each token's row.
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int x = 0; x < 4; ++x)
                        acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(pg.k[j][x]), __uint_as_float(qa[rb * NS + j][x]),
                                                                     acc[rb], 0, 0, 0);
            } else {
#pragma unroll
                for (int j = 0; j < NS; ++j) acc[rb] = mfma_16x16x32<F16>(pg.k[j], qa[rb * NS + j], acc[rb]);
            }
        }
        float hb = 0.0f;
        if constexpr (H8) hb = grp < 2 ? 0.0f : pg.hneg;
        // Online softmax of query row 16*rb + l%16 (rows >= G are q = 0 rows
        // whose results are never stored; p @ v keeps MFMA rows apart).  The
        // row blocks' softmax chains are independent and sit in one basic
        // block, ahead of the rescale branches, so that they interleave.
        auto fmax_ = [](float x, float y) { return fmaxf(x, y); };
        auto fadd_ = [](float x, float y) { return x + y; };
        float a[RB];
        u32x2 ph[RB], pl[RB];
        f32x4v_t pf[RB];
        bool rescale[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[i] = acc[rb][i] * scale;
                if constexpr (MASK) sc[i] = sc[i] - pg.mask[i];
                if constexpr (H8) sc[i] += hb;
            }
            const float mx = cross4_reduce(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmax_);
            const float mn = fmaxf(st.m[rb], mx);
            a[rb] = expf(st.m[rb] - mn);
            f32x4v_t pr;
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[i] = expf(sc[i] - mn);
            st.l[rb] = st.l[rb] * a[rb] + cross4_reduce((pr[0] + pr[1]) + (pr[2] + pr[3]), fadd_);
            st.m[rb] = mn;
            rescale[rb] = __builtin_amdgcn_ballot_w64(16 * rb + t < G && a[rb] != 1.0f) != 0;
            if constexpr (F32) pf[rb] = pr;
            else split4(pr, ph[rb], pl[rb]);
        }
        // o <- o * a + p @ v on the matrix cores: v_mfma_f32_16x16x16 with
        // M = query rows, K = the page's 16 tokens, N = 16 head dims.  p is
        // fp32 and enters as hi + lo (split4), two products per MFMA step;
        // the lane's scores are already its A operand (query row l%16,
        // tokens 4*(l/16)..+3).  MFMA e covers head dims DV*n + e (n = l%16):
        // lane (n, l/16) supplies V[tokens 4*(l/16)..+3][DV*n + e] straight
        // from its page registers (one 16-bit half of pg.v[i][e/2] per token)
        // and accumulates o rows 4*(l/16)..+3.  Once the running maxima
        // settle, a == 1 for every row and o * a == o exactly, so the rescale
        // is skipped for the whole wave.
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rescale[rb]) {
                // A real branch (the empty asm keeps it from being turned into
                // selects): the multiply is rare, and o stays in the matrix
                // cores' accumulator registers otherwise.  o row 4*(l/16) + j
                // takes the factor of query row 4*(l/16) + j, held by lane
                // 4*(l/16) + j.
                asm volatile("");
                f32x4v_t a4;
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[j] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * grp + j) * 4, __float_as_int(a[rb])));
#pragma unroll
                for (int e = 0; e < DV; ++e) st.o[rb][e] = st.o[rb][e] * a4;
            }
        }
        if constexpr (F32) {
            // MFMA i pairs token 4*g + i of lane group g: the lane's own score
            // pf[i] and V value pg.v[i][e].
#pragma unroll
            for (int e = 0; e < DV; ++e)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        st.o[rb][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(pf[rb][i], __uint_as_float(pg.v[i][e]), st.o[rb][e], 0, 0, 0);
        } else {
#pragma unroll
            for (int e = 0; e < DV; ++e) {
                const u32 sel = (e & 1) ? 0x07060302u : 0x05040100u;
                const u32x2 bv = {__builtin_amdgcn_perm(pg.v[1][e >> 1], pg.v[0][e >> 1], sel),
                                  __builtin_amdgcn_perm(pg.v[3][e >> 1], pg.v[2][e >> 1], sel)};
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    st.o[rb][e] = mfma16(ph[rb], bv, st.o[rb][e]);
                    st.o[rb][e] = mfma16(pl[rb], bv, st.o[rb][e]);
                }
            }
        }
    }

    // q rows as the score MFMA's B operand, row block rb in qa[rb*NS ..]
    // (rows >= G are zero).
    __device__ static void load_q(u32x4 (&qa)[NQ], const u16* q, i64 qs) {
        const int lane = threadIdx.x & 63, t = lane & 15, grp = lane >> 4;
        const char* qb = reinterpret_cast<const char*>(q);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                qa[rb * NS + j] = u32x4{0u, 0u, 0u, 0u};
                const i64 e = (16 * rb + t) * qs + (F32 ? 16 * j + 4 * grp : 32 * j + 8 * grp);
                if (16 * rb + t < G) qa[rb * NS + j] = *reinterpret_cast<const u32x4*>(qb + e * ES);
            }
        }
    }

    __device__ static void init(State& st) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            st.m[rb] = -__builtin_inff();
            st.l[rb] = 0.0f;
#pragma unroll
            for (int e = 0; e < DV; ++e) st.o[rb][e] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    // Writes st as a partial.  The stores carry sc1, the cache policy of the
    // agent-scope atomic stores of the memory model (see coherent_store):
    // they are written through to memory, where a wave of another XCD reads
    // them.  o is stored 128 bits per lane: lane n's four head dims
    // DV*n + 4c .. +3 of a row sit at positions 64c + 4n .. +3 (part_dim maps
    // back), so the 16 lanes of a row group write 256 contiguous bytes per
    // (row, c).
    __device__ static void store(const State& st, float* part) {
        const int lane = threadIdx.x & 63, t = lane & 15, grp = lane >> 4;
        const buf_rsrc rp = __builtin_amdgcn_make_buffer_rsrc(part, 0, -1, 0x00020000);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (grp == 0 && 16 * rb + t < G) {
                coherent_store(part + kPartM + 16 * rb + t, st.m[rb]);
                coherent_store(part + kPartM + G + 16 * rb + t, st.l[rb]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int g = 16 * rb + 4 * grp + j;
                if (g < G) {
#pragma unroll
                    for (int c = 0; c < DV / 4; ++c) {
                        const u32x4 w = {__float_as_uint(st.o[rb][4 * c][j]), __float_as_uint(st.o[rb][4 * c + 1][j]),
                                         __float_as_uint(st.o[rb][4 * c + 2][j]), __float_as_uint(st.o[rb][4 * c + 3][j])};
                        __builtin_amdgcn_raw_buffer_store_b128(w, rp, static_cast<u32>((g * D + 64 * c + 4 * t) * 4), 0, 16);
                    }
                }
            }
        }
    }
};

// Head dim held at position p of a partial's o row (see DecodeWave::store).
template <int D>
__device__ inline int part_dim(int p) {
    return (D / 16) * ((p & 63) >> 2) + 4 * (p >> 6) + (p & 3);
}

// Balanced split of a decode launch over the resident waves.  The units'
// pages are concatenated in unit order (page prefix pre[0..U], pre[U] = T)
// and so are their scheduling costs: a non-empty unit costs its pages plus
// kUnitCost leading positions that hold no page, for the work a wave does
// at every unit it starts (partial store, q switch, stalled ring), so that
// ranges with many short units get fewer pages (cost prefix cpre[0..U],
// cpre[U] = TC).  Wave w of W <= TC owns cost positions [w*TC/W,
// (w+1)*TC/W), i.e. the pages [page_at(w*TC/W), page_at((w+1)*TC/W)).  A
// wave writes one partial per unit it touches, into slot unit + w (slots are
// distinct because the first wave of unit u+1 is at least the last wave of
// unit u); unit u's partials are the consecutive slots u + wf .. u + wl, wf
// and wl the waves of its first page (cost position cpre[u] + kUnitCost)
// and last page (cpre[u+1] - 1).  A wave whose cost range holds no page
// lies before the first page of a unit, never between two waves of one.
struct DecodeSplit {
    static constexpr int kMaxUnits = 4096;  // prefixes held in LDS by every block
    static constexpr int kUnitCost = 3;
    __device__ static int cost(int pages) { return pages > 0 ? pages + kUnitCost : 0; }
    // Wave holding cost position p: the largest w with w*TC/W <= p.
    __device__ static i64 wave_of(i64 p, i64 TC, i64 W) { return ((p + 1) * W - 1) / TC; }
    // Largest u in [0, U) with pre[u] <= s, for 0 <= s < pre[U] (a non-empty unit).
    __device__ static int unit_of(const int* pre, int U, i64 s) {
        int lo = 0, hi = U;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (pre[mid] <= s) lo = mid;
            else hi = mid;
        }
        return lo;
    }
    // First page at or after cost position v (T for v >= TC).
    __device__ static i64 page_at(const int* pre, const int* cpre, int U, i64 v) {
        if (v >= cpre[U]) return pre[U];
        const int u = unit_of(cpre, U, v);
        const i64 off = v - cpre[u] - kUnitCost;
        return pre[u] + (off > 0 ? off : 0);
    }
};

// i64 held by lane i (i wave-uniform), as a wave-uniform value.
__device__ inline i64 readlane64(i64 x, int i) {
    const u64 b = static_cast<u64>(x);
    const u32 lo = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(b)), i));
    const u32 hi = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(b >> 32)), i));
    return static_cast<i64>((static_cast<u64>(hi) << 32) | lo);
}

// Element offsets of one page: K^T tile, V tile, mask row.
struct PageOffs {
    i64 k, v, m;
};

// The addressing hooks of a decode launch (see DecodeStream), from lambdas.
template <class P, class B, class Q, class S, class C>
struct DecodeFns {
    P page;
    B bases;
    Q q;
    S slot;
    C combine;
};
template <class P, class B, class Q, class S, class C>
__device__ inline DecodeFns<P, B, Q, S, C> decode_fns(P p, B b, Q q, S s, C c) {
    return DecodeFns<P, B, Q, S, C>{p, b, q, s, c};
}

// One decode wave's pages [s, b) of the launch (units laid end to end, see
// DecodeSplit; a "page" here is one 16-token step) folded as a single
// stream: the NB-page register ring keeps loading across unit boundaries and
// across the 64-page runs of page-table offsets (lane i of a run holds page
// r0+i's offsets; the next run is read 64 pages ahead; with two 8-token pages
// per step, 32 steps of two pages each), so the wave never waits for a page
// table or q read.
//
// At the end of a unit's pages in this wave the partial is stored and its
// completion deferred: vector memory operations of a wave complete in issue
// order, so NB folded pages later (page loads issued after the stores have
// returned) the stores are complete and the arrival is counted; NB pages
// after that the count's old value has returned, and the last arriver folds
// the unit's partials.  A second unit end while one is pending, and the end
// of the stream, complete it at once (waiting for the stores).
//
// F provides: page(h, PageOffs&) per lane, h = the step's index times
// DW::kHalves plus the page's half (k < 0 for a half the unit does not
// have); bases(PageOffs, kp, vp, mp);
// q(u) (q tile of unit u, or null when out of range); slot(u) (this wave's
// partial of unit u); combine(u, parts, first_slot).
template <class DW, int NB, bool ORDERED>
struct DecodeStream {
    struct Pending {
        int unit, parts, phase, wait;  // phase 0: none, 1: stores issued, 2: arrival issued
        i64 first;                     // first partial slot of the unit
        int old_v;                     // arrival count before this wave's (lane 0)
    };

    // ORDERED: the whole wave executes an agent-scope release fence before
    // lane 0's arrival RMW (its partial stores are complete and written back
    // before the count moves), and the last arriver an agent-scope acquire
    // fence before it reads the partials.
    __device__ static void arrive_issue(Pending& pd, int* cnt) {
        if constexpr (ORDERED) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        int r = 0;
        if ((threadIdx.x & 63) == 0) r = __hip_atomic_fetch_add(cnt + pd.unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pd.old_v = r;
    }
    template <class F>
    __device__ static void finish(Pending& pd, int* cnt, F& f) {
        bool last = true;
        if (pd.parts > 1) {
            last = __builtin_amdgcn_readfirstlane(pd.old_v) == pd.parts - 1;
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            if constexpr (ORDERED)
                if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        if (last) {
            f.combine(pd.unit, pd.parts, pd.first);
            if (pd.parts > 1) reset_count(cnt + pd.unit);
        }
        pd.phase = 0;
    }
    // Completes a pending unit now.
    template <class F>
    __device__ static void flush(Pending& pd, int* cnt, F& f) {
        if (pd.phase == 0) return;
        if (pd.phase == 1) {
            publish();
            if (pd.parts > 1) arrive_issue(pd, cnt);
        }
        finish(pd, cnt, f);
    }
    // One folded page of progress on a pending unit.
    template <class F>
    __device__ static void tick(Pending& pd, int* cnt, F& f) {
        if (pd.phase == 0 || --pd.wait > 0) return;
        if (pd.phase == 1 && pd.parts > 1) {
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            arrive_issue(pd, cnt);
            pd.phase = 2;
            pd.wait = NB;
            return;
        }
        finish(pd, cnt, f);
    }

    // Next unit after u with at least one page.
    __device__ static int next_unit(const int* pre, int u) {
        int n = u + 1;
        while (__builtin_amdgcn_readfirstlane(pre[n + 1]) == __builtin_amdgcn_readfirstlane(pre[n])) ++n;
        return n;
    }

    template <class F>
    __device__ static void run(F& f, const int* pre, const int* cpre, int U, i64 TC, i64 W, i64 w, i64 s, i64 b, int* cnt,
                               float scale, i64 ks, i64 vs, i64 qs) {
        const int lane = threadIdx.x & 63;
        const typename DW::Lanes ln = DW::lanes(ks, vs);
        // Page-table runs: lane i holds the offsets of page i%HS of step
        // r0 + i/HS (f.page takes that half-step index, HS*step + half).
        constexpr int HS = DW::kHalves, RL = 64 / HS;
        auto run_of = [&](i64 g0, PageOffs& po) { f.page(HS * g0 + lane < HS * b ? HS * g0 + lane : HS * b - 1, po); };
        i64 r0 = s;
        PageOffs rc, rn;
        run_of(s, rc);
        rn = rc;
        // Step g's offsets are read from the current run only: the run moves
        // on just before the first step past it is loaded, so the next run's
        // registers are read RL steps after their load was issued.  (A select
        // between the two runs here would make every page load wait for the
        // most recent page-table read, i.e. for the whole ring.)
        auto load = [&](typename DW::Page& pg, i64 g) {
            const bool real = g < b;
            if (real && g - r0 == RL) {
                r0 += RL;
                rc = rn;
                if (r0 + RL < b) run_of(r0 + RL, rn);
            }
            const int li = HS * static_cast<int>((real ? g : b - 1) - r0);
            PageOffs po;
            po.k = readlane64(rc.k, li);
            po.v = readlane64(rc.v, li);
            po.m = readlane64(rc.m, li);
            const u16 *kp, *vp;
            const float* mp;
            f.bases(po, kp, vp, mp);
            if constexpr (HS == 2) {
                // A step's second page (k < 0: the unit has no such page).
                PageOffs p2;
                p2.k = readlane64(rc.k, li + 1);
                p2.v = readlane64(rc.v, li + 1);
                p2.m = readlane64(rc.m, li + 1);
                const bool two = p2.k >= 0;
                if (!two) p2 = po;
                const u16 *kp2, *vp2;
                const float* mp2;
                f.bases(p2, kp2, vp2, mp2);
                DW::load_pair(pg, kp, vp, mp, kp2, vp2, mp2, ln, two);
            } else {
                // Past the stream's end the ring is still filled (so that
                // every step waits for the same number of loads) with loads
                // that read nothing.  The lane offsets stay the same
                // registers on every path: a lane-offset temporary could
                // share registers with a page load in flight, and the wait
                // for that write would drain the ring.
                DW::load_page(pg, kp, vp, mp, ln, real);
            }
        };
        // The first pages go out before anything else is read.
        typename DW::Page pg[NB];
#pragma unroll
        for (int i = 0; i < NB - 1; ++i) load(pg[i], s + i);
        if (s + RL < b) run_of(s + RL, rn);
        // Unit state.
        int u = DecodeSplit::unit_of(pre, U, s);
        u = __builtin_amdgcn_readfirstlane(u);
        i64 eu = __builtin_amdgcn_readfirstlane(pre[u + 1]);
        if (eu > b) eu = b;
        typename DW::State st;
        DW::init(st);
        u32x4 qa[DW::NQ], qn[DW::NQ];
        // A q tile out of range (error already flagged) folds with q = 0;
        // every step runs, so that its page waits order the partial stores.
        auto get_q = [&](u32x4 (&dst)[DW::NQ], int unit) {
            const u16* qp = f.q(unit);
            if (qp) {
                DW::load_q(dst, qp, qs);
            } else {
#pragma unroll
                for (int j = 0; j < DW::NQ; ++j) dst[j] = u32x4{0u, 0u, 0u, 0u};
            }
        };
        get_q(qa, u);
        // The first pages and q are waited for here, once: a load into q's
        // registers still in flight where the stream loop begins would make
        // the compiler's wait counts drain the ring at every loop iteration.
        wait_vmcnt<0>();
        int un = u;
        if (DW::kPrefetchQ && eu < b) {
            un = next_unit(pre, u);
            get_q(qn, un);
        }
        Pending pd;
        pd.phase = 0;
        for (i64 g = s;; g += NB) {
#pragma unroll
            for (int i = 0; i < NB; ++i) {
                const i64 gi = g + i;
                load(pg[(i + NB - 1) % NB], gi + NB - 1);
                DW::step(st, pg[i], qa, scale);
                tick(pd, cnt, f);
                if (gi + 1 == eu) {
                    // Unit u's pages in this wave are folded.
                    flush(pd, cnt, f);
                    const i64 cs = __builtin_amdgcn_readfirstlane(cpre[u]);
                    const i64 ce = __builtin_amdgcn_readfirstlane(cpre[u + 1]);
                    const i64 wf = DecodeSplit::wave_of(cs + DecodeSplit::kUnitCost, TC, W);
                    const i64 wl = DecodeSplit::wave_of(ce - 1, TC, W);
                    pd.unit = u;
                    pd.parts = static_cast<int>(wl - wf + 1);
                    pd.first = u + wf;
                    DW::store(st, f.slot(u));
                    pd.phase = 1;
                    pd.wait = NB;
                    if (eu >= b) {
                        flush(pd, cnt, f);
                        return;
                    }
                    if constexpr (DW::kPrefetchQ) {
                        u = un;
                        eu = __builtin_amdgcn_readfirstlane(pre[u + 1]);
                        if (eu > b) eu = b;
                        DW::init(st);
#pragma unroll
                        for (int j = 0; j < DW::NQ; ++j) qa[j] = qn[j];
                        if (eu < b) {
                            un = next_unit(pre, u);
                            get_q(qn, un);
                        }
                    } else {
                        // q is read here, behind the whole ring: the wait
                        // keeps the load out of the loop's later wait counts.
                        u = next_unit(pre, u);
                        eu = __builtin_amdgcn_readfirstlane(pre[u + 1]);
                        if (eu > b) eu = b;
                        DW::init(st);
                        get_q(qa, u);
                        wait_vmcnt<0>();
                    }
                }
            }
        }
    }
};

template <int G, int D, int ACC = 16>
struct DecodeCombine {
    static constexpr int DPL = D / 64;
    static constexpr int CB = 2;  // partials loaded together
    // Query rows folded per pass: R * DPL <= ACC accumulators per lane, so
    // the combine (inlined where a unit completes, with the page ring in
    // flight) needs the same registers for every G.
    static_assert(ACC >= DPL, "combine pass width");
    static constexpr int R = (ACC / DPL < G) ? ACC / DPL : G;
    __device__ static void fold(int g0, float (&mm)[R], float (&ll)[R], float (&oo)[R][DPL], const float* mc, const float* lc,
                                const float (*oc)[DPL]) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (g0 + r < G) {
                const float mn = fmaxf(mm[r], mc[r]);
                const float a = expf(mm[r] - mn), b = expf(mc[r] - mn);
                ll[r] = ll[r] * a + lc[r] * b;
#pragma unroll
                for (int j = 0; j < DPL; ++j) oo[r][j] = oo[r][j] * a + oc[r][j] * b;
                mm[r] = mn;
            }
        }
    }
    // Rows g0 .. g0+R-1 (those below G) of partial pc.
    __device__ static void load_rows(int g0, const float* pc, float (&mc)[R], float (&lc)[R], float (&oc)[R][DPL]) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int g = g0 + r;
            if (g < G) {
                mc[r] = coherent_load(pc + G * D + g);
                lc[r] = coherent_load(pc + G * D + G + g);
#pragma unroll
                for (int j = 0; j < DPL; ++j) oc[r][j] = coherent_load(pc + g * D + DPL * lane + j);
            }
        }
    }
    // Folds nch partials (page order) into the unit's accumulators; with out
    // non-null also writes out = o / l (the normalisation launch folded in).
    // Rows pass by pass; each row folds its partials in page order.
    __device__ static void run(i64 nch, const float* part, i64 pstride, float* m, i64 ms3, float* l, i64 ls3, float* o,
                               i64 os3, i64 os4, float* out, i64 us3, i64 us4) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int g0 = 0; g0 < G; g0 += R) {
            float mm[R], ll[R], oo[R][DPL];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int g = g0 + r;
                mm[r] = 0.0f;
                ll[r] = 0.0f;
#pragma unroll
                for (int j = 0; j < DPL; ++j) oo[r][j] = 0.0f;
                if (g < G) {
                    mm[r] = m[g * ms3];
                    ll[r] = l[g * ls3];
#pragma unroll
                    for (int j = 0; j < DPL; ++j) oo[r][j] = o[g * os3 + part_dim<D>(DPL * lane + j) * os4];
                }
            }
            i64 c = 0;
            for (; c + CB <= nch; c += CB) {
                float mc[CB][R], lc[CB][R], oc[CB][R][DPL];
#pragma unroll
                for (int b = 0; b < CB; ++b) load_rows(g0, part + (c + b) * pstride, mc[b], lc[b], oc[b]);
#pragma unroll
                for (int b = 0; b < CB; ++b) fold(g0, mm, ll, oo, mc[b], lc[b], oc[b]);
            }
            for (; c < nch; ++c) {
                float mc[R], lc[R], oc[R][DPL];
                load_rows(g0, part + c * pstride, mc, lc, oc);
                fold(g0, mm, ll, oo, mc, lc, oc);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int g = g0 + r;
                if (g < G) {
                    if (lane == 0) {
                        m[g * ms3] = mm[r];
                        l[g * ls3] = ll[r];
                    }
#pragma unroll
                    for (int j = 0; j < DPL; ++j) o[g * os3 + part_dim<D>(DPL * lane + j) * os4] = oo[r][j];
                    if (out) {
#pragma unroll
                        for (int j = 0; j < DPL; ++j) out[g * us3 + part_dim<D>(DPL * lane + j) * us4] = oo[r][j] / ll[r];
                    }
                }
            }
        }
    }
    // out = o / l of a unit no page folds into (its accumulators as they are).
    __device__ static void normalize(const float* o, i64 os3, i64 os4, const float* l, i64 ls3, float* out, i64 us3, i64 us4) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float lg = l[g * ls3];
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const int d = DPL * lane + j;
                out[g * us3 + d * us4] = o[g * os3 + d * os4] / lg;
            }
        }
    }
};

}  // namespace ptowsp
