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
__device__ inline i64 indirect_index(const LaunchArgs& A, int k, const i64* vars, int nvars) {
    const IndirectTerm& t = A.ind[k];
    i64 off = t.c;
    for (int v = 0; v < nvars; ++v) off += t.coef[v] * vars[v];
    i64 idx = 0;
    if (off >= 0 && off < t.span) idx = t.base[off];
    if (off < 0 || off >= t.span || idx < 0 || idx >= t.bound) {
        *A.err = 1;
        idx = 0;
    }
    return idx * t.stride;
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

__device__ inline u16 f32_to_half_bits(float f) { return __builtin_bit_cast(u16, static_cast<_Float16>(f)); }

// Round-to-nearest-even f32 -> bf16 (NaN stays NaN).
__device__ inline u16 f32_to_bf16_bits(float f) {
    const u32 x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<u16>((x >> 16) | 0x40u);
    return static_cast<u16>((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
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
//     at g ^ (k & 3); the MFMA B operand is read with ds_read_b64_tr_b16,
//     which transposes 16-bit elements across each group of 16 lanes.
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
typedef __amdgpu_buffer_rsrc_t buf_rsrc;

template <bool F16>
__device__ inline f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

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

template <int BM, int BN, int BK, int WM, int WN, bool F16>
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
    static constexpr int kLdsElems = 2 * STAGE;
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
            const int c = (((p >> 1) ^ (k & 3)) << 1) | (p & 1);
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
                const int pn = (((n >> 4) ^ e) << 4) | (n & 15);
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

    // K steps it0 .. iters-1; off(it, soa, sob) gives step it's byte offsets
    // from the step-0 origins pa / pb.  ACC: the block starts from C.
    template <bool ACC, class Off>
    __device__ static void run(u16* lds, const u16* pa, int lda, const u16* pb, int ldb, float* pc, int ldc, i64 it0,
                               i64 iters, Off off) {
        const u32x4 ra = buffer_words(pa), rb = buffer_words(pb);
        const buf_rsrc rc = __builtin_amdgcn_make_buffer_rsrc(pc, 0, -1, 0x00020000);
        Offs o;
        offsets(o, lda, ldb);
        Acc acc;
        if constexpr (ACC) {
            c_io<false>(acc, rc, ldc);
        } else {
#pragma unroll
            for (int i = 0; i < FI; ++i)
#pragma unroll
                for (int j = 0; j < FJ; ++j) acc.v[i][j] = f32x16{};
        }
        wait_vmcnt<0>();
        __syncthreads();  // the previous block's last stage reads are done
        int soa, sob;
        off(it0, soa, sob);
        load(lds, o, ra, soa, rb, sob);
        for (i64 it = it0; it < iters; ++it) {
            wait_vmcnt<0>();
            __syncthreads();
            const int cur = static_cast<int>((it - it0) & 1);
            if (it + 1 < iters) {
                off(it + 1, soa, sob);
                load(lds + (cur ^ 1) * STAGE, o, ra, soa, rb, sob);
            }
            mma(acc, lds + cur * STAGE);
        }
        c_io<true>(acc, rc, ldc);
    }
};

// ---------------------------------------------------------------------------
// Decode: online softmax over 16-token pages (flashinfer_decode pattern)
// ---------------------------------------------------------------------------
//
// The pages of one unit (sequence b, KV group g) are split into chunks; one
// wave folds a chunk into a partial (m, l, o) for the unit's G query rows,
// starting from (-inf, 0, 0), and DecodeCombine folds the partials of a unit
// in chunk order into the accumulators.  Per page:
//  * scores on MFMA v_mfma_f32_16x16x32 (one per 32-wide head-dim slice):
//    A = the K page (lane l: token l%16, head dims 8*(l/16)..+7 of the slice),
//    B = q^T (lane l: query row l%16, zero for rows >= G); lane l then holds
//    query row l%16 for tokens 4*(l/16)..+3;
//  * row max / row sum over the 16 tokens: 4 values in the lane, then lanes
//    l^16 and l^32;
//  * p and the rescale factor pass through LDS; p @ v runs in fp32 on the
//    VALU with lane l owning head-dim columns (D/64)*l ..; the sum over the 16
//    tokens runs in token order, mul then add (as the oracle's TMATMUL).

typedef float f32x4v_t __attribute__((ext_vector_type(4)));

template <bool F16>
__device__ inline f32x4v_t mfma_16x16x32(u32x4 a, u32x4 b, f32x4v_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

// 16-bit float (bf16 or f16) in the low / high half of a dword, as f32.
template <bool F16>
__device__ inline float h16_lo(u32 w) {
    if constexpr (F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<u16>(w & 0xFFFFu)));
    else return __uint_as_float(w << 16);
}
template <bool F16>
__device__ inline float h16_hi(u32 w) {
    if constexpr (F16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<u16>(w >> 16)));
    else return __uint_as_float(w & 0xFFFF0000u);
}

// Orders LDS traffic between the lanes of one wave (LDS executes a wave's
// instructions in order; this keeps the compiler from reordering them).
__device__ inline void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

template <int G, int D, bool F16, bool MASK>
struct DecodeWave {
    static_assert(G >= 1 && G <= 16 && (D == 64 || D == 128 || D == 256), "decode shape");
    static constexpr int NS = D / 32;    // head-dim slices, one MFMA each
    static constexpr int DPL = D / 64;   // head-dim columns per lane in p @ v
    static constexpr int kLdsFloats = G * 16 + 16;  // p rows, then the rescale factors
    // Chunk partial layout: m[G], l[G], o[G][D].
    static constexpr int kPartFloats = 2 * G + G * D;

    struct Page {
        u32x4 k[NS];
        u32 v[16 * (DPL == 4 ? 2 : 1)];  // DPL 1: one 16-bit value per token (low half)
        f32x4v_t mask;
    };

    // kp: K page (token t at kp + t*ks, head dims contiguous); vp: V page
    // (token t at vp + t*vs, head dims contiguous); mp: mask row (contiguous).
    __device__ static void load_page(Page& pg, const u16* kp, i64 ks, const u16* vp, i64 vs, const float* mp) {
        const int lane = threadIdx.x & 63, t = lane & 15, quad = lane >> 4;
#pragma unroll
        for (int j = 0; j < NS; ++j)
            pg.k[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + t * ks + 32 * j + 8 * quad));
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
            if constexpr (DPL == 4) {
                const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vp + tt * vs + 4 * lane));
                pg.v[2 * tt] = w.x;
                pg.v[2 * tt + 1] = w.y;
            } else if constexpr (DPL == 2) {
                pg.v[tt] = __builtin_nontemporal_load(reinterpret_cast<const u32*>(vp + tt * vs + 2 * lane));
            } else {
                pg.v[tt] = vp[tt * vs + lane];
            }
        }
        if constexpr (MASK) pg.mask = *reinterpret_cast<const f32x4v_t*>(mp + 4 * quad);
    }

    // Folds pages [p0, p1) into part; ptrs(p, kp, vp, mp) gives page p's bases.
    template <class PagePtrs>
    __device__ static void run(i64 p0, i64 p1, const u16* q, i64 qs, float scale, PagePtrs ptrs, i64 ks, i64 vs, float* lds,
                               float* part) {
        const int lane = threadIdx.x & 63, h = lane & 15, quad = lane >> 4;
        u32x4 qb[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            qb[j] = u32x4{0u, 0u, 0u, 0u};
            if (h < G) qb[j] = *reinterpret_cast<const u32x4*>(q + h * qs + 32 * j + 8 * quad);
        }
        float m = -__builtin_inff(), l = 0.0f;
        float o[G][DPL];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < DPL; ++j) o[g][j] = 0.0f;
        Page cur, nxt;
        const u16 *kp, *vp;
        const float* mp;
        ptrs(p0, kp, vp, mp);
        load_page(cur, kp, ks, vp, vs, mp);
        for (i64 p = p0; p < p1; ++p) {
            if (p + 1 < p1) {
                ptrs(p + 1, kp, vp, mp);
                load_page(nxt, kp, ks, vp, vs, mp);
            }
            f32x4v_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < NS; ++j) acc = mfma_16x16x32<F16>(cur.k[j], qb[j], acc);
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[i] = acc[i] * scale;
                if constexpr (MASK) sc[i] = sc[i] - cur.mask[i];
            }
            float pm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            pm = fmaxf(pm, __shfl_xor(pm, 16));
            pm = fmaxf(pm, __shfl_xor(pm, 32));
            const float mn = fmaxf(m, pm);
            const float a = expf(m - mn);
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = expf(sc[i] - mn);
            float ps = ((e[0] + e[1]) + e[2]) + e[3];
            ps = ps + __shfl_xor(ps, 16);
            ps = ps + __shfl_xor(ps, 32);
            l = l * a + ps;
            m = mn;
            if (h < G) {
                *reinterpret_cast<f32x4v_t*>(lds + h * 16 + 4 * quad) = f32x4v_t{e[0], e[1], e[2], e[3]};
                if (quad == 0) lds[G * 16 + h] = a;
            }
            wave_lds_fence();
            float pv[G][DPL];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int j = 0; j < DPL; ++j) pv[g][j] = 0.0f;
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) {
                f32x4v_t pg4[G];
#pragma unroll
                for (int g = 0; g < G; ++g) pg4[g] = *reinterpret_cast<const f32x4v_t*>(lds + g * 16 + 4 * t4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tt = 4 * t4 + i;
                    float vv[DPL];
                    if constexpr (DPL == 4) {
                        vv[0] = h16_lo<F16>(cur.v[2 * tt]);
                        vv[1] = h16_hi<F16>(cur.v[2 * tt]);
                        vv[2] = h16_lo<F16>(cur.v[2 * tt + 1]);
                        vv[3] = h16_hi<F16>(cur.v[2 * tt + 1]);
                    } else if constexpr (DPL == 2) {
                        vv[0] = h16_lo<F16>(cur.v[tt]);
                        vv[1] = h16_hi<F16>(cur.v[tt]);
                    } else {
                        vv[0] = h16_lo<F16>(cur.v[tt]);
                    }
#pragma unroll
                    for (int g = 0; g < G; ++g)
#pragma unroll
                        for (int j = 0; j < DPL; ++j) pv[g][j] = pv[g][j] + pg4[g][i] * vv[j];
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float ag = lds[G * 16 + g];
#pragma unroll
                for (int j = 0; j < DPL; ++j) o[g][j] = o[g][j] * ag + pv[g][j];
            }
            wave_lds_fence();
            cur = nxt;
        }
        if (quad == 0 && h < G) {
            part[h] = m;
            part[G + h] = l;
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < DPL; ++j) part[2 * G + g * D + DPL * lane + j] = o[g][j];
    }
};

// Folds the chunk partials of one unit, in chunk order, into its (m, l, o)
// accumulators: m' = max(m, mc), l' = l*e^(m-m') + lc*e^(mc-m'), o likewise.
template <int G, int D>
struct DecodeCombine {
    static constexpr int DPL = D / 64;
    __device__ static void run(i64 nch, const float* part, i64 pstride, float* m, i64 ms3, float* l, i64 ls3, float* o,
                               i64 os3, i64 os4) {
        const int lane = threadIdx.x & 63;
        float mm[G], ll[G], oo[G][DPL];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            mm[g] = m[g * ms3];
            ll[g] = l[g * ls3];
#pragma unroll
            for (int j = 0; j < DPL; ++j) oo[g][j] = o[g * os3 + (DPL * lane + j) * os4];
        }
        for (i64 c = 0; c < nch; ++c) {
            const float* pc = part + c * pstride;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float mc = pc[g], lc = pc[G + g];
                const float mn = fmaxf(mm[g], mc);
                const float a = expf(mm[g] - mn), b = expf(mc - mn);
                ll[g] = ll[g] * a + lc * b;
#pragma unroll
                for (int j = 0; j < DPL; ++j) oo[g][j] = oo[g][j] * a + pc[2 * G + g * D + DPL * lane + j] * b;
                mm[g] = mn;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (lane == 0) {
                m[g * ms3] = mm[g];
                l[g * ls3] = ll[g];
            }
#pragma unroll
            for (int j = 0; j < DPL; ++j) o[g * os3 + (DPL * lane + j) * os4] = oo[g][j];
        }
    }
};

}  // namespace ptowsp
