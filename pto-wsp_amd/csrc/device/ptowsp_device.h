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
// GEMM tiles: C[M,N] (fp32) from A[M,K] x B[K,N] (bf16 or f16) on MFMA
// ---------------------------------------------------------------------------
//
// One workgroup (4 waves, 2x2) owns the M x N tile; wave (wm, wn) computes
// the (M/2) x (N/2) quadrant as 32x32 blocks of v_mfma_f32_32x32x16_*.
// K steps are staged through LDS, double-buffered: A keeps its [m][k]
// layout; B is transposed on the way in (register 4x8 transpose) to
// Bt[n][k], so both MFMA operands are read as 8 consecutive k values.
// Lane l of a 32x32x16 MFMA holds row/col (l % 32), k = 8*(l/32) .. +7, and
// accumulator element e sits at row (e/4)*8 + (l/32)*4 + e%4, col l % 32.

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <bool F16>
__device__ inline f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

template <int M, int N, int K, bool F16>
struct GemmTile {
    static_assert(M % 64 == 0 && N % 64 == 0 && K % 16 == 0, "GEMM tile shape");
    static constexpr int AP = K + 8;  // LDS row pitch (16-bit elements) of A[m][k]
    static constexpr int BP = K + 8;  // LDS row pitch of Bt[n][k]
    static constexpr int ABUF = M * AP;
    static constexpr int BBUF = N * BP;
    static constexpr int kStage = ABUF + BBUF;
    static constexpr int kLdsElems = 2 * kStage;
    static constexpr int BI = M / 64, BJ = N / 64;
    static constexpr int ACH = M * K / 8;
    static constexpr int AQ = (ACH + 255) / 256;
    static constexpr int BBLK = (K / 4) * (N / 8);
    static constexpr int BQ = (BBLK + 255) / 256;

    struct Regs {
        u32x4 a[AQ];
        u32x4 b[BQ][4];
    };
    struct Acc {
        f32x16 v[BI][BJ];
    };

    // A element (m,k) at pa[m*s3a + k]; B element (k,n) at pb[k*s3b + n].
    __device__ static void gload(Regs& r, const u16* pa, i64 s3a, const u16* pb, i64 s3b) {
        const int tid = threadIdx.x;
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int c = tid + q * 256;
            if (c < ACH) {
                const int row = c / (K / 8), col = (c % (K / 8)) * 8;
                r.a[q] = *reinterpret_cast<const u32x4*>(pa + row * s3a + col);
            }
        }
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int blk = tid + q * 256;
            if (blk < BBLK) {
                const int k0 = (blk / (N / 8)) * 4, n0 = (blk % (N / 8)) * 8;
#pragma unroll
                for (int i = 0; i < 4; ++i) r.b[q][i] = *reinterpret_cast<const u32x4*>(pb + (k0 + i) * s3b + n0);
            }
        }
    }

    __device__ static void lstore(u16* stage, const Regs& r) {
        const int tid = threadIdx.x;
        u16* as = stage;
        u16* bs = stage + ABUF;
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int c = tid + q * 256;
            if (c < ACH) {
                const int row = c / (K / 8), col = (c % (K / 8)) * 8;
                *reinterpret_cast<u32x4*>(as + row * AP + col) = r.a[q];
            }
        }
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int blk = tid + q * 256;
            if (blk < BBLK) {
                const int k0 = (blk / (N / 8)) * 4, n0 = (blk % (N / 8)) * 8;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    // words w of rows k0..k0+3 hold columns n0+2w (low half) and n0+2w+1 (high half)
                    const u32 x0 = r.b[q][0][w], x1 = r.b[q][1][w], x2 = r.b[q][2][w], x3 = r.b[q][3][w];
                    u32x2 lo, hi;
                    lo.x = (x0 & 0xFFFFu) | (x1 << 16);
                    lo.y = (x2 & 0xFFFFu) | (x3 << 16);
                    hi.x = (x0 >> 16) | (x1 & 0xFFFF0000u);
                    hi.y = (x2 >> 16) | (x3 & 0xFFFF0000u);
                    *reinterpret_cast<u32x2*>(bs + (n0 + 2 * w) * BP + k0) = lo;
                    *reinterpret_cast<u32x2*>(bs + (n0 + 2 * w + 1) * BP + k0) = hi;
                }
            }
        }
    }

    __device__ static void zero(Acc& a) {
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
            for (int j = 0; j < BJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) a.v[i][j][e] = 0.0f;
    }

    // acc = A_stage x B_stage over the K of one stage, into a zeroed accumulator.
    __device__ static void mma(Acc& acc, const u16* stage) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = wave >> 1, wn = wave & 1;
        const u16* as = stage;
        const u16* bs = stage + ABUF;
        const int r = lane & 31, kh = (lane >> 5) * 8;
#pragma unroll
        for (int kk = 0; kk < K; kk += 16) {
            u32x4 af[BI], bf[BJ];
#pragma unroll
            for (int i = 0; i < BI; ++i)
                af[i] = *reinterpret_cast<const u32x4*>(as + (wm * (M / 2) + i * 32 + r) * AP + kk + kh);
#pragma unroll
            for (int j = 0; j < BJ; ++j)
                bf[j] = *reinterpret_cast<const u32x4*>(bs + (wn * (N / 2) + j * 32 + r) * BP + kk + kh);
#pragma unroll
            for (int i = 0; i < BI; ++i)
#pragma unroll
                for (int j = 0; j < BJ; ++j) acc.v[i][j] = mfma_32x32x16<F16>(af[i], bf[j], acc.v[i][j]);
        }
    }

    // c = c + a, elementwise fp32 (the TADD of the accumulate pattern).
    __device__ static void add(Acc& c, const Acc& a) {
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
            for (int j = 0; j < BJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) c.v[i][j][e] = c.v[i][j][e] + a.v[i][j][e];
    }

    template <bool STORE>
    __device__ static void c_io(Acc& c, float* pc, i64 s3c) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
        for (int i = 0; i < BI; ++i)
#pragma unroll
            for (int j = 0; j < BJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = wm * (M / 2) + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                    const int col = wn * (N / 2) + j * 32 + (lane & 31);
                    if constexpr (STORE) pc[row * s3c + col] = c.v[i][j][e];
                    else c.v[i][j][e] = pc[row * s3c + col];
                }
    }
};

}  // namespace ptowsp
