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

template <int NV, int VW, int G>
__device__ inline void row_load(RowSlice<NV, VW>& r, const float* p, i64 s4, int j) {
    if constexpr (VW == 4) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const float4 x = *reinterpret_cast<const float4*>(p + (k * G + j) * 4);
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

template <int NV, int VW, int G>
__device__ inline void row_store(float* p, const RowSlice<NV, VW>& r, i64 s4, int j) {
    if constexpr (VW == 4) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
            *reinterpret_cast<float4*>(p + (k * G + j) * 4) =
                make_float4(r.v[k * 4 + 0], r.v[k * 4 + 1], r.v[k * 4 + 2], r.v[k * 4 + 3]);
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

}  // namespace ptowsp
