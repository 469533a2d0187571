// Shared host/device helpers for the gfx950 logic-layer kernels.
//
// Every extern "C" entry point returns a status code (CL_OK on success) and records a
// message for the calling thread; nothing here ever calls exit().  Launches are
// asynchronous on the stream the caller passes.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/compactlogic_hip.h"

namespace cl {

// ---------------------------------------------------------------- error state
void set_error(const char* fmt, ...);
void clear_error();

#define CL_REQUIRE(cond, code, ...)      \
    do {                                 \
        if (!(cond)) {                   \
            ::cl::set_error(__VA_ARGS__); \
            return (code);               \
        }                                \
    } while (0)

#define CL_ARG(cond, ...) CL_REQUIRE(cond, CL_ERR_INVALID_ARGUMENT, __VA_ARGS__)

// Check the launch that was just enqueued.
int check_launch(const char* what);

// Runs the statement block with scalar_t bound to the element type of `dtype`.
#define CL_DTYPE_SWITCH(dtype, ...)                                                     \
    do {                                                                                \
        if ((dtype) == CL_DTYPE_F32) {                                                  \
            using scalar_t = float;                                                     \
            __VA_ARGS__                                                                 \
        } else if ((dtype) == CL_DTYPE_F64) {                                           \
            using scalar_t = double;                                                    \
            __VA_ARGS__                                                                 \
        } else {                                                                        \
            ::cl::set_error("unsupported dtype code %d (expected CL_DTYPE_F32 or F64)", \
                            int(dtype));                                                \
            return CL_ERR_INVALID_ARGUMENT;                                             \
        }                                                                               \
    } while (0)

// As CL_DTYPE_SWITCH, and CL_DTYPE_F16 binds scalar_t to __half (storage only: kernels
// compute in acc_t<scalar_t>).
#define CL_DTYPE_SWITCH_F16(dtype, ...)                                                 \
    do {                                                                                \
        if ((dtype) == CL_DTYPE_F32) {                                                  \
            using scalar_t = float;                                                     \
            __VA_ARGS__                                                                 \
        } else if ((dtype) == CL_DTYPE_F64) {                                           \
            using scalar_t = double;                                                    \
            __VA_ARGS__                                                                 \
        } else if ((dtype) == CL_DTYPE_F16) {                                           \
            using scalar_t = __half;                                                    \
            __VA_ARGS__                                                                 \
        } else {                                                                        \
            ::cl::set_error("unsupported dtype code %d (expected CL_DTYPE_F32, F64 or F16)", \
                            int(dtype));                                                \
            return CL_ERR_INVALID_ARGUMENT;                                             \
        }                                                                               \
    } while (0)

// Arithmetic type of a storage type: half is loaded, summed in fp32 and rounded once on store.
template <typename S>
struct AccType {
    using type = S;
};
template <>
struct AccType<__half> {
    using type = float;
};
template <typename S>
using acc_t = typename AccType<S>::type;

template <typename S>
__device__ __forceinline__ acc_t<S> to_acc(S v) {
    if constexpr (sizeof(S) == 2)
        return __half2float(v);
    else
        return v;
}

template <typename S>
__device__ __forceinline__ S from_acc(acc_t<S> v) {
    if constexpr (sizeof(S) == 2)
        return __float2half_rn(v);
    else
        return v;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Division of x < 2^31 by a fixed d >= 1 as a multiply and a shift (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, round-up method at N = 31):
// with l = ceil(log2 d) and m = ceil(2^(31 + l) / d), which is below 2^32, floor(x / d) =
// floor(x * m / 2^(31 + l)) for every x < 2^31, since m * d - 2^(31 + l) < d <= 2^l.
struct FastDiv {
    uint32_t m;
    uint32_t s;
    uint32_t d;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    const uint64_t num = uint64_t(1) << (31 + l);
    return FastDiv{uint32_t((num + d - 1) / d), 31 + l, d};
}

__device__ __host__ __forceinline__ uint32_t fast_div(uint32_t x, const FastDiv& f) {
    return uint32_t((uint64_t(x) * f.m) >> f.s);
}

// ---------------------------------------------------------------- gate algebra
//
// Opcode g in 0..15 stores its truth table in its four bits, MSB first over the input
// combinations AB = 00, 01, 10, 11 (the table of compactlogic/cuda/utils.cuh:122-139):
//     f(A, B) = (g >> (3 - (2A + B))) & 1.
// The relaxed operator is the unique multilinear interpolation of that table,
//     f(a, b) = c0 + c1*a + c2*b + c3*a*b,
// with c0 = f00, c1 = f10 - f00, c2 = f01 - f00, c3 = f11 - f10 - f01 + f00.
// Its partial derivatives are df/da = c1 + c3*b and df/db = c2 + c3*a.
template <typename T>
struct Coef4 {
    T c0, c1, c2, c3;
};

template <typename T>
__device__ __host__ __forceinline__ Coef4<T> gate_coef(int g) {
    const int f00 = (g >> 3) & 1;
    const int f01 = (g >> 2) & 1;
    const int f10 = (g >> 1) & 1;
    const int f11 = g & 1;
    Coef4<T> c;
    c.c0 = T(f00);
    c.c1 = T(f10 - f00);
    c.c2 = T(f01 - f00);
    c.c3 = T(f11 - f10 - f01 + f00);
    return c;
}

// Relaxed operator value, evaluated as c3*(a*b) + (c2*b + (c1*a + c0)).
template <typename T>
__device__ __forceinline__ T relaxed_op(const Coef4<T>& c, T a, T b) {
    return fma(c.c3, a * b, fma(c.c2, b, fma(c.c1, a, c.c0)));
}

// Bitwise operator on packed words: each output bit selects the truth-table entry for its
// (a, b) bit pair.  Branch-free: four minterm masks.
template <typename W>
__device__ __forceinline__ W bitwise_op(int g, W a, W b) {
    const W m00 = W(0) - W((g >> 3) & 1);
    const W m01 = W(0) - W((g >> 2) & 1);
    const W m10 = W(0) - W((g >> 1) & 1);
    const W m11 = W(0) - W(g & 1);
    return (~a & ~b & m00) | (~a & b & m01) | (a & ~b & m10) | (a & b & m11);
}

// ---------------------------------------------------------------- wave helpers (wave64)
constexpr int kWave = 64;

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// DPP lane permutation of a 32- or 64-bit value (64-bit values move as two halves).
template <int CTRL, typename T>
__device__ __forceinline__ T dpp_move(T v) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(
            T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const int lo = __builtin_amdgcn_update_dpp(0, int(uint32_t(u)), CTRL, 0xF, 0xF, false);
        const int hi = __builtin_amdgcn_update_dpp(0, int(uint32_t(u >> 32)), CTRL, 0xF, 0xF, false);
        return __builtin_bit_cast(T, (uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
    }
}

template <typename T>
__device__ __forceinline__ T read_lane(T v, int lane) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane(int(uint32_t(u)), lane);
        const uint32_t hi = __builtin_amdgcn_readlane(int(uint32_t(u >> 32)), lane);
        return __builtin_bit_cast(T, (uint64_t(hi) << 32) | lo);
    }
}

// Sum over all 64 lanes, returned as a wave-uniform (scalar) value.  Each 16-lane row is
// reduced with DPP (quad swaps 1 and 2, then row rotations by 4 and 8; a full-row rotation
// sum leaves the row total in every lane whatever the rotation direction), and the four row
// totals are added in lane order, so the result does not depend on scheduling.
template <typename T>
__device__ __forceinline__ T wave_total(T v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x124>(v);  // row_ror:4
    v += dpp_move<0x128>(v);  // row_ror:8
    return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}

// Wave index inside the workgroup, as a scalar (uniform) value.
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// ---------------------------------------------------------------- vector access
template <typename T, int VEC>
struct Vec;

template <typename T>
struct Vec<T, 1> {
    T v[1];
};
template <typename T>
struct Vec<T, 2> {
    T v[2];
};
template <typename T>
struct Vec<T, 4> {
    T v[4];
};
template <typename T>
struct Vec<T, 8> {
    T v[8];
};

template <typename T, int VEC>
__device__ __forceinline__ Vec<T, VEC> vload(const T* p) {
    Vec<T, VEC> r;
    if constexpr (VEC == 4 && sizeof(T) == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        r.v[0] = __builtin_bit_cast(T, t.x);
        r.v[1] = __builtin_bit_cast(T, t.y);
        r.v[2] = __builtin_bit_cast(T, t.z);
        r.v[3] = __builtin_bit_cast(T, t.w);
    } else if constexpr (VEC == 2 && sizeof(T) == 8) {
        const double2 t = *reinterpret_cast<const double2*>(p);
        r.v[0] = __builtin_bit_cast(T, t.x);
        r.v[1] = __builtin_bit_cast(T, t.y);
    } else if constexpr (VEC == 8 && sizeof(T) == 2) {
        const uint4 t = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.v[2 * i] = __builtin_bit_cast(T, uint16_t(w[i] & 0xFFFFu));
            r.v[2 * i + 1] = __builtin_bit_cast(T, uint16_t(w[i] >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) r.v[i] = p[i];
    }
    return r;
}

template <typename T, int VEC>
__device__ __forceinline__ void vstore(T* p, const Vec<T, VEC>& r) {
    if constexpr (VEC == 4 && sizeof(T) == 4) {
        float4 t;
        t.x = __builtin_bit_cast(float, r.v[0]);
        t.y = __builtin_bit_cast(float, r.v[1]);
        t.z = __builtin_bit_cast(float, r.v[2]);
        t.w = __builtin_bit_cast(float, r.v[3]);
        *reinterpret_cast<float4*>(p) = t;
    } else if constexpr (VEC == 2 && sizeof(T) == 8) {
        double2 t;
        t.x = __builtin_bit_cast(double, r.v[0]);
        t.y = __builtin_bit_cast(double, r.v[1]);
        *reinterpret_cast<double2*>(p) = t;
    } else if constexpr (VEC == 8 && sizeof(T) == 2) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = uint32_t(__builtin_bit_cast(uint16_t, r.v[2 * i])) |
                   (uint32_t(__builtin_bit_cast(uint16_t, r.v[2 * i + 1])) << 16);
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) p[i] = r.v[i];
    }
}

// Widest vector of T that keeps 16-byte loads, when the row length and base allow it.
template <typename T>
constexpr int wide_vec() {
    return 16 / int(sizeof(T));
}

// Cross-entropy of GroupSum scores given as per-tile class partials of the classifier head
// (the last dense layer's fused forward, dense_tiled.hip): part[(t * 2 + slot) * batch + n] is
// the sum over tile t's rows (tile_rows consecutive rows) of class (t * tile_rows / gsz) + slot.
// Adds them per (sample, class) into `nslices` slices, then the softmax, the loss terms and
// their mean as cl_group_sum_cross_entropy_forward does (groupsum.hip).
int ce_from_tile_partials(int dtype, const void* part, int64_t batch, int64_t features,
                          int64_t k, int64_t tile_rows, double tau, const int64_t* labels,
                          int64_t ignore_index, void* out, void* probs, void* loss, void* count,
                          void* slices, int64_t nslices, void* term, hipStream_t stream);

}  // namespace cl
