// Dense LogicLayer kernels for gfx950.
//
// Layout (as the reference binding, compactlogic/cuda/difflogic_kernel.cu:10-20):
//   x, grad_x: [in_dim, batch]   y, grad_y: [out_dim, batch]   a, b, w, gate_seq: [out_dim, G]
//
// Work decomposition.  One wave64 owns one neuron row (forward / eval / weight gradient) or
// one input row (input gradient) over a chunk of the batch; its lanes stream the batch
// dimension with 16-byte vector accesses, so every row gather is a fully coalesced read of
// contiguous memory.  The per-row metadata (indices, probabilities, opcodes) is wave-uniform
// and read through scalar loads.
//
// Collapsing.  The relaxed operator of opcode s is c0 + c1*a + c2*b + c3*a*b, affine in each
// coefficient, so consecutive slots that share an input pair collapse into one set of four
// coefficients (K = sum_g w_g * c[s_g]).  Each such run then costs two row gathers instead
// of two per slot, and its weight gradient follows from four batch moments
// (sum gy, sum gy*a, sum gy*b, sum gy*a*b).  The entry points over the reference's int64
// indices detect runs on the fly; the *_runs entry points take them from a prebuilt plan.
#include "common.h"

#include <algorithm>
#include <initializer_list>

namespace cl {
namespace {

constexpr int kWaves = 4;  // waves per workgroup (256 threads)

template <typename T>
__device__ __forceinline__ T qnan() {
    return T(__builtin_nan(""));
}

// Collapsed coefficients of the run [g0, g0+len) of one neuron: lane l takes slots
// g0 + l, g0 + l + 64, ..., and the four partial sums are reduced across the wave.  The
// result is wave-uniform.
template <typename T>
__device__ __forceinline__ Coef4<T> run_coef(const T* __restrict__ wrow,
                                             const uint8_t* __restrict__ grow, int g0, int len) {
    T p0 = 0, p1 = 0, p2 = 0, p3 = 0;
    for (int g = g0 + lane_id(); g < g0 + len; g += kWave) {
        const T wg = wrow[g];
        const Coef4<T> c = gate_coef<T>(grow[g]);
        p0 = fma(wg, c.c0, p0);
        p1 = fma(wg, c.c1, p1);
        p2 = fma(wg, c.c2, p2);
        p3 = fma(wg, c.c3, p3);
    }
    Coef4<T> k;
    k.c0 = wave_total(p0);
    k.c1 = wave_total(p1);
    k.c2 = wave_total(p2);
    k.c3 = wave_total(p3);
    return k;
}

template <typename T>
__device__ __forceinline__ Coef4<T> load_coef(const T* __restrict__ kc, int64_t r) {
    Coef4<T> k;
    k.c0 = kc[4 * r + 0];
    k.c1 = kc[4 * r + 1];
    k.c2 = kc[4 * r + 2];
    k.c3 = kc[4 * r + 3];
    return k;
}

// acc += K(xa, xb) over the wave's U vectors of the batch chunk starting at b0.
template <typename T, int VEC, int U>
__device__ __forceinline__ void accum_run(Vec<T, VEC> (&acc)[U], const T* __restrict__ xa,
                                          const T* __restrict__ xb, const Coef4<T>& k, int64_t b0,
                                          int64_t B) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = b0 + int64_t(u) * kWave * VEC;
        if (idx < B) {
            const Vec<T, VEC> va = vload<T, VEC>(xa + idx);
            const Vec<T, VEC> vb = vload<T, VEC>(xb + idx);
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[u].v[i] += relaxed_op(k, va.v[i], vb.v[i]);
        }
    }
}

template <typename T, int VEC, int U>
__device__ __forceinline__ void store_rows(T* __restrict__ yrow, const Vec<T, VEC> (&acc)[U],
                                           int64_t b0, int64_t B, bool poison) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = b0 + int64_t(u) * kWave * VEC;
        if (idx < B) {
            Vec<T, VEC> r = acc[u];
            if (poison) {
#pragma unroll
                for (int i = 0; i < VEC; ++i) r.v[i] = qnan<T>();
            }
            vstore<T, VEC>(yrow + idx, r);
        }
    }
}

// ------------------------------------------------------------------------------------------
// Forward over the reference's int64 indices (runs detected on the fly).
template <typename T, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_forward(const T* __restrict__ x,
                                                       const int64_t* __restrict__ a,
                                                       const int64_t* __restrict__ b,
                                                       const T* __restrict__ w,
                                                       const uint8_t* __restrict__ gs,
                                                       T* __restrict__ y, int64_t in_dim,
                                                       int64_t out_dim, int64_t B, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;
    const int64_t* arow = a + o * G;
    const int64_t* brow = b + o * G;
    const T* wrow = w + o * G;
    const uint8_t* grow = gs + o * G;

    Vec<T, VEC> acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[u].v[i] = T(0);

    bool bad = false;
    int g = 0;
    while (g < G) {
        const int64_t ia = arow[g], ib = brow[g];
        int g1 = g + 1;
        while (g1 < G && arow[g1] == ia && brow[g1] == ib) ++g1;
        if (uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim)) {
            bad = true;
        } else {
            const Coef4<T> k = run_coef(wrow, grow, g, g1 - g);
            accum_run<T, VEC, U>(acc, x + ia * B, x + ib * B, k, b0, B);
        }
        g = g1;
    }
    store_rows<T, VEC, U>(y + o * B, acc, b0, B, bad);
}

// Forward through a run plan.  The run coefficients are also written to `kc` (4 per run)
// when it is given, for the backward pass to reuse.
template <typename T, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_forward_runs(
    const T* __restrict__ x, const T* __restrict__ w, const uint8_t* __restrict__ gs,
    const int32_t* __restrict__ run_ptr, const int2* __restrict__ run_ab,
    const int32_t* __restrict__ run_gl, T* __restrict__ y, T* __restrict__ kc, int64_t in_dim,
    int64_t out_dim, int64_t num_runs, int64_t B, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;
    const T* wrow = w + o * G;
    const uint8_t* grow = gs + o * G;

    Vec<T, VEC> acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[u].v[i] = T(0);

    bool bad = false;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) {
        bad = true;
        r1 = r0;
    }
    for (int64_t r = r0; r < r1; ++r) {
        const int2 ab = run_ab[r];
        const int gl = run_gl[r];
        const int g0 = gl & 0xff, len = gl >> 8;
        if (uint32_t(ab.x) >= uint64_t(in_dim) || uint32_t(ab.y) >= uint64_t(in_dim) ||
            g0 + len > G) {
            bad = true;
            continue;
        }
        const Coef4<T> k = run_coef(wrow, grow, g0, len);
        if (kc != nullptr && blockIdx.y == 0 && lane_id() == 0) {
            kc[4 * r + 0] = k.c0;
            kc[4 * r + 1] = k.c1;
            kc[4 * r + 2] = k.c2;
            kc[4 * r + 3] = k.c3;
        }
        accum_run<T, VEC, U>(acc, x + int64_t(ab.x) * B, x + int64_t(ab.y) * B, k, b0, B);
    }
    store_rows<T, VEC, U>(y + o * B, acc, b0, B, bad);
}

// Run coefficients only (for a backward pass without a preceding forward).
template <typename T>
__global__ __launch_bounds__(256) void k_dense_run_coefs(const T* __restrict__ w,
                                                         const uint8_t* __restrict__ gs,
                                                         const int32_t* __restrict__ run_ptr,
                                                         const int32_t* __restrict__ run_gl,
                                                         T* __restrict__ kc, int64_t out_dim,
                                                         int64_t num_runs, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) return;
    for (int64_t r = r0; r < r1; ++r) {
        const int gl = run_gl[r];
        const int g0 = gl & 0xff, len = gl >> 8;
        Coef4<T> k{qnan<T>(), qnan<T>(), qnan<T>(), qnan<T>()};
        if (g0 + len <= G) k = run_coef(w + o * G, gs + o * G, g0, len);
        if (lane_id() == 0) {
            kc[4 * r + 0] = k.c0;
            kc[4 * r + 1] = k.c1;
            kc[4 * r + 2] = k.c2;
            kc[4 * r + 3] = k.c3;
        }
    }
}

// ------------------------------------------------------------------------------------------
// Batch moments of one run: S1 = sum gy, Sa = sum gy*a, Sb = sum gy*b, Sab = sum gy*a*b over
// the whole batch, reduced across the wave (every lane returns the totals).
template <typename T, int VEC>
__device__ __forceinline__ Coef4<T> run_moments(const T* __restrict__ gyrow,
                                                const T* __restrict__ xa,
                                                const T* __restrict__ xb, int64_t B) {
    T s1 = 0, sa = 0, sb = 0, sab = 0;
    for (int64_t idx = int64_t(lane_id()) * VEC; idx < B; idx += kWave * VEC) {
        const Vec<T, VEC> g = vload<T, VEC>(gyrow + idx);
        const Vec<T, VEC> va = vload<T, VEC>(xa + idx);
        const Vec<T, VEC> vb = vload<T, VEC>(xb + idx);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            s1 += g.v[i];
            const T ga = g.v[i] * va.v[i];
            sa += ga;
            sb = fma(g.v[i], vb.v[i], sb);
            sab = fma(ga, vb.v[i], sab);
        }
    }
    Coef4<T> m;
    m.c0 = wave_total(s1);
    m.c1 = wave_total(sa);
    m.c2 = wave_total(sb);
    m.c3 = wave_total(sab);
    return m;
}

// grad_w[o, g] for g in [g0, g0+len) from the run's moments m = (S1, Sa, Sb, Sab).
template <typename T>
__device__ __forceinline__ void write_run_grad_w(T* __restrict__ gwrow,
                                                 const uint8_t* __restrict__ grow, int g0,
                                                 int len, const Coef4<T>& m, bool poison) {
    for (int g = g0 + lane_id(); g < g0 + len; g += kWave) {
        const Coef4<T> c = gate_coef<T>(grow[g]);
        T v = fma(c.c3, m.c3, fma(c.c2, m.c2, fma(c.c1, m.c1, c.c0 * m.c0)));
        if (poison) v = qnan<T>();
        gwrow[g] = v;
    }
}

// Weight gradient over the reference's int64 indices: one wave per neuron, whole batch.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void k_dense_backward_w(const T* __restrict__ x,
                                                          const int64_t* __restrict__ a,
                                                          const int64_t* __restrict__ b,
                                                          const uint8_t* __restrict__ gs,
                                                          const T* __restrict__ gy,
                                                          T* __restrict__ gw, int64_t in_dim,
                                                          int64_t out_dim, int64_t B, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t* arow = a + o * G;
    const int64_t* brow = b + o * G;
    const uint8_t* grow = gs + o * G;
    int g = 0;
    while (g < G) {
        const int64_t ia = arow[g], ib = brow[g];
        int g1 = g + 1;
        while (g1 < G && arow[g1] == ia && brow[g1] == ib) ++g1;
        const bool bad = uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim);
        Coef4<T> m{T(0), T(0), T(0), T(0)};
        if (!bad) m = run_moments<T, VEC>(gy + o * B, x + ia * B, x + ib * B, B);
        write_run_grad_w<T>(gw + o * G, grow, g, g1 - g, m, bad);
        g = g1;
    }
}

// Weight gradient through a run plan: one wave per neuron, whole batch.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void k_dense_backward_w_runs(
    const T* __restrict__ x, const uint8_t* __restrict__ gs, const T* __restrict__ gy,
    const int32_t* __restrict__ run_ptr, const int2* __restrict__ run_ab,
    const int32_t* __restrict__ run_gl, T* __restrict__ gw, int64_t in_dim, int64_t out_dim,
    int64_t num_runs, int64_t B, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const uint8_t* grow = gs + o * G;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) {
        // Corrupt plan: poison the whole row.
        for (int g = lane_id(); g < G; g += kWave) gw[o * G + g] = qnan<T>();
        return;
    }
    for (int64_t r = r0; r < r1; ++r) {
        const int2 ab = run_ab[r];
        const int gl = run_gl[r];
        const int g0 = gl & 0xff, len = gl >> 8;
        if (g0 + len > G) continue;
        const bool bad = uint32_t(ab.x) >= uint64_t(in_dim) || uint32_t(ab.y) >= uint64_t(in_dim);
        Coef4<T> m{T(0), T(0), T(0), T(0)};
        if (!bad)
            m = run_moments<T, VEC>(gy + o * B, x + int64_t(ab.x) * B, x + int64_t(ab.y) * B, B);
        write_run_grad_w<T>(gw + o * G, grow, g0, len, m, bad);
    }
}

// ------------------------------------------------------------------------------------------
// Input gradient through the reference's inverse index: one wave per input row i over a batch
// chunk; every entry is one (neuron, slot, operand side) use of x_i.
template <typename T, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_backward_x(
    const T* __restrict__ x, const int64_t* __restrict__ a, const int64_t* __restrict__ b,
    const T* __restrict__ w, const uint8_t* __restrict__ gs, const T* __restrict__ gy,
    const int64_t* __restrict__ start, const int64_t* __restrict__ yidx,
    const int8_t* __restrict__ gcode, int64_t num_entries, T* __restrict__ gx, int64_t in_dim,
    int64_t out_dim, int64_t B, int G) {
    const int64_t i = int64_t(blockIdx.x) * kWaves + wave_id();
    if (i >= in_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;

    Vec<T, VEC> acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[u].v[v] = T(0);

    bool bad = false;
    int64_t e0 = start[i], e1 = start[i + 1];
    if (e0 < 0 || e1 < e0 || e1 > num_entries) {
        bad = true;
        e1 = e0;
    }
    for (int64_t e = e0; e < e1; ++e) {
        const int64_t yo = yidx[e];
        const int code = gcode[e];
        const bool side_a = code >= 0;
        const int g = side_a ? code : -code - 1;
        if (uint64_t(yo) >= uint64_t(out_dim) || g >= G) {
            bad = true;
            continue;
        }
        const int64_t other = side_a ? b[yo * G + g] : a[yo * G + g];
        if (uint64_t(other) >= uint64_t(in_dim)) {
            bad = true;
            continue;
        }
        const T wg = w[yo * G + g];
        const Coef4<T> c = gate_coef<T>(gs[yo * G + g]);
        const T kself = side_a ? c.c1 : c.c2;
        const T* xo = x + other * B;
        const T* gyr = gy + yo * B;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = b0 + int64_t(u) * kWave * VEC;
            if (idx < B) {
                const Vec<T, VEC> vo = vload<T, VEC>(xo + idx);
                const Vec<T, VEC> vg = vload<T, VEC>(gyr + idx);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const T dydx = wg * fma(c.c3, vo.v[v], kself);
                    acc[u].v[v] = fma(dydx, vg.v[v], acc[u].v[v]);
                }
            }
        }
    }
    store_rows<T, VEC, U>(gx + i * B, acc, b0, B, bad);
}

// Input gradient (and, with WANT_GW, the weight gradient) through the run plan's inverse
// index, reading the run coefficients K written by the forward pass.
//
// WPR waves share one input row and split its batch (WPR = 1: four rows per workgroup).
// With WANT_GW the workgroup covers the whole batch (gridDim.y == 1): the weight moments of
// run r are reduced at its operand-a entry, which lives in exactly one row, so every weight
// gradient is written exactly once and no atomics are needed.  With WPR > 1 the per-wave
// partial moments meet in LDS and are added in wave order.
constexpr int kPendingRuns = 16;

template <typename T, int VEC, int U, int WPR, bool WANT_GX, bool WANT_GW>
__global__ __launch_bounds__(256) void k_dense_backward_runs(
    const T* __restrict__ x, const T* __restrict__ kc, const uint8_t* __restrict__ gs,
    const T* __restrict__ gy, const int2* __restrict__ run_ab, const int32_t* __restrict__ run_gl,
    const int32_t* __restrict__ run_y, const int32_t* __restrict__ inv_ptr,
    const int32_t* __restrict__ inv_entry, T* __restrict__ gx, T* __restrict__ gw, int64_t in_dim,
    int64_t out_dim, int64_t num_runs, int64_t B, int G) {
    static_assert(kWaves % WPR == 0, "waves per row must divide the workgroup");
    constexpr int kRowsPerBlock = kWaves / WPR;
    constexpr bool kShared = WANT_GW && WPR > 1;
    __shared__ T mom[kShared ? kPendingRuns : 1][WPR][4];
    __shared__ int pend[kShared ? kPendingRuns : 1][2];

    const int wave = wave_id();
    const int part = wave % WPR;
    const int64_t i = int64_t(blockIdx.x) * kRowsPerBlock + wave / WPR;
    if (i >= in_dim) return;  // uniform across the workgroup when WPR == kWaves
    // batch element of unroll step u: ((u * WPR + part) * 64 + lane) * VEC, within chunk y
    const int64_t chunk0 = int64_t(blockIdx.y) * (int64_t(WPR) * kWave * VEC * U);
    auto elem = [&](int u) -> int64_t {
        return chunk0 + (int64_t(u) * WPR + part) * (kWave * VEC) + int64_t(lane_id()) * VEC;
    };
    const T* xi = x + i * B;

    Vec<T, VEC> acc[U];
    Vec<T, VEC> self[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
            acc[u].v[v] = T(0);
            self[u].v[v] = T(0);
        }
        if (WANT_GW) {
            const int64_t idx = elem(u);
            if (idx < B) self[u] = vload<T, VEC>(xi + idx);
        }
    }

    int npend = 0;
    auto flush = [&](int n) {
        for (int j = wave; j < n; j += kWaves) {
            Coef4<T> m;
            m.c0 = mom[j][0][0];
            m.c1 = mom[j][0][1];
            m.c2 = mom[j][0][2];
            m.c3 = mom[j][0][3];
            for (int q = 1; q < WPR; ++q) {
                m.c0 += mom[j][q][0];
                m.c1 += mom[j][q][1];
                m.c2 += mom[j][q][2];
                m.c3 += mom[j][q][3];
            }
            const int64_t yo = pend[j][0];
            const int gl = pend[j][1];
            write_run_grad_w<T>(gw + yo * G, gs + yo * G, gl & 0xff, gl >> 8, m, false);
        }
    };

    bool bad = false;
    int64_t e0 = inv_ptr[i], e1 = inv_ptr[i + 1];
    if (e0 < 0 || e1 < e0 || e1 > 2 * num_runs) {
        bad = true;
        e1 = e0;
    }
    for (int64_t e = e0; e < e1; ++e) {
        const int ent = inv_entry[e];
        const int64_t r = ent >> 1;
        const int side = ent & 1;
        if (r >= num_runs || ent < 0) {
            bad = true;
            continue;
        }
        const int64_t yo = run_y[r];
        const int2 ab = run_ab[r];
        const int gl = run_gl[r];
        const int64_t other = side ? ab.x : ab.y;
        if (uint64_t(yo) >= uint64_t(out_dim) || uint64_t(other) >= uint64_t(in_dim) ||
            (gl & 0xff) + (gl >> 8) > G) {
            bad = true;
            continue;
        }
        const Coef4<T> k = load_coef(kc, r);
        const T kself = side ? k.c2 : k.c1;
        const T* xo = x + other * B;
        const T* gyr = gy + yo * B;
        const bool moments = WANT_GW && side == 0;
        T s1 = 0, sa = 0, sb = 0, sab = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = elem(u);
            if (idx < B) {
                const Vec<T, VEC> vo = vload<T, VEC>(xo + idx);
                const Vec<T, VEC> vg = vload<T, VEC>(gyr + idx);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    if (WANT_GX) acc[u].v[v] = fma(fma(k.c3, vo.v[v], kself), vg.v[v], acc[u].v[v]);
                    if (moments) {
                        const T ga = vg.v[v] * self[u].v[v];
                        s1 += vg.v[v];
                        sa += ga;
                        sb = fma(vg.v[v], vo.v[v], sb);
                        sab = fma(ga, vo.v[v], sab);
                    }
                }
            }
        }
        if (moments) {
            Coef4<T> m;
            m.c0 = wave_total(s1);
            m.c1 = wave_total(sa);
            m.c2 = wave_total(sb);
            m.c3 = wave_total(sab);
            if constexpr (kShared) {
                if (lane_id() == 0) {
                    mom[npend][part][0] = m.c0;
                    mom[npend][part][1] = m.c1;
                    mom[npend][part][2] = m.c2;
                    mom[npend][part][3] = m.c3;
                    if (part == 0) {
                        pend[npend][0] = int(yo);
                        pend[npend][1] = gl;
                    }
                }
                if (++npend == kPendingRuns) {
                    __syncthreads();
                    flush(npend);
                    __syncthreads();
                    npend = 0;
                }
            } else {
                write_run_grad_w<T>(gw + yo * G, gs + yo * G, gl & 0xff, gl >> 8, m, false);
            }
        }
    }
    if constexpr (kShared) {
        __syncthreads();
        flush(npend);
    }
    if (WANT_GX) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = elem(u);
            if (idx < B) {
                Vec<T, VEC> r = acc[u];
                if (bad) {
#pragma unroll
                    for (int v = 0; v < VEC; ++v) r.v[v] = qnan<T>();
                }
                vstore<T, VEC>(gx + i * B + idx, r);
            }
        }
    }
}

// Discrete forward with the argmax slot, relaxed formula (exact on {0, 1} inputs).
template <typename T, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_eval(const T* __restrict__ x,
                                                    const int64_t* __restrict__ a,
                                                    const int64_t* __restrict__ b,
                                                    const uint8_t* __restrict__ wslot,
                                                    const uint8_t* __restrict__ gs,
                                                    T* __restrict__ y, int64_t in_dim,
                                                    int64_t out_dim, int64_t B, int G) {
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;
    const int s = wslot[o];
    bool bad = s >= G;
    int64_t ia = 0, ib = 0;
    Coef4<T> c{T(0), T(0), T(0), T(0)};
    if (!bad) {
        ia = a[o * G + s];
        ib = b[o * G + s];
        c = gate_coef<T>(gs[o * G + s]);
        bad = uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim);
    }
    Vec<T, VEC> acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[u].v[v] = T(0);
    if (!bad) accum_run<T, VEC, U>(acc, x + ia * B, x + ib * B, c, b0, B);
    store_rows<T, VEC, U>(y + o * B, acc, b0, B, bad);
}

// ------------------------------------------------------------------------------------------
// Host side.

// Per-lane vector width: 16-byte accesses when every row start stays aligned.
template <typename T>
int pick_vec(int64_t B, std::initializer_list<const void*> ptrs) {
    const int wide = wide_vec<T>();
    if (B % wide != 0) return 1;
    for (const void* p : ptrs)
        if (p && !aligned(p, 16)) return 1;
    return wide;
}

constexpr int kChunkUnroll = 4;
#ifndef CL_FWD_UNROLL
#define CL_FWD_UNROLL 2
#endif
#ifndef CL_FUSED_WPR
#define CL_FUSED_WPR 4
#endif
constexpr int kFwdUnroll = CL_FWD_UNROLL;      // 16-byte vectors per lane in the plan forward
constexpr int kFusedWpr = CL_FUSED_WPR;        // waves sharing one row in the fused backward
constexpr int kFusedMaxUnroll = 8;

inline dim3 rows_grid(int64_t rows, int64_t B, int vec, int unroll) {
    const int64_t chunk = int64_t(kWave) * vec * unroll;
    const int64_t gy = B == 0 ? 1 : ceil_div(B, chunk);
    return dim3(unsigned(ceil_div(rows, kWaves)), unsigned(gy), 1);
}

int check_dims(int64_t in_dim, int64_t out_dim, int64_t B, int64_t G) {
    CL_ARG(in_dim >= 0 && out_dim >= 0 && B >= 0, "negative dimension (in=%lld out=%lld batch=%lld)",
           (long long)in_dim, (long long)out_dim, (long long)B);
    CL_ARG(G >= 1 && G <= 128, "num_gates must be in [1, 128], got %lld", (long long)G);
    CL_ARG(ceil_div(std::max<int64_t>(in_dim, out_dim), kWaves) < (int64_t(1) << 31),
           "too many rows for one launch");
    return CL_OK;
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_dense_forward(int dtype, const void* x, const int64_t* a, const int64_t* b,
                                const void* w, const uint8_t* gate_seq, void* y, int64_t in_dim,
                                int64_t out_dim, int64_t batch, int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (out_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && a && b && w && gate_seq && y, "null pointer argument");
    CL_DTYPE_SWITCH(dtype, {
        const int vec = pick_vec<scalar_t>(batch, {x, y});
        const dim3 grid = rows_grid(out_dim, batch, vec, kChunkUnroll);
        auto* xs = static_cast<const scalar_t*>(x);
        auto* ws = static_cast<const scalar_t*>(w);
        auto* ys = static_cast<scalar_t*>(y);
        if (vec == wide_vec<scalar_t>())
            k_dense_forward<scalar_t, wide_vec<scalar_t>(), kChunkUnroll>
                <<<grid, 256, 0, as_stream(stream)>>>(xs, a, b, ws, gate_seq, ys, in_dim, out_dim,
                                                     batch, int(num_gates));
        else
            k_dense_forward<scalar_t, 1, kChunkUnroll><<<grid, 256, 0, as_stream(stream)>>>(
                xs, a, b, ws, gate_seq, ys, in_dim, out_dim, batch, int(num_gates));
    });
    return check_launch("cl_dense_forward");
}

extern "C" int cl_dense_forward_runs(int dtype, const void* x, const void* w,
                                     const uint8_t* gate_seq, const int32_t* run_ptr,
                                     const int32_t* run_ab, const int32_t* run_gl, void* y,
                                     void* run_coef, int64_t in_dim, int64_t out_dim,
                                     int64_t num_runs, int64_t batch, int64_t num_gates,
                                     void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (out_dim == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(w && gate_seq && run_ptr && run_ab && run_gl, "null pointer argument");
    CL_ARG(batch == 0 || (x && y), "null pointer argument");
    CL_ARG(aligned(run_ab, 8), "run_ab must be 8-byte aligned");
    const int64_t b_launch = std::max<int64_t>(batch, 1);  // batch 0 still fills run_coef
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        constexpr int W = wide_vec<T>();
        const int vec = pick_vec<T>(batch, {x, y});
        auto* xs = static_cast<const T*>(x);
        auto* ws = static_cast<const T*>(w);
        auto* ys = static_cast<T*>(y);
        auto* kc = static_cast<T*>(run_coef);
        auto* ab = reinterpret_cast<const int2*>(run_ab);
        hipStream_t s = as_stream(stream);
        if (batch == 0) {
            if (kc)
                k_dense_run_coefs<T><<<dim3(unsigned(ceil_div(out_dim, kWaves))), 256, 0, s>>>(
                    ws, gate_seq, run_ptr, run_gl, kc, out_dim, num_runs, int(num_gates));
        } else if (vec == W) {
            const dim3 grid = rows_grid(out_dim, b_launch, W, kFwdUnroll);
            k_dense_forward_runs<T, W, kFwdUnroll><<<grid, 256, 0, s>>>(
                xs, ws, gate_seq, run_ptr, ab, run_gl, ys, kc, in_dim, out_dim, num_runs, batch,
                int(num_gates));
        } else {
            const dim3 grid = rows_grid(out_dim, b_launch, 1, kChunkUnroll);
            k_dense_forward_runs<T, 1, kChunkUnroll><<<grid, 256, 0, s>>>(
                xs, ws, gate_seq, run_ptr, ab, run_gl, ys, kc, in_dim, out_dim, num_runs, batch,
                int(num_gates));
        }
    });
    return check_launch("cl_dense_forward_runs");
}

extern "C" int cl_dense_run_coefs(int dtype, const void* w, const uint8_t* gate_seq,
                                  const int32_t* run_ptr, const int32_t* run_gl, void* run_coef,
                                  int64_t out_dim, int64_t num_runs, int64_t num_gates,
                                  void* stream) {
    clear_error();
    CL_ARG(out_dim >= 0 && num_runs >= 0, "negative shape");
    CL_ARG(num_gates >= 1 && num_gates <= 128, "num_gates must be in [1, 128]");
    if (out_dim == 0) return CL_OK;
    CL_ARG(w && gate_seq && run_ptr && run_gl && run_coef, "null pointer argument");
    CL_DTYPE_SWITCH(dtype, {
        k_dense_run_coefs<scalar_t><<<dim3(unsigned(ceil_div(out_dim, kWaves))), 256, 0,
                                      as_stream(stream)>>>(
            static_cast<const scalar_t*>(w), gate_seq, run_ptr, run_gl,
            static_cast<scalar_t*>(run_coef), out_dim, num_runs, int(num_gates));
    });
    return check_launch("cl_dense_run_coefs");
}

extern "C" int cl_dense_backward_w(int dtype, const void* x, const int64_t* a, const int64_t* b,
                                   const uint8_t* gate_seq, const void* grad_y, void* grad_w,
                                   int64_t in_dim, int64_t out_dim, int64_t batch,
                                   int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (out_dim == 0) return CL_OK;
    CL_ARG(a && b && gate_seq && grad_w, "null pointer argument");
    CL_ARG(batch == 0 || (x && grad_y), "null pointer argument");
    CL_ARG(in_dim > 0 || batch == 0, "in_dim is 0 but out_dim > 0");
    CL_DTYPE_SWITCH(dtype, {
        const int vec = pick_vec<scalar_t>(batch, {x, grad_y});
        const dim3 grid(unsigned(ceil_div(out_dim, kWaves)), 1, 1);
        auto* xs = static_cast<const scalar_t*>(x);
        auto* gys = static_cast<const scalar_t*>(grad_y);
        auto* gws = static_cast<scalar_t*>(grad_w);
        if (vec == wide_vec<scalar_t>())
            k_dense_backward_w<scalar_t, wide_vec<scalar_t>()><<<grid, 256, 0, as_stream(stream)>>>(
                xs, a, b, gate_seq, gys, gws, std::max<int64_t>(in_dim, 1), out_dim, batch,
                int(num_gates));
        else
            k_dense_backward_w<scalar_t, 1><<<grid, 256, 0, as_stream(stream)>>>(
                xs, a, b, gate_seq, gys, gws, std::max<int64_t>(in_dim, 1), out_dim, batch,
                int(num_gates));
    });
    return check_launch("cl_dense_backward_w");
}

extern "C" int cl_dense_backward_x(int dtype, const void* x, const int64_t* a, const int64_t* b,
                                   const void* w, const uint8_t* gate_seq, const void* grad_y,
                                   const int64_t* start, const int64_t* y_index,
                                   const int8_t* gate_code, int64_t num_entries, void* grad_x,
                                   int64_t in_dim, int64_t out_dim, int64_t batch,
                                   int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (in_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(num_entries >= 0, "negative num_entries");
    CL_ARG(x && a && b && w && gate_seq && grad_y && start && grad_x, "null pointer argument");
    CL_ARG(num_entries == 0 || (y_index && gate_code), "null inverse-index pointer");
    CL_DTYPE_SWITCH(dtype, {
        const int vec = pick_vec<scalar_t>(batch, {x, grad_y, grad_x});
        const dim3 grid = rows_grid(in_dim, batch, vec, kChunkUnroll);
        auto* xs = static_cast<const scalar_t*>(x);
        auto* ws = static_cast<const scalar_t*>(w);
        auto* gys = static_cast<const scalar_t*>(grad_y);
        auto* gxs = static_cast<scalar_t*>(grad_x);
        if (vec == wide_vec<scalar_t>())
            k_dense_backward_x<scalar_t, wide_vec<scalar_t>(), kChunkUnroll>
                <<<grid, 256, 0, as_stream(stream)>>>(xs, a, b, ws, gate_seq, gys, start, y_index,
                                                     gate_code, num_entries, gxs, in_dim, out_dim,
                                                     batch, int(num_gates));
        else
            k_dense_backward_x<scalar_t, 1, kChunkUnroll><<<grid, 256, 0, as_stream(stream)>>>(
                xs, a, b, ws, gate_seq, gys, start, y_index, gate_code, num_entries, gxs, in_dim,
                out_dim, batch, int(num_gates));
    });
    return check_launch("cl_dense_backward_x");
}

namespace cl {
namespace {

// The fused input + weight gradient kernel splits each row's batch over kFusedWpr waves and
// covers up to kFusedMaxUnroll vectors per lane.
template <typename T>
constexpr int64_t fused_max_batch() {
    return int64_t(kFusedWpr) * kWave * wide_vec<T>() * kFusedMaxUnroll;
}

template <typename T, int U>
void launch_fused(const T* x, const T* kc, const uint8_t* gs, const T* gy, const int2* ab,
                  const int32_t* gl, const int32_t* ry, const int32_t* ip, const int32_t* ie, T* gx,
                  T* gw, int64_t in_dim, int64_t out_dim, int64_t R, int64_t B, int G,
                  hipStream_t s) {
    constexpr int W = wide_vec<T>();
    const dim3 grid(unsigned(ceil_div(in_dim, kWaves / kFusedWpr)), 1, 1);
    k_dense_backward_runs<T, W, U, kFusedWpr, true, true>
        <<<grid, 256, 0, s>>>(x, kc, gs, gy, ab, gl, ry, ip, ie, gx, gw, in_dim, out_dim, R, B, G);
}

}  // namespace
}  // namespace cl

extern "C" int cl_dense_backward_runs(int dtype, const void* x, const void* run_coef,
                                      const uint8_t* gate_seq, const void* grad_y,
                                      const int32_t* run_ptr, const int32_t* run_ab,
                                      const int32_t* run_gl, const int32_t* run_y,
                                      const int32_t* inv_ptr, const int32_t* inv_entry,
                                      void* grad_x, void* grad_w, int64_t in_dim, int64_t out_dim,
                                      int64_t num_runs, int64_t batch, int64_t num_gates,
                                      void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    CL_ARG(num_runs >= 0 && num_runs < (int64_t(1) << 30), "num_runs out of range");
    if (!grad_x && !grad_w) return CL_OK;
    if (out_dim == 0 && (in_dim == 0 || batch == 0 || !grad_x)) return CL_OK;
    CL_ARG(gate_seq && run_ptr && run_ab && run_gl, "null pointer argument");
    CL_ARG(batch == 0 || (x && grad_y), "null pointer argument");
    CL_ARG(aligned(run_ab, 8), "run_ab must be 8-byte aligned");
    if (grad_x)
        CL_ARG(run_coef && run_y && inv_ptr && inv_entry,
               "grad_x needs run_coef, run_y, inv_ptr and inv_entry");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        auto* xs = static_cast<const T*>(x);
        auto* kc = static_cast<const T*>(run_coef);
        auto* gys = static_cast<const T*>(grad_y);
        auto* gxs = static_cast<T*>(grad_x);
        auto* gws = static_cast<T*>(grad_w);
        auto* ab = reinterpret_cast<const int2*>(run_ab);
        const int G = int(num_gates);
        const int vec = pick_vec<T>(batch, {x, grad_y, grad_x});
        constexpr int W = wide_vec<T>();
        const bool fuse = grad_x && grad_w && vec == W && batch > 0 &&
                          batch <= fused_max_batch<T>() && in_dim > 0;
        if (fuse) {
            const int64_t per_unroll = int64_t(kFusedWpr) * kWave * W;
            const int64_t U = ceil_div(batch, per_unroll);
            if (U <= 1)
                launch_fused<T, 1>(xs, kc, gate_seq, gys, ab, run_gl, run_y, inv_ptr, inv_entry,
                                   gxs, gws, in_dim, out_dim, num_runs, batch, G, s);
            else if (U <= 2)
                launch_fused<T, 2>(xs, kc, gate_seq, gys, ab, run_gl, run_y, inv_ptr, inv_entry,
                                   gxs, gws, in_dim, out_dim, num_runs, batch, G, s);
            else if (U <= 4)
                launch_fused<T, 4>(xs, kc, gate_seq, gys, ab, run_gl, run_y, inv_ptr, inv_entry,
                                   gxs, gws, in_dim, out_dim, num_runs, batch, G, s);
            else
                launch_fused<T, kFusedMaxUnroll>(xs, kc, gate_seq, gys, ab, run_gl, run_y,
                                                 inv_ptr, inv_entry, gxs, gws, in_dim, out_dim,
                                                 num_runs, batch, G, s);
        } else {
            if (grad_x && in_dim > 0 && batch > 0) {
                const dim3 grid = rows_grid(in_dim, batch, vec, kChunkUnroll);
                if (vec == W)
                    k_dense_backward_runs<T, W, kChunkUnroll, 1, true, false><<<grid, 256, 0, s>>>(
                        xs, kc, gate_seq, gys, ab, run_gl, run_y, inv_ptr, inv_entry, gxs, nullptr,
                        in_dim, out_dim, num_runs, batch, G);
                else
                    k_dense_backward_runs<T, 1, kChunkUnroll, 1, true, false><<<grid, 256, 0, s>>>(
                        xs, kc, gate_seq, gys, ab, run_gl, run_y, inv_ptr, inv_entry, gxs, nullptr,
                        in_dim, out_dim, num_runs, batch, G);
                if (int rc = check_launch("cl_dense_backward_runs(grad_x)")) return rc;
            }
            if (grad_w && out_dim > 0) {
                const int vw = pick_vec<T>(batch, {x, grad_y});
                const dim3 grid(unsigned(ceil_div(out_dim, kWaves)), 1, 1);
                const int64_t ind = std::max<int64_t>(in_dim, 1);
                if (vw == W)
                    k_dense_backward_w_runs<T, W><<<grid, 256, 0, s>>>(
                        xs, gate_seq, gys, run_ptr, ab, run_gl, gws, ind, out_dim, num_runs, batch, G);
                else
                    k_dense_backward_w_runs<T, 1><<<grid, 256, 0, s>>>(
                        xs, gate_seq, gys, run_ptr, ab, run_gl, gws, ind, out_dim, num_runs, batch, G);
            }
        }
    });
    return check_launch("cl_dense_backward_runs");
}

extern "C" int cl_dense_eval(int dtype, const void* x, const int64_t* a, const int64_t* b,
                             const uint8_t* w_slot, const uint8_t* gate_seq, void* y,
                             int64_t in_dim, int64_t out_dim, int64_t batch, int64_t num_gates,
                             void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (out_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && a && b && w_slot && gate_seq && y, "null pointer argument");
    CL_DTYPE_SWITCH(dtype, {
        const int vec = pick_vec<scalar_t>(batch, {x, y});
        const dim3 grid = rows_grid(out_dim, batch, vec, kChunkUnroll);
        auto* xs = static_cast<const scalar_t*>(x);
        auto* ys = static_cast<scalar_t*>(y);
        if (vec == wide_vec<scalar_t>())
            k_dense_eval<scalar_t, wide_vec<scalar_t>(), kChunkUnroll>
                <<<grid, 256, 0, as_stream(stream)>>>(xs, a, b, w_slot, gate_seq, ys, in_dim,
                                                     out_dim, batch, int(num_gates));
        else
            k_dense_eval<scalar_t, 1, kChunkUnroll><<<grid, 256, 0, as_stream(stream)>>>(
                xs, a, b, w_slot, gate_seq, ys, in_dim, out_dim, batch, int(num_gates));
    });
    return check_launch("cl_dense_eval");
}
