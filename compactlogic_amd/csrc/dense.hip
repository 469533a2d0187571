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
// (sum gy, sum gy*a, sum gy*b, sum gy*a*b).  These entry points take the reference's int64
// indices and detect runs on the fly; the module's training path (dense_tiled.hip) takes
// them from a prebuilt plan.
#include "common.h"

#include <algorithm>
#include <initializer_list>

namespace cl {
namespace {

constexpr int kWaves = 4;  // waves per workgroup (256 threads)

// Storage type S (float, double or __half) and arithmetic type A = acc_t<S>: half rows are
// widened on load, summed in fp32 and rounded once on store.
template <typename S>
__device__ __forceinline__ S qnan() {
    return from_acc<S>(acc_t<S>(__builtin_nan("")));
}

// Collapsed coefficients of the run [g0, g0+len) of one neuron: lane l takes slots
// g0 + l, g0 + l + 64, ..., and the four partial sums are reduced across the wave.  The
// result is wave-uniform.
template <typename S>
__device__ __forceinline__ Coef4<acc_t<S>> run_coef(const S* __restrict__ wrow,
                                                    const uint8_t* __restrict__ grow, int g0,
                                                    int len) {
    using A = acc_t<S>;
    A p0 = 0, p1 = 0, p2 = 0, p3 = 0;
    for (int g = g0 + lane_id(); g < g0 + len; g += kWave) {
        const A wg = to_acc(wrow[g]);
        const Coef4<A> c = gate_coef<A>(grow[g]);
        p0 = fma(wg, c.c0, p0);
        p1 = fma(wg, c.c1, p1);
        p2 = fma(wg, c.c2, p2);
        p3 = fma(wg, c.c3, p3);
    }
    Coef4<A> k;
    k.c0 = wave_total(p0);
    k.c1 = wave_total(p1);
    k.c2 = wave_total(p2);
    k.c3 = wave_total(p3);
    return k;
}

// acc += K(xa, xb) over the wave's U vectors of the batch chunk starting at b0.
template <typename S, int VEC, int U>
__device__ __forceinline__ void accum_run(Vec<acc_t<S>, VEC> (&acc)[U], const S* __restrict__ xa,
                                          const S* __restrict__ xb, const Coef4<acc_t<S>>& k,
                                          int64_t b0, int64_t B) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = b0 + int64_t(u) * kWave * VEC;
        if (idx < B) {
            const Vec<S, VEC> va = vload<S, VEC>(xa + idx);
            const Vec<S, VEC> vb = vload<S, VEC>(xb + idx);
#pragma unroll
            for (int i = 0; i < VEC; ++i)
                acc[u].v[i] += relaxed_op(k, to_acc(va.v[i]), to_acc(vb.v[i]));
        }
    }
}

template <typename S, int VEC, int U>
__device__ __forceinline__ void store_rows(S* __restrict__ yrow,
                                           const Vec<acc_t<S>, VEC> (&acc)[U], int64_t b0,
                                           int64_t B, bool poison) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = b0 + int64_t(u) * kWave * VEC;
        if (idx < B) {
            Vec<S, VEC> r;
#pragma unroll
            for (int i = 0; i < VEC; ++i) r.v[i] = poison ? qnan<S>() : from_acc<S>(acc[u].v[i]);
            vstore<S, VEC>(yrow + idx, r);
        }
    }
}

template <typename A, int VEC, int U>
__device__ __forceinline__ void zero_acc(Vec<A, VEC> (&acc)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[u].v[i] = A(0);
}

// ------------------------------------------------------------------------------------------
// Forward over the reference's int64 indices (runs detected on the fly).
template <typename S, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_forward(const S* __restrict__ x,
                                                       const int64_t* __restrict__ a,
                                                       const int64_t* __restrict__ b,
                                                       const S* __restrict__ w,
                                                       const uint8_t* __restrict__ gs,
                                                       S* __restrict__ y, int64_t in_dim,
                                                       int64_t out_dim, int64_t B, int G) {
    using A = acc_t<S>;
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;
    const int64_t* arow = a + o * G;
    const int64_t* brow = b + o * G;
    const S* wrow = w + o * G;
    const uint8_t* grow = gs + o * G;

    Vec<A, VEC> acc[U];
    zero_acc(acc);
    bool bad = false;
    int g = 0;
    while (g < G) {
        const int64_t ia = arow[g], ib = brow[g];
        int g1 = g + 1;
        while (g1 < G && arow[g1] == ia && brow[g1] == ib) ++g1;
        if (uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim)) {
            bad = true;
        } else {
            const Coef4<A> k = run_coef(wrow, grow, g, g1 - g);
            accum_run<S, VEC, U>(acc, x + ia * B, x + ib * B, k, b0, B);
        }
        g = g1;
    }
    store_rows<S, VEC, U>(y + o * B, acc, b0, B, bad);
}

// ------------------------------------------------------------------------------------------
// Batch moments of one run: S1 = sum gy, Sa = sum gy*a, Sb = sum gy*b, Sab = sum gy*a*b over
// the whole batch, reduced across the wave (every lane returns the totals).
template <typename S, int VEC>
__device__ __forceinline__ Coef4<acc_t<S>> run_moments(const S* __restrict__ gyrow,
                                                       const S* __restrict__ xa,
                                                       const S* __restrict__ xb, int64_t B) {
    using A = acc_t<S>;
    A s1 = 0, sa = 0, sb = 0, sab = 0;
    for (int64_t idx = int64_t(lane_id()) * VEC; idx < B; idx += kWave * VEC) {
        const Vec<S, VEC> g = vload<S, VEC>(gyrow + idx);
        const Vec<S, VEC> va = vload<S, VEC>(xa + idx);
        const Vec<S, VEC> vb = vload<S, VEC>(xb + idx);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const A gi = to_acc(g.v[i]), ai = to_acc(va.v[i]), bi = to_acc(vb.v[i]);
            s1 += gi;
            const A ga = gi * ai;
            sa += ga;
            sb = fma(gi, bi, sb);
            sab = fma(ga, bi, sab);
        }
    }
    Coef4<A> m;
    m.c0 = wave_total(s1);
    m.c1 = wave_total(sa);
    m.c2 = wave_total(sb);
    m.c3 = wave_total(sab);
    return m;
}

// grad_w[o, g] for g in [g0, g0+len) from the run's moments m = (S1, Sa, Sb, Sab).
template <typename S>
__device__ __forceinline__ void write_run_grad_w(S* __restrict__ gwrow,
                                                 const uint8_t* __restrict__ grow, int g0,
                                                 int len, const Coef4<acc_t<S>>& m, bool poison) {
    using A = acc_t<S>;
    for (int g = g0 + lane_id(); g < g0 + len; g += kWave) {
        const Coef4<A> c = gate_coef<A>(grow[g]);
        const A v = fma(c.c3, m.c3, fma(c.c2, m.c2, fma(c.c1, m.c1, c.c0 * m.c0)));
        gwrow[g] = poison ? qnan<S>() : from_acc<S>(v);
    }
}

// Weight gradient over the reference's int64 indices: one wave per neuron, whole batch.
template <typename S, int VEC>
__global__ __launch_bounds__(256) void k_dense_backward_w(const S* __restrict__ x,
                                                          const int64_t* __restrict__ a,
                                                          const int64_t* __restrict__ b,
                                                          const uint8_t* __restrict__ gs,
                                                          const S* __restrict__ gy,
                                                          S* __restrict__ gw, int64_t in_dim,
                                                          int64_t out_dim, int64_t B, int G) {
    using A = acc_t<S>;
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
        Coef4<A> m{A(0), A(0), A(0), A(0)};
        if (!bad) m = run_moments<S, VEC>(gy + o * B, x + ia * B, x + ib * B, B);
        write_run_grad_w<S>(gw + o * G, grow, g, g1 - g, m, bad);
        g = g1;
    }
}

// ------------------------------------------------------------------------------------------
// Input gradient through the reference's inverse index: one wave per input row i over a batch
// chunk; every entry is one (neuron, slot, operand side) use of x_i.
template <typename S, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_backward_x(
    const S* __restrict__ x, const int64_t* __restrict__ a, const int64_t* __restrict__ b,
    const S* __restrict__ w, const uint8_t* __restrict__ gs, const S* __restrict__ gy,
    const int64_t* __restrict__ start, const int64_t* __restrict__ yidx,
    const int8_t* __restrict__ gcode, int64_t num_entries, S* __restrict__ gx, int64_t in_dim,
    int64_t out_dim, int64_t B, int G) {
    using A = acc_t<S>;
    const int64_t i = int64_t(blockIdx.x) * kWaves + wave_id();
    if (i >= in_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;

    Vec<A, VEC> acc[U];
    zero_acc(acc);
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
        const A wg = to_acc(w[yo * G + g]);
        const Coef4<A> c = gate_coef<A>(gs[yo * G + g]);
        const A kself = side_a ? c.c1 : c.c2;
        const S* xo = x + other * B;
        const S* gyr = gy + yo * B;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = b0 + int64_t(u) * kWave * VEC;
            if (idx < B) {
                const Vec<S, VEC> vo = vload<S, VEC>(xo + idx);
                const Vec<S, VEC> vg = vload<S, VEC>(gyr + idx);
#pragma unroll
                for (int v = 0; v < VEC; ++v) {
                    const A dydx = wg * fma(c.c3, to_acc(vo.v[v]), kself);
                    acc[u].v[v] = fma(dydx, to_acc(vg.v[v]), acc[u].v[v]);
                }
            }
        }
    }
    store_rows<S, VEC, U>(gx + i * B, acc, b0, B, bad);
}

// Discrete forward with the argmax slot, relaxed formula (exact on {0, 1} inputs).
template <typename S, int VEC, int U>
__global__ __launch_bounds__(256) void k_dense_eval(const S* __restrict__ x,
                                                    const int64_t* __restrict__ a,
                                                    const int64_t* __restrict__ b,
                                                    const uint8_t* __restrict__ wslot,
                                                    const uint8_t* __restrict__ gs,
                                                    S* __restrict__ y, int64_t in_dim,
                                                    int64_t out_dim, int64_t B, int G) {
    using A = acc_t<S>;
    const int64_t o = int64_t(blockIdx.x) * kWaves + wave_id();
    if (o >= out_dim) return;
    const int64_t b0 = int64_t(blockIdx.y) * (kWave * VEC * U) + int64_t(lane_id()) * VEC;
    const int s = wslot[o];
    bool bad = s >= G;
    int64_t ia = 0, ib = 0;
    Coef4<A> c{A(0), A(0), A(0), A(0)};
    if (!bad) {
        ia = a[o * G + s];
        ib = b[o * G + s];
        c = gate_coef<A>(gs[o * G + s]);
        bad = uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim);
    }
    Vec<A, VEC> acc[U];
    zero_acc(acc);
    if (!bad) accum_run<S, VEC, U>(acc, x + ia * B, x + ib * B, c, b0, B);
    store_rows<S, VEC, U>(y + o * B, acc, b0, B, bad);
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
    CL_DTYPE_SWITCH_F16(dtype, {
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
    CL_DTYPE_SWITCH_F16(dtype, {
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
    CL_DTYPE_SWITCH_F16(dtype, {
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

extern "C" int cl_dense_eval(int dtype, const void* x, const int64_t* a, const int64_t* b,
                             const uint8_t* w_slot, const uint8_t* gate_seq, void* y,
                             int64_t in_dim, int64_t out_dim, int64_t batch, int64_t num_gates,
                             void* stream) {
    clear_error();
    if (int rc = check_dims(in_dim, out_dim, batch, num_gates)) return rc;
    if (out_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && a && b && w_slot && gate_seq && y, "null pointer argument");
    CL_DTYPE_SWITCH_F16(dtype, {
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
