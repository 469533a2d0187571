// Dense LogicLayer training path for gfx950: batch-chunk tiles pinned to XCDs.
//
// Why tiles: every activation row is gathered by about two consumers (the neurons wired to
// it), so a gather kernel that streams whole rows reads each row twice from beyond the L2.
// Here the batch is cut into chunks of CS samples (one LPN-lane group of 16-byte vectors per
// row), and all work on chunk c runs on one XCD: workgroups are dispatched round-robin over
// the 8 XCDs of an MI355X, so workgroup w runs on XCD w % 8, and chunk c is given only to
// workgroups w with w % 8 == c % 8.  The chunk's band of the activation matrix (rows x CS
// samples, 1.5-3 MB at 12000 rows) then stays in that XCD's 4 MB L2 and the second gather of
// a row hits L2.  Outputs use ordinary write-back stores (see vst_stream).
//
// Per layer and training step:
//   k_prep        logits -> softmax probabilities and the collapsed coefficients K of every
//                 run (K = sum over the run's slots of p_g * (c0, c1, c2, c3)[gate_g])
//   k_fwd_tiled   y[o, chunk] = sum over runs of K0 + K1 a + K2 b + K3 a b
//   k_bwd_tiled   grad_x[i, chunk] through the inverse index, and per-chunk batch moments
//                 (sum gy, gy a, gy b, gy a b) of every run at its operand-a entry
//   k_moments     the same moments per neuron when no input gradient is needed
//   k_finalize    moments summed over chunks in chunk order -> gradient per slot -> softmax
//                 backward (optional) -> gradient of the logits
// Every reduction has a fixed order, so results are bitwise reproducible.
#include "common.h"

#include <algorithm>
#include <initializer_list>
#include <type_traits>

namespace cl {
namespace {

constexpr int kXcds = 8;  // MI355X: 8 XCDs of 32 CUs

template <typename T, int N>
struct VT {
    typedef T type __attribute__((ext_vector_type(N)));
};
template <typename T>
struct VT<T, 1> {
    typedef T type;
};

template <typename V>
__device__ __forceinline__ V vld(const void* p) {
    return *reinterpret_cast<const V*>(p);
}

// One 16-byte load of an int4 record (the HIP struct type may be split into narrower loads).
__device__ __forceinline__ int4 ld_rec(const int4* p) {
    typedef int I4 __attribute__((ext_vector_type(4)));
    const I4 v = *reinterpret_cast<const I4*>(p);
    return make_int4(v[0], v[1], v[2], v[3]);
}

// Lane accesses of the forward / backward tiled kernels are this many 16-byte vectors wide.
// One for both: with connections='random' (16 runs per neuron) two-vector backward lanes
// measured 0.346 ms per 12000 -> 12000 layer against 0.335 ms with one (2.78 -> 2.69 ms per
// step); 8-lane chunks were far slower (0.58 ms: the per-chunk run work doubles).
// Runs of a neuron the tiled forward gathers together (connections='random': 0.134 -> 0.111 ms
// per 12000 -> 12000 layer against one at a time; eight measured 0.124 ms).
constexpr int kFwdRunBatch = 4;
// Inverse-index entries the tiled backward gathers together (connections='random': 0.367 ->
// 0.314 ms per 12000 -> 12000 layer against one at a time; two 0.342, eight 0.339 ms).
constexpr int kBwdEntryBatch = 4;
#ifndef CL_FWD_VEC_MULT
#define CL_FWD_VEC_MULT 1
#endif
#ifndef CL_BWD_VEC_MULT
#define CL_BWD_VEC_MULT 1
#endif
#ifndef CL_FUSED_VEC_MULT
#define CL_FUSED_VEC_MULT 1
#endif

// Store of an output row segment.  Regular (write-back) stores measure faster inside a
// training step than non-temporal ones: the next kernel reads these rows right away and then
// finds them in the Infinity Cache.
template <typename V>
__device__ __forceinline__ void vst_stream(void* p, V v) {
    *reinterpret_cast<V*>(p) = v;
}

template <typename T, int N>
__device__ __forceinline__ T hsum(typename VT<T, N>::type v) {
    if constexpr (N == 1) {
        return v;
    } else if constexpr (N == 2) {
        return v[0] + v[1];
    } else if constexpr (N == 4) {
        return (v[0] + v[1]) + (v[2] + v[3]);
    } else {
        return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    }
}

// The product moments of one run over a lane's U vectors of a whole-batch row, summed over
// the wave: m1 = sum g*a, m2 = sum g*b, m3 = sum g*a*b.  Every product is rounded before it is
// added (no contraction into fused multiply-adds), so the kernels that compute a neuron's
// moments from the same rows (k_wgrad_rows from the stored gradient, k_bwd_rows' first-layer
// mode from the gradient it holds) produce the same bits.
template <typename T, int VEC, int U>
__device__ __forceinline__ void run_moments(const typename VT<T, VEC>::type (&g)[U],
                                            const typename VT<T, VEC>::type (&a)[U],
                                            const typename VT<T, VEC>::type (&b)[U], T& m1,
                                            T& m2, T& m3) {
#pragma clang fp contract(off)
    using V = typename VT<T, VEC>::type;
    T s2 = 0, s3 = 0, s4 = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const V ga = g[u] * a[u];
        s2 += hsum<T, VEC>(ga);
        s3 += hsum<T, VEC>(g[u] * b[u]);
        s4 += hsum<T, VEC>(ga * b[u]);
    }
    m1 = wave_total(s2);
    m2 = wave_total(s3);
    m3 = wave_total(s4);
}

// Softmax backward of a slot gradient gp with probability p (0 on lanes past the slots):
// p * (gp - sum_h p_h gp_h), without contraction (see run_moments).
template <typename T>
__device__ __forceinline__ T softmax_back(T p, T gp) {
#pragma clang fp contract(off)
    const T pg = p * gp;
    return p * (gp - wave_total(pg));
}

template <typename T>
__device__ __forceinline__ T nan_of() {
    return T(__builtin_nan(""));
}

// Sum over each group of LPN consecutive lanes (LPN in {4, 8, 16}); the total is valid at the
// group's first lane (for LPN = 16 at every lane of the group).  DPP stays inside a 16-lane
// row, and the group leader only ever reads lanes of its own group: row_ror:n delivers to
// lane l the value of lane (l - n) mod 16, so row_ror:12 brings lane l + 4 to lane l.
template <int LPN, typename T>
__device__ __forceinline__ T group_sum(T v) {
    v += dpp_move<0xB1>(v);                           // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);                           // quad_perm [2,3,0,1]
    if constexpr (LPN >= 8) v += dpp_move<0x12C>(v);  // row_ror:12 (lane l + 4)
    if constexpr (LPN >= 16) v += dpp_move<0x128>(v); // row_ror:8
    return v;
}

template <typename T>
__device__ __forceinline__ T row16_max(T v) {
    v = fmax(v, dpp_move<0xB1>(v));
    v = fmax(v, dpp_move<0x4E>(v));
    v = fmax(v, dpp_move<0x124>(v));
    v = fmax(v, dpp_move<0x128>(v));
    return v;
}

// Workgroup -> (chunk, tile).  With at least kXcds chunks, chunk c is handled only by the
// workgroups w with w % kXcds == c % kXcds, all tiles of chunk c before those of chunk
// c + kXcds.  With fewer chunks the tiles of each chunk are spread over all XCDs.
struct TileMap {
    int64_t nchunks;
    int64_t ntiles;
};

__host__ __device__ __forceinline__ int64_t tile_grid(const TileMap& m) {
    if (m.nchunks >= kXcds) return kXcds * ((m.nchunks + kXcds - 1) / kXcds) * m.ntiles;
    return m.nchunks * m.ntiles;
}

__device__ __forceinline__ bool map_tile(const TileMap& m, int64_t w, int64_t& c, int64_t& t) {
    // grids stay below 2^32 workgroups and tile counts below 2^31: 32-bit divisions
    const uint32_t nt = uint32_t(m.ntiles);
    if (m.nchunks >= kXcds) {
        const uint32_t x = uint32_t(w) % kXcds, j = uint32_t(w) / kXcds;
        c = x + kXcds * int64_t(j / nt);
        t = j % nt;
    } else {
        c = uint32_t(w) / nt;
        t = uint32_t(w) % nt;
    }
    return c < m.nchunks;
}

constexpr int kMaxSlotGroups = 8;  // G <= 128 = 8 groups of 16 slots

// ------------------------------------------------------------------------------------------
// k_prep: 16 lanes per neuron; lane l holds slots l, l+16, ...
template <typename T>
__global__ __launch_bounds__(256) void k_prep(const T* __restrict__ w, int softmax,
                                              const uint8_t* __restrict__ gs,
                                              const int32_t* __restrict__ run_ptr,
                                              const int32_t* __restrict__ run_gl,
                                              const int32_t* __restrict__ inv_pos,
                                              T* __restrict__ probs, T* __restrict__ kc,
                                              T* __restrict__ inv_coef, int64_t out_dim,
                                              int64_t num_runs, int G) {
    const int64_t o = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
    const int l = threadIdx.x & 15;
    if (o >= out_dim) return;  // uniform per 16-lane row
    const int ng = (G + 15) >> 4;
    T p[kMaxSlotGroups];
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        p[m] = (m < ng && g < G) ? w[o * G + g] : T(0);
    }
    if (softmax) {
        T mx = -T(__builtin_inf());
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m)
            if (m < ng && l + 16 * m < G) mx = fmax(mx, p[m]);
        mx = row16_max(mx);
        T s = 0;
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const bool ok = m < ng && l + 16 * m < G;
            p[m] = ok ? exp(p[m] - mx) : T(0);
            s += p[m];
        }
        s = group_sum<16>(s);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) p[m] = p[m] / s;
    }
    if (probs) {
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            if (m < ng && g < G) probs[o * G + g] = p[m];
        }
    }
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) return;
    // The row's gate codes, and the records of its runs 16 at a time (one per lane, handed
    // round by lane shuffles), are loaded before the runs are walked: no load waits inside.
    int code[kMaxSlotGroups];
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        code[m] = (m < ng && g < G) ? int(gs[o * G + g]) : 0;
    }
    const int row_lane0 = int(threadIdx.x) & ~15;
    for (int64_t rb = r0; rb < r1; rb += 16) {
    const int64_t rl = rb + l;
    const bool have = rl < r1;
    const int gl_l = have ? run_gl[rl] : 0;
    const int pa_l = (have && inv_coef) ? inv_pos[2 * rl] : -1;
    const int pb_l = (have && inv_coef) ? inv_pos[2 * rl + 1] : -1;
    const int nb = int(r1 - rb < 16 ? r1 - rb : 16);
    for (int q = 0; q < nb; ++q) {
        const int64_t r = rb + q;
        const int gl = __shfl(gl_l, row_lane0 + q);
        const int64_t pa = __shfl(pa_l, row_lane0 + q), pb = __shfl(pb_l, row_lane0 + q);
        const int g0 = gl & 0xff, g1 = g0 + (gl >> 8);
        T k0 = 0, k1 = 0, k2 = 0, k3 = 0;
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            if (m < ng && g >= g0 && g < g1 && g < G) {
                const Coef4<T> c = gate_coef<T>(code[m]);
                k0 = fma(p[m], c.c0, k0);
                k1 = fma(p[m], c.c1, k1);
                k2 = fma(p[m], c.c2, k2);
                k3 = fma(p[m], c.c3, k3);
            }
        }
        k0 = group_sum<16>(k0);
        k1 = group_sum<16>(k1);
        k2 = group_sum<16>(k2);
        k3 = group_sum<16>(k3);
        if (l == 0) {
            if (g1 > G) k0 = k1 = k2 = k3 = nan_of<T>();
            kc[4 * r + 0] = k0;
            kc[4 * r + 1] = k1;
            kc[4 * r + 2] = k2;
            kc[4 * r + 3] = k3;
            if (inv_coef) {
                // (own-operand coefficient, c3) of the run's two inverse-index entries
                if (uint64_t(pa) < uint64_t(2 * num_runs)) {
                    inv_coef[2 * pa + 0] = k1;
                    inv_coef[2 * pa + 1] = k3;
                }
                if (uint64_t(pb) < uint64_t(2 * num_runs)) {
                    inv_coef[2 * pb + 0] = k2;
                    inv_coef[2 * pb + 1] = k3;
                }
            }
        }
    }
    }
}

// ------------------------------------------------------------------------------------------
// k_fwd_tiled: LPN lanes per neuron row segment, NPG neurons per lane group (256 / LPN * NPG
// neurons per tile).  nab[o] = (a, b of the first run, first run, end run) is one load, after
// which the coefficients and both gathers of every neuron of the group are issued together.
// Neurons with several runs continue through run_ab for the others.
template <typename T, int VEC, int LPN, int NPG>
__device__ __forceinline__ void fwd_tile(const T* __restrict__ x, const T* __restrict__ kc,
                                         const int4* __restrict__ nab,
                                         const int2* __restrict__ run_ab, T* __restrict__ y,
                                         int64_t in_dim, int64_t out_dim, int64_t num_runs,
                                         int64_t B, int64_t c, int64_t t) {
    using V = typename VT<T, VEC>::type;
    using V4 = typename VT<T, 4>::type;
    constexpr int GROUPS = 256 / LPN;
    const int64_t obase = (t * GROUPS + threadIdx.x / LPN) * NPG;
    const int64_t idx = c * (LPN * VEC) + int64_t(threadIdx.x % LPN) * VEC;
    if (obase >= out_dim || idx >= B) return;
    int4 rec[NPG];
#pragma unroll
    for (int j = 0; j < NPG; ++j)
        rec[j] = obase + j < out_dim ? nab[obase + j] : make_int4(0, 0, 0, 0);
    V4 k[NPG];
    V va[NPG], vb[NPG];
    bool ok[NPG];
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        ok[j] = obase + j < out_dim && rec[j].z >= 0 && rec[j].z < rec[j].w &&
                rec[j].w <= num_runs && uint32_t(rec[j].x) < uint64_t(in_dim) &&
                uint32_t(rec[j].y) < uint64_t(in_dim);
        if (ok[j]) {
            k[j] = vld<V4>(kc + 4 * int64_t(rec[j].z));
            va[j] = vld<V>(x + int64_t(rec[j].x) * B + idx);
            vb[j] = vld<V>(x + int64_t(rec[j].y) * B + idx);
        }
    }
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        const int64_t o = obase + j;
        if (o >= out_dim) break;
        V acc = V(nan_of<T>());
        if (ok[j]) {
            acc = k[j][3] * (va[j] * vb[j]) + k[j][2] * vb[j] + k[j][1] * va[j] + k[j][0];
            int64_t r = int64_t(rec[j].z) + 1;
            // the further runs kFwdRunBatch at a time: their records and rows are in flight
            // together, the additions stay in run order
            bool badr = false;
            for (; r + kFwdRunBatch <= rec[j].w; r += kFwdRunBatch) {
                int2 ab[kFwdRunBatch];
                V4 kr[kFwdRunBatch];
#pragma unroll
                for (int q = 0; q < kFwdRunBatch; ++q) {
                    ab[q] = run_ab[r + q];
                    kr[q] = vld<V4>(kc + 4 * (r + q));
                }
                V a[kFwdRunBatch], b[kFwdRunBatch];
#pragma unroll
                for (int q = 0; q < kFwdRunBatch; ++q) {
                    const bool v = uint32_t(ab[q].x) < uint64_t(in_dim) &&
                                   uint32_t(ab[q].y) < uint64_t(in_dim);
                    badr = badr || !v;
                    a[q] = vld<V>(x + int64_t(v ? ab[q].x : 0) * B + idx);
                    b[q] = vld<V>(x + int64_t(v ? ab[q].y : 0) * B + idx);
                }
                if (badr) break;
#pragma unroll
                for (int q = 0; q < kFwdRunBatch; ++q)
                    acc += kr[q][3] * (a[q] * b[q]) + kr[q][2] * b[q] + kr[q][1] * a[q] + kr[q][0];
            }
            if (badr) {
                r = rec[j].w;
                acc = V(nan_of<T>());
            }
            for (; r < rec[j].w; ++r) {
                const int2 ab = run_ab[r];
                if (uint32_t(ab.x) >= uint64_t(in_dim) || uint32_t(ab.y) >= uint64_t(in_dim)) {
                    acc = V(nan_of<T>());
                    break;
                }
                const V4 kr = vld<V4>(kc + 4 * r);
                const V a = vld<V>(x + int64_t(ab.x) * B + idx);
                const V b = vld<V>(x + int64_t(ab.y) * B + idx);
                acc += kr[3] * (a * b) + kr[2] * b + kr[1] * a + kr[0];
            }
        }
        vst_stream<V>(y + o * B + idx, acc);
    }
}

template <typename T, int VEC, int LPN, int NPG>
__global__ __launch_bounds__(256) void k_fwd_tiled(const T* __restrict__ x,
                                                   const T* __restrict__ kc,
                                                   const int4* __restrict__ nab,
                                                   const int2* __restrict__ run_ab,
                                                   T* __restrict__ y, int64_t in_dim,
                                                   int64_t out_dim, int64_t num_runs, int64_t B,
                                                   TileMap tm) {
    int64_t c, t;
    if (map_tile(tm, blockIdx.x, c, t))
        fwd_tile<T, VEC, LPN, NPG>(x, kc, nab, run_ab, y, in_dim, out_dim, num_runs, B, c, t);
}

// ------------------------------------------------------------------------------------------
// Butterfly reductions over each group of LPN consecutive lanes (LPN in {4, 8, 16}) that
// leave the result in every lane of the group: quad permutes, then the mirror inside each
// half row (lane i <-> 7 - i), then the mirror inside the row (i <-> 15 - i).  Each step adds
// two partial sums of the same set of lanes, so all lanes end with bitwise the same value.
template <int LPN, typename T>
__device__ __forceinline__ T group_allsum(T v) {
    v += dpp_move<0xB1>(v);                            // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);                            // quad_perm [2,3,0,1]
    if constexpr (LPN >= 8) v += dpp_move<0x141>(v);   // row_half_mirror
    if constexpr (LPN >= 16) v += dpp_move<0x140>(v);  // row_mirror
    return v;
}

template <int LPN, typename T>
__device__ __forceinline__ T group_allmax(T v) {
    v = fmax(v, dpp_move<0xB1>(v));
    v = fmax(v, dpp_move<0x4E>(v));
    if constexpr (LPN >= 8) v = fmax(v, dpp_move<0x141>(v));
    if constexpr (LPN >= 16) v = fmax(v, dpp_move<0x140>(v));
    return v;
}

// exp and 1/s of the fused forward's softmax.  fp32 uses the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: about 1 ulp each, and one of each per slot in place of the
// range-reduced exp and the IEEE divide); the softmax of 16 slots stays within 1e-6 relative.
#ifndef CL_FUSED_FAST
#define CL_FUSED_FAST 1
#endif

template <typename T>
__device__ __forceinline__ T fused_exp(T v) {
    if constexpr (CL_FUSED_FAST && sizeof(T) == 4)
        return __builtin_amdgcn_exp2f(v * 1.44269504088896340736f);
    else
        return exp(v);
}

template <typename T>
__device__ __forceinline__ T fused_rcp(T v) {
    if constexpr (CL_FUSED_FAST && sizeof(T) == 4)
        return __builtin_amdgcn_rcpf(v);
    else
        return T(1) / v;
}

// k_fwd_fused: k_prep and k_fwd_tiled in one pass for layers whose neurons are single runs of
// at most 16 slots.  Lane l of a neuron's LPN-lane group holds slots l, l + LPN, ... (16 / LPN
// of them); the logits are loaded together with the row gathers, so the softmax and the
// collapse to K run while the gathers are in flight.  All lanes of a group stay active until
// the last reduction (DPP reads its neighbours), partial-chunk lanes only skip their row
// accesses.  The tile's writer chunk (t mod nchunks) stores probs and the inverse-index
// coefficients that the backward pass reads.
//
// HEAD (the last layer of a classifier, followed by GroupSum and the cross-entropy): the
// outputs are not stored.  Each lane adds its rows' outputs into two class sums (the class of
// the tile's first row, and the next class), the tile's lane groups add theirs in LDS in row
// order, and the tile writes part[(t * 2 + slot) * B + n]; a tile spans at most two classes
// (gsz >= 256 / LPN * NPG rows, checked by the host).
template <typename T, int VEC, int LPN, int NPG, bool COEF, bool HEAD>
__device__ __forceinline__ void fwd_fused_tile(const T* __restrict__ x, const T* __restrict__ w,
                                               int softmax, const uint8_t* __restrict__ gs,
                                               const int4* __restrict__ nab,
                                               const int32_t* __restrict__ inv_pos,
                                               T* __restrict__ probs, T* __restrict__ inv_coef,
                                               T* __restrict__ y, int64_t in_dim, int64_t out_dim,
                                               int64_t num_runs, int64_t B, int G,
                                               const TileMap& tm, int64_t c, int64_t t,
                                               T* __restrict__ part, int64_t gsz,
                                               T* __restrict__ red) {
    using V = typename VT<T, VEC>::type;
    constexpr int GROUPS = 256 / LPN;
    constexpr int SPL = 16 / LPN;
    const int64_t obase = (t * GROUPS + threadIdx.x / LPN) * NPG;
    // uniform per lane group; the head's lane groups past the end stay for the tile's barrier
    if (!HEAD && obase >= out_dim) return;
    const int64_t ob = obase < out_dim ? obase : 0;  // clamped row for the loads
    const int l = threadIdx.x % LPN;
    const int64_t idx = c * (LPN * VEC) + int64_t(l) * VEC;
    const bool col = idx < B;
    const int64_t off = col ? idx : 0;
    const bool writer = uint32_t(c) == uint32_t(t) % uint32_t(tm.nchunks);
    // Every load is unconditional (a clamped address, the value masked after it arrives): a
    // load under a branch makes the compiler wait there for all loads in flight, which would
    // serialize the logits, the records and the row gathers.
    bool live[NPG];
    int4 rec[NPG];
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        live[j] = obase + j < out_dim;
        rec[j] = ld_rec(nab + (live[j] ? obase + j : ob));
    }
    T p[NPG][SPL];
    int code[NPG][SPL];
#pragma unroll
    for (int j = 0; j < NPG; ++j)
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
            const int g = l + LPN * m;
            const int64_t wi = (live[j] ? obase + j : ob) * G + (g < G ? g : 0);
            p[j][m] = w[wi];
            code[j][m] = gs[wi];
        }
    V va[NPG], vb[NPG];
    bool ok[NPG];
    int2 ipos[NPG];
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        ok[j] = live[j] && rec[j].z >= 0 && rec[j].w == rec[j].z + 1 && rec[j].w <= num_runs &&
                uint32_t(rec[j].x) < uint64_t(in_dim) && uint32_t(rec[j].y) < uint64_t(in_dim);
        va[j] = vld<V>(x + int64_t(ok[j] ? rec[j].x : 0) * B + off);
        vb[j] = vld<V>(x + int64_t(ok[j] ? rec[j].y : 0) * B + off);
        // entry positions of the run's two sides, for the tile's writer chunk
        if constexpr (COEF) {
            const int64_t rz = ok[j] ? rec[j].z : 0;
            ipos[j] = make_int2(inv_pos[2 * rz], inv_pos[2 * rz + 1]);
        }
    }
#pragma unroll
    for (int j = 0; j < NPG; ++j)
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
            const bool v = live[j] && l + LPN * m < G;
            p[j][m] = v ? p[j][m] : -T(__builtin_inf());
            code[j][m] = v ? code[j][m] : 0;
        }
    // head: the first row of the tile's second class
    const int64_t bound = HEAD ? (t * GROUPS * NPG / gsz + 1) * gsz : 0;
    V h0 = V(T(0)), h1 = V(T(0));
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        const int64_t o = obase + j;
        if (softmax) {
            T mx = p[j][0];
#pragma unroll
            for (int m = 1; m < SPL; ++m) mx = fmax(mx, p[j][m]);
            mx = group_allmax<LPN>(mx);
            T s = 0;
#pragma unroll
            for (int m = 0; m < SPL; ++m) {
                p[j][m] = l + LPN * m < G ? fused_exp(p[j][m] - mx) : T(0);
                s += p[j][m];
            }
            s = group_allsum<LPN>(s);
            const T inv = fused_rcp(s);
#pragma unroll
            for (int m = 0; m < SPL; ++m) p[j][m] = p[j][m] * inv;
        } else {
#pragma unroll
            for (int m = 0; m < SPL; ++m)
                if (l + LPN * m >= G) p[j][m] = T(0);
        }
        T k0 = 0, k1 = 0, k2 = 0, k3 = 0;
#pragma unroll
        for (int m = 0; m < SPL; ++m) {
            const Coef4<T> cf = gate_coef<T>(code[j][m]);
            k0 = fma(p[j][m], cf.c0, k0);
            k1 = fma(p[j][m], cf.c1, k1);
            k2 = fma(p[j][m], cf.c2, k2);
            k3 = fma(p[j][m], cf.c3, k3);
        }
        k0 = group_allsum<LPN>(k0);
        k1 = group_allsum<LPN>(k1);
        k2 = group_allsum<LPN>(k2);
        k3 = group_allsum<LPN>(k3);
        if (o >= out_dim) break;
        if (writer) {
            if (probs) {
#pragma unroll
                for (int m = 0; m < SPL; ++m)
                    if (l + LPN * m < G) probs[o * G + l + LPN * m] = p[j][m];
            }
            if constexpr (COEF) {
                if (ok[j] && l == 0) {
                    const int64_t pa = ipos[j].x, pb = ipos[j].y;
                    if (uint64_t(pa) < uint64_t(2 * num_runs)) {
                        inv_coef[2 * pa + 0] = k1;
                        inv_coef[2 * pa + 1] = k3;
                    }
                    if (uint64_t(pb) < uint64_t(2 * num_runs)) {
                        inv_coef[2 * pb + 0] = k2;
                        inv_coef[2 * pb + 1] = k3;
                    }
                }
            }
        }
        if (col) {
            V acc = V(nan_of<T>());
            if (ok[j]) acc = k3 * (va[j] * vb[j]) + k2 * vb[j] + k1 * va[j] + k0;
            if constexpr (HEAD) {
                if (o < bound) h0 += acc;
                else h1 += acc;
            } else {
                vst_stream<V>(y + o * B + idx, acc);
            }
        }
    }
    if constexpr (HEAD) {
        // red[(group * 2 + slot) * LPN * VEC + column]: the lane groups' sums, added in group
        // (= row) order by the thread of each (slot, column)
        constexpr int CW = LPN * VEC;
        const int grp = threadIdx.x / LPN;
        const T* e0 = reinterpret_cast<const T*>(&h0);  // V is T itself when VEC == 1
        const T* e1 = reinterpret_cast<const T*>(&h1);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            red[(grp * 2 + 0) * CW + l * VEC + i] = e0[i];
            red[(grp * 2 + 1) * CW + l * VEC + i] = e1[i];
        }
        __syncthreads();
        const int64_t first = t * GROUPS * NPG;
        for (int e = threadIdx.x; e < 2 * CW; e += 256) {
            const int slot = e / CW, cc = e % CW;
            T sum = T(0);
#pragma unroll 8
            for (int g = 0; g < GROUPS; ++g) sum += red[(g * 2 + slot) * CW + cc];
            const int64_t n = c * CW + cc;
            if (n < B && first < out_dim) part[(t * 2 + slot) * B + n] = sum;
        }
    }
}

template <typename T, int VEC, int LPN, int NPG, bool COEF, bool HEAD>
__global__ __launch_bounds__(256) void k_fwd_fused(const T* __restrict__ x, const T* __restrict__ w,
                                                   int softmax, const uint8_t* __restrict__ gs,
                                                   const int4* __restrict__ nab,
                                                   const int32_t* __restrict__ inv_pos,
                                                   T* __restrict__ probs, T* __restrict__ inv_coef,
                                                   T* __restrict__ y, int64_t in_dim,
                                                   int64_t out_dim, int64_t num_runs, int64_t B,
                                                   int G, TileMap tm, T* __restrict__ part,
                                                   int64_t gsz) {
    __shared__ T red[HEAD ? 2 * 256 * VEC : 1];
    int64_t c, t;
    if (map_tile(tm, blockIdx.x, c, t))  // uniform per workgroup
        fwd_fused_tile<T, VEC, LPN, NPG, COEF, HEAD>(x, w, softmax, gs, nab, inv_pos, probs,
                                                     inv_coef, y, in_dim, out_dim, num_runs, B,
                                                     G, tm, c, t, part, gsz, red);
}

// ------------------------------------------------------------------------------------------
// Softmax + run coefficients of neuron o held by a 16-lane row (lane l: slots l, l+16, ...).
template <typename T, int NG = kMaxSlotGroups>
struct SlotProbs {
    T p[NG];
};

// NG: slot groups of 16 held per lane (a compile-time bound on (G + 15) / 16).
template <typename T, int NG = kMaxSlotGroups>
__device__ __forceinline__ SlotProbs<T, NG> slot_probs(const T* __restrict__ w, int softmax,
                                                       int64_t o, int l, int G) {
    constexpr int kMaxSlotGroups = NG;
    const int ng = (G + 15) >> 4;
    SlotProbs<T, NG> sp;
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        sp.p[m] = (m < ng && g < G) ? w[o * G + g] : T(0);
    }
    if (softmax) {
        T mx = -T(__builtin_inf());
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m)
            if (m < ng && l + 16 * m < G) mx = fmax(mx, sp.p[m]);
        mx = row16_max(mx);
        T s = 0;
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const bool ok = m < ng && l + 16 * m < G;
            sp.p[m] = ok ? exp(sp.p[m] - mx) : T(0);
            s += sp.p[m];
        }
        s = group_sum<16>(s);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) sp.p[m] = sp.p[m] / s;
    }
    return sp;
}

// K of the run [g0, g1) from the row's probabilities; every lane of the row gets the result.
template <typename T, int NG = kMaxSlotGroups>
__device__ __forceinline__ Coef4<T> row_run_coef(const SlotProbs<T, NG>& sp,
                                                 const uint8_t* __restrict__ grow, int l, int g0,
                                                 int g1, int G) {
    constexpr int kMaxSlotGroups = NG;
    const int ng = (G + 15) >> 4;
    T k0 = 0, k1 = 0, k2 = 0, k3 = 0;
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        if (m < ng && g >= g0 && g < g1 && g < G) {
            const Coef4<T> c = gate_coef<T>(grow[g]);
            k0 = fma(sp.p[m], c.c0, k0);
            k1 = fma(sp.p[m], c.c1, k1);
            k2 = fma(sp.p[m], c.c2, k2);
            k3 = fma(sp.p[m], c.c3, k3);
        }
    }
    Coef4<T> k;
    k.c0 = group_sum<16>(k0);
    k.c1 = group_sum<16>(k1);
    k.c2 = group_sum<16>(k2);
    k.c3 = group_sum<16>(k3);
    return k;
}

// k_wgrad_full: weight gradient per neuron over the whole batch (16 lanes per neuron), with
// the softmax backward when `probs` is given.  Used when no input gradient is needed, so no
// per-chunk moments or finalize pass are required.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void k_wgrad_full(const T* __restrict__ x, const T* __restrict__ gy,
                                                    const uint8_t* __restrict__ gs,
                                                    const T* __restrict__ probs,
                                                    const int32_t* __restrict__ run_ptr,
                                                    const int2* __restrict__ run_ab,
                                                    const int32_t* __restrict__ run_gl,
                                                    T* __restrict__ grad_w, int64_t in_dim,
                                                    int64_t out_dim, int64_t num_runs, int64_t B,
                                                    int G) {
    using V = typename VT<T, VEC>::type;
    const int64_t o = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
    if (o >= out_dim) return;  // uniform per 16-lane row
    const int l = threadIdx.x & 15;
    const int ng = (G + 15) >> 4;
    T gp[kMaxSlotGroups];
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) gp[m] = T(0);
    bool bad = false;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) {
        bad = true;
        r1 = r0;
    }
    const T* gyr = gy + o * B;
    for (int64_t r = r0; r < r1; ++r) {
        const int2 ab = run_ab[r];
        const int gl = run_gl[r];
        const int g0 = gl & 0xff, g1 = g0 + (gl >> 8);
        const bool ok = uint32_t(ab.x) < uint64_t(in_dim) && uint32_t(ab.y) < uint64_t(in_dim);
        bad = bad || !ok;
        T s1 = 0, sa = 0, sb = 0, sab = 0;
        if (ok) {
            const T* xa = x + int64_t(ab.x) * B;
            const T* xb = x + int64_t(ab.y) * B;
            for (int64_t idx = int64_t(l) * VEC; idx < B; idx += 16 * VEC) {
                const V vg = vld<V>(gyr + idx);
                const V va = vld<V>(xa + idx);
                const V vb = vld<V>(xb + idx);
                const V ga = vg * va;
                s1 += hsum<T, VEC>(vg);
                sa += hsum<T, VEC>(ga);
                sb += hsum<T, VEC>(vg * vb);
                sab += hsum<T, VEC>(ga * vb);
            }
        }
        s1 = group_sum<16>(s1);
        sa = group_sum<16>(sa);
        sb = group_sum<16>(sb);
        sab = group_sum<16>(sab);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            if (m < ng && g >= g0 && g < g1 && g < G) {
                const Coef4<T> cf = gate_coef<T>(gs[o * G + g]);
                gp[m] = fma(cf.c3, sab, fma(cf.c2, sb, fma(cf.c1, sa, cf.c0 * s1)));
            }
        }
    }
    if (probs) {
        T dot = 0;
        T p[kMaxSlotGroups];
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            p[m] = (m < ng && g < G) ? probs[o * G + g] : T(0);
            dot = fma(p[m], gp[m], dot);
        }
        dot = group_sum<16>(dot);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) gp[m] = p[m] * (gp[m] - dot);
    }
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        if (m < ng && g < G) grad_w[o * G + g] = bad ? nan_of<T>() : gp[m];
    }
}

// k_wgrad_rows: the same with one wave per neuron over the whole batch (lane l holds samples
// (u * 64 + l) * VEC .. +VEC-1, u < U), for batches of at most 64 * VEC * U samples and at
// most 64 slots (lane g owns slot g).  grad_y of the neuron is loaded once for all its runs;
// each run's moments are wave totals, so no partial sums leave the wave.  Loads are
// unconditional (clamped, masked afterwards) so they are in flight together, and run o's
// pair is fetched with run_ptr[o]: in a layer of single-run neurons run o is neuron o's
// only run, and its row gathers need no second round trip.
template <typename T, int VEC, int U, bool HAS_P>
__global__ __launch_bounds__(256) void k_wgrad_rows(const T* __restrict__ x,
                                                    const T* __restrict__ gy,
                                                    const uint8_t* __restrict__ gs,
                                                    const T* __restrict__ probs,
                                                    const int32_t* __restrict__ run_ptr,
                                                    const int2* __restrict__ run_ab,
                                                    const int32_t* __restrict__ run_gl,
                                                    T* __restrict__ grad_w, int64_t in_dim,
                                                    int64_t out_dim, int64_t num_runs, int64_t B,
                                                    int G) {
    using V = typename VT<T, VEC>::type;
    const int lane = threadIdx.x & 63;
    const int64_t o = int64_t(blockIdx.x) * 4 + wave_id();
    if (o >= out_dim) return;  // uniform per wave
    int64_t off[U];
    bool in[U];
    V vg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = int64_t(u * 64 + lane) * VEC;
        in[u] = idx < B;
        off[u] = in[u] ? idx : 0;
        vg[u] = vld<V>(gy + o * B + off[u]);
    }
    const int gl = lane < G ? lane : 0;
    const int code = gs[o * G + gl];
    const T p = HAS_P ? probs[o * G + gl] : T(0);
    const int64_t oc = o < num_runs ? o : num_runs - 1;
    const int2 ab_o = run_ab[oc];
    const int gl_o = run_gl[oc];
    bool bad = false;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) {
        bad = true;
        r1 = r0;
    }
    T s1 = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        vg[u] = in[u] ? vg[u] : V(T(0));
        s1 += hsum<T, VEC>(vg[u]);
    }
    const T m0 = wave_total(s1);
    T gp = T(0);
    for (int64_t r = r0; r < r1; ++r) {
        int2 ab = ab_o;
        int glr = gl_o;
        if (r != oc) {
            ab = run_ab[r];
            glr = run_gl[r];
        }
        const int g0 = glr & 0xff, g1 = g0 + (glr >> 8);
        const bool ok = uint32_t(ab.x) < uint64_t(in_dim) && uint32_t(ab.y) < uint64_t(in_dim);
        if (!ok) {
            bad = true;
            ab = make_int2(0, 0);
        }
        V va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            va[u] = vld<V>(x + int64_t(ab.x) * B + off[u]);
            vb[u] = vld<V>(x + int64_t(ab.y) * B + off[u]);
        }
        T m1, m2, m3;
        run_moments<T, VEC, U>(vg, va, vb, m1, m2, m3);
        const Coef4<T> cf = gate_coef<T>(code);
        const T v = fma(cf.c3, m3, fma(cf.c2, m2, fma(cf.c1, m1, cf.c0 * m0)));
        if (lane >= g0 && lane < g1 && lane < G) gp = v;
    }
    if constexpr (HAS_P) gp = softmax_back(lane < G ? p : T(0), gp);
    if (lane < G) grad_w[o * G + lane] = bad ? nan_of<T>() : gp;
}

// ------------------------------------------------------------------------------------------
// k_bwd_tiled: LPN lanes per input-row segment, NPG rows per lane group.  Rows are taken in
// processing-slot order (descending entry count, so the rows of a group and the groups of a
// wave have nearly equal work), and slot_rec[slot] = (input row, first entry, end entry) is
// one load.  Entry e of the inverse index carries a record (neuron, other input, run, side)
// and the coefficients (own-operand K, K3) written by k_prep; entries are taken
// kBwdEntryBatch at a time, their records and row gathers in flight together.
// part[(r * nchunks + c) * 4 + j] receives the chunk-c moments of run r (WANT_GW) at the
// run's operand-a entry.
template <typename T, int VEC, int LPN, int NPG, bool WANT_GX, bool WANT_GW>
__device__ __forceinline__ void bwd_tile(
    const T* __restrict__ x, const T* __restrict__ gy, const int4* __restrict__ slot_rec,
    const int4* __restrict__ inv_rec, const T* __restrict__ inv_coef, T* __restrict__ gx,
    T* __restrict__ part,
    int64_t in_dim, int64_t out_dim, int64_t num_runs, int64_t B, const TileMap& tm, int64_t c,
    int64_t t) {
    using V = typename VT<T, VEC>::type;
    using V2 = typename VT<T, 2>::type;
    using V4 = typename VT<T, 4>::type;
    constexpr int GROUPS = 256 / LPN;
    const int64_t slot0 = (t * GROUPS + threadIdx.x / LPN) * NPG;
    if (slot0 >= in_dim) return;  // uniform per lane group
    const int64_t idx = c * (LPN * VEC) + int64_t(threadIdx.x % LPN) * VEC;
    const bool col = idx < B;
    const bool leader = (threadIdx.x % LPN) == 0;

    int64_t row[NPG], e0[NPG], deg[NPG];
    bool live[NPG], bad[NPG];
    int64_t maxdeg = 0;
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        live[j] = slot0 + j < in_dim;
        const int4 sr = live[j] ? slot_rec[slot0 + j] : make_int4(0, 0, 0, 0);
        row[j] = sr.x;
        e0[j] = sr.y;
        deg[j] = int64_t(sr.z) - sr.y;
        bad[j] = false;
        if (live[j] && (uint64_t(row[j]) >= uint64_t(in_dim) || sr.y < 0 || deg[j] < 0 ||
                        sr.z > 2 * num_runs)) {
            live[j] = false;  // corrupt slot record: nothing is read or written for it
            deg[j] = 0;
        }
        if (!live[j]) deg[j] = 0;
        maxdeg = deg[j] > maxdeg ? deg[j] : maxdeg;
    }
    V xi[NPG], acc[NPG];
#pragma unroll
    for (int j = 0; j < NPG; ++j) {
        acc[j] = V(T(0));
        xi[j] = V(T(0));
        if (WANT_GW && live[j] && col) xi[j] = vld<V>(x + row[j] * B + idx);
    }
    // Entries are taken kBwdEntryBatch at a time: the batch's records and coefficients, then
    // all of its row gathers, are in flight together (every load unconditional: an unused
    // entry reads entry e0 and row 0, lanes past the batch read sample 0, and both are masked
    // afterwards); the accumulation order is the entry order.
    constexpr int EB = kBwdEntryBatch;
    const int64_t off = col ? idx : 0;
#pragma unroll
    for (int j = 0; j < NPG; ++j)
        if (!live[j]) e0[j] = 0;  // a dead or corrupt slot's unused loads read entry 0
    for (int64_t k = 0; k < maxdeg; k += EB) {
        int4 cur[NPG][EB];
        V2 ck[NPG][EB];
        bool use[NPG][EB];
#pragma unroll
        for (int j = 0; j < NPG; ++j)
#pragma unroll
            for (int q = 0; q < EB; ++q) {
                use[j][q] = k + q < deg[j];
                const int64_t e = e0[j] + (use[j][q] ? k + q : 0);
                cur[j][q] = inv_rec[e];
                ck[j][q] = vld<V2>(inv_coef + 2 * e);
            }
        V vo[NPG][EB], vg[NPG][EB];
#pragma unroll
        for (int j = 0; j < NPG; ++j)
#pragma unroll
            for (int q = 0; q < EB; ++q) {
                if (use[j][q] && (uint64_t(cur[j][q].x) >= uint64_t(out_dim) ||
                                  uint64_t(cur[j][q].y) >= uint64_t(in_dim) ||
                                  uint64_t(cur[j][q].z) >= uint64_t(num_runs))) {
                    bad[j] = true;
                    use[j][q] = false;
                }
                const bool u = use[j][q];
                vo[j][q] = vld<V>(x + int64_t(u ? cur[j][q].y : 0) * B + off);
                vg[j][q] = vld<V>(gy + int64_t(u ? cur[j][q].x : 0) * B + off);
            }
#pragma unroll
        for (int j = 0; j < NPG; ++j)
#pragma unroll
            for (int q = 0; q < EB; ++q) {
                if (!use[j][q]) continue;
                const V o = col ? vo[j][q] : V(T(0));
                const V g = col ? vg[j][q] : V(T(0));
                if (WANT_GX) acc[j] += (ck[j][q][0] + ck[j][q][1] * o) * g;
                if (WANT_GW && cur[j][q].w == 0) {
                    const V ga = g * xi[j];
                    T s1 = hsum<T, VEC>(g), sa = hsum<T, VEC>(ga);
                    T sb = hsum<T, VEC>(g * o), sab = hsum<T, VEC>(ga * o);
                    s1 = group_sum<LPN>(s1);
                    sa = group_sum<LPN>(sa);
                    sb = group_sum<LPN>(sb);
                    sab = group_sum<LPN>(sab);
                    if (leader) {
                        V4 mv;
                        mv[0] = s1;
                        mv[1] = sa;
                        mv[2] = sb;
                        mv[3] = sab;
                        *reinterpret_cast<V4*>(part + (int64_t(cur[j][q].z) * tm.nchunks + c) * 4) = mv;
                    }
                }
            }
    }
    if (WANT_GX && col) {
#pragma unroll
        for (int j = 0; j < NPG; ++j) {
            if (!live[j]) continue;
            V r = acc[j];
            if (bad[j]) r = V(nan_of<T>());
            vst_stream<V>(gx + row[j] * B + idx, r);
        }
    }
}

template <typename T, int VEC, int LPN, int NPG, bool WANT_GX, bool WANT_GW>
__global__ __launch_bounds__(256) void k_bwd_tiled(
    const T* __restrict__ x, const T* __restrict__ gy, const int4* __restrict__ slot_rec,
    const int4* __restrict__ inv_rec, const T* __restrict__ inv_coef, T* __restrict__ gx,
    T* __restrict__ part,
    int64_t in_dim, int64_t out_dim, int64_t num_runs, int64_t B, TileMap tm) {
    int64_t c, t;
    if (map_tile(tm, blockIdx.x, c, t))
        bwd_tile<T, VEC, LPN, NPG, WANT_GX, WANT_GW>(x, gy, slot_rec, inv_rec, inv_coef, gx, part,
                                                     in_dim, out_dim, num_runs, B, tm, c, t);
}

// ------------------------------------------------------------------------------------------
// k_bwd_part: the input gradient and per-chunk moments through tiles of kPartRows consecutive
// processing slots.  A workgroup takes TPW = 16 / LPN tiles of one batch chunk; lane group g
// owns slot row g % 16 of tile g / 16.
//   1. Every lane group loads its own row segment x_i and leaves a copy in LDS.
//   2. Internal runs of each tile (both inputs in the tile; listed by tile_ptr / tile_run /
//      tile_loc) are spread over the tile's lane groups: grad_y of the run's neuron is read
//      once, both inputs come from LDS, and the two contributions gy (K1 + K3 b) and
//      gy (K2 + K3 a) go to the LDS slots of the run's two entries, the chunk moments to
//      `part`.
//   3. Each owner adds its row's entries in entry order: an internal entry's contribution from
//      its LDS slot, an external one from the row gathers of bwd_tile.
// The sum of every row keeps the entry order, so results are bitwise reproducible.
constexpr int kPartRows = 16;
constexpr int kPartMaxSlots = 64;

template <typename T, int VEC, int LPN, bool WANT_GX, bool WANT_GW>
__global__ __launch_bounds__(256) void k_bwd_part(
    const T* __restrict__ x, const T* __restrict__ gy, const int4* __restrict__ slot_rec,
    const int4* __restrict__ inv_rec, const T* __restrict__ inv_coef,
    const int32_t* __restrict__ inv_slot, const int32_t* __restrict__ tile_ptr,
    const int4* __restrict__ tile_run, const int32_t* __restrict__ tile_loc,
    int64_t num_internal, T* __restrict__ gx, T* __restrict__ part, int64_t in_dim,
    int64_t out_dim, int64_t num_runs, int64_t B, int slots, TileMap tm) {
    using V = typename VT<T, VEC>::type;
    using V2 = typename VT<T, 2>::type;
    using V4 = typename VT<T, 4>::type;
    constexpr int CH = LPN * VEC;              // samples per chunk
    constexpr int TPW = 16 / LPN;              // tiles per workgroup
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T* xs = reinterpret_cast<T*>(smem_raw);    // [TPW][kPartRows][CH]
    T* cs = xs + TPW * kPartRows * CH;         // [TPW][slots][CH]
    int64_t c, t;
    if (!map_tile(tm, blockIdx.x, c, t)) return;  // uniform per workgroup
    const int g = threadIdx.x / LPN, l = threadIdx.x % LPN;
    const int tl = g / kPartRows, rg = g % kPartRows;
    const int64_t tile = t * TPW + tl;
    const int64_t slot = tile * kPartRows + rg;
    const int64_t idx = c * CH + int64_t(l) * VEC;
    const bool col = idx < B;
    const bool leader = l == 0;
    T* xs_t = xs + tl * kPartRows * CH;
    T* cs_t = cs + int64_t(tl) * slots * CH;

    // 1. own row
    bool live = slot < in_dim;
    const int4 sr = live ? slot_rec[slot] : make_int4(0, 0, 0, 0);
    const int64_t row = sr.x, e0 = sr.y;
    int64_t deg = int64_t(sr.z) - sr.y;
    if (live && (uint64_t(row) >= uint64_t(in_dim) || sr.y < 0 || deg < 0 || sr.z > 2 * num_runs))
        live = false;  // corrupt slot record: nothing is read or written for it
    if (!live) deg = 0;
    V xi = V(T(0));
    if (live && col) xi = vld<V>(x + row * B + idx);
    *reinterpret_cast<V*>(xs_t + rg * CH + l * VEC) = xi;
    __syncthreads();

    // 2. internal runs of the tile
    const int64_t ntiles = (in_dim + kPartRows - 1) / kPartRows;
    if (tile < ntiles) {
        const int64_t ip0 = tile_ptr[tile], ip1 = tile_ptr[tile + 1];
        const bool ok_range = ip0 >= 0 && ip1 >= ip0 && ip1 <= num_internal &&
                              ip1 - ip0 <= slots / 2;
        for (int64_t k = ok_range ? ip0 + rg : ip1; k < ip1; k += kPartRows) {
            const int4 tr = tile_run[k];
            const int loc = tile_loc[k];
            const int al = loc & 0xff, bl = (loc >> 8) & 0xff;
            const int sa = (loc >> 16) & 0xff, sb = (loc >> 24) & 0xff;
            if (uint64_t(tr.x) >= uint64_t(out_dim) || uint64_t(tr.y) >= uint64_t(num_runs) ||
                uint64_t(tr.z) >= uint64_t(2 * num_runs) ||
                uint64_t(tr.w) >= uint64_t(2 * num_runs) || al >= kPartRows || bl >= kPartRows ||
                sa >= slots || sb >= slots)
                continue;  // corrupt record: skipped, nothing is read or written for it
            V vg = V(T(0));
            if (col) vg = vld<V>(gy + int64_t(tr.x) * B + idx);
            const V2 ka = vld<V2>(inv_coef + 2 * int64_t(tr.z));
            const V2 kb = vld<V2>(inv_coef + 2 * int64_t(tr.w));
            const V va = *reinterpret_cast<const V*>(xs_t + al * CH + l * VEC);
            const V vb = *reinterpret_cast<const V*>(xs_t + bl * CH + l * VEC);
            if (WANT_GX) {
                *reinterpret_cast<V*>(cs_t + sa * CH + l * VEC) = (ka[0] + ka[1] * vb) * vg;
                *reinterpret_cast<V*>(cs_t + sb * CH + l * VEC) = (kb[0] + kb[1] * va) * vg;
            }
            if (WANT_GW) {
                const V ga = vg * va;
                T s1 = hsum<T, VEC>(vg), s2 = hsum<T, VEC>(ga);
                T s3 = hsum<T, VEC>(vg * vb), s4 = hsum<T, VEC>(ga * vb);
                s1 = group_sum<LPN>(s1);
                s2 = group_sum<LPN>(s2);
                s3 = group_sum<LPN>(s3);
                s4 = group_sum<LPN>(s4);
                if (leader) {
                    V4 mv;
                    mv[0] = s1;
                    mv[1] = s2;
                    mv[2] = s3;
                    mv[3] = s4;
                    *reinterpret_cast<V4*>(part + (int64_t(tr.y) * tm.nchunks + c) * 4) = mv;
                }
            }
        }
    }
    __syncthreads();

    // 3. the row's entries in entry order
    V acc = V(T(0));
    bool bad = false;
    int4 rec = make_int4(0, 0, 0, 0);
    V2 kk = V2(T(0));
    int sl = -1;
    if (deg > 0) {
        rec = inv_rec[e0];
        kk = vld<V2>(inv_coef + 2 * e0);
        sl = inv_slot[e0];
    }
    for (int64_t k = 0; k < deg; ++k) {
        const int4 cur = rec;
        const V2 ck = kk;
        const int cs_slot = sl;
        if (k + 1 < deg) {
            rec = inv_rec[e0 + k + 1];
            kk = vld<V2>(inv_coef + 2 * (e0 + k + 1));
            sl = inv_slot[e0 + k + 1];
        }
        if (cs_slot >= 0) {
            if (cs_slot >= slots) {
                bad = true;
                continue;
            }
            if (WANT_GX) acc += *reinterpret_cast<const V*>(cs_t + cs_slot * CH + l * VEC);
            continue;
        }
        if (uint64_t(cur.x) >= uint64_t(out_dim) || uint64_t(cur.y) >= uint64_t(in_dim) ||
            uint64_t(cur.z) >= uint64_t(num_runs)) {
            bad = true;
            continue;
        }
        V vo = V(T(0)), vg = V(T(0));
        if (col) {
            vo = vld<V>(x + int64_t(cur.y) * B + idx);
            vg = vld<V>(gy + int64_t(cur.x) * B + idx);
        }
        if (WANT_GX) acc += (ck[0] + ck[1] * vo) * vg;
        if (WANT_GW && cur.w == 0) {
            const V ga = vg * xi;
            T s1 = hsum<T, VEC>(vg), s2 = hsum<T, VEC>(ga);
            T s3 = hsum<T, VEC>(vg * vo), s4 = hsum<T, VEC>(ga * vo);
            s1 = group_sum<LPN>(s1);
            s2 = group_sum<LPN>(s2);
            s3 = group_sum<LPN>(s3);
            s4 = group_sum<LPN>(s4);
            if (leader) {
                V4 mv;
                mv[0] = s1;
                mv[1] = s2;
                mv[2] = s3;
                mv[3] = s4;
                *reinterpret_cast<V4*>(part + (int64_t(cur.z) * tm.nchunks + c) * 4) = mv;
            }
        }
    }
    if (WANT_GX && live && col) {
        V r = acc;
        if (bad) r = V(nan_of<T>());
        vst_stream<V>(gx + row * B + idx, r);
    }
}

// ------------------------------------------------------------------------------------------
// k_bwd_rows: one wave per input row over the whole batch (lane l holds samples
// (u * 64 + l) * VEC .. +VEC-1, u < U), for batches of at most 64 * VEC * U samples.  Every
// gather moves a whole 64 * VEC * U-sample row segment, and the moments of a run are complete
// inside the wave that handles its operand-a entry, so for layers of single-run neurons that
// wave also applies the finalize (moments -> slot gradients -> softmax backward) and writes
// the neuron's logits gradient: no moments buffer and no finalize launch.  Workgroup w (four
// rows) takes slot block (w % 8) * nblk + w / 8, so XCD w % 8 walks one contiguous stretch of
// the processing order, whose rows share neighbours.
//
// The kernel is bound by memory latency (a handful of dependent round trips per wave), so
// every load is unconditional: lanes past the batch read sample 0 and are masked afterwards,
// and an invalid record reads row 0 and poisons the result.  A load under a branch would make
// the compiler wait for all loads in flight at the branch's end.  Entries are taken EPI at a
// time (the records are wave-uniform), so their row gathers are in flight together; the
// input gradient still adds the entries in entry order.  With gy_magic != 0 the gradient of
// neuron o is row o / gsz of grad_y (one row per GroupSum class: the fused classifier head),
// gy_magic = ceil(2^32 / gsz) with out_dim * gsz <= 2^32, so the multiply-high is exact.
// Waves per SIMD the row backward asks the register allocator for: four (at most 128 VGPRs)
// where the fp32 kernel fits them without spilling (rows of up to 1024 samples); more waves
// per SIMD keep more rows' gathers in flight, which is what bounds this kernel.
#ifndef CL_FIRST_WAVES
#define CL_FIRST_WAVES 4
#endif
#ifndef CL_BWD_ROWS_S4
#define CL_BWD_ROWS_S4 12  // entries per row from which four waves share a row
#endif
#ifndef CL_BWD_ROWS_S2
#define CL_BWD_ROWS_S2 6   // ... two waves
#endif
#ifndef CL_FIRST_EPI4
#define CL_FIRST_EPI4 1
#endif
template <typename T, int U, bool FIRST = false>
constexpr int bwd_rows_waves() { return sizeof(T) == 4 && U <= 4 ? (FIRST ? CL_FIRST_WAVES : 4) : 1; }

#ifndef CL_BWD_ROWS_EPI4
#define CL_BWD_ROWS_EPI4 2
#endif

// The layer before, when its input needs no gradient (the first layer of a network): its
// logits gradient is a function of the gradient of its output, which is the input gradient
// the row backward computes, so the row backward finishes it for the neuron of each row
// instead of storing that gradient (k_bwd_rows with FIRST).  Single-run neurons with the
// softmax inside; x0 [in_dim, B] is the layer's input, nab its plan's (a, b, run_ptr[o],
// run_ptr[o + 1]) per neuron.
template <typename T>
struct FirstLayer {
    const T* x0;
    const int4* nab;
    const uint8_t* gs;
    const T* probs;
    T* grad_w;
    int64_t in_dim;
    int64_t num_runs;
    int G;
};

// S > 1 (rows with many entries, e.g. a narrow input feeding a wide layer): S waves of a
// workgroup share a row, wave `part` taking the contiguous part of its entries
// [deg * part / S, deg * (part + 1) / S); the parts' input-gradient sums meet in LDS and are
// added in part order (deterministic; the association differs from S = 1 by rounding).
template <typename T, int VEC, int U, bool WANT_GW, bool HAS_P, bool FIRST = false, int S = 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_rows_waves<T, U, FIRST>())))
void k_bwd_rows(
    const T* __restrict__ x, const T* __restrict__ gy, const int4* __restrict__ slot_rec,
    const int4* __restrict__ inv_rec, const T* __restrict__ inv_coef,
    const uint8_t* __restrict__ gs, const T* __restrict__ probs,
    const int32_t* __restrict__ run_ptr, T* __restrict__ grad_w, T* __restrict__ gx,
    int64_t in_dim, int64_t out_dim, int64_t num_runs, int64_t B, int G, int64_t nblk,
    uint32_t gy_magic, FirstLayer<T> first = {}) {
    static_assert(S == 1 || S == 2 || S == 4, "1, 2 or 4 waves per row");
    static_assert(S == 1 || !FIRST, "the first-layer mode takes one wave per row");
    using V = typename VT<T, VEC>::type;
    using V2 = typename VT<T, 2>::type;
    constexpr int EPI = U <= 2 ? 2 : U <= 4 ? (FIRST ? CL_FIRST_EPI4 : CL_BWD_ROWS_EPI4) : 1;
    const int lane = threadIdx.x & 63;
    const int64_t w = blockIdx.x;
    const int wv = wave_id();
    const int64_t slot = ((w % kXcds) * nblk + w / kXcds) * (4 / S) + wv / S;
    const int part = wv % S;
    if constexpr (S == 1) {
        if (slot >= in_dim) return;  // uniform per wave
    }
    // with S > 1 every wave reaches the closing barrier: an idle one only skips its work
    bool active = slot < in_dim;
    int4 sr = active ? slot_rec[slot] : make_int4(0, 0, 0, 0);
    if (uint64_t(sr.x) >= uint64_t(in_dim) || sr.y < 0 || sr.z < sr.y || sr.z > 2 * num_runs) {
        if constexpr (S == 1) return;  // corrupt slot record: nothing is read or written for it
        active = false;
        sr = make_int4(0, 0, 0, 0);
    }
    const int64_t row = sr.x, e0 = sr.y;
    const int64_t deg = int64_t(sr.z) - sr.y;
    const int64_t klo = active ? deg * part / S : 0, khi = active ? deg * (part + 1) / S : 0;
    int32_t off[U];  // batch offsets (rows of at most 64 * 8 * VEC samples)
    bool in[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = int64_t(u * 64 + lane) * VEC;
        in[u] = idx < B;
        off[u] = in[u] ? idx : 0;
    }
    V xi[U], acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        acc[u] = V(T(0));
        xi[u] = V(T(0));
        if constexpr (WANT_GW) xi[u] = vld<V>(x + row * B + off[u]);
    }
    const int gl = lane < G ? lane : 0;  // slot of this lane in the finalize (clamped)
    bool bad = false;
    // the first layer's wiring of this neuron, loaded with the rows rather than after them
    // (uniform: kept in scalar registers through the entry loop)
    int4 nab1 = make_int4(0, 0, 0, 0);
    if constexpr (FIRST) {
        const int4 t = first.nab[row];
        nab1 = make_int4(__builtin_amdgcn_readfirstlane(t.x), __builtin_amdgcn_readfirstlane(t.y),
                         __builtin_amdgcn_readfirstlane(t.z), __builtin_amdgcn_readfirstlane(t.w));
    }
    for (int64_t k = klo; k < khi; k += EPI) {
        int4 cur[EPI];
        V2 ck[EPI];
        bool use[EPI];
        V vo[EPI][U], vg[EPI][U];
        int rp0[EPI], rp1[EPI], code[EPI];
        T p[EPI];
#pragma unroll
        for (int q = 0; q < EPI; ++q) {
            const int64_t e = e0 + (k + q < khi ? k + q : k);
            cur[q] = inv_rec[e];
            ck[q] = vld<V2>(inv_coef + 2 * e);
            use[q] = k + q < khi;
            const bool ok = uint64_t(cur[q].x) < uint64_t(out_dim) &&
                            uint64_t(cur[q].y) < uint64_t(in_dim) &&
                            uint64_t(cur[q].z) < uint64_t(num_runs);
            if (use[q] && !ok) bad = true;
            use[q] = use[q] && ok;
            if (!ok) cur[q] = make_int4(0, 0, 0, 1);  // reads row 0, side b: no finalize
        }
#pragma unroll
        for (int q = 0; q < EPI; ++q) {
            // grad_y row of the neuron: its own, or its class's (o / gsz as a multiply-high)
            const int64_t gyr = gy_magic ? int64_t(__umulhi(uint32_t(cur[q].x), gy_magic))
                                         : int64_t(cur[q].x);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                vo[q][u] = vld<V>(x + int64_t(cur[q].y) * B + off[u]);
                vg[q][u] = vld<V>(gy + gyr * B + off[u]);
            }
            // the finalize's per-neuron data is loaded with the rows, not after the moments
            if constexpr (WANT_GW) {
                rp0[q] = run_ptr[cur[q].x];
                rp1[q] = run_ptr[cur[q].x + 1];
                code[q] = gs[int64_t(cur[q].x) * G + gl];
                p[q] = HAS_P ? probs[int64_t(cur[q].x) * G + gl] : T(0);
            }
        }
        // all gathers of the step are issued before any of them is waited for
        __builtin_amdgcn_sched_barrier(0);
        // Everything below is computed for every entry, used or not, and only the stores
        // are conditional: a value used under a branch would let the compiler sink its load
        // into that branch and wait for it there.  An unused entry adds -0, which leaves every
        // sum bitwise unchanged.
#pragma unroll
        for (int q = 0; q < EPI; ++q) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const V t = (ck[q][0] + ck[q][1] * vo[q][u]) * vg[q][u];
#pragma unroll
                for (int i = 0; i < VEC; ++i) acc[u][i] += use[q] ? t[i] : -T(0);
            }
            if constexpr (WANT_GW) {
                T s1 = 0, s2 = 0, s3 = 0, s4 = 0;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const V g = in[u] ? vg[q][u] : V(T(0));
                    const V ga = g * xi[u];
                    s1 += hsum<T, VEC>(g);
                    s2 += hsum<T, VEC>(ga);
                    s3 += hsum<T, VEC>(g * vo[q][u]);
                    s4 += hsum<T, VEC>(ga * vo[q][u]);
                }
                const T m0 = wave_total(s1), m1 = wave_total(s2);
                const T m2 = wave_total(s3), m3 = wave_total(s4);
                const Coef4<T> cf = gate_coef<T>(code[q]);
                T gp = lane < G ? fma(cf.c3, m3, fma(cf.c2, m2, fma(cf.c1, m1, cf.c0 * m0))) : T(0);
                if constexpr (HAS_P) {
                    const T pl = lane < G ? p[q] : T(0);
                    gp = pl * (gp - wave_total(pl * gp));
                }
                const bool single = rp0[q] == cur[q].z && rp1[q] == cur[q].z + 1;
                if (use[q] && cur[q].w == 0 && lane < G)
                    grad_w[int64_t(cur[q].x) * G + lane] = single ? gp : nan_of<T>();
            }
        }
    }
    if constexpr (FIRST) {
        // acc is the gradient of the first layer's neuron `row` (what the input-gradient store
        // below would write); its moments against the neuron's two inputs, in the order of
        // k_wgrad_rows, give bitwise the logits gradient that kernel computes from the stored
        // gradient.
        const bool single = nab1.z >= 0 && nab1.w == nab1.z + 1 && nab1.w <= first.num_runs;
        const bool ok = single && uint32_t(nab1.x) < uint64_t(first.in_dim) &&
                        uint32_t(nab1.y) < uint64_t(first.in_dim);
        const int64_t ra = ok ? nab1.x : 0, rb = ok ? nab1.y : 0;
        const int gl1 = lane < first.G ? lane : 0;
        const int code1 = first.gs[row * first.G + gl1];
        const T p1 = first.probs[row * first.G + gl1];
        V va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            va[u] = vld<V>(first.x0 + ra * B + off[u]);
            vb[u] = vld<V>(first.x0 + rb * B + off[u]);
        }
        T s1 = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc[u] = in[u] ? acc[u] : V(T(0));
            s1 += hsum<T, VEC>(acc[u]);
        }
        const T m0 = wave_total(s1);
        T m1, m2, m3;
        run_moments<T, VEC, U>(acc, va, vb, m1, m2, m3);
        const Coef4<T> cf = gate_coef<T>(code1);
        const T v = fma(cf.c3, m3, fma(cf.c2, m2, fma(cf.c1, m1, cf.c0 * m0)));
        const T gp = softmax_back(lane < first.G ? p1 : T(0), lane < first.G ? v : T(0));
        if (lane < first.G) first.grad_w[row * first.G + lane] = (bad || !ok) ? nan_of<T>() : gp;
    } else {
        if constexpr (S > 1) {
            __shared__ V red[4][U][64];
            __shared__ int red_bad[4];
            if (part > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u) red[wv][u][lane] = acc[u];
                if (lane == 0) red_bad[wv] = bad ? 1 : 0;
            }
            __syncthreads();
            if (part > 0 || !active) return;
#pragma unroll
            for (int q = 1; q < S; ++q) {
#pragma unroll
                for (int u = 0; u < U; ++u) acc[u] += red[wv + q][u][lane];
                bad = bad || red_bad[wv + q] != 0;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (in[u]) vst_stream<V>(gx + row * B + off[u], bad ? V(nan_of<T>()) : acc[u]);
    }
}

// k_moments: the per-chunk moments of every run, per neuron (used when grad_x is not needed).
template <typename T, int VEC, int LPN>
__global__ __launch_bounds__(256) void k_moments(const T* __restrict__ x, const T* __restrict__ gy,
                                                 const int32_t* __restrict__ run_ptr,
                                                 const int2* __restrict__ run_ab,
                                                 T* __restrict__ part, int64_t in_dim,
                                                 int64_t out_dim, int64_t num_runs, int64_t B,
                                                 TileMap tm) {
    using V = typename VT<T, VEC>::type;
    using V4 = typename VT<T, 4>::type;
    constexpr int NT = 256 / LPN;
    int64_t c, t;
    if (!map_tile(tm, blockIdx.x, c, t)) return;
    const int64_t o = t * NT + threadIdx.x / LPN;
    if (o >= out_dim) return;  // uniform per lane group
    const int64_t idx = c * (LPN * VEC) + int64_t(threadIdx.x % LPN) * VEC;
    const bool col = idx < B;
    const bool leader = (threadIdx.x % LPN) == 0;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) return;
    V vg = V(T(0));
    if (col) vg = vld<V>(gy + o * B + idx);
    const T s1 = group_sum<LPN>(hsum<T, VEC>(vg));
    for (int64_t r = r0; r < r1; ++r) {
        const int2 ab = run_ab[r];
        V va = V(T(0)), vb = V(T(0));
        const bool ok = uint32_t(ab.x) < uint64_t(in_dim) && uint32_t(ab.y) < uint64_t(in_dim);
        if (col && ok) {
            va = vld<V>(x + int64_t(ab.x) * B + idx);
            vb = vld<V>(x + int64_t(ab.y) * B + idx);
        }
        const V ga = vg * va;
        const T sa = group_sum<LPN>(hsum<T, VEC>(ga));
        const T sb = group_sum<LPN>(hsum<T, VEC>(vg * vb));
        const T sab = group_sum<LPN>(hsum<T, VEC>(ga * vb));
        if (leader) {
            V4 mv;
            mv[0] = ok ? s1 : nan_of<T>();
            mv[1] = sa;
            mv[2] = sb;
            mv[3] = sab;
            *reinterpret_cast<V4*>(part + (r * tm.nchunks + c) * 4) = mv;
        }
    }
}

// ------------------------------------------------------------------------------------------
// k_finalize: 16 lanes per neuron.  Moments of each run are summed over the chunks (lane l
// takes chunks l, l+16, ..., then a fixed lane tree), expanded to the run's slots, and, when
// `probs` is given, passed through the softmax backward: dL/dlogit_g = p_g (dL/dp_g - sum_h
// p_h dL/dp_h).
template <typename T>
__global__ __launch_bounds__(256) void k_finalize(const T* __restrict__ part, int64_t nchunks,
                                                  const uint8_t* __restrict__ gs,
                                                  const T* __restrict__ probs,
                                                  const int32_t* __restrict__ run_ptr,
                                                  const int32_t* __restrict__ run_gl,
                                                  T* __restrict__ grad_w, int64_t out_dim,
                                                  int64_t num_runs, int G) {
    const int64_t o = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
    const int l = threadIdx.x & 15;
    if (o >= out_dim) return;  // uniform per 16-lane row
    const int ng = (G + 15) >> 4;
    T gp[kMaxSlotGroups];
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) gp[m] = T(0);
    bool bad = false;
    int64_t r0 = run_ptr[o], r1 = run_ptr[o + 1];
    if (r0 < 0 || r1 < r0 || r1 > num_runs) {
        bad = true;
        r1 = r0;
    }
    for (int64_t r = r0; r < r1; ++r) {
        const int gl = run_gl[r];
        const int g0 = gl & 0xff, g1 = g0 + (gl >> 8);
        T m0 = 0, m1 = 0, m2 = 0, m3 = 0;
        const T* pr = part + r * nchunks * 4;
        for (int64_t cc = l; cc < nchunks; cc += 16) {
            m0 += pr[cc * 4 + 0];
            m1 += pr[cc * 4 + 1];
            m2 += pr[cc * 4 + 2];
            m3 += pr[cc * 4 + 3];
        }
        m0 = group_sum<16>(m0);
        m1 = group_sum<16>(m1);
        m2 = group_sum<16>(m2);
        m3 = group_sum<16>(m3);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            if (m < ng && g >= g0 && g < g1 && g < G) {
                const Coef4<T> cf = gate_coef<T>(gs[o * G + g]);
                gp[m] = fma(cf.c3, m3, fma(cf.c2, m2, fma(cf.c1, m1, cf.c0 * m0)));
            }
        }
    }
    if (probs) {
        T dot = 0;
        T p[kMaxSlotGroups];
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) {
            const int g = l + 16 * m;
            p[m] = (m < ng && g < G) ? probs[o * G + g] : T(0);
            dot = fma(p[m], gp[m], dot);
        }
        dot = group_sum<16>(dot);
#pragma unroll
        for (int m = 0; m < kMaxSlotGroups; ++m) gp[m] = p[m] * (gp[m] - dot);
    }
#pragma unroll
    for (int m = 0; m < kMaxSlotGroups; ++m) {
        const int g = l + 16 * m;
        if (m < ng && g < G) grad_w[o * G + g] = bad ? nan_of<T>() : gp[m];
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_zero(T* __restrict__ p, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        p[i] = T(0);
}

// ------------------------------------------------------------------------------------------
// Host-side tiling choice.

struct Tiling {
    int vec;   // elements per 16-byte access (1 when the batch does not allow vectors)
    int lpn;   // lanes per row segment
    int64_t chunk;
    TileMap map;
};

// Narrowest lane group first that still leaves every XCD a chunk; bands of at most
// `lpn_max` lanes keep a chunk's activation band within one XCD's L2.
// Lane vector width: `mult` 16-byte vectors when the batch allows it, else one, else scalars.
template <typename T>
Tiling choose_tiling(int64_t B, int64_t rows, int mult, int lpn_max, int rows_per_group = 1) {
    Tiling tl;
    constexpr int W = wide_vec<T>();
    tl.vec = B % (W * mult) == 0 ? W * mult : (B % W == 0 ? W : 1);
    tl.lpn = lpn_max;
    while (tl.lpn > 4 && ceil_div(B, int64_t(tl.lpn) * tl.vec) < kXcds) tl.lpn >>= 1;
    tl.chunk = int64_t(tl.lpn) * tl.vec;
    tl.map.nchunks = ceil_div(B, tl.chunk);
    tl.map.ntiles = ceil_div(rows, int64_t(256 / tl.lpn) * rows_per_group);
    return tl;
}

}  // namespace
}  // namespace cl

using namespace cl;

#ifndef CL_FWD_LPN
#define CL_FWD_LPN 16
#endif
#ifndef CL_BWD_LPN
#define CL_BWD_LPN 16
#endif
#ifndef CL_FWD_NPG
#define CL_FWD_NPG 2
#endif
#ifndef CL_BWD_NPG
#define CL_BWD_NPG 1
#endif

namespace {

// The tiling (and with it the chunk count of the moments buffer) depends on the batch alone:
// 16-byte vectors whenever batch % (16 / sizeof(T)) == 0, which then requires 16-byte aligned
// row buffers.
template <typename T>
bool vec_ok(int64_t B) {
    return B % wide_vec<T>() == 0;
}

bool all_aligned(std::initializer_list<const void*> ptrs) {
    for (const void* p : ptrs)
        if (p && !aligned(p, 16)) return false;
    return true;
}

int check_plan_dims(int64_t in_dim, int64_t out_dim, int64_t B, int64_t G, int64_t R) {
    CL_ARG(in_dim >= 0 && out_dim >= 0 && B >= 0, "negative dimension");
    CL_ARG(G >= 1 && G <= 128, "num_gates must be in [1, 128], got %lld", (long long)G);
    CL_ARG(R >= 0 && R < (int64_t(1) << 30), "num_runs out of range");
    CL_ARG(in_dim < (int64_t(1) << 31) && out_dim < (int64_t(1) << 31), "too many rows");
    return CL_OK;
}

}  // namespace

namespace {

// Calls f(std::integral_constant<int, VEC>, std::integral_constant<int, LPN>) for the
// tiling's vector width and lane-group size.
template <typename T, int MULT, typename F>
void with_tiling(const Tiling& tl, F&& f) {
    constexpr int W = wide_vec<T>();
    using I = std::integral_constant<int, 1>;
    using IW = std::integral_constant<int, W>;
    using IM = std::integral_constant<int, W * MULT>;
    using L4 = std::integral_constant<int, 4>;
    using L8 = std::integral_constant<int, 8>;
    using L16 = std::integral_constant<int, 16>;
    auto by_lanes = [&](auto vc) {
        if (tl.lpn == 16) f(vc, L16{});
        else if (tl.lpn == 8) f(vc, L8{});
        else f(vc, L4{});
    };
    if (MULT > 1 && tl.vec == W * MULT) by_lanes(IM{});
    else if (tl.vec == W) by_lanes(IW{});
    else by_lanes(I{});
}

}  // namespace

extern "C" int cl_dense_prep(int dtype, const void* w, int softmax, const uint8_t* gate_seq,
                             const int32_t* run_ptr, const int32_t* run_gl,
                             const int32_t* inv_pos, void* probs, void* run_coef,
                             void* inv_coef, int64_t out_dim, int64_t num_runs,
                             int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(1, out_dim, 0, num_gates, num_runs)) return rc;
    if (out_dim == 0) return CL_OK;
    CL_ARG(w && gate_seq && run_ptr && run_gl && run_coef, "null pointer argument");
    CL_ARG(!inv_coef || inv_pos, "inv_coef needs inv_pos");
    CL_DTYPE_SWITCH(dtype, {
        k_prep<scalar_t><<<unsigned(ceil_div(out_dim, 16)), 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(w), softmax, gate_seq, run_ptr, run_gl, inv_pos,
            static_cast<scalar_t*>(probs), static_cast<scalar_t*>(run_coef),
            static_cast<scalar_t*>(inv_coef), out_dim, num_runs, int(num_gates));
    });
    return check_launch("cl_dense_prep");
}

extern "C" int cl_dense_forward_tiled(int dtype, const void* x, const void* run_coef,
                                      const int32_t* nab, const int32_t* run_ab, void* y,
                                      int64_t in_dim, int64_t out_dim, int64_t num_runs,
                                      int64_t batch, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, 1, num_runs)) return rc;
    if (out_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && run_coef && nab && run_ab && y, "null pointer argument");
    CL_ARG(aligned(run_ab, 8) && aligned(nab, 16) && aligned(run_coef, 16),
           "run_ab / nab / run_coef misaligned");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        CL_ARG(!vec_ok<T>(batch) || all_aligned({x, y}), "x and y must be 16-byte aligned");
        const Tiling tl = choose_tiling<T>(batch, out_dim, CL_FWD_VEC_MULT, CL_FWD_LPN, CL_FWD_NPG);
        const unsigned grid = unsigned(tile_grid(tl.map));
        auto* xs = static_cast<const T*>(x);
        auto* kc = static_cast<const T*>(run_coef);
        auto* nb = reinterpret_cast<const int4*>(nab);
        auto* ab = reinterpret_cast<const int2*>(run_ab);
        auto* ys = static_cast<T*>(y);
        with_tiling<T, CL_FWD_VEC_MULT>(tl, [&](auto vc, auto lc) {
            k_fwd_tiled<T, decltype(vc)::value, decltype(lc)::value, CL_FWD_NPG>
                <<<grid, 256, 0, s>>>(xs, kc, nb, ab, ys, in_dim, out_dim, num_runs, batch, tl.map);
        });
    });
    return check_launch("cl_dense_forward_tiled");
}

extern "C" int cl_dense_forward_fused(int dtype, const void* x, const void* w, int softmax,
                                      const uint8_t* gate_seq, const int32_t* nab,
                                      const int32_t* inv_pos, void* probs, void* inv_coef,
                                      void* y, int64_t in_dim, int64_t out_dim,
                                      int64_t num_runs, int64_t batch, int64_t num_gates,
                                      void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, num_gates, num_runs)) return rc;
    CL_ARG(num_gates <= 16, "the fused forward takes at most 16 slots, got %lld",
           (long long)num_gates);
    CL_ARG(batch >= 1, "the fused forward needs batch >= 1 (use cl_dense_prep)");
    if (out_dim == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && w && gate_seq && nab && y, "null pointer argument");
    CL_ARG(!inv_coef || inv_pos, "inv_coef needs inv_pos");
    CL_ARG(aligned(nab, 16), "nab misaligned");
    CL_ARG(num_runs >= 1, "num_runs must be >= 1 when out_dim > 0");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        CL_ARG(!vec_ok<T>(batch) || all_aligned({x, y}), "x and y must be 16-byte aligned");
        const Tiling tl = choose_tiling<T>(batch, out_dim, CL_FUSED_VEC_MULT, CL_FWD_LPN, CL_FWD_NPG);
        const unsigned grid = unsigned(tile_grid(tl.map));
        auto* xs = static_cast<const T*>(x);
        auto* ws = static_cast<const T*>(w);
        auto* nb = reinterpret_cast<const int4*>(nab);
        auto* pr = static_cast<T*>(probs);
        auto* ic = static_cast<T*>(inv_coef);
        auto* ys = static_cast<T*>(y);
        with_tiling<T, CL_FUSED_VEC_MULT>(tl, [&](auto vc, auto lc) {
            constexpr int VEC = decltype(vc)::value, LPN = decltype(lc)::value;
            if (ic)
                k_fwd_fused<T, VEC, LPN, CL_FWD_NPG, true, false><<<grid, 256, 0, s>>>(
                    xs, ws, softmax, gate_seq, nb, inv_pos, pr, ic, ys, in_dim, out_dim, num_runs,
                    batch, int(num_gates), tl.map, nullptr, 0);
            else
                k_fwd_fused<T, VEC, LPN, CL_FWD_NPG, false, false><<<grid, 256, 0, s>>>(
                    xs, ws, softmax, gate_seq, nb, inv_pos, pr, ic, ys, in_dim, out_dim, num_runs,
                    batch, int(num_gates), tl.map, nullptr, 0);
        });
    });
    return check_launch("cl_dense_forward_fused");
}

extern "C" int cl_dense_weight_grad(int dtype, const void* x, const void* grad_y,
                                    const uint8_t* gate_seq, const void* probs,
                                    const int32_t* run_ptr, const int32_t* run_ab,
                                    const int32_t* run_gl, void* grad_w, int64_t in_dim,
                                    int64_t out_dim, int64_t num_runs, int64_t batch,
                                    int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, num_gates, num_runs)) return rc;
    if (out_dim == 0) return CL_OK;
    CL_ARG(gate_seq && run_ptr && run_ab && run_gl && grad_w, "null pointer argument");
    CL_ARG(batch == 0 || (x && grad_y), "null pointer argument");
    CL_ARG(aligned(run_ab, 8), "run_ab misaligned");
    CL_ARG(num_runs >= 1, "num_runs must be >= 1 when out_dim > 0");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        constexpr int W = wide_vec<T>();
        const bool v = vec_ok<T>(batch);
        CL_ARG(!v || all_aligned({x, grad_y}), "x and grad_y must be 16-byte aligned");
        const unsigned grid = unsigned(ceil_div(out_dim, 16));
        auto* xs = static_cast<const T*>(x);
        auto* gys = static_cast<const T*>(grad_y);
        auto* pr = static_cast<const T*>(probs);
        auto* ab = reinterpret_cast<const int2*>(run_ab);
        auto* gw = static_cast<T*>(grad_w);
        if (v && batch > 0 && num_gates <= 64 && batch <= 64 * W * 8) {
            const unsigned wgrid = unsigned(ceil_div(out_dim, int64_t(4)));
            auto go = [&](auto uc) {
                constexpr int U = decltype(uc)::value;
                if (pr)
                    k_wgrad_rows<T, W, U, true><<<wgrid, 256, 0, s>>>(
                        xs, gys, gate_seq, pr, run_ptr, ab, run_gl, gw,
                        std::max<int64_t>(in_dim, 1), out_dim, num_runs, batch, int(num_gates));
                else
                    k_wgrad_rows<T, W, U, false><<<wgrid, 256, 0, s>>>(
                        xs, gys, gate_seq, pr, run_ptr, ab, run_gl, gw,
                        std::max<int64_t>(in_dim, 1), out_dim, num_runs, batch, int(num_gates));
            };
            const int64_t per_u = 64 * W;
            if (batch <= per_u) go(std::integral_constant<int, 1>{});
            else if (batch <= 2 * per_u) go(std::integral_constant<int, 2>{});
            else if (batch <= 4 * per_u) go(std::integral_constant<int, 4>{});
            else go(std::integral_constant<int, 8>{});
        } else if (v)
            k_wgrad_full<T, W><<<grid, 256, 0, s>>>(xs, gys, gate_seq, pr, run_ptr, ab, run_gl, gw,
                                                   std::max<int64_t>(in_dim, 1), out_dim, num_runs,
                                                   batch, int(num_gates));
        else
            k_wgrad_full<T, 1><<<grid, 256, 0, s>>>(xs, gys, gate_seq, pr, run_ptr, ab, run_gl, gw,
                                                   std::max<int64_t>(in_dim, 1), out_dim, num_runs,
                                                   batch, int(num_gates));
    });
    return check_launch("cl_dense_weight_grad");
}

extern "C" int cl_dense_tiled_chunks(int dtype, int64_t batch, int64_t in_dim, int64_t out_dim,
                                     int64_t* nchunks) {
    clear_error();
    CL_ARG(nchunks && batch >= 0, "bad argument");
    // Chunks of the backward tiling: they depend on the batch (and dtype) only.
    (void)in_dim;
    (void)out_dim;
    CL_DTYPE_SWITCH(dtype, {
        const int64_t b = std::max<int64_t>(batch, 1);
        *nchunks = choose_tiling<scalar_t>(b, 1, CL_BWD_VEC_MULT, CL_BWD_LPN).map.nchunks;
    });
    return CL_OK;
}

extern "C" int cl_dense_backward_tiled(int dtype, const void* x, const void* grad_y,
                                       const int32_t* run_ptr, const int32_t* run_ab,
                                       const int32_t* slot_rec, const int32_t* inv_rec,
                                       const void* inv_coef, void* grad_x, void* moments,
                                       int64_t nchunks,
                                       int64_t in_dim, int64_t out_dim, int64_t num_runs,
                                       int64_t batch, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, 1, num_runs)) return rc;
    if (!grad_x && !moments) return CL_OK;
    if (batch == 0) {
        // Empty batch: all moments are zero (a fill kernel, so the call stays graph-safe).
        CL_ARG(!moments || nchunks >= 1, "nchunks must be >= 1");
        if (moments && num_runs > 0) {
            const int64_t n = num_runs * nchunks * 4;
            CL_DTYPE_SWITCH(dtype, {
                k_zero<scalar_t><<<unsigned(std::min<int64_t>(ceil_div(n, 256), 65535)), 256, 0,
                                   as_stream(stream)>>>(static_cast<scalar_t*>(moments), n);
            });
        }
        return check_launch("cl_dense_backward_tiled(zero)");
    }
    CL_ARG(x && grad_y, "null pointer argument");
    if (grad_x)
        CL_ARG(slot_rec && inv_rec && inv_coef && aligned(slot_rec, 16) && aligned(inv_rec, 16) &&
                   aligned(inv_coef, 8),
               "grad_x needs slot_rec, inv_rec (16-byte aligned) and inv_coef");
    if (moments) CL_ARG(aligned(moments, 16), "moments must be 16-byte aligned");
    if (moments && !grad_x)
        CL_ARG(run_ptr && run_ab && aligned(run_ab, 8), "moments need run_ptr and run_ab");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const bool v = vec_ok<T>(batch);
        CL_ARG(!v || all_aligned({x, grad_y, grad_x}), "row buffers must be 16-byte aligned");
        auto* xs = static_cast<const T*>(x);
        auto* gys = static_cast<const T*>(grad_y);
        auto* ab = reinterpret_cast<const int2*>(run_ab);
        auto* rec = reinterpret_cast<const int4*>(inv_rec);
        auto* srec = reinterpret_cast<const int4*>(slot_rec);
        auto* ic = static_cast<const T*>(inv_coef);
        auto* gxs = static_cast<T*>(grad_x);
        auto* mom = static_cast<T*>(moments);
        if (grad_x && in_dim > 0) {
            const Tiling tl = choose_tiling<T>(batch, in_dim, CL_BWD_VEC_MULT, CL_BWD_LPN, CL_BWD_NPG);
            const unsigned grid = unsigned(tile_grid(tl.map));
            if (moments) {
                CL_ARG(nchunks == tl.map.nchunks, "moments buffer must use the backward chunk count");
                with_tiling<T, CL_BWD_VEC_MULT>(tl, [&](auto vc, auto lc) {
                    k_bwd_tiled<T, decltype(vc)::value, decltype(lc)::value, CL_BWD_NPG, true, true>
                        <<<grid, 256, 0, s>>>(xs, gys, srec, rec, ic, gxs, mom,
                                              in_dim, out_dim, num_runs, batch, tl.map);
                });
            } else {
                with_tiling<T, CL_BWD_VEC_MULT>(tl, [&](auto vc, auto lc) {
                    k_bwd_tiled<T, decltype(vc)::value, decltype(lc)::value, CL_BWD_NPG, true, false>
                        <<<grid, 256, 0, s>>>(xs, gys, srec, rec, ic, gxs, mom,
                                              in_dim, out_dim, num_runs, batch, tl.map);
                });
            }
        } else if (moments && out_dim > 0) {
            const Tiling tl = choose_tiling<T>(batch, out_dim, CL_BWD_VEC_MULT, CL_BWD_LPN);
            CL_ARG(nchunks == tl.map.nchunks, "moments buffer must use the backward chunk count");
            const unsigned grid = unsigned(tile_grid(tl.map));
            with_tiling<T, CL_BWD_VEC_MULT>(tl, [&](auto vc, auto lc) {
                k_moments<T, decltype(vc)::value, decltype(lc)::value><<<grid, 256, 0, s>>>(
                    xs, gys, run_ptr, ab, mom, in_dim, out_dim, num_runs, batch, tl.map);
            });
        }
    });
    return check_launch("cl_dense_backward_tiled");
}

extern "C" int cl_dense_backward_part(int dtype, const void* x, const void* grad_y,
                                      const int32_t* slot_rec, const int32_t* inv_rec,
                                      const void* inv_coef, const int32_t* inv_slot,
                                      const int32_t* tile_ptr, const int32_t* tile_run,
                                      const int32_t* tile_loc, int64_t num_internal,
                                      int64_t part_slots, void* grad_x,
                                      void* moments, int64_t nchunks, int64_t in_dim,
                                      int64_t out_dim, int64_t num_runs, int64_t batch,
                                      void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, 1, num_runs)) return rc;
    CL_ARG(part_slots >= 2 && part_slots <= kPartMaxSlots && part_slots % 2 == 0,
           "part_slots must be even and in [2, %d]", kPartMaxSlots);
    CL_ARG(grad_x, "grad_x is required (use cl_dense_backward_tiled for moments alone)");
    CL_ARG(num_internal >= 0 && (num_internal == 0 || (tile_run && tile_loc)),
           "tile_run / tile_loc missing");
    if (batch == 0 || in_dim == 0)
        return cl_dense_backward_tiled(dtype, x, grad_y, nullptr, nullptr, slot_rec, inv_rec,
                                       inv_coef, grad_x, moments, nchunks, in_dim, out_dim,
                                       num_runs, batch, stream);
    CL_ARG(x && grad_y && slot_rec && inv_rec && inv_coef && inv_slot && tile_ptr,
           "null pointer argument");
    CL_ARG(aligned(slot_rec, 16) && aligned(inv_rec, 16) && aligned(inv_coef, 8) &&
               (!tile_run || aligned(tile_run, 16)),
           "slot_rec / inv_rec / tile_run must be 16-byte aligned, inv_coef 8-byte aligned");
    if (moments) CL_ARG(aligned(moments, 16), "moments must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const bool v = vec_ok<T>(batch);
        CL_ARG(!v || all_aligned({x, grad_y, grad_x}), "row buffers must be 16-byte aligned");
        const Tiling tl = choose_tiling<T>(batch, in_dim, CL_BWD_VEC_MULT, CL_BWD_LPN, 1);
        if (moments)
            CL_ARG(nchunks == tl.map.nchunks, "moments buffer must use the backward chunk count");
        const unsigned grid = unsigned(tile_grid(tl.map));
        auto* xs = static_cast<const T*>(x);
        auto* gys = static_cast<const T*>(grad_y);
        auto* rec = reinterpret_cast<const int4*>(inv_rec);
        auto* srec = reinterpret_cast<const int4*>(slot_rec);
        auto* trun = reinterpret_cast<const int4*>(tile_run);
        auto* ic = static_cast<const T*>(inv_coef);
        auto* gxs = static_cast<T*>(grad_x);
        auto* mom = static_cast<T*>(moments);
        with_tiling<T, CL_BWD_VEC_MULT>(tl, [&](auto vc, auto lc) {
            constexpr int VEC = decltype(vc)::value, LPN = decltype(lc)::value;
            const size_t lds = size_t(16 / LPN) * (kPartRows + part_slots) * LPN * VEC * sizeof(T);
            if (moments)
                k_bwd_part<T, VEC, LPN, true, true><<<grid, 256, lds, s>>>(
                    xs, gys, srec, rec, ic, inv_slot, tile_ptr, trun, tile_loc, num_internal, gxs, mom, in_dim,
                    out_dim, num_runs, batch, int(part_slots), tl.map);
            else
                k_bwd_part<T, VEC, LPN, true, false><<<grid, 256, lds, s>>>(
                    xs, gys, srec, rec, ic, inv_slot, tile_ptr, trun, tile_loc, num_internal, gxs, mom, in_dim,
                    out_dim, num_runs, batch, int(part_slots), tl.map);
        });
    });
    return check_launch("cl_dense_backward_part");
}

namespace {
// The first layer for k_bwd_rows' FIRST mode, untyped (see FirstLayer).
struct FirstArgs {
    const void* x0;
    const int32_t* nab;
    const uint8_t* gs;
    const void* probs;
    void* grad_w;
    int64_t in_dim, num_runs, G;
};

int backward_rows_impl(int dtype, const void* x, const void* grad_y, const int32_t* slot_rec,
                       const int32_t* inv_rec, const void* inv_coef, const uint8_t* gate_seq,
                       const void* probs, const int32_t* run_ptr, void* grad_w, void* grad_x,
                       int64_t in_dim, int64_t out_dim, int64_t num_runs, int64_t batch,
                       int64_t num_gates, uint32_t gy_magic, void* stream,
                       const FirstArgs* fa = nullptr) {
    if (int rc = check_plan_dims(in_dim, out_dim, batch, num_gates, num_runs)) return rc;
    CL_ARG(num_gates <= 64, "the row backward takes at most 64 slots, got %lld",
           (long long)num_gates);
    CL_ARG(grad_x || fa, "grad_x is required");
    if (in_dim == 0 || batch == 0) return CL_OK;
    CL_ARG(x && grad_y && slot_rec && inv_rec && inv_coef, "null pointer argument");
    CL_ARG(!grad_w || (gate_seq && run_ptr), "grad_w needs gate_seq and run_ptr");
    CL_ARG(aligned(slot_rec, 16) && aligned(inv_rec, 16) && aligned(inv_coef, 8),
           "slot_rec / inv_rec must be 16-byte aligned, inv_coef 8-byte aligned");
    if (fa) {
        CL_ARG(!grad_x, "the first layer's logits gradient replaces the input gradient");
        CL_ARG(grad_w && probs, "the first-layer mode needs grad_w and the softmax");
        CL_ARG(fa->x0 && fa->nab && fa->gs && fa->probs && fa->grad_w, "null pointer argument");
        CL_ARG(fa->G >= 1 && fa->G <= 64, "the first layer has 1 to 64 slots, got %lld",
               (long long)fa->G);
        CL_ARG(fa->in_dim >= 1 && fa->num_runs >= 0, "bad first-layer shape");
        CL_ARG(aligned(fa->nab, 16) && aligned(fa->x0, 16), "nab and x0 must be 16-byte aligned");
    }
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        constexpr int W = wide_vec<T>();
        CL_ARG(batch % W == 0 && batch <= 64 * W * 8,
               "the row backward needs batch %% %d == 0 and batch <= %d", W, 64 * W * 8);
        CL_ARG(all_aligned({x, grad_y}) && (!grad_x || aligned(grad_x, 16)),
               "row buffers must be 16-byte aligned");
        FirstLayer<T> first{};
        if (fa)
            first = FirstLayer<T>{static_cast<const T*>(fa->x0),
                                  reinterpret_cast<const int4*>(fa->nab), fa->gs,
                                  static_cast<const T*>(fa->probs), static_cast<T*>(fa->grad_w),
                                  fa->in_dim, fa->num_runs, int(fa->G)};
        // waves per row: rows with many entries (a narrow input feeding a wide layer) share
        // their entries among 2 or 4 waves
        const int64_t avg = in_dim > 0 ? 2 * num_runs / in_dim : 0;
        const int S = fa ? 1 : avg >= CL_BWD_ROWS_S4 ? 4 : avg >= CL_BWD_ROWS_S2 ? 2 : 1;
        const int64_t nblk = ceil_div(ceil_div(in_dim, int64_t(4 / S)), int64_t(kXcds));
        CL_ARG(kXcds * nblk < (int64_t(1) << 31), "too many rows");
        const unsigned grid = unsigned(kXcds * nblk);
        auto go = [&](auto uc) {
            constexpr int U = decltype(uc)::value;
            auto* xs = static_cast<const T*>(x);
            auto* gys = static_cast<const T*>(grad_y);
            auto* srec = reinterpret_cast<const int4*>(slot_rec);
            auto* rec = reinterpret_cast<const int4*>(inv_rec);
            auto* ic = static_cast<const T*>(inv_coef);
            auto* pr = static_cast<const T*>(probs);
            auto* gw = static_cast<T*>(grad_w);
            auto* gxs = static_cast<T*>(grad_x);
            auto launch = [&](auto gwc, auto pc) {
                constexpr bool GW = decltype(gwc)::value, HP = decltype(pc)::value;
                if (S == 4)
                    k_bwd_rows<T, W, U, GW, HP, false, 4><<<grid, 256, 0, s>>>(
                        xs, gys, srec, rec, ic, gate_seq, pr, run_ptr, gw, gxs, in_dim, out_dim,
                        num_runs, batch, int(num_gates), nblk, gy_magic);
                else if (S == 2)
                    k_bwd_rows<T, W, U, GW, HP, false, 2><<<grid, 256, 0, s>>>(
                        xs, gys, srec, rec, ic, gate_seq, pr, run_ptr, gw, gxs, in_dim, out_dim,
                        num_runs, batch, int(num_gates), nblk, gy_magic);
                else
                    k_bwd_rows<T, W, U, GW, HP><<<grid, 256, 0, s>>>(
                        xs, gys, srec, rec, ic, gate_seq, pr, run_ptr, gw, gxs, in_dim, out_dim,
                        num_runs, batch, int(num_gates), nblk, gy_magic);
            };
            using Y = std::true_type;
            using N = std::false_type;
            if (fa)
                k_bwd_rows<T, W, U, true, true, true>
                    <<<grid, 256, 0, s>>>(xs, gys, srec, rec, ic, gate_seq, pr, run_ptr, gw,
                                          nullptr, in_dim, out_dim, num_runs, batch,
                                          int(num_gates), nblk, gy_magic, first);
            else if (grad_w && probs) launch(Y{}, Y{});
            else if (grad_w) launch(Y{}, N{});
            else launch(N{}, N{});
        };
        const int64_t per_u = 64 * W;
        if (batch <= per_u) go(std::integral_constant<int, 1>{});
        else if (batch <= 2 * per_u) go(std::integral_constant<int, 2>{});
        else if (batch <= 4 * per_u) go(std::integral_constant<int, 4>{});
        else go(std::integral_constant<int, 8>{});
    });
    return check_launch("cl_dense_backward_rows");
}
}  // namespace

extern "C" int cl_dense_backward_rows_first(
    int dtype, const void* x, const void* grad_y, const int32_t* slot_rec,
    const int32_t* inv_rec, const void* inv_coef, const uint8_t* gate_seq, const void* probs,
    const int32_t* run_ptr, void* grad_w, int64_t in_dim, int64_t out_dim, int64_t num_runs,
    int64_t batch, int64_t num_gates, const void* x0, int64_t in0_dim, const int32_t* nab0,
    int64_t num_runs0, const uint8_t* gate_seq0, const void* probs0, void* grad_w0,
    int64_t num_gates0, void* stream) {
    clear_error();
    const FirstArgs fa{x0, nab0, gate_seq0, probs0, grad_w0, in0_dim, num_runs0, num_gates0};
    return backward_rows_impl(dtype, x, grad_y, slot_rec, inv_rec, inv_coef, gate_seq, probs,
                              run_ptr, grad_w, nullptr, in_dim, out_dim, num_runs, batch,
                              num_gates, 0, stream, &fa);
}

extern "C" int cl_dense_backward_rows(int dtype, const void* x, const void* grad_y,
                                      const int32_t* slot_rec, const int32_t* inv_rec,
                                      const void* inv_coef, const uint8_t* gate_seq,
                                      const void* probs, const int32_t* run_ptr, void* grad_w,
                                      void* grad_x, int64_t in_dim, int64_t out_dim,
                                      int64_t num_runs, int64_t batch, int64_t num_gates,
                                      void* stream) {
    clear_error();
    return backward_rows_impl(dtype, x, grad_y, slot_rec, inv_rec, inv_coef, gate_seq, probs,
                              run_ptr, grad_w, grad_x, in_dim, out_dim, num_runs, batch,
                              num_gates, 0, stream);
}

// ------------------------------------------------------------------------------------------
// The classifier head: the last dense layer, GroupSum(k, tau) and the mean cross-entropy in
// one autograd step.  The forward runs the fused forward kernel in its HEAD mode (the layer's
// outputs are never stored: each tile writes the sums of its rows by class), adds the tiles'
// partials per class and takes the softmax / loss as the GroupSum cross-entropy does.  The
// backward writes the class gradients [k, batch] (every row of a class has the same one) and
// runs the row backward with grad_y row o / gsz for neuron o.  Against the layer followed by
// GroupSum's cross-entropy this saves writing and re-reading the layer's output and its
// gradient (2 * 2 * out_dim * batch elements).
namespace {
constexpr int64_t kHeadSlices = 4;

struct HeadShape {
    Tiling tl;
    int64_t tile_rows, gsz, part_elems, slice_elems;
};

template <typename T>
bool head_shape(int64_t out_dim, int64_t batch, int64_t k, HeadShape& h) {
    h.tl = choose_tiling<T>(batch, out_dim, CL_FUSED_VEC_MULT, CL_FWD_LPN, CL_FWD_NPG);
    h.tile_rows = int64_t(256 / h.tl.lpn) * CL_FWD_NPG;
    h.gsz = ceil_div(out_dim, k);
    h.part_elems = h.tl.map.ntiles * 2 * batch;
    h.slice_elems = kHeadSlices * k * batch;
    // a tile spans at most two classes; o / gsz is an exact multiply-high for o < out_dim
    return h.tile_rows <= h.gsz && uint64_t(out_dim) * uint64_t(h.gsz) <= (uint64_t(1) << 32);
}
}  // namespace

extern "C" int cl_dense_group_sum_cross_entropy_workspace_size(int dtype, int64_t out_dim,
                                                              int64_t batch, int64_t k,
                                                              int64_t* forward_bytes,
                                                              int64_t* backward_bytes) {
    clear_error();
    CL_ARG(forward_bytes && backward_bytes, "null pointer argument");
    CL_ARG(out_dim >= 1 && batch >= 1 && k >= 1, "bad shape");
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        HeadShape h;
        if (!head_shape<T>(out_dim, batch, k, h)) {
            *forward_bytes = *backward_bytes = -1;  // the fused head does not apply
        } else {
            *forward_bytes = (h.part_elems + h.slice_elems + 2 * batch) * int64_t(sizeof(T));
            *backward_bytes = k * batch * int64_t(sizeof(T));
        }
    });
    return CL_OK;
}

extern "C" int cl_dense_group_sum_cross_entropy_forward(
    int dtype, const void* x, const void* w, int softmax, const uint8_t* gate_seq,
    const int32_t* nab, const int32_t* inv_pos, void* probs, void* inv_coef, int64_t in_dim,
    int64_t out_dim, int64_t num_runs, int64_t batch, int64_t num_gates, int64_t k, double tau,
    const int64_t* labels, int64_t ignore_index, void* scores, void* ce_probs, void* loss,
    void* count, void* workspace, int64_t workspace_bytes, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(in_dim, out_dim, batch, num_gates, num_runs)) return rc;
    CL_ARG(num_gates <= 16, "the fused forward takes at most 16 slots, got %lld",
           (long long)num_gates);
    CL_ARG(batch >= 1 && out_dim >= 1 && in_dim >= 1 && k >= 1, "bad shape");
    CL_ARG(num_runs >= 1, "num_runs must be >= 1 when out_dim > 0");
    CL_ARG(x && w && gate_seq && nab && inv_pos && inv_coef && labels && scores && ce_probs &&
               loss && count && workspace,
           "null pointer argument");
    CL_ARG(aligned(nab, 16), "nab misaligned");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        HeadShape h;
        CL_ARG(head_shape<T>(out_dim, batch, k, h),
               "the fused head needs classes of at least %d rows (and out_dim * rows per "
               "class <= 2^32)", 256 / CL_FWD_LPN * CL_FWD_NPG);
        const int64_t need = (h.part_elems + h.slice_elems + 2 * batch) * int64_t(sizeof(T));
        CL_ARG(workspace_bytes >= need,
               "workspace of %lld bytes needed (cl_dense_group_sum_cross_entropy_workspace_size)",
               (long long)need);
        CL_ARG(!vec_ok<T>(batch) || all_aligned({x, workspace}),
               "x and the workspace must be 16-byte aligned");
        T* part = static_cast<T*>(workspace);
        T* slices = part + h.part_elems;
        T* term = slices + h.slice_elems;
        const unsigned grid = unsigned(tile_grid(h.tl.map));
        with_tiling<T, CL_FUSED_VEC_MULT>(h.tl, [&](auto vc, auto lc) {
            constexpr int VEC = decltype(vc)::value, LPN = decltype(lc)::value;
            k_fwd_fused<T, VEC, LPN, CL_FWD_NPG, true, true><<<grid, 256, 0, s>>>(
                static_cast<const T*>(x), static_cast<const T*>(w), softmax, gate_seq,
                reinterpret_cast<const int4*>(nab), inv_pos, static_cast<T*>(probs),
                static_cast<T*>(inv_coef), nullptr, in_dim, out_dim, num_runs, batch,
                int(num_gates), h.tl.map, part, h.gsz);
        });
        if (int rc = check_launch("cl_dense_group_sum_cross_entropy_forward(layer)")) return rc;
        return ce_from_tile_partials(dtype, part, batch, out_dim, k, h.tile_rows, tau, labels,
                                     ignore_index, scores, ce_probs, loss, count, slices,
                                     kHeadSlices, term, s);
    });
    return CL_OK;
}

extern "C" int cl_dense_group_sum_cross_entropy_backward(
    int dtype, const void* x, const void* ce_probs, const int64_t* labels, int64_t ignore_index,
    const void* grad_loss, const void* count, int64_t k, double tau, const int32_t* slot_rec,
    const int32_t* inv_rec, const void* inv_coef, const uint8_t* gate_seq, const void* probs,
    const int32_t* run_ptr, void* grad_w, void* grad_x, int64_t in_dim, int64_t out_dim,
    int64_t num_runs, int64_t batch, int64_t num_gates, void* workspace,
    int64_t workspace_bytes, void* stream) {
    clear_error();
    CL_ARG(out_dim >= 1 && batch >= 1 && k >= 1, "bad shape");
    CL_ARG(workspace, "null pointer argument");
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        HeadShape h;
        CL_ARG(head_shape<T>(out_dim, batch, k, h), "the fused head does not apply to this shape");
        CL_ARG(workspace_bytes >= k * batch * int64_t(sizeof(T)),
               "workspace of %lld bytes needed", (long long)(k * batch * int64_t(sizeof(T))));
        CL_ARG(aligned(workspace, 16), "workspace must be 16-byte aligned");
        // class gradients, [k, batch]: grad_scores[n, c] / tau of the cross-entropy
        if (int rc = cl_group_sum_cross_entropy_backward(dtype, ce_probs, labels, ignore_index,
                                                         grad_loss, count, batch, k, k, tau,
                                                         workspace, 1, batch, stream))
            return rc;
        const uint32_t magic =
            h.gsz == 1 ? 0u : uint32_t(((uint64_t(1) << 32) + uint64_t(h.gsz) - 1) / uint64_t(h.gsz));
        return backward_rows_impl(dtype, x, workspace, slot_rec, inv_rec, inv_coef, gate_seq,
                                  probs, run_ptr, grad_w, grad_x, in_dim, out_dim, num_runs, batch,
                                  num_gates, magic, stream);
    });
    return CL_OK;
}

extern "C" int cl_dense_backward_finalize(int dtype, const void* moments, int64_t nchunks,
                                          const uint8_t* gate_seq, const void* probs,
                                          const int32_t* run_ptr, const int32_t* run_gl,
                                          void* grad_w, int64_t out_dim, int64_t num_runs,
                                          int64_t num_gates, void* stream) {
    clear_error();
    if (int rc = check_plan_dims(1, out_dim, 0, num_gates, num_runs)) return rc;
    if (out_dim == 0) return CL_OK;
    CL_ARG(nchunks >= 1, "nchunks must be >= 1");
    CL_ARG(gate_seq && run_ptr && run_gl && grad_w, "null pointer argument");
    CL_ARG(num_runs == 0 || moments, "null moments");
    CL_DTYPE_SWITCH(dtype, {
        k_finalize<scalar_t><<<unsigned(ceil_div(out_dim, 16)), 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(moments), nchunks, gate_seq,
            static_cast<const scalar_t*>(probs), run_ptr, run_gl,
            static_cast<scalar_t*>(grad_w), out_dim, num_runs, int(num_gates));
    });
    return check_launch("cl_dense_backward_finalize");
}
