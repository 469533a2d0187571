// Window path of the ConvLayer for gfx950: layers whose output channels each read a single
// input channel (ConvLayer's default num_chn = 1 wiring, compactlogic/compactlogic.py:678-683).
//
// Every slot of output channel c then reads two taps of the same input plane inside one
// KW x KW window anchored at (oy*s + oy0, ox*s + ox0), KW <= 3.  With the window values
// v_0 .. v_{P-1} (P = KW^2, zero outside the plane) the relaxed layer is a quadratic form
//     y = K + sum_k alpha_k v_k + sum_{k <= l} beta_kl v_k v_l
// whose coefficients collapse all G slots (slot g with taps (a, b) adds p_g * c0 to K,
// p_g * c1 to alpha_a, p_g * c2 to alpha_b and p_g * c3 to beta_{min(a,b) max(a,b)}).  So:
//   k_win_prep      softmax of the logits and the coefficients of every channel, summed in
//                   slot order (one wave per channel, lane j owns coefficient j)
//   k_win_fwd       one thread per output position of one (sample, input channel): loads the
//                   window once, evaluates every output channel reading that input channel
//   k_win_bwd_x     one workgroup per (sample, input channel): per position the derivative
//                   of sum_c gy_c y_c with respect to each window value, accumulated into an
//                   LDS copy of the input plane one window position at a time (positions map
//                   to distinct pixels for a fixed window index, so no two threads collide and
//                   the summation order is fixed)
//   k_win_moments   per (input channel, pair of output channels, sample chunk): the moments
//                   sum gy, sum gy v_k, sum gy v_k v_l over the chunk, reduced in a fixed order
//   k_win_finalize  moments summed over chunks in order -> gradient of every slot -> softmax
//                   backward -> gradient of the logits
// The coefficient block of a channel is [K, alpha_0 .. alpha_{P-1}, beta_00, beta_01, ...,
// beta_{P-1,P-1}] (upper triangle by rows), padded to a multiple of 4.
#include "common.h"

#include <algorithm>

namespace cl {
namespace {

template <int KW>
struct Win {
    static constexpr int P = KW * KW;
    static constexpr int NP = P * (P + 1) / 2;
    static constexpr int CW = (1 + P + NP + 3) & ~3;
};

// Index of beta_kl (k <= l) inside the coefficient block.
__host__ __device__ constexpr int beta_at(int P, int k, int l) {
    return 1 + P + k * P - k * (k - 1) / 2 + (l - k);
}

int coef_width(int kw) {
    switch (kw) {
        case 1: return Win<1>::CW;
        case 2: return Win<2>::CW;
        case 3: return Win<3>::CW;
        default: return 0;
    }
}

// ------------------------------------------------------------------------------------------
template <typename T, int KW>
__global__ __launch_bounds__(256) void k_win_prep(const T* __restrict__ w, int softmax,
                                                  const uint8_t* __restrict__ gs,
                                                  const int32_t* __restrict__ slot_win,
                                                  T* __restrict__ probs, T* __restrict__ coef,
                                                  int64_t Cout, int G) {
    constexpr int P = Win<KW>::P, CW = Win<KW>::CW;
    const int64_t c = int64_t(blockIdx.x) * 4 + wave_id();
    if (c >= Cout) return;  // uniform per wave
    const int l = lane_id();
    // every load of the channel first (lane g holds gate g's logit, opcode and taps)
    T p = l < G ? w[c * G + l] : T(0);
    const int op = l < G ? int(gs[c * G + l]) : 0;
    const int rec_l = l < G ? slot_win[c * G + l] : 0;
    if (softmax) {
        T m = l < G ? p : -__builtin_inf();
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = std::max(m, __shfl_xor(m, off, kWave));
        const T e = l < G ? T(exp(p - m)) : T(0);
        p = e / wave_total(e);
    }
    if (probs && l < G) probs[c * G + l] = p;
    T acc = 0;
    for (int g = 0; g < G; ++g) {
        const T pg = read_lane(p, g);
        const Coef4<T> cf = gate_coef<T>(uint8_t(read_lane(op, g)));
        const int rec = read_lane(rec_l, g);
        const int ka = rec & 0xff, kb = (rec >> 8) & 0xff;
        const int lo = std::min(ka, kb), hi = std::max(ka, kb);
        T add = 0;
        if (l == 0) add += pg * cf.c0;
        if (l == 1 + ka) add += pg * cf.c1;
        if (l == 1 + kb) add += pg * cf.c2;
        if (l == beta_at(P, lo, hi)) add += pg * cf.c3;
        acc += add;
    }
    if (l < CW) coef[c * CW + l] = acc;
}

// Window values of the thread's output position; zero outside the plane or past the end.
// INTERIOR: every window of every active position lies inside the plane (checked on the host),
// so only `active` is tested.
template <typename T, int KW, bool INTERIOR = false>
__device__ __forceinline__ void load_window(T (&v)[KW * KW], const T* __restrict__ plane, int H,
                                            int W, int by, int bx, bool active) {
#pragma unroll
    for (int kh = 0; kh < KW; ++kh) {
#pragma unroll
        for (int kw = 0; kw < KW; ++kw) {
            const int yy = by + kh, xx = bx + kw;
            const bool ok = active && (INTERIOR || (unsigned(yy) < unsigned(H) &&
                                                    unsigned(xx) < unsigned(W)));
            v[kh * KW + kw] = ok ? plane[yy * W + xx] : T(0);
        }
    }
}

struct WinDims {
    int64_t N, Cin, Cout;
    int H, W, Ho, Wo, stride, oy0, ox0;
};

// ------------------------------------------------------------------------------------------
// Block = BS threads over the output positions of sample n and input channel ch, and part
// `part` of split equal parts of the channel's output channels
// (blockIdx.x = ((n * Cin + ch) * pchunks + chunk) * split + part).
//
// PACK (small planes): a block of 256 threads takes spb = 256 / hw samples of input channel ch
// instead (blockIdx.x = ((n / spb) * Cin + ch) * split + part; thread t: sample t / hw, position
// t % hw), so that few lanes idle; pchunks is then spb.
template <typename T, int KW, int SPLIT, bool PACK, bool INTERIOR>
__global__ __launch_bounds__(256) void k_win_fwd(const T* __restrict__ x, const T* __restrict__ coef,
                                                 const int32_t* __restrict__ grp_ptr,
                                                 const int32_t* __restrict__ chan_order,
                                                 T* __restrict__ y, int pchunks, WinDims d) {
    constexpr int P = Win<KW>::P, CW = Win<KW>::CW;
    const int64_t blk = blockIdx.x / SPLIT;
    const int part = int(blockIdx.x % SPLIT);
    const int hw = d.Ho * d.Wo;
    int64_t ch, n;
    int pos;
    if constexpr (PACK) {
        ch = blk % d.Cin;
        const int s = int(threadIdx.x) / hw;
        pos = int(threadIdx.x) - s * hw;
        n = (blk / d.Cin) * pchunks + s;
        if (s >= pchunks || n >= d.N) return;
    } else {
        const int chunk = int(blk % pchunks);
        const int64_t nc = blk / pchunks;
        ch = nc % d.Cin;
        n = nc / d.Cin;
        pos = chunk * int(blockDim.x) + int(threadIdx.x);
    }
    const int g0 = grp_ptr[ch], g1 = grp_ptr[ch + 1];
    const int c0 = g0 + (g1 - g0) * part / SPLIT;
    const int c1 = g0 + (g1 - g0) * (part + 1) / SPLIT;
    if (c0 == c1 || pos >= hw) return;
    const int oy = pos / d.Wo, ox = pos - oy * d.Wo;
    T v[P];
    load_window<T, KW, INTERIOR>(v, x + (n * d.Cin + ch) * int64_t(d.H) * d.W, d.H, d.W,
                                 oy * d.stride + d.oy0, ox * d.stride + d.ox0, true);
    T* yn = y + n * d.Cout * hw + pos;
#pragma unroll 2
    for (int i = c0; i < c1; ++i) {
        const int c = chan_order[i];
        const T* cf = coef + int64_t(c) * CW;
        T acc = cf[0];
#pragma unroll
        for (int k = 0; k < P; ++k) {
            T t = cf[1 + k];
#pragma unroll
            for (int l = k; l < P; ++l) t = fma(cf[beta_at(P, k, l)], v[l], t);
            acc = fma(v[k], t, acc);
        }
        yn[int64_t(c) * hw] = acc;
    }
}

// ------------------------------------------------------------------------------------------
// Block (sample n, input channel ch): BS >= Ho * Wo threads, one per output position; the
// input-gradient plane of (n, ch) is built in LDS and written out whole.
//
// LDS layout of the plane (WinPlane): rows and columns split by their phase modulo ps (the
// stride, or 1 when the split plane does not fit), pixel (yy, xx) at
// ((yy % ps) * hs + yy / ps) * pitch + (yy % ps) * rgap + (xx % ps) * ws + xx / ps, with hs, ws
// the rows / columns of one phase.  Tap k of output position (oy, ox) then lands at base + tap[k], base =
// oy * pitch + ox when ps is the stride (> 1), else base = by * pitch + bx for the window's
// corner (by, bx); with pitch congruent to Wo modulo 32 the 32 lanes of a half-wave
// (consecutive positions) add to 32 distinct banks.  With pos = oy * Wo + ox both bases are
// oy * la + pos * lb + lc for uniform la, lb, lc, taken modulo 2^32 (exact for every lane
// that adds, whose index lies in the plane).
//
// The plane is written out in row-major order; when the block size is a multiple of ps * W a
// thread keeps one column and its LDS index moves by st_step per pass (else st_step = 0 and
// every pixel's index is computed).  The gap rgap between the phases' row blocks makes row
// yy + 1 start W banks after row yy when yy % ps < ps - 1, so that a half-wave reading ps
// rows of ps * W <= 32 pixels meets each bank once.
struct WinPlane {
    int ps, hs, ws, pitch, rgap, words, st_step, la, lb, lc;
    int tap[9];
    float inv_w, inv_ps, inv_wo;  // 1 / W, 1 / ps and 1 / Wo rounded to float
    FastDiv div_cin;
};

// floor(x / d) from inv = 1 / d rounded to float, for 0 <= x < 2^22: (x + 0.5) inv carries a
// relative error below 2^-23, less than the distance 0.5 / d of (x + 0.5) / d to the nearest
// integer.  Full-rate float instructions in place of 32-bit integer products.
__device__ __forceinline__ int small_div(int x, float inv) {
    return int(fmaf(float(x), inv, 0.5f * inv));
}

// LDS index of pixel i of the H x W plane in the WinPlane layout (i < 2^22, so every product
// below fits 24 bits).
__device__ __forceinline__ int win_plane_at(int i, int W, const WinPlane& lp) {
    const int yy = small_div(i, lp.inv_w), xx = i - __mul24(yy, W);
    const int qy = small_div(yy, lp.inv_ps), qx = small_div(xx, lp.inv_ps);
    const int py = yy - __mul24(qy, lp.ps);
    return __mul24(__mul24(py, lp.hs) + qy, lp.pitch) + __mul24(py, lp.rgap) +
           __mul24(xx - __mul24(qx, lp.ps), lp.ws) + qx;
}

template <typename T, int KW, bool INTERIOR>
__global__ __launch_bounds__(1024) void k_win_bwd_x(const T* __restrict__ x,
                                                    const T* __restrict__ gy,
                                                    const T* __restrict__ coef,
                                                    const int32_t* __restrict__ grp_ptr,
                                                    const int32_t* __restrict__ chan_order,
                                                    T* __restrict__ gx, WinDims d, WinPlane lp) {
    constexpr int P = Win<KW>::P, NP = Win<KW>::NP, CW = Win<KW>::CW;
    extern __shared__ __align__(16) unsigned char smem[];
    T* plane = reinterpret_cast<T*>(smem);
    // block = plane n * Cin + ch (fewer than 2^31 blocks)
    const uint32_t n = fast_div(blockIdx.x, lp.div_cin), ch = blockIdx.x - n * uint32_t(d.Cin);
    const int hw = d.Ho * d.Wo, HW = d.H * d.W;
    const int words = lp.words;
    const int pos = threadIdx.x;
    const bool active = pos < hw;
    const int oy = active ? small_div(pos, lp.inv_wo) : 0, ox = active ? pos - oy * d.Wo : 0;
    const int by = oy * d.stride + d.oy0, bx = ox * d.stride + d.ox0;
    const int lane_base =
        int(uint32_t(oy) * uint32_t(lp.la) + uint32_t(pos) * uint32_t(lp.lb) + uint32_t(lp.lc));
    const T* xplane = x + int64_t(blockIdx.x) * HW;
    T v[P];
    load_window<T, KW, INTERIOR>(v, xplane, d.H, d.W, by, bx, active);
    // A_k = sum_c gy_c alpha_kc, B_kl = sum_c gy_c beta_klc over the channels reading ch
    T A[P], B[NP];
#pragma unroll
    for (int k = 0; k < P; ++k) A[k] = 0;
#pragma unroll
    for (int q = 0; q < NP; ++q) B[q] = 0;
    const int c0 = grp_ptr[ch], c1 = grp_ptr[ch + 1];
    const T* gyn = gy + int64_t(n) * d.Cout * hw + pos;
    for (int i = c0; i < c1; ++i) {
        const int c = chan_order[i];
        const T g = active ? gyn[int64_t(c) * hw] : T(0);
        const T* cf = coef + int64_t(c) * CW;
#pragma unroll
        for (int k = 0; k < P; ++k) A[k] = fma(g, cf[1 + k], A[k]);
#pragma unroll
        for (int q = 0; q < NP; ++q) B[q] = fma(g, cf[1 + P + q], B[q]);
    }
    // +0 in 16-byte stores (the allocation is rounded up to 16 bytes)
    const int zvec = (words * int(sizeof(T)) + 15) / 16;
    uint4* zero = reinterpret_cast<uint4*>(smem);
    for (int i = threadIdx.x; i < zvec; i += blockDim.x) zero[i] = uint4{0, 0, 0, 0};
    __syncthreads();
#pragma unroll
    for (int k = 0; k < P; ++k) {
        // d(sum_c gy_c y_c)/dv_k = A_k + sum_{l != k} B_{kl} v_l + 2 B_kk v_k
        T dk = A[k];
#pragma unroll
        for (int l = 0; l < P; ++l) {
            const int q = (l < k ? beta_at(P, l, k) : beta_at(P, k, l)) - 1 - P;
            dk = fma(l == k ? T(2) * B[q] : B[q], v[l], dk);
        }
        const int yy = by + k / KW, xx = bx + k % KW;
        if (active && (INTERIOR || (unsigned(yy) < unsigned(d.H) && unsigned(xx) < unsigned(d.W))))
            plane[lane_base + lp.tap[k]] += dk;
        __syncthreads();
    }
    T* gplane = gx + int64_t(blockIdx.x) * HW;
    if (lp.st_step) {
        int i = threadIdx.x;
        for (int at = i < HW ? win_plane_at(i, d.W, lp) : 0; i < HW; i += blockDim.x)
            gplane[i] = plane[at], at += lp.st_step;
    } else {
        for (int i = threadIdx.x; i < HW; i += blockDim.x)
            gplane[i] = plane[win_plane_at(i, d.W, lp)];
    }
}

// ------------------------------------------------------------------------------------------
// Moments: block (ch, sub-block sb of CB channels, sample chunk q) of 256 threads; the
// threads stride over the chunk's (sample, position) elements.  part[q, c, j] for j < CW.
// The closing reduction adds quads with DPP, then the 16 quad sums of each of the 4 waves in
// a fixed order through LDS.
template <typename T, int KW, int CB, bool INTERIOR>
__global__ __launch_bounds__(256) void k_win_moments(const T* __restrict__ x,
                                                     const T* __restrict__ gy,
                                                     const int32_t* __restrict__ grp_ptr,
                                                     const int32_t* __restrict__ chan_order,
                                                     T* __restrict__ part, int nsub, int nq,
                                                     WinDims d) {
    constexpr int P = Win<KW>::P, NM = 1 + P + Win<KW>::NP, CW = Win<KW>::CW;
    constexpr int BS = 256;
    __shared__ T red[BS / 4][CB * NM];
    const int q = blockIdx.y;
    const int64_t ch = blockIdx.x / nsub;
    const int sb = blockIdx.x % nsub;
    const int g0 = grp_ptr[ch] + sb * CB, g1 = std::min(grp_ptr[ch + 1], g0 + CB);
    if (g0 >= g1) return;  // uniform per block
    int cs[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) cs[j] = g0 + j < g1 ? chan_order[g0 + j] : -1;
    const int hw = d.Ho * d.Wo, HW = d.H * d.W;
    const int64_t n0 = q * d.N / nq, n1 = (q + 1) * d.N / nq;
    const int64_t cnt = (n1 - n0) * hw;
    T S[CB][NM];
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int m = 0; m < NM; ++m) S[j][m] = 0;
    // element e = (n - n0) * hw + oy * Wo + ox, advanced by BS per step without a division
    const int dn = BS / hw, dp = BS % hw;
    const int dy = dp / d.Wo, dx = dp % d.Wo;
    int64_t n = n0 + threadIdx.x / hw;
    const int pos0 = threadIdx.x % hw;
    int oy = pos0 / d.Wo, ox = pos0 % d.Wo;
    for (int64_t e = threadIdx.x; e < cnt; e += BS) {
        const int pos = oy * d.Wo + ox;
        T v[P];
        load_window<T, KW, INTERIOR>(v, x + (n * d.Cin + ch) * int64_t(HW), d.H, d.W,
                                     oy * d.stride + d.oy0, ox * d.stride + d.ox0, true);
        const T* gyn = gy + int64_t(n) * d.Cout * hw + pos;
        n += dn;
        oy += dy;
        ox += dx;
        if (ox >= d.Wo) {
            ox -= d.Wo;
            ++oy;
        }
        if (oy >= d.Ho) {
            oy -= d.Ho;
            ++n;
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const T g = cs[j] >= 0 ? gyn[int64_t(cs[j]) * hw] : T(0);
            S[j][0] += g;
#pragma unroll
            for (int k = 0; k < P; ++k) {
                const T gv = g * v[k];
                S[j][1 + k] += gv;
#pragma unroll
                for (int l = k; l < P; ++l) S[j][beta_at(P, k, l)] = fma(gv, v[l], S[j][beta_at(P, k, l)]);
            }
        }
    }
    const bool quad_lead = (threadIdx.x & 3) == 0;
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            T t = S[j][m];
            t += dpp_move<0xB1>(t);  // quad_perm [1,0,3,2]
            t += dpp_move<0x4E>(t);  // quad_perm [2,3,0,1]
            if (quad_lead) red[threadIdx.x >> 2][j * NM + m] = t;
        }
    __syncthreads();
    for (int i = threadIdx.x; i < CB * CW; i += BS) {
        const int j = i / CW, m = i % CW;
        if (cs[j] < 0) continue;
        T t = 0;
        if (m < NM)
            for (int r = 0; r < BS / 4; ++r) t += red[r][j * NM + m];
        part[(int64_t(q) * d.Cout + cs[j]) * CW + m] = t;
    }
}

// ------------------------------------------------------------------------------------------
// Moments of input channels read by many output channels (cfg3's first layer: about 28 per
// input channel), as a register-tiled product on the VALU.  For input channel ch the moments
// of its output channels c are M[c][m] = sum_e gy_c(e) f_m(e) over the elements e = (sample,
// position), with the 64 features f_m(e) = [1, v_k, v_k v_l (k <= l), 0 ...] of e's window in
// the coefficient-block order (padded with zeros past NM).  One wave per (ch, tile of 32 of its
// channels, element chunk q): the elements are taken 32 at a time; the wave stages the 32 x 32
// grad_y values and the 32 x 64 features in LDS, then lane (cq, fg) adds gy * f for channels
// 4 cq .. 4 cq + 3 and features 8 fg .. 8 fg + 7 of every staged element, in element order.
// The window is loaded once per element for all the tile's channels (the per-channel-pair
// kernel above loads it once per pair).  Feature group fg sits at LDS offsets off0(fg) and
// off0(fg) ^ 4 (floats) of an element's row, so the eight groups' 16-byte reads of a half
// fall on distinct banks.
constexpr int kMmTile = 32;     // output channels per wave
constexpr int kMmSlab = 32;     // elements staged at a time
constexpr int kMmFeat = 64;     // features per element (>= NM, padded)
#ifndef CL_WIN_MM_NWAVES
#define CL_WIN_MM_NWAVES 4
#endif
constexpr int kMmWaves = CL_WIN_MM_NWAVES;  // waves per workgroup, each taking every kMmWaves-th slab

// LDS position of feature m in an element's row: group fg = m / 8 owns floats 8 fg .. 8 fg + 7;
// its first half (features 8 fg .. + 3) sits in the upper four of them when fg >= 4.
__host__ __device__ constexpr int mm_first(int fg) { return 8 * fg + 4 * (fg >> 2); }
__host__ __device__ constexpr int mm_second(int fg) { return 8 * fg + 4 * (1 - (fg >> 2)); }
__host__ __device__ constexpr int mm_pos(int m) {
    return ((m & 7) < 4 ? mm_first(m >> 3) : mm_second(m >> 3)) + (m & 3);
}

// (k, l) of the quadratic moments in coefficient-block order (row-major upper triangle)
template <int P>
struct BetaPairs {
    int k[P * (P + 1) / 2], l[P * (P + 1) / 2];
    constexpr BetaPairs() : k(), l() {
        int r = 0;
        for (int a = 0; a < P; ++a)
            for (int b = a; b < P; ++b) {
                k[r] = a;
                l[r] = b;
                ++r;
            }
    }
};

template <typename T, int KW>
__global__ __launch_bounds__(kMmWaves * 64) void k_win_moments_mm(
    const T* __restrict__ x, const T* __restrict__ gy, const int32_t* __restrict__ grp_ptr,
    const int32_t* __restrict__ chan_order, T* __restrict__ part, int ntile, int nq,
    WinDims d) {
    constexpr int P = Win<KW>::P, NM = 1 + P + Win<KW>::NP, CW = Win<KW>::CW;
    static_assert(NM <= kMmFeat, "too many features");
    typedef T V4 __attribute__((ext_vector_type(4)));
    // per wave: rows padded by 4 floats, so the staging writes of 32 elements spread over
    // 8 banks; the closing reduction reuses the feature buffers
    // (declared as 16-byte vectors, so the compiler knows the reads below are aligned)
    constexpr int GW = (kMmTile + 4) / 4, FW = (kMmFeat + 4) / 4;
    __shared__ V4 gs4[kMmWaves][kMmSlab][GW];    // [element][channel / 4]
    __shared__ V4 fs4[kMmWaves][kMmSlab][FW];    // [element][feature position / 4]
    static_assert(kMmWaves == 1 || sizeof(fs4) >= (kMmWaves - 1) * 64 * 32 * sizeof(T),
                  "reduction space");
    T* const gsw = reinterpret_cast<T*>(&gs4[0][0][0]);
    T* const fsw = reinterpret_cast<T*>(&fs4[0][0][0]);
    const int wv = wave_id(), lane = threadIdx.x & 63;
    const int q = blockIdx.y;
    const int ch = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    const int g0 = grp_ptr[ch] + tile * kMmTile, g1 = std::min(grp_ptr[ch + 1], g0 + kMmTile);
    if (g0 >= g1) return;  // uniform per workgroup
    const int hw = d.Ho * d.Wo, HW = d.H * d.W;
    const int E = int(d.N) * hw;  // < 2^31 (checked by the host)
    const int e0 = int(int64_t(q) * E / nq), e1 = int(int64_t(q + 1) * E / nq);
    const int nslab = (e1 - e0 + kMmSlab - 1) / kMmSlab;
    const int rounds = (nslab + kMmWaves - 1) / kMmWaves;  // equal for every wave
    // staging roles: element se = lane % 32; grad_y channels (lane / 32) * 16 .. + 15 of the
    // tile (clamped to a valid channel, masked after the load); features: lanes < 32 write
    // feature positions of features 0 .. 31, the others of 32 .. 63
    const int se = lane % kMmSlab, half = lane / kMmSlab;
    int coff[kMmTile / 2];
    bool cok[kMmTile / 2];
#pragma unroll
    for (int j = 0; j < kMmTile / 2; ++j) {
        const int gi = g0 + half * (kMmTile / 2) + j;
        cok[j] = gi < g1;
        coff[j] = chan_order[cok[j] ? gi : g0] * hw;
    }
    const int cq = lane / 8, fg = lane % 8;
    const int o0 = mm_first(fg) / 4, o1 = mm_second(fg) / 4;   // in 16-byte vectors
    T acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = T(0);
    constexpr BetaPairs<P> bp{};
    // The global loads of a slab (its window values and grad_y) are issued one slab ahead,
    // before the wave computes on the previous one, so the wave itself hides their latency.
    // Every load is unconditional (clamped address, value masked when used).
    auto issue = [&](int r, T (&vr)[P], T (&gr)[kMmTile / 2], bool& live, bool (&tin)[P]) {
        const int e = e0 + (r * kMmWaves + wv) * kMmSlab + se;
        live = r < rounds && e < e1;
        const int ec = live ? e : e0;
        const int n = ec / hw, pos = ec - n * hw;
        const int oy = pos / d.Wo, ox = pos - oy * d.Wo;
        const int by = oy * d.stride + d.oy0, bx = ox * d.stride + d.ox0;
        const T* plane = x + (int64_t(n) * d.Cin + ch) * HW;
#pragma unroll
        for (int k = 0; k < P; ++k) {
            const int yy = by + k / KW, xx = bx + k % KW;
            tin[k] = live && unsigned(yy) < unsigned(d.H) && unsigned(xx) < unsigned(d.W);
            vr[k] = plane[tin[k] ? yy * d.W + xx : 0];
        }
        const T* gyn = gy + int64_t(n) * d.Cout * hw + pos;
#pragma unroll
        for (int j = 0; j < kMmTile / 2; ++j) gr[j] = gyn[coff[j]];
    };
    T vn[P] = {}, gn[kMmTile / 2] = {};
    bool liven = false, tinn[P] = {};
    if (rounds > 0) issue(0, vn, gn, liven, tinn);  // an empty chunk reads nothing
    for (int r = 0; r < rounds; ++r) {
        T v[P], gv[kMmTile / 2];
#pragma unroll
        for (int k = 0; k < P; ++k) v[k] = tinn[k] ? vn[k] : T(0);
#pragma unroll
        for (int j = 0; j < kMmTile / 2; ++j) gv[j] = (liven && cok[j]) ? gn[j] : T(0);
        // features of the element: f_0 = 1, f_{1+k} = v_k, f_{beta(k,l)} = v_k v_l, zeros
        // past NM (a masked element has v = 0 and gy = 0)
        T f[kMmFeat / 2];
#pragma unroll
        for (int i = 0; i < kMmFeat / 2; ++i) {
            T lo = T(0), hi = T(0);  // features i and kMmFeat / 2 + i
            const int m0 = i, m1 = kMmFeat / 2 + i;
            if (m0 == 0) lo = T(1);
            else if (m0 <= P) lo = v[m0 - 1];
            else if (m0 < NM) lo = v[bp.k[m0 - 1 - P]] * v[bp.l[m0 - 1 - P]];
            if (m1 <= P) hi = v[m1 - 1];
            else if (m1 < NM) hi = v[bp.k[m1 - 1 - P]] * v[bp.l[m1 - 1 - P]];
            f[i] = half == 0 ? lo : hi;
        }
        // this wave's buffers only: a wave-level barrier orders its reads of the previous
        // slab before the writes, and the writes before the reads below
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        T* const frow = fsw + (wv * kMmSlab + se) * (FW * 4);
        T* const grow = gsw + (wv * kMmSlab + se) * (GW * 4);
#pragma unroll
        for (int m = 0; m < kMmFeat / 2; ++m) frow[mm_pos(half * (kMmFeat / 2) + m)] = f[m];
#pragma unroll
        for (int j = 0; j < kMmTile / 2; ++j) grow[half * (kMmTile / 2) + j] = gv[j];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        issue(r + 1, vn, gn, liven, tinn);   // the next slab's loads, in flight meanwhile
#pragma unroll 4
        for (int k = 0; k < kMmSlab; ++k) {
            const V4 gq = gs4[wv][k][cq];
            const V4 fa = fs4[wv][k][o0];
            const V4 fb = fs4[wv][k][o1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[i][j] = fma(gq[i], fa[j], acc[i][j]);
                    acc[i][4 + j] = fma(gq[i], fb[j], acc[i][4 + j]);
                }
            }
        }
    }
    // the waves' sums added in wave order by wave 0
    if constexpr (kMmWaves > 1) __syncthreads();
    T* red = fsw;
    if (kMmWaves > 1 && wv > 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) red[((wv - 1) * 32 + i * 8 + j) * 64 + lane] = acc[i][j];
    }
    if constexpr (kMmWaves > 1) __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int w = 1; w < kMmWaves; ++w)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[i][j] += red[((w - 1) * 32 + i * 8 + j) * 64 + lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gi = g0 + cq * 4 + i;
        if (gi >= g1) continue;
        const int c = chan_order[gi];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int m = fg * 8 + j;
            if (m < CW) part[(int64_t(q) * d.Cout + c) * CW + m] = acc[i][j];
        }
    }
}

// k_win_moments_mx: the fp32 form of k_win_moments_mm on the matrix cores.  Per slab of
// kMmSlab elements a wave stages grad_y and the window row (1, v_0 .. v_{P-1}, 0, ...) of each
// element (pitch kMxWP) in its own LDS buffers, then runs the product
//     M[c][m] += sum_e grad_y[c][e] f_m(e)
// as 16x16x4 fp32 MFMA tiles: A = grad_y (16 channels x 4 elements: lane i + 16 k holds
// channel i of element k), B = features (4 elements x 16 features: lane j + 16 k holds feature
// j of element k, formed as the product of the two window-row entries that define it, read
// from LDS), D = 16 x 16 moments (register r of lane l: channel 4 (l / 16) + r, feature
// l % 16).  A wave holds 2 x 4 tiles (32 channels x 64 features).  grad_y is fetched as
// 16-byte vectors of four consecutive elements of one channel when the plane size is a
// multiple of 4 (G4: chunks then start at multiples of 4, so a vector never spans two samples
// or two chunks) and staged [channel][element] (pitch kMxEP: the A reads of a half-wave fall
// in distinct banks); otherwise one element per lane, staged [element][channel] (pitch
// kMxGP).  The slab's global loads are issued one slab ahead; the waves' sums are added in
// wave order as in k_win_moments_mm.
constexpr int kMxGP = 48;  // [element][channel]: 32 channels + 16
constexpr int kMxEP = 34;  // [channel][element]: 32 elements + 2
constexpr int kMxWP = 12;  // 1, v_0 .. v_8, then zeros

template <int KW, bool G4>
__global__ __launch_bounds__(kMmWaves * 64) void k_win_moments_mx(
    const float* __restrict__ x, const float* __restrict__ gy, const int32_t* __restrict__ grp_ptr,
    const int32_t* __restrict__ chan_order, float* __restrict__ part, int ntile, int nq,
    WinDims d) {
    constexpr int P = Win<KW>::P, NM = 1 + P + Win<KW>::NP, CW = Win<KW>::CW;
    static_assert(P + 2 <= kMxWP && NM <= kMmFeat && kMmTile == 32 && kMmSlab == 32, "layout");
    static_assert(kMmSlab * kMxEP <= kMmSlab * kMxGP, "staging space");
    typedef float F4 __attribute__((ext_vector_type(4)));
    typedef float F2 __attribute__((ext_vector_type(2)));
    __shared__ F4 gs4[kMmWaves][kMmSlab * kMxGP / 4];
    __shared__ F4 ws4[kMmWaves][kMmSlab * kMxWP / 4];
    static_assert(sizeof(gs4) >= kMmWaves * 64 * 16 * sizeof(float), "reduction space");
    const int wv = wave_id(), lane = threadIdx.x & 63;
    float* const gsw = reinterpret_cast<float*>(&gs4[wv][0]);
    float* const wsw = reinterpret_cast<float*>(&ws4[wv][0]);
    const int q = blockIdx.y;
    const int ch = blockIdx.x / ntile, tile = blockIdx.x % ntile;
    const int g0 = grp_ptr[ch] + tile * kMmTile, g1 = std::min(grp_ptr[ch + 1], g0 + kMmTile);
    if (g0 >= g1) return;  // uniform per workgroup
    const int hw = d.Ho * d.Wo, HW = d.H * d.W;
    const int E = int(d.N) * hw;  // < 2^31 (checked by the host)
    int e0, e1;
    if constexpr (G4) {
        e0 = 4 * int(int64_t(q) * (E / 4) / nq);
        e1 = 4 * int(int64_t(q + 1) * (E / 4) / nq);
    } else {
        e0 = int(int64_t(q) * E / nq);
        e1 = int(int64_t(q + 1) * E / nq);
    }
    const int nslab = (e1 - e0 + kMmSlab - 1) / kMmSlab;
    const int rounds = (nslab + kMmWaves - 1) / kMmWaves;  // equal for every wave
    // window staging: element se = lane % 32, taps KH * half .. + KH - 1 (the window row's
    // constant entries, 1 and the zeros past P, are stored once here)
    constexpr int KH = (P + 1) / 2;
    const int se = lane % kMmSlab, half = lane / kMmSlab;
    if (half == 0) {
        wsw[se * kMxWP] = 1.f;
#pragma unroll
        for (int k = P + 1; k < kMxWP; ++k) wsw[se * kMxWP + k] = 0.f;
    }
    // grad_y staging: G4: four elements 4 quad .. + 3 of channels cg + 8 u (u < 4);
    // otherwise element se of channels 16 half .. + 15
    constexpr int NG = G4 ? 4 : kMmTile / 2;  // loads per lane
    const int quad = lane & 7, cg = lane >> 3;
    int coff[NG];
    bool cok[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const int gi = G4 ? g0 + cg + 8 * j : g0 + half * (kMmTile / 2) + j;
        cok[j] = gi < g1;
        coff[j] = chan_order[cok[j] ? gi : g0] * hw;
    }
    // MFMA roles: element row ek = lane / 16 of each group of four; feature 16 t + lane % 16
    // of tile t is w[fa[t]] * w[fb[t]] of the element's window row
    const int ek = lane / 16, li = lane % 16;
    const float* pwa[4];
    const float* pwb[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int m = 16 * t + li;
        int a = P + 1, b = P + 1;  // a zero entry: features past NM
        if (m == 0) {
            a = b = 0;
        } else if (m <= P) {
            a = 0;
            b = m;
        } else if (m < NM) {
            // pair r of the upper triangle by rows: (k, l) = (row, row + offset in the row)
            // (a lane-indexed table would be held in registers)
            int r = m - 1 - P, row = 0, len = P;
            while (r >= len) {
                r -= len;
                ++row;
                --len;
            }
            a = row + 1;
            b = row + r + 1;
        }
        pwa[t] = wsw + ek * kMxWP + a;
        pwb[t] = wsw + ek * kMxWP + b;
    }
    // A operand of step kk, channel tile mi: pga[kk * dA + mi * dM]
    const float* const pga = G4 ? gsw + li * kMxEP + ek : gsw + ek * kMxGP + li;
    constexpr int dA = G4 ? 4 : 4 * kMxGP, dM = G4 ? 16 * kMxEP : 16;
    F4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i][t] = F4{0.f, 0.f, 0.f, 0.f};
    auto issue = [&](int r, float (&vr)[KH], float (&gr)[kMmTile / 2], bool& live, bool& gl,
                     bool (&tin)[KH]) {
        const int sb = e0 + (r * kMmWaves + wv) * kMmSlab;
        {
            const int e = sb + se;
            live = r < rounds && e < e1;
            const int ec = live ? e : e0;
            const int n = ec / hw, pos = ec - n * hw;
            const int oy = pos / d.Wo, ox = pos - oy * d.Wo;
            const int by = oy * d.stride + d.oy0, bx = ox * d.stride + d.ox0;
            const float* plane = x + (int64_t(n) * d.Cin + ch) * HW;
#pragma unroll
            for (int j = 0; j < KH; ++j) {
                // tap j of half 0, tap KH + j of half 1 (P itself: the zero entry)
                const int dy = half ? (KH + j) / KW : j / KW, dx = half ? (KH + j) % KW : j % KW;
                const bool tap = !half || KH + j < P;
                const int yy = by + dy, xx = bx + dx;
                tin[j] = live && tap && unsigned(yy) < unsigned(d.H) && unsigned(xx) < unsigned(d.W);
                vr[j] = plane[tin[j] ? yy * d.W + xx : 0];
            }
            if constexpr (!G4) {
                gl = live;
                const float* gyn = gy + int64_t(n) * d.Cout * hw + pos;
#pragma unroll
                for (int j = 0; j < NG; ++j) gr[j] = gyn[coff[j]];
            }
        }
        if constexpr (G4) {
            const int e = sb + 4 * quad;
            gl = r < rounds && e < e1;  // e1 is a multiple of 4: the whole vector is live
            const int ec = gl ? e : e0;
            const int n = ec / hw, pos = ec - n * hw;
            const float* gyn = gy + int64_t(n) * d.Cout * hw + pos;
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const F4 v = *reinterpret_cast<const F4*>(gyn + coff[j]);
                gr[4 * j] = v[0];
                gr[4 * j + 1] = v[1];
                gr[4 * j + 2] = v[2];
                gr[4 * j + 3] = v[3];
            }
        }
    };
    float vn[KH] = {}, gn[kMmTile / 2] = {};
    bool liven = false, gln = false, tinn[KH] = {};
    if (rounds > 0) issue(0, vn, gn, liven, gln, tinn);  // an empty chunk reads nothing
    for (int r = 0; r < rounds; ++r) {
        float wv_[KH];
#pragma unroll
        for (int j = 0; j < KH; ++j) wv_[j] = tinn[j] ? vn[j] : 0.f;
        // a masked element or channel: grad_y 0 (its window row may hold anything finite)
        float gv[kMmTile / 2];
#pragma unroll
        for (int j = 0; j < kMmTile / 2; ++j) gv[j] = (gln && cok[G4 ? j / 4 : j]) ? gn[j] : 0.f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (G4) {
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                F2* gdst = reinterpret_cast<F2*>(gsw + (cg + 8 * j) * kMxEP + 4 * quad);
                gdst[0] = F2{gv[4 * j], gv[4 * j + 1]};
                gdst[1] = F2{gv[4 * j + 2], gv[4 * j + 3]};
            }
        } else {
            F4* gdst = reinterpret_cast<F4*>(gsw + se * kMxGP + half * (kMmTile / 2));
#pragma unroll
            for (int j = 0; j < kMmTile / 8; ++j)
                gdst[j] = F4{gv[4 * j], gv[4 * j + 1], gv[4 * j + 2], gv[4 * j + 3]};
        }
        {
            float* wdst = wsw + se * kMxWP + 1 + half * KH;
#pragma unroll
            for (int j = 0; j < KH; ++j) wdst[j] = wv_[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        issue(r + 1, vn, gn, liven, gln, tinn);   // the next slab's loads, in flight meanwhile
        // operands of step kk + 1 are read from LDS while the MFMAs of step kk run; every
        // read is a lane base plus a compile-time offset
        float a0 = pga[0], a1 = pga[dM], wa[4], wb[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            wa[t] = pwa[t][0];
            wb[t] = pwb[t][0];
        }
#pragma unroll
        for (int kk = 0; kk < kMmSlab / 4; ++kk) {
            float b[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) b[t] = wa[t] * wb[t];
            const float c0 = a0, c1 = a1;
            if (kk + 1 < kMmSlab / 4) {
                constexpr int dw = 4 * kMxWP;
                a0 = pga[(kk + 1) * dA];
                a1 = pga[(kk + 1) * dA + dM];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    wa[t] = pwa[t][(kk + 1) * dw];
                    wb[t] = pwb[t][(kk + 1) * dw];
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc[0][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(c0, b[t], acc[0][t], 0, 0, 0);
                acc[1][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(c1, b[t], acc[1][t], 0, 0, 0);
            }
        }
    }
    // the waves' sums added in wave order, one channel tile at a time: every wave stores its
    // 16 sums of the tile, then wave w adds feature tile w of all four waves and stores it
    static_assert(kMmWaves == 4, "one feature tile per wave in the closing reduction");
    float* red = reinterpret_cast<float*>(&gs4[0][0]);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(wv * 16 + t * 4 + r) * 64 + lane] = acc[i][t][r];
        __syncthreads();
        const int m = 16 * wv + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sum = red[(wv * 4 + r) * 64 + lane];
#pragma unroll
            for (int w = 1; w < kMmWaves; ++w) sum += red[(w * 16 + wv * 4 + r) * 64 + lane];
            const int gi = g0 + 16 * i + 4 * ek + r;
            if (gi < g1 && m < CW) part[(int64_t(q) * d.Cout + chan_order[gi]) * CW + m] = sum;
        }
    }
}

// One workgroup of four waves per channel: wave w sums the moments of chunks w, w + 4, ...
// (lane j: moment j, eight chunks' loads in flight at a time, additions in chunk order), the
// four partial sums are added in wave order, then slot g (lane g of the first wave) takes
// c0 S0 + c1 S_a + c2 S_b + c3 S_ab; with probs the softmax backward.
template <typename T, int KW>
__global__ __launch_bounds__(256) void k_win_finalize(const T* __restrict__ part, int nq,
                                                      const uint8_t* __restrict__ gs,
                                                      const int32_t* __restrict__ slot_win,
                                                      const T* __restrict__ probs,
                                                      T* __restrict__ grad_w, int64_t Cout,
                                                      int G) {
    constexpr int P = Win<KW>::P, CW = Win<KW>::CW;
    __shared__ T sums[4][64];
    const int64_t c = blockIdx.x;
    const int w = wave_id(), l = lane_id();
    // the slot's taps, opcode and probability loaded with the moments (wave 0 uses them)
    int rec = 0, op = 0;
    T pl = T(0);
    if (w == 0 && l < G) {
        rec = slot_win[c * G + l];
        op = gs[c * G + l];
        if (probs) pl = probs[c * G + l];
    }
    T s = 0;
    if (l < CW) {
        int q = w;
        for (; q + 7 * 4 < nq; q += 8 * 4) {
            T t[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) t[i] = part[(int64_t(q + 4 * i) * Cout + c) * CW + l];
#pragma unroll
            for (int i = 0; i < 8; ++i) s += t[i];
        }
        for (; q < nq; q += 4) s += part[(int64_t(q) * Cout + c) * CW + l];
    }
    sums[w][l] = s;
    __syncthreads();
    if (w != 0) return;
    s = ((sums[0][l] + sums[1][l]) + sums[2][l]) + sums[3][l];
    T gw = 0;
    int ia = 0, ib = 0, iab = 0;
    Coef4<T> cf = gate_coef<T>(0);
    if (l < G) {
        const int ka = rec & 0xff, kb = (rec >> 8) & 0xff;
        ia = 1 + ka;
        ib = 1 + kb;
        iab = beta_at(P, std::min(ka, kb), std::max(ka, kb));
        cf = gate_coef<T>(uint8_t(op));
    }
    const T s0 = read_lane(s, 0);
    const T sa = __shfl(s, ia, kWave), sb = __shfl(s, ib, kWave), sab = __shfl(s, iab, kWave);
    if (l < G) gw = fma(cf.c3, sab, fma(cf.c2, sb, fma(cf.c1, sa, cf.c0 * s0)));
    if (probs) {
        const T p = pl;
        const T dot = wave_total(p * gw);
        gw = p * (gw - dot);
    }
    if (l < G) grad_w[c * G + l] = gw;
}

int win_dims(WinDims& d, int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
             int64_t stride, int64_t h_out, int64_t w_out, int64_t oy0, int64_t ox0, int64_t kw) {
    CL_ARG(N >= 0 && Cin >= 1 && Cout >= 0 && H >= 1 && W >= 1, "bad shape");
    CL_ARG(h_out >= 1 && w_out >= 1 && stride >= 1, "bad output plane or stride");
    CL_ARG(kw >= 1 && kw <= 3, "window width must be 1, 2 or 3");
    CL_ARG(H * W < (int64_t(1) << 24) && h_out * w_out < (int64_t(1) << 24),
           "planes too large for the window path");
    CL_ARG(oy0 > -128 && oy0 < 128 && ox0 > -128 && ox0 < 128, "bad window origin");
    d = WinDims{N, Cin, Cout, int(H), int(W), int(h_out), int(w_out), int(stride), int(oy0),
                int(ox0)};
    return CL_OK;
}

template <typename F>
int with_kw(int64_t kw, F&& f) {
    switch (kw) {
        case 1: return f(std::integral_constant<int, 1>());
        case 2: return f(std::integral_constant<int, 2>());
        case 3: return f(std::integral_constant<int, 3>());
        default: set_error("window width must be 1, 2 or 3"); return CL_ERR_INVALID_ARGUMENT;
    }
}

// Every kw x kw window of every output position lies inside the H x W plane.
bool win_interior(int64_t H, int64_t W, int64_t stride, int64_t h_out, int64_t w_out,
                  int64_t oy0, int64_t ox0, int64_t kw) {
    return oy0 >= 0 && ox0 >= 0 && (h_out - 1) * stride + oy0 + kw <= H &&
           (w_out - 1) * stride + ox0 + kw <= W;
}

int block_for(int64_t hw, int cap) {
    int64_t b = ceil_div(hw, 64) * 64;
    return int(std::min<int64_t>(b, cap));
}

#ifndef CL_WIN_CB
#define CL_WIN_CB 2
#endif
constexpr int kWinCB = CL_WIN_CB;  // output channels per moments block

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_conv_window_coef_width(int64_t kw, int64_t* width) {
    clear_error();
    CL_ARG(width, "null pointer argument");
    const int w = coef_width(int(kw));
    CL_ARG(w > 0, "window width must be 1, 2 or 3");
    *width = w;
    return CL_OK;
}

extern "C" int cl_conv_window_prep(int dtype, const void* w, int softmax, const uint8_t* gate_seq,
                                   const int32_t* slot_win, void* probs, void* coef,
                                   int64_t Cout, int64_t num_gates, int64_t kw, void* stream) {
    clear_error();
    CL_ARG(Cout >= 0 && num_gates >= 1 && num_gates <= 64, "num_gates must be in [1, 64]");
    if (Cout == 0) return CL_OK;
    CL_ARG(w && gate_seq && slot_win && coef, "null pointer argument");
    const unsigned blocks = unsigned(ceil_div(Cout, 4));
    CL_DTYPE_SWITCH(dtype, {
        int rc = with_kw(kw, [&](auto K) {
            k_win_prep<scalar_t, decltype(K)::value><<<blocks, 256, 0, as_stream(stream)>>>(
                static_cast<const scalar_t*>(w), softmax, gate_seq, slot_win,
                static_cast<scalar_t*>(probs), static_cast<scalar_t*>(coef), Cout,
                int(num_gates));
            return CL_OK;
        });
        if (rc) return rc;
    });
    return check_launch("cl_conv_window_prep");
}

extern "C" int cl_conv_window_forward(int dtype, const void* x, const void* coef,
                                      const int32_t* grp_ptr, const int32_t* chan_order, void* y,
                                      int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                                      int64_t stride, int64_t h_out, int64_t w_out, int64_t oy0,
                                      int64_t ox0, int64_t kw, void* stream) {
    clear_error();
    WinDims d;
    if (int rc = win_dims(d, N, Cin, H, W, Cout, stride, h_out, w_out, oy0, ox0, kw)) return rc;
    if (N == 0 || Cout == 0) return CL_OK;
    CL_ARG(x && coef && grp_ptr && chan_order && y, "null pointer argument");
    const int hw = d.Ho * d.Wo;
    const int bs = block_for(hw, 256);
    // planes of at most 128 positions that would leave more than a tenth of a block idle take
    // several samples per 256-thread block
    const bool pack = hw <= 128 && (bs - hw) * 10 > bs;
    const int64_t pchunks = pack ? 256 / hw : ceil_div(hw, bs);
    // wide channel groups (many output channels per input channel on average) are split over
    // two blocks of threads: twice the waves for the same window loads per channel
    const int split = Cout >= 8 * Cin ? 2 : 1;
    const int64_t blocks = (pack ? ceil_div(N, pchunks) : N * pchunks) * Cin * split;
    CL_ARG(blocks < (int64_t(1) << 32), "conv layer too large for one launch");
    const bool interior = win_interior(H, W, stride, h_out, w_out, oy0, ox0, kw);
    CL_DTYPE_SWITCH(dtype, {
        int rc = with_kw(kw, [&](auto K) {
            auto go = [&](auto sc, auto pc) {
                constexpr int KWV = decltype(K)::value, SCV = decltype(sc)::value;
                constexpr bool PCV = decltype(pc)::value;
                auto kern = interior ? k_win_fwd<scalar_t, KWV, SCV, PCV, true>
                                     : k_win_fwd<scalar_t, KWV, SCV, PCV, false>;
                kern<<<unsigned(blocks), pack ? 256 : bs, 0, as_stream(stream)>>>(
                    static_cast<const scalar_t*>(x), static_cast<const scalar_t*>(coef), grp_ptr,
                    chan_order, static_cast<scalar_t*>(y), int(pchunks), d);
            };
            using S1 = std::integral_constant<int, 1>;
            using S2 = std::integral_constant<int, 2>;
            if (pack) {
                if (split == 2) go(S2{}, std::true_type{});
                else go(S1{}, std::true_type{});
            } else {
                if (split == 2) go(S2{}, std::false_type{});
                else go(S1{}, std::false_type{});
            }
            return CL_OK;
        });
        if (rc) return rc;
    });
    return check_launch("cl_conv_window_forward");
}

extern "C" int cl_conv_window_backward_x(int dtype, const void* x, const void* grad_y,
                                         const void* coef, const int32_t* grp_ptr,
                                         const int32_t* chan_order, void* grad_x, int64_t N,
                                         int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                                         int64_t stride, int64_t h_out, int64_t w_out,
                                         int64_t oy0, int64_t ox0, int64_t kw, void* stream) {
    clear_error();
    WinDims d;
    if (int rc = win_dims(d, N, Cin, H, W, Cout, stride, h_out, w_out, oy0, ox0, kw)) return rc;
    if (N == 0) return CL_OK;
    CL_ARG(x && grad_y && coef && grp_ptr && chan_order && grad_x, "null pointer argument");
    const int64_t hw = h_out * w_out;
    CL_ARG(hw <= 1024, "the window input gradient needs h_out * w_out <= 1024");
    const size_t tsize = dtype == CL_DTYPE_F64 ? 8 : 4;
    // the plane's LDS layout (see WinPlane): split by the stride's phases with the pitch padded
    // to Wo modulo 32 when that fits, else split unpadded, else the plain rows
    // words of the layout with the gap between phase row blocks (taken modulo 32)
    auto gap = [&](int64_t ps, int64_t pitch) {
        return ps > 1 ? ((W - ceil_div(H, ps) * pitch) % 32 + 32) % 32 : int64_t(0);
    };
    auto plane_words = [&](int64_t ps, int64_t pitch, int64_t rgap) {
        return ps * ceil_div(H, ps) * pitch + (ps - 1) * rgap;
    };
    const int64_t cap = 65536 / int64_t(tsize);
    WinPlane lp;
    int64_t ps = stride, pitch = stride * ceil_div(W, stride), rgap = 0;
    while (pitch % 32 != w_out % 32) ++pitch;
    rgap = gap(ps, pitch);
    if (plane_words(ps, pitch, rgap) > cap) pitch = stride * ceil_div(W, stride), rgap = 0;
    if (plane_words(ps, pitch, rgap) > cap) ps = 1, pitch = W;
    lp.ps = int(ps);
    lp.hs = int(ceil_div(H, ps));
    lp.ws = int(ceil_div(W, ps));
    lp.pitch = int(pitch);
    lp.rgap = int(rgap);
    lp.words = int(plane_words(ps, pitch, rgap));
    // lane bases (see WinPlane), reduced modulo 2^32
    const int64_t la = ps > 1 ? pitch - w_out : stride * (pitch - w_out);
    const int64_t lb = ps > 1 ? 1 : stride, lc = ps > 1 ? 0 : oy0 * pitch + ox0;
    lp.la = int(uint32_t(uint64_t(la)));
    lp.lb = int(uint32_t(uint64_t(lb)));
    lp.lc = int(uint32_t(uint64_t(lc)));
    for (int k = 0; k < 9; ++k) {
        if (ps == 1) {  // relative to the window's corner
            lp.tap[k] = int(k / kw * pitch + k % kw);
            continue;
        }
        // row / column of tap k relative to the position's phase origin (floor division)
        const int64_t r = oy0 + k / kw, c = ox0 + k % kw;
        const int64_t qr = r >= 0 ? r / ps : -((-r + ps - 1) / ps);
        const int64_t qc = c >= 0 ? c / ps : -((-c + ps - 1) / ps);
        lp.tap[k] = int(((r - qr * ps) * lp.hs + qr) * pitch + (r - qr * ps) * rgap +
                        (c - qc * ps) * lp.ws + qc);
    }
    lp.inv_w = 1.0f / float(W);
    lp.inv_ps = 1.0f / float(ps);
    lp.inv_wo = 1.0f / float(w_out);
    lp.div_cin = make_fastdiv(uint32_t(Cin));
    const size_t lds = size_t(ceil_div(int64_t(lp.words) * int64_t(tsize), 16) * 16);
    CL_ARG(lds <= 65536, "the window input gradient needs the input plane in 64 KiB of LDS");
    const int bs = block_for(hw, 1024);
    // a pass of bs pixels moves whole rows; with bs / W rows a multiple of ps, every thread's
    // phase stays fixed and its index moves by bs / (W ps) phase rows
    lp.st_step = bs % (W * ps) == 0 ? int(bs / (W * ps) * pitch) : 0;
    const int64_t blocks = N * Cin;
    CL_ARG(blocks < (int64_t(1) << 31), "conv layer too large for one launch");
    // every window of every output position inside the plane: no bounds tests
    const bool interior = win_interior(H, W, stride, h_out, w_out, oy0, ox0, kw);
    CL_DTYPE_SWITCH(dtype, {
        int rc = with_kw(kw, [&](auto K) {
            constexpr int KWV = decltype(K)::value;
            auto kern = interior ? k_win_bwd_x<scalar_t, KWV, true>
                                 : k_win_bwd_x<scalar_t, KWV, false>;
            kern<<<unsigned(blocks), bs, lds, as_stream(stream)>>>(
                static_cast<const scalar_t*>(x), static_cast<const scalar_t*>(grad_y),
                static_cast<const scalar_t*>(coef), grp_ptr, chan_order,
                static_cast<scalar_t*>(grad_x), d, lp);
            return CL_OK;
        });
        if (rc) return rc;
    });
    return check_launch("cl_conv_window_backward_x");
}

#ifndef CL_WIN_BLOCKS
#define CL_WIN_BLOCKS 768  // resident workgroups of the chunked moments kernel (three per CU)
#endif
#ifndef CL_WIN_MIN_ITERS
#define CL_WIN_MIN_ITERS 8
#endif

// Input channels read by at least this many output channels take the tiled moments kernel.
#ifndef CL_WIN_MX
#define CL_WIN_MX 1
#endif
#ifndef CL_WIN_MM_MIN_GROUP
#define CL_WIN_MM_MIN_GROUP 8
#endif
#ifndef CL_WIN_MM_BLOCKS
#define CL_WIN_MM_BLOCKS 1024  // resident workgroups of the fp32 tiled moments kernel (four per CU)
#endif

namespace {
bool use_mm(int64_t max_group) { return max_group >= CL_WIN_MM_MIN_GROUP; }

// element chunks of the tiled moments kernel: about CL_WIN_MM_BLOCKS workgroups, at least
// two staged slabs of elements per wave
int64_t mm_chunks(int64_t N, int64_t Cin, int64_t max_group, int64_t hw) {
    const int64_t ntile = ceil_div(max_group, kMmTile);
    // at most one round of resident workgroups: a few left over would run as a second round
    const int64_t want = std::max<int64_t>(1, CL_WIN_MM_BLOCKS / (Cin * ntile));
    const int64_t most = std::max<int64_t>(1, N * hw / (2 * kMmWaves * kMmSlab));
    return std::max<int64_t>(1, std::min(want, most));
}
}  // namespace

extern "C" int cl_conv_window_chunks(int64_t N, int64_t Cin, int64_t max_group, int64_t hw,
                                     int64_t* nq) {
    clear_error();
    CL_ARG(nq && N >= 0 && Cin >= 1 && max_group >= 0 && hw >= 1, "bad argument");
    if (use_mm(max_group)) {
        *nq = std::min<int64_t>(mm_chunks(N, Cin, max_group, hw), 65535);
        return CL_OK;
    }
    // one round of resident blocks (a few left over would run as a second round), but at
    // least 8 (sample, position) elements per thread so that the closing reduction stays
    // small against the loop
    const int64_t nsub = std::max<int64_t>(1, ceil_div(max_group, kWinCB));
    const int64_t want = std::max<int64_t>(1, CL_WIN_BLOCKS / (Cin * nsub));
    const int64_t most = N * hw / (256 * CL_WIN_MIN_ITERS);
    *nq = std::max<int64_t>(1, std::min<int64_t>(std::min(want, most), std::max<int64_t>(N, 1)));
    return CL_OK;
}

extern "C" int cl_conv_window_moments(int dtype, const void* x, const void* grad_y,
                                      const int32_t* grp_ptr, const int32_t* chan_order,
                                      void* moments, int64_t nq, int64_t max_group, int64_t N,
                                      int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                                      int64_t stride, int64_t h_out, int64_t w_out, int64_t oy0,
                                      int64_t ox0, int64_t kw, void* stream) {
    clear_error();
    WinDims d;
    if (int rc = win_dims(d, N, Cin, H, W, Cout, stride, h_out, w_out, oy0, ox0, kw)) return rc;
    if (Cout == 0) return CL_OK;
    CL_ARG(grp_ptr && chan_order && moments, "null pointer argument");
    CL_ARG(N == 0 || (x && grad_y), "null pointer argument");
    CL_ARG(nq >= 1 && nq < 65536 && max_group >= 0, "bad chunk count");
    if (use_mm(max_group)) {
        const int64_t ntile = ceil_div(max_group, kMmTile);
        const int64_t bx = Cin * ntile;
        CL_ARG(bx < (int64_t(1) << 31), "conv layer too large for one launch");
        CL_ARG(N * h_out * w_out < (int64_t(1) << 31), "too many (sample, position) elements");
        const dim3 grid(unsigned(bx), unsigned(nq), 1);
#if CL_WIN_MX
        if (dtype == CL_DTYPE_F32) {
            // 16-byte grad_y vectors: planes of a multiple of 4 elements, an aligned tensor
            const bool g4 = (h_out * w_out) % 4 == 0 && aligned(grad_y, 16);
            int rc = with_kw(kw, [&](auto K) {
                auto go = [&](auto gc) {
                    k_win_moments_mx<decltype(K)::value, decltype(gc)::value>
                        <<<grid, kMmWaves * 64, 0, as_stream(stream)>>>(
                        static_cast<const float*>(x), static_cast<const float*>(grad_y), grp_ptr,
                        chan_order, static_cast<float*>(moments), int(ntile), int(nq), d);
                };
                if (g4) go(std::true_type{});
                else go(std::false_type{});
                return CL_OK;
            });
            if (rc) return rc;
            return check_launch("cl_conv_window_moments");
        }
#endif
        CL_DTYPE_SWITCH(dtype, {
            int rc = with_kw(kw, [&](auto K) {
                k_win_moments_mm<scalar_t, decltype(K)::value>
                    <<<grid, kMmWaves * 64, 0, as_stream(stream)>>>(
                    static_cast<const scalar_t*>(x), static_cast<const scalar_t*>(grad_y),
                    grp_ptr, chan_order, static_cast<scalar_t*>(moments), int(ntile), int(nq), d);
                return CL_OK;
            });
            if (rc) return rc;
        });
        return check_launch("cl_conv_window_moments");
    }
    const int64_t nsub = std::max<int64_t>(1, ceil_div(max_group, kWinCB));
    const int64_t bx = Cin * nsub;
    CL_ARG(bx < (int64_t(1) << 31), "conv layer too large for one launch");
    const int bs = 256;
    const dim3 grid(unsigned(bx), unsigned(nq), 1);
    const bool interior = win_interior(H, W, stride, h_out, w_out, oy0, ox0, kw);
    CL_DTYPE_SWITCH(dtype, {
        int rc = with_kw(kw, [&](auto K) {
            constexpr int KWV = decltype(K)::value;
            auto kern = interior ? k_win_moments<scalar_t, KWV, kWinCB, true>
                                 : k_win_moments<scalar_t, KWV, kWinCB, false>;
            kern<<<grid, bs, 0, as_stream(stream)>>>(
                static_cast<const scalar_t*>(x), static_cast<const scalar_t*>(grad_y), grp_ptr,
                chan_order, static_cast<scalar_t*>(moments), int(nsub), int(nq), d);
            return CL_OK;
        });
        if (rc) return rc;
    });
    return check_launch("cl_conv_window_moments");
}

extern "C" int cl_conv_window_finalize(int dtype, const void* moments, int64_t nq,
                                       const uint8_t* gate_seq, const int32_t* slot_win,
                                       const void* probs, void* grad_w, int64_t Cout,
                                       int64_t num_gates, int64_t kw, void* stream) {
    clear_error();
    CL_ARG(Cout >= 0 && num_gates >= 1 && num_gates <= 64, "num_gates must be in [1, 64]");
    if (Cout == 0) return CL_OK;
    CL_ARG(moments && gate_seq && slot_win && grad_w, "null pointer argument");
    CL_ARG(nq >= 1, "bad chunk count");
    CL_ARG(Cout < (int64_t(1) << 31), "too many output channels");
    const unsigned blocks = unsigned(Cout);
    CL_DTYPE_SWITCH(dtype, {
        int rc = with_kw(kw, [&](auto K) {
            k_win_finalize<scalar_t, decltype(K)::value><<<blocks, 256, 0, as_stream(stream)>>>(
                static_cast<const scalar_t*>(moments), int(nq), gate_seq, slot_win,
                static_cast<const scalar_t*>(probs), static_cast<scalar_t*>(grad_w), Cout,
                int(num_gates));
            return CL_OK;
        });
        if (rc) return rc;
    });
    return check_launch("cl_conv_window_finalize");
}
