// Logic-tree convolution block (ConvLogic): third_party/convlogic_source_code/src/convlogic/
// convlogic_layer.py:85-360 (ConvLogicLayer, forward_python_full :236-321), treelogic_layer.py:
// 33-130 (TreeLogicLayer), cuda/full_convlogic_kernel.cu:10-701, cuda/convlogic_kernel.cu,
// cuda/treelogic_kernel.cu.
//
// Per output channel c and conv position (oy, ox), eight taps selection[c][k] =
// ch << 16 | row << 8 | col read x[n, ch, oy*sh + row - ph, ox*sw + col - pw] (0 outside the
// image).  Nodes 0..3 are relaxed gates on the tap pairs (2q, 2q + 1).  The complete block adds
// node 4 on the outputs of nodes (0, 1), node 5 on (2, 3), node 6 on (4, 5), and a 2x2 / stride 2
// max pool in which the first maximum in row-major window order wins (strict >).
//
// Every node's 16 probabilities w_prob[c][q][:] collapse to the four coefficients of
// K0 + K1 a + K2 b + K3 a b (the multilinear form of the gate mixture), so a node costs one
// evaluation whatever the mixture.  With TreeDims::softmax set, the 16 values are the node's
// logits and the probabilities are their softmax, taken where the coefficients are collapsed
// (once per workgroup and channel), and the finalize returns the gradient of the logits.
//
// Backward (all deterministic, no float atomics in global memory):
//   k_tree_nodes   per (sample, channel, pooled window): recompute the winner position's
//                  taps and nodes, propagate grad_y to the four conv gates (stored for the input
//                  gradient) and form the node moments (sum gy a b, gy a, gy b, gy); each
//                  workgroup reduces its items in a fixed order into one partial per channel;
//   k_tree_gather  per (sample, group of input channels): the input gradient accumulated in
//                  LDS.  Each lane group walks the (channel, tap) uses of one input channel in
//                  a fixed order; within one use the positions are distinct (a tap offset maps
//                  positions one to one), so every LDS word receives its additions in a fixed
//                  order and the result is bitwise reproducible;
//   k_tree_finalize  partials summed in block order, moments -> gradient of every probability
//                  (or, from logits, of every logit: the softmax backward p (g - sum p g)).
#include "common.h"

namespace cl {
namespace {

constexpr int kTaps = 8;
constexpr int kMaxNodes = 7;
constexpr int kGatherBatch = 4;  // channel uses whose loads the input-gradient gather overlaps
constexpr int kNodeItems = 16;   // most items per thread of the backward node kernel
#ifndef CL_TREE_NODE_WGS
#define CL_TREE_NODE_WGS 512      // workgroups the backward node kernel aims for
#endif

template <typename T>
__device__ __forceinline__ T quiet_nan() {
    return T(__builtin_nan(""));
}

struct TreeDims {
    int n, cin, h, w, cout, ho, wo, sh, sw, ph, pw;
    int complete;
    int softmax;  // the weights are logits: softmax over each node's 16 values on load
    int regular;  // the caller guarantees every tap lies in the window and reads a channel < cin
    int y_rows;   // complete form: y / grad_y element (n, c, p) at (c * P + p) * n_total + n
    int P;  // items per (sample, channel): pooled windows (complete) or conv positions
    int node_items;  // items per thread of the backward node kernel (set by node_blocks)
    // complete block forward: when set, the collapsed coefficients [cout][7][4] (of the
    // probabilities, or of the logits' softmax) written by the workgroups of sample 0, in the
    // order k_tree_coefs forms them, for the backward to take instead of forming them again
    void* coefs;
    FastDiv div_p, div_wp;  // by P, and by the windows per pooled row (complete) or wo
    FastDiv div_wo;         // by wo (conv positions -> rows)
};

// Pooled output / its gradient of (sample n, channel c, window p): NCHW, or with y_rows the
// feature-major [c * P + p][n] rows a following dense layer reads without a transpose.
__device__ __forceinline__ int64_t y_at(const TreeDims& d, int n, int c, int p) {
    return d.y_rows ? (int64_t(c) * d.P + p) * d.n + n : (int64_t(n) * d.cout + c) * d.P + p;
}

// Decoded tap: channel, row and column offset relative to the output position (pad removed).
struct TapOff {
    int ch, dy, dx;
};

__device__ __forceinline__ TapOff decode_tap(int32_t s, int ph, int pw) {
    TapOff t;
    t.ch = (s >> 16) & 0xFFFF;
    t.dy = ((s >> 8) & 0xFF) - ph;
    t.dx = (s & 0xFF) - pw;
    return t;
}

// Tap value at conv position (oy, ox), zero outside the image.  Branch-free: the load always
// goes to an address inside the sample (element 0 when the tap is outside) and the value is
// selected afterwards, so 32 taps do not become 32 divergent branches.
template <typename T>
__device__ __forceinline__ T tap_value(const T* __restrict__ xn, const TreeDims& d, const TapOff& t,
                                       int oy, int ox) {
    const int iy = oy * d.sh + t.dy, ix = ox * d.sw + t.dx;
    const bool ok = uint32_t(iy) < uint32_t(d.h) && uint32_t(ix) < uint32_t(d.w) &&
                    uint32_t(t.ch) < uint32_t(d.cin);
    const T v = xn[ok ? (t.ch * d.h + iy) * d.w + ix : 0];
    return ok ? v : T(0);
}

template <typename T>
__device__ __forceinline__ T node(const T* k, T a, T b) {
    return fma(k[3], a * b, fma(k[2], b, fma(k[1], a, k[0])));
}

// The 16 probabilities of a node from its weights: the weights themselves, or with `softmax`
// their softmax exp(w - max) * (1 / sum), one division per node (every workgroup of a forward
// recomputes the softmax of its channels).  The exponential is the accurate library one: the
// hardware exp2 form is off by a few 1e-7 relative, which the input gradient's cancelling sums
// turn into absolute errors above 1e-6.
template <typename T>
__device__ __forceinline__ void node_probs(const T* __restrict__ w, bool softmax, T (&p)[16]) {
#pragma unroll
    for (int g = 0; g < 16; ++g) p[g] = w[g];
    if (softmax) {
        T mx = p[0];
#pragma unroll
        for (int g = 1; g < 16; ++g) mx = fmax(mx, p[g]);
        T sum = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            p[g] = exp(p[g] - mx);
            sum += p[g];
        }
        const T inv = T(1) / sum;
#pragma unroll
        for (int g = 0; g < 16; ++g) p[g] = p[g] * inv;
    }
}

// Collapse w_prob[c][q][:] for q < nodes into sk[q][0..3]; taps of channel c into st.  Called by
// the whole workgroup, followed by a barrier.
template <typename T>
__device__ __forceinline__ void load_channel(const T* __restrict__ w_prob,
                                             const int32_t* __restrict__ sel, int c, int nodes,
                                             const TreeDims& d, T (*sk)[4], TapOff* st,
                                             int* bad) {
    const int t = threadIdx.x;
    if (t < nodes * 4) {
        const int q = t >> 2, m = t & 3;
        T p[16];
        node_probs(w_prob + (int64_t(c) * nodes + q) * 16, d.softmax != 0, p);
        T acc = 0;
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const Coef4<T> cf = gate_coef<T>(g);
            const T cm = m == 0 ? cf.c0 : m == 1 ? cf.c1 : m == 2 ? cf.c2 : cf.c3;
            acc = fma(p[g], cm, acc);
        }
        sk[q][m] = acc;
    }
    if (t >= 32 && t < 32 + kTaps) {
        const int k = t - 32;
        st[k] = decode_tap(sel[c * kTaps + k], d.ph, d.pw);
        if (st[k].ch >= d.cin) *bad = 1;
    }
}

// Node values at conv position (oy, ox): taps v, gates g (nodes 0..3), tree t (nodes 4, 5), r.
template <typename T, bool COMPLETE>
struct Eval {
    T v[kTaps], g[4], t[2], r;
};

template <typename T, bool COMPLETE>
__device__ __forceinline__ void eval_at(const T* __restrict__ xn, const TreeDims& d,
                                        const TapOff* st, T (*sk)[4], int oy, int ox,
                                        Eval<T, COMPLETE>& e) {
#pragma unroll
    for (int k = 0; k < kTaps; ++k) e.v[k] = tap_value(xn, d, st[k], oy, ox);
#pragma unroll
    for (int q = 0; q < 4; ++q) e.g[q] = node(sk[q], e.v[2 * q], e.v[2 * q + 1]);
    if constexpr (COMPLETE) {
        e.t[0] = node(sk[4], e.g[0], e.g[1]);
        e.t[1] = node(sk[5], e.g[2], e.g[3]);
        e.r = node(sk[6], e.t[0], e.t[1]);
    }
}

// One item of the conv-gates-only form with global taps: (sample, conv position) of channel c.
template <typename T>
__device__ __forceinline__ void fwd_gates_item(const T* __restrict__ x, const TreeDims& d,
                                               const TapOff* st, T (*sk)[4], bool bad, int c,
                                               int64_t item, T* __restrict__ y) {
    const int64_t total = int64_t(d.n) * d.P;
    if (item >= total) return;
    int n, p;
    if (total < (int64_t(1) << 31)) {  // uniform: 32-bit multiply-shift division
        n = int(fast_div(uint32_t(item), d.div_p));
        p = int(item) - n * d.P;
    } else {
        n = int(item / d.P);
        p = int(item % d.P);
    }
    const int oy = int(fast_div(uint32_t(p), d.div_wp));
    const T* xn = x + int64_t(n) * d.cin * d.h * d.w;
    Eval<T, false> e;
    eval_at<T, false>(xn, d, st, sk, oy, p - oy * d.wo, e);
    const int64_t pos = (int64_t(n) * d.cout + c) * d.P + p;
#pragma unroll
    for (int q = 0; q < 4; ++q) y[pos * 4 + q] = bad ? quiet_nan<T>() : e.g[q];
}

// ------------------------------------------------------------------------------------------
// Forward of the conv gates alone: one thread per (sample, conv position) of the workgroup's
// channel (blockIdx.y); y [N, C, Ho, Wo, 4].
template <typename T>
__global__ __launch_bounds__(256) void k_tree_fwd(const T* __restrict__ x, const T* __restrict__ w_prob,
                                                  const int32_t* __restrict__ sel, TreeDims d,
                                                  T* __restrict__ y) {
    __shared__ T sk[kMaxNodes][4];
    __shared__ TapOff st[kTaps];
    __shared__ int bad;
    const int c = blockIdx.y;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    load_channel(w_prob, sel, c, 4, d, sk, st, &bad);
    __syncthreads();
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;
    fwd_gates_item(x, d, st, sk, bad != 0, c, item, y);
}

constexpr int kFwdItems = 8;  // passes of 256 items per forward workgroup

// One item of the complete block with global taps: (sample, window) * 4 + q of channel c,
// the quad's four lanes together (every lane of the quad calls it).
template <typename T>
__device__ __forceinline__ void fwd_q_item(const T* __restrict__ x, const TreeDims& d,
                                           const TapOff* st, T (*sk)[4], bool bad, int c,
                                           int64_t item, int64_t total, T* __restrict__ y,
                                           T* __restrict__ x2, T* __restrict__ x3,
                                           int32_t* __restrict__ idx) {
    const int wp = d.wo / 2;
    const T nan = quiet_nan<T>();
    {
        const bool live = item < total;  // (n, window) * 4 + q
        const int64_t it = live ? item : 0;
        const int q = int(it & 3);
        const int64_t win = it >> 2;
        int n, p, py;
        if (total < (int64_t(1) << 31)) {  // uniform: 32-bit multiply-shift division
            n = int(fast_div(uint32_t(win), d.div_p));
            p = int(win) - n * d.P;
        } else {
            n = int(win / d.P);
            p = int(win % d.P);
        }
        py = int(fast_div(uint32_t(p), d.div_wp));
        const int oy = 2 * py + (q >> 1), ox = 2 * (p - py * wp) + (q & 1);
        const T* xn = x + int64_t(n) * d.cin * d.h * d.w;
        Eval<T, true> e;
        eval_at<T, true>(xn, d, st, sk, oy, ox, e);
        const int64_t cell = int64_t(n) * d.cout + c;
        if (live) {
            const int64_t pos = cell * d.ho * d.wo + int64_t(oy) * d.wo + ox;
            if (x2) {
#pragma unroll
                for (int k = 0; k < 4; ++k) x2[pos * 4 + k] = bad ? nan : e.g[k];
            }
            if (x3) {
                x3[pos * 2 + 0] = bad ? nan : e.t[0];
                x3[pos * 2 + 1] = bad ? nan : e.t[1];
            }
        }
        // first maximum over the quad: (0 vs 1), (2 vs 3), then (01 vs 23); the later lane
        // wins only when strictly greater.  A NaN never wins (it enters as -inf with winner
        // -1), so a window of NaNs keeps the reference's -inf / -1.
        const bool num = e.r == e.r;
        T r = num ? e.r : -T(__builtin_inf());
        int wi = num ? oy * d.wo + ox : -1;
        {
            const T ro = dpp_move<0xB1>(r);        // quad_perm [1,0,3,2]
            const int wo_ = dpp_move<0xB1>(wi);
            const bool take = (q & 1) ? !(r > ro) : (ro > r);  // odd lane: partner is earlier
            r = take ? ro : r;
            wi = take ? wo_ : wi;
        }
        {
            const T ro = dpp_move<0x4E>(r);        // quad_perm [2,3,0,1]
            const int wo_ = dpp_move<0x4E>(wi);
            const bool take = (q & 2) ? !(r > ro) : (ro > r);
            r = take ? ro : r;
            wi = take ? wo_ : wi;
        }
        if (live && q == 0) {
            y[y_at(d, n, c, p)] = bad ? nan : r;
            if (idx) idx[cell * d.P + p] = wi;
        }
    }
}

// Complete block, quad form: one thread per conv position, the four positions of a pooling
// window in the four lanes of a quad (lane order (0,0), (0,1), (1,0), (1,1)), so each thread
// gathers 8 taps instead of 32 and the pool is two quad-DPP steps that keep the earlier lane
// on ties (strict >, as the first-maximum rule).  Lane 0 of the quad stores y and the winner.
template <typename T>
__global__ __launch_bounds__(256) void k_tree_fwd_q(const T* __restrict__ x, const T* __restrict__ w_prob,
                                                    const int32_t* __restrict__ sel, TreeDims d,
                                                    T* __restrict__ y, T* __restrict__ x2,
                                                    T* __restrict__ x3, int32_t* __restrict__ idx) {
    __shared__ T sk[kMaxNodes][4];
    __shared__ TapOff st[kTaps];
    __shared__ int bad;
    const int c = blockIdx.y;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    load_channel(w_prob, sel, c, 7, d, sk, st, &bad);
    __syncthreads();
    if (d.coefs && blockIdx.x == 0 && threadIdx.x < kMaxNodes * 4)
        static_cast<T*>(d.coefs)[int64_t(c) * kMaxNodes * 4 + threadIdx.x] =
            sk[threadIdx.x >> 2][threadIdx.x & 3];
    const int64_t total = int64_t(d.n) * d.P * 4;
    // kFwdItems passes of 256 items per workgroup: the channel's coefficients are collapsed
    // once for all of them.
    for (int pass = 0; pass < kFwdItems; ++pass) {
        const int64_t item = (int64_t(blockIdx.x) * kFwdItems + pass) * 256 + threadIdx.x;
        if ((item & ~int64_t(255)) >= total) break;  // uniform per workgroup
        fwd_q_item(x, d, st, sk, bad != 0, c, item, total, y, x2, x3, idx);
    }
}

// ------------------------------------------------------------------------------------------
// LDS-staged forward (both forms).  A workgroup takes one sample (blockIdx.x) and a group of
// cg output channels (blockIdx.y).  It stages the sample's whole input in LDS once, zero
// padded, so a tap is one LDS read at a fixed per-lane base plus a per-channel offset: no
// bounds test, no per-tap index arithmetic beyond one add.  Staged layout of input channel ch,
// padded row iy (0 <= iy < H + 2 ph), padded column ix:
//     ch * cs + iy * rp + (ix % sw) * ws + ix / sw
// Columns are split by their phase modulo the stride, so the taps of neighbouring positions
// (ox, ox + 1) are neighbouring words; the row pitch rp is chosen on the host so that the two
// conv rows of a half-wave fall on distinct banks where it can be.  Tap k of channel c at
// conv position (oy, ox) then reads word  oy * sh * rp + ox + off[c][k]  with
//     off[c][k] = ch * cs + row * rp + (col % sw) * ws + col / sw.
// A channel whose taps leave the kernel window (row >= kh or col >= kw; the selection sampler
// never draws one) or read an input channel >= C is skipped here; k_tree_fwd_fix, launched
// after this kernel, computes it with the global-memory gather and its bounds tests (NaN for
// an out-of-range channel, as in the other forms).
//
// Lanes: IP items per channel (four per pooling window in the complete form, one per conv
// position otherwise).  When IP >= 64 a wave walks one channel's items 64 at a time; when
// IP < 64 a wave holds 64 / IP channels side by side.  The quad layout and the first-maximum
// pool are those of k_tree_fwd_q.
struct TreeLds {
    int rp, ws, cs;      // row pitch, phase block width, channel stride (elements)
    int cg;              // output channels per workgroup
    int kh, kw;          // kernel window
    int ip;              // items per channel
    FastDiv div_pos;     // items -> conv rows: windows per pooled row (complete) or wo
    FastDiv div_hw, div_w, div_sw;  // staging: element -> (channel, row, column), phase
    int idx32;           // n * cout * P < 2^31: output and winner indices in 32 bits
};

constexpr int kTapFlagIrregular = 1;
constexpr int kTapFlagBad = 2;

// LDS of a staged workgroup: the sample's planes, then per channel of the group its NK
// collapsed coefficients, its 8 tap offsets (bytes) and its flag.
template <typename T, int NK>
struct StagedLds {
    T* plane;
    T* coef;
    int* toff;
    int* tflag;
};

template <typename T, int NK>
__device__ __forceinline__ StagedLds<T, NK> staged_lds(unsigned char* raw, const TreeDims& d,
                                                       const TreeLds& g) {
    StagedLds<T, NK> L;
    L.plane = reinterpret_cast<T*>(raw);
    L.coef = L.plane + d.cin * g.cs;                             // [cg][NK]
    L.toff = reinterpret_cast<int*>(L.coef + g.cg * NK);         // [cg][8]
    L.tflag = L.toff + g.cg * kTaps;                             // [cg]
    return L;
}

// Prologue of the staged kernels (whole workgroup, ends with a barrier): the channel group's
// collapsed coefficients (the order of load_channel), tap offsets and flags, and sample n's
// zero-padded input.
template <typename T, int NODES>
__device__ __forceinline__ void stage_sample(const T* __restrict__ x, const T* __restrict__ w_prob,
                                             const int32_t* __restrict__ sel, const TreeDims& d,
                                             const TreeLds& g, int n, int c_lo, int c_n,
                                             const StagedLds<T, NODES * 4>& L) {
    const int planes = d.cin * g.cs;
    const int tid = threadIdx.x, nt = blockDim.x;
    for (int i = tid; i < planes; i += nt) L.plane[i] = T(0);
    // One thread per (channel, node): the four coefficients in the order of load_channel.
    for (int i = tid; i < c_n * NODES; i += nt) {
        T p[16];
        node_probs(w_prob + (int64_t(c_lo) * NODES + i) * 16, d.softmax != 0, p);
        T a0 = 0, a1 = 0, a2 = 0, a3 = 0;
#pragma unroll
        for (int gi = 0; gi < 16; ++gi) {
            const Coef4<T> cf = gate_coef<T>(gi);
            const T pg = p[gi];
            a0 = fma(pg, cf.c0, a0);
            a1 = fma(pg, cf.c1, a1);
            a2 = fma(pg, cf.c2, a2);
            a3 = fma(pg, cf.c3, a3);
        }
        L.coef[i * 4 + 0] = a0;
        L.coef[i * 4 + 1] = a1;
        L.coef[i * 4 + 2] = a2;
        L.coef[i * 4 + 3] = a3;
    }
    __syncthreads();
    for (int cc = tid; cc < c_n; cc += nt) {
        int flag = 0;
        for (int k = 0; k < kTaps; ++k) {
            const int32_t s = sel[int64_t(c_lo + cc) * kTaps + k];
            const int ch = (s >> 16) & 0xFFFF, row = (s >> 8) & 0xFF, col = s & 0xFF;
            if (ch >= d.cin) flag |= kTapFlagBad;
            if (row >= g.kh || col >= g.kw) flag |= kTapFlagIrregular;
            const uint32_t cq = fast_div(uint32_t(col), g.div_sw);
            L.toff[cc * kTaps + k] =  // bytes
                (ch * g.cs + row * g.rp + (col - int(cq) * d.sw) * g.ws + int(cq)) *
                int(sizeof(T));
        }
        L.tflag[cc] = flag;
        if (flag) {  // skipped by the staged kernels (a fix-up kernel takes it)
#pragma unroll
            for (int k = 0; k < kTaps; ++k) L.toff[cc * kTaps + k] = 0;  // in-bounds reads
        }
    }
    {
        const T* xn = x + int64_t(n) * d.cin * d.h * d.w;
        const int e_n = d.cin * d.h * d.w;
        for (int e = tid; e < e_n; e += nt) {
            const int ch = int(fast_div(uint32_t(e), g.div_hw));
            const int rem = e - ch * d.h * d.w;
            const int iy = int(fast_div(uint32_t(rem), g.div_w));
            const int ix = rem - iy * d.w + d.pw;
            const int xq = int(fast_div(uint32_t(ix), g.div_sw));
            L.plane[ch * g.cs + (iy + d.ph) * g.rp + (ix - xq * d.sw) * g.ws + xq] = xn[e];
        }
    }
    __syncthreads();
}

template <typename T, bool COMPLETE, bool INTER>
__device__ __forceinline__ void tree_fwd_lds(const T* __restrict__ x, const T* __restrict__ w_prob,
                                             const int32_t* __restrict__ sel, const TreeDims& d,
                                             const TreeLds& g, T* __restrict__ y,
                                             T* __restrict__ x2, T* __restrict__ x3,
                                             int32_t* __restrict__ idx) {
    constexpr int NODES = COMPLETE ? 7 : 4;
    constexpr int NK = NODES * 4;
    extern __shared__ __align__(16) unsigned char tree_lds[];
    const int n = blockIdx.x;
    const int c_lo = blockIdx.y * g.cg;
    const int c_n = min(g.cg, d.cout - c_lo);
    const StagedLds<T, NK> L = staged_lds<T, NK>(tree_lds, d, g);
    T* plane = L.plane;
    const T* coef = L.coef;
    const int* toff = L.toff;
    const int* tflag = L.tflag;
    const int tid = threadIdx.x, nt = blockDim.x;
    stage_sample<T, NODES>(x, w_prob, sel, d, g, n, c_lo, c_n, L);
    if (COMPLETE && d.coefs && n == 0) {
        T* kco = static_cast<T*>(d.coefs) + int64_t(c_lo) * NK;
        for (int i = threadIdx.x; i < c_n * NK; i += blockDim.x) kco[i] = coef[i];
    }

    const int lane = tid & 63, wave = tid >> 6, nw = nt >> 6;
    const int cpw = g.ip >= 64 ? 1 : 64 / g.ip;
    const int sub = g.ip >= 64 ? 0 : lane / g.ip;
    const int r0 = lane - sub * (g.ip >= 64 ? 0 : g.ip);
    const int row_step = d.sh * g.rp;
    const int wp = COMPLETE ? d.wo / 2 : d.wo;
    // Items are (window, q) with q = item & 3, and every chunk of a wave starts at a multiple
    // of 4 items, so a lane's q is fixed: lane & 3.
    const int q_lane = COMPLETE ? (lane & 3) : 0;
    {
        for (int it = wave * cpw; it < c_n; it += nw * cpw) {
            const int cc = it + sub;
            const int cl_ = (sub < cpw && cc < c_n) ? cc : it;
            const int flag = tflag[cl_];
            // flagged: k_tree_fwd_fix, or, when the caller guaranteed regular taps (no fix-up
            // launch), NaN outputs that make the broken guarantee visible
            const bool cok = sub < cpw && cc < c_n && (flag == 0 || d.regular != 0);
            const bool poison = flag != 0;
            T k[NODES][4];
#pragma unroll
            for (int q = 0; q < NODES; ++q)
#pragma unroll
                for (int m = 0; m < 4; ++m) k[q][m] = coef[cl_ * NK + q * 4 + m];
            int off[kTaps];
#pragma unroll
            for (int t = 0; t < kTaps; ++t) off[t] = toff[cl_ * kTaps + t];
            const int c = c_lo + cl_;
            const int64_t cell = int64_t(n) * d.cout + c;
            // 32-bit output / winner index of window p: base + p * step (when g.idx32)
            const uint32_t ybase = d.y_rows ? uint32_t(c) * uint32_t(d.P) * uint32_t(d.n) + n
                                            : uint32_t(cell) * uint32_t(d.P);
            const uint32_t ystep = d.y_rows ? uint32_t(d.n) : 1u;
            const uint32_t ibase = uint32_t(cell) * uint32_t(d.P);
            for (int j = 0; j < g.ip; j += 64) {
                const int r = j + r0;
                const bool live = cok && r < g.ip;
                const int re = live ? r : q_lane;  // a dead lane keeps its quad position
                int oy, ox, p;
                if constexpr (COMPLETE) {
                    p = re >> 2;
                    const int py = int(fast_div(uint32_t(p), g.div_pos));
                    const int px = p - py * wp;
                    oy = 2 * py + (q_lane >> 1);
                    ox = 2 * px + (q_lane & 1);
                } else {
                    p = re;
                    oy = int(fast_div(uint32_t(p), g.div_pos));
                    ox = p - oy * wp;
                }
                // Every lane reads in bounds: a dead lane sits at a valid position of a channel
                // whose offsets are valid (or 0 for a flagged one), and drops what it reads.
                T v[kTaps];
                {
                    const int base = (oy * row_step + ox) * int(sizeof(T));
                    const char* pl = reinterpret_cast<const char*>(plane) + base;
#pragma unroll
                    for (int t = 0; t < kTaps; ++t) v[t] = *reinterpret_cast<const T*>(pl + off[t]);
                }
                T gv[4];
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) gv[qq] = node(k[qq], v[2 * qq], v[2 * qq + 1]);
                if constexpr (!COMPLETE) {
                    if (live) {
                        const int64_t pos = cell * d.P + p;
#pragma unroll
                        for (int qq = 0; qq < 4; ++qq) y[pos * 4 + qq] = poison ? quiet_nan<T>() : gv[qq];
                    }
                } else {
                    const T t0 = node(k[4], gv[0], gv[1]);
                    const T t1 = node(k[5], gv[2], gv[3]);
                    const T rv = node(k[6], t0, t1);
                    if (INTER && live) {
                        const int64_t pos = cell * d.ho * d.wo + int64_t(oy) * d.wo + ox;
                        if (x2) {
#pragma unroll
                            for (int qq = 0; qq < 4; ++qq)
                                x2[pos * 4 + qq] = poison ? quiet_nan<T>() : gv[qq];
                        }
                        if (x3) {
                            x3[pos * 2 + 0] = poison ? quiet_nan<T>() : t0;
                            x3[pos * 2 + 1] = poison ? quiet_nan<T>() : t1;
                        }
                    }
                    // No NaN enters the quad (one enters as -inf), so for the later lane of a
                    // pair "not strictly greater than the earlier one" is ro >= rr.
                    const bool num = rv == rv;
                    T rr = num ? rv : -T(__builtin_inf());
                    int wi = num ? oy * d.wo + ox : -1;
                    // The comparisons are wave masks; the lane parity picks between them in
                    // scalar code (lanes with q & 1: 0xAAAA...; with q & 2: 0xCCCC...).
                    {
                        const T ro = dpp_move<0xB1>(rr);
                        const int wo_ = dpp_move<0xB1>(wi);
                        const uint64_t gt = __ballot(ro > rr), ge = __ballot(ro >= rr);
                        const bool take = __builtin_amdgcn_inverse_ballot_w64(
                            (ge & 0xAAAAAAAAAAAAAAAAull) | (gt & 0x5555555555555555ull));
                        rr = take ? ro : rr;
                        wi = take ? wo_ : wi;
                    }
                    {
                        const T ro = dpp_move<0x4E>(rr);
                        const int wo_ = dpp_move<0x4E>(wi);
                        const uint64_t gt = __ballot(ro > rr), ge = __ballot(ro >= rr);
                        const bool take = __builtin_amdgcn_inverse_ballot_w64(
                            (ge & 0xCCCCCCCCCCCCCCCCull) | (gt & 0x3333333333333333ull));
                        rr = take ? ro : rr;
                        wi = take ? wo_ : wi;
                    }
                    if (live && q_lane == 0) {
                        if (g.idx32) {
                            y[ybase + uint32_t(p) * ystep] = poison ? quiet_nan<T>() : rr;
                            if (idx) idx[ibase + uint32_t(p)] = poison ? -1 : wi;
                        } else {
                            y[y_at(d, n, c, p)] = poison ? quiet_nan<T>() : rr;
                            if (idx) idx[cell * d.P + p] = poison ? -1 : wi;
                        }
                    }
                }
            }
        }
    }
}

// fp32 without the intermediates fits 64 VGPRs: two workgroups of 16 waves per CU.
template <bool COMPLETE>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8))) void k_tree_fwd_lds_f32(
    const float* __restrict__ x, const float* __restrict__ w_prob, const int32_t* __restrict__ sel,
    TreeDims d, TreeLds g, float* __restrict__ y, float* __restrict__ x2, float* __restrict__ x3,
    int32_t* __restrict__ idx) {
    tree_fwd_lds<float, COMPLETE, false>(x, w_prob, sel, d, g, y, x2, x3, idx);
}

template <typename T, bool COMPLETE, bool INTER>
__global__ __launch_bounds__(1024) void k_tree_fwd_lds(
    const T* __restrict__ x, const T* __restrict__ w_prob, const int32_t* __restrict__ sel,
    TreeDims d, TreeLds g, T* __restrict__ y, T* __restrict__ x2, T* __restrict__ x3,
    int32_t* __restrict__ idx) {
    tree_fwd_lds<T, COMPLETE, INTER>(x, w_prob, sel, d, g, y, x2, x3, idx);
}

// The channels k_tree_fwd_lds skips.  Each workgroup checks 256 channels, one per thread, and
// returns when all of them are regular (the usual case: one short launch of a few
// workgroups); each flagged one is then computed by the whole workgroup with the global
// gather over every sample.
constexpr int kFixChannels = 256;

template <typename T, bool COMPLETE>
__global__ __launch_bounds__(256) void k_tree_fwd_fix(const T* __restrict__ x,
                                                      const T* __restrict__ w_prob,
                                                      const int32_t* __restrict__ sel, TreeDims d,
                                                      int kh, int kw, T* __restrict__ y,
                                                      T* __restrict__ x2, T* __restrict__ x3,
                                                      int32_t* __restrict__ idx) {
    __shared__ int flagged[kFixChannels];
    __shared__ int nflagged;
    __shared__ T sk[kMaxNodes][4];
    __shared__ TapOff st[kTaps];
    __shared__ int bad;
    if (threadIdx.x == 0) nflagged = 0;
    __syncthreads();
    {
        const int c = blockIdx.x * kFixChannels + threadIdx.x;
        bool f = false;
        if (c < d.cout) {
#pragma unroll
            for (int k = 0; k < kTaps; ++k) {
                const int32_t s = sel[int64_t(c) * kTaps + k];
                f |= ((s >> 16) & 0xFFFF) >= d.cin || ((s >> 8) & 0xFF) >= kh ||
                     (s & 0xFF) >= kw;
            }
        }
        if (f) flagged[atomicAdd(&nflagged, 1)] = c;  // LDS atomic
    }
    __syncthreads();
    const int nf = nflagged;
    for (int i = 0; i < nf; ++i) {  // uniform
        const int c = flagged[i];
        if (threadIdx.x == 0) bad = 0;
        __syncthreads();
        load_channel(w_prob, sel, c, COMPLETE ? 7 : 4, d, sk, st, &bad);
        __syncthreads();
        if constexpr (COMPLETE) {
            const int64_t total = int64_t(d.n) * d.P * 4;
            for (int64_t item = threadIdx.x; (item & ~int64_t(255)) < total; item += 256)
                fwd_q_item(x, d, st, sk, bad != 0, c, item, total, y, x2, x3, idx);
        } else {
            const int64_t total = int64_t(d.n) * d.P;
            for (int64_t item = threadIdx.x; item < total; item += 256)
                fwd_gates_item(x, d, st, sk, bad != 0, c, item, y);
        }
        __syncthreads();  // sk / st are rewritten for the next channel
    }
}

// Backward through nodes 6, 4 and 5 of the complete block at one position: the upstream
// gradients gc of the four conv gates, and the moments of nodes 4, 5 and 6.
template <typename T, typename K>
__device__ __forceinline__ void node_grads(const K& k, const T* g, const T* t, T gy, T* gc,
                                           T* mom) {
    const T gt0 = gy * fma(k[6][3], t[1], k[6][1]);
    const T gt1 = gy * fma(k[6][3], t[0], k[6][2]);
    gc[0] = gt0 * fma(k[4][3], g[1], k[4][1]);
    gc[1] = gt0 * fma(k[4][3], g[0], k[4][2]);
    gc[2] = gt1 * fma(k[5][3], g[3], k[5][1]);
    gc[3] = gt1 * fma(k[5][3], g[2], k[5][2]);
    const T gts[2] = {gt0, gt1};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const T a = g[2 * j], b = g[2 * j + 1], gg = gts[j];
        mom[(4 + j) * 4 + 0] += gg * a * b;
        mom[(4 + j) * 4 + 1] += gg * a;
        mom[(4 + j) * 4 + 2] += gg * b;
        mom[(4 + j) * 4 + 3] += gg;
    }
    mom[24] += gy * t[0] * t[1];
    mom[25] += gy * t[0];
    mom[26] += gy * t[1];
    mom[27] += gy;
}

// Moments of the four conv gates (nodes 0..3) at one position: taps v, upstream gradients gc.
template <typename T>
__device__ __forceinline__ void gate_moments(const T* v, const T* gc, T* mom) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const T a = v[2 * q], b = v[2 * q + 1], g = gc[q];
        mom[q * 4 + 0] += g * a * b;
        mom[q * 4 + 1] += g * a;
        mom[q * 4 + 2] += g * b;
        mom[q * 4 + 3] += g;
    }
}

// One item of the backward node pass with global taps: (sample, window) of channel c for the
// complete block (recomputed at the window's winner), (sample, position) otherwise; adds its
// node moments to mom[node * 4 + (gab, ga, gb, g)] and stores the four conv-gate gradients
// when gconv is given (complete block).
template <typename T, bool COMPLETE, bool REC>
__device__ __forceinline__ void nodes_item(const T* __restrict__ grad_y, const T* __restrict__ x,
                                           const int32_t* __restrict__ idx, const TreeDims& d,
                                           const TapOff* st, T (*sk)[4], int c, int64_t item,
                                           int64_t total, T* __restrict__ radd,
                                           int32_t* __restrict__ rtgt, T* mom) {
    int n, p;
    if (total < (int64_t(1) << 31)) {  // uniform: 32-bit multiply-shift division
        n = int(fast_div(uint32_t(item), d.div_p));
        p = int(item) - n * d.P;
    } else {
        n = int(item / d.P);
        p = int(item % d.P);
    }
    const T* xn = x + int64_t(n) * d.cin * d.h * d.w;
    const int64_t cell = int64_t(n) * d.cout + c;
    T gc[4];
    Eval<T, COMPLETE> e;
    if constexpr (COMPLETE) {
        const int win = idx[cell * d.P + p];
        const bool live = win >= 0 && win < d.ho * d.wo;
        const int w0 = live ? win : 0;
        const int wy = int(fast_div(uint32_t(w0), d.div_wo));
        eval_at<T, true>(xn, d, st, sk, wy, w0 - wy * d.wo, e);
        const T gy = live ? grad_y[y_at(d, n, c, p)] : T(0);
        node_grads<T>(sk, e.g, e.t, gy, gc, mom);
        if constexpr (REC) {  // the input gradient's contribution of every tap: use (c, k), item
            const int wx = w0 - wy * d.wo;
#pragma unroll
            for (int k = 0; k < kTaps; ++k) {
                const int q = k >> 1;
                const int iy = wy * d.sh + st[k].dy, ix = wx * d.sw + st[k].dx;
                const bool ok = live && uint32_t(iy) < uint32_t(d.h) &&
                                uint32_t(ix) < uint32_t(d.w) && uint32_t(st[k].ch) < uint32_t(d.cin);
                const int64_t at = (int64_t(c) * kTaps + k) * total + item;
                radd[at] = gc[q] * fma(sk[q][3], e.v[k ^ 1], (k & 1) ? sk[q][2] : sk[q][1]);
                rtgt[at] = ok ? iy * d.w + ix : -1;
            }
        }
    } else {
        const int oy = int(fast_div(uint32_t(p), d.div_wo));
        eval_at<T, false>(xn, d, st, sk, oy, p - oy * d.wo, e);
#pragma unroll
        for (int q = 0; q < 4; ++q) gc[q] = grad_y[(cell * d.P + p) * 4 + q];
    }
    gate_moments<T>(e.v, gc, mom);
}

// ------------------------------------------------------------------------------------------
// Backward, node part: per item the upstream gradients of the four conv gates (complete; the
// conv-only block reads them from grad_y) and the node moments, reduced over the workgroup's
// items into part[(c * nblk + blk) * NODES * 4 + q * 4 + m] with
// m = (sum gy a b, sum gy a, sum gy b, sum gy).  With REC (complete, input gradient wanted)
// it also stores, per tap k of the channel and item, the tap's input-gradient contribution
//     radd = gconv[q] * (k even ? K1 + K3 x_partner : K2 + K3 x_partner),  q = k / 2,
// and the input-plane position it adds to (rtgt, -1 for none), both at (c * 8 + k) * items +
// item, for k_tree_gather_rec.  The blk == 0 workgroup of each channel also stores the
// collapsed coefficients kc[c][q][:] for the conv-only gather.
template <typename T, bool COMPLETE, bool REC>
__global__ __launch_bounds__(256) void k_tree_nodes(const T* __restrict__ grad_y, const T* __restrict__ x,
                                                    const T* __restrict__ w_prob,
                                                    const int32_t* __restrict__ sel,
                                                    const int32_t* __restrict__ idx, TreeDims d,
                                                    T* __restrict__ radd, int32_t* __restrict__ rtgt,
                                                    T* __restrict__ part, T* __restrict__ kc) {
    constexpr int NODES = COMPLETE ? 7 : 4;
    constexpr int NM = NODES * 4;
    __shared__ T sk[kMaxNodes][4];
    __shared__ TapOff st[kTaps];
    __shared__ int bad;
    __shared__ T red[4][NM];
    const int c = blockIdx.y;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    load_channel(w_prob, sel, c, NODES, d, sk, st, &bad);
    __syncthreads();
    if (blockIdx.x == 0 && threadIdx.x < NM) kc[int64_t(c) * NM + threadIdx.x] = sk[threadIdx.x >> 2][threadIdx.x & 3];
    T mom[NM];
#pragma unroll
    for (int i = 0; i < NM; ++i) mom[i] = T(0);
    // d.node_items items per thread (strided by the workgroup size), so the moments of that
    // many items are summed in registers before the wave reductions
    const int64_t total = int64_t(d.n) * d.P;
    for (int it = 0; it < d.node_items; ++it) {
        const int64_t item = (int64_t(blockIdx.x) * d.node_items + it) * 256 + threadIdx.x;
        if (item >= total) break;
        nodes_item<T, COMPLETE, REC>(grad_y, x, idx, d, st, sk, c, item, total, radd, rtgt, mom);
    }
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < NM; ++i) {
        const T s = wave_total(mom[i]);
        if (lane == 0) red[wv][i] = s;
    }
    __syncthreads();
    if (threadIdx.x < NM) {
        const int i = threadIdx.x;
        const T s = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
        part[(int64_t(c) * gridDim.x + blockIdx.x) * NM + i] = bad ? quiet_nan<T>() : s;
    }
}

// ------------------------------------------------------------------------------------------
// Backward, input gradient.  Workgroup (spw samples, channel group); LDS holds the gradient of
// CG input channels of each sample.  A lane group of PW * spw lanes (PW = items per pass, a power
// of two <= 64; spw samples, each with PW lanes) owns one input channel at a time and walks its
// uses ent[ent_ptr[ch] ..) = c * 8 + k in order, so one use's taps and coefficients serve all
// spw samples; lane pl of a sample handles items pl, pl + PW, ...  Each (sample, channel) plane
// is added to by its own lanes only, in use order.  For use (c, k) at item p (conv position win, the pooled
// window's winner when complete) the tap reads (iy, ix) = (oy*sh + dy_k, ox*sw + dx_k) and adds
//   gconv[n, c, p, k/2] * (k even ? K1 + K3 x_partner : K2 + K3 x_partner)
// of node k/2, x_partner being the other tap of the node at the same position.
template <typename T, bool COMPLETE>
__global__ __launch_bounds__(256) void k_tree_gather(const T* __restrict__ gsrc, const T* __restrict__ x,
                                                     const int32_t* __restrict__ sel,
                                                     const int32_t* __restrict__ idx,
                                                     const int32_t* __restrict__ ent_ptr,
                                                     const int32_t* __restrict__ ent,
                                                     const T* __restrict__ kc, TreeDims d, int cg,
                                                     int pw_lanes, int spw, int band_rows,
                                                     T* __restrict__ grad_x) {
    constexpr int NODES = COMPLETE ? 7 : 4;
    extern __shared__ unsigned char smem_raw[];
    T* gx = reinterpret_cast<T*>(smem_raw);  // [spw][cg][band rows * w]
    const int n0 = blockIdx.x * spw;
    const int ch0 = blockIdx.y * cg;
    const int nch = min(cg, d.cin - ch0);
    // the workgroup's band of input rows [y0, y1) (the whole plane when it fits LDS); every
    // use is walked by every band and adds only to its own rows, in the same order
    const int y0 = blockIdx.z * band_rows, y1 = min(d.h, y0 + band_rows);
    const int hw = (y1 - y0) * d.w;
    for (int i = threadIdx.x; i < spw * nch * hw; i += 256) gx[i] = T(0);
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int PW = pw_lanes;
    // a lane group of PW * spw lanes: spw samples, PW items of each
    const int GL = PW * spw;
    const int groups_per_wave = 64 / GL;
    const int sub = lane / GL, gl = lane % GL, sl = gl / PW, pl = gl % PW;
    const int n = n0 + sl;
    const bool n_ok = n < d.n;
    const T* xn = x + int64_t(n_ok ? n : 0) * d.cin * d.h * d.w;  // the whole sample
    T* gxs = gx + sl * nch * hw;
    // channel slot handled by this lane group in pass `it`: wave-major so a wave's groups take
    // consecutive channels
    for (int base = 0; base < nch; base += 4 * groups_per_wave) {
        const int chl = base + wv * groups_per_wave + sub;
        const bool have = chl < nch;
        const int ch = ch0 + chl;
        const int e0 = have ? ent_ptr[ch] : 0, e1 = have ? ent_ptr[ch + 1] : 0;
        // trip count uniform over the wave: the largest use count of its groups
        int cnt = e1 - e0;
        for (int off = 32; off > 0; off >>= 1) cnt = max(cnt, __shfl_xor(cnt, off, 64));
        // uses in batches of kGatherBatch: the records, coefficients and gradients of a batch
        // are loaded together, then its additions are applied in use order
        for (int j = 0; j < cnt; j += kGatherBatch) {
            bool on[kGatherBatch];
            TapOff tk[kGatherBatch], tp[kGatherBatch];
            T kown[kGatherBatch], k3[kGatherBatch];
            int64_t cell[kGatherBatch];
            int kn[kGatherBatch];
#pragma unroll
            for (int i = 0; i < kGatherBatch; ++i) {
                on[i] = n_ok && j + i < e1 - e0;
                const int u = j + i < e1 - e0 ? ent[e0 + j + i] : 0;
                const int c = u >> 3, k = u & 7;
                tk[i] = decode_tap(sel[c * kTaps + k], d.ph, d.pw);
                tp[i] = decode_tap(sel[c * kTaps + (k ^ 1)], d.ph, d.pw);
                const T* kq = kc + (int64_t(c) * NODES + (k >> 1)) * 4;
                kown[i] = (k & 1) ? kq[2] : kq[1];
                k3[i] = kq[3];
                cell[i] = int64_t(n) * d.cout + c;
                kn[i] = k >> 1;
            }
            for (int p = pl; p < d.P; p += PW) {
                int tgt[kGatherBatch];
                T add[kGatherBatch];
#pragma unroll
                for (int i = 0; i < kGatherBatch; ++i) {
                    int win = p;
                    if constexpr (COMPLETE) win = on[i] ? idx[cell[i] * d.P + p] : -1;
                    const bool wok = on[i] && win >= 0 && win < d.ho * d.wo;
                    const int w0 = wok ? win : 0;
                    const int oy = int(fast_div(uint32_t(w0), d.div_wo)), ox = w0 - oy * d.wo;
                    const int iy = oy * d.sh + tk[i].dy, ix = ox * d.sw + tk[i].dx;
                    const bool ok = wok && iy >= y0 && iy < y1 && ix >= 0 && ix < d.w;
                    tgt[i] = ok ? (iy - y0) * d.w + ix : -1;
                    const T xp = ok ? tap_value(xn, d, tp[i], oy, ox) : T(0);
                    const T g = ok ? gsrc[(cell[i] * d.P + p) * 4 + kn[i]] : T(0);
                    add[i] = g * fma(k3[i], xp, kown[i]);
                }
#pragma unroll
                for (int i = 0; i < kGatherBatch; ++i)
                    if (tgt[i] >= 0) atomicAdd(&gxs[(ch - ch0) * hw + tgt[i]], add[i]);
            }
        }
    }
    __syncthreads();
    const int64_t plane = int64_t(d.h) * d.w;
    for (int i = threadIdx.x; i < spw * nch * hw; i += 256) {
        const int si = i / (nch * hw), r = i % (nch * hw);
        const int chl = r / hw, rr = r - chl * hw;
        if (n0 + si < d.n)
            grad_x[(int64_t(n0 + si) * d.cin + ch0 + chl) * plane + int64_t(y0) * d.w + rr] = gx[i];
    }
}

// Backward, input gradient of the complete block from the node pass's contributions: the
// workgroup and lane-group layout of k_tree_gather, but a use (c, k) at item (n, p) needs only
// its contribution and target (radd / rtgt at (c * 8 + k) * items + n * P + p), loaded for a
// batch of kRecBatch uses at once; the additions are applied in use order, as there.
#ifndef CL_TREE_REC_BATCH
#define CL_TREE_REC_BATCH 8
#endif
constexpr int kRecBatch = CL_TREE_REC_BATCH;

template <typename T>
__global__ __launch_bounds__(256) void k_tree_gather_rec(const T* __restrict__ radd,
                                                         const int32_t* __restrict__ rtgt,
                                                         const int32_t* __restrict__ ent_ptr,
                                                         const int32_t* __restrict__ ent,
                                                         TreeDims d, int cg, int pw_lanes,
                                                         int spw, int band_rows,
                                                         T* __restrict__ grad_x) {
    extern __shared__ unsigned char smem_raw[];
    T* gx = reinterpret_cast<T*>(smem_raw);  // [spw][cg][band rows * w]
    const int n0 = blockIdx.x * spw;
    const int ch0 = blockIdx.y * cg;
    const int nch = min(cg, d.cin - ch0);
    const int y0 = blockIdx.z * band_rows, y1 = min(d.h, y0 + band_rows);
    const int hw = (y1 - y0) * d.w, base_pos = y0 * d.w;
    for (int i = threadIdx.x; i < spw * nch * hw; i += 256) gx[i] = T(0);
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int PW = pw_lanes;
    const int GL = PW * spw;
    const int groups_per_wave = 64 / GL;
    const int sub = lane / GL, gl = lane % GL, sl = gl / PW, pl = gl % PW;
    const int n = n0 + sl;
    const bool n_ok = n < d.n;
    // record indices fit 32 bits (checked by the host)
    const uint32_t total = uint32_t(d.n) * uint32_t(d.P);
    const uint32_t nrow = uint32_t(n_ok ? n : 0) * uint32_t(d.P);
    T* gxs = gx + sl * nch * hw;
    for (int base = 0; base < nch; base += 4 * groups_per_wave) {
        const int chl = base + wv * groups_per_wave + sub;
        const bool have = chl < nch;
        const int ch = ch0 + chl;
        const int e0 = have ? ent_ptr[ch] : 0, e1 = have ? ent_ptr[ch + 1] : 0;
        int cnt = e1 - e0;
        for (int off = 32; off > 0; off >>= 1) cnt = max(cnt, __shfl_xor(cnt, off, 64));
        for (int j = 0; j < cnt; j += kRecBatch) {
            bool on[kRecBatch];
            uint32_t urow[kRecBatch];
#pragma unroll
            for (int i = 0; i < kRecBatch; ++i) {
                on[i] = n_ok && j + i < e1 - e0;
                urow[i] = uint32_t(on[i] ? ent[e0 + j + i] : 0) * total + nrow;
            }
            for (int p = pl; p < d.P; p += PW) {
                int32_t tg[kRecBatch];
                T ad[kRecBatch];
#pragma unroll
                for (int i = 0; i < kRecBatch; ++i) {
                    tg[i] = rtgt[urow[i] + p];
                    ad[i] = radd[urow[i] + p];
                }
#pragma unroll
                for (int i = 0; i < kRecBatch; ++i) {
                    const int rel = tg[i] - base_pos;
                    if (on[i] && tg[i] >= 0 && rel >= 0 && rel < hw)
                        atomicAdd(&gxs[(ch - ch0) * hw + rel], ad[i]);
                }
            }
        }
    }
    __syncthreads();
    const int64_t plane = int64_t(d.h) * d.w;
    for (int i = threadIdx.x; i < spw * nch * hw; i += 256) {
        const int si = i / (nch * hw), r = i % (nch * hw);
        const int chl = r / hw, rr = r - chl * hw;
        if (n0 + si < d.n)
            grad_x[(int64_t(n0 + si) * d.cin + ch0 + chl) * plane + int64_t(y0) * d.w + rr] = gx[i];
    }
}

// grad_w[c][q][g] = c0(g) M3 + c1(g) M1 + c2(g) M2 + c3(g) M0 with M the node's moments summed
// over the nblk partials in block order.  One thread per (c, q, g).
// Gradient of gate g of one node from its moments m = (sum gy a b, sum gy a, sum gy b,
// sum gy): of the probability, or with the node's logits of the logit.
template <typename T>
__device__ __forceinline__ T finalize_one(const T (&m)[4], const T* __restrict__ logits, int g) {
    auto prob_grad = [&](int h) {
        const Coef4<T> cf = gate_coef<T>(h);
        return fma(cf.c3, m[0], fma(cf.c2, m[2], fma(cf.c1, m[1], cf.c0 * m[3])));
    };
    if (!logits) return prob_grad(g);
    // softmax backward: every lane of the node forms all 16 probabilities and their
    // gradients itself, so the sum over the node is taken in one fixed order
    T p[16];
    node_probs(logits, true, p);
    T dot = 0, pg = 0;
#pragma unroll
    for (int h = 0; h < 16; ++h) {
        dot = fma(p[h], prob_grad(h), dot);
        pg = h == g ? p[h] : pg;  // a select per slot: no dynamic index into registers
    }
    return pg * (prob_grad(g) - dot);
}

template <typename T>
__global__ __launch_bounds__(256) void k_tree_finalize(const T* __restrict__ part, int64_t cout,
                                                       int nodes, int64_t nblk,
                                                       const T* __restrict__ logits,
                                                       T* __restrict__ grad_w) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= cout * nodes * 16) return;
    const int g = int(i & 15);
    const int64_t cq = i >> 4;
    const int64_t c = cq / nodes, q = cq % nodes;
    T m[4] = {0, 0, 0, 0};
    for (int64_t b = 0; b < nblk; ++b) {
        const T* src = part + ((c * nblk + b) * nodes + q) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) m[j] += src[j];
    }
    grad_w[i] = finalize_one<T>(m, logits ? logits + cq * 16 : nullptr, g);
}

// ------------------------------------------------------------------------------------------
// Staged backward of the complete block (float or double, when a sample's input fits LDS).
// A workgroup takes one sample and a group of cg output channels, stages the sample's input in
// LDS once (rows [-ph, hs - ph) and columns [-pw, ws - pw) of every input channel, zero outside
// the image, hs = (ho - 1) sh + kh, ws = (wo - 1) sw + kw: every tap inside the kernel window
// reads it without a bounds test), and computes per (channel, window) item what k_tree_nodes
// computes: the node values at the window's winner, the conv-gate gradients and the 28 node
// moments.  Lane group of L lanes per channel (L from P alone, so the summation order of a
// channel's moments is the same in every mode): lane l takes windows l, l + L, ... in order,
// then the L lanes are combined by an xor tree; the channel's sums for the sample go to
// part[(c * n + sample) * 32 + (node * 4 + m)] (28 of 32 words), summed over the samples in
// order by k_tree_moments.
//   MODE 0  moments only;
//   MODE 1  with the input gradient: every tap's contribution (the radd of k_tree_nodes) stays
//           in LDS, then lane groups of PL lanes per input channel walk its uses in use order
//           (for P <= PL the order of k_tree_gather_rec, so every plane word takes its
//           additions in the same order) into the sample's input gradient in LDS, stored once;
//           cg = cout;
//   MODE 2  with the conv-gate gradients stored for k_tree_gather (contributions that do not
//           fit LDS).
// A tap outside the kernel window (never drawn by the sampler) is read from global memory with
// bounds tests; a channel with a tap channel >= C gets NaN moments and that tap adds nothing.
struct TreeStage {
    int hs, ws, plane;  // staged rows, columns, words per input channel
    int kh, kw;
    int cg, groups;     // channels per workgroup, workgroups per sample
    int lanes;          // L: lanes per channel in the node phase (power of two)
    int glanes;         // PL: lanes per input channel in the gather (power of two, <= 64)
    int vec;            // rows of x (and grad_x) are whole 16-byte vectors, aligned
    int ul_words;       // MODE 1: room for the packed use list after the gradient planes
    int balance;        // MODE 1: input channels gathered in an order by use count
    int x_words;        // staged input (MODE 1: also the input gradient, after the node phase)
    int c_words;        // contributions (MODE 1)
    int64_t per_xcd;    // workgroups per XCD
    FastDiv div_hw, div_w, div_h, div_rv;  // by h * w, w, h, and the vectors per row
};

constexpr int kMomStride = 32;  // words per (channel, sample) moment record (28 used)

// A channel use u = c * 8 + k for the staged gather: its contribution slot
// c * 8 + ((k + c / 4) & 7) (the bank rotation of the contribution array) in the low 16 bits,
// the tap's column and row (selection bits 0..15) in the high 16.
__device__ __forceinline__ uint32_t pack_use(int u, int32_t sv) {
    const int c = u >> 3, k = u & 7;
    return uint32_t(c * 8 + ((k + (c >> 2)) & 7)) | (uint32_t(sv & 0xFFFF) << 16);
}

#ifndef CL_TREE_NT
#define CL_TREE_NT 1     // moment records stored non-temporally
#endif
#ifndef CL_TREE_UB
#define CL_TREE_UB 8     // channel uses a gather batch reads before its additions
#endif
#ifndef CL_TREE_NT_GX
#define CL_TREE_NT_GX 0  // the staged input gradient stored non-temporally (slower: 47 vs 38 us)
#endif

template <typename V>
__device__ __forceinline__ void nt_store(bool nt, V v, V* p) {
    if (nt) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <typename T, int MODE, int NT>
__global__ __launch_bounds__(NT) void k_tree_bwd_staged(
    const T* __restrict__ grad_y, const T* __restrict__ x, const T* __restrict__ kc,
    const int32_t* __restrict__ sel, const int32_t* __restrict__ idx,
    const int32_t* __restrict__ ent_ptr, const int32_t* __restrict__ ent, TreeDims d,
    TreeStage g, T* __restrict__ part, T* __restrict__ gconv, T* __restrict__ grad_x) {
    constexpr int VEC = 16 / sizeof(T);  // elements per 16-byte load or store
    typedef T V __attribute__((ext_vector_type(VEC)));
    constexpr int SB = 8;                 // staging loads in flight per thread
    constexpr int UB = CL_TREE_UB;        // channel uses whose records load together
    extern __shared__ unsigned char smem_raw[];
    T* xs = reinterpret_cast<T*>(smem_raw);
    // MODE 1: contributions cb[p * cs + cl * 8 + ((k + (cl >> 2)) & 7)] (the rotation by cl / 4
    // spreads a wave's stores of one tap over all banks; cs = cg * 8 + 1) and the winners'
    // input positions wins[p * (cg + 1) + cl] = (wy sh) << 16 | (wx sw), or -1 for none
    T* cb = xs + g.x_words;
    int* wins = reinterpret_cast<int*>(cb + g.c_words);
    // workgroups of one XCD take consecutive (sample, group) pairs: a sample's groups share
    // its staged input through that XCD's L2
    const int64_t bx = blockIdx.x;
    const int64_t j = (bx % 8) * g.per_xcd + bx / 8;
    if (j >= int64_t(d.n) * g.groups) return;  // whole workgroup, before any barrier
    const int n = int(j / g.groups), grp = int(j - int64_t(n) * g.groups);
    const int c0 = grp * g.cg, cg = min(g.cg, d.cout - c0);
    const int hw = d.h * d.w, nx = d.cin * hw;
    const T* xn = x + int64_t(n) * nx;
    const int t = threadIdx.x;
    const int cs = g.cg * kTaps + 1, wsd = g.cg + 1;

    // Node phase state.  Lane group of L lanes per channel; every lane walks cpl windows per
    // channel (those past P only keep the group in step for the xor tree).  The channel's
    // coefficients and taps and the first window's records are loaded before the staging,
    // and each window's records one window ahead of its use.
    const int L = g.lanes;
    const int l = t & (L - 1);
    const int cpl = (d.P + L - 1) / L;
    const int slots = NT / L;
    int cl = t / L;
    T sk[kMaxNodes][4];
    // staged word offsets of the taps (below 2^16: the LDS holds 40960 words), two 16-bit
    // halves a register; flags: bit k tap k staged, bit 8 a tap channel >= C
    uint32_t soff[kTaps / 2];
    uint32_t flags = 0;
    typedef T V4 __attribute__((ext_vector_type(4)));
    auto load_channel_regs = [&](int cc) {
        const int c = c0 + cc;
        // one vector load per node (the host checks kc's 16-byte alignment)
        const V4* kv = reinterpret_cast<const V4*>(kc) + int64_t(c) * kMaxNodes;
#pragma unroll
        for (int q = 0; q < kMaxNodes; ++q) {
            const V4 v = kv[q];
#pragma unroll
            for (int m = 0; m < 4; ++m) sk[q][m] = v[m];
        }
        flags = 0;
#pragma unroll
        for (int k = 0; k < kTaps; ++k) {
            const int32_t sv = sel[c * kTaps + k];
            const int ch = (sv >> 16) & 0xFFFF, row = (sv >> 8) & 0xFF, col = sv & 0xFF;
            const bool in = ch < d.cin && row < g.kh && col < g.kw;
            const uint32_t o = in ? uint32_t(ch * g.plane + row * g.ws + col) : 0u;
            if (k & 1) soff[k >> 1] |= o << 16;
            else soff[k >> 1] = o;
            flags |= uint32_t(in) << k | uint32_t(ch >= d.cin) << 8;
        }
    };
    int wn = -1;
    T gn = T(0);
    // item indices in 32 bits: the host checks n * cout * P < 2^31
    auto load_item = [&](int cc, int p) {
        const bool ok = cc < cg && p < d.P;
        const uint32_t c = uint32_t(c0 + (ok ? cc : 0)), pp = ok ? uint32_t(p) : 0u;
        const uint32_t at = (uint32_t(n) * uint32_t(d.cout) + c) * uint32_t(d.P) + pp;
        wn = ok ? idx[at] : -1;
        gn = ok ? grad_y[d.y_rows ? (c * uint32_t(d.P) + pp) * uint32_t(d.n) + uint32_t(n) : at]
                : T(0);
    };
    if (cl < cg) load_channel_regs(cl);
    load_item(cl, l);

    // staging: zero the region, then the sample with 16-byte loads (rows of whole vectors)
    // or element by element
    {
        V* xv = reinterpret_cast<V*>(xs);
        for (int i = t; i < g.x_words / VEC; i += NT) xv[i] = V(T(0));
        for (int i = (g.x_words / VEC) * VEC + t; i < g.x_words; i += NT) xs[i] = T(0);
    }
    __syncthreads();
    if (g.vec) {
        const V* src = reinterpret_cast<const V*>(xn);
        const int rv = d.w / VEC;  // vectors per input row
        const int nv = nx / VEC;
        for (int i0 = 0; i0 < nv; i0 += SB * NT) {
            V v[SB];
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int i = i0 + u * NT + t;
                if (i < nv) v[u] = src[i];
            }
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int i = i0 + u * NT + t;
                if (i >= nv) continue;
                const int r = int(fast_div(uint32_t(i), g.div_rv)), cv = i - r * rv;
                const int ch = int(fast_div(uint32_t(r), g.div_h)), iy = r - ch * d.h;
                const int sy = iy + d.ph;
                if (sy >= g.hs) continue;
                const int sx0 = cv * VEC + d.pw;
                T* dst = xs + ch * g.plane + sy * g.ws;
#pragma unroll
                for (int e = 0; e < VEC; ++e)
                    if (sx0 + e < g.ws) dst[sx0 + e] = v[u][e];
            }
        }
    } else {
        for (int i0 = 0; i0 < nx; i0 += SB * NT) {
            T v[SB];
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int i = i0 + u * NT + t;
                v[u] = i < nx ? xn[i] : T(0);
            }
#pragma unroll
            for (int u = 0; u < SB; ++u) {
                const int i = i0 + u * NT + t;
                if (i >= nx) continue;
                const int ch = int(fast_div(uint32_t(i), g.div_hw)), r = i - ch * hw;
                const int iy = int(fast_div(uint32_t(r), g.div_w)), ix = r - iy * d.w;
                const int sy = iy + d.ph, sx = ix + d.pw;
                if (sy < g.hs && sx < g.ws) xs[ch * g.plane + sy * g.ws + sx] = v[u];
            }
        }
    }
    __syncthreads();

    // node phase
    for (; cl < cg; cl += slots) {
        const int c = c0 + cl;
        const uint32_t cell = uint32_t(n) * uint32_t(d.cout) + uint32_t(c);
        T mom[28];
#pragma unroll
        for (int i = 0; i < 28; ++i) mom[i] = T(0);
        for (int i = 0; i < cpl; ++i) {
            const int p = l + i * L;
            const int win = wn;
            const T gyv = gn;
            if (i + 1 < cpl) load_item(cl, p + L);
            else load_item(cl + slots, l);
            if (p >= d.P) continue;
            const bool live = win >= 0 && win < d.ho * d.wo;
            const int w0 = live ? win : 0;
            const int wy = int(fast_div(uint32_t(w0), d.div_wo)), wx = w0 - wy * d.wo;
            const int pos = wy * d.sh * g.ws + wx * d.sw;
            T v[kTaps];
#pragma unroll
            for (int k = 0; k < kTaps; ++k)
                v[k] = xs[((k & 1) ? soff[k >> 1] >> 16 : soff[k >> 1] & 0xFFFFu) + pos];
            if ((flags & 0xFFu) != 0xFFu) {
#pragma unroll
                for (int k = 0; k < kTaps; ++k)
                    if (!((flags >> k) & 1))
                        v[k] = tap_value(xn, d, decode_tap(sel[c * kTaps + k], d.ph, d.pw),
                                         wy, wx);
            }
            T gg[4], tt[2], gc[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) gg[q] = node(sk[q], v[2 * q], v[2 * q + 1]);
            tt[0] = node(sk[4], gg[0], gg[1]);
            tt[1] = node(sk[5], gg[2], gg[3]);
            const T gy = live ? gyv : T(0);
            node_grads<T>(sk, gg, tt, gy, gc, mom);
            gate_moments<T>(v, gc, mom);
            if constexpr (MODE == 1) {
                const int rot = cl >> 2;
#pragma unroll
                for (int k = 0; k < kTaps; ++k) {
                    const int q = k >> 1;
                    cb[p * cs + cl * kTaps + ((k + rot) & 7)] =
                        gc[q] * fma(sk[q][3], v[k ^ 1], (k & 1) ? sk[q][2] : sk[q][1]);
                }
                wins[p * wsd + cl] = live ? ((wy * d.sh) << 16 | (wx * d.sw)) : -1;
            }
            if constexpr (MODE == 2) {
#pragma unroll
                for (int q = 0; q < 4; ++q) gconv[(cell * uint32_t(d.P) + p) * 4 + q] = gc[q];
            }
        }
        // the channel's lanes combined in a fixed xor tree (the whole group is active)
        for (int o = 1; o < L; o <<= 1) {
#pragma unroll
            for (int i = 0; i < 28; ++i) mom[i] += __shfl_xor(mom[i], o, 64);
        }
        if (l == 0 && part) {
            // streamed past L2: the records are read by the next launch only
            T* dst = part + (uint32_t(c) * uint32_t(d.n) + uint32_t(n)) * kMomStride;
#pragma unroll
            for (int i = 0; i < 28; ++i)
                nt_store<T>(CL_TREE_NT, (flags >> 8) ? quiet_nan<T>() : mom[i], dst + i);
        }
        if (cl + slots < cg) load_channel_regs(cl + slots);
    }
    if constexpr (MODE == 1) {
        __syncthreads();  // the staged input is dead: its words take the input gradient
        for (int i = t; i < nx; i += NT) xs[i] = T(0);
        // the use list with its taps, packed u | row << 16 | col << 24 (u = c * 8 + k), into
        // the words after the gradient planes when it fits there (g.ul_words), loaded by all
        // threads at once
        const int ea = ent_ptr[0], eb = ent_ptr[d.cin];
        const bool in_lds = ea >= 0 && eb >= ea && eb - ea <= g.ul_words;
        uint32_t* ul = reinterpret_cast<uint32_t*>(xs + nx);
        if (in_lds) {
            for (int e0 = ea; e0 < eb; e0 += 4 * NT) {
                int u4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int e = e0 + q * NT + t;
                    u4[q] = e < eb ? ent[e] : -1;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int e = e0 + q * NT + t;
                    const bool ok = uint32_t(u4[q]) < uint32_t(cg * kTaps);
                    const int32_t sv = sel[ok ? u4[q] : 0];
                    if (e < eb) ul[e - ea] = ok ? pack_use(u4[q], sv) : 0xFFFFFFFFu;
                }
            }
        }
        // Channels dealt to the lane groups in an order by use count (a counting sort by
        // LDS atomics): a wave's groups then walk about as many uses each, where in channel
        // order the wave waits for its busiest channel.  Each channel's additions keep their
        // order, so the order of the channels changes no result.
        int* perm = wins + d.P * (g.cg + 1);  // after the winners: [cin], then [64]
        int* hist = perm + d.cin;
        int bin = 0, pos = 0;
        if (g.balance) {
            if (t < 64) hist[t] = 0;
            __syncthreads();
            if (t < d.cin) {
                const int cnt = ent_ptr[t + 1] - ent_ptr[t];
                bin = 63 - min(max(cnt, 0), 63);  // busiest first
                pos = atomicAdd(&hist[bin], 1);
            }
            __syncthreads();
            if (t < 64) {  // exclusive scan of the 64 bins by the first wave
                const int h = hist[t];
                int incl = h;
                for (int o = 1; o < 64; o <<= 1) {
                    const int v = __shfl_up(incl, o, 64);
                    if (t >= o) incl += v;
                }
                hist[t] = incl - h;
            }
            __syncthreads();
            if (t < d.cin) perm[hist[bin] + pos] = t;
        }
        __syncthreads();
        const int PL = g.glanes;
        const int pl = t & (PL - 1);
        for (int chs = t / PL; chs < d.cin; chs += NT / PL) {
            const int ch = g.balance ? perm[chs] : chs;
            const int e0 = ent_ptr[ch], e1 = ent_ptr[ch + 1];
            T* gp = xs + ch * hw;
            for (int e = e0; e < e1; e += UB) {
                uint32_t rb[UB];
                if (in_lds) {
#pragma unroll
                    for (int i = 0; i < UB; ++i) {
                        const int ee = e + i - ea;
                        rb[i] = e + i < e1 && uint32_t(ee) < uint32_t(eb - ea) ? ul[ee]
                                                                                 : 0xFFFFFFFFu;
                    }
                } else {
                    int ub[UB];
#pragma unroll
                    for (int i = 0; i < UB; ++i) ub[i] = e + i < e1 ? ent[e + i] : -1;
#pragma unroll
                    for (int i = 0; i < UB; ++i) {
                        const bool ok = uint32_t(ub[i]) < uint32_t(cg * kTaps);
                        const int32_t sv = sel[ok ? ub[i] : 0];
                        rb[i] = ok ? pack_use(ub[i], sv) : 0xFFFFFFFFu;
                    }
                }
                // per window pass: the batch's winners and contributions read first, then
                // its additions in use order (within one use the windows add to distinct
                // pixels, so each plane word takes its additions in a fixed order: by window
                // pass, then by use)
                for (int p = pl; p < d.P; p += PL) {
                    int tg[UB];
                    T cv[UB];
#pragma unroll
                    for (int i = 0; i < UB; ++i) {
                        const bool on = rb[i] != 0xFFFFFFFFu;
                        const int slot = on ? int(rb[i] & 0xFFFF) : 0, c = slot >> 3;
                        const int pk = wins[p * wsd + c];
                        cv[i] = cb[p * cs + slot];
                        const int iy = (pk >> 16) + int(rb[i] >> 24) - d.ph;
                        const int ix = (pk & 0xFFFF) + int((rb[i] >> 16) & 0xFF) - d.pw;
                        tg[i] = on && pk >= 0 && uint32_t(iy) < uint32_t(d.h) &&
                                        uint32_t(ix) < uint32_t(d.w)
                                    ? iy * d.w + ix
                                    : -1;
                    }
#pragma unroll
                    for (int i = 0; i < UB; ++i)
                        if (tg[i] >= 0) gp[tg[i]] += cv[i];
                }
            }
        }
        __syncthreads();
        T* gxn = grad_x + int64_t(n) * nx;
        if (g.vec) {
            V* gv = reinterpret_cast<V*>(gxn);
            const V* lv = reinterpret_cast<const V*>(xs);
            for (int i = t; i < nx / VEC; i += NT) nt_store<V>(CL_TREE_NT_GX, lv[i], gv + i);
        } else {
            for (int i = t; i < nx; i += NT) nt_store<T>(CL_TREE_NT_GX, xs[i], gxn + i);
        }
    }
}

// Collapsed coefficients kc[c][q][:] of every node (from the logits with d.softmax).
template <typename T>
__global__ __launch_bounds__(64) void k_tree_coefs(const T* __restrict__ w_prob,
                                                   const int32_t* __restrict__ sel, TreeDims d,
                                                   T* __restrict__ kc) {
    __shared__ T sk[kMaxNodes][4];
    __shared__ TapOff st[kTaps];
    __shared__ int bad;
    const int c = blockIdx.x;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    load_channel(w_prob, sel, c, kMaxNodes, d, sk, st, &bad);
    __syncthreads();
    if (threadIdx.x < kMaxNodes * 4)
        kc[int64_t(c) * kMaxNodes * 4 + threadIdx.x] = sk[threadIdx.x >> 2][threadIdx.x & 3];
}

// The staged pass's moment records summed over the samples, then the weight gradient as in
// k_tree_finalize.  Workgroup per channel: thread (s, i) sums moment i over the s-th of 32
// contiguous runs of samples in order, the 32 run sums are added in a fixed tree, and threads
// (q, g) finish node q's gate g.
template <typename T>
__global__ __launch_bounds__(1024) void k_tree_moments(const T* __restrict__ part, int n,
                                                       const T* __restrict__ logits,
                                                       T* __restrict__ grad_w) {
    __shared__ T run[32][28];
    __shared__ T mom[28];
    const int c = blockIdx.x, t = threadIdx.x;
    const int s = t >> 5, i = t & 31;
    const int per = (n + 31) / 32;
    if (i < 28) {
        const T* src = part + int64_t(c) * n * kMomStride + i;
        const int lo = min(n, s * per), hi = min(n, lo + per);
        T a = 0;
        int k = lo;
        for (; k + 4 <= hi; k += 4) {
            const T v0 = src[int64_t(k) * kMomStride], v1 = src[int64_t(k + 1) * kMomStride];
            const T v2 = src[int64_t(k + 2) * kMomStride], v3 = src[int64_t(k + 3) * kMomStride];
            a += v0;
            a += v1;
            a += v2;
            a += v3;
        }
        for (; k < hi; ++k) a += src[int64_t(k) * kMomStride];
        run[s][i] = a;
    }
    __syncthreads();
    if (t < 28) {
        T r[32];
#pragma unroll
        for (int k = 0; k < 32; ++k) r[k] = run[k][t];
#pragma unroll
        for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
            for (int k = 0; k < w; ++k) r[k] = r[k] + r[k + w];
        mom[t] = r[0];
    }
    __syncthreads();
    if (t < kMaxNodes * 16) {
        const int q = t >> 4, gg = t & 15;
        const T m[4] = {mom[q * 4 + 0], mom[q * 4 + 1], mom[q * 4 + 2], mom[q * 4 + 3]};
        const int64_t at = (int64_t(c) * kMaxNodes + q) * 16 + gg;
        grad_w[at] = finalize_one<T>(m, logits ? logits + (int64_t(c) * kMaxNodes + q) * 16
                                               : nullptr, gg);
    }
}

// ------------------------------------------------------------------------------------------
// One tree level (TreeLogicLayer): x[..., 2j], x[..., 2j + 1] -> y[..., j] with node j of the
// element's channel.  x is [N, C, S, 2 * xo] (S = H * W), y [N, C, S, xo].
template <typename T>
__global__ __launch_bounds__(256) void k_level_fwd(const T* __restrict__ x, const T* __restrict__ w_prob,
                                                   int64_t n, int64_t c_dim, int64_t s, int xo,
                                                   T* __restrict__ y) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;  // (n, c, s, j)
    const int64_t total = n * c_dim * s * xo;
    if (i >= total) return;
    const int j = int(i % xo);
    const int64_t c = (i / xo / s) % c_dim;
    const T* p = w_prob + (c * xo + j) * 16;
    T k[4] = {0, 0, 0, 0};
    for (int g = 0; g < 16; ++g) {
        const Coef4<T> cf = gate_coef<T>(g);
        k[0] = fma(p[g], cf.c0, k[0]);
        k[1] = fma(p[g], cf.c1, k[1]);
        k[2] = fma(p[g], cf.c2, k[2]);
        k[3] = fma(p[g], cf.c3, k[3]);
    }
    const int64_t base = (i / xo) * 2 * xo + 2 * j;
    y[i] = node(k, x[base], x[base + 1]);
}

// Tree level backward: grad_x elementwise, node moments per workgroup (fixed order) into
// part[(c * nblk + blk) * xo * 4 + j * 4 + m]; the workgroup's items all have channel
// blockIdx.y (items are (n, s) pairs).
template <typename T>
__global__ __launch_bounds__(256) void k_level_bwd(const T* __restrict__ grad_y, const T* __restrict__ x,
                                                   const T* __restrict__ w_prob, int64_t n,
                                                   int64_t c_dim, int64_t s, int xo,
                                                   T* __restrict__ grad_x, T* __restrict__ part) {
    constexpr int kMaxOut = 4;
    __shared__ T sk[kMaxOut][4];
    __shared__ T red[4][kMaxOut * 4];
    const int c = blockIdx.y;
    if (threadIdx.x < xo * 4) {
        const int j = threadIdx.x >> 2, m = threadIdx.x & 3;
        const T* p = w_prob + (int64_t(c) * xo + j) * 16;
        T acc = 0;
        for (int g = 0; g < 16; ++g) {
            const Coef4<T> cf = gate_coef<T>(g);
            acc = fma(p[g], m == 0 ? cf.c0 : m == 1 ? cf.c1 : m == 2 ? cf.c2 : cf.c3, acc);
        }
        sk[j][m] = acc;
    }
    __syncthreads();
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;
    T mom[kMaxOut * 4];
#pragma unroll
    for (int i = 0; i < kMaxOut * 4; ++i) mom[i] = T(0);
    if (item < n * s) {
        const int64_t nn = item / s, ss = item % s;
        const int64_t row = (nn * c_dim + c) * s + ss;
#pragma unroll
        for (int j = 0; j < kMaxOut; ++j) {
            if (j >= xo) continue;
            const T a = x[row * 2 * xo + 2 * j], b = x[row * 2 * xo + 2 * j + 1];
            const T g = grad_y[row * xo + j];
            if (grad_x) {
                grad_x[row * 2 * xo + 2 * j] = g * fma(sk[j][3], b, sk[j][1]);
                grad_x[row * 2 * xo + 2 * j + 1] = g * fma(sk[j][3], a, sk[j][2]);
            }
            mom[j * 4 + 0] = g * a * b;
            mom[j * 4 + 1] = g * a;
            mom[j * 4 + 2] = g * b;
            mom[j * 4 + 3] = g;
        }
    }
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < kMaxOut * 4; ++i) {
        if (i >= xo * 4) continue;  // uniform
        const T t = wave_total(mom[i]);
        if (lane == 0) red[wv][i] = t;
    }
    __syncthreads();
    if (threadIdx.x < xo * 4) {
        const int i = threadIdx.x;
        part[(int64_t(c) * gridDim.x + blockIdx.x) * xo * 4 + i] =
            (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
    }
}

// ------------------------------------------------------------------------------------------
// Packed discrete block: rows of 64-bit words, one row per (channel, y, x) of the NCHW input
// (row = (ch * H + y) * W + x); output rows (c * Hp + py) * Wp + px (complete) or
// ((c * Ho + oy) * Wo + ox) * 4 + q (conv gates only).  gates[c * nodes + q] is node q's opcode;
// the pool of {0, 1} values is the OR of the window.
//
// Every input pixel is read by many output rows (all taps of all output channels that name
// its channel), so the words are cut into chunks of kPkChunk and a workgroup evaluates a block
// of output rows over one chunk.  Chunk j runs only on XCD j % 8 (workgroup w runs on XCD
// w % 8), all row blocks of a chunk before the next chunk of that XCD: the chunk's slice of
// the input (rows x 256 B) stays in the XCD's L2 while every output row reads it.
//
// A lane holds WPL consecutive words of one row (WPL = 2: 16-byte loads and stores), so a
// row's opcodes, tap offsets and bounds are worked out once per WPL words.  Tap loads are
// unconditional (a tap outside the image reads row 0 and is masked to zero afterwards) and the
// row index is 32-bit (the input holds fewer than 2^31 rows), leaving one 64-bit multiply-add
// per load.
constexpr int kPkChunk = 32;  // words per chunk (one 256-byte row segment)

// Opcode g as four minterm masks: result bit = m[a][b] of the (a, b) bit pair.
struct GateMask {
    uint32_t m00, m01, m10, m11;
};

__device__ __forceinline__ GateMask gate_mask(int g) {
    GateMask m;
    m.m00 = 0u - uint32_t((g >> 3) & 1);
    m.m01 = 0u - uint32_t((g >> 2) & 1);
    m.m10 = 0u - uint32_t((g >> 1) & 1);
    m.m11 = 0u - uint32_t(g & 1);
    return m;
}

template <int N>
struct Bits {
    uint32_t v[N];
};

template <int N>
__device__ __forceinline__ Bits<N> apply_gate(const GateMask& m, const Bits<N>& a,
                                              const Bits<N>& b) {
    Bits<N> o;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t if_b = (a.v[i] & m.m11) | (~a.v[i] & m.m01);
        const uint32_t if_not_b = (a.v[i] & m.m10) | (~a.v[i] & m.m00);
        o.v[i] = (b.v[i] & if_b) | (~b.v[i] & if_not_b);
    }
    return o;
}

template <int WPL>
__device__ __forceinline__ Bits<2 * WPL> load_words(const uint64_t* p, uint32_t mask) {
    Bits<2 * WPL> r;
    if constexpr (WPL == 2) {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        r.v[0] = q.x & mask, r.v[1] = q.y & mask, r.v[2] = q.z & mask, r.v[3] = q.w & mask;
    } else {
        const uint2 q = *reinterpret_cast<const uint2*>(p);
        r.v[0] = q.x & mask, r.v[1] = q.y & mask;
    }
    return r;
}

template <int WPL>
__device__ __forceinline__ void store_words(uint64_t* p, const Bits<2 * WPL>& r) {
    if constexpr (WPL == 2) {
        *reinterpret_cast<uint4*>(p) = make_uint4(r.v[0], r.v[1], r.v[2], r.v[3]);
    } else {
        *reinterpret_cast<uint2*>(p) = make_uint2(r.v[0], r.v[1]);
    }
}

// At most four waves per SIMD: the tap offsets, gate masks and loaded words then fit in
// registers without scratch.
template <int WPL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4))) void k_tree_packed(
    const uint64_t* __restrict__ x, int64_t words, const uint8_t* __restrict__ gates,
    const int32_t* __restrict__ sel, TreeDims d, int64_t nchunks, int64_t rblocks,
    uint64_t* __restrict__ y) {
    constexpr int kLanes = kPkChunk / WPL;  // lanes per row segment
    constexpr int kRows = 256 / kLanes;     // output rows per workgroup
    constexpr int N = 2 * WPL;              // 32-bit halves per lane
    // Grid, row and chunk counts are below 2^31 (checked by the caller): 32-bit index math.
    uint32_t chunk, rb;
    const uint32_t wg = blockIdx.x, nrb = uint32_t(rblocks);
    if (nchunks >= 8) {
        const uint32_t j = wg / 8;
        chunk = wg % 8 + 8 * (j / nrb);
        rb = j % nrb;
    } else {
        chunk = wg / nrb;
        rb = wg % nrb;
    }
    if (chunk >= uint32_t(nchunks)) return;  // uniform per workgroup
    const uint32_t r = rb * kRows + threadIdx.x / kLanes;
    const int64_t w = int64_t(chunk) * kPkChunk + (threadIdx.x % kLanes) * WPL;
    if (r >= uint32_t(d.cout) * uint32_t(d.P) || w >= words) return;
    const int c = int(r / uint32_t(d.P)), p = int(r % uint32_t(d.P));
    const int nodes = d.complete ? 7 : 4;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < kTaps; ++k) bad |= ((sel[c * kTaps + k] >> 16) & 0xFFFF) >= d.cin;
    const char* xw = reinterpret_cast<const char*>(x + w);
    const uint32_t row_stride = uint32_t(words) * 8u;  // bytes; words < 2^28 (caller)
    // Tap value at conv position (oy, ox).  Row arithmetic is unsigned 32-bit: for a tap inside
    // the image the wrapped sum equals the row (ch * H + iy) * W + ix < 2^31.
    auto tap = [&](const TapOff& t, uint32_t base, int oy, int ox) -> Bits<N> {
        const int iy = oy * d.sh + t.dy, ix = ox * d.sw + t.dx;
        const bool ok = (!bad) & (unsigned(iy) < unsigned(d.h)) & (unsigned(ix) < unsigned(d.w));
        const uint32_t row = ok ? base + uint32_t(oy * d.sh) * uint32_t(d.w) + uint32_t(ox * d.sw)
                                : 0u;
        return load_words<WPL>(
            reinterpret_cast<const uint64_t*>(xw + uint64_t(row) * uint64_t(row_stride)),
            ok ? ~0u : 0u);
    };
    auto plane_base = [&](const TapOff& t) -> uint32_t {
        return (uint32_t(t.ch) * uint32_t(d.h) + uint32_t(t.dy)) * uint32_t(d.w) + uint32_t(t.dx);
    };
    Bits<N> out;
    if (d.complete) {
        GateMask gm[kMaxNodes];
#pragma unroll
        for (int q = 0; q < kMaxNodes; ++q) gm[q] = gate_mask(gates[c * nodes + q] & 15);
        TapOff t[kTaps];
        uint32_t base[kTaps];
#pragma unroll
        for (int k = 0; k < kTaps; ++k) {
            t[k] = decode_tap(sel[c * kTaps + k], d.ph, d.pw);
            base[k] = plane_base(t[k]);
        }
        const int wp = d.wo / 2;
        const int py = p / wp, px = p % wp;
#pragma unroll
        for (int i = 0; i < N; ++i) out.v[i] = 0;
#pragma unroll
        for (int dy2 = 0; dy2 < 2; ++dy2)
#pragma unroll
            for (int dx2 = 0; dx2 < 2; ++dx2) {
                const int oy = 2 * py + dy2, ox = 2 * px + dx2;
                Bits<N> g[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    g[q] = apply_gate(gm[q], tap(t[2 * q], base[2 * q], oy, ox),
                                      tap(t[2 * q + 1], base[2 * q + 1], oy, ox));
                const Bits<N> r3 = apply_gate(gm[6], apply_gate(gm[4], g[0], g[1]),
                                              apply_gate(gm[5], g[2], g[3]));
#pragma unroll
                for (int i = 0; i < N; ++i) out.v[i] |= r3.v[i];
            }
    } else {
        const int q = p & 3, pos = p >> 2;
        const int oy = pos / d.wo, ox = pos % d.wo;
        const TapOff ta = decode_tap(sel[c * kTaps + 2 * q], d.ph, d.pw);
        const TapOff tb = decode_tap(sel[c * kTaps + 2 * q + 1], d.ph, d.pw);
        out = apply_gate(gate_mask(gates[c * nodes + q] & 15), tap(ta, plane_base(ta), oy, ox),
                         tap(tb, plane_base(tb), oy, ox));
    }
    if (bad) {
#pragma unroll
        for (int i = 0; i < N; ++i) out.v[i] = ~0u;
    }
    store_words<WPL>(y + int64_t(r) * words + w, out);
}

template <typename T>
__global__ __launch_bounds__(256) void k_zero(T* __restrict__ p, int64_t count) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < count) p[i] = T(0);
}

// Zero `count` elements with a kernel (not a memset node, so the call stays graph-safe).
template <typename T>
int zero_fill(void* p, int64_t count, hipStream_t s, const char* what) {
    if (count <= 0 || !p) return CL_OK;
    CL_ARG(ceil_div(count, 256) < (int64_t(1) << 31), "tensor too large");
    k_zero<T><<<unsigned(ceil_div(count, 256)), 256, 0, s>>>(static_cast<T*>(p), count);
    return check_launch(what);
}

int tree_dims(TreeDims& d, int64_t n, int64_t cin, int64_t h, int64_t w, int64_t cout, int sh,
              int sw, int ph, int pw, int kh, int kw, int complete) {
    CL_ARG(n >= 0 && cin >= 1 && h >= 1 && w >= 1 && cout >= 0, "bad block shape");
    CL_ARG(sh >= 1 && sw >= 1 && ph >= 0 && pw >= 0 && kh >= 1 && kw >= 1,
           "bad stride / padding / kernel");
    CL_ARG(cin <= 0xFFFF && h <= 4096 && w <= 4096 && kh <= 255 && kw <= 255 && ph <= 255 &&
               pw <= 255,
           "block dimensions beyond the selection encoding");
    const int64_t ho = (h + 2 * ph - kh) / sh + 1, wo = (w + 2 * pw - kw) / sw + 1;
    CL_ARG(h + 2 * ph >= kh && w + 2 * pw >= kw && ho > 0 && wo > 0,
           "invalid output shape: H_out=%lld, W_out=%lld", (long long)ho, (long long)wo);
    if (complete)
        CL_ARG(ho % 2 == 0 && wo % 2 == 0,
               "Output height and width after convolution must be divisible by 2 for 2x2 max "
               "pooling, but got H_out=%lld, W_out=%lld",
               (long long)ho, (long long)wo);
    const int64_t P = complete ? (ho / 2) * (wo / 2) : ho * wo;
    CL_ARG(cin * h * w < (int64_t(1) << 31), "one sample's input must have fewer than 2^31 elements");
    CL_ARG(n * cin * h * w < (int64_t(1) << 40) && cout * P < (int64_t(1) << 31) &&
               n * P < (int64_t(1) << 40) && cout < 65536,
           "block too large");
    d.n = int(n);
    d.coefs = nullptr;
    d.cin = int(cin);
    d.h = int(h);
    d.w = int(w);
    d.cout = int(cout);
    d.ho = int(ho);
    d.wo = int(wo);
    d.sh = sh;
    d.sw = sw;
    d.ph = ph;
    d.pw = pw;
    d.complete = complete ? 1 : 0;
    d.softmax = 0;
    d.regular = 0;
    d.y_rows = 0;
    d.P = int(P);
    d.div_p = make_fastdiv(uint32_t(std::max<int64_t>(P, 1)));
    d.div_wp = make_fastdiv(uint32_t(std::max<int64_t>(complete ? wo / 2 : wo, 1)));
    d.div_wo = make_fastdiv(uint32_t(std::max<int64_t>(wo, 1)));
    return CL_OK;
}

// Items per lane-group pass of the gather kernel: the next power of two >= P, at most 64.
int gather_lanes(int P) {
    int pw = 1;
    while (pw < P && pw < 64) pw <<= 1;
    return pw;
}

constexpr int64_t kGatherLdsBytes = 64 * 1024;

constexpr int64_t kFwdLdsLimit = 160 * 1024;  // LDS of one gfx950 CU
constexpr int kFwdLdsThreads = 1024;
constexpr int kMaxDevices = 64;

// Geometry of an LDS-staged kernel with `ip` items per (sample, channel), or false when one
// sample's padded input does not fit or staging does not pay: a sample's items must number
// at least `ratio` times its input elements (the forward asks 2; conv1 of the tree reading of
// cfg3 has 7).
template <typename T>
bool plan_tree_lds(const TreeDims& d, int kh, int kw, int ip, int ratio, TreeLds& g,
                   int& groups, int64_t& lds) {
    const int hpad = d.h + 2 * d.ph, wpad = d.w + 2 * d.pw;
    g.kh = kh;
    g.kw = kw;
    g.ws = (wpad + d.sw - 1) / d.sw;
    g.ip = ip;
    const int base = d.sw * g.ws;
    const int64_t tab = int64_t(d.complete ? 28 : 16) * sizeof(T) + (kTaps + 1) * 4;
    const int64_t staged = int64_t(d.cin) * d.h * d.w;
    if (int64_t(d.cout) * g.ip < ratio * staged) return false;
    auto total = [&](int rp, int64_t cg) {
        return int64_t(d.cin) * hpad * rp * int64_t(sizeof(T)) + cg * tab;
    };
    // Row pitch: conv rows oy and oy + 1 are sh * rp words apart; 16 banks apart (mod 32)
    // puts the two rows of a half-wave on distinct banks.
    int rp = base;
    for (int e = 0; e <= 16; ++e)
        if ((int64_t(d.sh) * (base + e)) % 32 == 16) {
            rp = base + e;
            break;
        }
    if (total(rp, 1) > kFwdLdsLimit) rp = base;
    if (total(rp, 1) > kFwdLdsLimit) return false;
    if (int64_t(d.cin) * hpad * rp >= (int64_t(1) << 30)) return false;
    g.rp = rp;
    g.cs = hpad * rp;
    // Channel groups: enough workgroups to fill the chip twice while every workgroup still
    // computes at least twice as many items as it stages input elements; then as many more
    // as LDS needs.
    int64_t G = 1;
    while (int64_t(d.n) * G < 512 && 2 * G <= d.cout &&
           ceil_div(d.cout, 2 * G) * g.ip >= staged)
        G *= 2;
    while (total(rp, ceil_div(d.cout, G)) > kFwdLdsLimit) ++G;
    g.cg = int(ceil_div(d.cout, G));
    groups = int(ceil_div(d.cout, g.cg));
    lds = total(rp, g.cg);
    g.div_pos = make_fastdiv(uint32_t(d.complete ? d.wo / 2 : d.wo));
    g.idx32 = int64_t(d.n) * d.cout * d.P < (int64_t(1) << 31) ? 1 : 0;
    g.div_hw = make_fastdiv(uint32_t(d.h * d.w));
    g.div_w = make_fastdiv(uint32_t(d.w));
    g.div_sw = make_fastdiv(uint32_t(d.sw));
    return groups < 65536;
}

// Above 64 KiB of LDS a kernel needs the attribute, set once per device and kernel.
template <typename K>
int reserve_lds(K* kern, int64_t lds, bool* reserved, const char* what) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("cannot query the device");
        return CL_ERR_HIP;
    }
    if (lds > 64 * 1024 && !reserved[dev]) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                int(kFwdLdsLimit)) != hipSuccess) {
            set_error("cannot reserve %lld bytes of LDS for %s", (long long)lds, what);
            return CL_ERR_HIP;
        }
        reserved[dev] = true;
    }
    return CL_OK;
}

template <typename T, bool COMPLETE>
int launch_tree_fwd_lds(const TreeDims& d, const TreeLds& g, int groups, int64_t lds,
                        const T* x, const T* w_prob, const int32_t* sel, T* y, T* x2, T* x3,
                        int32_t* idx, hipStream_t s) {
    void (*kern)(const T*, const T*, const int32_t*, TreeDims, TreeLds, T*, T*, T*, int32_t*);
    const bool inter = x2 != nullptr || x3 != nullptr;
    if constexpr (sizeof(T) == 4) {
        if (!inter) kern = &k_tree_fwd_lds_f32<COMPLETE>;
        else kern = &k_tree_fwd_lds<T, COMPLETE, true>;
    } else {
        kern = inter ? &k_tree_fwd_lds<T, COMPLETE, true> : &k_tree_fwd_lds<T, COMPLETE, false>;
    }
    static bool reserved[2][kMaxDevices] = {};  // per kernel chosen below
    if (int rc = reserve_lds(kern, lds, reserved[inter ? 1 : 0], "the tree block forward"))
        return rc;
    kern<<<dim3(unsigned(d.n), unsigned(groups)), kFwdLdsThreads, size_t(lds), s>>>(
        x, w_prob, sel, d, g, y, x2, x3, idx);
    if (int rc = check_launch("cl_tree_conv_forward")) return rc;
    if (d.regular) return CL_OK;  // no channel for the fix-up pass, by the caller's guarantee
    k_tree_fwd_fix<T, COMPLETE><<<unsigned(ceil_div(d.cout, kFixChannels)), kFixChannels, 0, s>>>(
        x, w_prob, sel, d, g.kh, g.kw, y, x2, x3, idx);
    return check_launch("cl_tree_conv_forward");
}

// Partial moment blocks per channel of the backward node pass, and the items per thread: about
// CL_TREE_NODE_WGS workgroups in all (more waves in flight than one block per channel gives
// small planes), at most kNodeItems items per thread.
inline int64_t node_blocks(const TreeDims& d, int* node_items = nullptr) {
    const int64_t total = int64_t(d.n) * d.P;
    const int64_t per_item_round = 256;
    int64_t nblk = std::max<int64_t>(1, ceil_div(int64_t(CL_TREE_NODE_WGS), int64_t(d.cout)));
    nblk = std::min(nblk, std::max<int64_t>(1, ceil_div(total, per_item_round)));
    int64_t items = ceil_div(total, nblk * per_item_round);
    if (items > kNodeItems) {
        items = kNodeItems;
        nblk = ceil_div(total, per_item_round * kNodeItems);
    }
    if (node_items) *node_items = int(std::max<int64_t>(1, items));
    return nblk;
}

// The complete block's input-gradient contributions: radd (T) then rtgt (int32), one of each
// per (channel, tap, item).
inline int64_t tree_records(const TreeDims& d) { return int64_t(d.cout) * kTaps * d.n * d.P; }

#ifndef CL_TREE_STAGED_BWD
#define CL_TREE_STAGED_BWD 1  // the staged backward of the complete block where it fits
#endif
#ifndef CL_TREE_LMAX
#define CL_TREE_LMAX 4  // most lanes per channel in the staged backward's node phase
#endif
#ifndef CL_TREE_STAGED_NT1
#define CL_TREE_STAGED_NT1 1024  // threads of the float form with the input gradient
#endif

// Plan of k_tree_bwd_staged, or false when it does not apply (then the node pass with global
// taps runs).  The decision and the lane count L depend on the shape and type alone, not on
// whether the input gradient is wanted, so the weight gradient is the same either way.
struct StagePlan {
    TreeStage g;
    int mode, threads;
    int64_t lds;
    unsigned grid;
};

bool plan_tree_stage(const TreeDims& d, int kh, int kw, bool want_gx, size_t tsize,
                     StagePlan& sp) {
    if (!CL_TREE_STAGED_BWD || !d.complete || d.P < 1 || kh < 1 || kw < 1) return false;
    TreeStage& g = sp.g;
    g.kh = kh;
    g.kw = kw;
    g.hs = (d.ho - 1) * d.sh + kh;
    g.ws = (d.wo - 1) * d.sw + kw;
    g.plane = g.hs * g.ws;
    int L = 1;  // min(CL_TREE_LMAX, largest power of two <= P / 2), at least 1
    while (2 * L <= CL_TREE_LMAX && 4 * L <= d.P) L *= 2;
    g.lanes = L;
    g.glanes = gather_lanes(d.P);
    // float: 1024 threads (16 waves, one workgroup per CU); double: 512 (its registers)
    sp.threads = tsize == 4 ? CL_TREE_STAGED_NT1 : 512;
    const int64_t xw = int64_t(d.cin) * g.plane, nx = int64_t(d.cin) * d.h * d.w;
    if (xw * int64_t(tsize) > kFwdLdsLimit || nx >= (int64_t(1) << 31)) return false;
    // MODE 1: staged input / input gradient (+ the packed use list when it fits), the
    // contributions and the winners, for all channels in one workgroup
    const int64_t c1 = int64_t(d.P) * (int64_t(d.cout) * kTaps + 1);
    const int64_t w1 = int64_t(d.P) * (d.cout + 1);
    auto lds_of = [&](int64_t xwords) { return (xwords + c1) * int64_t(tsize) + w1 * 4; };
    int64_t x1 = std::max(xw, nx + int64_t(d.cout) * kTaps);
    if (lds_of(x1) > kFwdLdsLimit) x1 = std::max(xw, nx);
    if (want_gx && lds_of(x1) <= kFwdLdsLimit && int64_t(d.cout) * kTaps < 65535) {
        sp.mode = 1;
        g.cg = d.cout;
        g.x_words = int(x1);
        g.c_words = int(c1);
        g.ul_words = int(x1 - nx);
        sp.lds = lds_of(x1);
        // the gather's channel order by use count (after the winners), when it fits
        g.balance = (d.cin <= sp.threads &&
                     sp.lds + (int64_t(d.cin) + 64) * 4 <= kFwdLdsLimit) ? 1 : 0;
        if (g.balance) sp.lds += (int64_t(d.cin) + 64) * 4;
    } else {
        sp.mode = want_gx ? 2 : 0;
        // channel groups only where the samples alone leave CUs idle
        const int slots = sp.threads / L;
        const int64_t groups = std::min<int64_t>(ceil_div(d.cout, slots),
                                                 std::max<int64_t>(1, ceil_div(256, d.n)));
        g.cg = int(ceil_div(d.cout, groups));
        g.x_words = int(xw);
        g.c_words = 0;
        g.ul_words = 0;
        g.balance = 0;
        sp.lds = xw * int64_t(tsize);
    }
    g.groups = int(ceil_div(d.cout, g.cg));
    g.per_xcd = ceil_div(int64_t(d.n) * g.groups, int64_t(8));
    if (8 * g.per_xcd >= (int64_t(1) << 31)) return false;
    // 32-bit item, moment-record and conv-gate-gradient indices
    const int64_t items = int64_t(d.n) * d.cout * d.P;
    if (items * 4 >= (int64_t(1) << 31) || int64_t(d.cout) * d.n * kMomStride >= (int64_t(1) << 31))
        return false;
    sp.grid = unsigned(8 * g.per_xcd);
    g.div_hw = make_fastdiv(uint32_t(d.h * d.w));
    g.div_w = make_fastdiv(uint32_t(d.w));
    g.div_h = make_fastdiv(uint32_t(d.h));
    g.div_rv = make_fastdiv(uint32_t(std::max(1, d.w / int(16 / tsize))));
    g.vec = 0;  // set by the caller, which sees the pointers
    return true;
}

template <typename T>
int64_t tree_workspace_bytes(const TreeDims& d, bool grad_x, int kh, int kw) {
    const int nodes = d.complete ? 7 : 4;
    StagePlan sp;
    if (plan_tree_stage(d, kh, kw, grad_x, sizeof(T), sp)) {
        // moment records [cout][n][32], coefficients [cout][7][4], conv-gate gradients
        int64_t b = int64_t(d.cout) * d.n * kMomStride * sizeof(T);
        b = (b + 255) / 256 * 256;
        b += int64_t(d.cout) * nodes * 4 * sizeof(T);
        if (sp.mode == 2) {
            b = (b + 255) / 256 * 256;
            b += int64_t(d.n) * d.cout * d.P * 4 * sizeof(T);
        }
        return b;
    }
    const int64_t nblk = node_blocks(d);
    int64_t b = 0;
    if (d.complete && grad_x) {
        b += tree_records(d) * int64_t(sizeof(T));
        b = (b + 255) / 256 * 256;
        b += tree_records(d) * 4;
    }
    b = (b + 255) / 256 * 256;
    b += int64_t(d.cout) * nblk * nodes * 4 * sizeof(T);  // partial moments
    b = (b + 255) / 256 * 256;
    b += int64_t(d.cout) * nodes * 4 * sizeof(T);  // collapsed coefficients
    return b;
}

}  // namespace
}  // namespace cl

using namespace cl;

namespace {
int tree_conv_forward_impl(int dtype, const void* x, const void* w_prob,
                           const int32_t* selection, int64_t n, int64_t c_in, int64_t h,
                           int64_t w, int64_t c_out, int stride_h, int stride_w, int pad_h,
                           int pad_w, int kernel_h, int kernel_w, int complete, void* y, void* x2,
                           void* x3, int32_t* indices, int softmax, int regular, int y_rows,
                           void* coefs, void* stream) {
    TreeDims d;
    if (int rc = tree_dims(d, n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w, kernel_h,
                           kernel_w, complete))
        return rc;
    CL_ARG(!y_rows || complete, "the feature-major output is for the complete block");
    CL_ARG(!coefs || complete, "the coefficient output is for the complete block");
    CL_ARG(!coefs || aligned(coefs, 16), "coefs must be 16-byte aligned");
    d.coefs = coefs;
    d.softmax = softmax ? 1 : 0;
    d.regular = regular ? 1 : 0;
    d.y_rows = y_rows ? 1 : 0;
    if (n == 0 || c_out == 0) return CL_OK;
    CL_ARG(x && w_prob && selection && y, "null pointer argument");
    const unsigned gx = unsigned(ceil_div(int64_t(d.n) * d.P, 256));
    const dim3 grid(gx, unsigned(d.cout));
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        TreeLds g;
        int groups = 0;
        int64_t lds = 0;
        if (plan_tree_lds<T>(d, kernel_h, kernel_w, complete ? 4 * d.P : d.P, 2, g, groups,
                             lds)) {
            const T* xs = static_cast<const T*>(x);
            const T* ws = static_cast<const T*>(w_prob);
            if (complete)
                return launch_tree_fwd_lds<T, true>(d, g, groups, lds, xs, ws, selection,
                                                    static_cast<T*>(y), static_cast<T*>(x2),
                                                    static_cast<T*>(x3), indices, s);
            return launch_tree_fwd_lds<T, false>(d, g, groups, lds, xs, ws, selection,
                                                 static_cast<T*>(y), nullptr, nullptr, nullptr,
                                                 s);
        }
        if (complete) {
            const unsigned gq = unsigned(ceil_div(int64_t(d.n) * d.P * 4, 256 * kFwdItems));
            k_tree_fwd_q<T><<<dim3(gq, unsigned(d.cout)), 256, 0, s>>>(
                static_cast<const T*>(x), static_cast<const T*>(w_prob), selection, d,
                static_cast<T*>(y), static_cast<T*>(x2), static_cast<T*>(x3), indices);
        }
        else
            k_tree_fwd<T><<<grid, 256, 0, s>>>(static_cast<const T*>(x),
                                               static_cast<const T*>(w_prob), selection, d,
                                               static_cast<T*>(y));
    });
    return check_launch("cl_tree_conv_forward");
}
}  // namespace

extern "C" int cl_tree_conv_forward(int dtype, const void* x, const void* w_prob,
                                    const int32_t* selection, int64_t n, int64_t c_in, int64_t h,
                                    int64_t w, int64_t c_out, int stride_h, int stride_w,
                                    int pad_h, int pad_w, int kernel_h, int kernel_w,
                                    int complete, void* y, void* x2, void* x3, int32_t* indices,
                                    void* stream) {
    clear_error();
    return tree_conv_forward_impl(dtype, x, w_prob, selection, n, c_in, h, w, c_out, stride_h,
                                  stride_w, pad_h, pad_w, kernel_h, kernel_w, complete, y, x2, x3,
                                  indices, 0, 0, 0, nullptr, stream);
}

extern "C" int cl_tree_conv_forward_softmax(int dtype, const void* x, const void* w_logits,
                                            const int32_t* selection, int64_t n, int64_t c_in,
                                            int64_t h, int64_t w, int64_t c_out, int stride_h,
                                            int stride_w, int pad_h, int pad_w, int kernel_h,
                                            int kernel_w, int complete, void* y, void* x2,
                                            void* x3, int32_t* indices, int regular_taps,
                                            int y_rows, void* stream) {
    clear_error();
    return tree_conv_forward_impl(dtype, x, w_logits, selection, n, c_in, h, w, c_out, stride_h,
                                  stride_w, pad_h, pad_w, kernel_h, kernel_w, complete, y, x2, x3,
                                  indices, 1, regular_taps, y_rows, nullptr, stream);
}

extern "C" int cl_tree_conv_forward_softmax_coefs(int dtype, const void* x, const void* w_logits,
                                                  const int32_t* selection, int64_t n,
                                                  int64_t c_in, int64_t h, int64_t w,
                                                  int64_t c_out, int stride_h, int stride_w,
                                                  int pad_h, int pad_w, int kernel_h,
                                                  int kernel_w, void* y, void* x2, void* x3,
                                                  int32_t* indices, int regular_taps, int y_rows,
                                                  void* coefs, void* stream) {
    clear_error();
    CL_ARG(coefs, "null pointer argument");
    return tree_conv_forward_impl(dtype, x, w_logits, selection, n, c_in, h, w, c_out, stride_h,
                                  stride_w, pad_h, pad_w, kernel_h, kernel_w, 1, y, x2, x3,
                                  indices, 1, regular_taps, y_rows, coefs, stream);
}

extern "C" int cl_tree_conv_workspace(int dtype, int64_t n, int64_t c_in, int64_t h, int64_t w,
                                      int64_t c_out, int stride_h, int stride_w, int pad_h,
                                      int pad_w, int kernel_h, int kernel_w, int complete,
                                      int grad_x, int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    TreeDims d;
    if (int rc = tree_dims(d, n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w, kernel_h,
                           kernel_w, complete))
        return rc;
    CL_DTYPE_SWITCH(dtype, {
        *bytes = tree_workspace_bytes<scalar_t>(d, grad_x != 0, kernel_h, kernel_w);
    });
    return CL_OK;
}

namespace {
template <typename T>
int tree_backward_staged(const TreeDims& d, const StagePlan& sp, const T* gy, const T* xs,
                         const T* wp, const int32_t* sel, const int32_t* idx,
                         const int32_t* ent_ptr, const int32_t* ent, T* grad_x, T* grad_w,
                         void* workspace, const T* coefs_in, hipStream_t s) {
    unsigned char* ws = static_cast<unsigned char*>(workspace);
    T* part = reinterpret_cast<T*>(ws);
    int64_t off = (int64_t(d.cout) * d.n * kMomStride * sizeof(T) + 255) / 256 * 256;
    T* kc = reinterpret_cast<T*>(ws + off);
    off += int64_t(d.cout) * kMaxNodes * 4 * sizeof(T);
    off = (off + 255) / 256 * 256;
    T* gconv = sp.mode == 2 ? reinterpret_cast<T*>(ws + off) : nullptr;
    TreeStage g = sp.g;
    g.vec = (d.w % (16 / int(sizeof(T))) == 0 && aligned(xs, 16) &&
             (!grad_x || aligned(grad_x, 16))) ? 1 : 0;
    if (coefs_in) {
        CL_ARG(aligned(coefs_in, 16), "coefs must be 16-byte aligned");
        kc = const_cast<T*>(coefs_in);  // read only
    } else {
        k_tree_coefs<T><<<unsigned(d.cout), 64, 0, s>>>(wp, sel, d, kc);
        if (int rc = check_launch("cl_tree_conv_backward(coefficients)")) return rc;
    }
    T* pw = grad_w ? part : nullptr;
    static bool reserved[3][2][kMaxDevices] = {};
    const int ti = sizeof(T) == 4 ? 0 : 1;
    auto go = [&](auto kern) -> int {
        if (int rc = reserve_lds(kern, sp.lds, reserved[sp.mode][ti], "the tree block backward"))
            return rc;
        kern<<<sp.grid, unsigned(sp.threads), size_t(sp.lds), s>>>(
            gy, xs, kc, sel, idx, ent_ptr, ent, d, g, pw, gconv, grad_x);
        return check_launch("cl_tree_conv_backward(staged)");
    };
    constexpr int NT = sizeof(T) == 4 ? CL_TREE_STAGED_NT1 : 512;
    int rc = sp.mode == 1 ? go(&k_tree_bwd_staged<T, 1, NT>)
             : sp.mode == 2 ? go(&k_tree_bwd_staged<T, 2, NT>)
                            : go(&k_tree_bwd_staged<T, 0, NT>);
    if (rc) return rc;
    if (grad_w) {
        k_tree_moments<T><<<unsigned(d.cout), 1024, 0, s>>>(part, d.n, d.softmax ? wp : nullptr,
                                                            grad_w);
        if (int rc2 = check_launch("cl_tree_conv_backward(moments)")) return rc2;
    }
    if (sp.mode == 2) {
        const int64_t row_bytes = int64_t(d.w) * int64_t(sizeof(T));
        CL_ARG(row_bytes <= kGatherLdsBytes,
               "input rows of more than %lld bytes are not supported by the input gradient",
               (long long)kGatherLdsBytes);
        const int band_rows = int(std::min<int64_t>(d.h, kGatherLdsBytes / row_bytes));
        const int nbands = int(ceil_div(d.h, band_rows));
        const int64_t hw_bytes = int64_t(band_rows) * row_bytes;
        const int pw_lanes = gather_lanes(d.P);
        int spw = std::max(1, 32 / pw_lanes);
        while (spw > 1 && int64_t(spw) * hw_bytes > kGatherLdsBytes) spw >>= 1;
        const int cg = int(std::max<int64_t>(1, std::min<int64_t>(
            std::min<int64_t>(d.cin, 4 * (64 / (pw_lanes * spw))),
            kGatherLdsBytes / (hw_bytes * spw))));
        CL_ARG(nbands < 65536, "input planes too tall for the input gradient");
        const dim3 g2(unsigned(ceil_div(d.n, spw)), unsigned(ceil_div(d.cin, cg)),
                      unsigned(nbands));
        const size_t lds = size_t(spw) * size_t(cg) * size_t(hw_bytes);
        k_tree_gather<T, true><<<g2, 256, lds, s>>>(gconv, xs, sel, idx, ent_ptr, ent, kc, d,
                                                    cg, pw_lanes, spw, band_rows, grad_x);
        if (int rc2 = check_launch("cl_tree_conv_backward(gather)")) return rc2;
    }
    return CL_OK;
}

int tree_conv_backward_impl(int dtype, const void* grad_y, const void* x, const void* w_prob,
                            const int32_t* selection, const int32_t* indices,
                            const int32_t* ent_ptr, const int32_t* ent, int64_t n, int64_t c_in,
                            int64_t h, int64_t w, int64_t c_out, int stride_h, int stride_w,
                            int pad_h, int pad_w, int kernel_h, int kernel_w, int complete,
                            void* grad_x, void* grad_w, void* workspace, int64_t workspace_bytes,
                            int softmax, int y_rows, const void* coefs, void* stream) {
    TreeDims d;
    if (int rc = tree_dims(d, n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w, kernel_h,
                           kernel_w, complete))
        return rc;
    CL_ARG(!y_rows || complete, "the feature-major gradient is for the complete block");
    d.softmax = softmax ? 1 : 0;
    d.y_rows = y_rows ? 1 : 0;
    if (!grad_x && !grad_w) return CL_OK;
    const int nodes = complete ? 7 : 4;
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        if (n == 0 || c_out == 0) {  // no items: zero gradients
            if (grad_x)
                if (int rc = zero_fill<T>(grad_x, n * c_in * h * w, s, "cl_tree_conv_backward"))
                    return rc;
            if (grad_w)
                if (int rc = zero_fill<T>(grad_w, c_out * nodes * 16, s, "cl_tree_conv_backward"))
                    return rc;
            return CL_OK;
        }
        CL_ARG(grad_y && x && w_prob && selection, "null pointer argument");
        CL_ARG(!complete || indices, "the complete block's backward needs the pooling indices");
        CL_ARG(!grad_x || (ent_ptr && ent), "the input gradient needs the channel use index");
        const int64_t need = tree_workspace_bytes<T>(d, grad_x != nullptr, kernel_h, kernel_w);
        CL_ARG(workspace && workspace_bytes >= need,
               "workspace of %lld bytes needed (see cl_tree_conv_workspace)", (long long)need);
        CL_ARG(aligned(workspace, 256), "workspace must be 256-byte aligned");
        StagePlan sp;
        if (plan_tree_stage(d, kernel_h, kernel_w, grad_x != nullptr, sizeof(T), sp))
            return tree_backward_staged<T>(d, sp, static_cast<const T*>(grad_y),
                                           static_cast<const T*>(x),
                                           static_cast<const T*>(w_prob), selection, indices,
                                           ent_ptr, ent, static_cast<T*>(grad_x),
                                           static_cast<T*>(grad_w), workspace,
                                           static_cast<const T*>(coefs), s);
        const int64_t nblk = node_blocks(d, &d.node_items);
        unsigned char* ws = static_cast<unsigned char*>(workspace);
        T* radd = nullptr;
        int32_t* rtgt = nullptr;
        int64_t off = 0;
        if (complete && grad_x) {
            radd = reinterpret_cast<T*>(ws);
            off = (tree_records(d) * int64_t(sizeof(T)) + 255) / 256 * 256;
            rtgt = reinterpret_cast<int32_t*>(ws + off);
            off += tree_records(d) * 4;
        }
        off = (off + 255) / 256 * 256;
        T* part = reinterpret_cast<T*>(ws + off);
        off += int64_t(d.cout) * nblk * nodes * 4 * sizeof(T);
        off = (off + 255) / 256 * 256;
        T* kc = reinterpret_cast<T*>(ws + off);
        const dim3 grid(unsigned(nblk), unsigned(d.cout));
        const T* gy = static_cast<const T*>(grad_y);
        const T* xs = static_cast<const T*>(x);
        const T* wp = static_cast<const T*>(w_prob);
        if (complete && radd)
            k_tree_nodes<T, true, true><<<grid, 256, 0, s>>>(gy, xs, wp, selection, indices, d,
                                                             radd, rtgt, part, kc);
        else if (complete)
            k_tree_nodes<T, true, false><<<grid, 256, 0, s>>>(gy, xs, wp, selection, indices, d,
                                                              nullptr, nullptr, part, kc);
        else
            k_tree_nodes<T, false, false><<<grid, 256, 0, s>>>(gy, xs, wp, selection, indices, d,
                                                               nullptr, nullptr, part, kc);
        if (int rc = check_launch("cl_tree_conv_backward(nodes)")) return rc;
        if (grad_w) {
            k_tree_finalize<T><<<unsigned(ceil_div(int64_t(d.cout) * nodes * 16, 256)), 256, 0, s>>>(
                part, d.cout, nodes, nblk, softmax ? wp : nullptr, static_cast<T*>(grad_w));
            if (int rc = check_launch("cl_tree_conv_backward(finalize)")) return rc;
        }
        if (grad_x) {
            const int64_t row_bytes = int64_t(d.w) * int64_t(sizeof(T));
            CL_ARG(row_bytes <= kGatherLdsBytes,
                   "input rows of more than %lld bytes are not supported by the input gradient",
                   (long long)kGatherLdsBytes);
            // planes beyond LDS: bands of rows, one workgroup per band
            const int band_rows = int(std::min<int64_t>(d.h, kGatherLdsBytes / row_bytes));
            const int nbands = int(ceil_div(d.h, band_rows));
            const int64_t hw_bytes = int64_t(band_rows) * row_bytes;
            // one pass of the workgroup's lane groups per channel group: more workgroups
            // (each staging only its channels) keep more waves in flight
            const int pw_lanes = gather_lanes(d.P);
            // small pooled planes: a lane group takes several samples of a channel, so the
            // loads of a use's taps and coefficients serve PW * spw lanes
            int spw = std::max(1, 32 / pw_lanes);
            while (spw > 1 && int64_t(spw) * hw_bytes > kGatherLdsBytes) spw >>= 1;
            const int cg = int(std::max<int64_t>(1, std::min<int64_t>(
                std::min<int64_t>(d.cin, 4 * (64 / (pw_lanes * spw))),
                kGatherLdsBytes / (hw_bytes * spw))));
            const dim3 g2(unsigned(ceil_div(d.n, spw)), unsigned(ceil_div(d.cin, cg)),
                          unsigned(nbands));
            CL_ARG(nbands < 65536, "input planes too tall for the input gradient");
            const size_t lds = size_t(spw) * size_t(cg) * size_t(hw_bytes);
            CL_ARG(!complete || tree_records(d) < (int64_t(1) << 32),
                   "too many tap contributions for the input gradient");
            if (complete)
                k_tree_gather_rec<T><<<g2, 256, lds, s>>>(radd, rtgt, ent_ptr, ent, d, cg,
                                                          pw_lanes, spw, band_rows,
                                                          static_cast<T*>(grad_x));
            else
                k_tree_gather<T, false><<<g2, 256, lds, s>>>(gy, xs, selection, indices, ent_ptr,
                                                             ent, kc, d, cg, pw_lanes, spw,
                                                             band_rows, static_cast<T*>(grad_x));
            if (int rc = check_launch("cl_tree_conv_backward(gather)")) return rc;
        }
    });
    return CL_OK;
}
}  // namespace

extern "C" int cl_tree_conv_backward(int dtype, const void* grad_y, const void* x,
                                     const void* w_prob, const int32_t* selection,
                                     const int32_t* indices, const int32_t* ent_ptr,
                                     const int32_t* ent, int64_t n, int64_t c_in, int64_t h,
                                     int64_t w, int64_t c_out, int stride_h, int stride_w,
                                     int pad_h, int pad_w, int kernel_h, int kernel_w,
                                     int complete, void* grad_x, void* grad_w, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    clear_error();
    return tree_conv_backward_impl(dtype, grad_y, x, w_prob, selection, indices, ent_ptr, ent, n,
                                   c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w, kernel_h,
                                   kernel_w, complete, grad_x, grad_w, workspace,
                                   workspace_bytes, 0, 0, nullptr, stream);
}

extern "C" int cl_tree_conv_backward_softmax(int dtype, const void* grad_y, const void* x,
                                             const void* w_logits, const int32_t* selection,
                                             const int32_t* indices, const int32_t* ent_ptr,
                                             const int32_t* ent, int64_t n, int64_t c_in,
                                             int64_t h, int64_t w, int64_t c_out, int stride_h,
                                             int stride_w, int pad_h, int pad_w, int kernel_h,
                                             int kernel_w, int complete, void* grad_x,
                                             void* grad_w, void* workspace,
                                             int64_t workspace_bytes, int y_rows,
                                             void* stream) {
    clear_error();
    return tree_conv_backward_impl(dtype, grad_y, x, w_logits, selection, indices, ent_ptr, ent,
                                   n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w,
                                   kernel_h, kernel_w, complete, grad_x, grad_w, workspace,
                                   workspace_bytes, 1, y_rows, nullptr, stream);
}

extern "C" int cl_tree_conv_backward_softmax_coefs(int dtype, const void* grad_y, const void* x,
                                                   const void* w_logits,
                                                   const int32_t* selection,
                                                   const int32_t* indices,
                                                   const int32_t* ent_ptr, const int32_t* ent,
                                                   int64_t n, int64_t c_in, int64_t h, int64_t w,
                                                   int64_t c_out, int stride_h, int stride_w,
                                                   int pad_h, int pad_w, int kernel_h,
                                                   int kernel_w, void* grad_x, void* grad_w,
                                                   void* workspace, int64_t workspace_bytes,
                                                   int y_rows, const void* coefs, void* stream) {
    clear_error();
    CL_ARG(coefs, "null pointer argument");
    return tree_conv_backward_impl(dtype, grad_y, x, w_logits, selection, indices, ent_ptr, ent,
                                   n, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w,
                                   kernel_h, kernel_w, 1, grad_x, grad_w, workspace,
                                   workspace_bytes, 1, y_rows, coefs, stream);
}

extern "C" int cl_tree_level_forward(int dtype, const void* x, const void* w_prob, int64_t n,
                                     int64_t channels, int64_t positions, int64_t out_bits,
                                     void* y, void* stream) {
    clear_error();
    CL_ARG(n >= 0 && channels >= 0 && positions >= 0, "negative shape");
    CL_ARG(out_bits >= 1 && out_bits <= 4, "Xout > 4 is not supported");
    const int64_t total = n * channels * positions * out_bits;
    if (total == 0) return CL_OK;
    CL_ARG(x && w_prob && y, "null pointer argument");
    CL_ARG(ceil_div(total, 256) < (int64_t(1) << 31), "tensor too large");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        k_level_fwd<T><<<unsigned(ceil_div(total, 256)), 256, 0, s>>>(
            static_cast<const T*>(x), static_cast<const T*>(w_prob), n, channels, positions,
            int(out_bits), static_cast<T*>(y));
    });
    return check_launch("cl_tree_level_forward");
}

extern "C" int cl_tree_level_workspace(int dtype, int64_t n, int64_t channels, int64_t positions,
                                       int64_t out_bits, int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    CL_ARG(n >= 0 && channels >= 0 && positions >= 0 && out_bits >= 1 && out_bits <= 4,
           "bad shape");
    const int64_t nblk = ceil_div(n * positions, 256);
    CL_DTYPE_SWITCH(dtype, { *bytes = channels * nblk * out_bits * 4 * int64_t(sizeof(scalar_t)); });
    return CL_OK;
}

extern "C" int cl_tree_level_backward(int dtype, const void* grad_y, const void* x,
                                      const void* w_prob, int64_t n, int64_t channels,
                                      int64_t positions, int64_t out_bits, void* grad_x,
                                      void* grad_w, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
    clear_error();
    CL_ARG(n >= 0 && channels >= 0 && positions >= 0, "negative shape");
    CL_ARG(out_bits >= 1 && out_bits <= 4, "Xout > 4 is not supported");
    if (!grad_x && !grad_w) return CL_OK;
    hipStream_t s = as_stream(stream);
    const int64_t items = n * positions;
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        if (items == 0 || channels == 0) {  // no items: zero weight gradient
            if (grad_w)
                return zero_fill<T>(grad_w, channels * out_bits * 16, s, "cl_tree_level_backward");
            return CL_OK;
        }
        CL_ARG(grad_y && x && w_prob, "null pointer argument");
        const int64_t nblk = ceil_div(items, 256);
        CL_ARG(nblk < (int64_t(1) << 31) && channels < 65536, "tensor too large");
        const int64_t need = channels * nblk * out_bits * 4 * int64_t(sizeof(T));
        CL_ARG(workspace && workspace_bytes >= need,
               "workspace of %lld bytes needed (see cl_tree_level_workspace)", (long long)need);
        T* part = static_cast<T*>(workspace);
        k_level_bwd<T><<<dim3(unsigned(nblk), unsigned(channels)), 256, 0, s>>>(
            static_cast<const T*>(grad_y), static_cast<const T*>(x), static_cast<const T*>(w_prob),
            n, channels, positions, int(out_bits), static_cast<T*>(grad_x), part);
        if (int rc = check_launch("cl_tree_level_backward")) return rc;
        if (grad_w) {
            k_tree_finalize<T><<<unsigned(ceil_div(channels * out_bits * 16, 256)), 256, 0, s>>>(
                part, channels, int(out_bits), nblk, nullptr, static_cast<T*>(grad_w));
        }
    });
    return check_launch("cl_tree_level_backward");
}

extern "C" int cl_tree_conv_eval_packed(const void* x, int64_t row_bytes, const uint8_t* gates,
                                        const int32_t* selection, int64_t c_in, int64_t h,
                                        int64_t w, int64_t c_out, int stride_h, int stride_w,
                                        int pad_h, int pad_w, int kernel_h, int kernel_w,
                                        int complete, void* y, void* stream) {
    clear_error();
    TreeDims d;
    if (int rc = tree_dims(d, 1, c_in, h, w, c_out, stride_h, stride_w, pad_h, pad_w, kernel_h,
                           kernel_w, complete))
        return rc;
    CL_ARG(row_bytes >= 0 && row_bytes % 8 == 0, "row_bytes must be a multiple of 8");
    const int64_t words = row_bytes / 8;
    const int64_t rows = int64_t(d.cout) * d.P * (complete ? 1 : 4);
    if (words == 0 || rows == 0) return CL_OK;
    CL_ARG(x && gates && selection && y, "null pointer argument");
    CL_ARG(aligned(x, 8) && aligned(y, 8), "packed rows must be 8-byte aligned");
    if (!complete) d.P *= 4;  // one output row per (position, gate)
    CL_ARG(words < (int64_t(1) << 28) && rows < (int64_t(1) << 31), "tensor too large");
    // Two words per lane when every lane's pair is whole and 16-byte aligned.
    const bool pairs = words % 2 == 0 && aligned(x, 16) && aligned(y, 16);
    const int64_t nchunks = ceil_div(words, kPkChunk);
    const int64_t rblocks = ceil_div(rows, pairs ? 16 : 8);
    const int64_t grid = nchunks >= 8 ? 8 * ceil_div(nchunks, 8) * rblocks : nchunks * rblocks;
    CL_ARG(grid < (int64_t(1) << 31), "tensor too large");
    const auto xs = static_cast<const uint64_t*>(x);
    const auto ys = static_cast<uint64_t*>(y);
    if (pairs)
        k_tree_packed<2><<<unsigned(grid), 256, 0, as_stream(stream)>>>(
            xs, words, gates, selection, d, nchunks, rblocks, ys);
    else
        k_tree_packed<1><<<unsigned(grid), 256, 0, as_stream(stream)>>>(
            xs, words, gates, selection, d, nchunks, rblocks, ys);
    return check_launch("cl_tree_conv_eval_packed");
}
