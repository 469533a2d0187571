// ConvLayer kernels for gfx950 (compactlogic/cuda/convlogic_kernel.cu semantics).
//
// Layout: x / grad_x [N, Cin, H, W] (unpadded), y / grad_y [N, Cout, Ho, Wo],
// offsets_ch (int32) / offsets_h / offsets_w (int8) [2, Cout, G] with the spatial offsets
// already shifted by -padding, w / gate_seq [Cout, G].  Tap (side, c, g) of output (oy, ox)
// reads x[n, ch, oy*stride + dh, ox*stride + dw], zero outside the input plane.
//
// forward / eval   one thread per output position, one output channel per workgroup row
//                  (grid.y), so the channel's slot metadata is wave-uniform (scalar loads).
// weight gradient  per-block partial sums over (n, position) for every slot, then a fixed-
//                  order sum over the blocks (deterministic, no atomics).
// input gradient   a deterministic gather: for stride s an input pixel (iy, ix) is reached by
//                  tap (side, c, g) only when iy = dh (mod s) and ix = dw (mod s), so the
//                  inverse index is bucketed by (input channel, dh mod s, dw mod s) and every
//                  entry a thread visits is phase-valid; only the range of oy, ox is checked.
#include "common.h"

#include <algorithm>

namespace cl {
namespace {

template <typename T>
__device__ __forceinline__ T cnan() {
    return T(__builtin_nan(""));
}

struct ConvDims {
    int64_t N, Cin, H, W, Cout, Ho, Wo;
    int G, stride;
};

template <typename T>
__device__ __forceinline__ T tap(const T* __restrict__ xn, const ConvDims& d, int ch, int yy,
                                 int xx) {
    return (yy >= 0 && yy < d.H && xx >= 0 && xx < d.W) ? xn[(int64_t(ch) * d.H + yy) * d.W + xx]
                                                          : T(0);
}

// ------------------------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_conv_fwd(const T* __restrict__ x,
                                                  const int32_t* __restrict__ och,
                                                  const int8_t* __restrict__ oh,
                                                  const int8_t* __restrict__ ow,
                                                  const T* __restrict__ w,
                                                  const uint8_t* __restrict__ gs,
                                                  T* __restrict__ y, ConvDims d) {
    const int64_t c = blockIdx.y;
    const int64_t hw = d.Ho * d.Wo;
    const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (e >= d.N * hw) return;
    const int64_t n = e / hw, p = e % hw;
    const int oy = int(p / d.Wo), ox = int(p % d.Wo);
    const T* xn = x + n * d.Cin * d.H * d.W;
    const int64_t G = d.G, side1 = d.Cout * G;
    T acc = 0;
    bool bad = false;
    for (int g = 0; g < d.G; ++g) {
        const int64_t s0 = c * G + g, s1 = side1 + s0;
        const int ch0 = och[s0], ch1 = och[s1];
        if (uint32_t(ch0) >= uint64_t(d.Cin) || uint32_t(ch1) >= uint64_t(d.Cin)) {
            bad = true;
            continue;
        }
        const T va = tap(xn, d, ch0, oy * d.stride + oh[s0], ox * d.stride + ow[s0]);
        const T vb = tap(xn, d, ch1, oy * d.stride + oh[s1], ox * d.stride + ow[s1]);
        acc = fma(w[s0], relaxed_op(gate_coef<T>(gs[s0]), va, vb), acc);
    }
    y[(n * d.Cout + c) * hw + p] = bad ? cnan<T>() : acc;
}

template <typename T>
__global__ __launch_bounds__(256) void k_conv_eval(const T* __restrict__ x,
                                                   const int32_t* __restrict__ och,
                                                   const int8_t* __restrict__ oh,
                                                   const int8_t* __restrict__ ow,
                                                   const uint8_t* __restrict__ wslot,
                                                   const uint8_t* __restrict__ gs,
                                                   T* __restrict__ y, ConvDims d) {
    const int64_t c = blockIdx.y;
    const int64_t hw = d.Ho * d.Wo;
    const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (e >= d.N * hw) return;
    const int64_t n = e / hw, p = e % hw;
    const int oy = int(p / d.Wo), ox = int(p % d.Wo);
    const int s = wslot[c];
    T out = cnan<T>();
    if (s < d.G) {
        const int64_t s0 = c * d.G + s, s1 = d.Cout * d.G + s0;
        const int ch0 = och[s0], ch1 = och[s1];
        if (uint32_t(ch0) < uint64_t(d.Cin) && uint32_t(ch1) < uint64_t(d.Cin)) {
            const T* xn = x + n * d.Cin * d.H * d.W;
            const T va = tap(xn, d, ch0, oy * d.stride + oh[s0], ox * d.stride + ow[s0]);
            const T vb = tap(xn, d, ch1, oy * d.stride + oh[s1], ox * d.stride + ow[s1]);
            out = relaxed_op(gate_coef<T>(gs[s0]), va, vb);
        }
    }
    y[(n * d.Cout + c) * hw + p] = out;
}

// ------------------------------------------------------------------------------------------
// Weight gradient, stage 1: block (b, c) sums gy * op_g(a, b) over its share of the (n, p)
// elements of channel c, for slots [g0, g0 + kSlots).
constexpr int kSlots = 16;

template <typename T>
__global__ __launch_bounds__(256) void k_conv_wgrad_partial(
    const T* __restrict__ x, const int32_t* __restrict__ och, const int8_t* __restrict__ oh,
    const int8_t* __restrict__ ow, const uint8_t* __restrict__ gs, const T* __restrict__ gy,
    T* __restrict__ part, int64_t per_block, ConvDims d) {
    __shared__ T red[4][kSlots];
    const int64_t b = blockIdx.x, c = blockIdx.y;
    const int g0 = blockIdx.z * kSlots;
    const int ns = std::min(kSlots, d.G - g0);
    const int64_t hw = d.Ho * d.Wo, total = d.N * hw;
    const int64_t e_begin = b * per_block, e_end = std::min(total, e_begin + per_block);
    const int64_t G = d.G, side1 = d.Cout * G;
    T acc[kSlots];
#pragma unroll
    for (int q = 0; q < kSlots; ++q) acc[q] = 0;
    for (int64_t e = e_begin + threadIdx.x; e < e_end; e += 256) {
        const int64_t n = e / hw, p = e % hw;
        const int oy = int(p / d.Wo), ox = int(p % d.Wo);
        const T* xn = x + n * d.Cin * d.H * d.W;
        const T gv = gy[(n * d.Cout + c) * hw + p];
#pragma unroll
        for (int q = 0; q < kSlots; ++q) {
            if (q < ns) {
                const int64_t s0 = c * G + g0 + q, s1 = side1 + s0;
                const int ch0 = och[s0], ch1 = och[s1];
                if (uint32_t(ch0) < uint64_t(d.Cin) && uint32_t(ch1) < uint64_t(d.Cin)) {
                    const T va = tap(xn, d, ch0, oy * d.stride + oh[s0], ox * d.stride + ow[s0]);
                    const T vb = tap(xn, d, ch1, oy * d.stride + oh[s1], ox * d.stride + ow[s1]);
                    acc[q] = fma(gv, relaxed_op(gate_coef<T>(gs[s0]), va, vb), acc[q]);
                } else {
                    acc[q] = cnan<T>();
                }
            }
        }
    }
    const int wv = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < kSlots; ++q) {
        const T t = wave_total(acc[q]);
        if ((threadIdx.x & 63) == 0) red[wv][q] = t;
    }
    __syncthreads();
    if (threadIdx.x < ns) {
        const int q = threadIdx.x;
        const T t = (red[0][q] + red[1][q]) + (red[2][q] + red[3][q]);
        part[(b * d.Cout + c) * G + g0 + q] = t;
    }
}

// Stage 2: grad_w[c, g] = sum over blocks in block order; with probs, the softmax backward.
template <typename T>
__global__ __launch_bounds__(256) void k_conv_wgrad_finish(const T* __restrict__ part,
                                                           int64_t nblocks,
                                                           const T* __restrict__ probs,
                                                           T* __restrict__ grad_w, int64_t Cout,
                                                           int G) {
    const int64_t c = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (c >= Cout) return;  // uniform per wave
    const int l = threadIdx.x & 63;
    for (int g0 = 0; g0 < G; g0 += 64) {
        const int g = g0 + l;
        T s = 0;
        if (g < G)
            for (int64_t b = 0; b < nblocks; ++b) s += part[(b * Cout + c) * G + g];
        if (probs) {
            // softmax backward needs the whole row: G <= 64 keeps it in one wave pass
            const T p = g < G ? probs[c * G + g] : T(0);
            const T dot = wave_total(p * s);
            s = p * (s - dot);
        }
        if (g < G) grad_w[c * G + g] = s;
    }
}

// ------------------------------------------------------------------------------------------
// Input gradient.  Workgroup (n, bucket k = ch * s^2 + py * s + px, pixel chunk): thread ->
// pixel (iy, ix) = (py + s*i, px + s*j) of that phase.  Entries of the bucket encode
// 2 * (c * G + g) + side.
template <typename T>
__global__ __launch_bounds__(64) void k_conv_bwd_x(
    const T* __restrict__ x, const int32_t* __restrict__ och, const int8_t* __restrict__ oh,
    const int8_t* __restrict__ ow, const T* __restrict__ w, const uint8_t* __restrict__ gs,
    const T* __restrict__ gy, const int32_t* __restrict__ inv_ptr,
    const int32_t* __restrict__ inv_ent, T* __restrict__ gx, int64_t chunks, ConvDims d) {
    const int s = d.stride;
    const int64_t nb = d.Cin * s * s;
    const int64_t blk = blockIdx.x;
    const int64_t chunk = blk % chunks;
    const int64_t k = (blk / chunks) % nb;
    const int64_t n = blk / (chunks * nb);
    if (n >= d.N) return;
    const int ch = int(k / (s * s)), py = int((k / s) % s), px = int(k % s);
    const int ph = int((d.H - py + s - 1) / s), pw = int((d.W - px + s - 1) / s);
    const int64_t li = chunk * 64 + threadIdx.x;
    if (li >= int64_t(ph) * pw) return;
    const int iy = py + s * int(li / pw), ix = px + s * int(li % pw);
    const T* xn = x + n * d.Cin * d.H * d.W;
    const T* gyn = gy + n * d.Cout * d.Ho * d.Wo;
    const int64_t G = d.G, side1 = d.Cout * G, hw = d.Ho * d.Wo;
    T acc = 0;
    bool bad = false;
    const int64_t e0 = inv_ptr[k], e1 = inv_ptr[k + 1];
    for (int64_t e = e0; e < e1; ++e) {
        const int ent = inv_ent[e];
        const int side = ent & 1;
        const int64_t sl = ent >> 1;  // c * G + g
        if (ent < 0 || sl >= side1) {
            bad = true;
            continue;
        }
        const int64_t c = sl / G;
        const int64_t self = side ? side1 + sl : sl, oth = side ? sl : side1 + sl;
        const int dy = int(iy) - oh[self], dx = int(ix) - ow[self];
        // dy, dx are multiples of s for every entry of this bucket
        const int oy = dy / s, ox = dx / s;
        if (dy < 0 || dx < 0 || oy >= d.Ho || ox >= d.Wo) continue;
        const int cho = och[oth];
        if (uint32_t(cho) >= uint64_t(d.Cin)) {
            bad = true;
            continue;
        }
        const T vo = tap(xn, d, cho, oy * s + oh[oth], ox * s + ow[oth]);
        const Coef4<T> cf = gate_coef<T>(gs[sl]);
        const T kself = side ? cf.c2 : cf.c1;
        const T dydx = w[sl] * fma(cf.c3, vo, kself);
        acc = fma(dydx, gyn[c * hw + int64_t(oy) * d.Wo + ox], acc);
    }
    gx[((n * d.Cin + ch) * d.H + iy) * d.W + ix] = bad ? cnan<T>() : acc;
}

// ------------------------------------------------------------------------------------------
// Packed layer from resolved index tables: y[o, :] = op_{g[o]}(x[ia[o], :], x[ib[o], :]);
// a negative index reads an all-zero row (a tap outside the input plane).  One wave per output
// row and chunk of 64 * U elements of type V (16-byte vectors when the rows allow it); lanes
// take consecutive elements, so every access is coalesced.
template <typename V, int U>
__global__ __launch_bounds__(256) void k_eval_packed_idx(const V* __restrict__ x,
                                                         const int32_t* __restrict__ ia,
                                                         const int32_t* __restrict__ ib,
                                                         const uint8_t* __restrict__ gate,
                                                         const int32_t* __restrict__ order,
                                                         V* __restrict__ y, int64_t in_dim,
                                                         int64_t out_dim, int64_t elems,
                                                         int64_t nblk) {
    // Workgroup (bx, chunk) takes row block (bx % 8) * nblk + bx / 8 of the processing order:
    // with gridDim.x a multiple of 8 it runs on XCD bx % 8, so each XCD walks one contiguous
    // stretch of the order, and rows that read the same input row (adjacent in the order)
    // find its words in that XCD's L2.
    const int64_t bx = blockIdx.x, chunk = blockIdx.y;
    const int64_t i = ((bx % 8) * nblk + bx / 8) * 4 + wave_id();
    if (i >= out_dim) return;
    const int64_t o = order ? int64_t(order[i]) : i;
    if (uint64_t(o) >= uint64_t(out_dim)) return;  // corrupt order entry: nothing is written
    const int64_t a = ia[o], b = ib[o];
    const int g = gate[o] & 15;
    const bool bad = a >= in_dim || b >= in_dim;
    const V zero = V(0);
    const V m00 = zero - V((g >> 3) & 1);
    const V m01 = zero - V((g >> 2) & 1);
    const V m10 = zero - V((g >> 1) & 1);
    const V m11 = zero - V(g & 1);
    // every load unconditional (row 0 for a negative or bad index, element 0 past the row's
    // end, masked afterwards), so the U loads of a lane are in flight together
    const V ka = (!bad && a >= 0) ? ~zero : zero;
    const V kb = (!bad && b >= 0) ? ~zero : zero;
    const int64_t ra = (!bad && a >= 0) ? a : 0, rb = (!bad && b >= 0) ? b : 0;
    const int64_t e0 = chunk * (64 * U) + lane_id();
    V va[U], vb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t e = e0 + int64_t(u) * 64;
        const int64_t off = e < elems ? e : 0;
        va[u] = x[ra * elems + off];
        vb[u] = x[rb * elems + off];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t e = e0 + int64_t(u) * 64;
        const V p = va[u] & ka, q = vb[u] & kb;
        V r = (~p & ~q & m00) | (~p & q & m01) | (p & ~q & m10) | (p & q & m11);
        if (bad) r = zero;
        // written once, read by the next layer only: bypass the caches
        if (e < elems) __builtin_nontemporal_store(r, y + o * elems + e);
    }
}

template <typename V>
int launch_eval_packed_idx(const void* x, const int32_t* ia, const int32_t* ib,
                           const uint8_t* gate, const int32_t* order, void* y, int64_t in_dim,
                           int64_t out_dim, int64_t row_bytes, hipStream_t s) {
    constexpr int U = 4;
    const int64_t elems = row_bytes / int64_t(sizeof(V));
    const int64_t nblk = ceil_div(ceil_div(out_dim, 4), 8);
    const int64_t nchunks = ceil_div(elems, 64 * U);
    CL_ARG(8 * nblk < (int64_t(1) << 31) && nchunks < 65536, "packed layer too large for one launch");
    const dim3 grid(unsigned(8 * nblk), unsigned(nchunks), 1);
    k_eval_packed_idx<V, U><<<grid, 256, 0, s>>>(static_cast<const V*>(x), ia, ib, gate, order,
                                                 static_cast<V*>(y), in_dim, out_dim, elems,
                                                 nblk);
    return CL_OK;
}

// Shapes given by the output plane (the backward passes take it from grad_y).
int conv_dims_out(ConvDims& d, int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                  int64_t G, int64_t stride, int64_t Ho, int64_t Wo) {
    CL_ARG(N >= 0 && Cin >= 1 && H >= 1 && W >= 1 && Cout >= 0, "bad input shape");
    CL_ARG(G >= 1 && G <= 128, "num_gates must be in [1, 128]");
    CL_ARG(stride >= 1, "bad stride");
    CL_ARG(Ho > 0 && Wo > 0, "Invalid output shape: h_out=%lld, w_out=%lld", (long long)Ho,
           (long long)Wo);
    CL_ARG(Cout < 65536, "c_out must be below 65536");
    CL_ARG(Cin * H * W < (int64_t(1) << 31) && Ho * Wo < (int64_t(1) << 31),
           "feature map too large for 32-bit pixel indices");
    d = ConvDims{N, Cin, H, W, Cout, Ho, Wo, int(G), int(stride)};
    return CL_OK;
}

// Shapes given by padding and kernel size (the forward passes).
int conv_dims(ConvDims& d, int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t G,
              int64_t stride, int64_t pad, int64_t ks) {
    CL_ARG(stride >= 1 && pad >= 0 && ks >= 1, "bad stride / padding / kernel size");
    CL_ARG(H + 2 * pad - ks >= 0 && W + 2 * pad - ks >= 0,
           "Invalid output shape: kernel size %lld exceeds the padded input", (long long)ks);
    const int64_t Ho = (H + 2 * pad - ks) / stride + 1, Wo = (W + 2 * pad - ks) / stride + 1;
    return conv_dims_out(d, N, Cin, H, W, Cout, G, stride, Ho, Wo);
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_conv_forward(int dtype, const void* x, const int32_t* offsets_ch,
                               const int8_t* offsets_h, const int8_t* offsets_w, const void* w,
                               const uint8_t* gate_seq, void* y, int64_t N, int64_t Cin,
                               int64_t H, int64_t W, int64_t Cout, int64_t num_gates,
                               int64_t stride, int64_t pad, int64_t ks, void* stream) {
    clear_error();
    ConvDims d;
    if (int rc = conv_dims(d, N, Cin, H, W, Cout, num_gates, stride, pad, ks)) return rc;
    if (N == 0 || Cout == 0) return CL_OK;
    CL_ARG(x && offsets_ch && offsets_h && offsets_w && w && gate_seq && y, "null pointer argument");
    const dim3 grid(unsigned(ceil_div(N * d.Ho * d.Wo, 256)), unsigned(Cout), 1);
    CL_DTYPE_SWITCH(dtype, {
        k_conv_fwd<scalar_t><<<grid, 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(x), offsets_ch, offsets_h, offsets_w,
            static_cast<const scalar_t*>(w), gate_seq, static_cast<scalar_t*>(y), d);
    });
    return check_launch("cl_conv_forward");
}

extern "C" int cl_conv_eval(int dtype, const void* x, const int32_t* offsets_ch,
                            const int8_t* offsets_h, const int8_t* offsets_w,
                            const uint8_t* w_slot, const uint8_t* gate_seq, void* y, int64_t N,
                            int64_t Cin, int64_t H, int64_t W, int64_t Cout, int64_t num_gates,
                            int64_t stride, int64_t pad, int64_t ks, void* stream) {
    clear_error();
    ConvDims d;
    if (int rc = conv_dims(d, N, Cin, H, W, Cout, num_gates, stride, pad, ks)) return rc;
    if (N == 0 || Cout == 0) return CL_OK;
    CL_ARG(x && offsets_ch && offsets_h && offsets_w && w_slot && gate_seq && y,
           "null pointer argument");
    const dim3 grid(unsigned(ceil_div(N * d.Ho * d.Wo, 256)), unsigned(Cout), 1);
    CL_DTYPE_SWITCH(dtype, {
        k_conv_eval<scalar_t><<<grid, 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(x), offsets_ch, offsets_h, offsets_w, w_slot, gate_seq,
            static_cast<scalar_t*>(y), d);
    });
    return check_launch("cl_conv_eval");
}

namespace {
int64_t wgrad_blocks(int64_t N, int64_t hw, int64_t Cout) {
    const int64_t total = N * hw;
    const int64_t want = std::max<int64_t>(1, 2048 / std::max<int64_t>(Cout, 1));
    return std::max<int64_t>(1, std::min<int64_t>(want, ceil_div(total, 1024)));
}
}  // namespace

extern "C" int cl_conv_backward_w_workspace(int dtype, int64_t N, int64_t Cin, int64_t H,
                                            int64_t W, int64_t Cout, int64_t num_gates,
                                            int64_t stride, int64_t h_out, int64_t w_out,
                                            int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    ConvDims d;
    if (int rc = conv_dims_out(d, N, Cin, H, W, Cout, num_gates, stride, h_out, w_out)) return rc;
    const int64_t nb = wgrad_blocks(N, d.Ho * d.Wo, Cout);
    *bytes = nb * Cout * num_gates * (dtype == CL_DTYPE_F64 ? 8 : 4);
    return CL_OK;
}

extern "C" int cl_conv_backward_w(int dtype, const void* x, const int32_t* offsets_ch,
                                  const int8_t* offsets_h, const int8_t* offsets_w,
                                  const uint8_t* gate_seq, const void* grad_y, const void* probs,
                                  void* grad_w, void* workspace, int64_t workspace_bytes,
                                  int64_t N, int64_t Cin, int64_t H, int64_t W, int64_t Cout,
                                  int64_t num_gates, int64_t stride, int64_t h_out,
                                  int64_t w_out, void* stream) {
    clear_error();
    ConvDims d;
    if (int rc = conv_dims_out(d, N, Cin, H, W, Cout, num_gates, stride, h_out, w_out)) return rc;
    if (Cout == 0) return CL_OK;
    CL_ARG(offsets_ch && offsets_h && offsets_w && gate_seq && grad_w, "null pointer argument");
    CL_ARG(N == 0 || (x && grad_y), "null pointer argument");
    CL_ARG(!probs || num_gates <= 64, "the fused softmax backward supports num_gates <= 64");
    const int64_t hw = d.Ho * d.Wo;
    const int64_t nb = wgrad_blocks(N, hw, Cout);
    const int64_t need = nb * Cout * num_gates * (dtype == CL_DTYPE_F64 ? 8 : 4);
    CL_ARG(workspace && workspace_bytes >= need, "workspace of %lld bytes required",
           (long long)need);
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const int64_t per_block = ceil_div(std::max<int64_t>(N * hw, 1), nb);
        const dim3 grid(unsigned(nb), unsigned(Cout), unsigned(ceil_div(num_gates, kSlots)));
        k_conv_wgrad_partial<T><<<grid, 256, 0, s>>>(
            static_cast<const T*>(x), offsets_ch, offsets_h, offsets_w, gate_seq,
            static_cast<const T*>(grad_y), static_cast<T*>(workspace), per_block, d);
        if (int rc = check_launch("cl_conv_backward_w(partial)")) return rc;
        k_conv_wgrad_finish<T><<<unsigned(ceil_div(Cout, 4)), 256, 0, s>>>(
            static_cast<const T*>(workspace), nb, static_cast<const T*>(probs),
            static_cast<T*>(grad_w), Cout, int(num_gates));
    });
    return check_launch("cl_conv_backward_w");
}

extern "C" int cl_conv_backward_x(int dtype, const void* x, const int32_t* offsets_ch,
                                  const int8_t* offsets_h, const int8_t* offsets_w, const void* w,
                                  const uint8_t* gate_seq, const void* grad_y,
                                  const int32_t* inv_ptr, const int32_t* inv_ent,
                                  void* grad_x, int64_t N, int64_t Cin, int64_t H, int64_t W,
                                  int64_t Cout, int64_t num_gates, int64_t stride, int64_t h_out,
                                  int64_t w_out, void* stream) {
    clear_error();
    ConvDims d;
    if (int rc = conv_dims_out(d, N, Cin, H, W, Cout, num_gates, stride, h_out, w_out)) return rc;
    if (N == 0) return CL_OK;
    CL_ARG(x && offsets_ch && offsets_h && offsets_w && w && gate_seq && grad_y && inv_ptr &&
               grad_x,
           "null pointer argument");
    const int64_t nbk = Cin * stride * stride;
    const int64_t pix = ceil_div(H, stride) * ceil_div(W, stride);
    const int64_t chunks = ceil_div(pix, 64);
    const int64_t blocks = N * nbk * chunks;
    CL_ARG(blocks < (int64_t(1) << 32), "conv input gradient too large for one launch");
    CL_DTYPE_SWITCH(dtype, {
        k_conv_bwd_x<scalar_t><<<unsigned(blocks), 64, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(x), offsets_ch, offsets_h, offsets_w,
            static_cast<const scalar_t*>(w), gate_seq, static_cast<const scalar_t*>(grad_y),
            inv_ptr, inv_ent, static_cast<scalar_t*>(grad_x), chunks, d);
    });
    return check_launch("cl_conv_backward_x");
}

extern "C" int cl_eval_packed_indexed(const void* x, const int32_t* ia, const int32_t* ib,
                                      const uint8_t* gate, const int32_t* order, void* y,
                                      int64_t in_dim, int64_t out_dim, int64_t row_bytes,
                                      void* stream) {
    clear_error();
    CL_ARG(in_dim >= 0 && out_dim >= 0 && row_bytes >= 0, "negative shape");
    if (out_dim == 0 || row_bytes == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && ia && ib && gate && y, "null pointer argument");
    CL_ARG(ceil_div(out_dim, 4) < (int64_t(1) << 31), "too many rows");
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    hipStream_t s = as_stream(stream);
    int rc;
    if (row_bytes % 16 == 0 && aligned(x, 16) && aligned(y, 16))
        rc = launch_eval_packed_idx<U4>(x, ia, ib, gate, order, y, in_dim, out_dim, row_bytes, s);
    else if (row_bytes % 8 == 0 && aligned(x, 8) && aligned(y, 8))
        rc = launch_eval_packed_idx<uint64_t>(x, ia, ib, gate, order, y, in_dim, out_dim, row_bytes, s);
    else if (row_bytes % 4 == 0 && aligned(x, 4) && aligned(y, 4))
        rc = launch_eval_packed_idx<uint32_t>(x, ia, ib, gate, order, y, in_dim, out_dim, row_bytes, s);
    else
        rc = launch_eval_packed_idx<uint8_t>(x, ia, ib, gate, order, y, in_dim, out_dim, row_bytes, s);
    if (rc) return rc;
    return check_launch("cl_eval_packed_indexed");
}
