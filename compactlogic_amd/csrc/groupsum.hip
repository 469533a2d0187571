// GroupSum forward / backward (compactlogic/compactlogic.py:450-468) for gfx950.
//
// The reference zero-pads the features to a multiple of k and sums k groups of
// gs = ceil(F / k) consecutive features, then divides by tau.  Padding columns contribute
// zero, so group c is simply features [c*gs, min((c+1)*gs, F)).
//
// A LogicLayer hands GroupSum a transposed view of its contiguous [F, batch] output, so the
// kernels take element strides and have a fast variant for each unit-stride direction:
//   batch-contiguous  (stride_batch == 1): lanes run along the batch, waves split the group
//   feature-contiguous (stride_feature == 1): one wave reduces one contiguous group
// and a plain strided variant for anything else.
#include "common.h"

#include <algorithm>

namespace cl {
namespace {

constexpr int kSplitWaves = 8;  // waves splitting one group in the batch-contiguous kernel

// ---- forward, batch-contiguous: block = (batch tile of 64*VEC samples, class c)
template <typename T, int VEC>
__global__ __launch_bounds__(kSplitWaves * 64) void k_gsum_fwd_bc(const T* __restrict__ x,
                                                                  int64_t B, int64_t F,
                                                                  int64_t sf, int64_t gsz,
                                                                  int64_t k, T tau,
                                                                  T* __restrict__ out) {
    __shared__ T part[kSplitWaves][64 * VEC];
    const int wv = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t c = blockIdx.y;
    const int64_t n0 = int64_t(blockIdx.x) * 64 * VEC + int64_t(lane) * VEC;
    const int64_t j0 = c * gsz;
    const int64_t j1 = std::min<int64_t>(j0 + gsz, F);
    Vec<T, VEC> s;
#pragma unroll
    for (int i = 0; i < VEC; ++i) s.v[i] = T(0);
    if (n0 < B) {
        for (int64_t j = j0 + wv; j < j1; j += kSplitWaves) {
            const Vec<T, VEC> v = vload<T, VEC>(x + j * sf + n0);
#pragma unroll
            for (int i = 0; i < VEC; ++i) s.v[i] += v.v[i];
        }
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) part[wv][lane * VEC + i] = s.v[i];
    __syncthreads();
    // Fixed-order combine of the wave partials (deterministic).
    for (int e = threadIdx.x; e < 64 * VEC; e += kSplitWaves * 64) {
        const int64_t n = int64_t(blockIdx.x) * 64 * VEC + e;
        if (n < B) {
            T t = part[0][e];
#pragma unroll
            for (int w = 1; w < kSplitWaves; ++w) t += part[w][e];
            out[n * k + c] = t / tau;
        }
    }
}

// ---- forward, batch-contiguous, split: block = (batch tile, class c, slice s of the
// group).  Each block writes the partial sum of its slice; k_gsum_finish adds the slices in
// slice order.  Used when a workspace is given, so that enough blocks fill the GPU.
constexpr int kPartWaves = 4;

template <typename T, int VEC>
__global__ __launch_bounds__(kPartWaves * 64) void k_gsum_partial(const T* __restrict__ x,
                                                                 int64_t B, int64_t F,
                                                                 int64_t sf, int64_t gsz,
                                                                 int64_t k, int64_t slice,
                                                                 T* __restrict__ part) {
    __shared__ T red[kPartWaves][64 * VEC];
    const int wv = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t c = blockIdx.y, sidx = blockIdx.z;
    const int64_t n0 = int64_t(blockIdx.x) * 64 * VEC + int64_t(lane) * VEC;
    const int64_t g_end = std::min<int64_t>((c + 1) * gsz, F);
    const int64_t j0 = c * gsz + sidx * slice;
    const int64_t j1 = std::min<int64_t>(j0 + slice, g_end);
    Vec<T, VEC> acc;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc.v[i] = T(0);
    if (n0 < B) {
        // the wave's rows eight at a time: the loads are issued together, the additions stay
        // in row order
        int64_t j = j0 + wv;
        for (; j + 7 * kPartWaves < j1; j += 8 * kPartWaves) {
            Vec<T, VEC> v[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) v[r] = vload<T, VEC>(x + (j + r * kPartWaves) * sf + n0);
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int i = 0; i < VEC; ++i) acc.v[i] += v[r].v[i];
        }
        for (; j < j1; j += kPartWaves) {
            const Vec<T, VEC> v = vload<T, VEC>(x + j * sf + n0);
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc.v[i] += v.v[i];
        }
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) red[wv][lane * VEC + i] = acc.v[i];
    __syncthreads();
    T* dst = part + (sidx * k + c) * B;
    for (int e = threadIdx.x; e < 64 * VEC; e += kPartWaves * 64) {
        const int64_t n = int64_t(blockIdx.x) * 64 * VEC + e;
        if (n < B) {
            T t = red[0][e];
#pragma unroll
            for (int w = 1; w < kPartWaves; ++w) t += red[w][e];
            dst[n] = t;
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_gsum_finish(const T* __restrict__ part, int64_t B,
                                                     int64_t k, int64_t nslices, T tau,
                                                     T* __restrict__ out) {
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;  // c * B + n
    if (item >= B * k) return;
    const int64_t c = item / B, n = item % B;
    const T* src = part + c * B + n;
    const int64_t step = k * B;
    // Loads are issued eight slices at a time; the additions stay in slice order.
    T t = 0;
    int64_t s = 0;
    for (; s + 8 <= nslices; s += 8) {
        T v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = src[(s + i) * step];
#pragma unroll
        for (int i = 0; i < 8; ++i) t += v[i];
    }
    for (; s < nslices; ++s) t += src[s * step];
    out[n * k + c] = t / tau;
}

// Slices per group for the split forward (1 = no split): about 256 (class, slice) workgroups
// per batch tile, at least 16 rows each.  More slices spread the partial sums over more
// workgroups but lengthen the per-sample slice sums that follow (k_ce_rows, k_gsum_finish);
// measured on the training lines, 256 per tile beat 1024 per batch at batch 256 (0.3531 ->
// 0.3503 ms for cfg3, 0.2846 -> 0.2811 ms for cfg3_tree) and equal it at batch 1024.
inline int64_t gsum_slices(int64_t B, int64_t F, int64_t k, int vec) {
    (void)B;
    (void)vec;
    const int64_t gsz = F == 0 ? 1 : ceil_div(F, k);
    const int64_t want = ceil_div(256, k);
    return std::max<int64_t>(1, std::min<int64_t>(want, ceil_div(gsz, 16)));
}

// ---- forward, feature-contiguous: one wave per (sample n, class c)
template <typename T>
__global__ __launch_bounds__(256) void k_gsum_fwd_fc(const T* __restrict__ x, int64_t B,
                                                     int64_t F, int64_t sb, int64_t gsz,
                                                     int64_t k, T tau, T* __restrict__ out) {
    const int64_t item = int64_t(blockIdx.x) * 4 + wave_id();
    if (item >= B * k) return;
    const int64_t n = item / k, c = item % k;
    const int64_t j0 = c * gsz;
    const int64_t j1 = std::min<int64_t>(j0 + gsz, F);
    const T* row = x + n * sb;
    T s = 0;
    for (int64_t j = j0 + lane_id(); j < j1; j += 64) s += row[j];
    s = wave_sum(s);
    if (lane_id() == 0) out[n * k + c] = s / tau;
}

// ---- forward, arbitrary strides: one thread per (n, c)
template <typename T>
__global__ __launch_bounds__(256) void k_gsum_fwd_generic(const T* __restrict__ x, int64_t B,
                                                          int64_t F, int64_t sb, int64_t sf,
                                                          int64_t gsz, int64_t k, T tau,
                                                          T* __restrict__ out) {
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (item >= B * k) return;
    const int64_t n = item / k, c = item % k;
    const int64_t j0 = c * gsz;
    const int64_t j1 = std::min<int64_t>(j0 + gsz, F);
    T s = 0;
    for (int64_t j = j0; j < j1; ++j) s += x[n * sb + j * sf];
    out[n * k + c] = s / tau;
}

template <typename T>
__device__ __forceinline__ T nan_of() {
    return T(__builtin_nan(""));
}

// ---- gradient of the class scores, as the backward kernels read it: src(n, c) is
// d loss / d out[n, c] divided by tau (the gradient each feature of group c receives).
template <typename T>
struct ScoreGrad {  // a given gradient g [B, k]
    const T* g;
    int64_t k;
    T tau;
    __device__ __forceinline__ T operator()(int64_t n, int64_t c) const { return g[n * k + c] / tau; }
};

// Mean cross-entropy of the scores: g[n, c] = gl * (p[n, c] - [c == y_n]) / count for a
// counted sample, 0 for an ignored one (y_n == ignore_index), NaN for a label outside [0, k).
// gl (the loss's upstream gradient) and count live in device memory.
template <typename T>
struct CrossEntropyGrad {
    const T* p;
    const int64_t* y;
    int64_t ignore;
    const T* gl;
    const T* count;
    int64_t k;
    T tau;
    __device__ __forceinline__ T operator()(int64_t n, int64_t c) const {
        // every load first (one round trip), then the selection
        const int64_t lab = y[n];
        const T pn = p[n * k + c], g = gl[0], cnt = count[0];
        if (lab == ignore) return T(0);
        if (lab < 0 || lab >= k) return nan_of<T>();
        const T d = pn - (lab == c ? T(1) : T(0));
        return d * (g / (cnt * tau));
    }
};

// ---- backward: grad_x[n, j] = src(n, j / gsz).  Elements are visited in memory order
// of grad_x: `inner` is the unit-stride dimension (batch or feature).
template <typename T, int VEC, bool BATCH_INNER, typename Src>
__global__ __launch_bounds__(256) void k_gsum_bwd(Src src, int64_t B, int64_t F, int64_t so,
                                                  int64_t gsz, T* __restrict__ gx) {
    // Rows: features (BATCH_INNER) or samples; inner: samples or features.
    const int64_t rows = BATCH_INNER ? F : B;
    const int64_t inner = BATCH_INNER ? B : F;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave_id();
    if (row >= rows) return;
    const int64_t i0 = (int64_t(blockIdx.y) * 64 + lane_id()) * VEC;
    if (i0 >= inner) return;
    Vec<T, VEC> v;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
        const int64_t n = BATCH_INNER ? i0 + i : row;
        const int64_t j = BATCH_INNER ? row : i0 + i;
        v.v[i] = src(n, j / gsz);
    }
    vstore<T, VEC>(gx + row * so + i0, v);
}

// ---- backward, batch-contiguous grad_x ([F, batch] in memory): block = (batch tile, class
// c, slice of the group's rows).  Each lane computes its g[n, c] / tau once and writes it
// down the rows of its slice.  The stores are ordinary write-back ones: the next kernel (the
// last layer's backward) reads these rows at once and finds them in the Infinity Cache;
// non-temporal stores measured 5 us slower per cfg2 step.
template <typename T, int VEC, typename Src>
__global__ __launch_bounds__(256) void k_gsum_bwd_rows(Src src, int64_t B, int64_t F, int64_t sf,
                                                       int64_t gsz, int64_t slice,
                                                       T* __restrict__ gx) {
    const int64_t n0 = (int64_t(blockIdx.x) * 64 + (threadIdx.x & 63)) * VEC;
    if (n0 >= B) return;
    const int64_t c = blockIdx.y;
    const int64_t j0 = c * gsz + int64_t(blockIdx.z) * slice;
    const int64_t j1 = std::min<int64_t>(std::min<int64_t>(j0 + slice, (c + 1) * gsz), F);
    Vec<T, VEC> v;
#pragma unroll
    for (int i = 0; i < VEC; ++i) v.v[i] = src(n0 + i, c);
    for (int64_t j = j0 + (threadIdx.x >> 6); j < j1; j += 4) vstore<T, VEC>(gx + j * sf + n0, v);
}

template <typename T, typename Src>
__global__ __launch_bounds__(256) void k_gsum_bwd_generic(Src src, int64_t B, int64_t F,
                                                          int64_t sb, int64_t sf, int64_t gsz,
                                                          T* __restrict__ gx) {
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (item >= B * F) return;
    const int64_t n = item / F, j = item % F;
    gx[n * sb + j * sf] = src(n, j / gsz);
}

// ---- mean cross-entropy of the scores.  k_ce_rows: workgroup of kCeSamples samples; its
// threads first add the group-sum slices of every (sample, class) pair (the split forward's
// finish, slices in order) into out and LDS, then one thread per sample takes the softmax
// (kept for the backward), its loss term and whether it counts.  k_ce_mean: one workgroup adds
// the terms in a fixed order.  Both are deterministic.
constexpr int kCeSamples = 16;
constexpr int kCeThreads = 256;

template <typename T>
__global__ __launch_bounds__(kCeThreads) void k_ce_rows(const T* __restrict__ part,
                                                        int64_t nslices, const int64_t* y,
                                                        int64_t B, int64_t k, int64_t ignore,
                                                        T tau, T* __restrict__ out,
                                                        T* __restrict__ p,
                                                        T* __restrict__ term) {
    extern __shared__ __align__(16) unsigned char ce_lds[];
    T* z = reinterpret_cast<T*>(ce_lds);  // [kCeSamples][k]
    const int64_t n0 = int64_t(blockIdx.x) * kCeSamples;
    const int64_t ns = std::min<int64_t>(kCeSamples, B - n0);
    const int64_t step = k * B;
    for (int64_t e = threadIdx.x; e < ns * k; e += kCeThreads) {
        const int64_t c = e % k, n = n0 + e / k;
        const T* src = part + c * B + n;
        T t = 0;
        int64_t sl = 0;
        // up to 32 slices per round of loads (one round for the usual slice counts); the
        // additions stay in slice order
        for (; sl + 32 <= nslices; sl += 32) {
            T v[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = src[(sl + i) * step];
#pragma unroll
            for (int i = 0; i < 32; ++i) t += v[i];
        }
        if (sl < nslices) {
            T v[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = sl + i < nslices ? src[(sl + i) * step] : T(0);
#pragma unroll
            for (int i = 0; i < 32; ++i)
                if (sl + i < nslices) t += v[i];
        }
        t = t / tau;
        out[n * k + c] = t;
        z[e] = t;
    }
    __syncthreads();
    if (threadIdx.x < ns) {
        const int64_t n = n0 + threadIdx.x;
        const T* zr = z + threadIdx.x * k;
        T mx = -T(__builtin_inf());
        for (int64_t c = 0; c < k; ++c) mx = fmax(mx, zr[c]);
        T sum = 0;
        for (int64_t c = 0; c < k; ++c) sum += exp(zr[c] - mx);
        const T inv = T(1) / sum;
        for (int64_t c = 0; c < k; ++c) p[n * k + c] = exp(zr[c] - mx) * inv;
        const int64_t lab = y[n];
        // term[n] = loss term, term[B + n] = 1 when the sample counts
        const bool counted = lab != ignore;
        term[n] = !counted ? T(0)
                  : (lab >= 0 && lab < k) ? (mx + log(sum)) - zr[lab] : nan_of<T>();
        term[B + n] = counted ? T(1) : T(0);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_scores_to_slices(const T* __restrict__ sc, int64_t B,
                                                          int64_t k, T* __restrict__ part) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;  // n * k + c
    if (i < B * k) part[(i % k) * B + i / k] = sc[i];
}

template <typename T>
__global__ __launch_bounds__(kCeThreads) void k_ce_mean(const T* __restrict__ term, int64_t B,
                                                        T* __restrict__ loss,
                                                        T* __restrict__ count) {
    __shared__ T sl[kCeThreads], sc[kCeThreads];
    T l = 0, c = 0;
    for (int64_t n = threadIdx.x; n < B; n += kCeThreads) {
        l += term[n];
        c += term[B + n];
    }
    sl[threadIdx.x] = l;
    sc[threadIdx.x] = c;
    __syncthreads();
    for (int h = kCeThreads / 2; h > 0; h >>= 1) {
        if (int(threadIdx.x) < h) {
            sl[threadIdx.x] += sl[threadIdx.x + h];
            sc[threadIdx.x] += sc[threadIdx.x + h];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        loss[0] = sl[0] / sc[0];  // no counted sample: 0 / 0 = NaN, the mean of nothing
        count[0] = sc[0];
    }
}

// ---- class sums of the classifier head's tile partials: block = (256 samples, class c,
// slice s of the tiles overlapping class c).  A tile overlapping class c starts in class c
// (slot 0) or in class c - 1 (slot 1): tiles are at most gsz rows.  Tiles in order.
template <typename T>
__global__ __launch_bounds__(256) void k_head_slices(const T* __restrict__ part, int64_t B,
                                                     int64_t F, int64_t gsz, int64_t k,
                                                     int64_t tile_rows, int64_t nslices,
                                                     T* __restrict__ slices) {
    const int64_t n = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (n >= B) return;
    const int64_t c = blockIdx.y, sl = blockIdx.z;
    const int64_t r0 = c * gsz, r1 = std::min<int64_t>((c + 1) * gsz, F);
    T acc = T(0);
    if (r0 < r1) {
        const int64_t t0 = r0 / tile_rows, t1 = (r1 - 1) / tile_rows;
        const int64_t per = (t1 - t0 + nslices) / nslices;  // ceil((t1 - t0 + 1) / nslices)
        const int64_t a = t0 + sl * per, b = std::min<int64_t>(a + per, t1 + 1);
        for (int64_t t = a; t < b; ++t) {
            const int64_t slot = (t * tile_rows) / gsz == c ? 0 : 1;
            acc += part[(t * 2 + slot) * B + n];
        }
    }
    slices[(sl * k + c) * B + n] = acc;
}

}  // namespace

int ce_from_tile_partials(int dtype, const void* part, int64_t batch, int64_t features,
                          int64_t k, int64_t tile_rows, double tau, const int64_t* labels,
                          int64_t ignore_index, void* out, void* probs, void* loss, void* count,
                          void* slices, int64_t nslices, void* term, hipStream_t s) {
    CL_ARG(batch >= 1 && features >= 1 && k >= 1 && tile_rows >= 1 && nslices >= 1,
           "bad head shape");
    CL_ARG(k * kCeSamples * 8 <= 64 * 1024, "k too large for the fused cross-entropy");
    const int64_t gsz = ceil_div(features, k);
    CL_ARG(tile_rows <= gsz, "tiles of %lld rows span more than two classes of %lld",
           (long long)tile_rows, (long long)gsz);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const dim3 grid(unsigned(ceil_div(batch, 256)), unsigned(k), unsigned(nslices));
        k_head_slices<T><<<grid, 256, 0, s>>>(static_cast<const T*>(part), batch, features, gsz,
                                              k, tile_rows, nslices, static_cast<T*>(slices));
        if (int rc = check_launch("cl_dense_group_sum_cross_entropy_forward(sums)")) return rc;
        k_ce_rows<T><<<unsigned(ceil_div(batch, kCeSamples)), kCeThreads,
                       size_t(kCeSamples * k * sizeof(T)), s>>>(
            static_cast<const T*>(slices), nslices, labels, batch, k, ignore_index, T(tau),
            static_cast<T*>(out), static_cast<T*>(probs), static_cast<T*>(term));
        if (int rc = check_launch("cl_dense_group_sum_cross_entropy_forward(rows)")) return rc;
        k_ce_mean<T><<<1, kCeThreads, 0, s>>>(static_cast<const T*>(term), batch,
                                              static_cast<T*>(loss), static_cast<T*>(count));
    });
    return check_launch("cl_dense_group_sum_cross_entropy_forward(mean)");
}

}  // namespace cl

using namespace cl;

namespace {
bool gsum_split_applies(int64_t batch, int64_t features, int64_t stride_batch) {
    return stride_batch == 1 && features > 0 && batch >= 64;
}
}  // namespace

extern "C" int cl_group_sum_workspace_size(int dtype, int64_t batch, int64_t features,
                                           int64_t stride_batch, int64_t stride_feature,
                                           int64_t k, int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    CL_ARG(batch >= 0 && features >= 0 && k >= 1, "bad shape");
    *bytes = 0;
    if (!gsum_split_applies(batch, features, stride_batch)) return CL_OK;
    CL_DTYPE_SWITCH(dtype, {
        constexpr int W = wide_vec<scalar_t>();
        const bool wide = batch % W == 0 && stride_feature % W == 0;
        const int64_t slices = gsum_slices(batch, features, k, wide ? W : 1);
        *bytes = slices > 1 ? slices * k * batch * int64_t(sizeof(scalar_t)) : 0;
    });
    return CL_OK;
}

extern "C" int cl_group_sum_forward(int dtype, const void* x, int64_t batch, int64_t features,
                                    int64_t stride_batch, int64_t stride_feature, int64_t k,
                                    double tau, void* out, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
    clear_error();
    CL_ARG(batch >= 0 && features >= 0, "negative shape");
    CL_ARG(k >= 1, "k must be >= 1, got %lld", (long long)k);
    CL_ARG(stride_batch >= 0 && stride_feature >= 0, "negative strides are not supported");
    CL_ARG(workspace_bytes >= 0, "negative workspace size");
    if (batch == 0) return CL_OK;
    CL_ARG(out, "null pointer argument");
    CL_ARG(features == 0 || x, "null pointer argument");
    const int64_t gsz = features == 0 ? 1 : ceil_div(features, k);
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const T* xs = static_cast<const T*>(x);
        T* os = static_cast<T*>(out);
        const T t = T(tau);
        constexpr int W = wide_vec<T>();
        if (gsum_split_applies(batch, features, stride_batch)) {
            const bool wide = batch % W == 0 && stride_feature % W == 0 && aligned(x, 16);
            const int vec = wide ? W : 1;
            const int64_t slices = gsum_slices(batch, features, k, vec);
            const int64_t need = slices * k * batch * int64_t(sizeof(T));
            if (slices > 1 && workspace && workspace_bytes >= need) {
                T* part = static_cast<T*>(workspace);
                const int64_t slice = ceil_div(gsz, slices);
                const dim3 grid(unsigned(ceil_div(batch, 64 * vec)), unsigned(k), unsigned(slices));
                if (wide)
                    k_gsum_partial<T, W><<<grid, kPartWaves * 64, 0, s>>>(
                        xs, batch, features, stride_feature, gsz, k, slice, part);
                else
                    k_gsum_partial<T, 1><<<grid, kPartWaves * 64, 0, s>>>(
                        xs, batch, features, stride_feature, gsz, k, slice, part);
                if (int rc = check_launch("cl_group_sum_forward(partial)")) return rc;
                k_gsum_finish<T><<<unsigned(ceil_div(batch * k, 256)), 256, 0, s>>>(
                    part, batch, k, slices, t, os);
            } else if (wide) {
                const dim3 grid(unsigned(ceil_div(batch, 64 * W)), unsigned(k), 1);
                k_gsum_fwd_bc<T, W><<<grid, kSplitWaves * 64, 0, s>>>(xs, batch, features,
                                                                      stride_feature, gsz, k, t, os);
            } else {
                const dim3 grid(unsigned(ceil_div(batch, 64)), unsigned(k), 1);
                k_gsum_fwd_bc<T, 1><<<grid, kSplitWaves * 64, 0, s>>>(xs, batch, features,
                                                                      stride_feature, gsz, k, t, os);
            }
        } else if (stride_feature == 1 || features <= 1) {
            const dim3 grid(unsigned(ceil_div(batch * k, 4)), 1, 1);
            k_gsum_fwd_fc<T><<<grid, 256, 0, s>>>(xs, batch, features, stride_batch, gsz, k, t, os);
        } else {
            const dim3 grid(unsigned(ceil_div(batch * k, 256)), 1, 1);
            k_gsum_fwd_generic<T><<<grid, 256, 0, s>>>(xs, batch, features, stride_batch,
                                                       stride_feature, gsz, k, t, os);
        }
    });
    return check_launch("cl_group_sum_forward");
}

namespace {
// grad_x from a gradient source, in grad_x's memory order (see the kernels above).
template <typename T, typename Src>
int launch_gsum_backward(const Src& src, int64_t batch, int64_t features, int64_t k,
                         T* gxs, int64_t stride_batch, int64_t stride_feature, hipStream_t s) {
    const int64_t gsz = ceil_div(features, k);
    constexpr int W = wide_vec<T>();
    if (stride_batch == 1) {
        const bool wide = batch % W == 0 && stride_feature % W == 0 && aligned(gxs, 16);
        const int vec = wide ? W : 1;
        const int64_t slice = std::max<int64_t>(std::min<int64_t>(gsz, 32), ceil_div(gsz, 65535));
        const dim3 grid(unsigned(ceil_div(batch, 64 * vec)), unsigned(k),
                        unsigned(ceil_div(gsz, slice)));
        if (wide)
            k_gsum_bwd_rows<T, W><<<grid, 256, 0, s>>>(src, batch, features, stride_feature, gsz,
                                                      slice, gxs);
        else
            k_gsum_bwd_rows<T, 1><<<grid, 256, 0, s>>>(src, batch, features, stride_feature, gsz,
                                                      slice, gxs);
    } else if (stride_feature == 1) {
        const bool wide = features % W == 0 && stride_batch % W == 0 && aligned(gxs, 16);
        const int vec = wide ? W : 1;
        const dim3 grid(unsigned(ceil_div(batch, 4)), unsigned(ceil_div(features, 64 * vec)), 1);
        if (wide)
            k_gsum_bwd<T, W, false><<<grid, 256, 0, s>>>(src, batch, features, stride_batch, gsz,
                                                        gxs);
        else
            k_gsum_bwd<T, 1, false><<<grid, 256, 0, s>>>(src, batch, features, stride_batch, gsz,
                                                        gxs);
    } else {
        const dim3 grid(unsigned(ceil_div(batch * features, 256)), 1, 1);
        k_gsum_bwd_generic<T><<<grid, 256, 0, s>>>(src, batch, features, stride_batch,
                                                   stride_feature, gsz, gxs);
    }
    return CL_OK;
}
}  // namespace

extern "C" int cl_group_sum_backward(int dtype, const void* grad_out, int64_t batch,
                                     int64_t features, int64_t k, double tau, void* grad_x,
                                     int64_t stride_batch, int64_t stride_feature, void* stream) {
    clear_error();
    CL_ARG(batch >= 0 && features >= 0, "negative shape");
    CL_ARG(k >= 1, "k must be >= 1, got %lld", (long long)k);
    CL_ARG(stride_batch >= 0 && stride_feature >= 0, "negative strides are not supported");
    if (batch == 0 || features == 0) return CL_OK;
    CL_ARG(grad_out && grad_x, "null pointer argument");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const ScoreGrad<T> src{static_cast<const T*>(grad_out), k, T(tau)};
        launch_gsum_backward<T>(src, batch, features, k, static_cast<T*>(grad_x), stride_batch,
                                stride_feature, s);
    });
    return check_launch("cl_group_sum_backward");
}

extern "C" int cl_group_sum_cross_entropy_workspace_size(int dtype, int64_t batch,
                                                         int64_t features, int64_t k,
                                                         int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    CL_ARG(batch >= 0 && features >= 0 && k >= 1, "bad shape");
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        constexpr int W = wide_vec<T>();
        const int64_t slices = gsum_slices(batch, features, k, W);
        *bytes = (slices * k * batch + 2 * batch) * int64_t(sizeof(T));
    });
    return CL_OK;
}

extern "C" int cl_group_sum_cross_entropy_forward(int dtype, const void* x, int64_t batch,
                                                  int64_t features, int64_t stride_batch,
                                                  int64_t stride_feature, int64_t k, double tau,
                                                  const int64_t* labels, int64_t ignore_index,
                                                  void* out, void* probs, void* loss,
                                                  void* count, void* workspace,
                                                  int64_t workspace_bytes, void* stream) {
    clear_error();
    CL_ARG(batch >= 0 && features >= 0, "negative shape");
    CL_ARG(k >= 1, "k must be >= 1, got %lld", (long long)k);
    CL_ARG(stride_batch >= 0 && stride_feature >= 0, "negative strides are not supported");
    CL_ARG(labels && probs && loss && count && out, "null pointer argument");
    CL_ARG(features == 0 || x, "null pointer argument");
    CL_ARG(k * kCeSamples * 8 <= 64 * 1024, "k too large for the fused cross-entropy");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const T t = T(tau);
        constexpr int W = wide_vec<T>();
        const int64_t gsz = features == 0 ? 1 : ceil_div(features, k);
        const bool split = gsum_split_applies(batch, features, stride_batch);
        const bool wide = split && batch % W == 0 && stride_feature % W == 0 && aligned(x, 16);
        // slices of the split forward (one slice: the plain sums, written by the same path)
        const int64_t slices = split ? gsum_slices(batch, features, k, wide ? W : 1) : 1;
        const int64_t need = (slices * k * batch + 2 * batch) * int64_t(sizeof(T));
        CL_ARG(need == 0 || (workspace && workspace_bytes >= need),
               "workspace of %lld bytes needed (cl_group_sum_cross_entropy_workspace_size)",
               (long long)need);
        T* part = static_cast<T*>(workspace);
        T* term = part + slices * k * batch;
        if (batch > 0) {
            if (split) {
                const int64_t slice = ceil_div(gsz, slices);
                const dim3 grid(unsigned(ceil_div(batch, 64 * (wide ? W : 1))), unsigned(k),
                                unsigned(slices));
                if (wide)
                    k_gsum_partial<T, W><<<grid, kPartWaves * 64, 0, s>>>(
                        static_cast<const T*>(x), batch, features, stride_feature, gsz, k,
                        slice, part);
                else
                    k_gsum_partial<T, 1><<<grid, kPartWaves * 64, 0, s>>>(
                        static_cast<const T*>(x), batch, features, stride_feature, gsz, k,
                        slice, part);
            } else {
                // the other layouts: their sums (tau = 1) into out, then out as one [k, batch]
                // slice; k_ce_rows overwrites out with the scores
                if (int rc = cl_group_sum_forward(dtype, x, batch, features, stride_batch,
                                                  stride_feature, k, 1.0, out, nullptr, 0,
                                                  stream))
                    return rc;
                k_scores_to_slices<T><<<unsigned(ceil_div(batch * k, 256)), 256, 0, s>>>(
                    static_cast<const T*>(out), batch, k, part);
            }
            if (int rc = check_launch("cl_group_sum_cross_entropy_forward(sums)")) return rc;
            k_ce_rows<T><<<unsigned(ceil_div(batch, kCeSamples)), kCeThreads,
                           size_t(kCeSamples * k * sizeof(T)), s>>>(
                part, slices, labels, batch, k, ignore_index, t, static_cast<T*>(out),
                static_cast<T*>(probs), term);
            if (int rc = check_launch("cl_group_sum_cross_entropy_forward(rows)")) return rc;
        }
        k_ce_mean<T><<<1, kCeThreads, 0, s>>>(term, batch, static_cast<T*>(loss),
                                              static_cast<T*>(count));
    });
    return check_launch("cl_group_sum_cross_entropy_forward");
}

extern "C" int cl_group_sum_cross_entropy_backward(int dtype, const void* probs,
                                                   const int64_t* labels, int64_t ignore_index,
                                                   const void* grad_loss, const void* count,
                                                   int64_t batch, int64_t features, int64_t k,
                                                   double tau, void* grad_x,
                                                   int64_t stride_batch, int64_t stride_feature,
                                                   void* stream) {
    clear_error();
    CL_ARG(batch >= 0 && features >= 0, "negative shape");
    CL_ARG(k >= 1, "k must be >= 1, got %lld", (long long)k);
    CL_ARG(stride_batch >= 0 && stride_feature >= 0, "negative strides are not supported");
    if (batch == 0 || features == 0) return CL_OK;
    CL_ARG(probs && labels && grad_loss && count && grad_x, "null pointer argument");
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        const CrossEntropyGrad<T> src{static_cast<const T*>(probs), labels, ignore_index,
                                      static_cast<const T*>(grad_loss),
                                      static_cast<const T*>(count), k, T(tau)};
        launch_gsum_backward<T>(src, batch, features, k, static_cast<T*>(grad_x), stride_batch,
                                stride_feature, s);
    });
    return check_launch("cl_group_sum_cross_entropy_backward");
}

// ------------------------------------------------------------------------------------------
// Allocation-free variant of cl_group_sum_cross_entropy_forward: the same kernels, with the
// workspace taken from a file-scope device array instead of the caller.  Each GPU holds its
// own copy of `scratch` for the life of the process.  Its device address is looked up once
// per device (hipGetSymbolAddress, with that device current) and kept in g_scratch_ptr; the
// array's name is never used as an address on the host.  The kernels write every workspace
// element they later read (slice partials, loss terms), so nothing needs clearing between
// calls.  Calls that overlap on one GPU (several streams, several host threads) race on the
// array.
#include <mutex>

namespace {
constexpr int64_t kCeScratchBytes = int64_t(8) << 20;  // 8 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kCeScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on `dev` (looked up on the first call for that device).
int scratch_on(int dev, void** out) {
    CL_ARG(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess) {
            set_error("hipGetDevice failed");
            return CL_ERR_HIP;
        }
        if (cur != dev && hipSetDevice(dev) != hipSuccess) {
            set_error("hipSetDevice(%d) failed", dev);
            return CL_ERR_HIP;
        }
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return CL_ERR_HIP;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CL_OK;
}
}  // namespace

extern "C" int cl_group_sum_cross_entropy_scratch_limit(int64_t* bytes) {
    clear_error();
    CL_ARG(bytes, "null pointer argument");
    *bytes = kCeScratchBytes;
    return CL_OK;
}

extern "C" int cl_group_sum_cross_entropy_forward_noalloc(
    int dtype, const void* x, int64_t batch, int64_t features, int64_t stride_batch,
    int64_t stride_feature, int64_t k, double tau, const int64_t* labels, int64_t ignore_index,
    void* out, void* probs, void* loss, void* count, void* stream) {
    clear_error();
    CL_ARG(batch >= 0 && features >= 0 && k >= 1, "bad shape");
    int64_t need = 0;
    if (int rc = cl_group_sum_cross_entropy_workspace_size(dtype, batch, features, k, &need))
        return rc;
    CL_ARG(need <= kCeScratchBytes,
           "cl_group_sum_cross_entropy_forward_noalloc: this shape needs %lld bytes of scratch, "
           "the limit is %lld (use cl_group_sum_cross_entropy_forward with a workspace)",
           (long long)need, (long long)kCeScratchBytes);
    int dev = -1;
    hipError_t e = stream ? hipStreamGetDevice(as_stream(stream), &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("cannot determine the stream's device: %s", hipGetErrorString(e));
        return CL_ERR_HIP;
    }
    void* ws = nullptr;
    if (int rc = scratch_on(dev, &ws)) return rc;
    return cl_group_sum_cross_entropy_forward(dtype, x, batch, features, stride_batch,
                                              stride_feature, k, tau, labels, ignore_index, out,
                                              probs, loss, count, ws, kCeScratchBytes, stream);
}
