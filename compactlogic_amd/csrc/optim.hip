// The optimizer half of a CompactLogic training step (experiments/experiment_script.py:280-293):
//   torch.nn.utils.clip_grad_norm_(params, max_norm)   then   torch.optim.Adam.step()
// over every parameter tensor, in two launches.
//
//   k_sq_partials   per-workgroup sums of g^2 over a slice of the parameters (all tensors taken
//                   as one concatenation), and the step counter advanced by one
//   k_adam_update   every workgroup adds the partials in a fixed order (the global norm),
//                   scales its gradients by min(1, max_norm / (norm + 1e-6)) and writes them
//                   back (as clip_grad_norm_ does), then applies Adam to its slice:
//                     m = beta1 m + (1 - beta1) g,  v = beta2 v + (1 - beta2) g^2,
//                     p -= (lr / (1 - beta1^t)) m / (sqrt(v) / sqrt(1 - beta2^t) + eps)
// The step count lives on the device, so a captured graph replays correct bias corrections.
// Every sum has a fixed order: results are bitwise reproducible.
#include "common.h"

namespace cl {
namespace {

constexpr int kOptThreads = 256;
constexpr int kOptPerThread = 4;                             // update: elements per thread
constexpr int64_t kOptChunk = kOptThreads * kOptPerThread;  // update: elements per workgroup
constexpr int kNormPerThread = 16;                           // norm: elements per thread
constexpr int64_t kNormChunk = kOptThreads * kNormPerThread; // norm: one partial per chunk
constexpr int kOptMaxTensors = 32;                           // per launch

template <typename T>
struct OptTensors {
    int n;
    int64_t start[kOptMaxTensors + 1];  // prefix offsets into the concatenation
    T* param[kOptMaxTensors];
    T* grad[kOptMaxTensors];
    T* m[kOptMaxTensors];
    T* v[kOptMaxTensors];
};

// Tensor holding concatenation element i (linear scan; at most kOptMaxTensors entries).
template <typename T>
__device__ __forceinline__ int tensor_of(const OptTensors<T>& ts, int64_t i) {
    int t = 0;
    while (t + 1 < ts.n && ts.start[t + 1] <= i) ++t;
    return t;
}

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    T s = 0;
    if (threadIdx.x == 0) {
        for (int i = 0; i < kOptThreads / 64; ++i) s += red[i];
        red[0] = s;
    }
    __syncthreads();
    s = red[0];
    __syncthreads();
    return s;
}

template <typename T>
__global__ __launch_bounds__(kOptThreads) void k_sq_partials(OptTensors<T> ts, T* __restrict__ part,
                                                             T* __restrict__ step) {
    __shared__ T red[kOptThreads / 64];
    const int64_t total = ts.start[ts.n];
    const int64_t base = int64_t(blockIdx.x) * kNormChunk;
    T s = 0;
#pragma unroll
    for (int k = 0; k < kNormPerThread; ++k) {
        const int64_t i = base + int64_t(k) * kOptThreads + threadIdx.x;
        if (i < total) {
            const int t = tensor_of(ts, i);
            const T g = ts.grad[t][i - ts.start[t]];
            s += g * g;
        }
    }
    s = block_sum(s, red);
    if (threadIdx.x == 0) {
        if (total > 0) part[blockIdx.x] = s;
        if (blockIdx.x == 0) step[0] = step[0] + T(1);
    }
}

template <typename T>
__global__ __launch_bounds__(kOptThreads) void k_adam_update(OptTensors<T> ts,
                                                             const T* __restrict__ part,
                                                             int64_t nparts,
                                                             const T* __restrict__ step, T lr,
                                                             T beta1, T beta2, T eps,
                                                             T max_norm, int clip) {
    __shared__ T red[kOptThreads / 64];
    // the global norm: every workgroup adds the same partials in the same order
    T s = 0;
    for (int64_t i = threadIdx.x; i < nparts; i += kOptThreads) s += part[i];
    const T sq = block_sum(s, red);
    T coef = T(1);
    if (clip) {
        const T c = max_norm / (sqrt(sq) + T(1e-6));
        coef = c < T(1) ? c : T(1);
    }
    // bias corrections once per workgroup
    if (threadIdx.x == 0) {
        const T t = step[0];
        red[0] = lr / (T(1) - pow(beta1, t));
        red[1] = sqrt(T(1) - pow(beta2, t));
    }
    __syncthreads();
    const T step_size = red[0], bc2_sqrt = red[1];
    const int64_t total = ts.start[ts.n];
    const int64_t base = int64_t(blockIdx.x) * kOptChunk;
#pragma unroll
    for (int k = 0; k < kOptPerThread; ++k) {
        const int64_t i = base + int64_t(k) * kOptThreads + threadIdx.x;
        if (i < total) {
            const int tt = tensor_of(ts, i);
            const int64_t j = i - ts.start[tt];
            T g = ts.grad[tt][j];
            if (clip) {
                g = g * coef;
                ts.grad[tt][j] = g;
            }
            T m = ts.m[tt][j], v = ts.v[tt][j];
            m = m + (T(1) - beta1) * (g - m);
            v = v * beta2 + (T(1) - beta2) * g * g;
            ts.m[tt][j] = m;
            ts.v[tt][j] = v;
            const T denom = sqrt(v) / bc2_sqrt + eps;
            ts.param[tt][j] = ts.param[tt][j] - step_size * (m / denom);
        }
    }
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_adam_clip_max_tensors(int64_t* n) {
    clear_error();
    CL_ARG(n, "null pointer argument");
    *n = kOptMaxTensors;
    return CL_OK;
}

extern "C" int cl_adam_clip_workspace(int64_t num_tensors, const int64_t* numels,
                                      int64_t* elements) {
    clear_error();
    CL_ARG(elements && (num_tensors == 0 || numels), "null pointer argument");
    CL_ARG(num_tensors >= 0 && num_tensors <= kOptMaxTensors, "at most %d tensors",
           kOptMaxTensors);
    int64_t total = 0;
    for (int64_t i = 0; i < num_tensors; ++i) {
        CL_ARG(numels[i] >= 0, "negative tensor size");
        total += numels[i];
    }
    *elements = ceil_div(total, kNormChunk);
    return CL_OK;
}

extern "C" int cl_adam_clip_step(int dtype, int64_t num_tensors, void* const* params,
                                 void* const* grads, void* const* exp_avg,
                                 void* const* exp_avg_sq, const int64_t* numels, void* step,
                                 double lr, double beta1, double beta2, double eps,
                                 double max_norm, void* workspace, int64_t workspace_elements,
                                 void* stream) {
    clear_error();
    CL_ARG(num_tensors >= 0 && num_tensors <= kOptMaxTensors, "at most %d tensors per call",
           kOptMaxTensors);
    CL_ARG(num_tensors == 0 || (params && grads && exp_avg && exp_avg_sq && numels),
           "null pointer argument");
    CL_ARG(step, "null step pointer");
    CL_ARG(lr >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1 && eps >= 0,
           "invalid Adam hyper-parameters");
    int64_t nparts = 0;
    if (int rc = cl_adam_clip_workspace(num_tensors, numels, &nparts)) return rc;
    CL_ARG(nparts < (int64_t(1) << 31), "too many parameters for one call");
    CL_ARG(nparts == 0 || (workspace && workspace_elements >= nparts),
           "workspace of %lld elements needed (cl_adam_clip_workspace)", (long long)nparts);
    hipStream_t s = as_stream(stream);
    CL_DTYPE_SWITCH(dtype, {
        using T = scalar_t;
        OptTensors<T> ts{};
        ts.n = int(num_tensors);
        ts.start[0] = 0;
        for (int i = 0; i < ts.n; ++i) {
            CL_ARG(numels[i] == 0 || (params[i] && grads[i] && exp_avg[i] && exp_avg_sq[i]),
                   "null tensor pointer at index %d", i);
            ts.param[i] = static_cast<T*>(params[i]);
            ts.grad[i] = static_cast<T*>(grads[i]);
            ts.m[i] = static_cast<T*>(exp_avg[i]);
            ts.v[i] = static_cast<T*>(exp_avg_sq[i]);
            ts.start[i + 1] = ts.start[i] + numels[i];
        }
        T* part = static_cast<T*>(workspace);
        T* st = static_cast<T*>(step);
        // one workgroup when there is nothing to update: it still advances the step count
        k_sq_partials<T><<<unsigned(nparts > 0 ? nparts : 1), kOptThreads, 0, s>>>(ts, part, st);
        if (int rc = check_launch("cl_adam_clip_step(norm)")) return rc;
        const int64_t ublocks = ceil_div(ts.start[ts.n], kOptChunk);
        CL_ARG(ublocks < (int64_t(1) << 31), "too many parameters for one call");
        if (nparts > 0)
            k_adam_update<T><<<unsigned(ublocks), kOptThreads, 0, s>>>(
                ts, part, nparts, st, T(lr), T(beta1), T(beta2), T(eps), T(max_norm),
                max_norm > 0 ? 1 : 0);
    });
    return check_launch("cl_adam_clip_step");
}
