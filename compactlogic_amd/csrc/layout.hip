// Layout change between the modules' [batch, features] tensors and the kernels' [features,
// batch] rows (compactlogic/compactlogic.py:100-101 does it with a torch transpose copy).
//
// One 64 x 64 tile per workgroup through LDS: the reads run along the source rows and the
// writes along the destination rows, both 64 consecutive elements per wave instruction.  The
// LDS tile has one padding column, so the column reads of the transposed pass fall in
// distinct banks.
#include "common.h"

namespace cl {
namespace {

constexpr int kTile = 64;

template <typename T>
__global__ __launch_bounds__(256) void k_transpose(const T* __restrict__ src, T* __restrict__ dst,
                                                   int64_t rows, int64_t cols) {
    __shared__ T tile[kTile][kTile + 1];
    const int64_t r0 = int64_t(blockIdx.y) * kTile;
    const int64_t c0 = int64_t(blockIdx.x) * kTile;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < kTile / 4; ++i) {
        const int rr = i * 4 + wv;
        const int64_t r = r0 + rr, c = c0 + lane;
        tile[rr][lane] = (r < rows && c < cols) ? src[r * cols + c] : T(0);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTile / 4; ++i) {
        const int cc = i * 4 + wv;
        const int64_t c = c0 + cc, r = r0 + lane;
        if (c < cols && r < rows) dst[c * rows + r] = tile[lane][cc];
    }
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_transpose(int dtype, const void* src, void* dst, int64_t rows, int64_t cols,
                            void* stream) {
    clear_error();
    CL_ARG(rows >= 0 && cols >= 0, "negative dimension");
    if (rows == 0 || cols == 0) return CL_OK;
    CL_ARG(src && dst, "null pointer argument");
    CL_ARG(src != dst, "cl_transpose does not work in place");
    const int64_t gx = ceil_div(cols, int64_t(kTile)), gy = ceil_div(rows, int64_t(kTile));
    CL_ARG(gx < (int64_t(1) << 31) && gy < 65536, "matrix too large for one launch");
    CL_DTYPE_SWITCH(dtype, {
        k_transpose<scalar_t><<<dim3(unsigned(gx), unsigned(gy)), 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(src), static_cast<scalar_t*>(dst), rows, cols);
    });
    return check_launch("cl_transpose");
}
