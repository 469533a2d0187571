// Layout change between the modules' [batch, features] tensors and the kernels' [features,
// batch] rows (compactlogic/compactlogic.py:100-101 does it with a torch transpose copy).
//
// Every tile goes through LDS: the reads run along the source rows and the writes along the
// destination rows.  The general kernel moves one 64 x 64 tile per workgroup, 64 consecutive
// elements per wave instruction; its LDS tile has one padding column, so the column reads of
// the transposed pass fall in distinct banks.
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

// fp32 with rows % 4 == cols % 4 == 0: one 32 x 32 tile per workgroup, one 16-byte load
// and one 16-byte store per thread.  Eight lanes cover a 128-byte row segment of the source
// on the way in and of the destination on the way out (each store gathers its four values
// from four LDS rows).  The small tile gives a 1024 x 784 input 800 workgroups: the layout
// change of a training step's input is a few MB, so it is bound by how many loads are in
// flight, not by bandwidth.
constexpr int kTile4 = 32;

__global__ __launch_bounds__(256) void k_transpose_v4(const float4* __restrict__ src,
                                                      float4* __restrict__ dst, int64_t rows,
                                                      int64_t cols) {
    __shared__ float tile[kTile4][kTile4 + 1];
    const int64_t r0 = int64_t(blockIdx.y) * kTile4;
    const int64_t c0 = int64_t(blockIdx.x) * kTile4;
    const int q = threadIdx.x & 7;    // 4-element group within the tile's 32 columns / rows
    const int rr = threadIdx.x >> 3;  // 0..31
    const int64_t cols4 = cols / 4, rows4 = rows / 4;
    {
        const int64_t r = r0 + rr, c = c0 + 4 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows && c < cols) v = src[r * cols4 + c / 4];
        tile[rr][4 * q + 0] = v.x;
        tile[rr][4 * q + 1] = v.y;
        tile[rr][4 * q + 2] = v.z;
        tile[rr][4 * q + 3] = v.w;
    }
    __syncthreads();
    const int cc = rr;
    const int64_t c = c0 + cc, r = r0 + 4 * q;
    if (c < cols && r < rows)
        dst[c * rows4 + r / 4] = make_float4(tile[4 * q + 0][cc], tile[4 * q + 1][cc],
                                             tile[4 * q + 2][cc], tile[4 * q + 3][cc]);
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
    if (dtype == CL_DTYPE_F32 && rows % 4 == 0 && cols % 4 == 0 && aligned(src, 16) &&
        aligned(dst, 16)) {
        const int64_t gx4 = ceil_div(cols, int64_t(kTile4)), gy4 = ceil_div(rows, int64_t(kTile4));
        CL_ARG(gx4 < (int64_t(1) << 31) && gy4 < 65536, "matrix too large for one launch");
        k_transpose_v4<<<dim3(unsigned(gx4), unsigned(gy4)), 256, 0, as_stream(stream)>>>(
            static_cast<const float4*>(src), static_cast<float4*>(dst), rows, cols);
        return check_launch("cl_transpose");
    }
    CL_DTYPE_SWITCH(dtype, {
        k_transpose<scalar_t><<<dim3(unsigned(gx), unsigned(gy)), 256, 0, as_stream(stream)>>>(
            static_cast<const scalar_t*>(src), static_cast<scalar_t*>(dst), rows, cols);
    });
    return check_launch("cl_transpose");
}
