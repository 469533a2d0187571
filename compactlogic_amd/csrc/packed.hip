// Bit-packed discrete inference for gfx950.
//
// A packed row is a little-endian bit string: bit j of the row (bit j%8 of byte j/8) is
// sample j.  This is the layout tensor_packbits_cuda writes for every word width
// (compactlogic/cuda/difflogic_kernel.cu:417-451: bit i of word w is sample bits*w + i, and
// words are stored little-endian), so any row can be processed as 64-bit words whatever
// width the caller packed it with, as long as the row byte length allows it.
#include "common.h"

#include <algorithm>
#include <type_traits>

namespace cl {
namespace {

// ------------------------------------------------------------------------------------------
// pack: t [rows, n] bool bytes -> rows of row_bytes bytes.  One thread builds one 8-byte
// chunk (or one byte when the row length is not a multiple of 8).
__device__ __forceinline__ uint64_t gather8(const uint8_t* p, int64_t avail) {
    // Eight 0/1 bytes -> eight bits, LSB = first byte.
    uint64_t v = 0;
    if (avail >= 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v |= uint64_t(p[i]) << (8 * i);
    } else {
        for (int i = 0; i < avail; ++i) v |= uint64_t(p[i]) << (8 * i);
    }
    // Multiplying by sum_j 2^(8j + 7 - j) moves byte i's bit to position 56 + i without
    // carries (all partial products land on distinct bits), so the top byte holds the bits.
    return (v * 0x0102040810204080ULL) >> 56;
}

template <typename W>
__global__ __launch_bounds__(256) void k_pack_bits(const uint8_t* __restrict__ t, int64_t rows,
                                                   int64_t n, int64_t row_words,
                                                   W* __restrict__ out) {
    const int64_t item = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (item >= rows * row_words) return;
    const int64_t r = item / row_words, wi = item % row_words;
    constexpr int kBytes = int(sizeof(W));
    const uint8_t* src = t + r * n;
    uint64_t word = 0;
#pragma unroll
    for (int q = 0; q < kBytes; ++q) {
        const int64_t s0 = (wi * kBytes + q) * 8;  // first sample of this output byte
        const int64_t avail = n - s0;
        if (avail > 0) word |= gather8(src + s0, avail) << (8 * q);
    }
    out[item] = W(word);
}

// ------------------------------------------------------------------------------------------
// Bitwise layer: y[o, :] = op(x[a, :], x[b, :]) with the argmax slot of neuron o.  One wave
// per neuron and word chunk; lanes stream VEC consecutive words.  The grid's x dimension
// runs over neurons first so the workgroups in flight cover one band of words of every
// row, and the band of x they gather from stays cache resident.  The output rows are
// written once and read by the next layer only, so 16-byte rows are stored non-temporally
// and leave the caches to the band being gathered (7% faster per pass at cfg4).
constexpr int kPackedU = 4;  // 16-byte vectors per lane and row (8 measures slower)

template <typename W, int VEC, int U>
__global__ __launch_bounds__(256) void k_eval_packed(const W* __restrict__ x,
                                                     const int64_t* __restrict__ a,
                                                     const int64_t* __restrict__ b,
                                                     const uint8_t* __restrict__ wslot,
                                                     const uint8_t* __restrict__ gs,
                                                     W* __restrict__ y, int64_t in_dim,
                                                     int64_t out_dim, int64_t words, int G) {
    const int64_t o = int64_t(blockIdx.x) * 4 + wave_id();
    if (o >= out_dim) return;
    // Every load is unconditional (clamped slot, row 0 for a bad record, word 0 past the
    // row's end, results masked afterwards): a load under a branch makes the compiler wait
    // for it inside the branch, which serialized the U steps of a lane.
    const int s = wslot[o];
    const int sc = s < G ? s : 0;
    int64_t ia = a[o * G + sc];
    int64_t ib = b[o * G + sc];
    const int g = gs[o * G + sc];
    const bool bad = s >= G || uint64_t(ia) >= uint64_t(in_dim) || uint64_t(ib) >= uint64_t(in_dim);
    if (bad) ia = ib = 0;
    const W* xa = x + ia * words;
    const W* xb = x + ib * words;
    W* yr = y + o * words;
    const int64_t w0 = int64_t(blockIdx.y) * (64 * VEC * U) + int64_t(lane_id()) * VEC;
    if constexpr (VEC == 2 && sizeof(W) == 8) {
        typedef unsigned int U4v __attribute__((ext_vector_type(4)));
        U4v va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = w0 + int64_t(u) * 64 * VEC;
            const int64_t off = idx < words ? idx : 0;
            va[u] = *reinterpret_cast<const U4v*>(xa + off);
            vb[u] = *reinterpret_cast<const U4v*>(xb + off);
        }
        const U4v keep = U4v(bad ? 0u : ~0u);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = w0 + int64_t(u) * 64 * VEC;
            U4v r;
            r.x = bitwise_op<uint32_t>(g, va[u].x, vb[u].x);
            r.y = bitwise_op<uint32_t>(g, va[u].y, vb[u].y);
            r.z = bitwise_op<uint32_t>(g, va[u].z, vb[u].z);
            r.w = bitwise_op<uint32_t>(g, va[u].w, vb[u].w);
            if (idx < words) __builtin_nontemporal_store(r & keep, reinterpret_cast<U4v*>(yr + idx));
        }
    } else {
        W va[U][VEC], vb[U][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const int64_t idx = w0 + int64_t(u) * 64 * VEC + v;
                const int64_t off = idx < words ? idx : 0;
                va[u][v] = xa[off];
                vb[u][v] = xb[off];
            }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                const int64_t idx = w0 + int64_t(u) * 64 * VEC + v;
                if (idx < words) yr[idx] = bad ? W(0) : bitwise_op<W>(g, va[u][v], vb[u][v]);
            }
    }
}

// ------------------------------------------------------------------------------------------
// Group popcount.  counts[n, c] = sum over the rows of group c of bit n.  Each thread owns
// one word column of one class and counts its group's rows "vertically" with bit-sliced
// counters: carry-save adders fold 16 rows into ones/twos/fours/eights slices and a
// sixteens word that ripples into the upper slices, so a row costs a handful of bitwise
// operations instead of one add per sample.  The per-sample counts are then read out of the
// slices, transposed through LDS, and written as contiguous [sample, class] rows.
template <typename W>
__device__ __forceinline__ void csa(W& h, W& l, W a, W b, W c) {
    const W u = a ^ b;
    h = (a & b) | (u & c);
    l = u ^ c;
}

template <typename W, int NB>
struct SliceCounter {
    W s[NB];  // s[k] holds bit k of every per-sample count

    __device__ __forceinline__ void clear() {
#pragma unroll
        for (int k = 0; k < NB; ++k) s[k] = 0;
    }
    // Add `v` (one bit per sample) with weight 2^level.
    __device__ __forceinline__ void add(W v, int level) {
        W carry = v;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            if (k >= level) {
                const W t = s[k] & carry;
                s[k] ^= carry;
                carry = t;
            }
        }
    }
    __device__ __forceinline__ int count(int bit) const {
        int c = 0;
#pragma unroll
        for (int k = 0; k < NB; ++k) c |= int((s[k] >> bit) & 1) << k;
        return c;
    }
};

// Every packed word is read once: non-temporal loads.  Column tiles of 32 words keep the LDS
// transpose tile at 41 KB, so three workgroups fit a CU (48 columns: two).
#ifndef CL_GBS_MAX_COLS
#define CL_GBS_MAX_COLS 32
#endif
constexpr int kGbsThreads = 512;
constexpr int kGbsMaxClasses = 16;  // classes per pass

template <typename W, int NB>
__global__ __launch_bounds__(kGbsThreads) void k_group_bit_sum(const W* __restrict__ x,
                                                               int64_t words, int64_t gsz,
                                                               int64_t k, int64_t n_valid,
                                                               int cols, int kb,
                                                               int32_t* __restrict__ counts) {
    constexpr int kBits = int(sizeof(W)) * 8;
    using CountT = typename std::conditional<NB <= 16, uint16_t, int32_t>::type;
    extern __shared__ __align__(16) unsigned char lds_raw[];
    CountT* lds = reinterpret_cast<CountT*>(lds_raw);  // [cols][kBits * kb + 1]
    const int row_stride = kBits * kb + 1;
    const int t = threadIdx.x;
    const int cls = t / cols, col = t % cols;
    const int64_t col0 = int64_t(blockIdx.x) * cols;
    const int64_t c0 = int64_t(blockIdx.y) * kb;
    const int64_t wc = col0 + col;
    const int64_t c = c0 + cls;

    if (cls < kb && c < k && wc < words) {
        const W* p = x + (c * gsz) * words + wc;
        SliceCounter<W, NB> cnt;
        cnt.clear();
        int64_t r = 0;
        W ones = 0, twos = 0, fours = 0, eights = 0;
        for (; r + 16 <= gsz; r += 16) {
            W v[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                v[q] = __builtin_nontemporal_load(p + (r + q) * words);
            }
            W twosA, twosB, foursA, foursB, eightsA, eightsB, sixteens;
            csa(twosA, ones, ones, v[0], v[1]);
            csa(twosB, ones, ones, v[2], v[3]);
            csa(foursA, twos, twos, twosA, twosB);
            csa(twosA, ones, ones, v[4], v[5]);
            csa(twosB, ones, ones, v[6], v[7]);
            csa(foursB, twos, twos, twosA, twosB);
            csa(eightsA, fours, fours, foursA, foursB);
            csa(twosA, ones, ones, v[8], v[9]);
            csa(twosB, ones, ones, v[10], v[11]);
            csa(foursA, twos, twos, twosA, twosB);
            csa(twosA, ones, ones, v[12], v[13]);
            csa(twosB, ones, ones, v[14], v[15]);
            csa(foursB, twos, twos, twosA, twosB);
            csa(eightsB, fours, fours, foursA, foursB);
            csa(sixteens, eights, eights, eightsA, eightsB);
            cnt.add(sixteens, 4);
        }
        for (; r < gsz; ++r) {
            // Remaining rows: add with weight 1 into the ones..eights slices.
            const W v = p[r * words];
            W carry = ones & v;
            ones ^= v;
            W t2 = twos & carry;
            twos ^= carry;
            carry = t2;
            t2 = fours & carry;
            fours ^= carry;
            carry = t2;
            t2 = eights & carry;
            eights ^= carry;
            carry = t2;
            cnt.add(carry, 4);
        }
        cnt.add(ones, 0);
        cnt.add(twos, 1);
        cnt.add(fours, 2);
        cnt.add(eights, 3);
        CountT* dst = lds + col * row_stride + cls;
        for (int bit = 0; bit < kBits; ++bit) dst[bit * kb] = CountT(cnt.count(bit));
    }
    __syncthreads();

    // Write [samples of this tile] x [kb classes]; consecutive threads write consecutive
    // classes of consecutive samples, so a tile with kb == k is one contiguous run.
    const int64_t s_base = col0 * kBits;
    const int64_t tile = int64_t(cols) * kBits * kb;
    const int kb_here = int(std::min<int64_t>(kb, k - c0));
    for (int64_t e = t; e < tile; e += kGbsThreads) {
        const int64_t sl = e / kb;
        const int cl = int(e % kb);
        const int64_t sample = s_base + sl;
        if (cl < kb_here && sample < n_valid) {
            const int64_t cc = sl / kBits, bit = sl % kBits;
            counts[sample * k + c0 + cl] = int32_t(lds[cc * row_stride + bit * kb + cl]);
        }
    }
}

template <typename W, int NB>
void launch_gbs(const W* x, int64_t words, int64_t gsz, int64_t k, int64_t n_valid,
                int32_t* counts, hipStream_t s) {
    constexpr int kBits = int(sizeof(W)) * 8;
    const size_t count_bytes = NB <= 16 ? 2 : 4;
    const int kb = int(std::min<int64_t>(k, kGbsMaxClasses));
    // Keep the LDS tile within 64 KiB (the default dynamic-LDS limit of a workgroup).
    const int lds_cols = int(65536 / ((kBits * kb + 1) * count_bytes));
    // Column tiles of whole 128-byte lines, so no cache line is split between workgroups.
    const int line_words = std::max(1, 128 / int(sizeof(W)));
    int cols = std::min(std::min(kGbsThreads / kb, lds_cols), CL_GBS_MAX_COLS);
    if (cols >= line_words) cols -= cols % line_words;
    const size_t lds = (size_t(cols) * (kBits * kb + 1) * count_bytes + 15) / 16 * 16;
    const dim3 grid(unsigned(ceil_div(words, cols)), unsigned(ceil_div(k, kb)), 1);
    k_group_bit_sum<W, NB><<<grid, kGbsThreads, lds, s>>>(x, words, gsz, k, n_valid, cols, kb,
                                                         counts);
}

// ------------------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_fill_splitmix64(uint64_t* __restrict__ out,
                                                         int64_t count, uint64_t base) {
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride)
        out[i] = splitmix64(base + uint64_t(i));
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_pack_bits(const uint8_t* t, int64_t rows, int64_t n, int32_t bit_count,
                            void* packed, int64_t* pad_len, void* stream) {
    clear_error();
    CL_REQUIRE(bit_count == 8 || bit_count == 16 || bit_count == 32 || bit_count == 64,
               CL_ERR_VALUE, "`bit_count` has to be in { 8, 16, 32, 64 }");
    CL_ARG(rows >= 0 && n >= 0, "negative shape");
    if (pad_len) *pad_len = (bit_count - n % bit_count) % bit_count;
    const int64_t words = ceil_div(n, bit_count);
    if (rows == 0 || words == 0) return CL_OK;
    CL_ARG(t && packed, "null pointer argument");
    hipStream_t s = as_stream(stream);
    const int64_t items = rows * words;
    const dim3 grid(unsigned(ceil_div(items, 256)), 1, 1);
    switch (bit_count) {
        case 8:
            k_pack_bits<uint8_t><<<grid, 256, 0, s>>>(t, rows, n, words, static_cast<uint8_t*>(packed));
            break;
        case 16:
            k_pack_bits<uint16_t><<<grid, 256, 0, s>>>(t, rows, n, words, static_cast<uint16_t*>(packed));
            break;
        case 32:
            k_pack_bits<uint32_t><<<grid, 256, 0, s>>>(t, rows, n, words, static_cast<uint32_t*>(packed));
            break;
        default:
            k_pack_bits<uint64_t><<<grid, 256, 0, s>>>(t, rows, n, words, static_cast<uint64_t*>(packed));
            break;
    }
    return check_launch("cl_pack_bits");
}

extern "C" int cl_dense_eval_packed(const void* x, const int64_t* a, const int64_t* b,
                                    const uint8_t* w_slot, const uint8_t* gate_seq, void* y,
                                    int64_t in_dim, int64_t out_dim, int64_t row_bytes,
                                    int64_t num_gates, void* stream) {
    clear_error();
    CL_ARG(in_dim >= 0 && out_dim >= 0 && row_bytes >= 0, "negative shape");
    CL_ARG(num_gates >= 1 && num_gates <= 128, "num_gates must be in [1, 128]");
    if (out_dim == 0 || row_bytes == 0) return CL_OK;
    CL_ARG(in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(x && a && b && w_slot && gate_seq && y, "null pointer argument");
    CL_ARG(ceil_div(out_dim, 4) < (int64_t(1) << 31), "too many rows");
    hipStream_t s = as_stream(stream);
    const int G = int(num_gates);
    const unsigned gx = unsigned(ceil_div(out_dim, 4));
    if (row_bytes % 16 == 0 && aligned(x, 16) && aligned(y, 16)) {
        constexpr int VEC = 2, U = kPackedU;
        const int64_t words = row_bytes / 8;
        const dim3 grid(gx, unsigned(ceil_div(words, 64 * VEC * U)), 1);
        k_eval_packed<uint64_t, VEC, U><<<grid, 256, 0, s>>>(
            static_cast<const uint64_t*>(x), a, b, w_slot, gate_seq, static_cast<uint64_t*>(y),
            in_dim, out_dim, words, G);
    } else if (row_bytes % 8 == 0 && aligned(x, 8) && aligned(y, 8)) {
        constexpr int VEC = 1, U = 8;
        const int64_t words = row_bytes / 8;
        const dim3 grid(gx, unsigned(ceil_div(words, 64 * VEC * U)), 1);
        k_eval_packed<uint64_t, VEC, U><<<grid, 256, 0, s>>>(
            static_cast<const uint64_t*>(x), a, b, w_slot, gate_seq, static_cast<uint64_t*>(y),
            in_dim, out_dim, words, G);
    } else {
        constexpr int VEC = 1, U = 8;
        const dim3 grid(gx, unsigned(ceil_div(row_bytes, 64 * VEC * U)), 1);
        k_eval_packed<uint8_t, VEC, U><<<grid, 256, 0, s>>>(
            static_cast<const uint8_t*>(x), a, b, w_slot, gate_seq, static_cast<uint8_t*>(y),
            in_dim, out_dim, row_bytes, G);
    }
    return check_launch("cl_dense_eval_packed");
}

extern "C" int cl_group_bit_sum(const void* packed, int64_t rows, int64_t row_bytes,
                                int64_t pad_len, int64_t k, int32_t* counts, void* stream) {
    clear_error();
    CL_ARG(rows >= 0 && row_bytes >= 0 && pad_len >= 0, "negative shape");
    CL_ARG(k >= 1, "k must be >= 1");
    CL_REQUIRE(rows % k == 0, CL_ERR_VALUE,
               "in_dim (%lld) has to be divisible by k (%lld) but it is not", (long long)rows,
               (long long)k);
    const int64_t n_valid = row_bytes * 8 - pad_len;
    CL_ARG(n_valid >= 0, "pad_len exceeds the packed length");
    if (n_valid == 0) return CL_OK;
    CL_ARG(packed && counts, "null pointer argument");
    const int64_t gsz = rows / k;
    CL_ARG(gsz < (int64_t(1) << 31), "group too large");
    hipStream_t s = as_stream(stream);
    if (row_bytes % 8 == 0 && aligned(packed, 8)) {
        const auto* x = static_cast<const uint64_t*>(packed);
        const int64_t words = row_bytes / 8;
        if (gsz < (1 << 16))
            launch_gbs<uint64_t, 16>(x, words, gsz, k, n_valid, counts, s);
        else
            launch_gbs<uint64_t, 32>(x, words, gsz, k, n_valid, counts, s);
    } else {
        const auto* x = static_cast<const uint8_t*>(packed);
        if (gsz < (1 << 16))
            launch_gbs<uint8_t, 16>(x, row_bytes, gsz, k, n_valid, counts, s);
        else
            launch_gbs<uint8_t, 32>(x, row_bytes, gsz, k, n_valid, counts, s);
    }
    return check_launch("cl_group_bit_sum");
}

extern "C" int cl_fill_splitmix64(uint64_t* out, int64_t count, uint64_t base, void* stream) {
    clear_error();
    CL_ARG(count >= 0, "negative count");
    if (count == 0) return CL_OK;
    CL_ARG(out, "null pointer argument");
    const int64_t blocks = std::min<int64_t>(ceil_div(count, 256), 1 << 20);
    k_fill_splitmix64<<<unsigned(blocks), 256, 0, as_stream(stream)>>>(out, count, base);
    return check_launch("cl_fill_splitmix64");
}
