// Whole-network packed inference for gfx950: every layer of a frozen dense network and the
// popcount GroupSum in one launch, with the activations of a 32-sample column held in LDS.
//
// The layer-by-layer path writes every layer's packed output to HBM and reads it back
// (F bytes / 8 per sample per layer, both ways).  Here a workgroup takes one 32-bit column of
// the packed input (32 samples), keeps the current layer's rows in LDS (one 32-bit word per
// row) and evaluates the next layer from them: gate o reads rows a_o and b_o of the previous
// layer from LDS and writes row o of the next.  The only HBM traffic is the input column and
// the class counts; the gate tables (8 bytes per gate) stay in L2, shared by all workgroups.
//
// Gate table entry (uint64): bits 0-19 byte offset of row a (4 * a), 20-39 that of row b,
// 40-43 opcode.  The opcode's truth table selects the result per bit with three bit-field
// inserts:
//     r = b ? (a ? f11 : f01) : (a ? f10 : f00)
// with f_xy the all-ones / all-zero masks of the truth-table entries (v_bfe_i32 of the opcode).
//
// Class counts: rows c*gs .. c*gs+gs-1 form class c.  Each class's rows are split into
// slices, one thread per slice; a thread adds its slice's words into NB-bit bit-sliced
// vertical counters (carry-save), and every (sample, class) count is then assembled from the
// slices' counter words by several threads whose partial sums are added at the end.  Integer
// sums: the result is exact and independent of the order.
#include "common.h"

#include <algorithm>

namespace cl {
namespace {

constexpr int kNetThreads = 1024;
constexpr int kNetMaxLayers = 16;
constexpr int kMaxCountBits = 12;  // vertical counter width: at most 4095 rows per slice
#ifndef CL_NET_NO_REGS
#define CL_NET_NO_REGS 0
#endif
constexpr bool kNetDisableRegs = CL_NET_NO_REGS;  // force the one-column-per-block kernel

struct PackedNet {
    int num_layers;
    int k;
    int slices;             // slices per class
    int rows[kNetMaxLayers + 1];
    int64_t table_off[kNetMaxLayers];
};

__device__ __forceinline__ uint32_t gate_word(uint32_t g, uint32_t a, uint32_t b) {
    // truth-table bits of opcode g, MSB first over AB = 00, 01, 10, 11
    const uint32_t f00 = uint32_t(__builtin_amdgcn_sbfe(int(g), 3, 1));
    const uint32_t f01 = uint32_t(__builtin_amdgcn_sbfe(int(g), 2, 1));
    const uint32_t f10 = uint32_t(__builtin_amdgcn_sbfe(int(g), 1, 1));
    const uint32_t f11 = uint32_t(__builtin_amdgcn_sbfe(int(g), 0, 1));
    const uint32_t hi = (a & f11) | (~a & f01);  // b = 1
    const uint32_t lo = (a & f10) | (~a & f00);  // b = 0
    return (b & hi) | (~b & lo);
}

template <int NB>
__device__ __forceinline__ void add_vertical(uint32_t (&v)[NB], uint32_t x) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint32_t carry = v[b] & x;
        v[b] ^= x;
        x = carry;
    }
}

// Column of the workgroup: XCD x (= w % 8) takes a contiguous range of columns, so the
// workgroups resident on one XCD read neighbouring 4-byte words of every input row and share
// their cache lines in that XCD's L2.
__device__ __forceinline__ int64_t net_column(int64_t w, int64_t cols) {
    const int64_t per = (cols + 7) / 8;
    return (w % 8) * per + w / 8;
}

template <int NB>
__global__ __launch_bounds__(kNetThreads) void k_packed_net(const uint32_t* __restrict__ x,
                                                            int64_t cols, int64_t nsamples,
                                                            const uint64_t* __restrict__ tables,
                                                            PackedNet net,
                                                            int32_t* __restrict__ counts,
                                                            int buf_words) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int64_t col = net_column(blockIdx.x, cols);
    if (col >= cols) return;  // uniform per block
    uint32_t* cur = lds;
    uint32_t* nxt = lds + buf_words;
    const int tid = threadIdx.x;
    for (int r = tid; r < net.rows[0]; r += kNetThreads) cur[r] = x[int64_t(r) * cols + col];
    __syncthreads();
    for (int l = 0; l < net.num_layers; ++l) {
        const uint64_t* t = tables + net.table_off[l];
        const int out = net.rows[l + 1];
        const unsigned char* src = reinterpret_cast<const unsigned char*>(cur);
        for (int o = tid; o < out; o += kNetThreads) {
            const uint64_t e = t[o];
            const uint32_t lo = uint32_t(e), hi = uint32_t(e >> 32);
            const uint32_t a = *reinterpret_cast<const uint32_t*>(src + (lo & 0xfffffu));
            const uint32_t b = *reinterpret_cast<const uint32_t*>(
                src + __builtin_amdgcn_ubfe(uint32_t(e >> 20), 0, 20));
            nxt[o] = gate_word(__builtin_amdgcn_ubfe(hi, 8, 4), a, b);
        }
        __syncthreads();
        uint32_t* s = cur;
        cur = nxt;
        nxt = s;
    }
    // class counts of the 32 samples of this column
    const int rows = net.rows[net.num_layers];
    const int gs = rows / net.k;
    const int S = net.slices;
    uint32_t* vc = nxt;                      // [k * S][NB] vertical counters
    int32_t* part = reinterpret_cast<int32_t*>(nxt + net.k * S * NB);  // [P][32 k] partials
    if (tid < net.k * S) {
        const int c = tid / S, j = tid % S;
        uint32_t v[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) v[b] = 0;
        for (int r = c * gs + j; r < (c + 1) * gs; r += S) add_vertical<NB>(v, cur[r]);
#pragma unroll
        for (int b = 0; b < NB; ++b) vc[tid * NB + b] = v[b];
    }
    __syncthreads();
    const int pairs = 32 * net.k;
    const int P = std::max(1, kNetThreads / pairs);  // threads per (sample, class) pair
    if (tid < pairs * P) {
        const int i = tid % pairs, p = tid / pairs;
        const int smp = i / net.k, c = i % net.k;
        int32_t n = 0;
        for (int j = p; j < S; j += P) {
            const uint32_t* vv = vc + (c * S + j) * NB;
#pragma unroll
            for (int b = 0; b < NB; ++b) n += int32_t((vv[b] >> smp) & 1u) << b;
        }
        part[p * pairs + i] = n;
    }
    __syncthreads();
    for (int i = tid; i < pairs; i += kNetThreads) {
        int32_t n = 0;
        for (int p = 0; p < P; ++p) n += part[p * pairs + i];
        const int64_t sample = col * 32 + i / net.k;
        if (sample < nsamples) counts[sample * net.k + i % net.k] = n;
    }
}

// ------------------------------------------------------------------------------------------
// Persistent variant for networks whose layers are at most 16383 rows wide and whose gates
// fit in TG registers per thread: every thread keeps its gates (the LDS byte offsets of both
// inputs, 16 bits each, and the opcode) in registers for the whole launch, so the gate
// tables are read once per workgroup instead of once per column, and each workgroup walks a
// range of columns, loading the next column's input words while it evaluates the current one.
constexpr int kSlotCap = 80;  // gate slots per thread (registers)

// Bit-sliced addition of the partner lane's number to this lane's: a += partner(a), W words
// (word i holds bit i of 32 counts), the sum fitting in W bits.  Each word is fetched from
// the partner inside the carry loop: all lanes fetch word i before any lane updates it, so
// one temporary register suffices.
// Only the low N words can be non-zero in either addend (N <= W).
template <int CTRL, int N, int W>
__device__ __forceinline__ void bs_add_dpp(uint32_t (&a)[W]) {
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t x = a[i], y = dpp_move<CTRL>(x);
        a[i] = x ^ y ^ c;
        c = (x & y) | (c & (x | y));
    }
}

template <int N, int W>
__device__ __forceinline__ void bs_add_xor(uint32_t (&a)[W], int d) {
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint32_t x = a[i], y = uint32_t(__shfl_xor(int(x), d, 64));
        a[i] = x ^ y ^ c;
        c = (x & y) | (c & (x | y));
    }
}

// Class counts of one column, one wave per class: lane l adds rows l, l + 64, ... of the
// class into (W - 6)-bit vertical counters, six butterfly steps of bit-sliced addition (DPP
// inside each 16-lane row, then lane shuffles across rows) leave the class total of all 32
// samples in every lane as W bit planes, and lane s < 32 reads off the count of sample s.
// Requires gs <= 2^W - 64 (per-lane counts fit W - 6 bits, the total W bits).  Integer sums:
// exact and independent of the order.
template <int W>
__device__ __forceinline__ void column_counts_wave(const uint32_t* last, const PackedNet& net,
                                                   int64_t col, int64_t nsamples,
                                                   int32_t* __restrict__ counts) {
    constexpr int LW = W - 6;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gs = net.rows[net.num_layers] / net.k;
    for (int c = wave; c < net.k; c += kNetThreads / 64) {  // uniform per wave
        uint32_t a[W];
#pragma unroll
        for (int i = 0; i < W; ++i) a[i] = 0;
#pragma unroll 1
        for (int r = c * gs + lane; r < (c + 1) * gs; r += 64) {
            // add one row's bits into the low LW words (per-lane counts stay below 2^LW)
            uint32_t x = last[r];
#pragma unroll
            for (int i = 0; i < LW; ++i) {
                const uint32_t carry = a[i] & x;
                a[i] ^= x;
                x = carry;
            }
        }
        // after step k the sums have at most LW + k bits: each step carries one word further
        constexpr auto n = [](int k) { return LW + k < W ? LW + k : W; };
        bs_add_dpp<0xB1, n(1)>(a);   // quad_perm [1,0,3,2]
        bs_add_dpp<0x4E, n(2)>(a);   // quad_perm [2,3,0,1]
        bs_add_dpp<0x124, n(3)>(a);  // row_ror:4
        bs_add_dpp<0x128, n(4)>(a);  // row_ror:8
        bs_add_xor<n(5)>(a, 16);
        bs_add_xor<n(6)>(a, 32);
        if (lane < 32) {
            int32_t n = 0;
#pragma unroll
            for (int i = 0; i < W; ++i) n |= int32_t((a[i] >> lane) & 1u) << i;
            const int64_t sample = col * 32 + lane;
            if (sample < nsamples) counts[sample * net.k + c] = n;
        }
    }
}

// k_packed_net_slots: persistent workgroups (columns col, col + gridDim/8, ... on XCD
// blockIdx % 8, a contiguous range of columns per XCD) with the gate tables in registers.
// Every layer owns J slots of a thread: slot q = l * J + j is gate row tid + 1024 j of layer
// l, so the layer of a slot, its output row and the LDS buffer it reads (l even: the first,
// odd: the second) are compile-time constants.  A layer issues the 2J row reads of its gates
// before computing them, then writes the J outputs, then meets the barrier.  Gate entry in a
// register: byte offset of row a | that of row b << 16 (rows < 16384); opcodes as nibbles.
// Slots past a layer's width hold entry 0: they read row 0 and write rows at or beyond the
// width, which no later step reads (each buffer spans at least 1024 J words), so no slot
// needs a branch.
#ifndef CL_NET_BATCH
#define CL_NET_BATCH 4
#endif
constexpr int kBatch = CL_NET_BATCH;  // gates whose row reads are in flight together

template <int CW, int J, int IPT>
__global__ __launch_bounds__(kNetThreads) void k_packed_net_slots(
    const uint32_t* __restrict__ x, int64_t cols, int64_t nsamples,
    const uint64_t* __restrict__ tables, PackedNet net, int32_t* __restrict__ counts,
    int buf_words) {
    constexpr int LMAX = kSlotCap / J < kNetMaxLayers ? kSlotCap / J : kNetMaxLayers;
    constexpr int TG = LMAX * J;
    extern __shared__ __align__(16) uint32_t lds[];
    const int tid = threadIdx.x;
    const int L = net.num_layers;
    uint32_t ent[TG];
    uint32_t ops[(TG + 7) / 8];
#pragma unroll
    for (int i = 0; i < (TG + 7) / 8; ++i) ops[i] = 0;
#pragma unroll
    for (int q = 0; q < TG; ++q) {
        const int l = q / J, o = tid + kNetThreads * (q % J);
        ent[q] = 0;  // no gate in this slot: reads row 0, writes past the layer's rows
        if (l < L && o < net.rows[l + 1]) {
            const uint64_t e = tables[net.table_off[l] + o];
            ent[q] = (uint32_t(e) & 0xffffu) | (__builtin_amdgcn_ubfe(uint32_t(e >> 20), 0, 16) << 16);
            ops[q / 8] |= __builtin_amdgcn_ubfe(uint32_t(e >> 32), 8, 4) << (4 * (q % 8));
        }
    }
    const int64_t per = (cols + 7) / 8;
    const int64_t nb8 = gridDim.x / 8;
    const int64_t c_first = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int64_t c_end = std::min(cols, (blockIdx.x % 8 + 1) * per);
    uint32_t in[IPT];
    auto fetch = [&](int64_t c) {
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int r = tid + kNetThreads * j;
            in[j] = (c < c_end && r < net.rows[0]) ? x[int64_t(r) * cols + c] : 0u;
        }
    };
    fetch(c_first);
    for (int64_t col = c_first; col < c_end; col += nb8) {
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int r = tid + kNetThreads * j;
            if (r < net.rows[0]) lds[r] = in[j];
        }
        fetch(col + nb8);
        __syncthreads();
        // The gate entries and opcode words are made opaque for every column: keeps the
        // compiler from hoisting per-gate values derived from them (the two LDS addresses,
        // the four truth-table masks) out of the column loop, which would need up to six more
        // registers per gate.
#pragma unroll
        for (int i = 0; i < (TG + 7) / 8; ++i) asm volatile("" : "+v"(ops[i]));
#pragma unroll
        for (int q = 0; q < TG; ++q) asm volatile("" : "+v"(ent[q]));
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            if (l < L) {  // uniform
                const unsigned char* cur =
                    reinterpret_cast<const unsigned char*>(lds + (l & 1) * buf_words);
                uint32_t* nxt = lds + ((l + 1) & 1) * buf_words;
                // the row reads of kBatch gates are issued together, then the gates computed
#pragma unroll
                for (int j0 = 0; j0 < J; j0 += kBatch) {
                    uint32_t va[kBatch], vb[kBatch];
#pragma unroll
                    for (int j = j0; j < j0 + kBatch && j < J; ++j) {
                        const uint32_t e = ent[l * J + j];
                        va[j - j0] = *reinterpret_cast<const uint32_t*>(cur + (e & 0xffffu));
                        vb[j - j0] = *reinterpret_cast<const uint32_t*>(cur + (e >> 16));
                    }
#pragma unroll
                    for (int j = j0; j < j0 + kBatch && j < J; ++j) {
                        const int q = l * J + j;
                        nxt[tid + kNetThreads * j] = gate_word(
                            (ops[q / 8] >> (4 * (q % 8))) & 15u, va[j - j0], vb[j - j0]);
                    }
                }
                __syncthreads();
            }
        }
        // the last layer's rows are in buffer L % 2
        column_counts_wave<CW>(lds + (L & 1) * buf_words, net, col, nsamples, counts);
        __syncthreads();  // the next column overwrites both buffers
    }
}

}  // namespace
}  // namespace cl

using namespace cl;

extern "C" int cl_packed_network_limits(int64_t* max_layers, int64_t* max_rows) {
    clear_error();
    CL_ARG(max_layers && max_rows, "null pointer argument");
    *max_layers = kNetMaxLayers;
    // two row buffers of 32-bit words within 160 KiB of LDS
    *max_rows = (160 * 1024) / (2 * 4);
    return CL_OK;
}

extern "C" int cl_packed_network(const void* x, int64_t row_bytes, int64_t nsamples,
                                 const uint64_t* tables, const int64_t* rows_host,
                                 int64_t num_layers, int64_t k, int32_t* counts, void* stream) {
    clear_error();
    CL_ARG(num_layers >= 1 && num_layers <= kNetMaxLayers, "1 to %d layers", kNetMaxLayers);
    CL_ARG(rows_host && k >= 1, "bad arguments");
    CL_ARG(row_bytes >= 0 && row_bytes % 4 == 0, "packed rows must be a multiple of 4 bytes");
    CL_ARG(nsamples >= 0 && nsamples <= row_bytes * 8, "more samples than packed bits");
    PackedNet net{};
    net.num_layers = int(num_layers);
    net.k = int(k);
    int max_rows = 0;
    int64_t off = 0;
    for (int l = 0; l <= num_layers; ++l) {
        const int64_t r = rows_host[l];
        CL_ARG(r >= 1 && r <= 20480, "layer widths must be in [1, 20480] for the fused pass");
        net.rows[l] = int(r);
        max_rows = std::max(max_rows, int(r));
        if (l < num_layers) {
            net.table_off[l] = off;
            off += rows_host[l + 1];
        }
    }
    const int last = net.rows[num_layers];
    if (last % k != 0) {
        set_error("in_dim (%d) has to be divisible by k (%lld) but it is not", last, (long long)k);
        return CL_ERR_VALUE;
    }
    // slices per class: one thread each, as many as fit
    const int gs = last / int(k);
    CL_ARG(int(k) <= kNetThreads, "k must be at most %d for the fused pass", kNetThreads);
    const int S = std::max(1, std::min(kNetThreads / int(k), gs));
    const int per_slice = int(ceil_div(gs, S));
    int NB = 1;
    while ((1 << NB) <= per_slice) ++NB;
    NB = NB <= 4 ? 4 : (NB <= 8 ? 8 : NB);
    CL_ARG(NB <= kMaxCountBits, "class groups too large for the fused pass");
    net.slices = S;
    const int pairs = 32 * int(k);
    const int P = std::max(1, kNetThreads / pairs);
    const int count_words = int(k) * S * NB + P * pairs;
    int buf_words = std::max(max_rows, count_words);
    size_t lds = size_t(2) * buf_words * 4;
    CL_ARG(lds <= 160 * 1024, "activations do not fit in LDS");
    const int64_t cols = row_bytes / 4;
    if (nsamples == 0 || cols == 0) return CL_OK;
    CL_ARG(x && tables && counts, "null pointer argument");
    CL_ARG(aligned(x, 4) && aligned(tables, 8), "misaligned buffers");
    const int64_t blocks = 8 * ceil_div(cols, 8);
    CL_ARG(blocks < (int64_t(1) << 31), "too many columns");
    int rc = CL_OK;
    // persistent slot-table variant when it applies: J slots of 1024 rows per layer
    int J = int(ceil_div(int64_t(*std::max_element(net.rows + 1, net.rows + num_layers + 1)),
                         int64_t(kNetThreads)));
    for (int cand : {1, 2, 4, 8, 12, 16}) {
        if (J <= cand) {
            J = cand;
            break;
        }
    }
    const bool slots = max_rows <= 16383 && net.rows[0] <= 4 * kNetThreads && J <= 16 &&
                       num_layers <= std::min(kSlotCap / J, kNetMaxLayers);
    if (slots && !kNetDisableRegs) {
        // every slot writes: a buffer spans the J * 1024 rows a thread's slots can address
        buf_words = std::max(buf_words, J * kNetThreads);
        lds = size_t(2) * buf_words * 4;
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            set_error("cannot query the device");
            return CL_ERR_HIP;
        }
        const int64_t want = std::max<int64_t>(8, (int64_t(cus) / 8) * 8);
        const int64_t pblocks = std::min<int64_t>(want, 8 * ceil_div(cols, 8));
        auto go = [&](auto nb, auto jc, auto ipt) {
            auto* kern = &k_packed_net_slots<decltype(nb)::value, decltype(jc)::value,
                                             decltype(ipt)::value>;
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) !=
                hipSuccess) {
                set_error("cannot reserve %zu bytes of LDS for the fused pass", lds);
                rc = CL_ERR_HIP;
                return;
            }
            kern<<<unsigned(pblocks), kNetThreads, lds, as_stream(stream)>>>(
                static_cast<const uint32_t*>(x), cols, nsamples, tables, net, counts, buf_words);
        };
        auto by_j = [&](auto nb, auto ipt) {
            using std::integral_constant;
            switch (J) {
                case 1: go(nb, integral_constant<int, 1>(), ipt); break;
                case 2: go(nb, integral_constant<int, 2>(), ipt); break;
                case 4: go(nb, integral_constant<int, 4>(), ipt); break;
                case 8: go(nb, integral_constant<int, 8>(), ipt); break;
                case 12: go(nb, integral_constant<int, 12>(), ipt); break;
                default: go(nb, integral_constant<int, 16>(), ipt); break;
            }
        };
        auto by_ipt = [&](auto nb) {
            if (net.rows[0] <= kNetThreads) by_j(nb, std::integral_constant<int, 1>());
            else by_j(nb, std::integral_constant<int, 4>());
        };
        // count width: gs <= 2^CW - 64
        if (gs <= 192) by_ipt(std::integral_constant<int, 8>());
        else if (gs <= 960) by_ipt(std::integral_constant<int, 10>());
        else if (gs <= 4032) by_ipt(std::integral_constant<int, 12>());
        else by_ipt(std::integral_constant<int, 15>());
        if (rc) return rc;
        return check_launch("cl_packed_network");
    }
    auto launch = [&](auto nb) {
        auto* kern = &k_packed_net<decltype(nb)::value>;
        // more than the default 64 KiB of dynamic LDS per workgroup
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess) {
            set_error("cannot reserve %zu bytes of LDS for the fused pass", lds);
            rc = CL_ERR_HIP;
            return;
        }
        kern<<<unsigned(blocks), kNetThreads, lds, as_stream(stream)>>>(
            static_cast<const uint32_t*>(x), cols, nsamples, tables, net, counts, buf_words);
    };
    if (NB == 4) launch(std::integral_constant<int, 4>());
    else if (NB == 8) launch(std::integral_constant<int, 8>());
    else launch(std::integral_constant<int, kMaxCountBits>());
    if (rc) return rc;
    return check_launch("cl_packed_network");
}
