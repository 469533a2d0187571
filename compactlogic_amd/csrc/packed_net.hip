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
constexpr int kSlotCap = 72;  // gate slots per thread (registers)

// Exchange with lane l ^ K inside each 32-lane half of the wave.
template <int K>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (K == 1) return dpp_move<0xB1>(v);         // quad_perm [1,0,3,2]
    else if constexpr (K == 2) return dpp_move<0x4E>(v);    // quad_perm [2,3,0,1]
    else if constexpr (K == 8) return dpp_move<0x128>(v);   // row_ror:8
    else return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), (K << 10) | 0x1F));  // xor mode
}

// One stage of the 32 x 32 bit transpose across a half-wave (row = lane, column = bit): lanes
// l and l ^ K swap the off-diagonal K x K blocks of every 2K x 2K block.  The lane with bit K
// clear keeps its columns c with c & K == 0 and takes the partner's same columns shifted up by
// K; the other keeps c & K != 0 and takes the partner's shifted down.  A rotation by K or
// 32 - K moves the wanted bits into place for either lane (the bits it wraps round are masked).
template <int K>
__device__ __forceinline__ uint32_t transpose_stage(uint32_t t, int lane) {
    constexpr uint32_t m = K == 16 ? 0x0000FFFFu
                           : K == 8 ? 0x00FF00FFu
                           : K == 4 ? 0x0F0F0F0Fu
                           : K == 2 ? 0x33333333u
                                    : 0x55555555u;  // columns c with c & K == 0
    const bool low = (lane & K) == 0;
    const uint32_t p = xor_lane<K>(t);
    const uint32_t sh = __builtin_amdgcn_alignbit(p, p, low ? 32 - K : K);  // rotate right
    const uint32_t keep = low ? m : ~m;
    return (t & keep) | (sh & ~keep);
}

// Adds the 1-bit numbers of x into the bit planes a[I..B) (a ripple of half adders).
template <int I, int B>
__device__ __forceinline__ void add_planes(uint32_t (&a)[B], uint32_t x) {
#pragma unroll
    for (int i = I; i < B; ++i) {
        const uint32_t carry = a[i] & x;
        a[i] ^= x;
        x = carry;
    }
}

// Full adder on bit planes: a, carry = a + x + y (sum bit and carry bit per sample).
__device__ __forceinline__ uint32_t full_add(uint32_t& a, uint32_t x, uint32_t y) {
    const uint32_t carry = (a & x) | (a & y) | (x & y);
    a ^= x ^ y;
    return carry;
}

// Class counts of one column, one wave per class.  Lane l adds rows l, l + 64, ... of the
// class into B bit planes (bit s of plane b = bit b of its count for sample s; four rows per
// step through three full adders); the lane's count is at most ceil(gs / 64) < 2^B.  Each
// plane, read across a half-wave, is a 32 x 32 bit matrix (row = lane, column = sample); five
// exchange stages transpose it, after which lane j holds column j and one popcount sums the
// plane over the half-wave's 32 lanes for sample j.  The two half-waves' sums are added.
// Integer sums: exact and independent of the order.
template <int B>
__device__ __forceinline__ void column_counts_wave(const uint32_t* last, int gs, int k,
                                                   int64_t col, int64_t nsamples,
                                                   int32_t* __restrict__ counts) {
    const int lane = threadIdx.x & 63;
    for (int c = wave_id(); c < k; c += kNetThreads / 64) {  // uniform per wave
        uint32_t a[B];
#pragma unroll
        for (int i = 0; i < B; ++i) a[i] = 0;
        const int end = (c + 1) * gs;
        int r = c * gs + lane;
#pragma unroll 1
        for (; r + 192 < end; r += 256) {
            const uint32_t x0 = last[r], x1 = last[r + 64], x2 = last[r + 128], x3 = last[r + 192];
            const uint32_t c1 = full_add(a[0], x0, x1);
            const uint32_t c2 = full_add(a[0], x2, x3);
            add_planes<2>(a, full_add(a[1], c1, c2));
        }
#pragma unroll 1
        for (; r < end; r += 64) add_planes<0>(a, last[r]);
        int32_t n = 0;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            uint32_t t = a[b];
            t = transpose_stage<16>(t, lane);
            t = transpose_stage<8>(t, lane);
            t = transpose_stage<4>(t, lane);
            t = transpose_stage<2>(t, lane);
            t = transpose_stage<1>(t, lane);
            n += int32_t(__builtin_popcount(t)) << b;
        }
        n += __shfl_xor(n, 32, 64);  // the other half-wave's rows
        if (lane < 32) {
            const int64_t sample = col * 32 + lane;
            if (sample < nsamples) counts[sample * k + c] = n;
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

// With J <= 12 the opcode nibbles live in LDS after the two row buffers (word i of thread t
// at i * 1024 + t, conflict-free), not in registers: with 1024-thread workgroups a wave has
// at most 128 VGPRs, and the gate entries alone take up to 72 of them.  A layer loads the two
// or three opcode words of its slots when it starts.  (Two buffers of 16 * 1024 rows leave no
// room for them: with J = 16 they stay in registers, next to 64 entries.)
constexpr int kOpsLdsMaxJ = 12;

template <int B, int J, int IPT>
__global__ __launch_bounds__(kNetThreads) void k_packed_net_slots(
    const uint32_t* __restrict__ x, int64_t cols, int64_t nsamples,
    const uint64_t* __restrict__ tables, PackedNet net, int32_t* __restrict__ counts,
    int buf_words) {
    constexpr int LMAX = kSlotCap / J < kNetMaxLayers ? kSlotCap / J : kNetMaxLayers;
    constexpr int TG = LMAX * J;
    constexpr int OW = (TG + 7) / 8;
    constexpr bool OPSL = J <= kOpsLdsMaxJ;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t* ops_lds = lds + 2 * buf_words;
    const int tid = threadIdx.x;
    const int L = net.num_layers;
    uint32_t ent[TG];
    uint32_t ops[OW];
#pragma unroll
    for (int i = 0; i < OW; ++i) ops[i] = 0;
#pragma unroll
    for (int q = 0; q < TG; ++q) {
        const int l = q / J, o = tid + kNetThreads * (q % J);
        // no gate in this slot: entry 0 reads row 0 and writes past the layer's rows
        const bool gate = l < L && o < net.rows[l + 1];
        uint64_t e = 0;
        if constexpr (TG <= 16) {
            // selects, not branches: a conditionally assigned array this small becomes one
            // vector register tuple, copied whole at every branch
            e = tables[gate ? net.table_off[l] + o : 0];
            e = gate ? e : 0;
        } else {
            if (gate) e = tables[net.table_off[l] + o];
        }
        ent[q] = 0;
        if (TG <= 16 || gate) {
            ent[q] = (uint32_t(e) & 0xffffu) | (__builtin_amdgcn_ubfe(uint32_t(e >> 20), 0, 16) << 16);
            ops[q / 8] |= __builtin_amdgcn_ubfe(uint32_t(e >> 32), 8, 4) << (4 * (q % 8));
        }
    }
    if constexpr (OPSL) {
#pragma unroll
        for (int i = 0; i < OW; ++i) ops_lds[i * kNetThreads + tid] = ops[i];
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
        if constexpr (!OPSL) {
#pragma unroll
            for (int i = 0; i < OW; ++i) asm volatile("" : "+v"(ops[i]));
        }
#pragma unroll
        for (int q = 0; q < TG; ++q) asm volatile("" : "+v"(ent[q]));
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            if (l < L) {  // uniform
                const unsigned char* cur =
                    reinterpret_cast<const unsigned char*>(lds + (l & 1) * buf_words);
                uint32_t* nxt = lds + ((l + 1) & 1) * buf_words;
                // the opcode words of this layer's slots (a constant range once unrolled)
                constexpr int NW = (J + 7) / 8 + 1;
                const int wlo = (l * J) / 8;
                uint32_t lw[NW];
#pragma unroll
                for (int i = 0; i < NW; ++i) {
                    const int wi = wlo + i < OW ? wlo + i : OW - 1;
                    lw[i] = OPSL ? ops_lds[wi * kNetThreads + tid] : ops[wi];
                }
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
                            (lw[q / 8 - wlo] >> (4 * (q % 8))) & 15u, va[j - j0], vb[j - j0]);
                    }
                }
                __syncthreads();
            }
        }
        // the last layer's rows are in buffer L % 2
        column_counts_wave<B>(lds + (L & 1) * buf_words, net.rows[L] / net.k, net.k, col,
                              nsamples, counts);
        __syncthreads();  // the next column overwrites both buffers
    }
}

// ------------------------------------------------------------------------------------------
// Wide-input fused pass.  An input wider than four rows per thread comes column-major: the
// words of column c are x[c * in_words + r] for rows r < in_words (k_eval_packed_cols writes
// this layout), so a workgroup loads its column with coalesced 16-byte loads however many
// rows the input has, where the row-major layout would pull a cache line per row for 4 bytes.
// LDS holds the column at words [0, in_words).  The first layer writes its slots
// j < J - HOLD to base[0] + tid + 1024 j, after the input, and keeps its last HOLD slots in
// registers until every thread has read the input; they then go to hold_base + 1024 h + tid,
// over the input.  Later layers write to base[l] + tid + 1024 j.  Gate entries hold absolute
// LDS word addresses (16 bits each), so the host can place each layer's rows anywhere in the
// 160 KiB (cols_plan) and builds the entries to match; the input's LDS words cannot hold
// both it and a full first layer when the input passes 24576 rows.
constexpr int kLdsWords = 40960;  // 160 KiB of LDS per workgroup

// Layers the gate-entry registers hold: 2 of 16 slots or 3 of 8 (with the input loads in
// flight beside them, more entries spill).
constexpr int cols_max_layers(int J) { return J == 16 ? 2 : 3; }

struct PackedNetCols {
    int num_layers;
    int k;
    int rows[kNetMaxLayers + 1];
    int64_t table_off[kNetMaxLayers];
    int base[kNetMaxLayers];  // LDS word of layer l's slot 0 (layer 0: its unheld slots)
    int hold_base;            // LDS word of layer 0's first held slot
    int in_words;             // words per input column, a multiple of 64
};

// 16-byte loads per thread that stage the widest input a plan with J - HOLD unheld
// first-layer slots admits
template <int J, int HOLD>
constexpr int cols_in_loads() {
    return (kLdsWords - kNetThreads * (J - HOLD) + 4 * kNetThreads - 1) / (4 * kNetThreads);
}

// Persistent like k_packed_net_slots (columns of one XCD contiguous, gate entries and opcodes
// in registers, the next column's input loaded while the current one is evaluated).  Entry
// register: LDS word of row a | that of row b << 16; opcodes as nibbles.
template <int B, int J, int HOLD>
__global__ __launch_bounds__(kNetThreads) void k_packed_net_cols(
    const uint4* __restrict__ x, int64_t cols, int64_t nsamples,
    const uint64_t* __restrict__ tables, PackedNetCols net, int32_t* __restrict__ counts) {
    constexpr int LMAX = cols_max_layers(J);
    constexpr int TG = LMAX * J;
    constexpr int OW = (TG + 7) / 8;
    constexpr int JB = J - HOLD;
    constexpr int IPT = cols_in_loads<J, HOLD>();
    extern __shared__ __align__(16) uint32_t lds[];
    const int tid = threadIdx.x;
    const int L = net.num_layers;
    uint32_t ent[TG];
    uint32_t ops[OW];
#pragma unroll
    for (int i = 0; i < OW; ++i) ops[i] = 0;
#pragma unroll
    for (int q = 0; q < TG; ++q) {
        // no gate in this slot: entry 0 reads word 0 and writes a row no later step reads
        const int l = q / J, o = tid + kNetThreads * (q % J);
        uint64_t e = 0;
        if (l < L && o < net.rows[l + 1]) e = tables[net.table_off[l] + o];
        ent[q] = uint32_t(e);
        ops[q / 8] |= (uint32_t(e >> 32) & 15u) << (4 * (q % 8));
    }
    const int in4 = net.in_words / 4;
    const int64_t per = (cols + 7) / 8;
    const int64_t nb8 = gridDim.x / 8;
    const int64_t c_first = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int64_t c_end = std::min(cols, (blockIdx.x % 8 + 1) * per);
    uint4 in[IPT];
    auto fetch = [&](int64_t c) {
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int i = tid + kNetThreads * j;
            in[j] = (c < c_end && i < in4) ? x[c * in4 + i] : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    fetch(c_first);
    for (int64_t col = c_first; col < c_end; col += nb8) {
        uint4* l4 = reinterpret_cast<uint4*>(lds);
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int i = tid + kNetThreads * j;
            if (i < in4) l4[i] = in[j];
        }
        fetch(col + nb8);
        __syncthreads();
        // opaque per column, as in k_packed_net_slots: no per-gate values hoisted out of the
        // column loop
#pragma unroll
        for (int i = 0; i < OW; ++i) asm volatile("" : "+v"(ops[i]));
#pragma unroll
        for (int q = 0; q < TG; ++q) asm volatile("" : "+v"(ent[q]));
#pragma unroll
        for (int l = 0; l < LMAX; ++l) {
            if (l < L) {  // uniform
                uint32_t* nxt = lds + net.base[l];
                constexpr int NW = (J + 7) / 8 + 1;
                const int wlo = (l * J) / 8;
                uint32_t lw[NW];
#pragma unroll
                for (int i = 0; i < NW; ++i) lw[i] = ops[wlo + i < OW ? wlo + i : OW - 1];
                uint32_t held[HOLD > 0 ? HOLD : 1];
#pragma unroll
                for (int j0 = 0; j0 < J; j0 += kBatch) {
                    uint32_t va[kBatch], vb[kBatch];
#pragma unroll
                    for (int j = j0; j < j0 + kBatch && j < J; ++j) {
                        const uint32_t e = ent[l * J + j];
                        va[j - j0] = lds[e & 0xffffu];
                        vb[j - j0] = lds[e >> 16];
                    }
#pragma unroll
                    for (int j = j0; j < j0 + kBatch && j < J; ++j) {
                        const int q = l * J + j;
                        const uint32_t r = gate_word((lw[q / 8 - wlo] >> (4 * (q % 8))) & 15u,
                                                     va[j - j0], vb[j - j0]);
                        if (HOLD > 0 && l == 0 && j >= JB) held[HOLD > 0 ? j - JB : 0] = r;
                        else nxt[tid + kNetThreads * j] = r;
                    }
                }
                __syncthreads();
                if constexpr (HOLD > 0) {
                    if (l == 0) {  // every thread has read the input: its words are free
#pragma unroll
                        for (int h = 0; h < HOLD; ++h)
                            lds[net.hold_base + kNetThreads * h + tid] = held[h];
                        __syncthreads();
                    }
                }
            }
        }
        column_counts_wave<B>(lds + net.base[L - 1], net.rows[L] / net.k, net.k, col,
                              nsamples, counts);
        __syncthreads();  // the next column overwrites the input words
    }
}

// Packed layers from resolved index tables with column-major output (the input layout of
// k_packed_net_cols): y[c * out_words + p] = word c of row order[p] (row p without an order)
// of the last layer, 0 for positions out_dim <= p < out_words.  The order only changes which
// rows run together: rows that read the same blocks of input rows, placed next to each other,
// keep the input words a column tile needs within one XCD's L2.  A layer's row o is op_{g[o]}(row ia[o], row ib[o]) of its input,
// a negative index reading a zero row and an index past the input's rows making row o zero
// (as k_eval_packed_idx).  With PAIR the kernel evaluates two layers composed, the first
// (t1) on x and the second (t2) on the first's rows, computing each first-layer row the
// second reads in place of storing the first layer: four input rows per output row instead
// of a full intermediate written and read back.
// Workgroups are mapped XCD-aware: XCD x (= blockIdx % 8) takes a contiguous range of column
// tiles and walks every row tile of one column tile before the next, so the input words of a
// column tile are read from HBM once, by one XCD, and the (up to four) reads of each input
// row by the rows of that tile hit its L2.
// A workgroup takes 64 rows x W words: a wave evaluates 16 rows, the indices of a row being
// uniform (scalar loads), and lane l takes words l, l + 64, ... (coalesced 4-byte loads of
// 64 words per input row); the tile is transposed through LDS (row stride W + 1: the column
// reads of a half-wave hit 32 banks) and each wave then writes the 64-row runs of W / 4
// words, 256 contiguous bytes each.
struct PackedTabs {
    const int32_t* ia;
    const int32_t* ib;
    const uint8_t* gate;
    int64_t in;  // rows of the layer's input
};

#ifndef CL_COLS_ROWS
#define CL_COLS_ROWS 64
#endif
constexpr int kColRows = CL_COLS_ROWS;  // rows per workgroup (16 per wave)
constexpr int kColThreads = kColRows * 4;
#ifndef CL_COLS_PAIR_RB
#define CL_COLS_PAIR_RB 8
#endif
#ifndef CL_COLS_NT_STORE
#define CL_COLS_NT_STORE 1
#endif

// Truth table of a gate whose input a (tt_a0) or b (tt_b0) is held at zero: the opcode
// that gives the same words without masking the operand (bits MSB first over AB = 00, 01,
// 10, 11, as gate_word reads them).
__device__ __forceinline__ uint32_t tt_a0(uint32_t g) {
    const uint32_t f00 = (g >> 3) & 1u, f01 = (g >> 2) & 1u;
    return (f00 << 3) | (f01 << 2) | (f00 << 1) | f01;
}
__device__ __forceinline__ uint32_t tt_b0(uint32_t g) {
    const uint32_t f00 = (g >> 3) & 1u, f10 = (g >> 1) & 1u;
    return (f00 << 3) | (f00 << 2) | (f10 << 1) | f10;
}

template <int W, bool PAIR>
__global__ __launch_bounds__(kColThreads) void k_eval_packed_cols(const uint32_t* __restrict__ x,
                                                          PackedTabs t1, PackedTabs t2,
                                                          const int32_t* __restrict__ order,
                                                          uint32_t* __restrict__ y,
                                                          int64_t out_dim, int64_t cols,
                                                          int64_t out_words, int64_t row_tiles,
                                                          int64_t tiles_per_xcd) {
    __shared__ uint32_t tile[kColRows][W + 1];
    constexpr int K = W / 64;          // words per lane
    constexpr int R = 16;              // rows per wave
    constexpr int NWV = kColRows / R;  // waves per workgroup
    constexpr int RB = PAIR ? CL_COLS_PAIR_RB : 8;  // rows whose loads are in flight together
    constexpr int NR = PAIR ? 4 : 2;   // input rows per output row
    const PackedTabs& tl = PAIR ? t2 : t1;  // the layer whose rows are written
    const int64_t i = blockIdx.x / 8;       // position in this XCD's walk
    const int64_t ct = (blockIdx.x % 8) * tiles_per_xcd + i / row_tiles;
    const int64_t o0 = (i % row_tiles) * kColRows, c0 = ct * W;
    if (c0 >= cols) return;  // past the last column tile (uniform per workgroup)
    const int w = wave_id(), lane = lane_id();
    // Lane r < R resolves row o0 + w * R + r: the input rows it reads (0 for one it does not)
    // and its opcodes, rewritten so that an operand read as zero (a negative index, a
    // first-layer row that is zero, a row written as zero) needs no mask: opcode 0 writes
    // zeros, tt_a0 / tt_b0 ignore the operand.  The wave's rows then take these values by
    // readlane, so no row waits on a chain of dependent scalar loads.
    int32_t src[NR];
    uint32_t ops = 0;  // output opcode | first-layer opcodes << 4, << 8
    {
        const int64_t p = o0 + w * R + lane;  // output position; the layer row order[p]
        int64_t o = p, a = -1, b = -1;
        bool row = lane < R && p < out_dim;
        if (row && order) {
            o = order[p];
            row = uint64_t(o) < uint64_t(out_dim);  // a corrupt entry writes zeros
        }
        if (row) {
            a = tl.ia[o];
            b = tl.ib[o];
        }
        const bool live = row && a < tl.in && b < tl.in;
        uint32_t g = live ? uint32_t(tl.gate[o] & 15) : 0u;
        if constexpr (PAIR) {
            // the two first-layer rows this row reads, each from two input rows
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int64_t p = s2 ? b : a;
                int64_t pa = -1, pb = -1;
                const bool has = live && p >= 0;
                if (has) {
                    pa = t1.ia[p];
                    pb = t1.ib[p];
                }
                const bool live1 = has && pa < t1.in && pb < t1.in;
                uint32_t g1 = live1 ? uint32_t(t1.gate[p] & 15) : 0u;
                if (pa < 0) g1 = tt_a0(g1);
                if (pb < 0) g1 = tt_b0(g1);
                if (!live1) g = s2 ? tt_b0(g) : tt_a0(g);
                ops |= g1 << (4 + 4 * s2);
                src[2 * s2] = live1 && pa >= 0 ? int32_t(pa) : 0;
                src[2 * s2 + 1] = live1 && pb >= 0 ? int32_t(pb) : 0;
            }
        } else {
            if (a < 0) g = tt_a0(g);
            if (b < 0) g = tt_b0(g);
            src[0] = live && a >= 0 ? int32_t(a) : 0;
            src[1] = live && b >= 0 ? int32_t(b) : 0;
        }
        ops |= g;
    }
    uint32_t lc[K];  // this lane's word offsets in a row (the row base is uniform)
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int64_t c = c0 + 64 * k + lane;
        lc[k] = uint32_t(c < cols ? c : 0);  // in bounds; the word is not stored
    }
#pragma unroll
    for (int i0 = 0; i0 < R; i0 += RB) {
        uint32_t v[RB][NR][K], f[RB];
#pragma unroll
        for (int ii = 0; ii < RB; ++ii) {
            f[ii] = __builtin_amdgcn_readlane(ops, i0 + ii);
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const uint32_t* rp = x + int64_t(__builtin_amdgcn_readlane(src[r], i0 + ii)) * cols;
#pragma unroll
                for (int k = 0; k < K; ++k) v[ii][r][k] = rp[lc[k]];
            }
        }
#pragma unroll
        for (int ii = 0; ii < RB; ++ii) {
            const uint32_t fl = f[ii];
#pragma unroll
            for (int k = 0; k < K; ++k) {
                uint32_t res;
                if constexpr (PAIR) {
                    const uint32_t u = gate_word((fl >> 4) & 15u, v[ii][0][k], v[ii][1][k]);
                    const uint32_t q = gate_word((fl >> 8) & 15u, v[ii][2][k], v[ii][3][k]);
                    res = gate_word(fl & 15u, u, q);
                } else {
                    res = gate_word(fl & 15u, v[ii][0][k], v[ii][1][k]);
                }
                tile[w * R + i0 + ii][64 * k + lane] = res;
            }
        }
    }
    __syncthreads();
    // store: wave w takes columns w, w + NWV, ...; a column's kColRows rows in 64-row pieces,
    // so each column is written as one contiguous run of kColRows words
    constexpr int PIECES = kColRows / 64;
#pragma unroll 4
    for (int j = w; j < W * PIECES; j += NWV) {
        const int cw = j / PIECES, rr = (j % PIECES) * 64 + lane;
        const int64_t c = c0 + cw, o = o0 + rr;
        if (c < cols && o < out_words) {
#if CL_COLS_NT_STORE
            // read once, by the fused pass: bypass the caches
            __builtin_nontemporal_store(tile[rr][cw], y + c * out_words + o);
#else
            y[c * out_words + o] = tile[rr][cw];
#endif
        }
    }
}

#ifndef CL_COLS_WORDS
#define CL_COLS_WORDS 128
#endif
constexpr int kColWords = CL_COLS_WORDS;  // words (32-sample columns) per workgroup

// LDS placement of the wide-input fused pass's layers (see k_packed_net_cols).
struct ColsPlan {
    int J = 0, hold = 0, in_words = 0, hold_base = 0, lds_words = 0;
    int base[kNetMaxLayers] = {};
};

bool spans_overlap(int a0, int a1, int b0, int b1) { return a0 < b1 && b0 < a1; }

// False when the network does not fit: a layer wider than 16 * 1024 rows, more layers than
// the entry registers hold (cols_max_layers), or an input whose column leaves no room for the first layer
// (holding at most two of its slots in registers).  Each later layer goes to the lowest of
// two places (after the held slots or word 0, else the top of LDS) that does not overlap the
// rows it reads.  Deterministic.
bool cols_plan(const int64_t* rows, int64_t L, ColsPlan& p) {
    if (L < 1 || L > kNetMaxLayers || rows[0] < 1) return false;
    int64_t maxw = 0;
    for (int64_t l = 1; l <= L; ++l) {
        if (rows[l] < 1) return false;
        maxw = std::max(maxw, rows[l]);
    }
    if (maxw > 16 * kNetThreads) return false;
    const int J = maxw <= 8 * kNetThreads ? 8 : 16;
    if (L > cols_max_layers(J)) return false;
    const int64_t in_words = ceil_div(rows[0], 64) * 64;
    if (in_words > kLdsWords) return false;
    const int span = J * kNetThreads;
    for (int hold : {0, 2}) {
        if (hold > 0 && L < 2) continue;  // the class counts read one contiguous layer
        const int split = (J - hold) * kNetThreads;
        if (in_words + split > kLdsWords || int64_t(hold) * kNetThreads > in_words) continue;
        ColsPlan q;
        q.J = J;
        q.hold = hold;
        q.in_words = int(in_words);
        q.hold_base = 0;
        q.base[0] = int(in_words);
        int end = int(in_words) + split;
        // the runs of LDS the layer being placed reads (layer 0's output is two)
        int r0a = q.base[0], r0b = q.base[0] + split, r1a = 0, r1b = hold * kNetThreads;
        bool ok = true;
        for (int64_t l = 1; l < L && ok; ++l) {
            ok = false;
            for (int c : {l == 1 ? hold * kNetThreads : 0, kLdsWords - span}) {
                if (c < 0 || c + span > kLdsWords || spans_overlap(c, c + span, r0a, r0b) ||
                    spans_overlap(c, c + span, r1a, r1b))
                    continue;
                q.base[l] = c;
                end = std::max(end, c + span);
                r0a = c;
                r0b = c + span;
                r1a = r1b = 0;
                ok = true;
                break;
            }
        }
        if (!ok) continue;
        q.lds_words = end;
        p = q;
        return true;
    }
    return false;
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
    const int gs = last / int(k);
    CL_ARG(int(k) <= kNetThreads, "k must be at most %d for the fused pass", kNetThreads);
    const int64_t cols = row_bytes / 4;
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
    // a lane of the class counts adds at most ceil(gs / 64) rows, fewer than 2^B
    const int per_lane = int(ceil_div(gs, 64));
    const bool slots = max_rows <= 16383 && net.rows[0] <= 4 * kNetThreads && J <= 16 &&
                       num_layers <= std::min(kSlotCap / J, kNetMaxLayers) && per_lane < 256;
    if (slots && !kNetDisableRegs) {
        // every slot writes: a buffer spans the J * 1024 rows a thread's slots can address
        const int buf_words = std::max(max_rows, J * kNetThreads);
        const int LMAX = std::min(kSlotCap / J, kNetMaxLayers);
        const size_t ops_bytes = size_t((LMAX * J + 7) / 8) * kNetThreads * 4;
        const size_t lds = size_t(2) * buf_words * 4 + (J <= kOpsLdsMaxJ ? ops_bytes : 0);
        CL_REQUIRE(lds <= 160 * 1024, CL_ERR_VALUE, "internal error: %zu bytes of LDS", lds);
        if (nsamples == 0 || cols == 0) return CL_OK;
        CL_ARG(x && tables && counts, "null pointer argument");
        CL_ARG(aligned(x, 4) && aligned(tables, 8), "misaligned buffers");
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
        if (per_lane < 8) by_ipt(std::integral_constant<int, 3>());
        else if (per_lane < 32) by_ipt(std::integral_constant<int, 5>());
        else by_ipt(std::integral_constant<int, 8>());
        if (rc) return rc;
        return check_launch("cl_packed_network");
    }
    // one column per workgroup; the class counts use the buffers as scratch
    // slices per class: one thread each, as many as fit
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
    const int buf_words = std::max(max_rows, count_words);
    const size_t lds = size_t(2) * buf_words * 4;
    CL_ARG(lds <= 160 * 1024, "activations do not fit in LDS");
    if (nsamples == 0 || cols == 0) return CL_OK;
    CL_ARG(x && tables && counts, "null pointer argument");
    CL_ARG(aligned(x, 4) && aligned(tables, 8), "misaligned buffers");
    const int64_t blocks = 8 * ceil_div(cols, 8);
    CL_ARG(blocks < (int64_t(1) << 31), "too many columns");
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

extern "C" int cl_packed_network_columns_layout(const int64_t* rows_host, int64_t num_layers,
                                                int64_t* applies, int64_t* in_words,
                                                int64_t* split, int64_t* hold_base,
                                                int64_t* base) {
    clear_error();
    CL_ARG(rows_host && applies && in_words && split && hold_base && base,
           "null pointer argument");
    CL_ARG(num_layers >= 1 && num_layers <= kNetMaxLayers, "1 to %d layers", kNetMaxLayers);
    ColsPlan p;
    *applies = cols_plan(rows_host, num_layers, p) ? 1 : 0;
    *in_words = p.in_words;
    *split = int64_t(p.J - p.hold) * kNetThreads;
    *hold_base = p.hold_base;
    for (int64_t l = 0; l < num_layers; ++l) base[l] = p.base[l];
    return CL_OK;
}

namespace {
int launch_packed_cols(const void* x, const PackedTabs& t1, const PackedTabs* t2,
                       const int32_t* order, void* y, int64_t out_dim, int64_t row_bytes,
                       int64_t out_words, void* stream) {
    CL_ARG(row_bytes % 4 == 0, "packed rows must be a multiple of 4 bytes");
    CL_ARG(out_words >= out_dim, "out_words (%lld) must be at least out_dim (%lld)",
           (long long)out_words, (long long)out_dim);
    const int64_t cols = row_bytes / 4;
    if (out_words == 0 || cols == 0) return CL_OK;
    CL_ARG(y && (out_dim == 0 || x), "null pointer argument");
    CL_ARG(aligned(x, 4) && aligned(y, 4), "misaligned buffers");
    const int64_t row_tiles = ceil_div(out_words, kColRows);
    const int64_t per_xcd = ceil_div(ceil_div(cols, kColWords), 8);
    CL_ARG(8 * per_xcd * row_tiles < (int64_t(1) << 31), "packed layer too large for one launch");
    const unsigned grid = unsigned(8 * per_xcd * row_tiles);
    auto* xs = static_cast<const uint32_t*>(x);
    auto* ys = static_cast<uint32_t*>(y);
    if (t2)
        k_eval_packed_cols<kColWords, true><<<grid, kColThreads, 0, as_stream(stream)>>>(
            xs, t1, *t2, order, ys, out_dim, cols, out_words, row_tiles, per_xcd);
    else
        k_eval_packed_cols<kColWords, false><<<grid, kColThreads, 0, as_stream(stream)>>>(
            xs, t1, t1, order, ys, out_dim, cols, out_words, row_tiles, per_xcd);
    return CL_OK;
}
}  // namespace

extern "C" int cl_eval_packed_indexed_columns(const void* x, const int32_t* ia,
                                              const int32_t* ib, const uint8_t* gate,
                                              const int32_t* order, void* y, int64_t in_dim,
                                              int64_t out_dim, int64_t row_bytes,
                                              int64_t out_words, void* stream) {
    clear_error();
    CL_ARG(in_dim >= 0 && out_dim >= 0 && row_bytes >= 0, "negative shape");
    CL_ARG(out_dim == 0 || in_dim > 0, "in_dim is 0 but out_dim > 0");
    CL_ARG(out_dim == 0 || (ia && ib && gate), "null pointer argument");
    const PackedTabs t{ia, ib, gate, in_dim};
    if (int rc = launch_packed_cols(x, t, nullptr, order, y, out_dim, row_bytes, out_words,
                                    stream))
        return rc;
    return check_launch("cl_eval_packed_indexed_columns");
}

extern "C" int cl_eval_packed_indexed_pair_columns(
    const void* x, const int32_t* ia1, const int32_t* ib1, const uint8_t* gate1,
    const int32_t* ia2, const int32_t* ib2, const uint8_t* gate2, const int32_t* order, void* y,
    int64_t in_dim, int64_t mid_dim, int64_t out_dim, int64_t row_bytes, int64_t out_words,
    void* stream) {
    clear_error();
    CL_ARG(in_dim >= 0 && mid_dim >= 0 && out_dim >= 0 && row_bytes >= 0, "negative shape");
    CL_ARG(out_dim == 0 || (mid_dim > 0 && in_dim > 0), "an empty layer feeds out_dim > 0 rows");
    CL_ARG(out_dim == 0 || (ia1 && ib1 && gate1 && ia2 && ib2 && gate2),
           "null pointer argument");
    const PackedTabs t1{ia1, ib1, gate1, in_dim}, t2{ia2, ib2, gate2, mid_dim};
    if (int rc = launch_packed_cols(x, t1, &t2, order, y, out_dim, row_bytes, out_words, stream))
        return rc;
    return check_launch("cl_eval_packed_indexed_pair_columns");
}

extern "C" int cl_packed_network_columns(const void* x, int64_t cols, int64_t in_words,
                                         int64_t nsamples, const uint64_t* tables,
                                         const int64_t* rows_host, int64_t num_layers, int64_t k,
                                         int32_t* counts, void* stream) {
    clear_error();
    CL_ARG(num_layers >= 1 && num_layers <= kNetMaxLayers, "1 to %d layers", kNetMaxLayers);
    CL_ARG(rows_host && k >= 1 && cols >= 0, "bad arguments");
    CL_ARG(nsamples >= 0 && nsamples <= cols * 32, "more samples than packed bits");
    ColsPlan p;
    CL_ARG(cols_plan(rows_host, num_layers, p),
           "the network does not fit the wide-input fused pass "
           "(cl_packed_network_columns_layout)");
    CL_ARG(in_words == p.in_words, "in_words must be %d for this network, got %lld",
           p.in_words, (long long)in_words);
    PackedNetCols net{};
    net.num_layers = int(num_layers);
    net.k = int(k);
    int64_t off = 0;
    for (int l = 0; l <= num_layers; ++l) {
        net.rows[l] = int(rows_host[l]);
        if (l < num_layers) {
            net.table_off[l] = off;
            off += rows_host[l + 1];
            net.base[l] = p.base[l];
        }
    }
    net.hold_base = p.hold_base;
    net.in_words = p.in_words;
    const int last = net.rows[num_layers];
    if (last % k != 0) {
        set_error("in_dim (%d) has to be divisible by k (%lld) but it is not", last, (long long)k);
        return CL_ERR_VALUE;
    }
    CL_ARG(k <= last, "k must be at most the last layer's width");
    const int per_lane = int(ceil_div(last / k, 64));
    CL_ARG(per_lane < 256, "class groups too large for the fused pass");
    if (nsamples == 0 || cols == 0) return CL_OK;
    CL_ARG(x && tables && counts, "null pointer argument");
    CL_ARG(aligned(x, 16) && aligned(tables, 8), "misaligned buffers");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        set_error("cannot query the device");
        return CL_ERR_HIP;
    }
    const int64_t want = std::max<int64_t>(8, (int64_t(cus) / 8) * 8);
    const int64_t pblocks = std::min<int64_t>(want, 8 * ceil_div(cols, 8));
    const size_t lds = size_t(p.lds_words) * 4;
    int rc = CL_OK;
    auto go = [&](auto nb, auto jc, auto hc) {
        auto* kern = &k_packed_net_cols<decltype(nb)::value, decltype(jc)::value,
                                        decltype(hc)::value>;
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) !=
            hipSuccess) {
            set_error("cannot reserve %zu bytes of LDS for the fused pass", lds);
            rc = CL_ERR_HIP;
            return;
        }
        kern<<<unsigned(pblocks), kNetThreads, lds, as_stream(stream)>>>(
            static_cast<const uint4*>(x), cols, nsamples, tables, net, counts);
    };
    using std::integral_constant;
    auto by_shape = [&](auto nb) {
        if (p.J == 8 && p.hold == 0) go(nb, integral_constant<int, 8>(), integral_constant<int, 0>());
        else if (p.J == 8) go(nb, integral_constant<int, 8>(), integral_constant<int, 2>());
        else if (p.hold == 0) go(nb, integral_constant<int, 16>(), integral_constant<int, 0>());
        else go(nb, integral_constant<int, 16>(), integral_constant<int, 2>());
    };
    if (per_lane < 8) by_shape(integral_constant<int, 3>());
    else if (per_lane < 32) by_shape(integral_constant<int, 5>());
    else by_shape(integral_constant<int, 8>());
    if (rc) return rc;
    return check_launch("cl_packed_network_columns");
}
