/* Bit-packed evaluator in plain C -- TEST INFRASTRUCTURE ONLY (CPU oracle).
 *
 * Follows (paths relative to the eth-sri/CompactLogic tree):
 *   bitwise gates   compactlogic/cuda/utils.cuh:141-178 (the 16-case table, restated here
 *                   case by case; the HIP kernels use a minterm-mask form instead)
 *   pack layout     compactlogic/cuda/difflogic_kernel.cu:417-462 (LSB = first sample,
 *                   pad_len = (bits - n % bits) % bits)
 *   layer eval      third_party/convlogic_source_code/src/difflogic/cuda/difflogic_kernel.cu:271-293
 *   group popcount  compactlogic/cuda/difflogic_kernel.cu:500-567 (counts [N, k])
 *   tree conv block third_party/convlogic_source_code/src/convlogic/convlogic_layer.py:236-321
 *                   with the argmax gates: 8 taps (sel = ch << 16 | row << 8 | col, zero outside
 *                   the image), gates on the tap pairs, on (0,1), (2,3) and their pair; 2x2
 *                   pool of {0, 1} values = OR
 * A packed row is a little-endian bit string: bit j of the row = bit j%8 of byte j/8.
 */
#include <stdint.h>
#include <string.h>

uint64_t oracle_gate_word(int g, uint64_t a, uint64_t b) {
    switch (g) {
        case 0: return 0;
        case 1: return a & b;
        case 2: return a & ~b;
        case 3: return a;
        case 4: return b & ~a;
        case 5: return b;
        case 6: return a ^ b;
        case 7: return a | b;
        case 8: return ~(a | b);
        case 9: return ~(a ^ b);
        case 10: return ~b;
        case 11: return ~b | a;
        case 12: return ~a;
        case 13: return ~a | b;
        case 14: return ~(a & b);
        default: return ~(uint64_t)0;
    }
}

/* Vigna's SplitMix64 output function applied to (x + golden gamma). */
uint64_t oracle_splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

void oracle_fill_splitmix64(uint64_t* out, int64_t count, uint64_t base) {
    for (int64_t i = 0; i < count; ++i) out[i] = oracle_splitmix64(base + (uint64_t)i);
}

/* t: [rows, n] bytes (0/1) -> out: [rows, row_bytes], row_bytes = ceil(n / bits) * bits / 8. */
void oracle_pack_bits(const uint8_t* t, int64_t rows, int64_t n, int bits, uint8_t* out) {
    const int64_t words = (n + bits - 1) / bits;
    const int64_t row_bytes = words * (bits / 8);
    memset(out, 0, (size_t)(rows * row_bytes));
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < n; ++j)
            if (t[r * n + j]) out[r * row_bytes + j / 8] |= (uint8_t)(1u << (j % 8));
}

/* One layer on packed rows (row_bytes multiple of 8): y[o] = op_g[o](x[ia[o]], x[ib[o]]),
 * a negative index reads an all-zero row. */
void oracle_eval_packed(const uint64_t* x, int64_t in_dim, int64_t words, const int64_t* ia,
                        const int64_t* ib, const uint8_t* g, int64_t out_dim, uint64_t* y) {
    (void)in_dim;
    for (int64_t o = 0; o < out_dim; ++o) {
        const uint64_t* xa = ia[o] >= 0 ? x + ia[o] * words : 0;
        const uint64_t* xb = ib[o] >= 0 ? x + ib[o] * words : 0;
        for (int64_t w = 0; w < words; ++w)
            y[o * words + w] = oracle_gate_word(g[o], xa ? xa[w] : 0, xb ? xb[w] : 0);
    }
}

/* counts[s, c] = number of rows of group c (rows c*gs .. c*gs+gs-1, gs = rows / k) whose bit s
 * is set, for s < n_valid. */
void oracle_group_bit_sum(const uint8_t* packed, int64_t rows, int64_t row_bytes,
                          int64_t n_valid, int64_t k, int32_t* counts) {
    const int64_t gs = rows / k;
    memset(counts, 0, (size_t)(n_valid * k) * sizeof(int32_t));
    for (int64_t c = 0; c < k; ++c)
        for (int64_t r = c * gs; r < (c + 1) * gs; ++r) {
            const uint8_t* row = packed + r * row_bytes;
            for (int64_t s = 0; s < n_valid; ++s) counts[s * k + c] += (row[s >> 3] >> (s & 7)) & 1;
        }
}

/* Complete packed tree block: x rows (ch * h + y) * w + x of `words` 64-bit words; gates
 * [c_out][7] opcodes; sel [c_out][8]; output rows (c * hp + py) * wp + px. */
void oracle_tree_block_bits(const uint64_t* x, int64_t words, const uint8_t* gates,
                            const int32_t* sel, int c_in, int h, int w, int c_out, int sh,
                            int sw, int ph, int pw, int kh, int kw, uint64_t* y) {
    const int ho = (h + 2 * ph - kh) / sh + 1, wo = (w + 2 * pw - kw) / sw + 1;
    const int hp = ho / 2, wp = wo / 2;
    for (int c = 0; c < c_out; ++c) {
        int ch[8], dy[8], dx[8];
        for (int k = 0; k < 8; ++k) {
            ch[k] = (sel[c * 8 + k] >> 16) & 0xFFFF;
            dy[k] = ((sel[c * 8 + k] >> 8) & 0xFF) - ph;
            dx[k] = (sel[c * 8 + k] & 0xFF) - pw;
        }
        const uint8_t* g = gates + (int64_t)c * 7;
        for (int py = 0; py < hp; ++py)
            for (int px = 0; px < wp; ++px) {
                uint64_t* out = y + (((int64_t)c * hp + py) * wp + px) * words;
                const uint64_t* tap[4][8];  /* NULL = zero word */
                for (int q = 0; q < 4; ++q) {
                    const int oy = 2 * py + (q >> 1), ox = 2 * px + (q & 1);
                    for (int k = 0; k < 8; ++k) {
                        const int iy = oy * sh + dy[k], ix = ox * sw + dx[k];
                        const int in = ch[k] < c_in && iy >= 0 && iy < h && ix >= 0 && ix < w;
                        tap[q][k] = in ? x + (((int64_t)ch[k] * h + iy) * w + ix) * words : 0;
                    }
                }
                for (int64_t j = 0; j < words; ++j) {
                    uint64_t acc = 0;
                    for (int q = 0; q < 4; ++q) {
                        uint64_t v[8], n[4];
                        for (int k = 0; k < 8; ++k) v[k] = tap[q][k] ? tap[q][k][j] : 0;
                        for (int k = 0; k < 4; ++k) n[k] = oracle_gate_word(g[k] & 15, v[2 * k], v[2 * k + 1]);
                        acc |= oracle_gate_word(g[6] & 15, oracle_gate_word(g[4] & 15, n[0], n[1]),
                                                oracle_gate_word(g[5] & 15, n[2], n[3]));
                    }
                    out[j] = acc;
                }
            }
    }
}
