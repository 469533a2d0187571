"""Bit-packed CPU evaluator -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes front end of packed_ref.c (built by ``make -C oracle``).  Follows the
reference files listed in packed_ref.c.  Pinned by tests/test_oracle.py against
numpy.packbits(bitorder='little'), a per-bit boolean evaluator using the truth table, unpacked
bit sums, and the published SplitMix64 output sequence.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.oracle_gate_word.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_gate_word.restype = ctypes.c_uint64
        L.oracle_splitmix64.argtypes = [ctypes.c_uint64]
        L.oracle_splitmix64.restype = ctypes.c_uint64
        L.oracle_fill_splitmix64.argtypes = [p, i64, ctypes.c_uint64]
        L.oracle_pack_bits.argtypes = [p, i64, i64, ctypes.c_int, p]
        L.oracle_eval_packed.argtypes = [p, i64, i64, p, p, p, i64, p]
        L.oracle_group_bit_sum.argtypes = [p, i64, i64, i64, i64, p]
        L.oracle_tree_block_bits.argtypes = [p, i64, p, p] + [ctypes.c_int] * 10 + [p]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def splitmix64(z: int) -> int:
    return int(lib().oracle_splitmix64(z & 0xFFFFFFFFFFFFFFFF))


def fill_splitmix64(count: int, base: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    lib().oracle_fill_splitmix64(_ptr(out), count, base & 0xFFFFFFFFFFFFFFFF)
    return out


def pack_bits(t: np.ndarray, bits: int) -> tuple[np.ndarray, int]:
    """bool [rows, n] -> (uint8 [rows, row_bytes], pad_len)."""
    t = np.ascontiguousarray(t, dtype=np.uint8)
    rows, n = t.shape
    words = -(-n // bits)
    out = np.empty((rows, words * bits // 8), dtype=np.uint8)
    lib().oracle_pack_bits(_ptr(t), rows, n, bits, _ptr(out))
    return out, (bits - n % bits) % bits


def eval_layer(x: np.ndarray, ia: np.ndarray, ib: np.ndarray, g: np.ndarray) -> np.ndarray:
    """x: uint64 [in, words] -> uint64 [out, words]; y[o] = op_g[o](x[ia[o]], x[ib[o]]),
    a negative index reads zeros."""
    x = np.ascontiguousarray(x.view(np.uint64))
    ia = np.ascontiguousarray(ia, dtype=np.int64)
    ib = np.ascontiguousarray(ib, dtype=np.int64)
    g = np.ascontiguousarray(g, dtype=np.uint8)
    y = np.empty((len(ia), x.shape[1]), dtype=np.uint64)
    lib().oracle_eval_packed(_ptr(x), x.shape[0], x.shape[1], _ptr(ia), _ptr(ib), _ptr(g),
                             len(ia), _ptr(y))
    return y


def resolve_slots(indices: np.ndarray, gate_sequence: np.ndarray, w_slot: np.ndarray):
    """(ia, ib, g) of every neuron's argmax slot (compactlogic/compactlogic.py:126-129)."""
    o = np.arange(indices.shape[1])
    s = np.asarray(w_slot).astype(np.int64)
    return indices[0][o, s], indices[1][o, s], np.asarray(gate_sequence)[o, s]


def resolve_conv_slots(offsets_ch, offsets_h, offsets_w, gate_sequence, w_slot, in_shape, stride,
                       out_hw):
    """(ia, ib, g) per output feature (c, oy, ox) of a frozen ConvLayer, following the loop of
    compiler/extract.py:130-174: the winner slot s = w_slot[c] reads input feature
    (ch * h + y) * w + x (NCHW, :101-102) at y = oy * stride + dh, x = ox * stride + dw, and a
    tap outside the input plane is the constant 0 (index -1 here)."""
    _, h, w = in_shape
    h_out, w_out = out_hw
    c_out = len(w_slot)
    ia = np.empty(c_out * h_out * w_out, dtype=np.int64)
    ib = np.empty_like(ia)
    g = np.empty(len(ia), dtype=np.uint8)
    for c in range(c_out):
        s = int(w_slot[c])
        taps = [(int(offsets_ch[side][c][s]), int(offsets_h[side][c][s]),
                 int(offsets_w[side][c][s])) for side in (0, 1)]
        for oy in range(h_out):
            for ox in range(w_out):
                o = (c * h_out + oy) * w_out + ox
                for side, dst in ((0, ia), (1, ib)):
                    ch, dh, dw = taps[side]
                    y, x = oy * stride + dh, ox * stride + dw
                    dst[o] = (ch * h + y) * w + x if (0 <= y < h and 0 <= x < w) else -1
                g[o] = int(gate_sequence[c][s])
    return ia, ib, g


def group_bit_sum(packed: np.ndarray, pad_len: int, k: int) -> np.ndarray:
    """uint rows [rows, *] -> int32 [N, k]; raises ValueError when rows % k != 0."""
    packed = np.ascontiguousarray(packed).view(np.uint8)
    rows, row_bytes = packed.shape
    if rows % k:
        raise ValueError(f"in_dim ({rows}) has to be divisible by k ({k}) but it is not")
    n = row_bytes * 8 - pad_len
    counts = np.empty((n, k), dtype=np.int32)
    lib().oracle_group_bit_sum(_ptr(packed), rows, row_bytes, n, k, _ptr(counts))
    return counts


def network_counts(x_words: np.ndarray, layers, k: int, pad_len: int = 0) -> np.ndarray:
    """Whole packed network: layers = [(ia, ib, g), ...] per layer; returns int32 [N, k]."""
    h = x_words
    for ia, ib, g in layers:
        h = eval_layer(h, ia, ib, g)
    return group_bit_sum(h, pad_len, k)


def tree_block_bits(x_words: np.ndarray, gates: np.ndarray, sel: np.ndarray, in_shape, stride,
                    pad, kernel) -> np.ndarray:
    """Complete packed tree block (pool = OR): uint64 rows [c_in * h * w, words] ->
    [c_out * hp * wp, words]."""
    xw = np.ascontiguousarray(x_words, dtype=np.uint64)
    g = np.ascontiguousarray(gates, dtype=np.uint8)
    s = np.ascontiguousarray(sel, dtype=np.int32)
    c_in, h, w = in_shape
    (sh, sw), (ph, pw), (kh, kw) = stride, pad, kernel
    ho, wo = (h + 2 * ph - kh) // sh + 1, (w + 2 * pw - kw) // sw + 1
    c_out = s.shape[0]
    y = np.empty((c_out * (ho // 2) * (wo // 2), xw.shape[1]), dtype=np.uint64)
    lib().oracle_tree_block_bits(_ptr(xw), xw.shape[1], _ptr(g), _ptr(s), c_in, h, w, c_out,
                                 sh, sw, ph, pw, kh, kw, _ptr(y))
    return y
