"""ctypes binding of libcompactlogic_hip.so (declarations in include/compactlogic_hip.h).

The library is built in-tree by ``compactlogic_amd.build``; this module only loads it.  There
is no fallback: if the library is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

# The in-tree build; nothing else is loaded.
LIB_PATH = Path(__file__).resolve().parent / "libcompactlogic_hip.so"

CL_OK = 0
CL_ERR_INVALID_ARGUMENT = 1
CL_ERR_VALUE = 2
CL_ERR_HIP = 3

CL_DTYPE_F32 = 0
CL_DTYPE_F64 = 1
CL_DTYPE_F16 = 2

ABI_VERSION = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_u64 = ctypes.c_uint64
_f64 = ctypes.c_double

# name -> argument types (restype is int for every entry point except cl_last_error)
SIGNATURES: dict[str, list] = {
    "cl_abi_version": [],
    "cl_dense_forward": [_int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_dense_backward_w": [_int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_dense_backward_x": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64,
                            _i64, _i64, _p],
    "cl_dense_eval": [_int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_dense_prep": [_int, _p, _int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "cl_dense_forward_tiled": [_int, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_dense_backward_part": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p, _p,
                               _i64, _i64, _i64, _i64, _i64, _p],
    "cl_dense_backward_rows": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                               _i64, _i64, _p],
    "cl_transpose": [_int, _p, _p, _i64, _i64, _p],
    "cl_tree_conv_forward": [_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _int, _int,
                             _int, _int, _int, _int, _p, _p, _p, _p, _p],
    "cl_tree_conv_workspace": [_int, _i64, _i64, _i64, _i64, _i64, _int, _int, _int, _int, _int,
                               _int, _int, _int, _p],
    "cl_tree_conv_backward": [_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                              _int, _int, _int, _int, _int, _int, _int, _p, _p, _p, _i64, _p],
    "cl_tree_conv_forward_softmax": [_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _int, _int,
                                     _int, _int, _int, _int, _int, _p, _p, _p, _p, _int, _int,
                                     _p],
    "cl_tree_conv_backward_softmax": [_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64,
                                      _i64, _int, _int, _int, _int, _int, _int, _int, _p, _p, _p,
                                      _i64, _int, _p],
    "cl_tree_conv_forward_softmax_coefs": [_int, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                           _int, _int, _int, _int, _int, _int, _p, _p, _p, _p,
                                           _int, _int, _p, _p],
    "cl_tree_conv_backward_softmax_coefs": [_int, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                            _i64, _i64, _int, _int, _int, _int, _int, _int, _p,
                                            _p, _p, _i64, _int, _p, _p],
    "cl_tree_level_forward": [_int, _p, _p, _i64, _i64, _i64, _i64, _p, _p],
    "cl_tree_level_workspace": [_int, _i64, _i64, _i64, _i64, _p],
    "cl_tree_level_backward": [_int, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p],
    "cl_tree_conv_eval_packed": [_p, _i64, _p, _p, _i64, _i64, _i64, _i64, _int, _int, _int, _int,
                                 _int, _int, _int, _p, _p],
    "cl_dense_forward_fused": [_int, _p, _p, _int, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                               _i64, _i64, _p],
    "cl_dense_weight_grad": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                             _p],
    "cl_dense_tiled_chunks": [_int, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "cl_dense_backward_tiled": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                _i64, _i64, _p],
    "cl_dense_backward_finalize": [_int, _p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "cl_conv_forward": [_int, _p, _p, _p, _p, _p, _p, _p] + [_i64] * 9 + [_p],
    "cl_conv_eval": [_int, _p, _p, _p, _p, _p, _p, _p] + [_i64] * 9 + [_p],
    "cl_conv_backward_w": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64] + [_i64] * 9 + [_p],
    "cl_conv_backward_w_workspace": [_int] + [_i64] * 9 + [ctypes.POINTER(_i64)],
    "cl_conv_backward_x": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p] + [_i64] * 9 + [_p],
    "cl_eval_packed_indexed": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "cl_conv_window_coef_width": [_i64, ctypes.POINTER(_i64)],
    "cl_conv_window_prep": [_int, _p, _int, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "cl_conv_window_forward": [_int, _p, _p, _p, _p, _p] + [_i64] * 11 + [_p],
    "cl_conv_window_backward_x": [_int, _p, _p, _p, _p, _p, _p] + [_i64] * 11 + [_p],
    "cl_conv_window_chunks": [_i64, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "cl_conv_window_moments": [_int, _p, _p, _p, _p, _p, _i64, _i64] + [_i64] * 11 + [_p],
    "cl_conv_window_finalize": [_int, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i64, _p],
    "cl_group_sum_forward": [_int, _p, _i64, _i64, _i64, _i64, _i64, _f64, _p, _p, _i64, _p],
    "cl_group_sum_workspace_size": [_int, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "cl_group_sum_backward": [_int, _p, _i64, _i64, _i64, _f64, _p, _i64, _i64, _p],
    "cl_group_sum_cross_entropy_forward": [_int, _p, _i64, _i64, _i64, _i64, _i64, _f64, _p,
                                           _i64, _p, _p, _p, _p, _p, _i64, _p],
    "cl_group_sum_cross_entropy_workspace_size": [_int, _i64, _i64, _i64, ctypes.POINTER(_i64)],
    "cl_group_sum_cross_entropy_backward": [_int, _p, _p, _i64, _p, _p, _i64, _i64, _i64, _f64,
                                            _p, _i64, _i64, _p],
    "cl_group_sum_cross_entropy_scratch_limit": [ctypes.POINTER(_i64)],
    "cl_dense_group_sum_cross_entropy_workspace_size": [_int, _i64, _i64, _i64,
                                                        ctypes.POINTER(_i64),
                                                        ctypes.POINTER(_i64)],
    "cl_dense_group_sum_cross_entropy_forward": [_int, _p, _p, _int, _p, _p, _p, _p, _p, _i64,
                                                 _i64, _i64, _i64, _i64, _i64, _f64, _p, _i64,
                                                 _p, _p, _p, _p, _p, _i64, _p],
    "cl_dense_group_sum_cross_entropy_backward": [_int, _p, _p, _p, _i64, _p, _p, _i64, _f64,
                                                  _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                                                  _i64, _i64, _i64, _p, _i64, _p],
    "cl_dense_backward_rows_first": [_int, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                     _i64, _i64, _p, _i64, _p, _i64, _p, _p, _p, _i64, _p],
    "cl_plan_locality_order": [ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i64, _i64,
                               ctypes.POINTER(_i32)],
    "cl_packed_bank_layout": [ctypes.POINTER(_i32), ctypes.POINTER(_i32),
                              ctypes.POINTER(_i32), ctypes.POINTER(_i32), _i64, _i64,
                              ctypes.POINTER(_i32)],
    "cl_adam_clip_max_tensors": [ctypes.POINTER(_i64)],
    "cl_adam_clip_workspace": [_i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "cl_adam_clip_step": [_int, _i64, _p, _p, _p, _p, ctypes.POINTER(_i64), _p, _f64, _f64,
                          _f64, _f64, _f64, _p, _i64, _p],
    "cl_group_sum_cross_entropy_forward_noalloc": [_int, _p, _i64, _i64, _i64, _i64, _i64, _f64,
                                                   _p, _i64, _p, _p, _p, _p, _p],
    "cl_pack_bits": [_p, _i64, _i64, _i32, _p, ctypes.POINTER(_i64), _p],
    "cl_dense_eval_packed": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_group_bit_sum": [_p, _i64, _i64, _i64, _i64, _p, _p],
    "cl_fill_splitmix64": [_p, _i64, _u64, _p],
    "cl_packed_network_limits": [ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "cl_packed_network": [_p, _i64, _i64, _p, ctypes.POINTER(_i64), _i64, _i64, _p, _p],
    "cl_packed_network_columns_layout": [ctypes.POINTER(_i64), _i64, ctypes.POINTER(_i64),
                                         ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                         ctypes.POINTER(_i64), ctypes.POINTER(_i64)],
    "cl_eval_packed_indexed_columns": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "cl_eval_packed_indexed_pair_columns": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64,
                                            _i64, _i64, _i64, _p],
    "cl_packed_network_columns": [_p, _i64, _i64, _i64, _p, ctypes.POINTER(_i64), _i64, _i64,
                                  _p, _p],
}

_lib = None


class CompactLogicError(RuntimeError):
    """Raised when an entry point of the HIP library reports a failure."""


def load() -> ctypes.CDLL:
    """Load (once) and return the in-tree HIP library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    p = LIB_PATH
    if not p.exists():
        raise CompactLogicError(
            f"HIP library not found at {p}; build it with `python -m compactlogic_amd.build`")
    lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _int
    lib.cl_last_error.argtypes = []
    lib.cl_last_error.restype = ctypes.c_char_p
    got = lib.cl_abi_version()
    if got != ABI_VERSION:
        raise CompactLogicError(f"ABI version mismatch: library {got}, bindings {ABI_VERSION}")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Invoke entry point `name`; translate a failure status into a Python exception."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != CL_OK:
        msg = lib.cl_last_error().decode(errors="replace")
        if rc == CL_ERR_VALUE:
            raise ValueError(msg)
        raise CompactLogicError(f"{name} failed (status {rc}): {msg}")
