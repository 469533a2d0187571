"""The C-ABI library loads without a GPU and exports every entry point the public header
declares, with the bindings' signature table covering the same set.  No compute calls."""
import ctypes
import re
from pathlib import Path

from compactlogic_amd import _capi

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(cl_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    assert {"cl_dense_forward", "cl_dense_backward_w", "cl_dense_backward_x", "cl_dense_eval",
            "cl_pack_bits", "cl_group_bit_sum", "cl_dense_eval_packed"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_capi.LIB_PATH))
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_bindings_cover_the_header():
    assert declared_symbols() == set(_capi.SIGNATURES) | {"cl_last_error"}


def test_abi_version_and_error_state():
    lib = _capi.load()
    assert lib.cl_abi_version() == _capi.ABI_VERSION
    assert lib.cl_last_error() == b""


def test_argument_errors_are_reported_without_a_device():
    lib = _capi.load()
    # Invalid num_gates is rejected before anything touches the device.
    rc = lib.cl_dense_forward(0, None, None, None, None, None, None, 4, 4, 4, 0, None)
    assert rc == _capi.CL_ERR_INVALID_ARGUMENT
    assert b"num_gates" in lib.cl_last_error()
    # groupbitsum divisibility is a ValueError, as in the reference binding.
    rc = lib.cl_group_bit_sum(None, 7, 8, 0, 2, None, None)
    assert rc == _capi.CL_ERR_VALUE
    assert b"divisible" in lib.cl_last_error()
    rc = lib.cl_pack_bits(None, 1, 1, 12, None, None, None)
    assert rc == _capi.CL_ERR_VALUE
