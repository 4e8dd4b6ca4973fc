"""The C-ABI library loads, exports every symbol include/sunshape_amd.h declares, and
its argument checks run on the host (no GPU calls are made here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sunshape_amd.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"^[A-Za-z_][\w \*]*?\b(ssq_\w+)\s*\(", src, flags=re.M))


def test_header_declares_expected_entry_points():
    from sunshape_amd import _native as N

    assert _declared_functions() == set(N.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    from sunshape_amd import _native as N

    assert os.path.exists(N.LIB_PATH), "run python -m sunshape_amd.build"
    lib = N.lib()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.ssq_abi_version() == N.ABI_VERSION == 5


def test_struct_layout_matches_library():
    """Wrong struct_size -> SSQ_ERR_ABI; right size with NULL tensors -> SSQ_ERR_INVALID."""
    from sunshape_amd import _native as N

    lib = N.lib()
    a = N.DecodeArgs()
    a.struct_size = ctypes.sizeof(N.DecodeArgs) + 8
    assert lib.ssq_decode(ctypes.byref(a), None, 0, None) == N.SSQ_ERR_ABI
    a = N.DecodeArgs()
    assert lib.ssq_decode(ctypes.byref(a), None, 0, None) == N.SSQ_ERR_INVALID
    assert b"non-NULL" in lib.ssq_last_error()
    e = N.EncodeArgs()
    e.struct_size = 4
    assert lib.ssq_encode(ctypes.byref(e), None) == N.SSQ_ERR_ABI
    e = N.EncodeArgs()
    assert lib.ssq_encode(ctypes.byref(e), None) == N.SSQ_ERR_INVALID
    assert lib.ssq_decode_workspace_size(ctypes.byref(N.DecodeArgs())) == 0


def test_host_side_argument_errors_name_the_problem():
    from sunshape_amd import _native as N

    lib = N.lib()
    a = N.DecodeArgs(q=1, perm=1, cent=1, codes=1, batch=1, num_q_heads=6, q_len=1, num_kv_heads=4,
                     head_dim=64, block_dim=8, n_blocks=8, n_centroids=256)
    assert lib.ssq_decode(ctypes.byref(a), None, 0, None) == N.SSQ_ERR_INVALID
    assert b"divisible" in lib.ssq_last_error()
    a.num_kv_heads = 2
    a.n_blocks = 7
    assert lib.ssq_attention_scores(ctypes.byref(a), None) == N.SSQ_ERR_INVALID
    assert b"n_blocks" in lib.ssq_last_error()
    a.n_blocks = 8
    a.heavy_mask[0] = 1
    assert lib.ssq_attention_scores(ctypes.byref(a), None) == N.SSQ_ERR_INVALID
    assert b"passthrough" in lib.ssq_last_error()
    assert lib.ssq_lut_build(None, 0, 0, 1, 64, None, None, 8, 256, 0, 0.0, None, None) == N.SSQ_ERR_INVALID
    assert lib.ssq_dequantize(None, 8, 4, None, None, 64, 8, 256, None, 0, None, 0, 0, None, 64, None) == N.SSQ_ERR_INVALID


def test_product_fails_loudly_without_library(monkeypatch):
    from sunshape_amd import _native as N

    monkeypatch.setattr(N, "_lib", None)
    monkeypatch.setattr(N, "LIB_PATH", "/nonexistent/libsunshape_amd.so")
    with pytest.raises(RuntimeError, match="not built"):
        N.lib()


def test_probe_library_exports_the_stream_read():
    """bench.py's bandwidth probe lives in its own library (not the decode ABI); build() makes it."""
    import ctypes as C

    from sunshape_amd.build import PROBE_PATH

    probe = C.CDLL(PROBE_PATH)
    assert hasattr(probe, "ssq_probe_stream_read")
