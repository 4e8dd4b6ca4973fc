"""ctypes mirrors of the C ABI's argument structs (include/sunshape_amd.h), without torch: the
binding (``_native``) and host-only tools that load the library without torch (the sanitized host
build's fuzz driver) share them.  The library checks ``struct_size``, so a drift between these and
the header is an SSQ_ERR_ABI, never a misread argument."""

from __future__ import annotations

import ctypes

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float


class DecodeArgs(ctypes.Structure):
    """Mirror of ``ssq_decode_args``."""

    _fields_ = [
        ("struct_size", _u32),
        ("q", _vp), ("q_dtype", _i32), ("q_sb", _i64), ("q_sh", _i64), ("q_sl", _i64),
        ("batch", _i32), ("num_q_heads", _i32), ("q_len", _i32), ("head_dim", _i32), ("num_kv_heads", _i32),
        ("has_scale", _i32), ("scale", _f32),
        ("perm", _vp), ("perm_sh", _i64),
        ("cent", _vp), ("cent_sh", _i64),
        ("block_dim", _i32), ("n_blocks", _i32), ("n_centroids", _i32),
        ("heavy_mask", ctypes.c_uint64 * 2),
        ("pt_dense", _i32), ("pt_dtype", _i32),
        ("pt", _vp), ("pt_sb", _i64), ("pt_sh", _i64), ("pt_st", _i64),
        ("layout", _i32), ("seq_len", _i32),
        ("codes", _vp), ("c_sb", _i64), ("c_sh", _i64), ("c_st", _i64),
        ("block_table", _vp), ("bt_sb", _i64), ("seq_lens", _vp), ("page_size", _i32),
        ("v", _vp), ("v_dtype", _i32), ("value_dim", _i32),
        ("v_sb", _i64), ("v_sh", _i64), ("v_st", _i64),
        ("mask", _vp), ("m_sb", _i64), ("m_sh", _i64), ("m_sl", _i64), ("m_st", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_sh", _i64), ("o_sl", _i64),
        ("lse", _vp),
        ("scores", _vp), ("s_sb", _i64), ("s_sh", _i64), ("s_sl", _i64),
        ("num_splits", _i32), ("kernel", _i32),
        ("code_bits", _i32),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(DecodeArgs)
        for k, v in kw.items():
            setattr(self, k, v)


class EncodeArgs(ctypes.Structure):
    """Mirror of ``ssq_encode_args``."""

    _fields_ = [
        ("struct_size", _u32),
        ("keys", _vp), ("k_dtype", _i32), ("k_sb", _i64), ("k_sh", _i64), ("k_ss", _i64),
        ("batch", _i32), ("num_kv_heads", _i32), ("seq_len", _i32), ("head_dim", _i32),
        ("perm", _vp), ("perm_sh", _i64),
        ("cent", _vp), ("cent_sh", _i64),
        ("metric", _vp), ("metric_sh", _i64),
        ("block_dim", _i32), ("n_blocks", _i32), ("n_centroids", _i32),
        ("heavy_mask", ctypes.c_uint64 * 2),
        ("codes", _vp), ("c_sb", _i64), ("c_sh", _i64), ("c_st", _i64),
        ("pt", _vp), ("pt_dtype", _i32), ("pt_dense", _i32), ("pt_sb", _i64), ("pt_sh", _i64), ("pt_st", _i64),
        ("slot_mapping", _vp), ("sm_sb", _i64), ("page_size", _i32),
        ("kernel", _i32),
        ("grid", _vp), ("grid_bytes", ctypes.c_uint64),
        ("direct_dist", _i32),
    ]

    def __init__(self, **kw):
        super().__init__()
        self.struct_size = ctypes.sizeof(EncodeArgs)
        for k, v in kw.items():
            setattr(self, k, v)
