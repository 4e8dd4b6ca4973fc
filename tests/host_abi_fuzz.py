"""Drives the library's host code (argument checks, kernel choice, launch plans, workspace sizes)
with arbitrary arguments, for tests/test_host_sanitizers.py.  Run as a script in a process whose
LD_PRELOAD holds the AddressSanitizer runtime, against the host-sanitized build
(sunshape_amd/build.py: build_host_sanitized), in a process that sees no GPU, so every launch a
plan reaches fails at the runtime instead of running.  Device pointers
are fake (aligned or not) addresses the host code only inspects, never dereferences.

usage: python host_abi_fuzz.py <libsunshape_amd_hostsan.so> <examples>
"""

import ctypes
import importlib.util
import os
import sys

from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("ssq_abi", os.path.join(HERE, "..", "sunshape_amd", "_abi.py"))
abi = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(abi)

lib = ctypes.CDLL(sys.argv[1])
N_EXAMPLES = int(sys.argv[2]) if len(sys.argv) > 2 else 1500
P = ctypes.POINTER
vp = ctypes.c_void_p
lib.ssq_decode_workspace_size.argtypes = [P(abi.DecodeArgs)]
lib.ssq_decode_workspace_size.restype = ctypes.c_size_t
lib.ssq_decode.argtypes = [P(abi.DecodeArgs), vp, ctypes.c_size_t, vp]
lib.ssq_decode_noalloc.argtypes = [P(abi.DecodeArgs), vp]
lib.ssq_attention_scores.argtypes = [P(abi.DecodeArgs), vp]
lib.ssq_encode.argtypes = [P(abi.EncodeArgs), vp]
lib.ssq_encode_grid_bytes.argtypes = [P(abi.EncodeArgs)]
lib.ssq_encode_grid_bytes.restype = ctypes.c_uint64
lib.ssq_encode_grid_build.argtypes = [P(abi.EncodeArgs), vp, ctypes.c_uint64, vp]
lib.ssq_dequantize.argtypes = [vp, ctypes.c_int64, ctypes.c_int32, vp, vp, ctypes.c_int32, ctypes.c_int32,
                               ctypes.c_int32, vp, ctypes.c_int32, vp, ctypes.c_int32, ctypes.c_int64, vp,
                               ctypes.c_int64, vp]
lib.ssq_pack_codes.argtypes = [vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, vp,
                               ctypes.c_int64, vp]
lib.ssq_last_error.restype = ctypes.c_char_p

ALIGNED = 1 << 32  # fake device addresses: multiples of 256, or off by a few bytes
ptr = st.one_of(st.just(0), st.integers(1, 1 << 20).map(lambda k: ALIGNED + 256 * k),
                st.integers(1, 1 << 20).map(lambda k: ALIGNED + 256 * k + 2), st.just(ALIGNED + 1))
stride = st.one_of(st.integers(-4, 4), st.sampled_from([0, 8, 16, 32, 64, 128, 129, 512, 4096, 1 << 20, 1 << 31,
                                                        -(1 << 20), (1 << 40)]))
dims = st.sampled_from([-1, 0, 1, 2, 16, 32, 48, 64, 96, 128, 192, 256, 512, 1024, 4096])
small = st.integers(-2, 130)
ncent = st.sampled_from([-1, 0, 1, 16, 64, 100, 255, 256, 257, 4096, 65535, 65536, (1 << 20), (1 << 20) + 1])
bdim = st.sampled_from([-1, 0, 1, 2, 3, 4, 8, 16, 17, 32])
dtype = st.integers(-1, 3)
u64 = st.one_of(st.just(0), st.integers(0, (1 << 64) - 1), st.sampled_from([1, 0xF, 0xF0, 1 << 63]))


@st.composite
def decode_args(draw):
    hd = draw(dims)
    bd = draw(bdim)
    nb = hd // bd if bd > 0 and draw(st.booleans()) else draw(small)
    a = abi.DecodeArgs(
        q=draw(ptr), q_dtype=draw(dtype), q_sb=draw(stride), q_sh=draw(stride), q_sl=draw(stride),
        batch=draw(small), num_q_heads=draw(st.sampled_from([-1, 0, 1, 7, 8, 14, 16, 32, 64, 128, 2048, 1 << 20])),
        q_len=draw(st.sampled_from([-1, 0, 1, 2, 3, 64, 512, 100000])), head_dim=hd,
        num_kv_heads=draw(st.sampled_from([-1, 0, 1, 2, 3, 8, 16])), has_scale=draw(st.integers(0, 1)),
        scale=draw(st.floats(allow_nan=True, allow_infinity=True, width=32)),
        perm=draw(ptr), perm_sh=draw(stride), cent=draw(ptr), cent_sh=draw(stride),
        block_dim=bd, n_blocks=nb, n_centroids=draw(ncent),
        pt_dense=draw(st.integers(0, 1)), pt_dtype=draw(dtype), pt=draw(ptr), pt_sb=draw(stride), pt_sh=draw(stride),
        pt_st=draw(stride), layout=draw(st.integers(-1, 2)),
        seq_len=draw(st.sampled_from([-1, 0, 1, 15, 16, 63, 64, 65, 1000, 8192, 32768, 1 << 20, (1 << 31) - 1])),
        codes=draw(ptr), c_sb=draw(stride), c_sh=draw(stride), c_st=draw(stride), block_table=draw(ptr),
        bt_sb=draw(stride), seq_lens=draw(ptr), page_size=draw(st.sampled_from([-1, 0, 7, 8, 16, 32, 64, 256, 512])),
        v=draw(ptr), v_dtype=draw(dtype), value_dim=draw(st.sampled_from([-8, 0, 8, 24, 64, 128, 256, 512])),
        v_sb=draw(stride), v_sh=draw(stride), v_st=draw(stride), mask=draw(ptr), m_sb=draw(stride),
        m_sh=draw(stride), m_sl=draw(stride), m_st=draw(stride), out=draw(ptr), o_sb=draw(stride), o_sh=draw(stride),
        o_sl=draw(stride), lse=draw(ptr), scores=draw(ptr), s_sb=draw(stride), s_sh=draw(stride), s_sl=draw(stride),
        num_splits=draw(st.sampled_from([-1, 0, 1, 2, 7, 64, 100000])), kernel=draw(st.integers(-1, 5)),
        code_bits=draw(st.sampled_from([-1, 0, 1, 3, 4, 5, 6, 7, 8, 9, 16, 32])))
    a.heavy_mask[0] = draw(u64)
    a.heavy_mask[1] = draw(u64)
    if draw(st.booleans()):
        a.struct_size = draw(st.integers(0, 1 << 16))
    return a


@st.composite
def encode_args(draw):
    hd = draw(dims)
    bd = draw(bdim)
    nb = hd // bd if bd > 0 and draw(st.booleans()) else draw(small)
    a = abi.EncodeArgs(
        keys=draw(ptr), k_dtype=draw(dtype), k_sb=draw(stride), k_sh=draw(stride), k_ss=draw(stride),
        batch=draw(small), num_kv_heads=draw(st.sampled_from([-1, 0, 1, 2, 8, 129])),
        seq_len=draw(st.sampled_from([-1, 0, 1, 25, 26, 1023, 1024, 16384, 1 << 24])), head_dim=hd,
        perm=draw(ptr), perm_sh=draw(stride), cent=draw(ptr), cent_sh=draw(stride), metric=draw(ptr),
        metric_sh=draw(stride), block_dim=bd, n_blocks=nb, n_centroids=draw(ncent), codes=draw(ptr),
        c_sb=draw(stride), c_sh=draw(stride), c_st=draw(stride), pt=draw(ptr), pt_dtype=draw(dtype),
        pt_dense=draw(st.integers(0, 1)), pt_sb=draw(stride), pt_sh=draw(stride), pt_st=draw(stride),
        slot_mapping=draw(ptr), sm_sb=draw(stride), page_size=draw(st.sampled_from([-1, 0, 1, 16, 4096])),
        kernel=draw(st.integers(-1, 4)), grid=draw(ptr),
        grid_bytes=draw(st.sampled_from([0, 1, 1 << 20, 1 << 40])), direct_dist=draw(st.integers(-1, 2)))
    a.heavy_mask[0] = draw(u64)
    a.heavy_mask[1] = draw(u64)
    if draw(st.booleans()):
        a.struct_size = draw(st.integers(0, 1 << 16))
    return a


# Consistent problems (contiguous strides, plausible shapes) that pass the argument checks and reach
# kernel choice, launch planning and workspace sizing, then optionally one field overwritten with
# an edge value: the shallow strategies above mostly stop at the first check.
DEC_EDGES = dict(q_sb=stride, q_sh=stride, q_sl=stride, batch=small, num_q_heads=small, q_len=small, head_dim=dims,
                 num_kv_heads=small, perm_sh=stride, cent_sh=stride, block_dim=bdim, n_blocks=small,
                 n_centroids=ncent, pt_sb=stride, pt_sh=stride, pt_st=stride, pt_dtype=dtype, seq_len=small,
                 c_sb=stride, c_sh=stride, c_st=stride, bt_sb=stride, page_size=small, value_dim=dims,
                 v_sb=stride, v_sh=stride, v_st=stride, m_sb=stride, m_sh=stride, m_sl=stride, m_st=stride,
                 o_sb=stride, o_sh=stride, o_sl=stride, s_sb=stride, s_sh=stride, s_sl=stride,
                 num_splits=st.integers(-1, 70000), kernel=st.integers(-1, 5), code_bits=st.integers(-1, 33),
                 q=ptr, v=ptr, pt=ptr, mask=ptr, out=ptr, lse=ptr, scores=ptr, codes=ptr, block_table=ptr,
                 seq_lens=ptr, q_dtype=dtype, v_dtype=dtype)


def _aligned(draw):
    return ALIGNED + 256 * draw(st.integers(1, 1 << 24))


@st.composite
def consistent_decode_args(draw):
    hd = draw(st.sampled_from([32, 64, 96, 128, 256]))
    bd = draw(st.sampled_from([b for b in (1, 2, 4, 8, 16) if hd % b == 0 and hd // b <= 128]))
    nb = hd // bd
    nc = draw(st.sampled_from([1, 16, 64, 256, 257, 4096, 65535, 65536, 1 << 20]))
    hkv = draw(st.sampled_from([1, 2, 8]))
    hq = hkv * draw(st.sampled_from([1, 2, 4, 7, 8, 16]))
    B, Lq = draw(st.integers(1, 4)), draw(st.sampled_from([1, 1, 2, 3, 8]))
    paged = draw(st.booleans())
    T = draw(st.sampled_from([1, 15, 16, 17, 255, 1024, 4096, 32768]))
    dv = draw(st.sampled_from([64, 128, hd]))
    scores_only = draw(st.integers(0, 3)) == 0
    width = 1 if nc <= 256 else 2 if nc <= 65535 else 4
    bits = draw(st.sampled_from([0, 0, 0, 4, 6, 8, 3])) if nc <= 256 else 0
    cw = -(-nb // (32 // bits)) if bits else nb  # code row length in elements of its storage
    a = abi.DecodeArgs(q=_aligned(draw), q_dtype=draw(st.integers(0, 2)), q_sl=hd, q_sh=Lq * hd, q_sb=hq * Lq * hd,
                       batch=B, num_q_heads=hq, q_len=Lq, head_dim=hd, num_kv_heads=hkv,
                       has_scale=draw(st.integers(0, 1)), scale=0.125, perm=_aligned(draw),
                       perm_sh=draw(st.sampled_from([0, hd])), cent=_aligned(draw),
                       cent_sh=draw(st.sampled_from([0, nb * nc * bd])), block_dim=bd, n_blocks=nb, n_centroids=nc,
                       layout=int(paged), seq_len=T, codes=_aligned(draw), code_bits=bits,
                       num_splits=draw(st.sampled_from([0, 0, 1, 2, 5])), kernel=draw(st.integers(0, 4)))
    heavy = [i for i in range(nb) if draw(st.integers(0, 7)) == 0] if draw(st.booleans()) else []
    for i in heavy:
        a.heavy_mask[i // 64] |= 1 << (i % 64)
    if paged:
        page = draw(st.sampled_from([8, 16, 32, 64]))
        pages = -(-T // page)
        a.page_size, a.block_table, a.bt_sb, a.seq_lens = page, _aligned(draw), pages, _aligned(draw)
        a.c_st, a.c_sh, a.c_sb = cw, page * cw, hkv * page * cw
    else:
        a.c_st, a.c_sh, a.c_sb = cw, T * cw, hkv * T * cw
    if heavy:
        a.pt_dense = draw(st.integers(0, 1))
        a.pt_dtype = draw(st.integers(0, 2))
        slots = nb if a.pt_dense else len(heavy)
        rows = page if paged else T
        a.pt, a.pt_st = _aligned(draw), slots * bd
        a.pt_sh, a.pt_sb = rows * slots * bd, hkv * rows * slots * bd
    if draw(st.booleans()):
        a.mask, a.m_st = _aligned(draw), 1
        a.m_sl = draw(st.sampled_from([0, T]))
        a.m_sh = draw(st.sampled_from([0, Lq * T]))
        a.m_sb = draw(st.sampled_from([0, hq * Lq * T]))
    if not scores_only:
        a.v, a.v_dtype, a.value_dim = _aligned(draw), draw(st.integers(1, 2)), dv
        if paged:
            a.v_st, a.v_sh, a.v_sb = page, dv * page, hkv * dv * page
        else:
            a.v_st, a.v_sh, a.v_sb = dv, T * dv, hkv * T * dv
        a.out, a.o_sl, a.o_sh, a.o_sb = _aligned(draw), dv, Lq * dv, hq * Lq * dv
        if draw(st.booleans()):
            a.lse = _aligned(draw)
    if scores_only or draw(st.integers(0, 3)) == 0:
        a.scores, a.s_sl, a.s_sh, a.s_sb = _aligned(draw), T, Lq * T, hq * Lq * T
    if draw(st.booleans()):
        name = draw(st.sampled_from(sorted(DEC_EDGES)))
        setattr(a, name, draw(DEC_EDGES[name]))
    return a


ENC_EDGES = dict(k_sb=stride, k_sh=stride, k_ss=stride, batch=small, num_kv_heads=small, seq_len=small,
                 head_dim=dims, perm_sh=stride, cent_sh=stride, metric_sh=stride, block_dim=bdim, n_blocks=small,
                 n_centroids=ncent, c_sb=stride, c_sh=stride, c_st=stride, pt_dtype=dtype, pt_sb=stride,
                 pt_sh=stride, pt_st=stride, sm_sb=stride, page_size=small, kernel=st.integers(-1, 4),
                 grid_bytes=st.sampled_from([0, 1, 1 << 20, 1 << 40]), direct_dist=st.integers(-1, 2),
                 keys=ptr, codes=ptr, pt=ptr, slot_mapping=ptr, grid=ptr, k_dtype=dtype)


@st.composite
def consistent_encode_args(draw):
    hd = draw(st.sampled_from([32, 64, 96, 128, 256]))
    bd = draw(st.sampled_from([b for b in (1, 2, 4, 8, 16) if hd % b == 0 and hd // b <= 128]))
    nb = hd // bd
    nc = draw(st.sampled_from([1, 16, 25, 64, 256, 257, 4096, 65536, 1 << 20]))
    hkv, B = draw(st.sampled_from([1, 2, 8])), draw(st.integers(1, 3))
    S = draw(st.sampled_from([1, 25, 26, 1000, 16384]))
    width = 1 if nc <= 256 else 2 if nc <= 65535 else 4
    a = abi.EncodeArgs(keys=_aligned(draw), k_dtype=draw(st.integers(0, 2)), k_ss=hd, k_sh=S * hd, k_sb=hkv * S * hd,
                       batch=B, num_kv_heads=hkv, seq_len=S, head_dim=hd, perm=_aligned(draw),
                       perm_sh=draw(st.sampled_from([0, hd])), cent=_aligned(draw),
                       cent_sh=draw(st.sampled_from([0, nb * nc * bd])), block_dim=bd, n_blocks=nb, n_centroids=nc,
                       codes=_aligned(draw), kernel=draw(st.integers(0, 3)), direct_dist=draw(st.integers(0, 1)))
    del width
    if draw(st.booleans()):
        a.metric, a.metric_sh = _aligned(draw), draw(st.sampled_from([0, hd * hd]))
    heavy = [i for i in range(nb) if draw(st.integers(0, 7)) == 0] if draw(st.booleans()) else []
    for i in heavy:
        a.heavy_mask[i // 64] |= 1 << (i % 64)
    slots = 0
    if heavy:
        a.pt_dense, a.pt_dtype = draw(st.integers(0, 1)), draw(st.integers(0, 2))
        slots = nb if a.pt_dense else len(heavy)
        a.pt = _aligned(draw)
    if draw(st.booleans()):
        page = draw(st.sampled_from([16, 64]))
        a.slot_mapping, a.sm_sb, a.page_size = _aligned(draw), S, page
        a.c_st, a.c_sh, a.c_sb = nb, page * nb, hkv * page * nb
        if heavy:
            a.pt_st, a.pt_sh, a.pt_sb = slots * bd, page * slots * bd, hkv * page * slots * bd
    else:
        a.c_st, a.c_sh, a.c_sb = nb, S * nb, hkv * S * nb
        if heavy:
            a.pt_st, a.pt_sh, a.pt_sb = slots * bd, S * slots * bd, hkv * S * slots * bd
    if draw(st.booleans()):
        a.grid = _aligned(draw)
        a.grid_bytes = lib.ssq_encode_grid_bytes(ctypes.byref(a))
    if draw(st.booleans()):
        name = draw(st.sampled_from(sorted(ENC_EDGES)))
        setattr(a, name, draw(ENC_EDGES[name]))
    return a


SETTINGS = settings(max_examples=N_EXAMPLES, deadline=None, derandomize=True, database=None,
                    suppress_health_check=list(HealthCheck))


@SETTINGS
@given(st.one_of(decode_args(), consistent_decode_args(), consistent_decode_args()))
def fuzz_decode(a):
    ws = lib.ssq_decode_workspace_size(ctypes.byref(a))
    rc = lib.ssq_decode(ctypes.byref(a), ALIGNED if ws else None, ws, None)
    assert rc in (0, 1, 2, 3, 4), rc
    if rc:
        assert lib.ssq_last_error()  # every failure names its reason
    rc = lib.ssq_attention_scores(ctypes.byref(a), None)
    assert rc in (0, 1, 2, 3, 4), rc
    rc = lib.ssq_decode_noalloc(ctypes.byref(a), None)
    assert rc in (0, 1, 2, 3, 4), rc


@SETTINGS
@given(st.one_of(encode_args(), consistent_encode_args(), consistent_encode_args()))
def fuzz_encode(a):
    n = lib.ssq_encode_grid_bytes(ctypes.byref(a))
    rc = lib.ssq_encode(ctypes.byref(a), None)
    assert rc in (0, 1, 2, 3, 4), rc
    rc = lib.ssq_encode_grid_build(ctypes.byref(a), a.grid, n, None)
    assert rc in (0, 1, 2, 3, 4), rc


@SETTINGS
@given(st.sampled_from([0, 1, 16, 1000]), st.sampled_from([-1, 0, 1, 2, 8, 128]), st.sampled_from([-1, 0, 1, 2, 4, 8]),
       ncent, u64, st.integers(0, 1), dtype, stride, stride, ptr)
def fuzz_misc(tokens, head_dim, bd, nc, hm, dense, pdt, c_st, o_st, p):
    mask = (ctypes.c_uint64 * 2)(hm, 0)
    rc = lib.ssq_dequantize(p, c_st, tokens, p, p, head_dim, bd, nc, ctypes.cast(mask, vp), dense, p, pdt, c_st, p,
                            o_st, None)
    assert rc in (0, 1, 2, 3, 4), rc
    rc = lib.ssq_pack_codes(p, c_st, tokens, head_dim, bd, p, o_st, None)
    assert rc in (0, 1, 2, 3, 4), rc


if __name__ == "__main__":
    fuzz_decode()
    fuzz_encode()
    fuzz_misc()
    print(f"host ABI fuzz: {3 * N_EXAMPLES} examples, no sanitizer report")
