"""Host-side behaviour of the drop-in Python surface (no GPU needed).

Gate strings follow sunshape/triton_kernels.py:327-363 and
sunshape/vllm_attn_backend.py:159-194; everything that would reach a kernel
with CPU tensors must raise instead (no CPU path exists)."""

import math

import pytest
import torch

from sunshape_amd import hip_ops
from sunshape_amd.codec import SunShapeBlockCodec, SunShapeQuantized, _invert_permutation
from sunshape_amd.hf import SunShapeBundle, default_block_dim, resolve_mode_alias
from sunshape_amd.integration.vllm import SunShapeVLLMRuntimeState
from sunshape_amd.kernels import _triton_fast_path_unavailable_reason, require_triton_fast_path
from sunshape_amd import synthetic
from sunshape_amd import vllm_attn_backend as VB


def _codec(nkv=None, mode="profileperm_baseline"):
    g = torch.Generator().manual_seed(0)
    D, bd = 64, 8
    shape = (() if nkv is None else (nkv,)) + (D // bd, 256, bd)
    cent = torch.randn(*shape, generator=g)
    perm = torch.randperm(D, generator=g) if nkv is None else torch.stack([torch.randperm(D, generator=g) for _ in range(nkv)])
    return SunShapeBlockCodec.from_buffers(perm, cent, mode=mode, device="cpu")


def test_codec_buffers_match_reference_layout():
    c = SunShapeBlockCodec(head_dim=64, block_dim=8, device="cpu")
    sd = c.state_dict()
    assert set(sd) == {"E", "E_inv", "centroids", "dsq_block_affinity", "dsq_active_blocks",
                       "mixed_high_precision_blocks", "mixed_block_mass", "permutation", "inv_permutation", "rotation"}
    assert sd["centroids"].shape == (8, 256, 8)
    assert sd["permutation"].dtype == torch.long
    with pytest.raises(ValueError):
        SunShapeBlockCodec(head_dim=64, block_dim=7, device="cpu")


def test_per_kv_head_codec_and_inverse_permutation():
    c = _codec(nkv=3)
    assert c.centroids.shape == (3, 8, 256, 8) and c.permutation.shape == (3, 64)
    x = torch.randn(5, 64)
    for h in range(3):
        y = c._forward_transform(x, kv_head=h)
        assert torch.equal(c._inverse_transform(y, kv_head=h), x)
    assert torch.equal(_invert_permutation(c.permutation)[1][c.permutation[1]], torch.arange(64))


def test_effective_permutation_identity_outside_profileperm_modes():
    c = _codec(mode="identity_baseline")
    assert torch.equal(c.effective_permutation(), torch.arange(64))
    assert not torch.equal(_codec().effective_permutation(), torch.arange(64))


def test_heavy_blocks_cached_and_refreshed():
    c = _codec(mode="profileperm_mixed_precision")
    assert c.heavy_blocks() is None
    c.mixed_high_precision_blocks[2] = True
    assert c.heavy_blocks()[2] is True and sum(c.heavy_blocks()) == 1
    c.mixed_high_precision_blocks[2] = False
    assert c.heavy_blocks() is None


def test_unsupported_modes_raise_with_reason():
    wide = SunShapeBlockCodec(head_dim=64, block_dim=8, n_centroids=1024, device="cpu")
    assert wide.unsupported_reason() is None  # 16-bit codes (the reference's int16 indices)
    with pytest.raises(RuntimeError, match="no CPU path"):
        wide.quantize(torch.randn(4, 64))
    c = SunShapeBlockCodec(head_dim=4, block_dim=4, n_centroids=(1 << 20) + 1, device="cpu")
    assert "2^20" in c.unsupported_reason()
    with pytest.raises(RuntimeError, match="2\\^20"):
        c.quantize(torch.randn(4, 4))
    rot = SunShapeBlockCodec(head_dim=64, block_dim=8, use_rotation=True, device="cpu")
    assert rot.unsupported_reason() is None and rot.rotation_matrix() is rot.rotation
    with pytest.raises(RuntimeError, match="no CPU path"):
        rot.quantize(torch.randn(4, 64))
    pro = _codec(mode="profileperm_localmetric_dsq")
    with pytest.raises(NotImplementedError):
        pro.fit(torch.randn(4, 64), torch.randn(4, 64))
    # no silent CPU path: a CPU tensor reaches the device check and raises
    with pytest.raises(RuntimeError, match="no CPU path"):
        pro.quantize(torch.randn(4, 64))


def test_encode_metric_selection():
    """SunShape-Pro and legacy modes encode under E (sunshape/codec.py:375-376); the others do not."""
    E = torch.randn(64, 64)
    for mode, has in (("profileperm_localmetric_dsq", True), ("legacy_strict", True),
                      ("profileperm_baseline", False), ("profileperm_mixed_precision", False),
                      ("identity_baseline", False)):
        cb = synthetic.make_codebook(1, 64, 8, 3)
        c = SunShapeBlockCodec.from_buffers(cb.perm[0], cb.centroids[0], mode=mode, metric=E, device="cpu")
        m = c.encode_metric()
        assert (m is not None) == has, mode
        if has:
            assert torch.equal(m, E)
    with pytest.raises(ValueError):
        SunShapeBlockCodec.from_buffers(torch.arange(64), torch.zeros(8, 256, 8), metric=torch.eye(32), device="cpu")


def test_scores_gate_reasons():
    c = _codec()
    q = torch.randn(4, 64)
    qk = SunShapeQuantized(torch.zeros(10, 8, dtype=torch.uint8), 64, 8, 8)
    assert "HIP device" in _triton_fast_path_unavailable_reason(c, q, qk)
    with pytest.raises(RuntimeError, match="HIP device"):
        require_triton_fast_path(c, q, qk)
    assert _triton_fast_path_unavailable_reason(c, q, object()) == "Quantized key must expose an .indices tensor."


def test_ops_reject_cpu_tensors_before_any_launch():
    c = _codec()
    with pytest.raises(RuntimeError, match="no CPU path"):
        hip_ops.attention_scores(torch.randn(2, 64), torch.zeros(5, 8, dtype=torch.uint8), c.permutation, c.centroids)
    with pytest.raises(RuntimeError, match="no CPU path"):
        hip_ops.encode(torch.randn(1, 1, 5, 64), c.permutation, c.centroids)
    with pytest.raises(RuntimeError, match="no CPU path"):
        c.quantize(torch.randn(3, 64))


def test_backend_gate_reasons():
    c = _codec()
    bundle = SunShapeBundle("m", [0], 1.0, 8, "profileperm_baseline", 0, 0, 0, {0: c})
    rs = SunShapeVLLMRuntimeState("p", "m", "sunshape_base", 1.0, 8, [0], bundle, "cpu")
    key = VB.SunShapeQuantizedKeys(quantized_heads=(), batch_size=2, num_kv_heads=2, seq_len=10)
    q = torch.randn(2, 4, 1, 64)
    v = torch.randn(2, 2, 10, 64)
    R = VB._quantized_fast_path_unavailable_reason
    kw = dict(runtime_state=rs, layer_idx=0, query=q, key=key, value=v, attn_mask=None, is_causal=False)
    assert R(**kw) is None
    assert R(**{**kw, "runtime_state": None}) == "No registered runtime state for quantized attention."
    assert R(**{**kw, "key": torch.randn(2, 2, 10, 64)}) == "Key payload is not SunShapeQuantizedKeys."
    assert R(**{**kw, "layer_idx": 5}) == "No codec for layer 5."
    assert R(**{**kw, "query": torch.randn(3, 4, 1, 64)}) == "Quantized key batch size does not match query batch size."
    assert R(**{**kw, "value": torch.randn(2, 2, 11, 64)}) == "Quantized key sequence length does not match value sequence length."
    assert R(**{**kw, "query": torch.randn(2, 3, 1, 64)}) == "Query head count must be divisible by kv-head count."
    assert R(**{**kw, "query": torch.randn(2, 4, 2, 64), "is_causal": True}) == \
        "Causal quantized fast path currently targets decode (query_len == 1)."
    assert R(**{**kw, "attn_mask": torch.zeros(10)}) == "Unsupported attention-mask rank for quantized fast path."
    # off the fused path a quantized payload is dequantized through the registered runtime, as the
    # reference does (sunshape/vllm_attn_backend.py:140-148, :306): none registered -> RuntimeError
    impl = VB.SunShapeAttentionImpl(layer_idx=0, runtime_state=rs)
    bad = VB.SunShapeQuantizedKeys(quantized_heads=(), batch_size=3, num_kv_heads=2, seq_len=10)
    with pytest.raises(RuntimeError, match="runtime state is required to dequantize"):
        impl.forward(q, bad, v)


def test_backend_dense_keys_go_to_delegate():
    seen = {}

    def delegate(q, k, v, **kw):
        seen.update(kw)
        return q + 1

    impl = VB.SunShapeAttentionImpl(delegate=delegate, layer_idx=None)
    VB.clear_registered_runtime()
    q = torch.randn(1, 2, 1, 8)
    out = impl.forward(q, torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8), scale=0.5)
    assert torch.equal(out, q + 1) and seen["scale"] == 0.5


def test_mask_view_matches_reference_slicing():
    B, Hq, Lq, T = 2, 6, 1, 7
    m2 = torch.randn(Lq, T)
    m3b = torch.randn(B, Lq, T)
    m3h = torch.randn(Hq, Lq, T)
    m4 = torch.randn(B, Hq, Lq, T)
    for m in (m2, m3b, m3h, m4):
        view = VB._mask_view(m, B, Hq, Lq, T).expand(B, Hq, Lq, T)
        for b in range(B):
            for kv in range(2):
                h0, h1 = kv * 3, kv * 3 + 3
                # reference: sunshape/vllm_attn_backend.py:197-213
                if m.ndim == 2:
                    ref = m.unsqueeze(0)
                elif m.ndim == 3:
                    ref = m[b].unsqueeze(0) if m.shape[0] == B else m[h0:h1]
                else:
                    ref = m[b, h0:h1]
                assert torch.equal(view[b, h0:h1], ref.expand(3, Lq, T))


def test_mode_registration_globals():
    VB.clear_registered_runtime()
    VB.clear_registered_handle()
    assert VB.get_mode() == VB.MODE_OFF
    rs = SunShapeVLLMRuntimeState("p", "m", "x", 1.0, 8, [], SunShapeBundle("m", [], 1.0, 8, "x", 0, 0, 0, {}), "cpu")
    VB.register_runtime_state(rs)
    assert VB.get_mode() == VB.MODE_ACTIVE and VB.get_registered_runtime() is rs
    assert VB.ensure_backend_registered()["runtime_loaded"]
    VB.clear_registered_runtime()
    assert VB.get_mode() == VB.MODE_OFF
    keys = VB.SunShapeQuantizedKeys(quantized_heads=("a", "b", "c", "d"), batch_size=2, num_kv_heads=2, seq_len=1)
    assert keys.head(1, 0) == "c"


def test_bundle_roundtrip_and_extension(tmp_path):
    c1 = _codec()
    c2 = _codec(nkv=2, mode="profileperm_mixed_precision")
    c2.mixed_high_precision_blocks[1] = True
    b = SunShapeBundle("model", [0, 5], 1.0, 8, "profileperm_baseline", 4096, 3, 42, {0: c1, 5: c2}, {"k": 1})
    path = b.save(tmp_path / "bundle.pt")
    obj = torch.load(path, weights_only=True)
    assert obj["format_version"] == 1 and "num_kv_heads" not in obj["codecs"]["0"]
    assert obj["codecs"]["5"]["num_kv_heads"] == 2
    b2 = SunShapeBundle.load(path, device="cpu")
    assert b2.layers == [0, 5] and b2.trace_meta == {"k": 1}
    for k, v in c2.state_dict().items():
        assert torch.equal(b2.codecs[5].state_dict()[k], v)
    assert b2.codecs[5].heavy_blocks()[1]
    torch.save({"nope": 1}, tmp_path / "bad.pt")
    with pytest.raises(ValueError):
        SunShapeBundle.load(tmp_path / "bad.pt", device="cpu")


def test_bundle_roundtrip_per_kv_head_metric(tmp_path):
    """A SunShape-Pro codec with one block metric per KV head ([Hkv, D, D]) saves and reloads."""
    g = torch.Generator().manual_seed(3)
    cent = torch.randn(2, 8, 256, 8, generator=g)
    perm = torch.stack([torch.randperm(64, generator=g) for _ in range(2)])
    E = torch.eye(64).expand(2, 64, 64) + 0.1 * torch.randn(2, 64, 64, generator=g)
    c = SunShapeBlockCodec.from_buffers(perm, cent, mode="profileperm_localmetric_dsq", metric=E, device="cpu")
    assert c.E.shape == (2, 64, 64) and c.E_inv.shape == (2, 64, 64)
    b = SunShapeBundle("model", [3], 1.0, 8, "profileperm_localmetric_dsq", 1, 0, 0, {3: c})
    b2 = SunShapeBundle.load(b.save(tmp_path / "pro.pt"), device="cpu")
    c2 = b2.codecs[3]
    for k, v in c.state_dict().items():
        assert torch.equal(c2.state_dict()[k], v), k
    assert torch.equal(c2.encode_metric(1), E[1])
    # the reference's one-metric-per-layer layout still loads into [D, D]
    c1 = SunShapeBlockCodec.from_buffers(perm[0], cent[0], mode="profileperm_localmetric_dsq", metric=E[0], device="cpu")
    b3 = SunShapeBundle.load(SunShapeBundle("m", [0], 1.0, 8, "x", 1, 0, 0, {0: c1}).save(tmp_path / "one.pt"),
                             device="cpu")
    assert b3.codecs[0].E.shape == (64, 64) and torch.equal(b3.codecs[0].E, E[0])


def test_mode_aliases_and_block_dim():
    assert resolve_mode_alias("sunshape_mixed") == "profileperm_mixed_precision"
    assert default_block_dim(1.0) == 8 and default_block_dim(4.0) == 2
    with pytest.raises(ValueError):
        resolve_mode_alias("nope")


def test_synthetic_configs_shapes():
    p = synthetic.config1()
    assert p["codes"].shape == (4096, 8) and p["centroids"].shape == (8, 256, 8)
    p = synthetic.config2(B=2, T=64)
    assert p["q"].shape == (2, 14, 1, 64) and p["q"].dtype == torch.bfloat16 and p["codes"].shape == (2, 2, 64, 8)
    p = synthetic.config4(B=2, T=64)
    assert p["code_pages"].shape == (8, 8, 16, 32) and p["v_pages"].shape == (8, 8, 128, 16)
    assert sorted(p["block_table"].flatten().tolist()) == list(range(8))
    p = synthetic.config5(B=1, S=32)
    assert p["heavy"].sum() == 4 and not p["centroids"][:, p["heavy"]].any()
    cb = synthetic.make_codebook(2, 64, 2, 0)
    # codebook coordinates follow the permuted per-dim sigma
    assert cb.centroids.shape == (2, 32, 256, 2)
    assert math.isclose(float(cb.sigma.min()), 0.1, rel_tol=2.0) and float(cb.sigma.max()) <= 3.0


def test_encode_search_grid_applies_only_where_it_is_exact_and_needs_a_device():
    """The codec's search grid serves block_dim 2 without a block metric; elsewhere (and when
    disabled) it is None, so the exhaustive encode runs.  Building one needs a device codebook."""
    g = torch.Generator().manual_seed(3)
    assert _codec().encode_search_grid(_codec().centroids) is None  # block_dim 8
    c2 = SunShapeBlockCodec.from_buffers(torch.randperm(64, generator=g), torch.randn(32, 256, 2, generator=g),
                                         device="cpu")
    c2.use_encode_grid = False
    assert c2.encode_search_grid(c2.centroids) is None
    c2.use_encode_grid = True
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        c2.encode_search_grid(c2.centroids)
    pro = SunShapeBlockCodec.from_buffers(torch.randperm(64, generator=g), torch.randn(32, 256, 2, generator=g),
                                          mode="profileperm_localmetric_dsq", metric=torch.eye(64), device="cpu")
    assert pro.encode_search_grid(pro.centroids) is None  # a block metric changes the distances


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus above 1 exits with a message before touching a device."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stderr + r.stdout)


def test_install_hooks_keyword_only_and_error_order(tmp_path):
    """sunshape/integration/vllm.py:284-300: keyword-only arguments; a missing bundle raises
    FileNotFoundError before vLLM is looked up; without vLLM it raises RuntimeError."""
    from sunshape_amd.integration.vllm import install_hooks

    kw = dict(model_name="m", mode="sunshape_base", bits_per_dim=4.0, block_dim=2, layers=[0])
    with pytest.raises(TypeError):
        install_hooks(str(tmp_path / "b.pt"), **kw)  # positional bundle_path is refused
    with pytest.raises(FileNotFoundError):
        install_hooks(bundle_path=tmp_path / "missing.pt", **kw)
    bundle = tmp_path / "b.pt"
    bundle.write_bytes(b"")
    try:
        import vllm  # noqa: F401
    except Exception:
        with pytest.raises(RuntimeError, match="vLLM is not installed"):
            install_hooks(bundle_path=bundle, **kw)


def test_encode_grid_budget_is_process_wide_lru(monkeypatch):
    """Encode search grids of every codec share one byte budget: the least recently used are dropped
    first, a grid larger than the budget is not built (the encode then scans every codeword), and a
    per-KV-head codec's one-head views share its grid.  Grids are stood in for by host buffers of the
    library's stated size (ssq_encode_grid_bytes)."""
    from sunshape_amd import codec as C
    from sunshape_amd import hip_ops

    built = []

    def fake_grid(cent, num_kv_heads=1):
        built.append(cent.data_ptr())
        return torch.empty(hip_ops.encode_grid_bytes(cent, num_kv_heads), dtype=torch.uint8)

    monkeypatch.setattr(C.hip_ops, "encode_grid", fake_grid)
    codecs = [SunShapeBlockCodec(head_dim=64, block_dim=2, num_kv_heads=2, device="cpu") for _ in range(32)]
    per = hip_ops.encode_grid_bytes(codecs[0].centroids)
    assert 20 << 20 <= per < 21 << 20  # 320 KiB per head and block, plus block headers
    old = C._GRID_BUDGET[0]
    try:
        C.set_encode_grid_budget(4 * per + 100)
        for c in codecs:
            assert c.encode_search_grid(c.centroids) is not None
            assert C.encode_grid_footprint() <= 4 * per + 100
        assert C.encode_grid_footprint() == 4 * per and len(built) == 32
        codecs[28].encode_search_grid(codecs[28].centroids)  # among the 4 most recent: a hit
        assert len(built) == 32
        head = codecs[28].encode_search_grid(codecs[28].codebook(1))  # one head's view of the same grid
        assert len(built) == 32 and head.numel() == per // 2
        codecs[0].encode_search_grid(codecs[0].centroids)  # evicted long ago: rebuilt, evicting the oldest
        assert len(built) == 33 and C.encode_grid_footprint() == 4 * per
        C.set_encode_grid_budget(per - 1)  # smaller than one grid: everything dropped, nothing built
        assert C.encode_grid_footprint() == 0
        assert codecs[5].encode_search_grid(codecs[5].centroids) is None and len(built) == 33
    finally:
        C.set_encode_grid_budget(old)


def test_encode_grid_cache_from_threads(monkeypatch):
    """Encodes on several threads share the grid budget: concurrent lookups, builds and evictions
    leave every returned grid whole and the footprint within the budget.  Grids are host stand-ins
    of the library's stated size."""
    import random
    import threading

    from sunshape_amd import codec as C
    from sunshape_amd import hip_ops

    monkeypatch.setattr(C.hip_ops, "encode_grid",
                        lambda cent, num_kv_heads=1: torch.empty(hip_ops.encode_grid_bytes(cent, num_kv_heads),
                                                                 dtype=torch.uint8))
    codecs = [SunShapeBlockCodec(head_dim=32, block_dim=2, device="cpu") for _ in range(12)]
    per = hip_ops.encode_grid_bytes(codecs[0].centroids)
    old = C._GRID_BUDGET[0]
    errors, done = [], []

    def work(seed):
        try:
            rng = random.Random(seed)
            for _ in range(150):
                c = codecs[rng.randrange(len(codecs))]
                g = c.encode_search_grid(c.centroids)
                assert g is not None and g.numel() == per
            done.append(seed)
        except Exception as e:  # reported below, with the thread's seed
            errors.append((seed, repr(e)))

    try:
        C.set_encode_grid_budget(3 * per)
        threads = [threading.Thread(target=work, args=(s,)) for s in range(8)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        assert len(done) == 8  # every thread ran its lookups to the end
        assert C.encode_grid_footprint() <= 3 * per
    finally:
        C.set_encode_grid_budget(old)
