"""The reference's import paths reach this library after sunshape_amd.compat.install() (no GPU).
Run in a child interpreter: the aliases are process-wide."""

import subprocess
import sys
import textwrap


def _run(code):
    return subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True, timeout=120)


def test_reference_import_paths_resolve_to_this_library():
    res = _run("""
        from sunshape_amd import compat
        compat.install()
        import sunshape.triton_kernels as tk
        from sunshape.codec import SunShapeBlockCodec
        from sunshape.vllm_attn_backend import SunShapeAttentionImpl, quantize_key_states
        from sunshape.integration.vllm import install_hooks, load_runtime_state
        from sunshape.hf import SunShapeBundle
        import sunshape_amd.codec, sunshape_amd.triton_kernels
        assert SunShapeBlockCodec is sunshape_amd.codec.SunShapeBlockCodec
        assert tk.sunshape_attention_scores is sunshape_amd.triton_kernels.sunshape_attention_scores
        assert compat.installed() and compat.install() is __import__("sunshape")
        try:
            import sunshape.server
        except ModuleNotFoundError:
            print("ok")
    """)
    assert res.returncode == 0, res.stderr
    assert res.stdout.strip() == "ok"


def test_install_refuses_to_shadow_an_imported_sunshape():
    res = _run("""
        import sys, types
        sys.modules["sunshape"] = types.ModuleType("sunshape")
        from sunshape_amd import compat
        try:
            compat.install()
        except RuntimeError as e:
            print("refused:", e)
    """)
    assert res.returncode == 0, res.stderr
    assert res.stdout.startswith("refused:")
