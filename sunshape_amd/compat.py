"""Run code written against the reference's import paths (``import sunshape...``) on this
library, without editing it.

``install()`` registers this package's modules in ``sys.modules`` under the reference's module
names, for the modules on the decode path:

    sunshape.codec              -> sunshape_amd.codec
    sunshape.triton_kernels     -> sunshape_amd.triton_kernels
    sunshape.vllm_attn_backend  -> sunshape_amd.vllm_attn_backend
    sunshape.hf                 -> sunshape_amd.hf
    sunshape.cache              -> sunshape_amd.cache
    sunshape.integration        -> sunshape_amd.integration
    sunshape.integration.vllm   -> sunshape_amd.integration.vllm

so that, for instance, a deployment whose own code (or the reference's
``codec.attention_scores``, sunshape/codec.py:404-408) imports ``sunshape.triton_kernels``
reaches these kernels.  It is opt-in and refuses to run when a ``sunshape`` package is already
imported or importable (``force=True`` overrides that): aliasing over the reference would make
it unreachable in this process.  The reference's modules outside the decode path (CLI, server,
fitting, evaluation) have no counterpart here, and importing them afterwards raises
ModuleNotFoundError.
"""

from __future__ import annotations

import importlib
import importlib.util
import sys
import types

ALIASES = {
    "sunshape.codec": "sunshape_amd.codec",
    "sunshape.triton_kernels": "sunshape_amd.triton_kernels",
    "sunshape.vllm_attn_backend": "sunshape_amd.vllm_attn_backend",
    "sunshape.hf": "sunshape_amd.hf",
    "sunshape.cache": "sunshape_amd.cache",
    "sunshape.integration": "sunshape_amd.integration",
    "sunshape.integration.vllm": "sunshape_amd.integration.vllm",
}


def installed() -> bool:
    return getattr(sys.modules.get("sunshape"), "__sunshape_amd_alias__", False)


def install(force: bool = False) -> types.ModuleType:
    """Register the aliases; returns the ``sunshape`` package module.  Idempotent."""
    if installed():
        return sys.modules["sunshape"]
    if not force:
        if "sunshape" in sys.modules:
            raise RuntimeError("a 'sunshape' package is already imported; install(force=True) would shadow it")
        if importlib.util.find_spec("sunshape") is not None:
            raise RuntimeError("a 'sunshape' package is importable; install(force=True) would shadow it")
    pkg = types.ModuleType("sunshape", "sunshape_amd under the reference's package name (sunshape_amd.compat)")
    pkg.__path__ = []  # a package, so that the submodule names below resolve
    pkg.__sunshape_amd_alias__ = True
    sys.modules["sunshape"] = pkg
    for alias, target in ALIASES.items():
        mod = importlib.import_module(target)
        sys.modules[alias] = mod
        parent, _, leaf = alias.rpartition(".")
        setattr(sys.modules[parent], leaf, mod)
    return pkg
