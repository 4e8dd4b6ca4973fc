"""Runtime state the decode call reads (drop-in for the parts of ``sunshape.integration.vllm``
on the decode path).

``SunShapeVLLMRuntimeState.codec_for_layer`` (sunshape/integration/vllm.py:127-158) and
``load_runtime_state`` (:237-265) are what ``SunShapeAttentionImpl`` needs.  The config /
engine-args / env export and ``install_hooks`` into a live vLLM (:18-81, :268-341) are
outside this library: ``install_hooks`` raises when vLLM is not importable, as the
reference does (:294-300).
"""

from __future__ import annotations

import importlib
import json
import os
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any, Iterable

import torch

DEFAULT_BACKEND_MODULE = "sunshape_amd.vllm_attn_backend"


@dataclass
class SunShapeVLLMConfig:
    """Launch description of a SunShape-enabled vLLM deployment (sunshape/integration/vllm.py:45-81)."""

    model_name: str
    bundle_path: str
    mode: str = "sunshape_base"
    bits_per_dim: float = 4.0
    block_dim: int = 2
    layers: list[int] = field(default_factory=list)
    backend_module: str = DEFAULT_BACKEND_MODULE
    connector_name: str = "SUNSHAPE"

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    def write_json(self, path: str | Path) -> Path:
        path = Path(path)
        path.write_text(json.dumps(self.to_dict(), indent=2))
        return path


@dataclass
class SunShapeVLLMHandle:
    config: SunShapeVLLMConfig
    hooks_installed: bool
    backend_module: str | None = None
    connector_registered: bool = False
    runtime_patch_available: bool = False
    vllm_version: str | None = None
    notes: list[str] = field(default_factory=list)

    def to_dict(self) -> dict[str, Any]:
        return {
            "config": self.config.to_dict(),
            "hooks_installed": self.hooks_installed,
            "backend_module": self.backend_module,
            "connector_registered": self.connector_registered,
            "runtime_patch_available": self.runtime_patch_available,
            "vllm_version": self.vllm_version,
            "notes": list(self.notes),
        }


@dataclass
class SunShapeVLLMRuntimeState:
    """Loaded bundle + metadata; the decode call asks it for a layer's codec."""

    bundle_path: str
    model_name: str
    mode: str
    bits_per_dim: float
    block_dim: int
    layers: list[int]
    bundle: Any
    device: str
    backend_module: str = DEFAULT_BACKEND_MODULE
    beta: bool = True

    def codec_for_layer(self, layer_idx: int):
        return self.bundle.codecs.get(int(layer_idx))

    def supports_layer(self, layer_idx: int) -> bool:
        return int(layer_idx) in self.bundle.codecs

    def to_dict(self) -> dict[str, Any]:
        return {
            "bundle_path": self.bundle_path,
            "model_name": self.model_name,
            "mode": self.mode,
            "bits_per_dim": self.bits_per_dim,
            "block_dim": self.block_dim,
            "layers": list(self.layers),
            "device": self.device,
            "backend_module": self.backend_module,
            "beta": self.beta,
            "trace_meta": dict(getattr(self.bundle, "trace_meta", {})),
        }


def load_runtime_state(
    *,
    bundle_path: str | Path,
    model_name: str,
    mode: str,
    bits_per_dim: float,
    block_dim: int,
    layers: Iterable[int],
    backend_module: str = DEFAULT_BACKEND_MODULE,
    device: str | torch.device | None = None,
) -> SunShapeVLLMRuntimeState:
    """sunshape/integration/vllm.py:237-265."""
    from ..hf import SunShapeBundle

    bundle_path = Path(bundle_path)
    if not bundle_path.exists():
        raise FileNotFoundError(f"SunShape vLLM bundle does not exist: {bundle_path}")
    device_obj = torch.device(device) if device is not None else torch.device("cuda")
    bundle = SunShapeBundle.load(bundle_path, device=device_obj)
    runtime_layers = [int(x) for x in layers] if layers else list(bundle.layers)
    return SunShapeVLLMRuntimeState(
        bundle_path=str(bundle_path), model_name=model_name, mode=mode, bits_per_dim=float(bits_per_dim),
        block_dim=int(block_dim), layers=runtime_layers, bundle=bundle, device=str(device_obj),
        backend_module=backend_module, beta=True,
    )


def install_hooks(
    *,
    bundle_path: str | Path,
    model_name: str,
    mode: str,
    bits_per_dim: float,
    block_dim: int,
    layers: Iterable[int],
) -> SunShapeVLLMHandle:
    """Register the bundle's runtime state with this library's attention backend inside a live
    vLLM (keyword-only, as sunshape/integration/vllm.py:284-291).

    Raises FileNotFoundError for a missing bundle and RuntimeError when vLLM is not importable
    (the reference's order, :293-300).  With vLLM present it loads the bundle
    (``load_runtime_state``), hands it to ``sunshape_amd.vllm_attn_backend`` and selects the
    backend through ``VLLM_ATTENTION_BACKEND``; patching vLLM's own modules is not done here.
    """
    bundle_path = Path(bundle_path)
    if not bundle_path.exists():
        raise FileNotFoundError(f"SunShape vLLM bundle does not exist: {bundle_path}")
    try:
        vllm = importlib.import_module("vllm")
    except Exception as exc:  # vLLM is not a dependency
        raise RuntimeError("vLLM is not installed; SunShape hooks cannot be installed.") from exc
    layer_list = [int(x) for x in layers]
    config = SunShapeVLLMConfig(model_name=model_name, bundle_path=str(bundle_path), mode=mode,
                                bits_per_dim=float(bits_per_dim), block_dim=int(block_dim), layers=layer_list)
    handle = SunShapeVLLMHandle(config=config, hooks_installed=False, backend_module=config.backend_module,
                                vllm_version=getattr(vllm, "__version__", None))
    backend = importlib.import_module(config.backend_module)
    state = load_runtime_state(bundle_path=bundle_path, model_name=model_name, mode=mode,
                               bits_per_dim=bits_per_dim, block_dim=block_dim, layers=layer_list,
                               backend_module=config.backend_module)
    backend.register_runtime_state(state)
    os.environ["VLLM_ATTENTION_BACKEND"] = config.connector_name
    handle.hooks_installed = True
    handle.notes.append("Registered SunShape runtime state with the attention backend.")
    return handle
