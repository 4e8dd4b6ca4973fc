"""SunShape bundle on-disk format (drop-in for ``SunShapeBundle`` of ``sunshape.hf``).

Format version 1 of sunshape/hf.py:273-338: a ``torch.save``'d dict with keys
format_version, model_name, layers, bits_per_dim, block_dim, mode, cal_points,
dsq_steps, seed, trace_meta and codecs{str(layer): {state_dict, head_dim,
block_dim, n_centroids, c, n_refine_dsq, mode}}.

Extension (backward compatible): a codec payload may carry ``num_kv_heads``;
its state_dict then holds centroids [Hkv, nb, nc, bd] and permutations
[Hkv, D].  Payloads without the key load as the reference's per-layer codec.

Loading uses ``torch.load(weights_only=True)``: the format holds only tensors
and plain containers, so nothing in a bundle file is executed.  Model loading,
trace extraction and fitting (the rest of sunshape/hf.py) are outside this
library.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

import torch

from .codec import SunShapeBlockCodec

FORMAT_VERSION = 1


def resolve_mode_alias(mode: str) -> str:
    """sunshape/hf.py:202-218."""
    aliases = {
        "sunshape_base": "profileperm_baseline",
        "profileperm_baseline": "profileperm_baseline",
        "profileperm_sigmaq": "profileperm_baseline",
        "sunshape_mixed": "profileperm_mixed_precision",
        "profileperm_mixed_precision": "profileperm_mixed_precision",
        "baseline": "identity_baseline",
        "identity_baseline": "identity_baseline",
        "sunshape_pro": "profileperm_localmetric_dsq",
        "profileperm_localmetric_dsq": "profileperm_localmetric_dsq",
        "profileperm_sigmaq_localmetric_dsq": "profileperm_localmetric_dsq",
        "rotated": "rotated",
    }
    if mode not in aliases:
        raise ValueError(f"Unknown SunShape mode alias: {mode}")
    return aliases[mode]


def default_block_dim(bits_per_dim: float) -> int:
    """sunshape/hf.py:221-222."""
    return 8 if bits_per_dim <= 1.0 else 2


@dataclass
class SunShapeBundle:
    model_name: str
    layers: list[int]
    bits_per_dim: float
    block_dim: int
    mode: str
    cal_points: int
    dsq_steps: int
    seed: int
    codecs: dict[int, SunShapeBlockCodec]
    trace_meta: dict = field(default_factory=dict)

    def make_cache(self, *, config=None, num_layers: int | None = None, store_codes: bool = False):
        """An HF cache whose bundle layers hold this bundle's codecs (sunshape/hf.py:267-268).

        store_codes=False is the reference's cache (keys quantised and dequantised, stored dense);
        store_codes=True keeps the codes (``SunShapeCodeLayer``; the model then attends with the
        ``"sunshape"`` attention implementation, ``cache.register_sunshape_attention``).
        """
        from .cache import SunShapeCache

        return SunShapeCache.from_codecs(codecs_dict=self.codecs, config=config, num_layers=num_layers,
                                         store_codes=store_codes)

    def state_dict(self) -> dict:
        """sunshape/hf.py:273-297."""
        codec_state = {}
        for layer_idx, codec in self.codecs.items():
            payload = {
                "state_dict": {k: v.detach().cpu() for k, v in codec.state_dict().items()},
                "head_dim": codec.head_dim,
                "block_dim": codec.block_dim,
                "n_centroids": codec.n_centroids,
                "c": codec.c,
                "n_refine_dsq": codec.n_refine_dsq,
                "mode": codec.mode,
            }
            if codec.num_kv_heads is not None:
                payload["num_kv_heads"] = int(codec.num_kv_heads)
            codec_state[str(layer_idx)] = payload
        return {
            "format_version": FORMAT_VERSION,
            "model_name": self.model_name,
            "layers": list(self.layers),
            "bits_per_dim": self.bits_per_dim,
            "block_dim": self.block_dim,
            "mode": self.mode,
            "cal_points": self.cal_points,
            "dsq_steps": self.dsq_steps,
            "seed": self.seed,
            "trace_meta": dict(self.trace_meta),
            "codecs": codec_state,
        }

    def save(self, path: str | Path) -> Path:
        """sunshape/hf.py:299-303."""
        path = Path(path)
        path.parent.mkdir(parents=True, exist_ok=True)
        torch.save(self.state_dict(), path)
        return path

    @classmethod
    def from_state_dict(cls, obj: dict, *, device: torch.device | None = None) -> "SunShapeBundle":
        if not isinstance(obj, dict) or "codecs" not in obj:
            raise ValueError("Invalid SunShape bundle file.")
        if int(obj.get("format_version", FORMAT_VERSION)) != FORMAT_VERSION:
            raise ValueError(f"Unsupported SunShape bundle format_version {obj.get('format_version')}")
        device = torch.device(device) if device is not None else torch.device("cuda")
        codecs: dict[int, SunShapeBlockCodec] = {}
        for layer_idx_str, payload in obj["codecs"].items():
            nkv = payload.get("num_kv_heads")
            codec = SunShapeBlockCodec(
                head_dim=int(payload["head_dim"]),
                block_dim=int(payload["block_dim"]),
                n_centroids=int(payload["n_centroids"]),
                c=float(payload.get("c", 5.0)),
                n_refine_dsq=int(payload.get("n_refine_dsq", 3)),
                mode=str(payload["mode"]),
                device=device,
                num_kv_heads=None if nkv is None else int(nkv),
            )
            codec.load_state_dict(payload["state_dict"])
            codec.to(device)
            codecs[int(layer_idx_str)] = codec
        return cls(
            model_name=str(obj["model_name"]),
            layers=[int(x) for x in obj["layers"]],
            bits_per_dim=float(obj["bits_per_dim"]),
            block_dim=int(obj["block_dim"]),
            mode=str(obj["mode"]),
            cal_points=int(obj["cal_points"]),
            dsq_steps=int(obj["dsq_steps"]),
            seed=int(obj["seed"]),
            codecs=codecs,
            trace_meta=dict(obj.get("trace_meta", {})),
        )

    @classmethod
    def load(cls, path: str | Path, *, device: torch.device | None = None) -> "SunShapeBundle":
        """sunshape/hf.py:305-338, with a loader that executes nothing from the file."""
        obj = torch.load(path, map_location="cpu", weights_only=True)
        return cls.from_state_dict(obj, device=device)
