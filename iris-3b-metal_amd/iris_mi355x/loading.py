"""Released-checkpoint loading for the MI355X engine.

A checkpoint directory holds ``config.yaml`` (a training or exported config whose ``model``
section describes the denoiser), ``model.safetensors`` (the ``IrisDiT`` state dict under the
reference's key names, FP32 or BF16) and, for Iris-3B Turbo, ``distill.yaml`` (the distillation
recipe that pins the four sampling sigmas). This mirrors src/iris_metal/loading.py:15-77 and
src/iris_metal/turbo.py:16-35:

- ``load_config`` reads the ``model`` section into a ``ModelConfig`` (unknown keys dropped,
  missing keys at the Iris-3B defaults, as ``inference_config`` merges over its schema);
- ``open_weights`` maps the safetensors file lazily: the header is read once, every key and
  shape is checked against the configuration's parameter schema (``strict`` like
  ``load_state_dict(strict=True)``), and a tensor is read from the file only when the engine
  asks for it, so the FP32 checkpoint is never resident as a whole;
- ``load_engine`` builds ``HipIris`` from the directory. The precision plan is the engine's:
  trunk and pixel-stage Linear weights BF16 (the reference keeps the pixel stage BF16 whenever
  the trunk is reduced precision), the per-pixel MLP, norm gains, adaLN biases and position
  tables FP32;
- ``load_turbo_sigmas`` accepts only the official deterministic four-step TDM recipe.

YAML is read with ``yaml.safe_load``; OmegaConf interpolations are not resolved (released
configs carry none in the sections read here).
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from pathlib import Path

import torch
import yaml

from .config import ModelConfig
from .sampling import TURBO_SIGMAS
from .weights import parameter_schema

CONFIG_FILE = "config.yaml"
WEIGHTS_FILE = "model.safetensors"
DISTILL_FILE = "distill.yaml"


def _read_yaml(path: Path) -> dict:
    with open(path, encoding="utf-8") as f:
        data = yaml.safe_load(f)
    if not isinstance(data, dict):
        raise ValueError(f"{path} does not hold a mapping")
    return data


def load_config(checkpoint: str | Path, overrides: dict | None = None) -> ModelConfig:
    """The ``model`` section of ``<checkpoint>/config.yaml`` (src/iris_metal/loading.py:15-17);
    ``overrides`` replaces individual model keys (``{"pixel": {...}}`` merges one level down)."""
    raw = _read_yaml(Path(checkpoint) / CONFIG_FILE)
    model = raw.get("model")
    if not isinstance(model, dict):
        raise ValueError(f"{CONFIG_FILE} has no 'model' mapping")
    model = dict(model)
    for key, value in (overrides or {}).items():
        if key == "pixel" and isinstance(value, dict):
            model["pixel"] = {**(model.get("pixel") or {}), **value}
        else:
            model[key] = value
    cfg = ModelConfig.from_mapping(model)
    cfg.validate()
    return cfg


class SafetensorsWeights(Mapping):
    """Read-only mapping over a safetensors file that reads each tensor on access (CPU)."""

    def __init__(self, path: str | Path):
        from safetensors import safe_open

        self.path = Path(path)
        self._file = safe_open(str(self.path), framework="pt", device="cpu")
        self._keys = list(self._file.keys())
        self._key_set = set(self._keys)

    def shape(self, key: str) -> tuple[int, ...]:
        return tuple(self._file.get_slice(key).get_shape())

    def __getitem__(self, key: str) -> torch.Tensor:
        if key not in self._key_set:
            raise KeyError(key)
        return self._file.get_tensor(key)

    def __contains__(self, key: object) -> bool:
        return key in self._key_set

    def __iter__(self) -> Iterator[str]:
        return iter(self._keys)

    def __len__(self) -> int:
        return len(self._keys)


def open_weights(checkpoint: str | Path, cfg: ModelConfig, strict: bool = True) -> SafetensorsWeights:
    """``<checkpoint>/model.safetensors`` checked against ``cfg``'s parameter schema: every
    expected key present with its shape, and (``strict``) no unexpected key."""
    weights = SafetensorsWeights(Path(checkpoint) / WEIGHTS_FILE)
    schema = parameter_schema(cfg)
    missing = sorted(set(schema) - set(weights))
    extra = sorted(set(weights) - set(schema)) if strict else []
    if missing or extra:
        raise ValueError(f"checkpoint does not match the model config: missing {missing[:5]}"
                         f"{' ...' if len(missing) > 5 else ''}, unexpected {extra[:5]}{' ...' if len(extra) > 5 else ''}")
    for name, spec in schema.items():
        shape = weights.shape(name)
        if shape != spec.shape:
            raise ValueError(f"checkpoint tensor {name} has shape {shape}, the config expects {spec.shape}")
    return weights


def load_engine(checkpoint: str | Path, device: str | torch.device = "cuda", overrides: dict | None = None,
                strict: bool = True, graphs: bool = True):
    """``HipIris`` for a released checkpoint directory (src/iris_metal/loading.py:67-77 and
    pipeline.py:133-142). Tensors are read, converted and moved one at a time."""
    from .engine import HipIris

    cfg = load_config(checkpoint, overrides)
    return HipIris(cfg, open_weights(checkpoint, cfg, strict), device=device, graphs=graphs)


def load_turbo_sigmas(checkpoint: str | Path) -> tuple[float, ...] | None:
    """The Turbo sampling sigmas from ``<checkpoint>/distill.yaml``, or None without that file;
    only the official deterministic four-step TDM recipe is accepted (turbo.py:16-35)."""
    path = Path(checkpoint) / DISTILL_FILE
    if not path.exists():
        return None
    dmd = _read_yaml(path).get("dmd")
    sigmas = dmd.get("sigmas") if isinstance(dmd, dict) else None
    official = (
        isinstance(sigmas, list)
        and all(type(s) in (int, float) for s in sigmas)  # (bool is not a number here)
        and tuple(float(s) for s in sigmas) == TURBO_SIGMAS
        and dmd.get("method") == "tdm"
        and dmd.get("deterministic") is True
    )
    if not official:
        raise ValueError("unsupported Turbo distill.yaml: expected official deterministic four-step TDM recipe")
    return TURBO_SIGMAS
