"""Downstream task engines on the HIP forward: monocular depth and one-step restoration.

Both fine-tunes run the whole Iris-3B forward once per image (or tile) on the embedding of the
empty prompt (src/iris3b/downstream/__init__.py:1-13). The reference serves them by keeping
the upstream predictors' image handling and replacing only the model call
(src/iris_metal/tasks.py:79-150): ``MetalDepth`` installs ``predict(rgb, embeddings, mask)`` as
``DepthPredictor.model``, ``MetalRestorer`` overrides ``Restorer.restore_tile(x)``. The classes
here are those two calls on ``HipIris``:

- ``HipDepth(rgb)`` = ``IrisDepth.forward`` (src/iris3b/downstream/depth.py:30-48): RGB plus a
  zero channel into the widened embedders, model time ``num_train_timesteps``, and the 1x1
  ``depth_reducer`` folded into the pixel head, so the engine writes ``[B, 1, H, W]`` directly;
- ``HipRestorer.restore_tile(x)`` = ``x - sigma * v(x, sigma * T)``
  (src/iris3b/downstream/restoration.py:135-142, src/iris_metal/tasks.py:144-150), the update
  in the FP32 flow kernel.

``read_export`` reads a task export directory (``config.yaml`` with ``model`` / ``flow`` /
``task`` sections, ``model.safetensors``, ``empty_prompt.safetensors``), checking every key
and shape, as ``load_export`` / ``_read_export`` do (src/iris3b/downstream/__init__.py:20-40,
src/iris_metal/tasks.py:69-76).
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from dataclasses import dataclass
from pathlib import Path

import torch

from . import kernels as K
from .config import ModelConfig
from .engine import HipIris, require_finite
from .loading import CONFIG_FILE, WEIGHTS_FILE, SafetensorsWeights, _read_yaml, load_config
from .weights import ParamSpec, parameter_schema

PROMPT_FILE = "empty_prompt.safetensors"
TASKS = ("depth", "restoration")


@dataclass(frozen=True)
class TaskExport:
    cfg: ModelConfig
    settings: dict
    num_train_timesteps: int
    prediction: str
    weights: Mapping
    prompt: dict


class Prefixed(Mapping):
    """The entries of ``weights`` under ``prefix``, with the prefix removed (``IrisDepth.pixel``)."""

    def __init__(self, weights: Mapping, prefix: str):
        self.weights, self.prefix = weights, prefix
        self._keys = [k[len(prefix):] for k in weights if k.startswith(prefix)]

    def __getitem__(self, key: str) -> torch.Tensor:
        return self.weights[self.prefix + key]

    def __contains__(self, key: object) -> bool:
        return isinstance(key, str) and (self.prefix + key) in self.weights

    def __iter__(self) -> Iterator[str]:
        return iter(self._keys)

    def __len__(self) -> int:
        return len(self._keys)


def task_schema(cfg: ModelConfig, task: str) -> dict[str, ParamSpec]:
    """State-dict keys and shapes of a task model: ``IrisDiT`` for restoration; for depth the
    ``IrisDepth`` module tree, ``pixel.*`` with both embedders taking one more input channel and
    ``depth_reducer`` a ``Conv2d(C, 1, 1)`` (src/iris3b/downstream/depth.py:26-39)."""
    if task not in TASKS:
        raise ValueError(f"unknown task {task!r} (known: {TASKS})")
    base = parameter_schema(cfg)
    if task == "restoration":
        return base
    c, pp = cfg.in_channels, cfg.patch_size ** 2
    schema = {f"pixel.{k}": v for k, v in base.items()}
    schema["pixel.s_embedder.proj.weight"] = ParamSpec((cfg.hidden_size, pp * (c + 1)), "linear")
    schema["pixel.pixel_embedder.proj.weight"] = ParamSpec((cfg.pixel.hidden_size, c + 1), "linear")
    schema["depth_reducer.weight"] = ParamSpec((1, c, 1, 1), "linear")
    schema["depth_reducer.bias"] = ParamSpec((1,), "linear")
    return schema


def check_weights(weights: Mapping, schema: dict[str, ParamSpec]) -> None:
    """Every schema key present with its shape and no other key (``load_state_dict(strict=True)``)."""
    missing = sorted(set(schema) - set(weights))
    extra = sorted(set(weights) - set(schema))
    if missing or extra:
        raise ValueError(f"task weights do not match the model config: missing {missing[:5]}, unexpected {extra[:5]}")
    for name, spec in schema.items():
        shape = weights.shape(name) if hasattr(weights, "shape") else tuple(weights[name].shape)
        if tuple(shape) != spec.shape:
            raise ValueError(f"task tensor {name} has shape {tuple(shape)}, the config expects {spec.shape}")


def read_export(path: str | Path, task: str) -> TaskExport:
    """A local task export directory (the reference also fetches one from the Hub; there is
    no network here)."""
    from safetensors.torch import load_file

    path = Path(path)
    raw = _read_yaml(path / CONFIG_FILE)
    settings = raw.get("task")
    if not isinstance(settings, dict):
        raise ValueError(f"{path} is not a depth or upscaling export (its {CONFIG_FILE} has no task)")
    if settings.get("name") != task:
        raise ValueError(f"{path} holds a {settings.get('name')!r} export, not {task!r}")
    cfg = load_config(path)
    flow = raw.get("flow") or {}
    weights = SafetensorsWeights(path / WEIGHTS_FILE)
    check_weights(weights, task_schema(cfg, task))
    prompt = load_file(str(path / PROMPT_FILE))
    if set(prompt) < {"embeddings", "mask"}:
        raise ValueError(f"{PROMPT_FILE} must hold 'embeddings' and 'mask'")
    return TaskExport(cfg, dict(settings), int(flow.get("num_train_timesteps", 1000)),
                      str(flow.get("prediction", "v")), weights, prompt)


class HipDepth:
    """Relative log depth (-1 near, +1 far) of ``[B, 3, H, W]`` RGB in ``[-1, 1]`` as ``[B, 1, H, W]``
    FP32: the model call of ``DepthPredictor`` (``IrisDepth.forward``)."""

    def __init__(self, cfg: ModelConfig, weights: Mapping, prompt: dict, num_train_timesteps: int = 1000,
                 device: str | torch.device = "cuda", graphs: bool = True):
        self.engine = HipIris(cfg, Prefixed(weights, "pixel."), device=device, graphs=graphs)
        if self.engine.in_channels != cfg.in_channels + 1:
            raise ValueError("the depth model's embedders must take RGB plus one channel")
        self.engine.fold_reducer(weights["depth_reducer.weight"], weights["depth_reducer.bias"])
        self.device = self.engine.device
        self.text = self.engine.encode_text(prompt["embeddings"], prompt["mask"])
        self.time = float(num_train_timesteps)
        self.patch = cfg.patch_size
        self._x: torch.Tensor | None = None

    @classmethod
    def from_export(cls, path: str | Path, device: str | torch.device = "cuda") -> "HipDepth":
        e = read_export(path, "depth")
        return cls(e.cfg, e.weights, e.prompt, e.num_train_timesteps, device)

    @torch.no_grad()
    def __call__(self, rgb: torch.Tensor, embeddings=None, mask=None) -> torch.Tensor:
        """``embeddings`` / ``mask`` are accepted for the upstream call signature and ignored:
        the empty prompt was encoded once at construction (src/iris_metal/tasks.py:88-99)."""
        batch, channels, height, width = rgb.shape
        if channels != 3:
            raise ValueError(f"depth takes [B, 3, H, W] RGB, got {tuple(rgb.shape)}")
        shape = (batch, 4, height, width)
        if self._x is None or tuple(self._x.shape) != shape:
            self._x = torch.zeros(shape, device=self.device, dtype=torch.float32)  # channel 3 stays zero
        self._x[:, :3].copy_(rgb)
        t = torch.full((batch,), self.time, device=self.device, dtype=torch.float32)
        return require_finite(self.engine(self._x, t, self.text.expand(batch, -1, -1)))


class HipRestorer:
    """One-step restoration of ``[B, 3, tile, tile]`` crops in ``[-1, 1]``: ``Restorer.restore_tile``."""

    def __init__(self, cfg: ModelConfig, weights: Mapping, prompt: dict, settings: dict,
                 num_train_timesteps: int = 1000, prediction: str = "v", device: str | torch.device = "cuda",
                 graphs: bool = True):
        if prediction != "v":
            raise ValueError("the restorer expects a v-prediction parent")
        self.engine = HipIris(cfg, weights, device=device, graphs=graphs)
        self.device = self.engine.device
        self.text = self.engine.encode_text(prompt["embeddings"], prompt["mask"])
        self.patch = cfg.patch_size
        self.tile = settings["tile"]
        self.sigma = settings["sigma"]
        self.time = settings["sigma"] * num_train_timesteps
        self._buffers: dict = {}

    @classmethod
    def from_export(cls, path: str | Path, device: str | torch.device = "cuda") -> "HipRestorer":
        e = read_export(path, "restoration")
        return cls(e.cfg, e.weights, e.prompt, e.settings, e.num_train_timesteps, e.prediction, device)

    @torch.no_grad()
    def restore_tile(self, x: torch.Tensor) -> torch.Tensor:
        """``x - sigma * v`` in FP32 (a new tensor; ``x`` is not modified)."""
        x = x.to(self.device, torch.float32).contiguous()
        key = tuple(x.shape)
        if key not in self._buffers:
            self._buffers = {key: (torch.empty_like(x), torch.empty_like(x))}
        v, out = self._buffers[key]
        t = torch.full((x.shape[0],), self.time, device=self.device, dtype=torch.float32)
        self.engine(x, t, self.text.expand(x.shape[0], -1, -1), out=v)
        K.flow_euler(x, v, self.sigma, None, None, out)
        return require_finite(out.clone())
