"""Parameter schema and synthetic weights of the Iris-3B denoiser.

``parameter_schema`` enumerates the reference ``IrisDiT`` ``state_dict`` keys and
shapes for a ``ModelConfig`` (module tree of src/iris3b/models/dit.py:65-193,
blocks/mmdit.py:37-82, blocks/single_stream.py:20-56, blocks/pit.py:31-64,
nn/embeddings.py:21-328, nn/modulation.py:258-334), so a real checkpoint saved by
the reference loads by name and the synthetic weights use the same names.

``synthetic_state_dict`` is the seeded weight recipe every parity test and the
benchmark use: keys in sorted order, one ``torch.Generator`` seeded once,
Linear weights/biases, adaLN cores and per-block adaLN biases ~ N(0, 0.02),
RMSNorm gains 1 + N(0, 0.02), the text position table ~ N(0, 1). The reference's
own init zeroes the head and every adaLN projection, which makes the predicted
flow identically zero (src/iris3b/models/dit.py:196-215), so it cannot serve
as a parity input.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from pathlib import Path

import torch

from .config import ModelConfig


@dataclass(frozen=True)
class ParamSpec:
    shape: tuple[int, ...]
    kind: str  # "linear" | "norm" | "adaln_bias" | "lowrank" | "pos"


def _linear(schema: dict, name: str, out_f: int, in_f: int, bias: bool = True) -> None:
    schema[f"{name}.weight"] = ParamSpec((out_f, in_f), "linear")
    if bias:
        schema[f"{name}.bias"] = ParamSpec((out_f,), "linear")


def _norm(schema: dict, name: str, dim: int) -> None:
    schema[f"{name}.weight"] = ParamSpec((dim,), "norm")


def _self_attention(schema: dict, name: str, dim: int, heads: int, qkv_bias: bool, qk_norm: bool) -> None:
    _linear(schema, f"{name}.qkv", 3 * dim, dim, qkv_bias)
    if qk_norm:
        _norm(schema, f"{name}.q_norm", dim // heads)
        _norm(schema, f"{name}.k_norm", dim // heads)
    _linear(schema, f"{name}.proj", dim, dim)


def _swiglu(schema: dict, name: str, dim: int, ratio: float) -> None:
    hidden = int(2 * int(dim * ratio) / 3)
    _linear(schema, f"{name}.w1", hidden, dim, False)
    _linear(schema, f"{name}.w3", hidden, dim, False)
    _linear(schema, f"{name}.w2", dim, hidden, False)


def _transformer_text(schema: dict, name: str, cfg: ModelConfig, text_dim: int) -> None:
    d = cfg.hidden_size
    _linear(schema, f"{name}.proj", d, text_dim)
    for i in range(2):
        b = f"{name}.blocks.{i}"
        _norm(schema, f"{b}.norm1", d)
        _self_attention(schema, f"{b}.attn", d, cfg.num_heads, cfg.qkv_bias, cfg.qk_norm)
        _norm(schema, f"{b}.norm2", d)
        _swiglu(schema, f"{b}.mlp", d, cfg.mlp_ratio)
    _norm(schema, f"{name}.norm", d)


def _adaln(schema: dict, name: str, cfg: ModelConfig) -> None:
    d = cfg.hidden_size
    if cfg.modulation == "per_block":
        _linear(schema, name, 6 * d, d)
    elif cfg.modulation == "shared_bias":
        schema[f"{name}.bias"] = ParamSpec((6 * d,), "adaln_bias")
    else:
        schema[f"{name}.down.weight"] = ParamSpec((cfg.modulation_rank, d), "lowrank")
        schema[f"{name}.adaln_up.weight"] = ParamSpec((6 * d, cfg.modulation_rank), "lowrank")


def core_names(cfg: ModelConfig) -> list[str]:
    """Shared adaLN cores (``modulation_cores.*``) a config builds (src/iris3b/models/dit.py:121-128)."""
    if cfg.modulation == "per_block":
        return []
    names = []
    alias = {"shared": "img"} if cfg.dual_depth else {}
    for i in range(cfg.depth):
        streams = ("img", "txt") if cfg.block_kind(i) == "mmdit" else ("shared",)
        for s in streams:
            key = f"adaln_{alias.get(s, s)}"
            if key not in names:
                names.append(key)
    return names


def parameter_schema(cfg: ModelConfig) -> dict[str, ParamSpec]:
    cfg.validate()
    d, p, hd = cfg.hidden_size, cfg.patch_size, cfg.head_dim
    kv_dim = cfg.kv_heads * hd
    gqa = cfg.kv_heads != cfg.num_heads
    s: dict[str, ParamSpec] = {}
    _linear(s, "s_embedder.proj", d, p * p * cfg.in_channels)
    _linear(s, "t_embedder.mlp.0", d, 256)
    _linear(s, "t_embedder.mlp.2", d, d)
    if cfg.text_adapter == "linear":
        _linear(s, "y_embedder.proj", d, cfg.text_dim)
        _norm(s, "y_embedder.norm", d)
    elif cfg.text_adapter == "blocks2":
        _transformer_text(s, "y_embedder", cfg, cfg.text_dim)
    else:
        td = cfg.text_dim
        hidden = int(td * cfg.text_lap_mlp_ratio)
        for i in range(2):
            b = f"y_embedder.layer_blocks.{i}"
            _norm(s, f"{b}.norm1", td)
            _self_attention(s, f"{b}.attn", td, cfg.text_lap_num_heads, False, False)
            _norm(s, f"{b}.norm2", td)
            _linear(s, f"{b}.mlp.0", hidden, td)
            _linear(s, f"{b}.mlp.2", td, hidden)
        _linear(s, "y_embedder.layer_pool", 1, cfg.text_lap_num_layers)
        _transformer_text(s, "y_embedder.refiner", cfg, td)
    if cfg.text_abs_pos_embed:
        s["y_pos_embedding"] = ParamSpec((1, cfg.text_len, d), "pos")
    for name in core_names(cfg):
        _linear(s, f"modulation_cores.{name}", 6 * d, d)

    for i in range(cfg.depth):
        b = f"blocks.{i}"
        text_out = cfg.text_out(i)
        if cfg.block_kind(i) == "mmdit":
            _norm(s, f"{b}.norm_x1", d)
            _norm(s, f"{b}.norm_x2", d)
            _norm(s, f"{b}.norm_y1", d)
            if text_out:
                _norm(s, f"{b}.norm_y2", d)
            for st in ("x", "y"):
                if gqa:
                    _linear(s, f"{b}.attn.q_proj_{st}", d, d, cfg.qkv_bias)
                    _linear(s, f"{b}.attn.k_proj_{st}", kv_dim, d, cfg.qkv_bias)
                    _linear(s, f"{b}.attn.v_proj_{st}", kv_dim, d, cfg.qkv_bias)
                else:
                    _linear(s, f"{b}.attn.qkv_{st}", 3 * d, d, cfg.qkv_bias)
            if cfg.qk_norm:
                for nm in ("q_norm_x", "k_norm_x", "q_norm_y", "k_norm_y"):
                    _norm(s, f"{b}.attn.{nm}", hd)
            _linear(s, f"{b}.attn.proj_x", d, d)
            if text_out:
                _linear(s, f"{b}.attn.proj_y", d, d)
            if cfg.gated_attention:
                _linear(s, f"{b}.attn_gate_x", d, d, False)
                if text_out:
                    _linear(s, f"{b}.attn_gate_y", d, d, False)
            if cfg.sandwich_norm:
                _norm(s, f"{b}.attn_post_norm_x", d)
                if text_out:
                    _norm(s, f"{b}.attn_post_norm_y", d)
            _swiglu(s, f"{b}.mlp_x", d, cfg.mlp_ratio)
            if text_out:
                _swiglu(s, f"{b}.mlp_y", d, cfg.mlp_ratio)
            if cfg.sandwich_norm:
                _norm(s, f"{b}.mlp_post_norm_x", d)
                if text_out:
                    _norm(s, f"{b}.mlp_post_norm_y", d)
            _adaln(s, f"{b}.adaln_img", cfg)
            _adaln(s, f"{b}.adaln_txt", cfg)
        else:
            _norm(s, f"{b}.norm1", d)
            _norm(s, f"{b}.norm2", d)
            if gqa:
                _linear(s, f"{b}.q_proj", d, d, cfg.qkv_bias)
                _linear(s, f"{b}.k_proj", kv_dim, d, cfg.qkv_bias)
                _linear(s, f"{b}.v_proj", kv_dim, d, cfg.qkv_bias)
            else:
                _linear(s, f"{b}.qkv", 3 * d, d, cfg.qkv_bias)
            if cfg.qk_norm:
                _norm(s, f"{b}.q_norm", hd)
                _norm(s, f"{b}.k_norm", hd)
            if cfg.gated_attention:
                _linear(s, f"{b}.attn_gate", d, d, False)
            _linear(s, f"{b}.attn_proj", d, d)
            if cfg.sandwich_norm:
                _norm(s, f"{b}.attn_post_norm", d)
            _swiglu(s, f"{b}.mlp", d, cfg.mlp_ratio)
            if cfg.sandwich_norm:
                _norm(s, f"{b}.mlp_post_norm", d)
            _adaln(s, f"{b}.adaln", cfg)

    px = cfg.pixel
    if not px.enabled:
        _norm(s, "final_layer.norm", d)
        _linear(s, "final_layer.linear", p * p * cfg.in_channels, d)
        return s
    hp, pp = px.hidden_size, p * p
    _linear(s, "pixel_embedder.proj", hp, cfg.in_channels)
    n_mod = 6 if px.modulation == "pre" else 4
    for i in range(px.depth):
        b = f"pixel_blocks.{i}"
        _norm(s, f"{b}.norm1", hp)
        _norm(s, f"{b}.norm2", hp)
        _linear(s, f"{b}.adaln", n_mod * hp * pp, d)
        _linear(s, f"{b}.compress", px.attn_hidden_size, pp * hp)
        _linear(s, f"{b}.expand", pp * hp, px.attn_hidden_size)
        _self_attention(s, f"{b}.attn", px.attn_hidden_size, px.num_heads, False, cfg.qk_norm)
        _linear(s, f"{b}.mlp.fc1", int(hp * px.mlp_ratio), hp)
        _linear(s, f"{b}.mlp.fc2", hp, int(hp * px.mlp_ratio))
    _norm(s, "final_layer.norm", hp)
    _linear(s, "final_layer.linear", cfg.in_channels, hp)
    return s


def parameter_count(cfg: ModelConfig) -> int:
    return sum(math.prod(spec.shape) for spec in parameter_schema(cfg).values())


def synthetic_state_dict(
    cfg: ModelConfig, seed: int = 0, std: float = 0.02, device: str | torch.device = "cpu",
    schema: dict[str, ParamSpec] | None = None,
) -> dict[str, torch.Tensor]:
    """FP32 weights by the seeded recipe above, in sorted key order.

    ``device`` selects where the generator draws; ``"cpu"`` is the canonical
    recipe, and a device generator gives a different (but again deterministic)
    draw that is much faster for the 3B-parameter model. ``schema`` replaces the
    denoiser's parameter schema (the downstream task models).
    """
    gen = torch.Generator(device=device).manual_seed(seed)
    out: dict[str, torch.Tensor] = {}
    for name, spec in sorted((parameter_schema(cfg) if schema is None else schema).items()):
        t = torch.randn(spec.shape, generator=gen, device=device, dtype=torch.float32)
        if spec.kind == "pos":
            pass
        elif spec.kind == "norm":
            t.mul_(std).add_(1.0)
        else:
            t.mul_(std)
        out[name] = t
    return out


def save_state_dict(state: dict[str, torch.Tensor], path: str | Path) -> None:
    from safetensors.torch import save_file

    save_file({k: v.detach().contiguous().cpu() for k, v in state.items()}, str(path))


def load_state_dict(path: str | Path, device: str | torch.device = "cpu") -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    return load_file(str(path), device=str(device))


def check_state_dict(cfg: ModelConfig, state: dict[str, torch.Tensor]) -> None:
    """Raise ``ValueError`` unless ``state`` has exactly the schema's keys and shapes."""
    schema = parameter_schema(cfg)
    missing = sorted(set(schema) - set(state))
    extra = sorted(set(state) - set(schema))
    if missing or extra:
        raise ValueError(f"state_dict mismatch: missing {missing[:5]}, unexpected {extra[:5]}")
    for name, spec in schema.items():
        if tuple(state[name].shape) != spec.shape:
            raise ValueError(f"{name} has shape {tuple(state[name].shape)}, expected {spec.shape}")
