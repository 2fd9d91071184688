"""Model shape configuration for the Iris-3B denoiser.

Plain dataclasses restating the fields of the reference's ``ModelConfig`` and
``PixelStageConfig`` (src/iris3b/config.py:26-120) that the forward pass reads.
The defaults are the Iris-3B architecture (src/iris3b/models/presets.py:15).
Training-only fields (REPA, activation checkpointing, optimizer) are omitted;
``from_mapping`` accepts a reference ``config.yaml`` ``model:`` section and
ignores the keys this file does not model.
"""

from __future__ import annotations

from dataclasses import dataclass, field, fields, replace

HEAD_DIM = 128
PIXEL_WIDTH = 16
PIXEL_HIDDEN = 64


@dataclass(frozen=True)
class PixelStageConfig:
    """Pixel-level PiT stage (src/iris3b/config.py:26-38)."""

    enabled: bool = True
    depth: int = 4
    hidden_size: int = 16
    attn_hidden_size: int = 1280
    num_heads: int = 10
    mlp_ratio: float = 4.0
    modulation: str = "post"  # "pre" (6 tuples, gated) | "post" (4 tuples)
    abs_pos_embed: bool = True


@dataclass(frozen=True)
class ModelConfig:
    """Patch-stage topology (src/iris3b/config.py:42-120)."""

    block: str = "single_stream"
    dual_depth: int = 8
    final_block_text: str = "keep"
    hidden_size: int = 2560
    depth: int = 24
    num_heads: int = 20
    num_kv_heads: int | None = 5
    gated_attention: bool = True
    sandwich_norm: bool = True
    patch_size: int = 16
    in_channels: int = 3
    mlp_ratio: float = 4.0
    qkv_bias: bool = False
    qk_norm: bool = True
    norm_eps: float = 1e-6
    modulation: str = "shared_bias"  # per_block | shared_lowrank | shared_bias
    modulation_rank: int = 64
    timestep_max_period: float = 10.0
    adaln_zero_init: bool = True
    rope_theta: float = 10000.0
    rope_scale: float = 16.0
    rope_aspect: str = "isotropic"
    rope_frame_pairs: int = 0
    rope_frame_theta: float = 10.0
    text_rope: bool = True
    text_rope_theta: float = 10000.0
    text_abs_pos_embed: bool = True
    text_dim: int = 2560
    text_len: int = 300
    text_adapter: str = "lap_blocks2"  # linear | blocks2 | lap_blocks2
    text_lap_num_layers: int = 12
    text_lap_num_heads: int = 32
    text_lap_mlp_ratio: float = 1.3
    pixel: PixelStageConfig = field(default_factory=PixelStageConfig)

    # -- derived shapes ------------------------------------------------------
    @property
    def kv_heads(self) -> int:
        return self.num_heads if self.num_kv_heads is None else self.num_kv_heads

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def mlp_hidden(self) -> int:
        """SwiGLU width, the 2/3 rule of src/iris3b/nn/mlp.py:24-40."""
        return int(2 * int(self.hidden_size * self.mlp_ratio) / 3)

    @property
    def pixels_per_patch(self) -> int:
        return self.patch_size * self.patch_size

    def block_kind(self, index: int) -> str:
        """``"mmdit"`` for the leading ``dual_depth`` blocks, then ``block``."""
        return "mmdit" if index < self.dual_depth else self.block

    def text_out(self, index: int) -> bool:
        """Whether block ``index`` builds its text output path (src/iris3b/models/dit.py:141-153)."""
        return self.final_block_text == "keep" or index < self.depth - 1

    def validate(self) -> None:
        if not 0 <= self.dual_depth <= self.depth:
            raise ValueError(f"dual_depth must be in [0, {self.depth}], got {self.dual_depth}")
        if self.final_block_text not in ("keep", "drop"):
            raise ValueError(f"unknown final_block_text {self.final_block_text!r}")
        if self.hidden_size % self.num_heads:
            raise ValueError(f"hidden_size {self.hidden_size} not divisible by num_heads {self.num_heads}")
        if self.kv_heads <= 0 or self.num_heads % self.kv_heads:
            raise ValueError(f"query heads {self.num_heads} must be divisible by KV heads {self.kv_heads}")
        if self.modulation not in ("per_block", "shared_lowrank", "shared_bias"):
            raise ValueError(f"unknown modulation {self.modulation!r}")
        if self.text_adapter not in ("linear", "blocks2", "lap_blocks2"):
            raise ValueError(f"unknown text_adapter {self.text_adapter!r}")
        if self.pixel.modulation not in ("pre", "post"):
            raise ValueError(f"unknown PiT modulation {self.pixel.modulation!r}")

    @classmethod
    def from_mapping(cls, values: dict) -> "ModelConfig":
        """Build from a reference ``config.yaml`` ``model`` mapping (unknown keys ignored)."""
        names = {f.name for f in fields(cls)}
        kwargs = {k: v for k, v in values.items() if k in names and k != "pixel"}
        pixel = values.get("pixel") or {}
        pnames = {f.name for f in fields(PixelStageConfig)}
        kwargs["pixel"] = PixelStageConfig(**{k: v for k, v in pixel.items() if k in pnames})
        return cls(**kwargs)


IRIS_3B = ModelConfig()

# The reference's CPU-sized unit-test model (tests/tiny_config.py:7-26): all MM-DiT,
# MHA with fused QKV, per-block adaLN, linear text adapter and a "pre" PiT stage.
TINY = ModelConfig(
    block="mmdit",
    dual_depth=0,
    hidden_size=64,
    depth=2,
    num_heads=4,
    num_kv_heads=None,
    gated_attention=False,
    sandwich_norm=False,
    patch_size=4,
    modulation="per_block",
    adaln_zero_init=False,
    rope_aspect="square",
    text_dim=32,
    text_len=16,
    text_adapter="linear",
    text_lap_num_layers=0,
    pixel=PixelStageConfig(depth=1, hidden_size=8, attn_hidden_size=64, num_heads=4, modulation="pre"),
)

# The released topology at toy width, 128-wide heads (tests/test_metal_engine.py:28-48).
RELEASED_TOPOLOGY = ModelConfig(
    block="single_stream",
    dual_depth=1,
    hidden_size=256,
    depth=3,
    num_heads=2,
    num_kv_heads=1,
    gated_attention=True,
    sandwich_norm=True,
    patch_size=4,
    modulation="shared_bias",
    adaln_zero_init=False,
    rope_aspect="isotropic",
    text_dim=64,
    text_len=16,
    text_adapter="lap_blocks2",
    text_lap_num_layers=3,
    text_lap_num_heads=4,
    pixel=PixelStageConfig(depth=2, hidden_size=16, attn_hidden_size=256, num_heads=2, modulation="post"),
)

PRESETS = {"iris-3b": IRIS_3B}


def get_preset(name: str, **overrides) -> ModelConfig:
    if name not in PRESETS:
        raise KeyError(f"unknown preset '{name}' (known: {sorted(PRESETS)})")
    return replace(PRESETS[name], **overrides)
