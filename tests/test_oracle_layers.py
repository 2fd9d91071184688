"""Pins the CPU oracle's layer functions.

Two kinds of check:
- golden vectors written by running the reference's unmodified ``iris3b.nn``
  package (``tests/golden/make_nn_golden.py``), compared to the oracle on the
  same weights and inputs;
- the reference's own known-answer tests (tests/test_layers.py,
  tests/test_single_stream_architecture.py), restated against the oracle.
"""

import math
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import load_file

from oracle import iris_oracle as O

GOLDEN = load_file(str(Path(__file__).parent / "golden" / "nn_golden.safetensors"))


def case(name: str) -> dict[str, torch.Tensor]:
    prefix = f"{name}/"
    return {k[len(prefix):]: v for k, v in GOLDEN.items() if k.startswith(prefix)}


def weights(name: str, prefix: str = "") -> dict[str, torch.Tensor]:
    return {f"{prefix}{k[2:]}": v for k, v in case(name).items() if k.startswith("w/")}


def exact(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert torch.equal(a, b), (a - b).abs().max()


# -- golden vectors ----------------------------------------------------------
def test_rope_tables_match_reference_bitwise():
    for name, kw in {
        "rope2d_iso": dict(head_dim=128, height=6, width=4, aspect="isotropic"),
        "rope2d_square": dict(head_dim=64, height=4, width=6, aspect="square"),
        "rope2d_frame": dict(head_dim=64, height=4, width=6, frame_pairs=2, frame_index=1),
    }.items():
        cis = O.rope_2d(**kw)
        exact(cis.real, case(name)["real"])
        exact(cis.imag, case(name)["imag"])
    cis = O.rope_1d(128, 9)
    exact(cis.real, case("rope1d")["real"])
    exact(cis.imag, case("rope1d")["imag"])


def test_apply_rope_matches_reference():
    c = case("apply_rope")
    q, k = O.apply_rope(c["q"], c["k"], O.rope_2d(128, 6, 4, aspect="isotropic"))
    torch.testing.assert_close(q, c["q_out"], rtol=0, atol=1e-6)
    torch.testing.assert_close(k, c["k_out"], rtol=0, atol=1e-6)


def test_rms_norm_and_adaln_tails_match_reference():
    w = weights("rmsnorm")["weight"]
    c = case("rmsnorm")
    exact(O.rms_norm(c["x"], w, 1e-6), c["y"])
    t = case("adaln_tails")
    exact(O.modulate(O.rms_norm(t["x"], w, 1e-6), t["shift"], t["scale"]), t["norm_modulate"])
    exact(t["x"] + t["gate"] * O.rms_norm(t["branch"], w, 1e-6), t["gated_norm_residual"])
    exact(t["x"] + O.modulate(t["branch"], t["shift"], t["scale"]), t["modulated_residual"])


def test_mlps_match_reference():
    torch.testing.assert_close(O.swiglu(weights("swiglu", "m."), "m", case("swiglu")["x"]), case("swiglu")["y"])
    torch.testing.assert_close(
        O.gelu_mlp(weights("gelu_mlp", "m."), "m", case("gelu_mlp")["x"]), case("gelu_mlp")["y"]
    )


def test_self_attention_matches_reference():
    c = case("self_attention")
    rope = O.rope_2d(128, 6, 4, aspect="isotropic")
    y = O.self_attention(weights("self_attention", "a."), "a", c["x"], 1, 1e-6, rope)
    torch.testing.assert_close(y, c["y"], rtol=1e-5, atol=1e-6)


def test_joint_attention_matches_reference():
    """Pins the ``[text | image]`` concatenation, per-stream norms and gates, GQA."""
    from iris_mi355x.config import ModelConfig

    c = case("joint_attention")
    cfg = ModelConfig(hidden_size=64, num_heads=4, num_kv_heads=2)
    p = weights("joint_attention", "blocks.0.attn.")
    hx, hy = c["x"], c["y"]
    qx, kx, vx = O._project(p, cfg, "blocks.0.attn.", "_x", hx)
    qy, ky, vy = O._project(p, cfg, "blocks.0.attn.", "_y", hy)
    qx, kx = O.norm(p, "blocks.0.attn.q_norm_x", qx, 1e-6), O.norm(p, "blocks.0.attn.k_norm_x", kx, 1e-6)
    qy, ky = O.norm(p, "blocks.0.attn.q_norm_y", qy, 1e-6), O.norm(p, "blocks.0.attn.k_norm_y", ky, 1e-6)
    qx, kx = O.apply_rope(qx, kx, O.rope_2d(16, 6, 4, aspect="isotropic"))
    qy, ky = O.apply_rope(qy, ky, O.rope_1d(16, 9))
    q, k, v = (torch.cat(pair, dim=1).transpose(1, 2) for pair in ((qy, qx), (ky, kx), (vy, vx)))
    out = O.attention(q, k, v).transpose(1, 2).reshape(2, 33, 64)
    ox = O.linear(p, "blocks.0.attn.proj_x", out[:, 9:] * c["gate_x"])
    oy = O.linear(p, "blocks.0.attn.proj_y", out[:, :9] * c["gate_y"])
    torch.testing.assert_close(ox, c["out_x"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(oy, c["out_y"], rtol=1e-5, atol=1e-6)


def test_embedders_match_reference():
    c = case("timestep")
    y = O.timestep_embed(weights("timestep", "t_embedder."), c["t"], 10.0)
    torch.testing.assert_close(y, c["y"], rtol=1e-5, atol=1e-6)
    c = case("pixel_embed")
    y = O.pixel_embed(weights("pixel_embed", "pixel_embedder."), c["x"], 4, True)
    torch.testing.assert_close(y, c["y"], rtol=1e-6, atol=1e-6)
    exact(O.sincos_2d(16, 8, 12), case("sincos")["y"])


def test_text_adapters_match_reference():
    from iris_mi355x.config import ModelConfig

    c = case("text_linear")
    cfg = ModelConfig(hidden_size=64, text_dim=32, text_len=16, text_adapter="linear", text_abs_pos_embed=False)
    torch.testing.assert_close(O.embed_text(weights("text_linear", "y_embedder."), cfg, c["y_in"]), c["y"])

    c = case("text_blocks2")
    y = O.transformer_text(weights("text_blocks2", "t."), "t", c["y_in"], c["mask"], 1, 1e-6)
    torch.testing.assert_close(y, c["y"], rtol=1e-5, atol=1e-5)

    c = case("text_lap")
    cfg = ModelConfig(hidden_size=128, num_heads=1, text_dim=32, text_len=16, text_lap_num_layers=3,
                      text_lap_num_heads=4, text_abs_pos_embed=False)
    y = O.embed_text(weights("text_lap", "y_embedder."), cfg, c["y_in"], c["mask"])
    torch.testing.assert_close(y, c["y"], rtol=1e-5, atol=1e-5)


def test_shared_modulation_matches_reference():
    from iris_mi355x.config import ModelConfig

    c = case("shared_core")
    p = {f"modulation_cores.adaln_img.{k}": v for k, v in weights("shared_core").items()}
    p["blocks.0.adaln_img.bias"] = weights("shared_bias")["bias"]
    for k, v in weights("shared_lowrank").items():
        p[f"blocks.0.adaln_img.{k}"] = v
    cfg = ModelConfig(hidden_size=64, dual_depth=1, depth=1, modulation="shared_bias")
    torch.testing.assert_close(O.modulation(p, cfg, "blocks.0", "img", c["cond"]), c["bias_out"])
    cfg = ModelConfig(hidden_size=64, dual_depth=1, depth=1, modulation="shared_lowrank", modulation_rank=8)
    torch.testing.assert_close(O.modulation(p, cfg, "blocks.0", "img", c["cond"]), c["lowrank_out"])


# -- the reference's known-answer tests, restated (tests/test_layers.py) ------
def test_rmsnorm_fp32_math():
    x = torch.randn(2, 3, 8) * 100
    expected = x / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    torch.testing.assert_close(O.rms_norm(x, torch.ones(8), 1e-6), expected, rtol=1e-6, atol=0)


def test_swiglu_two_thirds_width():
    from iris_mi355x.config import IRIS_3B, ModelConfig

    assert ModelConfig(hidden_size=1536).mlp_hidden == 4096  # test_layers.py:23-26
    assert IRIS_3B.mlp_hidden == 6826


def test_timestep_embedding_layout():
    feats = O.timestep_features(torch.tensor([3.0]), 8, 10.0)
    freqs = torch.exp(-math.log(10.0) * torch.arange(4).float() / 4)
    torch.testing.assert_close(feats[0, :4], torch.cos(3.0 * freqs))
    torch.testing.assert_close(feats[0, 4:], torch.sin(3.0 * freqs))


def test_rope2d_resolution_independent_span():
    a, b = O.rope_2d(64, 8, 8, scale=16.0), O.rope_2d(64, 32, 32, scale=16.0)
    assert a.shape == (64, 32) and b.shape == (1024, 32)
    torch.testing.assert_close(a[-1], b[-1], rtol=1e-5, atol=1e-6)


def test_rope2d_xy_interleave():
    cis = O.rope_2d(8, 2, 3, theta=10000.0, scale=16.0)
    torch.testing.assert_close(cis[1, 1], torch.complex(torch.tensor(1.0), torch.tensor(0.0)))
    assert cis[1, 0].angle().abs() > 0


def test_rope2d_default_matches_explicit_construction():
    head_dim, h, w, theta, scale = 64, 4, 6, 10000.0, 16.0
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 4)[: head_dim // 4].float() / head_dim)
    x_ang = torch.outer(torch.linspace(0, scale, w), freqs)
    y_ang = torch.outer(torch.linspace(0, scale, h), freqs)
    x_cis = torch.polar(torch.ones_like(x_ang), x_ang)[None, :, :].expand(h, w, -1)
    y_cis = torch.polar(torch.ones_like(y_ang), y_ang)[:, None, :].expand(h, w, -1)
    ref = torch.stack([x_cis, y_cis], dim=-1).reshape(h * w, head_dim // 2)
    assert torch.equal(O.rope_2d(head_dim, h, w, theta=theta, scale=scale), ref)


def test_rope2d_isotropic_aspect_preserves_ratio():
    h, w, scale, j = 4, 8, 16.0, 3
    freq = (1.0 / 10000.0 ** (torch.arange(0, 64, 4).float() / 64))[j]
    step = scale / (w - 1)
    iso = O.rope_2d(64, h, w, scale=scale, aspect="isotropic")
    torch.testing.assert_close(iso[1, 2 * j].angle(), step * freq)
    torch.testing.assert_close(iso[w, 2 * j + 1].angle(), step * freq)
    ratio = iso[-1, 2 * j].angle() / iso[-1, 2 * j + 1].angle()
    torch.testing.assert_close(ratio, torch.tensor((w - 1) / (h - 1)), rtol=1e-5, atol=1e-5)


def test_rope_square_and_isotropic_agree_on_square_grids():
    torch.testing.assert_close(O.rope_2d(128, 64, 64, aspect="square"), O.rope_2d(128, 64, 64, aspect="isotropic"))


def test_apply_rope_preserves_norm():
    q, k = torch.randn(2, 5, 4, 64), torch.randn(2, 5, 4, 64)
    q2, _ = O.apply_rope(q, k, O.rope_1d(64, 5))
    torch.testing.assert_close(q2.norm(dim=-1), q.norm(dim=-1), rtol=1e-4, atol=1e-4)


# -- attention (tests/test_single_stream_architecture.py:45-56) ----------------
def test_gqa_attention_matches_explicit_repeat_and_library_sdpa():
    torch.manual_seed(0)
    q, k, v = torch.randn(2, 4, 5, 8), torch.randn(2, 2, 5, 8), torch.randn(2, 2, 5, 8)
    expected = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1))
    torch.testing.assert_close(O.attention(q, k, v), expected)
    mask = torch.rand(2, 1, 5, 5) > 0.5
    mask |= torch.eye(5, dtype=torch.bool)
    expected = F.scaled_dot_product_attention(q, k.repeat_interleave(2, 1), v.repeat_interleave(2, 1), attn_mask=mask)
    torch.testing.assert_close(O.attention(q, k, v, mask), expected)


# -- unfold / fold glue (src/iris3b/models/dit.py:326, 370-374) ---------------
@pytest.mark.parametrize("hw", [(8, 12), (16, 16)])
def test_patchify_and_unpatchify_match_library_unfold_fold(hw):
    x = torch.randn(2, 3, *hw)
    exact(O.patchify(x, 4), F.unfold(x, kernel_size=4, stride=4).transpose(1, 2))
    out = torch.randn(2 * (hw[0] // 4) * (hw[1] // 4), 16, 3)
    folded = out.reshape(2, -1, 16, 3).permute(0, 3, 2, 1).reshape(2, 3 * 16, -1)
    exact(O.unpatchify(out, 2, *hw, 4), F.fold(folded, output_size=hw, kernel_size=4, stride=4))
