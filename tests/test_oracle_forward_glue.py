"""Pins the glue of the oracle's ``forward`` (src/iris3b/models/dit.py:263-281, 321-375) with
known answers.

The reference's ``IrisDiT`` cannot be imported here (its config module needs omegaconf), and its
blocks and layers are pinned by golden vectors elsewhere. What only ``IrisDiT.forward`` does is
glue: ``cond = silu(t_emb)``, text truncation and the ``y_pos_embedding`` add of ``embed_text``,
the ``[text | image]`` hand-over between blocks, the ``silu(t_emb + s)`` re-fusion feeding the
pixel stage, ``FinalLayer`` (RMSNorm, then Linear) and the fold. Here the weights are chosen so
that the whole forward has a closed form computed from library routines and pinned layers alone:

- zero query and key projections make every attention uniform, so each attention row is the
  mean of the value rows of the whole joint ``[text | image]`` sequence (text reaches the image
  rows through it); zero MLP output weights make every MLP branch exactly zero;
- each PiT block's adaLN bias sets its scales to -1, so ``modulate(branch, shift, -1)`` is
  ``shift`` ("post": the attention branch is replaced by ``shift1``, a Linear of the pixel
  stage's condition, the MLP branch by 0) or its output weights are zero so the branch is its
  bias ("pre": the gated residuals add ``gate1 * expand.bias`` and ``gate2 * fc2.bias``);
- the expected flow is then assembled from ``F.unfold``, ``F.linear``, ``F.fold``, RMSNorm
  restated from src/iris3b/nn/norms.py:15-21, and the golden-pinned timestep embedder, pixel
  embedder and text adapters.

Each plausible mistake in the glue, written into a copy of the oracle's source, must fail the
same comparison (``test_a_mutated_forward_fails``): the check is shown to discriminate.
The tiny config case uses config 1's inputs (64x64, 32 text tokens of which 16 are kept, t = 500).
"""

from __future__ import annotations

import inspect
import math
import textwrap
from dataclasses import replace

import pytest
import torch
import torch.nn.functional as F

from iris_mi355x.config import RELEASED_TOPOLOGY, TINY
from iris_mi355x.weights import synthetic_state_dict
from oracle import iris_oracle as O

RTOL, ATOL = 2e-5, 2e-6


def rms(x, w, eps=1e-6):
    """RMSNorm of src/iris3b/nn/norms.py:15-21 (FP32 statistics, gain after)."""
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def fold_pixels(out, batch, height, width, patch):
    """dit.py:370-374: ``[B*L, p*p, C] -> [B, C, H, W]`` through ``F.fold``."""
    n = (height // patch) * (width // patch)
    c = out.shape[-1]
    folded = out.reshape(batch, n, patch * patch, c).permute(0, 3, 2, 1).reshape(batch, c * patch * patch, n)
    return F.fold(folded, output_size=(height, width), kernel_size=patch, stride=patch)


def _draw(p, gen, name, fan_in=None, scale=1.0):
    t = p[name]
    std = scale / math.sqrt(fan_in if fan_in is not None else t.shape[-1])
    p[name] = torch.randn(t.shape, generator=gen) * std


def _uniform_attention_mean(h, w_v, heads, kv_heads, head_dim):
    """Rows of uniform attention over ``h`` ([B, N, D] joint rows): per query head, the mean of its
    K/V head's value rows (GQA: query head j reads K/V head j // (heads / kv_heads))."""
    v = F.linear(h, w_v).mean(1)  # [B, kv_heads * d]
    return v.reshape(-1, kv_heads, head_dim).repeat_interleave(heads // kv_heads, dim=1).reshape(v.shape[0], 1, -1)


# ------------------------------------------------------------------------------------------
# the released topology: lap_blocks2 adapter, shared_bias modulation, GQA with gate and
# sandwich norms, one dual block then single-stream blocks, "post" PiT
# ------------------------------------------------------------------------------------------
def released_case(final_block_text="keep", seed=5, n_in=None):
    cfg = replace(RELEASED_TOPOLOGY, final_block_text=final_block_text)
    p = synthetic_state_dict(cfg)
    g = torch.Generator().manual_seed(seed)
    d, hd = cfg.hidden_size, cfg.head_dim
    # inputs of O(1) everywhere, so that every glue term moves the output by O(1)
    for name in ("s_embedder.proj.weight", "t_embedder.mlp.0.weight", "t_embedder.mlp.2.weight",
                 "modulation_cores.adaln_img.weight", "modulation_cores.adaln_txt.weight"):
        _draw(p, g, name)
    for st in ("x", "y"):
        p[f"blocks.0.attn.q_proj_{st}.weight"].zero_()
        p[f"blocks.0.attn.k_proj_{st}.weight"].zero_()
        _draw(p, g, f"blocks.0.attn.v_proj_{st}.weight")
        p[f"blocks.0.attn_gate_{st}.weight"].zero_()
        p[f"blocks.0.mlp_{st}.w2.weight"].zero_()
    for i in range(1, cfg.depth):
        b = f"blocks.{i}"
        p[f"{b}.q_proj.weight"].zero_()
        p[f"{b}.k_proj.weight"].zero_()
        _draw(p, g, f"{b}.v_proj.weight")
        p[f"{b}.attn_gate.weight"].zero_()
        p[f"{b}.mlp.w2.weight"].zero_()
    px, pp = cfg.pixel, cfg.pixels_per_patch
    hp = px.hidden_size
    for i in range(px.depth):
        b = f"pixel_blocks.{i}"
        # adaLN rows of pixel q: [scale1 | shift1 | scale2 | shift2] (hp each; pit.py:89)
        w = torch.zeros(pp, 4, hp, d)
        w[:, 1] = torch.randn(pp, hp, d, generator=g) / math.sqrt(d)
        bias = torch.zeros(pp, 4, hp)
        bias[:, 0] = bias[:, 2] = -1.0
        p[f"{b}.adaln.weight"] = w.reshape(pp * 4 * hp, d)
        p[f"{b}.adaln.bias"] = bias.reshape(-1)
    p["final_layer.norm.weight"] = 0.5 + torch.rand(hp, generator=g)
    _draw(p, g, "final_layer.linear.weight")
    gen = torch.Generator().manual_seed(seed + 1)
    batch, height, width = 2, 16, 24  # a 4 x 6 patch grid: the fold's orientation shows
    x = torch.randn(batch, 3, height, width, generator=gen)
    t = torch.tensor([125.0, 850.0])
    if n_in is None:
        n_in = cfg.text_len + 4  # longer than text_len: embed_text keeps the first text_len
    states = torch.randn(batch, n_in, cfg.text_lap_num_layers, cfg.text_dim, generator=gen)
    mask = torch.zeros(batch, n_in, dtype=torch.long)
    mask[0, :5] = 1
    mask[1, :9] = 1
    mask[:, cfg.text_len:] = 1  # past text_len: must be cut with the states
    return cfg, p, (x, t, states, mask)


def released_expected(cfg, p, x, t, states, mask):
    eps, d, hd = cfg.norm_eps, cfg.hidden_size, cfg.head_dim
    heads, kv = cfg.num_heads, cfg.kv_heads
    batch, _, height, width = x.shape
    patch = cfg.patch_size
    n_txt = cfg.text_len
    s = F.linear(F.unfold(x, patch, stride=patch).transpose(1, 2), p["s_embedder.proj.weight"],
                 p["s_embedder.proj.bias"])
    t_emb = O.timestep_embed(p, t, cfg.timestep_max_period)  # [B, 1, D]
    cond = F.silu(t_emb)
    text = O.layerwise_text(p, cfg, states[:, :n_txt], mask[:, :n_txt])
    text = text + p["y_pos_embedding"][:, :text.shape[1]]  # the table's first rows

    def mods(core, bias):
        return (F.linear(cond, p[f"modulation_cores.{core}.weight"], p[f"modulation_cores.{core}.bias"])
                + p[bias]).chunk(6, dim=-1)

    # dual block 0: uniform joint attention over [text | image], zero MLPs
    xs1, xc1, xg1, *_ = mods("adaln_img", "blocks.0.adaln_img.bias")
    ys1, yc1, yg1, *_ = mods("adaln_txt", "blocks.0.adaln_txt.bias")
    hx = rms(s, p["blocks.0.norm_x1.weight"], eps) * (1 + xc1) + xs1
    hy = rms(text, p["blocks.0.norm_y1.weight"], eps) * (1 + yc1) + ys1
    vx = F.linear(hx, p["blocks.0.attn.v_proj_x.weight"])
    vy = F.linear(hy, p["blocks.0.attn.v_proj_y.weight"])
    mean = torch.cat([vy, vx], 1).mean(1).reshape(batch, kv, hd).repeat_interleave(heads // kv, 1).reshape(batch, 1, d)
    for st, gate in (("x", xg1), ("y", yg1)):
        a = rms(F.linear(0.5 * mean, p[f"blocks.0.attn.proj_{st}.weight"], p[f"blocks.0.attn.proj_{st}.bias"]),
                p[f"blocks.0.attn_post_norm_{st}.weight"], eps)
        if st == "x":
            s = s + gate * a
        else:
            text = text + gate * a
    # single-stream blocks over [text | image]
    for i in range(1, cfg.depth):
        b = f"blocks.{i}"
        s1, c1, g1, *_ = mods("adaln_img", f"{b}.adaln.bias")
        tokens = torch.cat([text, s], 1)
        h = rms(tokens, p[f"{b}.norm1.weight"], eps) * (1 + c1) + s1
        mean = _uniform_attention_mean(h, p[f"{b}.v_proj.weight"], heads, kv, hd)
        a = rms(F.linear(0.5 * mean, p[f"{b}.attn_proj.weight"], p[f"{b}.attn_proj.bias"]),
                p[f"{b}.attn_post_norm.weight"], eps)
        text, s = text + g1 * a, s + g1 * a
    # timestep re-fused into every patch token, then the pixel stage ("post": + shift1 per block)
    cond_pix = F.silu(t_emb + s).reshape(-1, d)
    pixels = O.pixel_embed(p, x, patch, cfg.pixel.abs_pos_embed)
    pp, hp = cfg.pixels_per_patch, cfg.pixel.hidden_size
    for i in range(cfg.pixel.depth):
        w = p[f"pixel_blocks.{i}.adaln.weight"].reshape(pp, 4, hp, d)[:, 1].reshape(pp * hp, d)
        pixels = pixels + F.linear(cond_pix, w).reshape(-1, pp, hp)
    out = F.linear(rms(pixels, p["final_layer.norm.weight"], eps), p["final_layer.linear.weight"],
                   p["final_layer.linear.bias"])
    return fold_pixels(out, batch, height, width, patch)


# ------------------------------------------------------------------------------------------
# the tiny config (tests/tiny_config.py:7-26): linear adapter, per-block adaLN, MHA with fused
# QKV, no gate or sandwich norms, all MM-DiT, "pre" PiT; config 1's inputs
# ------------------------------------------------------------------------------------------
def tiny_case(seed=7):
    cfg = TINY
    p = synthetic_state_dict(cfg)
    g = torch.Generator().manual_seed(seed)
    d = cfg.hidden_size
    for name in ("s_embedder.proj.weight", "t_embedder.mlp.0.weight", "t_embedder.mlp.2.weight",
                 "y_embedder.proj.weight"):
        _draw(p, g, name)
    for i in range(cfg.depth):
        b = f"blocks.{i}"
        for st in ("x", "y"):
            w = p[f"{b}.attn.qkv_{st}.weight"]
            w[: 2 * d] = 0.0  # q and k rows
            w[2 * d:] = torch.randn(d, d, generator=g) / math.sqrt(d)
            p[f"{b}.mlp_{st}.w2.weight"].zero_()
            _draw(p, g, f"{b}.attn.proj_{st}.weight")
            _draw(p, g, f"{b}.adaln_{st.replace('x', 'img').replace('y', 'txt')}.weight")
    px, pp = cfg.pixel, cfg.pixels_per_patch
    hp = px.hidden_size
    b = "pixel_blocks.0"
    _draw(p, g, f"{b}.adaln.weight")
    p[f"{b}.expand.weight"].zero_()
    p[f"{b}.expand.bias"] = torch.randn(pp * hp, generator=g)
    p[f"{b}.mlp.fc2.weight"].zero_()
    p[f"{b}.mlp.fc2.bias"] = torch.randn(hp, generator=g)
    p["final_layer.norm.weight"] = 0.5 + torch.rand(hp, generator=g)
    _draw(p, g, "final_layer.linear.weight")
    # config 1: x ~ N(0,1) [1, 3, 64, 64], then y ~ N(0,1) [1, 32, 32] from the same generator, t = 500
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(1, 3, 64, 64, generator=gen)
    y = torch.randn(1, 32, cfg.text_dim, generator=gen)
    return cfg, p, (x, torch.tensor([500.0]), y, None)


def tiny_expected(cfg, p, x, t, y, _mask):
    eps, d = cfg.norm_eps, cfg.hidden_size
    batch, _, height, width = x.shape
    patch, n_txt = cfg.patch_size, cfg.text_len
    s = F.linear(F.unfold(x, patch, stride=patch).transpose(1, 2), p["s_embedder.proj.weight"],
                 p["s_embedder.proj.bias"])
    t_emb = O.timestep_embed(p, t, cfg.timestep_max_period)
    cond = F.silu(t_emb)
    text = rms(F.linear(y[:, :n_txt], p["y_embedder.proj.weight"], p["y_embedder.proj.bias"]),
               p["y_embedder.norm.weight"], eps) + p["y_pos_embedding"][:, :n_txt]
    for i in range(cfg.depth):
        b = f"blocks.{i}"
        xs1, xc1, xg1, *_ = F.linear(cond, p[f"{b}.adaln_img.weight"], p[f"{b}.adaln_img.bias"]).chunk(6, -1)
        ys1, yc1, yg1, *_ = F.linear(cond, p[f"{b}.adaln_txt.weight"], p[f"{b}.adaln_txt.bias"]).chunk(6, -1)
        hx = rms(s, p[f"{b}.norm_x1.weight"], eps) * (1 + xc1) + xs1
        hy = rms(text, p[f"{b}.norm_y1.weight"], eps) * (1 + yc1) + ys1
        vx = F.linear(hx, p[f"{b}.attn.qkv_x.weight"][2 * d:])
        vy = F.linear(hy, p[f"{b}.attn.qkv_y.weight"][2 * d:])
        mean = torch.cat([vy, vx], 1).mean(1, keepdim=True)  # MHA: every head reads its own values
        s = s + xg1 * F.linear(mean, p[f"{b}.attn.proj_x.weight"], p[f"{b}.attn.proj_x.bias"])
        text = text + yg1 * F.linear(mean, p[f"{b}.attn.proj_y.weight"], p[f"{b}.attn.proj_y.bias"])
    cond_pix = F.silu(t_emb + s).reshape(-1, d)
    pixels = O.pixel_embed(p, x, patch, cfg.pixel.abs_pos_embed)
    pp, hp = cfg.pixels_per_patch, cfg.pixel.hidden_size
    b = "pixel_blocks.0"
    # adaLN rows of pixel q: [shift1 | scale1 | gate1 | shift2 | scale2 | gate2] (pit.py:85-88)
    mods = F.linear(cond_pix, p[f"{b}.adaln.weight"], p[f"{b}.adaln.bias"]).reshape(-1, pp, 6, hp)
    pixels = pixels + mods[:, :, 2] * p[f"{b}.expand.bias"].reshape(pp, hp)
    pixels = pixels + mods[:, :, 5] * p[f"{b}.mlp.fc2.bias"]
    out = F.linear(rms(pixels, p["final_layer.norm.weight"], eps), p["final_layer.linear.weight"],
                   p["final_layer.linear.bias"])
    return fold_pixels(out, batch, height, width, patch)


CASES = {
    "released_keep": (lambda: released_case("keep"), released_expected),
    "released_drop": (lambda: released_case("drop"), released_expected),
    "released_short_text": (lambda: released_case("keep", n_in=11), released_expected),
    "tiny_config1": (tiny_case, tiny_expected),
}


def _compare(forward, case):
    build, expected_fn = CASES[case]
    cfg, p, (x, t, y, mask) = build()
    want = expected_fn(cfg, p, x, t, y, mask)
    got = forward(p, cfg, x, t, y, mask)
    return got, want


@pytest.mark.parametrize("case", sorted(CASES))
def test_forward_glue_matches_closed_form(case):
    got, want = _compare(O.forward, case)
    assert got.shape == want.shape
    assert want.abs().max() > 0.1  # the answer is not trivially small
    torch.testing.assert_close(got, want, rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------------------------------
# the comparison discriminates: each plausible mistake in the glue fails it
# ------------------------------------------------------------------------------------------
def _mutant(edits):
    """A copy of the oracle's module namespace whose functions ``edits`` names are rebuilt from
    their source with one replacement each; returns that namespace's ``forward``."""
    ns = dict(vars(O))
    for fn, old, new in edits:
        src = textwrap.dedent(inspect.getsource(fn))
        assert src.count(old) == 1, f"{fn.__name__}: {old!r} not found once"
        exec(compile(src.replace(old, new), f"<mutant of {fn.__name__}>", "exec"), ns)
    if not any(fn is O.forward for fn, _, _ in edits):  # forward resolves the mutated helpers in ns
        exec(compile(textwrap.dedent(inspect.getsource(O.forward)), "<forward>", "exec"), ns)
    return ns["forward"]


MUTATIONS = {
    "refusion_silu_outside": [(O.forward, "s = F.silu(t_emb + s)", "s = F.silu(s) + t_emb")],
    "no_refusion": [(O.forward, "s = F.silu(t_emb + s)", "s = s")],
    "refusion_drops_t_emb": [(O.forward, "s = F.silu(t_emb + s)", "s = F.silu(s)")],
    "cond_without_silu": [(O.forward, "cond = F.silu(t_emb)", "cond = t_emb")],
    "head_without_norm": [(O.forward, 'out = linear(p, "final_layer.linear", rms_norm(pixels, p["final_layer.norm.weight"], cfg.norm_eps))',
                           'out = linear(p, "final_layer.linear", pixels)')],
    "head_norm_without_gain": [(O.forward, 'rms_norm(pixels, p["final_layer.norm.weight"], cfg.norm_eps)',
                                "rms_norm(pixels, None, cfg.norm_eps)")],
    "head_linear_before_norm": [(O.forward, 'out = linear(p, "final_layer.linear", rms_norm(pixels, p["final_layer.norm.weight"], cfg.norm_eps))',
                                 'out = rms_norm(linear(p, "final_layer.linear", pixels), None, cfg.norm_eps)')],
    "image_rows_first": [(O.forward, "torch.cat([text, s], dim=1)", "torch.cat([s, text], dim=1)")],
    "handover_rows_swapped": [(O.forward, "s, text = tokens[:, n_txt:], tokens[:, :n_txt]",
                               "s, text = tokens[:, :n_txt], tokens[:, n_txt:]")],
    "no_position_table": [(O.embed_text, 'y = y + p["y_pos_embedding"][:, : y.shape[1]]', "y = y")],
    "position_table_from_the_end": [(O.embed_text, 'p["y_pos_embedding"][:, : y.shape[1]]',
                                     'p["y_pos_embedding"][:, -y.shape[1]:]')],
    "text_not_truncated": [(O.embed_text, "y = y[:, : cfg.text_len]", "y = y")],
    "pixel_cond_before_trunk": [(O.forward, "cond_pix = s.reshape(", "cond_pix = F.silu(t_emb + linear(p, 's_embedder.proj', patchify(x, patch))).reshape(")],
    "patches_row_major_channels_last": [(O.forward, 's = linear(p, "s_embedder.proj", patchify(x, patch))',
                                         's = linear(p, "s_embedder.proj", patchify(x.transpose(2, 3), patch))')],
}


def _fails(forward, case):
    try:
        got, want = _compare(forward, case)
    except (RuntimeError, ValueError, IndexError):  # a shape mismatch is a failure too
        return True, "raised"
    if got.shape != want.shape:
        return True, "shape"
    err = (got - want).abs().max().item()
    return err > 100 * (ATOL + RTOL * want.abs().max().item()), f"max err {err:.3e}"


@pytest.mark.parametrize("mutation", sorted(MUTATIONS))
def test_a_mutated_forward_fails(mutation):
    """Every case either cannot apply the mistake (it depends on a branch the config does not take,
    e.g. the text hand-over of a dual-only trunk) or fails by at least 100x the tolerance; and at
    least one case fails."""
    forward = _mutant(MUTATIONS[mutation])
    results = {}
    for case in sorted(CASES):
        if mutation in ("image_rows_first", "handover_rows_swapped") and case.startswith("tiny"):
            continue  # all MM-DiT: no joined rows to hand over
        if mutation == "position_table_from_the_end" and case != "released_short_text":
            continue  # a whole table's worth of text: its first and last rows are the same rows
        if mutation == "text_not_truncated" and case == "released_short_text":
            continue  # fewer tokens than text_len: nothing to cut
        results[case] = _fails(forward, case)
    assert results and all(ok for ok, _ in results.values()), results


def test_unmutated_copy_passes():
    """The mutation harness itself leaves a faithful copy passing (so failures come from the edits)."""
    forward = _mutant([(O.forward, "cond = F.silu(t_emb)", "cond = F.silu(t_emb)")])
    for case in sorted(CASES):
        got, want = _compare(forward, case)
        torch.testing.assert_close(got, want, rtol=RTOL, atol=ATOL)


# ------------------------------------------------------------------------------------------
# rotary tables follow the token order of the patchify (dit.py:218-260, 326)
# ------------------------------------------------------------------------------------------
def test_image_rope_rows_follow_the_patch_token_order():
    """Token l of ``F.unfold`` is patch (row l // Wp, column l % Wp); its rotary row must rotate the
    first frequency pair by the column coordinate and the second by the row coordinate (x first,
    rope.py:19-82), with the isotropic step 16 / (max(Hp, Wp) - 1): on a 3 x 5 grid a swapped grid
    or a transposed coordinate gives other angles."""
    cfg = RELEASED_TOPOLOGY
    hp_, wp_ = 3, 5
    img, txt, pix = O.rope_tables(cfg, (hp_, wp_), 7)
    step = cfg.rope_scale / (max(hp_, wp_) - 1)
    f0 = 1.0  # the first frequency, theta ** 0
    for l in range(hp_ * wp_):
        row, col = divmod(l, wp_)
        ang = torch.angle(img[l, :2]).double()
        want = torch.tensor([col * step * f0, row * step * f0], dtype=torch.float64)
        want = torch.remainder(want + math.pi, 2 * math.pi) - math.pi
        torch.testing.assert_close(ang, want, rtol=0, atol=1e-5)
    assert img.shape == (hp_ * wp_, cfg.head_dim // 2)
    assert txt.shape == (7, cfg.head_dim // 2)  # one row per text token
    torch.testing.assert_close(torch.angle(txt[:, 0]).double(),
                               torch.remainder(torch.arange(7.0).double() + math.pi, 2 * math.pi) - math.pi,
                               rtol=0, atol=1e-5)
    ph = cfg.pixel.attn_hidden_size // cfg.pixel.num_heads
    assert pix.shape == (hp_ * wp_, ph // 2)
    torch.testing.assert_close(torch.angle(pix[:, :2]), torch.angle(O.rope_2d(ph, hp_, wp_, aspect=cfg.rope_aspect)[:, :2]))
