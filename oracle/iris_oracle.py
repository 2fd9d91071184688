"""FP32 CPU oracle of the Iris-3B denoiser forward, its text adapter and samplers.

TEST INFRASTRUCTURE ONLY. This module is the reference the HIP path is
compared against. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never
does, and it is never a fallback for the GPU path.

It restates the reference's PyTorch model semantics as plain functions over a
``state_dict`` (reference key names) in FP32, with explicit softmax attention
instead of a fused SDPA kernel. Each function cites the reference lines it
follows. How each function is pinned (reference tests restated, golden vectors
written by importing the unmodified ``iris3b.nn`` package, library routines,
closed forms) is listed in the test files ``tests/test_oracle_*.py``.

Parity status: every layer-level function is pinned by golden vectors of the
unmodified ``iris3b.nn`` modules. The blocks ``mmdit_block``,
``single_block`` and ``pit_block`` are pinned by golden vectors of the
unmodified reference block modules (blocks/mmdit.py, single_stream.py,
pit.py, loaded by file path) at the released topology and the tiny config.
The reference's ``IrisDiT`` itself cannot be imported here (its config module
needs omegaconf, which is absent); the glue of ``forward`` and ``embed_text``
that lives only in src/iris3b/models/dit.py:263-375 (``cond = silu(t_emb)``,
text truncation and the ``y_pos_embedding`` add, the block loop's hand-over
of ``[text | image]`` rows, the ``silu(t_emb + s)`` re-fusion, the
``FinalLayer`` RMSNorm then Linear, the fold) is pinned by closed-form
known answers at the released topology and the tiny config
(``tests/test_oracle_forward_glue.py``): weights that make every attention
uniform and every PiT branch a plain shift or bias give a flow computed from
library routines and golden-pinned layers alone, and each plausible mistake
written into a copy of this module's source fails that comparison.
The downstream wrappers ``depth_forward`` and ``restore_tile`` are pinned by
invariants of their own (``tests/test_tasks.py``): the zero fourth channel
equals the three-channel model with the sliced embedders, and a head that
predicts a constant flow moves every pixel by exactly ``-sigma`` times it.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

Tensor = torch.Tensor
Params = dict[str, Tensor]


# ----------------------------------------------------------------------------
# layers
# ----------------------------------------------------------------------------
def linear(p: Params, name: str, x: Tensor) -> Tensor:
    """``nn.Linear`` by state_dict name; bias optional."""
    return F.linear(x, p[f"{name}.weight"], p.get(f"{name}.bias"))


def rms_norm(x: Tensor, weight: Tensor | None, eps: float) -> Tensor:
    """src/iris3b/nn/norms.py:15-21: FP32 statistics, gain applied after."""
    x32 = x.float()
    normed = x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + eps)
    return normed if weight is None else weight * normed


def norm(p: Params, name: str, x: Tensor, eps: float) -> Tensor:
    """RMSNorm when ``name`` has a gain in ``p``, identity otherwise (nn.Identity slots)."""
    key = f"{name}.weight"
    return rms_norm(x, p[key], eps) if key in p else x


def modulate(x: Tensor, shift: Tensor, scale: Tensor) -> Tensor:
    """src/iris3b/nn/modulation.py:11-12."""
    return x * (1 + scale) + shift


def swiglu(p: Params, name: str, x: Tensor) -> Tensor:
    """src/iris3b/nn/mlp.py:24-40."""
    return linear(p, f"{name}.w2", F.silu(linear(p, f"{name}.w1", x)) * linear(p, f"{name}.w3", x))


def gelu_mlp(p: Params, name: str, x: Tensor) -> Tensor:
    """src/iris3b/nn/mlp.py:43-53 (exact-erf GELU)."""
    return linear(p, f"{name}.fc2", F.gelu(linear(p, f"{name}.fc1", x)))


# ----------------------------------------------------------------------------
# rotary tables (src/iris3b/nn/rope.py:19-101)
# ----------------------------------------------------------------------------
def rope_2d(
    head_dim: int,
    height: int,
    width: int,
    theta: float = 10000.0,
    scale: float = 16.0,
    aspect: str = "square",
    frame_pairs: int = 0,
    frame_theta: float = 10.0,
    frame_index: int = 0,
) -> Tensor:
    """Complex ``[height*width, head_dim//2]`` table; (x, y) frequency pairs interleaved."""
    n_pairs = head_dim // 4
    if not 0 <= frame_pairs < n_pairs:
        raise ValueError(f"rope: frame_pairs={frame_pairs} is not one of 0..{n_pairs - 1}")
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 4)[:n_pairs].float() / head_dim)
    freqs = freqs[: n_pairs - frame_pairs]
    if aspect == "square":
        xs, ys = torch.linspace(0, scale, width), torch.linspace(0, scale, height)
    elif aspect == "isotropic":
        step = scale / max(max(height, width) - 1, 1)
        xs, ys = torch.arange(width).float() * step, torch.arange(height).float() * step
    else:
        raise ValueError(f"rope: aspect must be 'square' or 'isotropic', got {aspect!r}")
    x_ang, y_ang = torch.outer(xs, freqs), torch.outer(ys, freqs)
    x_cis = torch.polar(torch.ones_like(x_ang), x_ang)[None, :, :].expand(height, width, -1)
    y_cis = torch.polar(torch.ones_like(y_ang), y_ang)[:, None, :].expand(height, width, -1)
    cis = torch.stack([x_cis, y_cis], dim=-1).reshape(height * width, -1)
    if frame_pairs:
        slots = 2 * frame_pairs
        f_freqs = 1.0 / frame_theta ** (torch.arange(slots).float() / slots)
        f_cis = torch.polar(torch.ones(slots), float(frame_index) * f_freqs)
        cis = torch.cat([cis, f_cis[None, :].expand(height * width, -1)], dim=-1)
    return cis


def rope_1d(head_dim: int, length: int, theta: float = 10000.0) -> Tensor:
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 2)[: head_dim // 2].float() / head_dim)
    ang = torch.outer(torch.arange(length).float(), freqs)
    return torch.polar(torch.ones_like(ang), ang)


def apply_rope(q: Tensor, k: Tensor, cis: Tensor) -> tuple[Tensor, Tensor]:
    """Rotate adjacent pairs of ``[B, N, H, d]`` by complex ``cis[N, d/2]`` in FP32."""
    fc = cis[None, :, None, :]

    def rot(t: Tensor) -> Tensor:
        c = torch.view_as_complex(t.float().reshape(*t.shape[:-1], -1, 2).contiguous())
        return torch.view_as_real(c * fc).flatten(3).to(t.dtype)

    return rot(q), rot(k)


# ----------------------------------------------------------------------------
# attention (src/iris3b/nn/attention.py:61-244)
# ----------------------------------------------------------------------------
def attention(q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None = None) -> Tensor:
    """softmax(q kᵀ / sqrt(d)) v over ``[B, H, N, d]``; grouped K/V heads are repeated.

    ``mask``: bool, broadcastable to ``[B, H, Nq, Nk]``, True = attend.
    Evaluated one head at a time to bound memory at the 1024² shapes.
    """
    heads, kv_heads = q.shape[1], k.shape[1]
    if heads != kv_heads:
        k = k.repeat_interleave(heads // kv_heads, dim=1)
        v = v.repeat_interleave(heads // kv_heads, dim=1)
    scale = 1.0 / math.sqrt(q.shape[-1])
    out = torch.empty(q.shape[:-1] + (v.shape[-1],), dtype=torch.float32, device=q.device)
    for h in range(heads):
        s = torch.matmul(q[:, h].float(), k[:, h].float().transpose(-1, -2).contiguous()) * scale
        if mask is not None:
            m = mask[:, min(h, mask.shape[1] - 1)] if mask.dim() == 4 else mask
            s = s.masked_fill(~m, float("-inf"))
        out[:, h] = torch.matmul(torch.softmax(s, dim=-1), v[:, h].float())
    return out


def self_attention(
    p: Params, name: str, x: Tensor, heads: int, eps: float, rope: Tensor | None = None, mask=None
) -> Tensor:
    """``SelfAttention.forward`` (attention.py:117-132): fused QKV, per-head QK norm, RoPE."""
    b, n, dim = x.shape
    q, k, v = linear(p, f"{name}.qkv", x).reshape(b, n, 3, heads, dim // heads).unbind(2)
    q, k = norm(p, f"{name}.q_norm", q, eps), norm(p, f"{name}.k_norm", k, eps)
    if rope is not None:
        q, k = apply_rope(q, k, rope)
    out = attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask)
    return linear(p, f"{name}.proj", out.transpose(1, 2).reshape(b, n, dim))


# ----------------------------------------------------------------------------
# embedders (src/iris3b/nn/embeddings.py)
# ----------------------------------------------------------------------------
def timestep_features(t: Tensor, freq_dim: int = 256, max_period: float = 10.0) -> Tensor:
    """embeddings.py:41-45: ``[cos | sin]`` of ``t * exp(-ln(P) k / n)``."""
    n = freq_dim // 2
    k = torch.arange(n, dtype=torch.float32, device=t.device)
    phase = torch.outer(t.float(), torch.exp(-math.log(max_period) * k / n))
    return torch.cat([phase.cos(), phase.sin()], dim=-1)


def timestep_embed(p: Params, t: Tensor, max_period: float) -> Tensor:
    """embeddings.py:47-52 -> ``[B, 1, D]``."""
    h = F.silu(linear(p, "t_embedder.mlp.0", timestep_features(t.reshape(-1), 256, max_period)))
    return linear(p, "t_embedder.mlp.2", h).reshape(t.shape[0], 1, -1)


def sincos_1d(dim: int, pos: Tensor) -> Tensor:
    """embeddings.py:269-274: FP64 ``[sin | cos]`` over ``dim`` channels."""
    omega = 1.0 / 10000.0 ** (torch.arange(dim // 2, dtype=torch.float64) / (dim / 2.0))
    out = torch.outer(pos.reshape(-1).double(), omega)
    return torch.cat([torch.sin(out), torch.cos(out)], dim=1)


def sincos_2d(dim: int, height: int, width: int) -> Tensor:
    """embeddings.py:277-288: ``[H*W, dim]``, first half from the x (column) coordinate."""
    ys, xs = torch.meshgrid(torch.arange(height, dtype=torch.float32), torch.arange(width, dtype=torch.float32), indexing="ij")
    return torch.cat([sincos_1d(dim // 2, xs), sincos_1d(dim // 2, ys)], dim=1).float()


def pixel_embed(p: Params, x: Tensor, patch: int, abs_pos: bool) -> Tensor:
    """embeddings.py:291-328: ``[B,C,H,W] -> [B*(H/p)*(W/p), p*p, hidden]``, row-major in patch."""
    b, _, h, w = x.shape
    tokens = linear(p, "pixel_embedder.proj", x.permute(0, 2, 3, 1))
    if abs_pos:
        tokens = tokens + sincos_2d(tokens.shape[-1], h, w).reshape(h, w, -1).to(tokens)
    tokens = tokens.reshape(b, h // patch, patch, w // patch, patch, -1).permute(0, 1, 3, 2, 4, 5)
    return tokens.reshape(b * (h // patch) * (w // patch), patch * patch, -1)


def patchify(x: Tensor, patch: int) -> Tensor:
    """``F.unfold(x, p, stride=p).transpose(1, 2)`` (dit.py:326) as a reshape:
    ``[B, C, H, W] -> [B, L, C*p*p]`` with channel-major, then row, then column order."""
    b, c, h, w = x.shape
    t = x.reshape(b, c, h // patch, patch, w // patch, patch).permute(0, 2, 4, 1, 3, 5)
    return t.reshape(b, (h // patch) * (w // patch), c * patch * patch)


def unpatchify(out: Tensor, batch: int, height: int, width: int, patch: int) -> Tensor:
    """The PiT head fold (dit.py:370-374): ``[B*L, p*p, C] -> [B, C, H, W]``."""
    c = out.shape[-1]
    t = out.reshape(batch, height // patch, width // patch, patch, patch, c).permute(0, 5, 1, 3, 2, 4)
    return t.reshape(batch, c, height, width)


# ----------------------------------------------------------------------------
# text adapters (embeddings.py:111-266) and embed_text (dit.py:263-281)
# ----------------------------------------------------------------------------
def transformer_text(p: Params, name: str, y: Tensor, mask: Tensor, heads: int, eps: float) -> Tensor:
    """``TransformerTextEmbedder``: pad keys masked, each query keeps its own position."""
    if mask.shape != y.shape[:2]:
        raise ValueError(f"text mask must be {tuple(y.shape[:2])}, got {tuple(mask.shape)}")
    eye = torch.eye(y.shape[1], dtype=torch.bool, device=y.device)
    keep = mask.bool()[:, None, None, :] | eye
    y = linear(p, f"{name}.proj", y)
    for i in range(2):
        b = f"{name}.blocks.{i}"
        y = y + self_attention(p, f"{b}.attn", rms_norm(y, p[f"{b}.norm1.weight"], eps), heads, eps, mask=keep)
        y = y + swiglu(p, f"{b}.mlp", rms_norm(y, p[f"{b}.norm2.weight"], eps))
    return rms_norm(y, p[f"{name}.norm.weight"], eps)


def layerwise_text(p: Params, cfg, y: Tensor, mask: Tensor) -> Tensor:
    """``LayerwiseTextEmbedder``: per-token attention over encoder layers, learned pool, refiner."""
    eps = cfg.norm_eps
    expected = (*mask.shape, cfg.text_lap_num_layers, cfg.text_dim)
    if tuple(y.shape) != expected:
        raise ValueError(f"layerwise text states must be {expected}, got {tuple(y.shape)}")
    b, n, layers, dim = y.shape
    h = y.reshape(b * n, layers, dim)
    for i in range(2):
        blk = f"y_embedder.layer_blocks.{i}"
        h = h + self_attention(p, f"{blk}.attn", rms_norm(h, p[f"{blk}.norm1.weight"], eps), cfg.text_lap_num_heads, eps)
        m = rms_norm(h, p[f"{blk}.norm2.weight"], eps)
        h = h + linear(p, f"{blk}.mlp.2", F.silu(linear(p, f"{blk}.mlp.0", m)))
    pooled = linear(p, "y_embedder.layer_pool", h.transpose(1, 2)).squeeze(-1).reshape(b, n, dim)
    return transformer_text(p, "y_embedder.refiner", pooled, mask, cfg.num_heads, eps)


def embed_text(p: Params, cfg, y: Tensor, mask: Tensor | None = None) -> Tensor:
    y = y[:, : cfg.text_len]
    if cfg.text_adapter == "linear":
        y = rms_norm(linear(p, "y_embedder.proj", y), p["y_embedder.norm.weight"], cfg.norm_eps)
    else:
        if mask is None:
            raise ValueError(f"text_adapter={cfg.text_adapter!r} requires y_mask")
        mask = mask[:, : cfg.text_len]
        if cfg.text_adapter == "blocks2":
            y = transformer_text(p, "y_embedder", y, mask, cfg.num_heads, cfg.norm_eps)
        else:
            y = layerwise_text(p, cfg, y, mask)
    if cfg.text_abs_pos_embed:
        y = y + p["y_pos_embedding"][:, : y.shape[1]]
    return y


# ----------------------------------------------------------------------------
# adaLN (src/iris3b/nn/modulation.py:258-334)
# ----------------------------------------------------------------------------
def modulation(p: Params, cfg, prefix: str, stream: str, cond: Tensor) -> Tensor:
    """``[B, 1, 6D]`` modulation of block ``prefix`` for ``stream`` (img | txt | shared)."""
    name = f"{prefix}.adaln" if stream == "shared" else f"{prefix}.adaln_{stream}"
    if cfg.modulation == "per_block":
        return linear(p, name, cond)
    core = {"shared": "img"}.get(stream, stream) if cfg.dual_depth else stream
    shared = linear(p, f"modulation_cores.adaln_{core}", cond)
    if cfg.modulation == "shared_bias":
        return shared + p[f"{name}.bias"]
    return shared + F.linear(F.linear(cond, p[f"{name}.down.weight"]), p[f"{name}.adaln_up.weight"])


# ----------------------------------------------------------------------------
# blocks
# ----------------------------------------------------------------------------
def _project(p: Params, cfg, prefix: str, suffix: str, h: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Q, K, V as ``[B, N, heads, d]`` from fused QKV (MHA) or separate projections (GQA)."""
    b, n, _ = h.shape
    hd = cfg.head_dim
    if f"{prefix}qkv{suffix}.weight" in p:
        return linear(p, f"{prefix}qkv{suffix}", h).reshape(b, n, 3, cfg.num_heads, hd).unbind(2)
    q = linear(p, f"{prefix}q_proj{suffix}", h).reshape(b, n, cfg.num_heads, hd)
    k = linear(p, f"{prefix}k_proj{suffix}", h).reshape(b, n, cfg.kv_heads, hd)
    v = linear(p, f"{prefix}v_proj{suffix}", h).reshape(b, n, cfg.kv_heads, hd)
    return q, k, v


def mmdit_block(p, cfg, i: int, x: Tensor, y: Tensor, cond: Tensor, rope_img, rope_txt):
    """``MMDiTBlock.forward`` + ``JointAttention`` (blocks/mmdit.py:84-128, attention.py:205-244)."""
    b = f"blocks.{i}"
    eps = cfg.norm_eps
    text_out = cfg.text_out(i)
    xs1, xc1, xg1, xs2, xc2, xg2 = modulation(p, cfg, b, "img", cond).chunk(6, dim=-1)
    ys1, yc1, yg1, ys2, yc2, yg2 = modulation(p, cfg, b, "txt", cond).chunk(6, dim=-1)
    hx = modulate(rms_norm(x, p[f"{b}.norm_x1.weight"], eps), xs1, xc1)
    hy = modulate(rms_norm(y, p[f"{b}.norm_y1.weight"], eps), ys1, yc1)

    n_txt = y.shape[1]
    qx, kx, vx = _project(p, cfg, f"{b}.attn.", "_x", hx)
    qy, ky, vy = _project(p, cfg, f"{b}.attn.", "_y", hy)
    qx, kx = norm(p, f"{b}.attn.q_norm_x", qx, eps), norm(p, f"{b}.attn.k_norm_x", kx, eps)
    qy, ky = norm(p, f"{b}.attn.q_norm_y", qy, eps), norm(p, f"{b}.attn.k_norm_y", ky, eps)
    qx, kx = apply_rope(qx, kx, rope_img)
    if rope_txt is not None:
        qy, ky = apply_rope(qy, ky, rope_txt)
    q, k, v = (torch.cat(pair, dim=1).transpose(1, 2) for pair in ((qy, qx), (ky, kx), (vy, vx)))
    out = attention(q, k, v).transpose(1, 2).reshape(x.shape[0], n_txt + x.shape[1], -1)
    out_x, out_y = out[:, n_txt:], out[:, :n_txt]
    if f"{b}.attn_gate_x.weight" in p:
        out_x = out_x * torch.sigmoid(linear(p, f"{b}.attn_gate_x", hx))
    x = x + xg1 * norm(p, f"{b}.attn_post_norm_x", linear(p, f"{b}.attn.proj_x", out_x), eps)
    mlp_x = swiglu(p, f"{b}.mlp_x", modulate(rms_norm(x, p[f"{b}.norm_x2.weight"], eps), xs2, xc2))
    x = x + xg2 * norm(p, f"{b}.mlp_post_norm_x", mlp_x, eps)
    if not text_out:
        return x, y
    if f"{b}.attn_gate_y.weight" in p:
        out_y = out_y * torch.sigmoid(linear(p, f"{b}.attn_gate_y", hy))
    y = y + yg1 * norm(p, f"{b}.attn_post_norm_y", linear(p, f"{b}.attn.proj_y", out_y), eps)
    mlp_y = swiglu(p, f"{b}.mlp_y", modulate(rms_norm(y, p[f"{b}.norm_y2.weight"], eps), ys2, yc2))
    return x, y + yg2 * norm(p, f"{b}.mlp_post_norm_y", mlp_y, eps)


def single_block(p, cfg, i: int, tokens: Tensor, n_txt: int, cond: Tensor, rope_img, rope_txt) -> Tensor:
    """``SingleStreamBlock.forward_joint`` (blocks/single_stream.py:90-143) over ``[text | image]``.
    Returns all rows, or only the image rows when the block has no text output."""
    b = f"blocks.{i}"
    eps = cfg.norm_eps
    s1, c1, g1, s2, c2, g2 = modulation(p, cfg, b, "shared", cond).chunk(6, dim=-1)
    h = modulate(rms_norm(tokens, p[f"{b}.norm1.weight"], eps), s1, c1)
    q, k, v = _project(p, cfg, f"{b}.", "", h)
    q, k = norm(p, f"{b}.q_norm", q, eps), norm(p, f"{b}.k_norm", k, eps)
    if rope_txt is not None:
        q, k = apply_rope(q, k, torch.cat([rope_txt, rope_img]))
    else:
        qi, ki = apply_rope(q[:, n_txt:], k[:, n_txt:], rope_img)
        q, k = torch.cat([q[:, :n_txt], qi], dim=1), torch.cat([k[:, :n_txt], ki], dim=1)
    out = attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    out = out.transpose(1, 2).reshape(tokens.shape)
    if not cfg.text_out(i):
        out, h, tokens = out[:, n_txt:], h[:, n_txt:], tokens[:, n_txt:]
    if f"{b}.attn_gate.weight" in p:
        out = out * torch.sigmoid(linear(p, f"{b}.attn_gate", h))
    tokens = tokens + g1 * norm(p, f"{b}.attn_post_norm", linear(p, f"{b}.attn_proj", out), eps)
    mlp = swiglu(p, f"{b}.mlp", modulate(rms_norm(tokens, p[f"{b}.norm2.weight"], eps), s2, c2))
    return tokens + g2 * norm(p, f"{b}.mlp_post_norm", mlp, eps)


def pit_block(p, cfg, i: int, x: Tensor, cond: Tensor, rope: Tensor, grid: tuple[int, int]) -> Tensor:
    """``PiTBlock.forward`` (blocks/pit.py:66-93), both modulation layouts."""
    b = f"pixel_blocks.{i}"
    eps = cfg.norm_eps
    px = cfg.pixel
    n_patches = grid[0] * grid[1]
    batch = x.shape[0] // n_patches

    def global_attn(h: Tensor) -> Tensor:
        compact = linear(p, f"{b}.compress", h.reshape(batch * n_patches, -1))
        a = self_attention(p, f"{b}.attn", compact.reshape(batch, n_patches, -1), px.num_heads, eps, rope)
        return linear(p, f"{b}.expand", a.reshape(batch * n_patches, -1)).reshape_as(h)

    mods = linear(p, f"{b}.adaln", cond).reshape(x.shape[0], cfg.pixels_per_patch, -1)
    n1, n2 = p[f"{b}.norm1.weight"], p[f"{b}.norm2.weight"]
    if px.modulation == "pre":
        shift1, scale1, gate1, shift2, scale2, gate2 = mods.chunk(6, dim=-1)
        x = x + gate1 * global_attn(modulate(rms_norm(x, n1, eps), shift1, scale1))
        return x + gate2 * gelu_mlp(p, f"{b}.mlp", modulate(rms_norm(x, n2, eps), shift2, scale2))
    scale1, shift1, scale2, shift2 = mods.chunk(4, dim=-1)
    x = x + modulate(global_attn(rms_norm(x, n1, eps)), shift1, scale1)
    return x + modulate(gelu_mlp(p, f"{b}.mlp", rms_norm(x, n2, eps)), shift2, scale2)


# ----------------------------------------------------------------------------
# the forward (src/iris3b/models/dit.py:283-375)
# ----------------------------------------------------------------------------
def rope_tables(cfg, grid: tuple[int, int], n_text: int):
    """(image, text or None, pixel-stage) complex tables (dit.py:218-260)."""
    img = rope_2d(
        cfg.head_dim, *grid, theta=cfg.rope_theta, scale=cfg.rope_scale, aspect=cfg.rope_aspect,
        frame_pairs=cfg.rope_frame_pairs, frame_theta=cfg.rope_frame_theta,
    )
    txt = rope_1d(cfg.head_dim, n_text, theta=cfg.text_rope_theta) if cfg.text_rope else None
    pix = None
    if cfg.pixel.enabled:
        pix = rope_2d(
            cfg.pixel.attn_hidden_size // cfg.pixel.num_heads, *grid, theta=cfg.rope_theta,
            scale=cfg.rope_scale, aspect=cfg.rope_aspect,
        )
    return img, txt, pix


@torch.no_grad()
def forward(p: Params, cfg, x: Tensor, t: Tensor, y: Tensor | None = None, y_mask: Tensor | None = None,
            prepared_text: Tensor | None = None, capture: tuple[int, ...] = ()) -> Tensor:
    """Predicted flow ``[B, C, H, W]`` for noised pixels ``x``, model time ``t`` and text.

    With ``capture`` the patch tokens after the given 1-based blocks are
    returned too, as ``(v, {index: tokens})``.
    """
    patch = cfg.patch_size
    batch, _, height, width = x.shape
    if height % patch or width % patch:
        raise ValueError(f"input {height}x{width} is not divisible by patch_size {patch}")
    grid = (height // patch, width // patch)
    x = x.float()
    s = linear(p, "s_embedder.proj", patchify(x, patch))
    t_emb = timestep_embed(p, t, cfg.timestep_max_period)
    cond = F.silu(t_emb)
    text = embed_text(p, cfg, y, y_mask) if prepared_text is None else prepared_text.float()
    rope_img, rope_txt, rope_pix = rope_tables(cfg, grid, text.shape[1])

    features = {}
    n_txt = text.shape[1]
    for i in range(cfg.depth):
        if cfg.block_kind(i) == "mmdit":
            s, text = mmdit_block(p, cfg, i, s, text, cond, rope_img, rope_txt)
        else:
            tokens = single_block(p, cfg, i, torch.cat([text, s], dim=1), n_txt, cond, rope_img, rope_txt)
            if cfg.text_out(i):
                s, text = tokens[:, n_txt:], tokens[:, :n_txt]
            else:
                s = tokens
        if i + 1 in capture:
            features[i + 1] = s
    s = F.silu(t_emb + s)

    if not cfg.pixel.enabled:
        out = linear(p, "final_layer.linear", rms_norm(s, p["final_layer.norm.weight"], cfg.norm_eps))
        c = cfg.in_channels
        out = out.reshape(batch * grid[0] * grid[1], c, patch * patch).transpose(1, 2)
        v = unpatchify(out, batch, height, width, patch)
    else:
        cond_pix = s.reshape(batch * grid[0] * grid[1], -1)
        pixels = pixel_embed(p, x, patch, cfg.pixel.abs_pos_embed)
        for i in range(cfg.pixel.depth):
            pixels = pit_block(p, cfg, i, pixels, cond_pix, rope_pix, grid)
        out = linear(p, "final_layer.linear", rms_norm(pixels, p["final_layer.norm.weight"], cfg.norm_eps))
        v = unpatchify(out, batch, height, width, patch)
    return (v, features) if capture else v


# ----------------------------------------------------------------------------
# samplers (src/iris3b/sampling.py:98-138, src/iris3b/flow/solver.py, schedule.py:24-25)
# ----------------------------------------------------------------------------
TURBO_SIGMAS = (1.0, 0.938, 0.833, 0.625)


# ----------------------------------------------------------------------------
# downstream tasks (src/iris3b/downstream/depth.py, restoration.py)
# ----------------------------------------------------------------------------
def depth_forward(p: Params, cfg, rgb: Tensor, embeddings: Tensor, mask: Tensor,
                  num_train_timesteps: int = 1000) -> Tensor:
    """``IrisDepth.forward`` (depth.py:41-48): RGB plus a zero channel after it into the widened
    embedders of the ``pixel.*`` denoiser at model time ``num_train_timesteps`` with the (empty)
    prompt, then the 1x1 ``depth_reducer`` -> ``[B, 1, H, W]``."""
    b, _, h, w = rgb.shape
    sub = {k[len("pixel."):]: v for k, v in p.items() if k.startswith("pixel.")}
    x = torch.cat([rgb.float(), torch.zeros(b, 1, h, w)], dim=1)
    t = torch.full((b,), float(num_train_timesteps))
    out = forward(sub, cfg, x, t, embeddings.expand(b, *embeddings.shape[1:]), y_mask=mask.expand(b, -1))
    return F.conv2d(out, p["depth_reducer.weight"], p["depth_reducer.bias"])


def restore_tile(p: Params, cfg, x: Tensor, embeddings: Tensor, mask: Tensor, sigma: float,
                 num_train_timesteps: int = 1000) -> Tensor:
    """``Restorer.restore_tile`` (restoration.py:135-142): one forward at model time
    ``sigma * num_train_timesteps`` with the (empty) prompt, then ``x - sigma * v``."""
    t = torch.full((x.shape[0],), sigma * num_train_timesteps)
    y = embeddings.expand(len(x), *embeddings.shape[1:])
    v = forward(p, cfg, x, t, y, y_mask=mask.expand(len(x), -1))
    return x.float() - sigma * v.float()


def turbo_sample(model_fn, noise: Tensor, sigmas=TURBO_SIGMAS, num_train_timesteps: int = 1000,
                 prediction: str = "v", check=None) -> Tensor:
    """Deterministic few-step flow-Euler without CFG; ``model_fn(x, t_model) -> out``."""
    x = noise.float()
    sigma = torch.full((x.shape[0], 1, 1, 1), sigmas[0], dtype=torch.float32, device=x.device)
    clean = x
    for i in range(len(sigmas)):
        out = model_fn(x, sigma.flatten() * num_train_timesteps).float()
        clean = out if prediction == "x" else x - sigma * out
        if i + 1 < len(sigmas):
            implied_noise = (x - (1 - sigma) * clean) / sigma
            sigma = torch.full_like(sigma, sigmas[i + 1])
            x = (1 - sigma) * clean + sigma * implied_noise
    if check is not None:
        check(clean)
    return clean.clamp(-1, 1)


def shift_sigma(sigma: Tensor, shift: float) -> Tensor:
    return shift * sigma / (1 + (shift - 1) * sigma)


def time_grid(steps: int, shift: float) -> list[float]:
    sigma = 1.0 - torch.linspace(1.0, 0.001, steps + 1, dtype=torch.float64)
    return shift_sigma(sigma, shift).flip(0).tolist()


def _lam(t: float) -> float:
    return math.inf if t <= 0.0 else math.log((1.0 - t) / t)


def dpm_sample(model_fn, z: Tensor, cond: Tensor, uncond: Tensor | None = None, steps: int = 50,
               order: int = 2, shift: float = 1.0, cfg_scale: float = 1.0,
               cfg_interval: tuple[float, float] = (0.0, 1.0), prediction: str = "v",
               num_timesteps: int = 1000) -> Tensor:
    """``FlowDPMSolver.sample`` (solver.py:111-141); ``model_fn(x, t_model, text) -> out``."""
    grid = time_grid(steps, shift)
    x = z
    history: list[tuple[float, Tensor]] = []
    for i in range(1, steps + 1):
        s, t = grid[i - 1], grid[i]
        lo, hi = cfg_interval
        use_cfg = uncond is not None and cfg_scale != 1.0 and lo < s < hi
        rows = 2 * x.shape[0] if use_cfg else x.shape[0]
        t_model = torch.full((rows,), s * num_timesteps, dtype=torch.float32, device=x.device)
        if use_cfg:
            out_u, out_c = model_fn(torch.cat([x, x]), t_model, torch.cat([uncond, cond])).chunk(2)
            out = out_u + cfg_scale * (out_c - out_u)
        else:
            out = model_fn(x, t_model, cond)
        x0 = out if prediction == "x" else x - s * out
        history.append((s, x0))
        step_order = min(i, order, steps + 1 - i)
        if step_order == 1:
            phi1 = math.expm1(-(_lam(t) - _lam(s)))
            x = (t / s) * x - (1.0 - t) * phi1 * x0
        else:
            (s1, x0_1), (s0, x0_0) = history[-2], history[-1]
            h, h0 = _lam(t) - _lam(s0), _lam(s0) - _lam(s1)
            d = (x0_0 - x0_1) / (h0 / h)
            phi1 = math.expm1(-h)
            x = (t / s0) * x - (1.0 - t) * phi1 * x0_0 - 0.5 * (1.0 - t) * phi1 * d
        if len(history) > 2:
            history.pop(0)
    return x
