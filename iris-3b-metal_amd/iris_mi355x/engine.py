"""``HipIris``: the Iris-3B velocity predictor ``(x, t, text) -> v`` on one MI355X.

Drop-in for the reference engine's call surface (``MetalIris``, src/iris_metal/model.py:113-217):
same constructor checks, ``__call__(x, t, text)`` with ``x`` ``[B, 3, H, W]``, model time
``t`` ``[B]`` and prepared text tokens ``[B, T, D]``, returning FP32 velocity, under no-grad,
without modifying its inputs. Every operation of the forward is one of the HIP kernels of
``libiris_hip.so``; torch only provides device memory and the stream.

Precision plan: residual streams (trunk and pixel stage), norm statistics, modulation,
rotary math and softmax are FP32; GEMM and attention operands are BF16 with FP32
accumulation; every activation crossing a GEMM is stored BF16 once.

Data layout in HBM (per call shape, allocated once and reused):
- dual-stream phase: image ``X`` ``[B*L, D]`` and text ``Y`` ``[B*T, D]`` FP32 residuals;
- single-stream phase: ``tok`` ``[B*N, D]`` FP32 with the text rows first in each batch (for one
  batch item ``Y`` and ``X`` are its first ``T`` and last ``L`` rows, so the join copies nothing);
- packed projections ``[rows, 6400]`` = ``q | k | v | gate``: one call per block over the packed
  weight (two GEMMs in one launch), the q | k | v one writing the attention inputs below
  straight from its store (Q / K normed and rotated; V transposed when each batch item is whole
  256-row tiles, else its V columns land here for ``v_heads_t``), the gate one its columns here;
- attention inputs ``q`` ``[B, 20, N_pad, 128]``, ``k`` ``[B, 5, N_pad, 128]``, ``v^T`` ``[B, 5, 128, N_pad]``;
- pixel stream ``[B*L, p*p, 16]`` FP32 and its BF16 normed copy, adaLN mods ``[B*L, p*p, 64]`` BF16.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels as K
from . import tables
from .config import ModelConfig

HEAD_DIM = K.HEAD_DIM


def check_supported(cfg: ModelConfig) -> None:
    """Reject topologies the fused forward does not handle (src/iris_metal/model.py:68-93)."""
    requirements = {
        "a pixel stage with post-modulated blocks": cfg.pixel.enabled and cfg.pixel.modulation == "post",
        "shared_bias modulation with a dual-stream prefix": cfg.modulation == "shared_bias" and cfg.dual_depth > 0,
        "a single-stream final block": cfg.block_kind(cfg.depth - 1) == "single_stream"
        and cfg.block == "single_stream",
        "grouped-query, gated, sandwich-normed, QK-normed attention": (
            cfg.num_kv_heads is not None
            and cfg.num_kv_heads < cfg.num_heads
            and cfg.gated_attention
            and cfg.sandwich_norm
            and cfg.qk_norm
        ),
        f"{HEAD_DIM}-wide attention heads": (
            cfg.hidden_size // cfg.num_heads == HEAD_DIM
            and cfg.pixel.attn_hidden_size // cfg.pixel.num_heads == HEAD_DIM
        ),
        "a masked text adapter with text RoPE and position table": (
            cfg.text_adapter != "linear" and cfg.text_rope and cfg.text_abs_pos_embed
        ),
        "16-channel pixels with a 64-wide MLP": cfg.pixel.hidden_size == K.PIXEL_WIDTH
        and int(cfg.pixel.hidden_size * cfg.pixel.mlp_ratio) == K.PIXEL_HIDDEN and cfg.in_channels == 3,
    }
    missing = [name for name, ok in requirements.items() if not ok]
    if missing:
        raise ValueError(f"HipIris supports the released Iris-3B topology; this model lacks {missing}")


def require_finite(result: torch.Tensor) -> torch.Tensor:
    """Raise rather than return an overflowed result (src/iris_metal/model.py:102-110)."""
    if not torch.isfinite(result).all():
        raise FloatingPointError("the model produced non-finite values; please report the input and settings")
    return result


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


@dataclass
class _Shape:
    batch: int
    height: int
    width: int
    n_text: int


class HipIris:
    """Velocity predictor over a ``state_dict`` with the reference's key names.

    ``HipIris(cfg, state_dict)`` or ``HipIris.from_module(dit)`` for an object exposing ``cfg``
    and ``state_dict()`` (an upstream ``IrisDiT``).

    With ``graphs=True`` (the default) the inputs are copied into buffers the engine owns, the
    forward over them is recorded once per input shape as a HIP graph (after one eager run,
    whose result that call returns) and replayed by later calls: one launch instead of ~330,
    whatever buffers the caller passes. The result is copied out of the engine's buffer.
    """

    def __init__(self, cfg: ModelConfig, state_dict: dict[str, torch.Tensor], device: str | torch.device = "cuda",
                 graphs: bool = True):
        cfg.validate()
        check_supported(cfg)
        self.cfg = cfg
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("HipIris runs on the GPU only")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.eps = cfg.norm_eps
        self.hidden_pad = _round_up(cfg.mlp_hidden, 64)
        self._prepare(state_dict)
        self._ws: dict | None = None
        self._ws_shape: _Shape | None = None
        self._tables: dict = {}
        self.graphs = graphs

    @classmethod
    def from_module(cls, dit, device: str | torch.device = "cuda") -> "HipIris":
        return cls(dit.cfg, dit.state_dict(), device)

    # -- weights ----------------------------------------------------------------------
    def _prepare(self, sd: dict[str, torch.Tensor]) -> None:
        cfg, dev = self.cfg, self.device

        def f32(name: str) -> torch.Tensor:
            return sd[name].detach().to(dev, torch.float32).contiguous()

        def bf(t: torch.Tensor) -> torch.Tensor:
            return t.detach().to(dev, torch.bfloat16).contiguous()

        def w(name: str) -> torch.Tensor:
            return bf(sd[f"{name}.weight"])

        def cat_rows(*names: str) -> torch.Tensor:
            return bf(torch.cat([sd[f"{n}.weight"].detach().float() for n in names], dim=0))

        def swiglu(prefix: str) -> tuple[torch.Tensor, torch.Tensor]:
            w1 = sd[f"{prefix}.w1.weight"].detach().float()
            w3 = sd[f"{prefix}.w3.weight"].detach().float()
            w2 = sd[f"{prefix}.w2.weight"].detach().float()
            packed = K.pack_swiglu(w1, w3, self.hidden_pad)
            w2p = torch.zeros(w2.shape[0], self.hidden_pad)
            w2p[:, : w2.shape[1]] = w2
            return bf(packed), bf(w2p)

        # the patch embedder's K (C*p*p) is zero-padded to the GEMM's multiple of 64; C is 3, or 4
        # for the depth fine-tune, whose embedders take an extra input channel after RGB
        # (src/iris3b/downstream/depth.py:30-39)
        s_w = sd["s_embedder.proj.weight"].detach().float()
        pp = cfg.patch_size ** 2
        self.in_channels = s_w.shape[1] // pp
        if s_w.shape[1] % pp or self.in_channels not in (3, 4):
            raise ValueError(f"s_embedder.proj takes {s_w.shape[1]} features: not 3 or 4 channels of {pp} pixels")
        if tuple(sd["pixel_embedder.proj.weight"].shape) != (K.PIXEL_WIDTH, self.in_channels):
            raise ValueError("pixel_embedder.proj does not take the patch embedder's input channels")
        self.patch_k = _round_up(s_w.shape[1], 64)
        self.s_w = bf(torch.nn.functional.pad(s_w, (0, self.patch_k - s_w.shape[1])))
        self.s_b = f32("s_embedder.proj.bias")
        self.t0_w, self.t0_b = w("t_embedder.mlp.0"), f32("t_embedder.mlp.0.bias")
        self.t2_w, self.t2_b = w("t_embedder.mlp.2"), f32("t_embedder.mlp.2.bias")
        self.core_img_w, self.core_img_b = w("modulation_cores.adaln_img"), f32("modulation_cores.adaln_img.bias")
        self.core_txt_w, self.core_txt_b = w("modulation_cores.adaln_txt"), f32("modulation_cores.adaln_txt.bias")

        img_bias, txt_bias = [], []
        self.blocks = []
        for i in range(cfg.depth):
            b = f"blocks.{i}"
            if cfg.block_kind(i) == "mmdit":
                blk = {"kind": "mmdit", "img_mod": len(img_bias), "txt_mod": len(txt_bias)}
                img_bias.append(f32(f"{b}.adaln_img.bias"))
                txt_bias.append(f32(f"{b}.adaln_txt.bias"))
                for st in ("x", "y"):
                    blk[f"qkvg_{st}"] = cat_rows(f"{b}.attn.q_proj_{st}", f"{b}.attn.k_proj_{st}",
                                                 f"{b}.attn.v_proj_{st}", f"{b}.attn_gate_{st}")
                    blk[f"proj_{st}_w"], blk[f"proj_{st}_b"] = w(f"{b}.attn.proj_{st}"), f32(f"{b}.attn.proj_{st}.bias")
                    blk[f"w13_{st}"], blk[f"w2_{st}"] = swiglu(f"{b}.mlp_{st}")
                    for nm in (f"norm_{st}1", f"norm_{st}2", f"attn_post_norm_{st}", f"mlp_post_norm_{st}"):
                        blk[nm] = f32(f"{b}.{nm}.weight")
                    for nm in (f"q_norm_{st}", f"k_norm_{st}"):
                        blk[nm] = f32(f"{b}.attn.{nm}.weight")
            else:
                blk = {"kind": "single", "img_mod": len(img_bias)}
                img_bias.append(f32(f"{b}.adaln.bias"))
                blk["qkvg"] = cat_rows(f"{b}.q_proj", f"{b}.k_proj", f"{b}.v_proj", f"{b}.attn_gate")
                blk["proj_w"], blk["proj_b"] = w(f"{b}.attn_proj"), f32(f"{b}.attn_proj.bias")
                blk["w13"], blk["w2"] = swiglu(f"{b}.mlp")
                for nm in ("norm1", "norm2", "attn_post_norm", "mlp_post_norm", "q_norm", "k_norm"):
                    blk[nm] = f32(f"{b}.{nm}.weight")
            self.blocks.append(blk)
        self.img_bias = torch.stack(img_bias).contiguous()
        self.txt_bias = torch.stack(txt_bias).contiguous()

        def fold(outer: str, inner: str) -> tuple[torch.Tensor, torch.Tensor]:
            """``outer(inner(x))`` of two Linears as one: W = W_o W_i, b = W_o b_i + b_o, from the
            BF16 weights the GEMMs would use, in FP32, W rounded to BF16 once."""
            wo, wi = w(outer).float(), w(inner).float()
            weight = bf(wo @ wi)
            bias = (wo @ f32(f"{inner}.bias") + f32(f"{outer}.bias")).contiguous()
            return weight, bias

        self.pix_w, self.pix_b = f32("pixel_embedder.proj.weight"), f32("pixel_embedder.proj.bias")
        self.pixel_blocks = []
        for j in range(cfg.pixel.depth):
            b = f"pixel_blocks.{j}"
            self.pixel_blocks.append({
                "norm1": f32(f"{b}.norm1.weight"), "norm2": f32(f"{b}.norm2.weight"),
                "adaln_w": w(f"{b}.adaln"), "adaln_b": f32(f"{b}.adaln.bias"),
                "compress_w": w(f"{b}.compress"), "compress_b": f32(f"{b}.compress.bias"),
                "qkv_w": w(f"{b}.attn.qkv"),
                "q_norm": f32(f"{b}.attn.q_norm.weight"), "k_norm": f32(f"{b}.attn.k_norm.weight"),
                # the attention's output projection and the expand Linear back to pixels, with nothing
                # between them (src/iris_metal/model.py:340-341), folded into one GEMM
                **dict(zip(("proj_expand_w", "proj_expand_b"), fold(f"{b}.expand", f"{b}.attn.proj"))),
                "fc1_w": f32(f"{b}.mlp.fc1.weight"), "fc1_b": f32(f"{b}.mlp.fc1.bias"),
                "fc2_w": f32(f"{b}.mlp.fc2.weight"), "fc2_b": f32(f"{b}.mlp.fc2.bias"),
            })
        self.final_norm = f32("final_layer.norm.weight")
        self.final_w, self.final_b = f32("final_layer.linear.weight"), f32("final_layer.linear.bias")
        self.out_channels = self.final_w.shape[0]
        self.t_freqs = tables.timestep_freqs(256, cfg.timestep_max_period, self.device)
        if "t_embedder.mlp.0.weight" in sd and sd["t_embedder.mlp.0.weight"].shape[1] != 256:
            raise ValueError("HipIris expects 256 timestep frequencies")
        self._prepare_text(sd, f32, w, swiglu)

    def _prepare_text(self, sd, f32, w, swiglu) -> None:
        """Weights of the masked text adapter (src/iris3b/nn/embeddings.py:110-266): the
        layer-wise blocks (``lap_blocks2`` only) with their MLP hidden width zero-padded to a
        multiple of 64 (padded columns are silu(0) = 0 and meet zero weights), the pool, the
        refiner, and the position table."""
        cfg, dev = self.cfg, self.device
        self.text_layer_blocks = []
        if cfg.text_adapter == "lap_blocks2":
            hidden = int(cfg.text_dim * cfg.text_lap_mlp_ratio)
            self.text_lap_hidden = _round_up(hidden, 64)
            for i in range(2):
                b = f"y_embedder.layer_blocks.{i}"
                m0 = sd[f"{b}.mlp.0.weight"].detach().float()
                m0b = sd[f"{b}.mlp.0.bias"].detach().float()
                m2 = sd[f"{b}.mlp.2.weight"].detach().float()
                pad = self.text_lap_hidden - hidden
                self.text_layer_blocks.append({
                    "norm1": f32(f"{b}.norm1.weight"), "norm2": f32(f"{b}.norm2.weight"),
                    "qkv_w": w(f"{b}.attn.qkv"),
                    "qkv_b": f32(f"{b}.attn.qkv.bias") if f"{b}.attn.qkv.bias" in sd else None,
                    "proj_w": w(f"{b}.attn.proj"), "proj_b": f32(f"{b}.attn.proj.bias"),
                    "mlp0_w": torch.nn.functional.pad(m0, (0, 0, 0, pad)).to(dev, torch.bfloat16).contiguous(),
                    "mlp0_b": torch.nn.functional.pad(m0b, (0, pad)).to(dev).contiguous(),
                    "mlp2_w": torch.nn.functional.pad(m2, (0, pad)).to(dev, torch.bfloat16).contiguous(),
                    "mlp2_b": f32(f"{b}.mlp.2.bias"),
                })
            self.text_pool_w = f32("y_embedder.layer_pool.weight")
            self.text_pool_b = f32("y_embedder.layer_pool.bias")
            refiner = "y_embedder.refiner"
        else:
            refiner = "y_embedder"
        self.text_one = torch.ones(1, device=dev)  # a one-layer pool: the FP32 -> BF16 cast of blocks2 input
        self.text_proj_w, self.text_proj_b = w(f"{refiner}.proj"), f32(f"{refiner}.proj.bias")
        self.text_blocks = []
        for i in range(2):
            b = f"{refiner}.blocks.{i}"
            blk = {"norm1": f32(f"{b}.norm1.weight"), "norm2": f32(f"{b}.norm2.weight"),
                   "qkv_w": w(f"{b}.attn.qkv"),
                   "qkv_b": f32(f"{b}.attn.qkv.bias") if f"{b}.attn.qkv.bias" in sd else None,
                   "q_norm": f32(f"{b}.attn.q_norm.weight"), "k_norm": f32(f"{b}.attn.k_norm.weight"),
                   "proj_w": w(f"{b}.attn.proj"), "proj_b": f32(f"{b}.attn.proj.bias")}
            blk["w13"], blk["w2"] = swiglu(f"{b}.mlp")
            self.text_blocks.append(blk)
        self.text_norm = f32(f"{refiner}.norm.weight")
        self.text_pos = f32("y_pos_embedding").reshape(-1, cfg.hidden_size)
        self._text_ws: dict | None = None

    # -- per-shape state ----------------------------------------------------------------
    def _workspace(self, shape: _Shape) -> dict:
        if self._ws is not None and self._ws_shape == shape:
            return self._ws
        self._ws = None  # (with the buffers it points into goes the recorded graph)
        cfg, dev = self.cfg, self.device
        B, T = shape.batch, shape.n_text
        p = cfg.patch_size
        hp, wp = shape.height // p, shape.width // p
        Lp = hp * wp
        N = T + Lp
        D = cfg.hidden_size
        H, Hkv = cfg.num_heads, cfg.kv_heads
        n_pad = _round_up(N, 64)
        l_pad = _round_up(Lp, 64)
        pp = p * p
        px = cfg.pixel
        qkvg_w = (H + 2 * Hkv) * HEAD_DIM + D
        bf16, f32 = torch.bfloat16, torch.float32

        def e(*s, dtype=bf16):
            return torch.empty(*s, device=dev, dtype=dtype)

        n_img, n_txt = self.img_bias.shape[0], self.txt_bias.shape[0]
        ws = {
            "L": Lp, "N": N, "n_pad": n_pad, "l_pad": l_pad, "grid": (hp, wp),
            "patches": torch.zeros(B * Lp, self.patch_k, device=dev, dtype=bf16),
            "X": e(B * Lp, D, dtype=f32), "Y": e(B * T, D, dtype=f32), "tok": e(B * N, D, dtype=f32),
            "tfeat": e(B, 256, dtype=f32), "th": e(B, D, dtype=f32), "temb": e(B, D, dtype=f32),
            "mods_img": e(n_img, B, 6 * D, dtype=f32), "mods_txt": e(n_txt, B, 6 * D, dtype=f32),
            "h_tok": e(B * N, D), "qkvg": e(B * N, qkvg_w), "attn": e(B * N, D), "branch": e(B * N, D),
            "hh": e(B * N, self.hidden_pad),
            "q": e(B, H, n_pad, HEAD_DIM), "k": e(B, Hkv, n_pad, HEAD_DIM),
            "vt": torch.zeros(B, Hkv, HEAD_DIM, n_pad, device=dev, dtype=bf16),
            "scond": e(B * Lp, D),
            "pixels": e(B * Lp, pp, K.PIXEL_WIDTH, dtype=f32), "hpix": e(B * Lp, pp, K.PIXEL_WIDTH),
            "mods_pix": e(B * Lp, pp, 4 * K.PIXEL_WIDTH),
            "cp": e(B * Lp, px.attn_hidden_size), "pq": e(B * Lp, 3 * px.attn_hidden_size),
            "pa": e(B * Lp, px.attn_hidden_size),
            "ex": e(B * Lp, pp * K.PIXEL_WIDTH),
            "qp": e(B, px.num_heads, l_pad, HEAD_DIM), "kp": e(B, px.num_heads, l_pad, HEAD_DIM),
            "vtp": torch.zeros(B, px.num_heads, HEAD_DIM, l_pad, device=dev, dtype=bf16),
        }
        # one batch item: the dual-stream residuals are the single-stream buffer's text and image
        # rows, so joining the streams (and the last block's image rows) moves nothing
        ws["joined_in_place"] = B == 1
        if B == 1:
            ws["Y"], ws["X"] = ws["tok"][:T], ws["tok"][T:]
        # text-stream scratch of the dual blocks lives after the image rows of the shared buffers
        key = ((hp, wp), T)
        if key not in self._tables:
            img = tables.rope_2d_angles(HEAD_DIM, hp, wp, cfg.rope_theta, cfg.rope_scale, cfg.rope_aspect,
                                        cfg.rope_frame_pairs, cfg.rope_frame_theta)
            pix = tables.rope_2d_angles(px.attn_hidden_size // px.num_heads, hp, wp, cfg.rope_theta,
                                        cfg.rope_scale, cfg.rope_aspect)
            txt = tables.rope_1d_angles(HEAD_DIM, T, cfg.text_rope_theta)
            self._tables = {key: {
                "rope": tables.cos_sin(txt, img, device=dev),
                "rope_pix": tables.cos_sin(pix, device=dev),
                "pos": tables.sincos_halves(K.PIXEL_WIDTH, shape.height, shape.width, dev),
            }}
        ws.update(self._tables[key])
        self._ws, self._ws_shape = ws, shape
        return ws

    # -- forward ------------------------------------------------------------------------
    @torch.no_grad()
    def __call__(self, x: torch.Tensor, t: torch.Tensor, text: torch.Tensor, out: torch.Tensor | None = None):
        """``x``: ``[B, 3, H, W]``; ``t``: model time ``[B]``; ``text``: ``[B, T, D]``; returns FP32 ``v``."""
        cfg = self.cfg
        p = cfg.patch_size
        batch, channels, height, width = x.shape
        if height % p or width % p:
            raise ValueError(f"input {height}x{width} is not divisible by patch_size {p}")
        if channels != self.in_channels:
            raise ValueError(f"expected {self.in_channels} input channels, got {channels}")
        if text.dim() != 3 or text.shape[0] != batch or text.shape[2] != cfg.hidden_size:
            raise ValueError(f"text must be [B, T, {cfg.hidden_size}] prepared tokens, got {tuple(text.shape)}")
        if t.numel() != batch:
            raise ValueError(f"t must hold one model time per sample, got {tuple(t.shape)}")
        dev = self.device
        shape = _Shape(batch, height, width, text.shape[1])
        ws = self._workspace(shape)
        if out is None:
            out = torch.empty(batch, self.out_channels, height, width, device=dev, dtype=torch.float32)
        elif (out.shape != (batch, self.out_channels, height, width) or out.dtype != torch.float32
              or not out.is_contiguous() or out.device != dev):
            raise ValueError(f"out must be a contiguous FP32 {(batch, self.out_channels, height, width)} tensor on {dev}")
        if not self.graphs:
            x = x.to(dev, torch.float32).contiguous()
            t = t.reshape(batch).to(dev, torch.float32).contiguous()
            text = text.to(dev, torch.float32).contiguous()
            self._forward(ws, x, t, text, out)
            return out
        if "graph" not in ws:
            ws["x_in"] = torch.empty(batch, self.in_channels, height, width, device=dev, dtype=torch.float32)
            ws["t_in"] = torch.empty(batch, device=dev, dtype=torch.float32)
            ws["text_in"] = torch.empty(text.shape, device=dev, dtype=torch.float32)
            ws["out_ws"] = torch.empty(batch, self.out_channels, height, width, device=dev, dtype=torch.float32)
            ws["graph"] = None
        args = (ws, ws["x_in"], ws["t_in"], ws["text_in"], ws["out_ws"])
        ws["x_in"].copy_(x)
        ws["t_in"].copy_(t.reshape(batch))
        ws["text_in"].copy_(text)
        if ws["graph"] is None:
            self._forward(*args)  # this call's result, and every lazy set-up before recording
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._forward(*args)
            ws["graph"] = graph
        else:
            ws["graph"].replay()
        out.copy_(ws["out_ws"])
        return out

    def _forward(self, ws: dict, x: torch.Tensor, t: torch.Tensor, text: torch.Tensor, out: torch.Tensor) -> None:
        cfg, eps = self.cfg, self.eps
        B = x.shape[0]
        T, Lp, N = text.shape[1], ws["L"], ws["N"]
        D = cfg.hidden_size
        p = cfg.patch_size
        pb0 = self.pixel_blocks[0]

        # patch tokens, the pixel stream and its first norm, from one read of x
        K.patchify_embed(x, p, self.pix_w, self.pix_b, ws["pos"][0], ws["pos"][1], pb0["norm1"], eps,
                         ws["patches"], ws["pixels"], ws["hpix"])
        K.linear(ws["patches"], self.s_w, self.s_b, out=ws["X"])

        self._conditioning(ws, t)

        Y = ws["Y"]
        K.copy_rows(text.reshape(B * T, D), Y, B, T, 0, T, 0, T)
        joined = False
        h_ready = False  # the next block's input norms were produced by the previous block
        for i, blk in enumerate(self.blocks):
            nxt = self.blocks[i + 1] if i + 1 < len(self.blocks) else None
            if blk["kind"] == "mmdit":
                fuse = nxt is not None and nxt["kind"] == "mmdit"
                self._dual_block(ws, blk, B, T, Lp, N, h_ready, nxt if fuse else None)
                h_ready = fuse
                continue
            if not joined:
                if not ws["joined_in_place"]:
                    K.copy_rows(Y, ws["tok"], B, T, 0, T, 0, N)
                    K.copy_rows(ws["X"], ws["tok"], B, Lp, 0, Lp, T, N)
                joined = True
            self._single_block(ws, blk, B, T, Lp, N, i == cfg.depth - 1, h_ready, nxt)
            h_ready = nxt is not None

        # pixel stage
        K.silu_add_rows(ws["X"], ws["temb"], Lp, ws["scond"])
        for j, pblk in enumerate(self.pixel_blocks):
            next_norm = self.pixel_blocks[j + 1]["norm1"] if j + 1 < len(self.pixel_blocks) else self.final_norm
            self._pixel_block(ws, pblk, B, Lp, next_norm)
        K.unpatchify_head(ws["hpix"], self.final_w, self.final_b, out, p)

    def _conditioning(self, ws: dict, t: torch.Tensor) -> None:
        """Timestep embedding, then both shared adaLN cores with every block's bias folded in."""
        K.timestep_features(t, self.t_freqs, ws["tfeat"])
        K.gemv(self.t0_w, ws["tfeat"], self.t0_b, ws["th"], out_silu=True)
        K.gemv(self.t2_w, ws["th"], self.t2_b, ws["temb"])
        K.gemv(self.core_img_w, ws["temb"], self.core_img_b, ws["mods_img"], extra_bias=self.img_bias, in_silu=True)
        K.gemv(self.core_txt_w, ws["temb"], self.core_txt_b, ws["mods_txt"], extra_bias=self.txt_bias, in_silu=True)

    @torch.no_grad()
    def block_forward(self, index: int, x: torch.Tensor, text: torch.Tensor, t: torch.Tensor,
                      grid: tuple[int, int]) -> tuple[torch.Tensor, torch.Tensor]:
        """One trunk block on its own: ``x`` image tokens ``[B, L, D]`` over a ``grid`` of patches
        (``L = grid[0] * grid[1]``), ``text`` tokens ``[B, T, D]``, model time ``t`` ``[B]``.
        Returns the block's ``(x, text)`` as the reference block's ``forward`` does
        (src/iris3b/models/blocks/mmdit.py:84-128, single_stream.py:69-88): FP32, the text
        returned unchanged by a block without a text output. The modulation comes from ``t``
        through the timestep embedder and the shared adaLN cores, as in the full forward."""
        cfg = self.cfg
        if not 0 <= index < cfg.depth:
            raise ValueError(f"block index must be in [0, {cfg.depth}), got {index}")
        B, Lp, D = x.shape
        T = text.shape[1]
        if grid[0] * grid[1] != Lp or text.shape[0] != B or text.shape[2] != D or D != cfg.hidden_size:
            raise ValueError(f"x must be [B, {grid[0] * grid[1]}, {cfg.hidden_size}] and text [B, T, "
                             f"{cfg.hidden_size}], got {tuple(x.shape)} and {tuple(text.shape)}")
        p = cfg.patch_size
        ws = self._workspace(_Shape(B, grid[0] * p, grid[1] * p, T))
        dev = self.device
        x = x.to(dev, torch.float32).contiguous()
        text = text.to(dev, torch.float32).contiguous()
        self._conditioning(ws, t.reshape(B).to(dev, torch.float32).contiguous())
        N = T + Lp
        if cfg.block_kind(index) == "mmdit":
            ws["X"].copy_(x.reshape(B * Lp, D))
            ws["Y"].copy_(text.reshape(B * T, D))
        else:
            K.copy_rows(text.reshape(B * T, D), ws["tok"], B, T, 0, T, 0, N)
            K.copy_rows(x.reshape(B * Lp, D), ws["tok"], B, Lp, 0, Lp, T, N)
        ws["block"] = (index, B, T, Lp, N)
        self.run_block()
        if cfg.block_kind(index) == "mmdit":
            return ws["X"].view(B, Lp, D).clone(), ws["Y"].view(B, T, D).clone()
        if not cfg.text_out(index):
            return ws["X"].view(B, Lp, D).clone(), text
        tok = ws["tok"].view(B, N, D)
        return tok[:, T:].clone(), tok[:, :T].clone()

    def run_block(self) -> None:
        """Run the block of the last ``block_forward`` call again, in place on the residual it
        left in the engine's workspace (for timing the block's kernels alone)."""
        ws = self._ws
        if ws is None or "block" not in ws:
            raise RuntimeError("run_block follows a block_forward call")
        index, B, T, Lp, N = ws["block"]
        blk = self.blocks[index]
        if blk["kind"] == "mmdit":
            self._dual_block(ws, blk, B, T, Lp, N, False, None)
        else:
            self._single_block(ws, blk, B, T, Lp, N, not self.cfg.text_out(index), False, None)

    def _mods(self, ws: dict, table: str, index: int, chunk: int) -> torch.Tensor:
        D = self.cfg.hidden_size
        return ws[table][index][:, chunk * D:(chunk + 1) * D].unsqueeze(1)

    def _dual_block(self, ws: dict, blk: dict, B: int, T: int, Lp: int, N: int, h_ready: bool,
                    nxt: dict | None) -> None:
        """One dual-stream block on the image ``X`` and text ``Y`` residuals. With ``h_ready`` the
        input norms are already in the ``h`` rows (fused into the previous block's last residual);
        with ``nxt`` (a dual block) this block's last residual also produces ``nxt``'s input norms."""
        cfg, eps = self.cfg, self.eps
        D, H, Hkv = cfg.hidden_size, cfg.num_heads, cfg.kv_heads
        X, Y = ws["X"].view(B, Lp, D), ws["Y"].view(B, T, D)
        xm = [self._mods(ws, "mods_img", blk["img_mod"], c) for c in range(6)]
        ym = [self._mods(ws, "mods_txt", blk["txt_mod"], c) for c in range(6)]
        qkvg_w = ws["qkvg"].shape[1]
        rows_x, rows_y = B * Lp, B * T
        hx, hy = ws["h_tok"][:rows_x], ws["h_tok"][rows_x:rows_x + rows_y]
        px, py = ws["qkvg"][:rows_x], ws["qkvg"][rows_x:rows_x + rows_y]
        ax, ay = ws["attn"][:rows_x], ws["attn"][rows_x:rows_x + rows_y]
        bx, by = ws["branch"][:rows_x], ws["branch"][rows_x:rows_x + rows_y]
        hhx, hhy = ws["hh"][:rows_x], ws["hh"][rows_x:rows_x + rows_y]
        bf16 = torch.bfloat16

        if not h_ready:
            K.rms_norm_modulate(X, blk["norm_x1"], xm[0], xm[1], eps, bf16, out=hx.view(B, Lp, D))
            K.rms_norm_modulate(Y, blk["norm_y1"], ym[0], ym[1], eps, bf16, out=hy.view(B, T, D))
        # q | k | v | gate in one launch, the Q / K norm + rotary in the store of the q | k | v
        # columns (text rows at positions 0.., image rows after them), the V heads transposed
        # there too or from its output, the gate columns a plain product beside them
        rope_c, rope_s = ws["rope"]
        q, k, vt = ws["q"], ws["k"], ws["vt"]
        gate_col = (H + 2 * Hkv) * HEAD_DIM
        fuse_vt = Lp % 256 == 0 and T % 256 == 0  # whole 256-row tiles per item (and T % 16 == 0)
        K.linear_qk_rope([hx, hy], [blk["qkvg_x"], blk["qkvg_y"]], [px, py], [blk["q_norm_x"], blk["q_norm_y"]],
                         [blk["k_norm_x"], blk["k_norm_y"]], rope_c, rope_s, eps, H, Hkv, q, k, [Lp, T], [T, 0],
                         vt=vt if fuse_vt else None)
        if not fuse_vt:
            for proj, rows, off in ((py, T, 0), (px, Lp, T)):
                K.v_heads_t(proj.view(B, rows, qkvg_w), Hkv, vt, (H + Hkv) * HEAD_DIM, off)
        K.flash_attention(q, k, vt, N, ay, ax, n_split=T, gate0=py[:, gate_col:], gate1=px[:, gate_col:])
        K.linear_grouped([ax, ay], [blk["proj_x_w"], blk["proj_y_w"]], [blk["proj_x_b"], blk["proj_y_b"]], [bx, by])
        K.gated_residual_grouped_([X, Y], [bx.view(B, Lp, D), by.view(B, T, D)],
                                  [blk["attn_post_norm_x"], blk["attn_post_norm_y"]], [xm[2], ym[2]], eps,
                                  [blk["norm_x2"], blk["norm_y2"]], [xm[3], ym[3]], [xm[4], ym[4]],
                                  [hx.view(B, Lp, D), hy.view(B, T, D)])
        K.linear_grouped([hx, hy], [blk["w13_x"], blk["w13_y"]], None, [hhx, hhy], swiglu=True)
        K.linear_grouped([hhx, hhy], [blk["w2_x"], blk["w2_y"]], None, [bx, by])
        if nxt is None:
            K.gated_residual_grouped_([X, Y], [bx.view(B, Lp, D), by.view(B, T, D)],
                                      [blk["mlp_post_norm_x"], blk["mlp_post_norm_y"]], [xm[5], ym[5]], eps)
        else:
            nx = [self._mods(ws, "mods_img", nxt["img_mod"], c) for c in range(2)]
            ny = [self._mods(ws, "mods_txt", nxt["txt_mod"], c) for c in range(2)]
            K.gated_residual_grouped_([X, Y], [bx.view(B, Lp, D), by.view(B, T, D)],
                                      [blk["mlp_post_norm_x"], blk["mlp_post_norm_y"]], [xm[5], ym[5]], eps,
                                      [nxt["norm_x1"], nxt["norm_y1"]], [nx[0], ny[0]], [nx[1], ny[1]],
                                      [hx.view(B, Lp, D), hy.view(B, T, D)])

    def _single_block(self, ws: dict, blk: dict, B: int, T: int, Lp: int, N: int, last: bool, h_ready: bool,
                      nxt: dict | None) -> None:
        """One single-stream block on ``tok`` (the last one continues on the image rows only).
        ``h_ready`` / ``nxt``: as for ``_dual_block``, with ``nxt`` a single-stream block."""
        cfg, eps = self.cfg, self.eps
        D, H, Hkv = cfg.hidden_size, cfg.num_heads, cfg.kv_heads
        tok = ws["tok"]
        m = [self._mods(ws, "mods_img", blk["img_mod"], c) for c in range(6)]
        rows = B * N
        h, proj = ws["h_tok"][:rows], ws["qkvg"][:rows]
        qkvg_w = proj.shape[1]
        if not h_ready:
            K.rms_norm_modulate(tok.view(B, N, D), blk["norm1"], m[0], m[1], eps, torch.bfloat16, out=h.view(B, N, D))
        rope_c, rope_s = ws["rope"]
        q, k, vt = ws["q"], ws["k"], ws["vt"]
        gate_col = (H + 2 * Hkv) * HEAD_DIM  # as in _dual_block
        fuse_vt = N % 256 == 0
        K.linear_qk_rope([h], [blk["qkvg"]], [proj], [blk["q_norm"]], [blk["k_norm"]],
                         rope_c, rope_s, eps, H, Hkv, q, k, [N], [0], vt=vt if fuse_vt else None)
        if not fuse_vt:
            K.v_heads_t(proj.view(B, N, qkvg_w), Hkv, vt, (H + Hkv) * HEAD_DIM)
        gate = proj[:, gate_col:]
        if not last:
            R, M, per_batch = tok, rows, N
            attn = ws["attn"][:rows]
            K.flash_attention(q, k, vt, N, None, attn, n_split=0, gate1=gate)
        else:
            # the text rows still feed attention but no output depends on them (model.py:307-308)
            R, M, per_batch = ws["X"], B * Lp, Lp
            if not ws["joined_in_place"]:
                K.copy_rows(tok, R, B, Lp, T, N, 0, Lp)
            attn = ws["attn"][:M]
            K.flash_attention(q, k, vt, N, None, attn, n_split=T, gate1=gate[T:],
                              out_batch_rows=(T, Lp), gate_batch_rows=(T, N))
        branch, hh = ws["branch"][:M], ws["hh"][:M]
        h2 = ws["h_tok"][:M]
        Rv = R.view(B, per_batch, D)
        K.linear(attn, blk["proj_w"], blk["proj_b"], out=branch)
        K.gated_residual_norm_modulate_(Rv, branch.view(B, per_batch, D), blk["attn_post_norm"], m[2], eps,
                                        blk["norm2"], m[3], m[4], h2.view(B, per_batch, D))
        K.linear(h2, blk["w13"], out=hh, swiglu=True)
        K.linear(hh, blk["w2"], out=branch)
        if nxt is None:
            K.gated_residual_rms_norm_(Rv, branch.view(B, per_batch, D), blk["mlp_post_norm"], m[5], eps)
        else:
            n1 = [self._mods(ws, "mods_img", nxt["img_mod"], c) for c in range(2)]
            K.gated_residual_norm_modulate_(Rv, branch.view(B, per_batch, D), blk["mlp_post_norm"], m[5], eps,
                                            nxt["norm1"], n1[0], n1[1], h.view(B, N, D))

    def _pixel_block(self, ws: dict, blk: dict, B: int, Lp: int, next_norm: torch.Tensor) -> None:
        cfg, eps = self.cfg, self.eps
        px = cfg.pixel
        heads = px.num_heads
        width = px.attn_hidden_size
        K.linear(ws["scond"], blk["adaln_w"], blk["adaln_b"], out=ws["mods_pix"].view(B * Lp, -1))
        K.linear(ws["hpix"].view(B * Lp, -1), blk["compress_w"], blk["compress_b"], out=ws["cp"])
        K.linear(ws["cp"], blk["qkv_w"], out=ws["pq"])
        rope_c, rope_s = ws["rope_pix"]
        pv = ws["pq"].view(B, Lp, 3 * width)
        K.qkv_prepare(pv, blk["q_norm"], blk["k_norm"], rope_c, rope_s, eps, heads, heads, ws["qp"], ws["kp"],
                      ws["vtp"], 0, width, 2 * width)
        K.flash_attention(ws["qp"], ws["kp"], ws["vtp"], Lp, None, ws["pa"], n_split=0)
        K.linear(ws["pa"], blk["proj_expand_w"], blk["proj_expand_b"], out=ws["ex"])
        K.pixel_mlp_(ws["pixels"], ws["ex"].view_as(ws["hpix"]), ws["mods_pix"], blk["norm2"],
                     (blk["fc1_w"], blk["fc1_b"]), (blk["fc2_w"], blk["fc2_b"]), next_norm, eps,
                     next_input=ws["hpix"])

    def fold_reducer(self, weight: torch.Tensor, bias: torch.Tensor) -> None:
        """Fold a 1x1 convolution over the three output channels into the head (the depth
        reducer, src/iris3b/downstream/depth.py:37, 47): the engine then returns
        ``conv(v) = sum_c weight[0, c] v_c + bias`` as ``[B, 1, H, W]``, in one head pass."""
        w = weight.detach().cpu().to(torch.float32).reshape(1, -1)
        if w.shape[1] != self.out_channels or self.out_channels != 3 or bias.numel() != 1:
            raise ValueError("fold_reducer takes a [1, 3, 1, 1] convolution and its bias over the 3-channel head")
        b = bias.detach().cpu().to(torch.float32).reshape(1)
        head_w, head_b = self.final_w.cpu(), self.final_b.cpu()
        self.final_w = (w @ head_w).to(self.device).contiguous()
        self.final_b = (w @ head_b + b).to(self.device).contiguous()
        self.out_channels = 1
        self._ws = None  # the output buffers and any recorded graph change shape

    def as_dit(self) -> "HipIrisDiT":
        """The upstream ``IrisDiT`` call surface over this engine (the Turbo route)."""
        return HipIrisDiT(self)

    # -- conditioning -------------------------------------------------------------------
    def _text_workspace(self, batch: int, n: int) -> dict:
        if self._text_ws is not None and self._text_ws["key"] == (batch, n):
            return self._text_ws
        cfg, dev = self.cfg, self.device
        D, H, td = cfg.hidden_size, cfg.num_heads, cfg.text_dim
        n_pad = _round_up(n, 64)
        rows = batch * n
        bf16, f32 = torch.bfloat16, torch.float32

        def e(*s, dtype=bf16):
            return torch.empty(*s, device=dev, dtype=dtype)

        ws = {
            "key": (batch, n), "n_pad": n_pad,
            "Y": e(rows, D, dtype=f32), "hy": e(rows, D), "qkv": e(rows, 3 * D), "att": e(rows, D),
            "br": e(rows, D), "hh": e(rows, self.hidden_pad), "pooled": e(rows, td),
            "q": e(batch, H, n_pad, HEAD_DIM), "k": e(batch, H, n_pad, HEAD_DIM),
            # V^T columns of tokens >= n must stay zero: v_heads_t never writes them
            "vt": torch.zeros(batch, H, HEAD_DIM, n_pad, device=dev, dtype=bf16),
            "kmask": e(batch, n_pad, dtype=torch.uint8),
            # the refiner has no RoPE: the fused QK-norm kernel runs with the identity rotation
            "cos": torch.ones(n_pad, HEAD_DIM // 2, device=dev), "sin": torch.zeros(n_pad, HEAD_DIM // 2, device=dev),
        }
        if cfg.text_adapter == "lap_blocks2":
            L = cfg.text_lap_num_layers
            r = rows * L
            ws.update({"H": e(r, td, dtype=f32), "hn": e(r, td), "lqkv": e(r, 3 * td), "latt": e(r, td),
                       "lbr": e(r, td), "lmh": e(r, self.text_lap_hidden)})
        else:
            ws["flat"] = e(rows, td, dtype=f32)
        self._text_ws = ws
        return ws

    @torch.no_grad()
    def encode_text(self, states: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """Encoder states -> trunk text tokens ``[B, T, D]`` FP32 (src/iris_metal/model.py:133-145),
        ``T = min(len, text_len)``: the masked text adapter (src/iris3b/nn/embeddings.py:143-266)
        plus the position table (src/iris3b/models/dit.py:263-281), once per prompt.

        ``states``: ``[B, T_in, layers, text_dim]`` for ``lap_blocks2``, ``[B, T_in, text_dim]`` for
        ``blocks2``; ``mask``: the encoder's ``[B, T_in]`` attention mask (1 = real token).
        BF16 GEMM operands with FP32 accumulation, FP32 residuals, norms and softmax."""
        cfg, eps, dev = self.cfg, self.eps, self.device
        D, H, td = cfg.hidden_size, cfg.num_heads, cfg.text_dim
        if mask is None:
            raise ValueError(f"text_adapter={cfg.text_adapter!r} requires the encoder's [B, T] attention mask")
        n = min(states.shape[1], cfg.text_len)
        lap = cfg.text_adapter == "lap_blocks2"
        if mask.dim() != 2:
            raise ValueError(f"text mask must be [B, T], got {tuple(mask.shape)}")
        if lap:
            expected = (mask.shape[0], min(mask.shape[1], cfg.text_len), cfg.text_lap_num_layers, td)
            got = (states.shape[0], n, *states.shape[2:])
            if states.dim() != 4 or got != expected:
                raise ValueError(f"layerwise text states must be {expected}, got {got}")
            L, lheads = cfg.text_lap_num_layers, cfg.text_lap_num_heads
            if L > 16 or td % lheads or td // lheads > 128:
                raise ValueError("HipIris.encode_text: at most 16 encoder layers and heads of at most 128 values")
        else:
            got = (states.shape[0], n)
            if states.dim() != 3 or states.shape[2] != td or got != (mask.shape[0], min(mask.shape[1], cfg.text_len)):
                raise ValueError(f"text states must be [B, T, {td}] with a matching [B, T] mask, got "
                                 f"{tuple(states.shape)} and {tuple(mask.shape)}")
        B = states.shape[0]
        if B == 0 or n == 0:
            return torch.empty(B, n, D, device=dev, dtype=torch.float32)
        ws = self._text_workspace(B, n)
        states = states.to(dev, torch.float32).contiguous()
        mask = mask.to(dev)
        if mask.dtype not in K._MASK_KINDS:
            mask = mask.to(torch.float32)
        if mask.stride(1) != 1:
            mask = mask.contiguous()
        K.text_key_mask(mask, n, ws["kmask"])
        rows = B * n
        Y = ws["Y"]

        if lap:
            # per-token attention over encoder layers, two pre-norm blocks, then the learned pool
            H_, hn, qkv, att, br, mh = (ws[k] for k in ("H", "hn", "lqkv", "latt", "lbr", "lmh"))
            T_in = states.shape[1]
            K.copy_rows(states.view(B * T_in * L, td), H_, B, n * L, 0, T_in * L, 0, n * L)
            K.residual_rms_norm(H_, None, self.text_layer_blocks[0]["norm1"], eps, hn)
            for i, blk in enumerate(self.text_layer_blocks):
                K.linear(hn, blk["qkv_w"], blk["qkv_b"], out=qkv)
                K.layer_attention(qkv, att, L, lheads)
                K.linear(att, blk["proj_w"], blk["proj_b"], out=br)
                K.residual_rms_norm(H_, br, blk["norm2"], eps, hn)
                K.linear(hn, blk["mlp0_w"], blk["mlp0_b"], out=mh, silu=True)
                K.linear(mh, blk["mlp2_w"], blk["mlp2_b"], out=br)
                if i + 1 < len(self.text_layer_blocks):
                    K.residual_rms_norm(H_, br, self.text_layer_blocks[i + 1]["norm1"], eps, hn)
            K.layer_pool(H_, br, self.text_pool_w, self.text_pool_b, L, ws["pooled"])
        else:
            T_in = states.shape[1]
            K.copy_rows(states.view(B * T_in, td), ws["flat"], B, n, 0, T_in, 0, n)
            K.layer_pool(ws["flat"], None, self.text_one, None, 1, ws["pooled"])  # FP32 -> BF16

        # refiner: Linear, two masked pre-norm blocks, RMSNorm, + position table
        K.linear(ws["pooled"], self.text_proj_w, self.text_proj_b, out=Y)
        hy, qkv, att, br, hh = ws["hy"], ws["qkv"], ws["att"], ws["br"], ws["hh"]
        q, k, vt, cos, sin = ws["q"], ws["k"], ws["vt"], ws["cos"], ws["sin"]
        out = torch.empty(B, n, D, device=dev, dtype=torch.float32)
        K.residual_rms_norm(Y, None, self.text_blocks[0]["norm1"], eps, hy)
        for i, blk in enumerate(self.text_blocks):
            K.linear(hy, blk["qkv_w"], blk["qkv_b"], out=qkv)
            pv = qkv.view(B, n, 3 * D)
            K.qkv_prepare(pv, blk["q_norm"], blk["k_norm"], cos, sin, eps, H, H, q, k, vt, 0, D, 2 * D)
            K.flash_attention_masked(q, k, vt, n, ws["kmask"], att)
            K.linear(att, blk["proj_w"], blk["proj_b"], out=br)
            K.residual_rms_norm(Y, br, blk["norm2"], eps, hy)
            K.linear(hy, blk["w13"], out=hh, swiglu=True)
            K.linear(hh, blk["w2"], out=br)
            if i + 1 < len(self.text_blocks):
                K.residual_rms_norm(Y, br, self.text_blocks[i + 1]["norm1"], eps, hy)
            else:
                K.residual_rms_norm(Y, br, self.text_norm, eps, out.view(rows, D), add_rows=self.text_pos[:n])
        return out


class HipIrisDiT:
    """``model(x, t, y, y_mask=, prepared_text=, precompute_modulation=).x`` over a ``HipIris``:
    the upstream ``IrisDiT.forward`` surface the reference Turbo route calls
    (src/iris_metal/pipeline.py:387-407, src/iris3b/models/dit.py:283-315)."""

    def __init__(self, engine: HipIris):
        self.engine = engine
        self.cfg = engine.cfg

    def __call__(self, x, t, y=None, y_mask=None, prepared_text=None, precompute_modulation=True, capture=()):
        if capture:
            raise ValueError("HipIrisDiT does not return intermediate block features")
        text = prepared_text if prepared_text is not None else self.engine.encode_text(y, y_mask)
        from types import SimpleNamespace

        return SimpleNamespace(x=self.engine(x, t.reshape(-1), text))
