"""Per-shape constant tables of the forward, built once per (grid, text length) on the host
and kept on the device, as the reference engine does (src/iris_metal/model.py:147-174).

- rotary tables: FP32 ``cos``/``sin`` ``[N, 64]`` for the trunk in ``[text | image]`` order and
  ``[L, 64]`` for the pixel stage (src/iris3b/nn/rope.py:19-89);
- the pixel stage's fixed 2-D sincos position table, stored separably as ``[W, 8]`` (x half)
  and ``[H, 8]`` (y half) since each half depends on one coordinate
  (src/iris3b/nn/embeddings.py:269-288);
- the timestep frequency bank ``exp(-ln(P) k / n)`` (src/iris3b/nn/embeddings.py:41-45).
"""

from __future__ import annotations

import math

import torch


def rope_2d_angles(head_dim: int, height: int, width: int, theta: float, scale: float, aspect: str,
                   frame_pairs: int = 0, frame_theta: float = 10.0, frame_index: int = 0) -> torch.Tensor:
    """Complex ``[H*W, head_dim/2]`` table of src/iris3b/nn/rope.py:19-82 (x, y pairs interleaved)."""
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
    x_cis = torch.polar(torch.ones(width, freqs.numel()), torch.outer(xs, freqs))
    y_cis = torch.polar(torch.ones(height, freqs.numel()), torch.outer(ys, freqs))
    cis = torch.stack(
        [x_cis[None, :, :].expand(height, width, -1), y_cis[:, None, :].expand(height, width, -1)], dim=-1
    ).reshape(height * width, -1)
    if frame_pairs:
        slots = 2 * frame_pairs
        f_freqs = 1.0 / frame_theta ** (torch.arange(slots).float() / slots)
        f_cis = torch.polar(torch.ones(slots), float(frame_index) * f_freqs)
        cis = torch.cat([cis, f_cis[None, :].expand(height * width, -1)], dim=-1)
    return cis


def rope_1d_angles(head_dim: int, length: int, theta: float) -> torch.Tensor:
    """Complex ``[length, head_dim/2]`` table of src/iris3b/nn/rope.py:85-89."""
    freqs = 1.0 / theta ** (torch.arange(0, head_dim, 2)[: head_dim // 2].float() / head_dim)
    ang = torch.outer(torch.arange(length).float(), freqs)
    return torch.polar(torch.ones_like(ang), ang)


def cos_sin(*tables: torch.Tensor, device) -> tuple[torch.Tensor, torch.Tensor]:
    cis = torch.view_as_real(torch.cat(tables))
    return cis[..., 0].contiguous().to(device), cis[..., 1].contiguous().to(device)


def sincos_halves(dim: int, height: int, width: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """``([W, dim/2], [H, dim/2])`` FP32: ``[sin | cos]`` of the column / row coordinate,
    computed in FP64 then rounded, as src/iris3b/nn/embeddings.py:269-288."""
    half = dim // 2
    omega = torch.arange(half // 2, dtype=torch.float64) / (half / 2.0)
    omega = 1.0 / 10000.0**omega

    def one(n: int) -> torch.Tensor:
        out = torch.outer(torch.arange(n, dtype=torch.float32).double(), omega)
        return torch.cat([torch.sin(out), torch.cos(out)], dim=1).float().contiguous()

    return one(width).to(device), one(height).to(device)


def timestep_freqs(freq_dim: int, max_period: float, device) -> torch.Tensor:
    n = freq_dim // 2
    k = torch.arange(n, dtype=torch.float32)
    return torch.exp(-math.log(max_period) * k / n).to(device)
