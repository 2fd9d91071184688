"""Tensor-level wrappers of the HIP kernels, with the reference's names and argument checks.

The first five functions keep the call surface of the reference's fused Metal kernels
(src/iris_metal/kernels.py:334-584: ``qk_norm_rope``, ``rms_norm_modulate``,
``gated_residual_rms_norm_``, ``pixel_rms_norm``, ``pixel_mlp_``): same arguments, same
meaning, ``ValueError`` on a bad argument before anything is launched. Unlike the reference
they have no CPU branch: every call runs the HIP kernel and raises on a tensor that is not
on the GPU. The rest wrap the kernels that replace the reference's PyTorch ops (``F.linear``,
``F.scaled_dot_product_attention``, the patchify / unpatchify reshapes and the sampler
updates). Outputs are allocated by the wrapper unless passed in, as in the reference.
"""

from __future__ import annotations

import torch

from . import _lib as L

HEAD_DIM = 128
PIXEL_WIDTH, PIXEL_HIDDEN = 16, 64


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _require_fp32(**tensors: torch.Tensor) -> None:
    for name, tensor in tensors.items():
        _require(tensor.dtype == torch.float32 and tensor.is_contiguous(), f"{name} must be contiguous FP32")


def _on_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("the HIP kernels need GPU tensors (there is no CPU path)")


def _per_batch(vector: torch.Tensor, batch: int, width: int) -> tuple[torch.Tensor, int]:
    """``[B, 1, D]`` modulation slice -> FP32 rows read in place when 16-byte aligned, and their stride."""
    rows = vector.reshape(batch, width)
    if rows.dtype != torch.float32:
        rows = rows.float()
    if rows.stride(1) != 1 or rows.stride(0) % 4 or rows.storage_offset() % 4:
        rows = rows.contiguous()
    return rows, rows.stride(0) if batch > 1 else width


# ---------------------------------------------------------------------------------------
# the reference's fused kernels
# ---------------------------------------------------------------------------------------
def qk_norm_rope(
    x: torch.Tensor,
    weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
    heads: int,
    col_offset: int = 0,
    out: torch.Tensor | None = None,
    offset: int = 0,
    out_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Fused per-head RMSNorm + RoPE + ``[B, N, H, D] -> [B, H, N, D]`` layout
    (src/iris_metal/kernels.py:334-397). ``x``: contiguous ``[B, N, W]`` whose columns
    ``[col_offset, col_offset + heads*128)`` hold the heads; ``cos``/``sin``: FP32
    ``[N_out, 64]``; rows land at ``offset + token`` of ``out`` (``[B, heads, N_out, 128]``)."""
    _require(heads > 0 and col_offset >= 0 and offset >= 0, "heads must be positive and offsets nonnegative")
    batch, tokens, width = x.shape
    if out is None:
        out = x.new_empty(batch, heads, tokens, HEAD_DIM, dtype=out_dtype or x.dtype)
    _on_gpu(x, out, weight, cos, sin)
    _require(
        col_offset + heads * HEAD_DIM <= width and x.is_contiguous(),
        "qk_norm_rope needs a contiguous [B, N, W] input holding the heads",
    )
    _require(
        out.shape[:2] == (batch, heads) and out.shape[3] == HEAD_DIM and out.is_contiguous(),
        f"qk_norm_rope output must be a contiguous [{batch}, {heads}, N, {HEAD_DIM}] tensor",
    )
    _require(
        cos.shape == sin.shape == (cos.shape[0], HEAD_DIM // 2) and offset + tokens <= min(cos.shape[0], out.shape[2]),
        "qk_norm_rope rotary tables or output do not cover the written rows",
    )
    _require_fp32(weight=weight, cos=cos, sin=sin)
    _require(weight.numel() == HEAD_DIM, f"qk_norm_rope gain must have {HEAD_DIM} entries")
    L.call(
        "iris_qk_norm_rope", L.ptr(x), L.dtype_code(x.dtype), L.ptr(out), L.dtype_code(out.dtype), L.ptr(weight),
        L.ptr(cos), L.ptr(sin), cos.shape[0], batch, tokens, out.shape[2], heads, offset, width, col_offset,
        float(eps), L.stream(),
    )
    return out


def rms_norm_modulate(
    x: torch.Tensor,
    weight: torch.Tensor,
    shift: torch.Tensor,
    scale: torch.Tensor,
    eps: float,
    out_dtype: torch.dtype,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``(rms_norm(x) * weight * (1 + scale) + shift).to(out_dtype)`` for ``x``: ``[B, N, D]`` and
    per-sample ``shift``/``scale``: ``[B, 1, D]`` (src/iris_metal/kernels.py:413-452)."""
    batch, tokens, width = x.shape
    _on_gpu(x, weight, shift, scale)
    _require(width % 128 == 0 and x.is_contiguous(), "rms_norm_modulate needs a contiguous input, width % 128 == 0")
    _require_fp32(weight=weight)
    _require(weight.numel() == width, "rms_norm_modulate gain width mismatch")
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    _require(out.shape == x.shape and out.is_contiguous() and out.dtype == out_dtype, "rms_norm_modulate: bad out")
    shift, shift_stride = _per_batch(shift, batch, width)
    scale, scale_stride = _per_batch(scale, batch, width)
    if shift_stride != scale_stride:  # the kernel takes one stride
        shift, scale = shift.contiguous(), scale.contiguous()
        shift_stride = width
    L.call(
        "iris_rms_norm_modulate", L.ptr(x), L.dtype_code(x.dtype), L.ptr(out), L.dtype_code(out_dtype),
        L.ptr(weight), L.ptr(shift), L.ptr(scale), batch * tokens, tokens, width, shift_stride, float(eps),
        L.stream(),
    )
    return out


def gated_residual_rms_norm_(
    residual: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, eps: float
) -> torch.Tensor:
    """``residual += gate * rms_norm(branch) * weight`` in place; ``residual``: FP32 ``[B, N, D]``
    (src/iris_metal/kernels.py:455-480)."""
    batch, tokens, width = residual.shape
    _on_gpu(residual, branch, weight, gate)
    _require(width % 128 == 0 and branch.shape == residual.shape, "gated_residual_rms_norm_ shape mismatch")
    _require(branch.is_contiguous(), "gated_residual_rms_norm_ needs a contiguous branch")
    _require_fp32(residual=residual, weight=weight)
    _require(weight.numel() == width, "gated_residual_rms_norm_ gain width mismatch")
    gate, gate_stride = _per_batch(gate, batch, width)
    L.call(
        "iris_gated_residual_rms_norm", L.ptr(residual), L.ptr(branch), L.dtype_code(branch.dtype), L.ptr(weight),
        L.ptr(gate), batch * tokens, tokens, width, gate_stride, float(eps), L.stream(),
    )
    return residual


def gated_residual_norm_modulate_(
    residual: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, eps: float,
    next_weight: torch.Tensor, next_shift: torch.Tensor, next_scale: torch.Tensor, out: torch.Tensor,
) -> torch.Tensor:
    """``gated_residual_rms_norm_`` then ``rms_norm_modulate`` of the updated residual into ``out``,
    in one pass over the row (the residual is read and written once)."""
    batch, tokens, width = residual.shape
    _on_gpu(residual, branch, weight, gate, next_weight, next_shift, next_scale, out)
    _require(width % 128 == 0 and branch.shape == residual.shape, "gated_residual_rms_norm_ shape mismatch")
    _require(branch.is_contiguous() and out.is_contiguous() and out.shape == residual.shape,
             "gated_residual_norm_modulate_ needs contiguous branch and output")
    _require_fp32(residual=residual, weight=weight, next_weight=next_weight)
    _require(weight.numel() == next_weight.numel() == width, "gated_residual_norm_modulate_ gain width mismatch")
    gate, gate_stride = _per_batch(gate, batch, width)
    shift, shift_stride = _per_batch(next_shift, batch, width)
    scale, scale_stride = _per_batch(next_scale, batch, width)
    if shift_stride != scale_stride:
        shift, scale = shift.contiguous(), scale.contiguous()
        shift_stride = width
    L.call(
        "iris_gated_residual_norm_modulate", L.ptr(residual), L.ptr(branch), L.dtype_code(branch.dtype),
        L.ptr(weight), L.ptr(gate), batch * tokens, tokens, width, gate_stride, float(eps), L.ptr(next_weight),
        L.ptr(shift), L.ptr(scale), shift_stride, L.ptr(out), L.dtype_code(out.dtype), L.stream(),
    )
    return out


def gated_residual_grouped_(residuals, branches, weights, gates, eps: float, next_weights=None, next_shifts=None,
                            next_scales=None, outs=None) -> None:
    """``gated_residual_rms_norm_`` (``outs`` None) or ``gated_residual_norm_modulate_`` of two
    streams (the image and text rows of a dual-stream block) in one launch, each on its own
    tensors; same results as the two calls."""
    _require(len(residuals) == len(branches) == len(weights) == len(gates) == 2, "gated_residual_grouped_ takes two")
    nxt = outs is not None
    width = residuals[0].shape[-1]
    keep, rows, per_batch, strides, nstrides, shifts, scales = [], [], [], [], [], [], []
    for i in range(2):
        residual, branch = residuals[i], branches[i]
        batch, tokens, w = residual.shape
        _on_gpu(residual, branch, weights[i], gates[i])
        _require(w == width and w % 128 == 0 and branch.shape == residual.shape and branch.is_contiguous(),
                 "gated_residual_grouped_ shape mismatch")
        _require(branch.dtype == branches[0].dtype, "gated_residual_grouped_: branch dtypes differ")
        _require_fp32(residual=residual, weight=weights[i])
        _require(weights[i].numel() == width, "gated_residual_grouped_ gain width mismatch")
        gate, gate_stride = _per_batch(gates[i], batch, width)
        keep.append(gate)
        rows.append(batch * tokens)
        per_batch.append(tokens)
        strides.append(gate_stride)
        if nxt:
            _on_gpu(next_weights[i], next_shifts[i], next_scales[i], outs[i])
            _require(outs[i].is_contiguous() and outs[i].shape == residual.shape and outs[i].dtype == outs[0].dtype,
                     "gated_residual_grouped_: bad output")
            _require_fp32(next_weight=next_weights[i])
            shift, shift_stride = _per_batch(next_shifts[i], batch, width)
            scale, scale_stride = _per_batch(next_scales[i], batch, width)
            if shift_stride != scale_stride:
                shift, scale = shift.contiguous(), scale.contiguous()
                shift_stride = width
            shifts.append(shift)
            scales.append(scale)
            nstrides.append(shift_stride)
    P = L.pointer_array
    L.call(
        "iris_gated_residual_grouped", 2, P([L.ptr(r) for r in residuals]), P([L.ptr(b) for b in branches]),
        L.dtype_code(branches[0].dtype), P([L.ptr(w) for w in weights]), P([L.ptr(g) for g in keep]),
        L.long_array(rows), L.long_array(per_batch), width, L.long_array(strides), float(eps),
        P([L.ptr(w) for w in next_weights]) if nxt else None, P([L.ptr(x) for x in shifts]) if nxt else None,
        P([L.ptr(x) for x in scales]) if nxt else None, L.long_array(nstrides) if nxt else None,
        P([L.ptr(o) for o in outs]) if nxt else None, L.dtype_code(outs[0].dtype) if nxt else L.BF16, L.stream(),
    )


def pixel_rms_norm(pixels: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rms_norm(pixels) * weight`` over the 16 channels of each pixel, stored BF16
    (src/iris_metal/kernels.py:486-498)."""
    _on_gpu(pixels, weight)
    _require(pixels.shape[-1] == PIXEL_WIDTH and pixels.is_contiguous(), "pixel_rms_norm needs 16-wide pixels")
    _require_fp32(weight=weight)
    _require(weight.numel() == PIXEL_WIDTH, "pixel_rms_norm gain width mismatch")
    out = torch.empty(pixels.shape, device=pixels.device, dtype=torch.bfloat16)
    n_pixels = pixels.numel() // PIXEL_WIDTH
    L.call("iris_pixel_rms_norm", L.ptr(pixels), L.dtype_code(pixels.dtype), L.ptr(out), L.ptr(weight), n_pixels,
           float(eps), L.stream())
    return out


def _linear_params(layer) -> tuple[torch.Tensor, torch.Tensor]:
    weight, bias = (layer.weight, layer.bias) if hasattr(layer, "weight") else layer
    return weight.detach().float().contiguous(), bias.detach().float().contiguous()


def pixel_mlp_(
    pixels: torch.Tensor,
    branch: torch.Tensor,
    mods: torch.Tensor,
    norm_weight: torch.Tensor,
    fc1,
    fc2,
    next_norm_weight: torch.Tensor,
    eps: float,
    next_input: torch.Tensor | None = None,
) -> torch.Tensor:
    """Finish a post-modulated PiT block in place; return the next block's normed input
    (src/iris_metal/kernels.py:527-584). ``pixels``: FP32 or BF16 ``[..., 16]`` (updated in
    place); ``branch``: BF16 ``[..., 16]``; ``mods``: BF16 ``[..., 64]`` (scale1, shift1,
    scale2, shift2); ``fc1``/``fc2``: ``nn.Linear`` (or ``(weight, bias)``) of 16 -> 64 -> 16."""
    _on_gpu(pixels, branch, mods, norm_weight, next_norm_weight)
    w1, b1 = _linear_params(fc1)
    w2, b2 = _linear_params(fc2)
    _require(
        pixels.shape[-1] == PIXEL_WIDTH
        and branch.shape == pixels.shape
        and mods.shape == (*pixels.shape[:-1], 4 * PIXEL_WIDTH)
        and w1.shape == (PIXEL_HIDDEN, PIXEL_WIDTH)
        and w2.shape == (PIXEL_WIDTH, PIXEL_HIDDEN)
        and b1.shape == (PIXEL_HIDDEN,)
        and b2.shape == (PIXEL_WIDTH,),
        "pixel_mlp_ needs the released pixel-stage widths",
    )
    _require(
        all(t.is_contiguous() for t in (pixels, branch, mods))
        and branch.dtype == torch.bfloat16
        and mods.dtype == torch.bfloat16
        and pixels.dtype in (torch.float32, torch.bfloat16),
        "pixel_mlp_ needs contiguous BF16 branch/mods and FP32 or BF16 pixels",
    )
    _require_fp32(norm_weight=norm_weight, next_norm_weight=next_norm_weight)
    _require(norm_weight.numel() == next_norm_weight.numel() == PIXEL_WIDTH, "pixel_mlp_ gain width mismatch")
    if next_input is None:
        next_input = torch.empty(pixels.shape, device=pixels.device, dtype=torch.bfloat16)
    n_pixels = pixels.numel() // PIXEL_WIDTH
    dev = pixels.device
    w1, b1, w2, b2 = (t.to(dev) for t in (w1, b1, w2, b2))
    L.call(
        "iris_pixel_mlp", L.ptr(pixels), L.dtype_code(pixels.dtype), L.ptr(branch), L.ptr(mods), L.ptr(norm_weight),
        L.ptr(w1), L.ptr(b1), L.ptr(w2), L.ptr(b2), L.ptr(next_norm_weight), L.ptr(next_input), n_pixels,
        float(eps), L.stream(),
    )
    return next_input


# ---------------------------------------------------------------------------------------
# kernels replacing the reference's PyTorch ops
# ---------------------------------------------------------------------------------------
def vt_positions(n: int) -> torch.Tensor:
    """Token held by each of ``n`` positions of the V^T layout (quads 1 and 2 of every 16
    positions swapped); the map is its own inverse."""
    i = torch.arange(n)
    quad = (i >> 2) & 3
    swapped = torch.where(quad == 1, 2, torch.where(quad == 2, 1, quad))
    return (i & ~15) | (swapped << 2) | (i & 3)


def v_heads_t(x: torch.Tensor, heads: int, out: torch.Tensor, col_offset: int = 0, offset: int = 0) -> torch.Tensor:
    """Write the V heads at ``col_offset`` of a BF16 ``[B, N, W]`` projection into ``out``
    (``[B, heads, 128, N_pad]``) transposed, token ``offset + t`` at position
    ``vt_positions(N_pad)[offset + t]`` (the layout ``flash_attention`` reads)."""
    batch, tokens, width = x.shape
    _on_gpu(x, out)
    _require(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "v_heads_t works on BF16")
    _require(x.is_contiguous() and out.is_contiguous(), "v_heads_t needs contiguous tensors")
    _require(out.shape[:3] == (batch, heads, HEAD_DIM), f"v_heads_t output must be [{batch}, {heads}, 128, N]")
    L.call("iris_v_heads_t", L.ptr(x), L.ptr(out), batch, tokens, out.shape[3], heads, offset, width, col_offset,
           L.stream())
    return out


def qkv_prepare(
    x: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    eps: float,
    heads: int,
    kv_heads: int,
    q: torch.Tensor,
    k: torch.Tensor,
    vt: torch.Tensor,
    q_col: int,
    k_col: int,
    v_col: int,
    offset: int = 0,
) -> None:
    """``qk_norm_rope`` of the Q heads and of the K heads and ``v_heads_t`` of the V heads of one
    BF16 ``[B, N, W]`` projection in one launch (same results as the three calls); ``q``:
    ``[B, heads, N_out, 128]``, ``k``: ``[B, kv_heads, N_out, 128]``, ``vt``:
    ``[B, kv_heads, 128, N_pad]``, all BF16, rows / positions from ``offset``."""
    batch, tokens, width = x.shape
    _on_gpu(x, q, k, vt, q_weight, k_weight, cos, sin)
    _require(all(t.dtype == torch.bfloat16 for t in (x, q, k, vt)), "qkv_prepare works on BF16")
    _require(x.is_contiguous() and q.is_contiguous() and k.is_contiguous() and vt.is_contiguous(),
             "qkv_prepare needs contiguous tensors")
    _require(q.shape == (batch, heads, q.shape[2], HEAD_DIM) and k.shape == (batch, kv_heads, q.shape[2], HEAD_DIM),
             "qkv_prepare: q / k must be [B, heads, N, 128] buffers of equal length")
    _require(vt.shape[:3] == (batch, kv_heads, HEAD_DIM), f"qkv_prepare: vt must be [{batch}, {kv_heads}, 128, N]")
    _require(cos.shape == sin.shape == (cos.shape[0], HEAD_DIM // 2), "qkv_prepare: rotary tables must be [N, 64]")
    _require_fp32(q_weight=q_weight, k_weight=k_weight, cos=cos, sin=sin)
    _require(q_weight.numel() == HEAD_DIM and k_weight.numel() == HEAD_DIM, "qkv_prepare: gains have 128 entries")
    L.call(
        "iris_qkv_prepare", L.ptr(x), L.ptr(q), L.ptr(k), L.ptr(vt), L.ptr(q_weight), L.ptr(k_weight), L.ptr(cos),
        L.ptr(sin), cos.shape[0], batch, tokens, q.shape[2], vt.shape[3], heads, kv_heads, offset, width, q_col,
        k_col, v_col, float(eps), L.stream(),
    )


def linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
    swiglu: bool = False,
    silu: bool = False,
) -> torch.Tensor:
    """``F.linear(x, weight, bias)`` on the MFMA GEMM; BF16 operands, FP32 accumulation.

    ``x``: BF16 ``[..., K]`` with contiguous rows; ``weight``: BF16 ``[N, K]``; ``bias``: FP32
    ``[N]``. With ``swiglu`` the weight is a ``pack_swiglu`` pair and the result is
    ``silu(x w1^T) * (x w3^T)``, N/2 wide; with ``silu`` the result is ``silu(x w^T + bias)``.
    K must be a multiple of 64."""
    _require(not (swiglu and silu), "linear: choose one epilogue")
    _on_gpu(x, weight, bias, out)
    _require(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16, "linear takes BF16 operands")
    _require(x.stride(-1) == 1 and weight.is_contiguous(), "linear needs row-contiguous operands")
    k = x.shape[-1]
    n = weight.shape[0]
    _require(weight.shape[1] == k, f"linear: weight {tuple(weight.shape)} does not match input width {k}")
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    n_out = n // 2 if swiglu else n
    if out is None:
        out = torch.empty(*x.shape[:-1], n_out, device=x.device, dtype=out_dtype)
    _require(out.shape[-1] == n_out and out.stride(-1) == 1, "linear: bad output")
    if bias is not None:
        _require_fp32(bias=bias)
        _require(bias.numel() == n, "linear: bias width mismatch")
    out2 = out.reshape(-1, n_out)
    L.call(
        "iris_gemm_bf16", L.ptr(x2), L.ptr(weight), L.ptr(bias), L.ptr(out2), L.dtype_code(out.dtype), m, n, k,
        x2.stride(0), weight.stride(0), out2.stride(0),
        L.EPI_SILU_MUL if swiglu else (L.EPI_SILU if silu else L.EPI_NONE), L.stream(),
    )
    return out


def linear_grouped(xs, weights, biases, outs, swiglu: bool = False) -> None:
    """Two ``linear`` calls of equal weight shape (one per stream of a dual block) in one launch."""
    _require(len(xs) == len(weights) == len(outs) == 2, "linear_grouped takes two problems")
    k = xs[0].shape[-1]
    n = weights[0].shape[0]
    for x, w, o in zip(xs, weights, outs):
        _on_gpu(x, w, o)
        _require(w.shape == (n, k) and x.shape[-1] == k and x.stride(-1) == 1, "linear_grouped: shape mismatch")
        _require(x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16, "linear_grouped takes BF16 operands")
    x2 = [x.reshape(-1, k) for x in xs]
    o2 = [o.reshape(-1, o.shape[-1]) for o in outs]
    _require(x2[0].stride(0) == x2[1].stride(0) and o2[0].stride(0) == o2[1].stride(0), "linear_grouped: strides differ")
    _require(outs[0].dtype == outs[1].dtype, "linear_grouped: output dtypes differ")
    bias_ptrs = None if biases is None else L.pointer_array([L.ptr(b) for b in biases])
    L.call(
        "iris_gemm_bf16_grouped", 2, L.pointer_array([L.ptr(x) for x in x2]),
        L.pointer_array([L.ptr(w) for w in weights]), bias_ptrs, L.pointer_array([L.ptr(o) for o in o2]),
        L.int_array([x.shape[0] for x in x2]), L.dtype_code(outs[0].dtype), n, k, x2[0].stride(0),
        weights[0].stride(0), o2[0].stride(0), L.EPI_SILU_MUL if swiglu else L.EPI_NONE, L.stream(),
    )


def pack_swiglu(w1: torch.Tensor, w3: torch.Tensor, hidden_pad: int) -> torch.Tensor:
    """Interleave SwiGLU ``w1``/``w3`` (``[H, D]``) in 32-row groups, zero-padded to ``hidden_pad``
    rows each: rows ``64p..64p+31`` are ``w1[32p:32p+32]``, rows ``64p+32..`` are ``w3[32p:..]``."""
    hidden, dim = w1.shape
    _require(w3.shape == w1.shape and hidden_pad % 32 == 0 and hidden_pad >= hidden, "pack_swiglu: bad shapes")
    pad = torch.zeros(2, hidden_pad, dim, dtype=w1.dtype, device=w1.device)
    pad[0, :hidden] = w1
    pad[1, :hidden] = w3
    return pad.reshape(2, hidden_pad // 32, 32, dim).transpose(0, 1).reshape(2 * hidden_pad, dim).contiguous()


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    vt: torch.Tensor,
    n: int,
    out0: torch.Tensor | None,
    out1: torch.Tensor | None,
    n_split: int = 0,
    gate0: torch.Tensor | None = None,
    gate1: torch.Tensor | None = None,
    out_batch_rows: tuple[int, int] | None = None,
    gate_batch_rows: tuple[int, int] | None = None,
    scale: float | None = None,
) -> None:
    """``softmax(q k^T / sqrt(128)) v`` over ``n`` joint tokens (GQA), written to two row
    segments: rows ``< n_split`` to ``out0`` and the rest to ``out1`` (``[rows, heads*128]``
    views with unit column stride), each optionally multiplied by ``sigmoid(gate)``.

    ``q``: ``[B, H, N_pad, 128]``, ``k``: ``[B, H_kv, N_pad, 128]``, ``vt``: ``[B, H_kv, 128, N_pad]``
    with zero columns from ``n`` on, all BF16."""
    batch, heads, n_pad, hd = q.shape
    kv_heads = k.shape[1]
    _on_gpu(q, k, vt, out0, out1, gate0, gate1)
    _require(hd == HEAD_DIM and k.shape == (batch, kv_heads, n_pad, HEAD_DIM), "flash_attention: bad q/k shapes")
    _require(vt.shape == (batch, kv_heads, HEAD_DIM, n_pad), "flash_attention: bad vt shape")
    _require(all(t.dtype == torch.bfloat16 and t.is_contiguous() for t in (q, k, vt)), "flash_attention: BF16 inputs")
    ref = out1 if out1 is not None else out0
    _require(ref is not None, "flash_attention: no output")
    for t in (out0, out1, gate0, gate1):
        if t is not None:
            _require(t.dtype == torch.bfloat16 and t.stride(-1) == 1, "flash_attention: BF16 row-major outputs/gates")
    ld_out = ref.stride(-2)
    if out0 is not None and out1 is not None:
        _require(out0.stride(-2) == ld_out, "flash_attention: output strides differ")
    gref = gate1 if gate1 is not None else gate0
    ld_gate = gref.stride(-2) if gref is not None else 0
    ob = out_batch_rows or (n_split, n - n_split)
    gb = gate_batch_rows or (n_split, n - n_split)
    scale = HEAD_DIM ** -0.5 if scale is None else scale
    L.call(
        "iris_flash_attn", L.ptr(q), L.ptr(k), L.ptr(vt), batch, heads, kv_heads, n, n_pad, n_split, float(scale),
        L.ptr(out0), L.ptr(out1), ld_out, ob[0], ob[1], L.ptr(gate0), L.ptr(gate1), ld_gate, gb[0], gb[1],
        L.stream(),
    )


def flash_attention_masked(q, k, vt, n: int, key_mask: torch.Tensor, out: torch.Tensor, scale: float | None = None):
    """The text refiner's attention: ``flash_attention`` where query ``i`` of batch ``b`` sees key
    ``j < n`` only if ``key_mask[b, j]`` or ``j == i`` (``mask | eye``, src/iris3b/nn/embeddings.py:199-201).
    ``key_mask``: uint8 ``[B, N_pad]`` from ``text_key_mask``; ``out``: BF16 ``[B, rows >= n, heads*128]``
    or ``[B*n, heads*128]`` with unit column stride."""
    batch, heads, n_pad, hd = q.shape
    kv_heads = k.shape[1]
    _on_gpu(q, k, vt, key_mask, out)
    _require(hd == HEAD_DIM and k.shape == (batch, kv_heads, n_pad, HEAD_DIM), "flash_attention_masked: bad q/k shapes")
    _require(vt.shape == (batch, kv_heads, HEAD_DIM, n_pad), "flash_attention_masked: bad vt shape")
    _require(all(t.dtype == torch.bfloat16 and t.is_contiguous() for t in (q, k, vt)),
             "flash_attention_masked: BF16 inputs")
    _require(key_mask.dtype == torch.uint8 and key_mask.shape == (batch, n_pad) and key_mask.is_contiguous(),
             f"flash_attention_masked: key_mask must be uint8 [{batch}, {n_pad}]")
    _require(out.dtype == torch.bfloat16 and out.stride(-1) == 1 and out.shape[-1] == heads * HEAD_DIM,
             "flash_attention_masked: BF16 row-major output")
    if out.dim() == 3:
        _require(out.shape[0] == batch and out.shape[1] >= n, "flash_attention_masked: output too small")
        batch_rows = out.stride(0) // out.stride(1)
        _require(out.stride(0) == batch_rows * out.stride(1), "flash_attention_masked: output batch stride")
    else:
        _require(out.shape[0] >= batch * n, "flash_attention_masked: output too small")
        batch_rows = n
    scale = HEAD_DIM ** -0.5 if scale is None else scale
    L.call("iris_flash_attn_masked", L.ptr(q), L.ptr(k), L.ptr(vt), batch, heads, kv_heads, n, n_pad, float(scale),
           L.ptr(key_mask), L.ptr(out), out.stride(-2), batch_rows, L.stream())
    return out


_MASK_KINDS = {torch.bool: 0, torch.uint8: 0, torch.int8: 0, torch.int32: 1, torch.float32: 2, torch.int64: 3}


def text_key_mask(mask: torch.Tensor, n: int, out: torch.Tensor) -> torch.Tensor:
    """``mask[:, :n].bool()`` as the zero-padded uint8 ``[B, N_pad]`` key mask of ``flash_attention_masked``."""
    _on_gpu(mask, out)
    _require(mask.dtype in _MASK_KINDS, f"text mask dtype {mask.dtype} not supported (bool, uint8, int32, int64, float32)")
    _require(mask.dim() == 2 and mask.stride(1) == 1 and mask.shape[1] >= n, "text mask must be [B, >= n] row-major")
    _require(out.dtype == torch.uint8 and out.dim() == 2 and out.shape[0] == mask.shape[0] and out.is_contiguous(),
             "text_key_mask: out must be uint8 [B, N_pad]")
    L.call("iris_text_key_mask", L.ptr(mask), _MASK_KINDS[mask.dtype], mask.stride(0), mask.shape[0], n, out.shape[1],
           L.ptr(out), L.stream())
    return out


def layer_attention(qkv: torch.Tensor, out: torch.Tensor, seq_len: int, heads: int, scale: float | None = None):
    """Attention of each text token over its ``seq_len`` encoder-layer states (no mask, no QK norm):
    ``qkv`` BF16 ``[S*seq_len, 3*heads*d]`` -> ``out`` BF16 ``[S*seq_len, heads*d]``
    (src/iris3b/nn/embeddings.py:139-141, src/iris3b/nn/attention.py:117-132)."""
    _on_gpu(qkv, out)
    rows, width3 = qkv.shape
    _require(qkv.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and qkv.is_contiguous() and out.is_contiguous(),
             "layer_attention works on contiguous BF16")
    _require(width3 % (3 * heads) == 0 and rows % seq_len == 0 and out.shape == (rows, width3 // 3),
             "layer_attention: bad shapes")
    d = width3 // (3 * heads)
    scale = d ** -0.5 if scale is None else scale
    L.call("iris_layer_attention", L.ptr(qkv), L.ptr(out), rows // seq_len, seq_len, heads, d, float(scale), L.stream())
    return out


def layer_pool(h: torch.Tensor, branch: torch.Tensor | None, weight: torch.Tensor, bias: torch.Tensor | None,
               layers: int, out: torch.Tensor) -> torch.Tensor:
    """``layer_pool((h + branch).transpose(1, 2)).squeeze(-1)`` over ``[R, layers, W]`` states
    (src/iris3b/nn/embeddings.py:262); ``h`` FP32, ``branch`` BF16 or None, ``out`` ``[R, W]``."""
    _on_gpu(h, branch, weight, bias, out)
    _require_fp32(h=h, weight=weight)
    width = h.shape[-1]
    rows = h.numel() // (layers * width)
    _require(h.is_contiguous() and h.numel() == rows * layers * width, "layer_pool: bad states")
    if branch is not None:
        _require(branch.dtype == torch.bfloat16 and branch.is_contiguous() and branch.numel() == h.numel(),
                 "layer_pool: branch must be BF16 like h")
    if bias is not None:
        _require_fp32(bias=bias)
    _require(weight.numel() == layers and (bias is None or bias.numel() == 1), "layer_pool: weight is [1, layers]")
    _require(out.is_contiguous() and out.numel() == rows * width, "layer_pool: bad out")
    L.call("iris_layer_pool", L.ptr(h), L.ptr(branch), L.ptr(weight), L.ptr(bias), rows, layers, width, L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def residual_rms_norm(residual: torch.Tensor, branch: torch.Tensor | None, weight: torch.Tensor, eps: float,
                      out: torch.Tensor, add_rows: torch.Tensor | None = None) -> torch.Tensor:
    """``residual += branch`` (in place, FP32), then ``out = rmsnorm(residual) * weight (+ add_rows)``
    (the pre-norm residual of src/iris3b/nn/embeddings.py:105-107, 139-141; ``add_rows``
    ``[P, W]`` is added to row ``r`` as ``add_rows[r % P]``)."""
    _on_gpu(residual, branch, weight, out, add_rows)
    _require_fp32(residual=residual, weight=weight)
    width = residual.shape[-1]
    rows = residual.numel() // width
    _require(residual.is_contiguous() and out.is_contiguous() and out.numel() == residual.numel(),
             "residual_rms_norm: contiguous residual and out of one shape")
    if branch is not None:
        _require(branch.is_contiguous() and branch.numel() == residual.numel(), "residual_rms_norm: bad branch")
    period = 0
    if add_rows is not None:
        _require_fp32(add_rows=add_rows)
        _require(add_rows.is_contiguous() and add_rows.shape[-1] == width, "residual_rms_norm: bad add_rows")
        period = add_rows.numel() // width
    _require(weight.numel() == width, "residual_rms_norm: weight width")
    L.call("iris_residual_rms_norm", L.ptr(residual), L.ptr(branch),
           L.dtype_code(branch.dtype) if branch is not None else L.F32, L.ptr(weight), L.ptr(add_rows), period, rows,
           width, float(eps), L.ptr(out), L.dtype_code(out.dtype), L.stream())
    return out


def gemv(
    weight: torch.Tensor,
    x: torch.Tensor,
    bias: torch.Tensor | None,
    out: torch.Tensor,
    extra_bias: torch.Tensor | None = None,
    in_silu: bool = False,
    out_silu: bool = False,
) -> torch.Tensor:
    """``out = act(act_in(x) W^T + bias)`` for a few rows ``x`` (FP32 ``[B, K]``), BF16 ``W``;
    with ``extra_bias`` (``[J, N]``) ``out[j] = y + extra_bias[j]`` (``out``: ``[J, B, N]``)."""
    n, k = weight.shape
    batch = x.shape[0]
    _on_gpu(weight, x, bias, out, extra_bias)
    _require(weight.dtype == torch.bfloat16 and weight.is_contiguous(), "gemv: BF16 contiguous weight")
    _require(x.shape == (batch, k) and x.dtype == torch.float32 and x.is_contiguous(), "gemv: FP32 [B, K] input")
    n_extra = 0 if extra_bias is None else extra_bias.shape[0]
    expect = (n_extra, batch, n) if n_extra else (batch, n)
    _require(tuple(out.shape) == expect and out.dtype == torch.float32 and out.is_contiguous(), "gemv: bad out")
    if bias is not None:
        _require_fp32(bias=bias)
    if extra_bias is not None:
        _require_fp32(extra_bias=extra_bias)
    L.call(
        "iris_gemv_bf16", L.ptr(weight), L.ptr(x), batch, n, k, L.ptr(bias), L.ptr(extra_bias), n_extra, L.ptr(out),
        L.ACT_SILU if in_silu else L.ACT_NONE, L.ACT_SILU if out_silu else L.ACT_NONE, L.stream(),
    )
    return out


def patchify_embed(x, patch, pix_w, pix_b, pos_x, pos_y, norm_weight, eps, patches, pixels, normed) -> None:
    """Patch matrix for the patch embedder, the embedded pixel stream and its first norm
    (src/iris_metal/model.py:188-189, 208-210)."""
    batch, channels, height, width = x.shape
    _on_gpu(x, patches, pixels, normed)
    _require(channels in (3, 4) and x.dtype == torch.float32 and x.is_contiguous(),
             "patchify_embed: FP32 [B, 3 or 4, H, W]")
    _require_fp32(pix_w=pix_w, pix_b=pix_b, pos_x=pos_x, pos_y=pos_y, norm_weight=norm_weight)
    _require(pix_w.shape == (PIXEL_WIDTH, channels), f"patchify_embed: pixel embedder weight must be [16, {channels}]")
    n_patches = (height // patch) * (width // patch)
    _require(patches.dtype == torch.bfloat16 and patches.stride(-1) == 1
             and patches.reshape(-1, patches.shape[-1]).shape[0] == batch * n_patches
             and patches.shape[-1] >= channels * patch * patch,
             "patchify_embed: patches must be BF16 [B*L, >= C*p*p]")
    _require(pixels.numel() == normed.numel() == batch * height * width * PIXEL_WIDTH
             and normed.dtype == torch.bfloat16, "patchify_embed: bad pixel buffers")
    L.call(
        "iris_patchify_embed", L.ptr(x), batch, channels, height, width, patch, L.ptr(patches), patches.stride(-2),
        L.ptr(pix_w), L.ptr(pix_b),
        L.ptr(pos_x), L.ptr(pos_y), L.ptr(norm_weight), float(eps), L.ptr(pixels), L.dtype_code(pixels.dtype),
        L.ptr(normed), L.stream(),
    )


def unpatchify_head(h, weight, bias, out, patch) -> torch.Tensor:
    """``out[b, c, y, x] = h[pixel] . weight[c] + bias[c]`` (src/iris_metal/model.py:214-217);
    3 output channels, or 1 for the depth head."""
    batch, channels, height, width = out.shape
    _on_gpu(h, weight, bias, out)
    _require(channels in (1, 3) and out.dtype == torch.float32 and out.is_contiguous(),
             "unpatchify_head: FP32 output of 1 or 3 channels")
    _require(h.dtype == torch.bfloat16 and h.is_contiguous(), "unpatchify_head: BF16 pixels")
    _require_fp32(weight=weight, bias=bias)
    _require(weight.shape == (channels, PIXEL_WIDTH) and bias.numel() == channels, "unpatchify_head: head shape")
    L.call("iris_unpatchify_head", L.ptr(h), L.ptr(weight), L.ptr(bias), L.ptr(out), channels, batch, height, width,
           patch, L.stream())
    return out


def timestep_features(t: torch.Tensor, freqs: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``[cos | sin](t * freqs)`` (src/iris3b/nn/embeddings.py:41-45); ``out``: FP32 ``[B, 2*len(freqs)]``."""
    _on_gpu(t, freqs, out)
    _require_fp32(t=t, freqs=freqs, out=out)
    _require(out.shape == (t.numel(), 2 * freqs.numel()), "timestep_features: bad out")
    L.call("iris_timestep_features", L.ptr(t), L.ptr(freqs), t.numel(), freqs.numel(), L.ptr(out), L.stream())
    return out


def copy_rows(src, dst, batch: int, rows: int, src_offset: int, src_batch_rows: int, dst_offset: int,
              dst_batch_rows: int) -> None:
    """``dst[b*dst_batch_rows + dst_offset + r] = src[b*src_batch_rows + src_offset + r]`` for FP32 rows."""
    _on_gpu(src, dst)
    _require_fp32(src=src, dst=dst)
    width = src.shape[-1]
    _require(dst.shape[-1] == width, "copy_rows: widths differ")
    _require(src.numel() >= batch * src_batch_rows * width and dst.numel() >= batch * dst_batch_rows * width,
             "copy_rows: buffers too small")
    L.call("iris_copy_rows", L.ptr(src), L.ptr(dst), batch, rows, width, src_batch_rows, src_offset, dst_batch_rows,
           dst_offset, L.stream())


def silu_add_rows(x, t, rows_per_batch: int, out) -> None:
    """``out[r] = silu(x[r] + t[r // rows_per_batch])`` (src/iris_metal/model.py:207)."""
    _on_gpu(x, t, out)
    _require_fp32(x=x, t=t)
    _require(out.shape == x.shape and out.is_contiguous(), "silu_add_rows: bad out")
    L.call("iris_silu_add_rows", L.ptr(x), L.ptr(t), x.shape[0], rows_per_batch, x.shape[1], L.ptr(out),
           L.dtype_code(out.dtype), L.stream())


def flow_euler(x, v, sigma: float, sigma_next: float | None, x_next, clean) -> None:
    """Turbo Euler step in the reference's FP32 operation order (src/iris3b/sampling.py:129-135)."""
    _on_gpu(x, v, x_next, clean)
    L.call("iris_flow_euler", L.ptr(x), L.ptr(v), x.numel(), float(sigma), float(sigma_next or 0.0),
           L.ptr(x_next) if sigma_next is not None else None, L.ptr(clean), L.stream())


def dpm1_update(x, v, s: float, c_x: float, c_x0: float, out) -> None:
    _on_gpu(x, v, out)
    L.call("iris_dpm1_update", L.ptr(x), L.ptr(v), x.numel(), float(s), float(c_x), float(c_x0), L.ptr(out),
           L.stream())


def dpm_update(x, v, x0_prev, s: float, c_x: float, c_x0: float, c_d: float, r0: float, x_next, x0_out) -> None:
    """One FlowDPMSolver step (src/iris3b/flow/solver.py:90-109): first order when ``x0_prev``
    is None, else second order; ``x0_out`` receives this step's ``x0 = x - s*v``."""
    tensors = [t for t in (x, v, x0_prev, x_next, x0_out) if t is not None]
    _on_gpu(*tensors)
    _require(all(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == x.numel() for t in tensors),
             "dpm_update needs contiguous FP32 tensors of one size")
    L.call("iris_dpm_update", L.ptr(x), L.ptr(v), L.ptr(x0_prev), x.numel(), float(s), float(c_x), float(c_x0),
           float(c_d), float(r0), L.ptr(x_next), L.ptr(x0_out), L.stream())


def cfg_combine(v_uncond, v_cond, scale: float, out) -> None:
    _on_gpu(v_uncond, v_cond, out)
    L.call("iris_cfg_combine", L.ptr(v_uncond), L.ptr(v_cond), v_cond.numel(), float(scale), L.ptr(out), L.stream())


def clamp(x, lo: float, hi: float, out) -> None:
    _on_gpu(x, out)
    L.call("iris_clamp", L.ptr(x), x.numel(), float(lo), float(hi), L.ptr(out), L.stream())
