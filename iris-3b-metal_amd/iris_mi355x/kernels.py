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


class _Check:
    """The host-side argument checks of one wrapper call, run before anything is launched.

    Created with the operation's name and the tensors that must live on the GPU (``None``
    entries are skipped); calling it with a condition and a description raises
    ``ValueError("<op>: <description>")`` when the condition is false. Methods cover the
    recurring expectations (FP32 gains of a given width, BF16 operands, contiguity)."""

    __slots__ = ("op",)

    def __init__(self, op: str, *tensors: torch.Tensor | None):
        self.op = op
        if any(t is not None and t.device.type != "cuda" for t in tensors):
            raise ValueError(f"{op}: the HIP kernels need GPU tensors (there is no CPU path)")

    def __call__(self, ok: bool, what: str) -> "_Check":
        if not ok:
            raise ValueError(f"{self.op}: {what}")
        return self

    def fp32(self, **tensors: torch.Tensor) -> "_Check":
        for name, t in tensors.items():
            self(t.dtype == torch.float32 and t.is_contiguous(), f"{name} must be contiguous FP32 (got {t.dtype})")
        return self

    def gains(self, width: int, **gains: torch.Tensor) -> "_Check":
        """Per-channel FP32 vectors of ``width`` entries (RMSNorm gains)."""
        self.fp32(**gains)
        for name, g in gains.items():
            self(g.numel() == width, f"{name}: gain width {g.numel()} does not match the {width} channels")
        return self

    def bf16(self, **tensors: torch.Tensor) -> "_Check":
        for name, t in tensors.items():
            self(t.dtype == torch.bfloat16 and t.is_contiguous(), f"{name} must be contiguous BF16 (got {t.dtype})")
        return self


def _mod_rows(vector: torch.Tensor, batch: int, width: int) -> tuple[torch.Tensor, int]:
    """A ``[B, 1, D]`` slice of a modulation vector as FP32 rows the kernels read with 16-byte
    loads: returned in place when its rows are unit-stride and 16-byte aligned (slices of the
    engine's ``[B, 6D]`` modulation table are), else as a packed copy; with the row stride in
    elements (``D`` for one row)."""
    rows = vector.reshape(batch, width)
    rows = rows if rows.dtype == torch.float32 else rows.float()
    in_place = rows.stride(1) == 1 and rows.storage_offset() % 4 == 0 and (batch == 1 or rows.stride(0) % 4 == 0)
    if not in_place:
        rows = rows.contiguous()
    return rows, (rows.stride(0) if batch > 1 else width)


def _mod_pair(shift: torch.Tensor, scale: torch.Tensor, batch: int,
              width: int) -> tuple[torch.Tensor, torch.Tensor, int]:
    """``_mod_rows`` of a shift and a scale that the kernel addresses with one row stride."""
    shift, stride_a = _mod_rows(shift, batch, width)
    scale, stride_b = _mod_rows(scale, batch, width)
    if stride_a != stride_b:
        shift, scale, stride_a = shift.contiguous(), scale.contiguous(), width
    return shift, scale, stride_a


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
    if heads <= 0 or min(col_offset, offset) < 0:
        raise ValueError(f"qk_norm_rope: heads must be positive and offsets nonnegative "
                         f"(heads={heads}, col_offset={col_offset}, offset={offset})")
    batch, tokens, width = x.shape
    if out is None:
        out = x.new_empty(batch, heads, tokens, HEAD_DIM, dtype=out_dtype or x.dtype)
    check = _Check("qk_norm_rope", x, out, weight, cos, sin)
    check(x.is_contiguous() and col_offset + heads * HEAD_DIM <= width,
          f"the contiguous [B, N, {width}] input does not hold {heads} heads from column {col_offset}")
    check(out.is_contiguous() and out.dim() == 4 and out.shape[:2] == (batch, heads) and out.shape[3] == HEAD_DIM,
          f"output must be a contiguous [{batch}, {heads}, N, {HEAD_DIM}] tensor")
    rows_needed = offset + tokens
    check(cos.shape == sin.shape and cos.dim() == 2 and cos.shape[1] == HEAD_DIM // 2
          and rows_needed <= cos.shape[0] and rows_needed <= out.shape[2],
          f"rotary tables or output do not cover the written rows (up to {rows_needed})")
    check.fp32(cos=cos, sin=sin).gains(HEAD_DIM, weight=weight)
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
    check = _Check("rms_norm_modulate", x, weight, shift, scale, out)
    check(x.is_contiguous() and width % 128 == 0, f"needs a contiguous input whose width is a multiple of 128 "
                                                  f"(got {width})")
    check.gains(width, weight=weight)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    check(out.is_contiguous() and out.shape == x.shape and out.dtype == out_dtype,
          f"out must be a contiguous {out_dtype} tensor of the input's shape")
    shift, scale, stride = _mod_pair(shift, scale, batch, width)
    L.call(
        "iris_rms_norm_modulate", L.ptr(x), L.dtype_code(x.dtype), L.ptr(out), L.dtype_code(out_dtype),
        L.ptr(weight), L.ptr(shift), L.ptr(scale), batch * tokens, tokens, width, stride, float(eps),
        L.stream(),
    )
    return out


def _residual_checks(check: _Check, residual: torch.Tensor, branch: torch.Tensor, width: int) -> None:
    check(width % 128 == 0 and branch.shape == residual.shape and branch.is_contiguous(),
          "the branch must be contiguous and shaped like the residual, of a width that is a multiple of 128")
    check.fp32(residual=residual)


def gated_residual_rms_norm_(
    residual: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, eps: float
) -> torch.Tensor:
    """``residual += gate * rms_norm(branch) * weight`` in place; ``residual``: FP32 ``[B, N, D]``
    (src/iris_metal/kernels.py:455-480)."""
    batch, tokens, width = residual.shape
    check = _Check("gated_residual_rms_norm_", residual, branch, weight, gate)
    _residual_checks(check, residual, branch, width)
    check.gains(width, weight=weight)
    gate, gate_stride = _mod_rows(gate, batch, width)
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
    check = _Check("gated_residual_norm_modulate_", residual, branch, weight, gate, next_weight, next_shift,
                   next_scale, out)
    _residual_checks(check, residual, branch, width)
    check(out.is_contiguous() and out.shape == residual.shape, "out must be contiguous and shaped like the residual")
    check.gains(width, weight=weight, next_weight=next_weight)
    gate, gate_stride = _mod_rows(gate, batch, width)
    shift, scale, stride = _mod_pair(next_shift, next_scale, batch, width)
    L.call(
        "iris_gated_residual_norm_modulate", L.ptr(residual), L.ptr(branch), L.dtype_code(branch.dtype),
        L.ptr(weight), L.ptr(gate), batch * tokens, tokens, width, gate_stride, float(eps), L.ptr(next_weight),
        L.ptr(shift), L.ptr(scale), stride, L.ptr(out), L.dtype_code(out.dtype), L.stream(),
    )
    return out


def gated_residual_grouped_(residuals, branches, weights, gates, eps: float, next_weights=None, next_shifts=None,
                            next_scales=None, outs=None) -> None:
    """``gated_residual_rms_norm_`` (``outs`` None) or ``gated_residual_norm_modulate_`` of two
    streams (the image and text rows of a dual-stream block) in one launch, each on its own
    tensors; same results as the two calls."""
    if not len(residuals) == len(branches) == len(weights) == len(gates) == 2:
        raise ValueError("gated_residual_grouped_ takes two streams")
    nxt = outs is not None
    width = residuals[0].shape[-1]
    groups = []  # per stream: (gate rows, rows, rows per batch, gate stride, shift, scale, stride)
    for i in range(2):
        residual, branch = residuals[i], branches[i]
        batch, tokens, w = residual.shape
        check = _Check(f"gated_residual_grouped_ (stream {i})", residual, branch, weights[i], gates[i],
                       *((next_weights[i], next_shifts[i], next_scales[i], outs[i]) if nxt else ()))
        check(w == width, "the two streams differ in width")
        _residual_checks(check, residual, branch, width)
        check(branch.dtype == branches[0].dtype, "the two branches differ in dtype")
        check.gains(width, weight=weights[i])
        gate, gate_stride = _mod_rows(gates[i], batch, width)
        entry = [gate, batch * tokens, tokens, gate_stride, None, None, 0]
        if nxt:
            check(outs[i].is_contiguous() and outs[i].shape == residual.shape and outs[i].dtype == outs[0].dtype,
                  "outputs must be contiguous, shaped like their residual, of one dtype")
            check.gains(width, next_weight=next_weights[i])
            entry[4:] = _mod_pair(next_shifts[i], next_scales[i], batch, width)
        groups.append(entry)
    P = L.pointer_array
    L.call(
        "iris_gated_residual_grouped", 2, P([L.ptr(r) for r in residuals]), P([L.ptr(b) for b in branches]),
        L.dtype_code(branches[0].dtype), P([L.ptr(w) for w in weights]), P([L.ptr(g[0]) for g in groups]),
        L.long_array([g[1] for g in groups]), L.long_array([g[2] for g in groups]), width,
        L.long_array([g[3] for g in groups]), float(eps),
        P([L.ptr(w) for w in next_weights]) if nxt else None, P([L.ptr(g[4]) for g in groups]) if nxt else None,
        P([L.ptr(g[5]) for g in groups]) if nxt else None, L.long_array([g[6] for g in groups]) if nxt else None,
        P([L.ptr(o) for o in outs]) if nxt else None, L.dtype_code(outs[0].dtype) if nxt else L.BF16, L.stream(),
    )


def pixel_rms_norm(pixels: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rms_norm(pixels) * weight`` over the 16 channels of each pixel, stored BF16
    (src/iris_metal/kernels.py:486-498)."""
    check = _Check("pixel_rms_norm", pixels, weight)
    check(pixels.is_contiguous() and pixels.shape[-1] == PIXEL_WIDTH, "needs contiguous 16-channel pixels")
    check.gains(PIXEL_WIDTH, weight=weight)
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
    scale2, shift2); ``fc1``/``fc2``: ``nn.Linear`` (or ``(weight, bias)``) of 16 -> 64 -> 16.
    The MLP rounds where the reference kernel does (src/iris_metal/kernels.py:268-280): the normed
    input, both weights, the pre-activation and the exact-erf GELU (correctly rounded) are BF16,
    the two products BF16 MFMA with FP32 sums; the stream and both modulations stay FP32."""
    check = _Check("pixel_mlp_", pixels, branch, mods, norm_weight, next_norm_weight)
    w1, b1 = _linear_params(fc1)
    w2, b2 = _linear_params(fc2)
    widths = (pixels.shape[-1], tuple(w1.shape), tuple(w2.shape), tuple(b1.shape), tuple(b2.shape))
    released = (PIXEL_WIDTH, (PIXEL_HIDDEN, PIXEL_WIDTH), (PIXEL_WIDTH, PIXEL_HIDDEN), (PIXEL_HIDDEN,), (PIXEL_WIDTH,))
    check(widths == released and branch.shape == pixels.shape
          and mods.shape == (*pixels.shape[:-1], 4 * PIXEL_WIDTH),
          "needs the released pixel-stage widths (16 channels, a 64-wide MLP, 64 modulation values per pixel)")
    check(pixels.dtype in (torch.float32, torch.bfloat16) and pixels.is_contiguous(),
          "pixels must be contiguous FP32 or BF16")
    check.bf16(branch=branch, mods=mods)
    check.gains(PIXEL_WIDTH, norm_weight=norm_weight, next_norm_weight=next_norm_weight)
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
    check = _Check("v_heads_t", x, out)
    check(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "works on BF16")
    check(x.is_contiguous() and out.is_contiguous(), "needs contiguous tensors")
    check(out.shape[:3] == (batch, heads, HEAD_DIM), f"output must be [{batch}, {heads}, 128, N]")
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
    check = _Check("qkv_prepare", x, q, k, vt, q_weight, k_weight, cos, sin)
    check(all(t.dtype == torch.bfloat16 for t in (x, q, k, vt)), "works on BF16")
    check(x.is_contiguous() and q.is_contiguous() and k.is_contiguous() and vt.is_contiguous(),
          "needs contiguous tensors")
    check(q.shape == (batch, heads, q.shape[2], HEAD_DIM) and k.shape == (batch, kv_heads, q.shape[2], HEAD_DIM),
          "q / k must be [B, heads, N, 128] buffers of equal length")
    check(vt.shape[:3] == (batch, kv_heads, HEAD_DIM), f"vt must be [{batch}, {kv_heads}, 128, N]")
    check(cos.shape == sin.shape == (cos.shape[0], HEAD_DIM // 2), "rotary tables must be [N, 64]")
    check.fp32(q_weight=q_weight, k_weight=k_weight, cos=cos, sin=sin)
    check(q_weight.numel() == HEAD_DIM and k_weight.numel() == HEAD_DIM, "gains have 128 entries")
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
    _Check("linear")(not (swiglu and silu), "choose one epilogue")
    check = _Check("linear", x, weight, bias, out)
    check(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16, "takes BF16 operands")
    check(x.stride(-1) == 1 and weight.is_contiguous(), "needs row-contiguous operands")
    k = x.shape[-1]
    n = weight.shape[0]
    check(weight.shape[1] == k, f"weight {tuple(weight.shape)} does not match input width {k}")
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    n_out = n // 2 if swiglu else n
    if out is None:
        out = torch.empty(*x.shape[:-1], n_out, device=x.device, dtype=out_dtype)
    check(out.shape[-1] == n_out and out.stride(-1) == 1, "bad output")
    if bias is not None:
        check.fp32(bias=bias)
        check(bias.numel() == n, "bias width mismatch")
    out2 = out.reshape(-1, n_out)
    L.call(
        "iris_gemm_bf16", L.ptr(x2), L.ptr(weight), L.ptr(bias), L.ptr(out2), L.dtype_code(out.dtype), m, n, k,
        x2.stride(0), weight.stride(0), out2.stride(0),
        L.EPI_SILU_MUL if swiglu else (L.EPI_SILU if silu else L.EPI_NONE), L.stream(),
    )
    return out


def linear_grouped(xs, weights, biases, outs, swiglu: bool = False) -> None:
    """Two ``linear`` calls of equal weight shape (one per stream of a dual block) in one launch."""
    _Check("linear_grouped")(len(xs) == len(weights) == len(outs) == 2, "takes two problems")
    k = xs[0].shape[-1]
    n = weights[0].shape[0]
    for x, w, o in zip(xs, weights, outs):
        check = _Check("linear_grouped", x, w, o)
        check(w.shape == (n, k) and x.shape[-1] == k and x.stride(-1) == 1, "shape mismatch")
        check(x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16, "takes BF16 operands")
    x2 = [x.reshape(-1, k) for x in xs]
    o2 = [o.reshape(-1, o.shape[-1]) for o in outs]
    check(x2[0].stride(0) == x2[1].stride(0) and o2[0].stride(0) == o2[1].stride(0), "strides differ")
    check(outs[0].dtype == outs[1].dtype, "output dtypes differ")
    bias_ptrs = None if biases is None else L.pointer_array([L.ptr(b) for b in biases])
    L.call(
        "iris_gemm_bf16_grouped", 2, L.pointer_array([L.ptr(x) for x in x2]),
        L.pointer_array([L.ptr(w) for w in weights]), bias_ptrs, L.pointer_array([L.ptr(o) for o in o2]),
        L.int_array([x.shape[0] for x in x2]), L.dtype_code(outs[0].dtype), n, k, x2[0].stride(0),
        weights[0].stride(0), o2[0].stride(0), L.EPI_SILU_MUL if swiglu else L.EPI_NONE, L.stream(),
    )


def linear_qk_rope(xs, weights, outs, q_weights, k_weights, cos: torch.Tensor, sin: torch.Tensor, eps: float,
                   heads: int, kv_heads: int, q: torch.Tensor, k: torch.Tensor, rows_per_batch, offsets,
                   vt: torch.Tensor | None = None) -> None:
    """``linear`` of one or two q | k | v (| gate) projections (one per stream of a dual block, in
    one launch) whose Q and K heads go to ``q`` / ``k`` normed and rotated exactly as
    ``qk_norm_rope`` writes them; the columns after them go to ``outs`` as ``linear`` writes them,
    except that with ``vt`` the ``kv_heads`` V heads go transposed into it exactly as ``v_heads_t``
    writes them (every ``rows_per_batch`` a multiple of 256 and every offset of 16), and ``outs``
    then receives only the columns after the V heads (the attention gate of a q | k | v | gate
    weight). Group ``i``'s rows are batch items of ``rows_per_batch[i]`` tokens, written at rows
    ``offsets[i] + token`` of ``q`` / ``k`` (``[B, heads, N, 128]`` / ``[B, kv_heads, N, 128]``,
    BF16) with gains ``q_weights[i]`` / ``k_weights[i]`` and the rotary tables' rows
    ``offsets[i] + token``."""
    groups = len(xs)
    check = _Check("linear_qk_rope", q, k, cos, sin)
    check(groups in (1, 2) and len(weights) == len(outs) == len(q_weights) == len(k_weights) == groups
          and len(rows_per_batch) == len(offsets) == groups, "takes one or two problems")
    kdim = xs[0].shape[-1]
    n = weights[0].shape[0]
    for x, w, o, rows in zip(xs, weights, outs, rows_per_batch):
        c = _Check("linear_qk_rope", x, w, o)
        c(x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and o.dtype == torch.bfloat16, "works on BF16")
        c(w.shape == (n, kdim) and w.is_contiguous() and x.shape[-1] == kdim and x.stride(-1) == 1,
          "shape mismatch")
        c(o.shape[-1] == n and o.stride(-1) == 1 and o.reshape(-1, n).shape[0] == x.reshape(-1, kdim).shape[0],
          "bad output")
        c(rows > 0 and x.reshape(-1, kdim).shape[0] % rows == 0, "rows are not whole batch items")
    x2 = [x.reshape(-1, kdim) for x in xs]
    o2 = [o.reshape(-1, n) for o in outs]
    check(all(x.stride(0) == x2[0].stride(0) for x in x2) and all(o.stride(0) == o2[0].stride(0) for o in o2),
          "strides differ")
    check(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and q.is_contiguous() and k.is_contiguous(),
          "q / k must be contiguous BF16")
    check(q.dim() == 4 and q.shape[1] == heads and q.shape[3] == HEAD_DIM
          and k.shape == (q.shape[0], kv_heads, q.shape[2], HEAD_DIM),
          "q / k must be [B, heads, N, 128] buffers of equal length")
    check(cos.shape == sin.shape == (cos.shape[0], HEAD_DIM // 2), "rotary tables must be [N, 64]")
    check.fp32(cos=cos, sin=sin, **{f"q_weight{i}": w for i, w in enumerate(q_weights)},
               **{f"k_weight{i}": w for i, w in enumerate(k_weights)})
    check(all(w.numel() == HEAD_DIM for w in (*q_weights, *k_weights)), "gains have 128 entries")
    for x, rows in zip(x2, rows_per_batch):
        check(x.shape[0] // rows <= q.shape[0], "more batch items than q / k hold")
    if vt is not None:
        check(vt.dtype == torch.bfloat16 and vt.is_contiguous() and vt.dim() == 4
              and vt.shape[:3] == (q.shape[0], kv_heads, HEAD_DIM) and vt.shape[3] % 64 == 0,
              f"vt must be a contiguous BF16 [{q.shape[0]}, {kv_heads}, 128, N] buffer, N % 64 == 0")
        check(all(r % 256 == 0 and o % 16 == 0 for r, o in zip(rows_per_batch, offsets)),
              "the V^T store needs rows_per_batch % 256 == 0 and offsets % 16 == 0")
        check(n >= (heads + 2 * kv_heads) * HEAD_DIM,
              f"with vt the weight must hold {heads} Q, {kv_heads} K and {kv_heads} V heads "
              f"(at least {(heads + 2 * kv_heads) * HEAD_DIM} rows), got {n}")
    L.call(
        "iris_gemm_bf16_qk_rope", groups, L.pointer_array([L.ptr(x) for x in x2]),
        L.pointer_array([L.ptr(w) for w in weights]), L.pointer_array([L.ptr(o) for o in o2]),
        L.int_array([x.shape[0] for x in x2]), n, kdim, x2[0].stride(0), weights[0].stride(0), o2[0].stride(0),
        L.pointer_array([L.ptr(w) for w in q_weights]), L.pointer_array([L.ptr(w) for w in k_weights]),
        L.int_array(list(rows_per_batch)), L.int_array(list(offsets)), L.ptr(cos), L.ptr(sin), cos.shape[0],
        L.ptr(q), L.ptr(k), heads, kv_heads, q.shape[2], L.ptr(vt), vt.shape[3] if vt is not None else 0,
        float(eps), L.stream(),
    )


def pack_swiglu(w1: torch.Tensor, w3: torch.Tensor, hidden_pad: int) -> torch.Tensor:
    """Interleave SwiGLU ``w1``/``w3`` (``[H, D]``) in 32-row groups, zero-padded to ``hidden_pad``
    rows each: rows ``64p..64p+31`` are ``w1[32p:32p+32]``, rows ``64p+32..`` are ``w3[32p:..]``."""
    hidden, dim = w1.shape
    _Check("pack_swiglu")(w3.shape == w1.shape and hidden_pad % 32 == 0 and hidden_pad >= hidden, "bad shapes")
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
    check = _Check("flash_attention", q, k, vt, out0, out1, gate0, gate1)
    check(hd == HEAD_DIM and k.shape == (batch, kv_heads, n_pad, HEAD_DIM), "bad q/k shapes")
    check(vt.shape == (batch, kv_heads, HEAD_DIM, n_pad), "bad vt shape")
    check(all(t.dtype == torch.bfloat16 and t.is_contiguous() for t in (q, k, vt)), "BF16 inputs")
    ref = out1 if out1 is not None else out0
    check(ref is not None, "no output")
    for t in (out0, out1, gate0, gate1):
        if t is not None:
            check(t.dtype == torch.bfloat16 and t.stride(-1) == 1, "BF16 row-major outputs/gates")
    ld_out = ref.stride(-2)
    if out0 is not None and out1 is not None:
        check(out0.stride(-2) == ld_out, "output strides differ")
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
    check = _Check("flash_attention_masked", q, k, vt, key_mask, out)
    check(hd == HEAD_DIM and k.shape == (batch, kv_heads, n_pad, HEAD_DIM), "bad q/k shapes")
    check(vt.shape == (batch, kv_heads, HEAD_DIM, n_pad), "bad vt shape")
    check(all(t.dtype == torch.bfloat16 and t.is_contiguous() for t in (q, k, vt)),
          "BF16 inputs")
    check(key_mask.dtype == torch.uint8 and key_mask.shape == (batch, n_pad) and key_mask.is_contiguous(),
          f"key_mask must be uint8 [{batch}, {n_pad}]")
    check(out.dtype == torch.bfloat16 and out.stride(-1) == 1 and out.shape[-1] == heads * HEAD_DIM,
          "BF16 row-major output")
    if out.dim() == 3:
        check(out.shape[0] == batch and out.shape[1] >= n, "output too small")
        batch_rows = out.stride(0) // out.stride(1)
        check(out.stride(0) == batch_rows * out.stride(1), "output batch stride")
    else:
        check(out.shape[0] >= batch * n, "output too small")
        batch_rows = n
    scale = HEAD_DIM ** -0.5 if scale is None else scale
    L.call("iris_flash_attn_masked", L.ptr(q), L.ptr(k), L.ptr(vt), batch, heads, kv_heads, n, n_pad, float(scale),
           L.ptr(key_mask), L.ptr(out), out.stride(-2), batch_rows, L.stream())
    return out


_MASK_KINDS = {torch.bool: 0, torch.uint8: 0, torch.int8: 0, torch.int32: 1, torch.float32: 2, torch.int64: 3}


def text_key_mask(mask: torch.Tensor, n: int, out: torch.Tensor) -> torch.Tensor:
    """``mask[:, :n].bool()`` as the zero-padded uint8 ``[B, N_pad]`` key mask of ``flash_attention_masked``."""
    check = _Check("text_key_mask", mask, out)
    check(mask.dtype in _MASK_KINDS, f"text mask dtype {mask.dtype} not supported (bool, uint8, int32, int64, float32)")
    check(mask.dim() == 2 and mask.stride(1) == 1 and mask.shape[1] >= n, "text mask must be [B, >= n] row-major")
    check(out.dtype == torch.uint8 and out.dim() == 2 and out.shape[0] == mask.shape[0] and out.is_contiguous(),
          "out must be uint8 [B, N_pad]")
    L.call("iris_text_key_mask", L.ptr(mask), _MASK_KINDS[mask.dtype], mask.stride(0), mask.shape[0], n, out.shape[1],
           L.ptr(out), L.stream())
    return out


def layer_attention(qkv: torch.Tensor, out: torch.Tensor, seq_len: int, heads: int, scale: float | None = None):
    """Attention of each text token over its ``seq_len`` encoder-layer states (no mask, no QK norm):
    ``qkv`` BF16 ``[S*seq_len, 3*heads*d]`` -> ``out`` BF16 ``[S*seq_len, heads*d]``
    (src/iris3b/nn/embeddings.py:139-141, src/iris3b/nn/attention.py:117-132)."""
    check = _Check("layer_attention", qkv, out)
    rows, width3 = qkv.shape
    check(qkv.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and qkv.is_contiguous() and out.is_contiguous(),
          "works on contiguous BF16")
    check(width3 % (3 * heads) == 0 and rows % seq_len == 0 and out.shape == (rows, width3 // 3),
          "bad shapes")
    d = width3 // (3 * heads)
    scale = d ** -0.5 if scale is None else scale
    L.call("iris_layer_attention", L.ptr(qkv), L.ptr(out), rows // seq_len, seq_len, heads, d, float(scale), L.stream())
    return out


def layer_pool(h: torch.Tensor, branch: torch.Tensor | None, weight: torch.Tensor, bias: torch.Tensor | None,
               layers: int, out: torch.Tensor) -> torch.Tensor:
    """``layer_pool((h + branch).transpose(1, 2)).squeeze(-1)`` over ``[R, layers, W]`` states
    (src/iris3b/nn/embeddings.py:262); ``h`` FP32, ``branch`` BF16 or None, ``out`` ``[R, W]``."""
    check = _Check("layer_pool", h, branch, weight, bias, out)
    check.fp32(h=h, weight=weight)
    width = h.shape[-1]
    rows = h.numel() // (layers * width)
    check(h.is_contiguous() and h.numel() == rows * layers * width, "bad states")
    if branch is not None:
        check(branch.dtype == torch.bfloat16 and branch.is_contiguous() and branch.numel() == h.numel(),
              "branch must be BF16 like h")
    if bias is not None:
        check.fp32(bias=bias)
    check(weight.numel() == layers and (bias is None or bias.numel() == 1), "weight is [1, layers]")
    check(out.is_contiguous() and out.numel() == rows * width, "bad out")
    L.call("iris_layer_pool", L.ptr(h), L.ptr(branch), L.ptr(weight), L.ptr(bias), rows, layers, width, L.ptr(out),
           L.dtype_code(out.dtype), L.stream())
    return out


def residual_rms_norm(residual: torch.Tensor, branch: torch.Tensor | None, weight: torch.Tensor, eps: float,
                      out: torch.Tensor, add_rows: torch.Tensor | None = None) -> torch.Tensor:
    """``residual += branch`` (in place, FP32), then ``out = rmsnorm(residual) * weight (+ add_rows)``
    (the pre-norm residual of src/iris3b/nn/embeddings.py:105-107, 139-141; ``add_rows``
    ``[P, W]`` is added to row ``r`` as ``add_rows[r % P]``)."""
    check = _Check("residual_rms_norm", residual, branch, weight, out, add_rows)
    check.fp32(residual=residual, weight=weight)
    width = residual.shape[-1]
    rows = residual.numel() // width
    check(residual.is_contiguous() and out.is_contiguous() and out.numel() == residual.numel(),
          "contiguous residual and out of one shape")
    if branch is not None:
        check(branch.is_contiguous() and branch.numel() == residual.numel(), "bad branch")
    period = 0
    if add_rows is not None:
        check.fp32(add_rows=add_rows)
        check(add_rows.is_contiguous() and add_rows.shape[-1] == width, "bad add_rows")
        period = add_rows.numel() // width
    check(weight.numel() == width, "weight width")
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
    check = _Check("gemv", weight, x, bias, out, extra_bias)
    check(weight.dtype == torch.bfloat16 and weight.is_contiguous(), "BF16 contiguous weight")
    check(x.shape == (batch, k) and x.dtype == torch.float32 and x.is_contiguous(), "FP32 [B, K] input")
    n_extra = 0 if extra_bias is None else extra_bias.shape[0]
    expect = (n_extra, batch, n) if n_extra else (batch, n)
    check(tuple(out.shape) == expect and out.dtype == torch.float32 and out.is_contiguous(), "bad out")
    if bias is not None:
        check.fp32(bias=bias)
    if extra_bias is not None:
        check.fp32(extra_bias=extra_bias)
    L.call(
        "iris_gemv_bf16", L.ptr(weight), L.ptr(x), batch, n, k, L.ptr(bias), L.ptr(extra_bias), n_extra, L.ptr(out),
        L.ACT_SILU if in_silu else L.ACT_NONE, L.ACT_SILU if out_silu else L.ACT_NONE, L.stream(),
    )
    return out


def patchify_embed(x, patch, pix_w, pix_b, pos_x, pos_y, norm_weight, eps, patches, pixels, normed) -> None:
    """Patch matrix for the patch embedder, the embedded pixel stream and its first norm
    (src/iris_metal/model.py:188-189, 208-210)."""
    batch, channels, height, width = x.shape
    check = _Check("patchify_embed", x, patches, pixels, normed)
    check(channels in (3, 4) and x.dtype == torch.float32 and x.is_contiguous(),
          "FP32 [B, 3 or 4, H, W]")
    check.fp32(pix_w=pix_w, pix_b=pix_b, pos_x=pos_x, pos_y=pos_y, norm_weight=norm_weight)
    check(pix_w.shape == (PIXEL_WIDTH, channels), f"pixel embedder weight must be [16, {channels}]")
    n_patches = (height // patch) * (width // patch)
    check(patches.dtype == torch.bfloat16 and patches.stride(-1) == 1
          and patches.reshape(-1, patches.shape[-1]).shape[0] == batch * n_patches
          and patches.shape[-1] >= channels * patch * patch,
          "patches must be BF16 [B*L, >= C*p*p]")
    check(pixels.numel() == normed.numel() == batch * height * width * PIXEL_WIDTH
          and normed.dtype == torch.bfloat16, "bad pixel buffers")
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
    check = _Check("unpatchify_head", h, weight, bias, out)
    check(channels in (1, 3) and out.dtype == torch.float32 and out.is_contiguous(),
          "FP32 output of 1 or 3 channels")
    check(h.dtype == torch.bfloat16 and h.is_contiguous(), "BF16 pixels")
    check.fp32(weight=weight, bias=bias)
    check(weight.shape == (channels, PIXEL_WIDTH) and bias.numel() == channels, "head shape")
    L.call("iris_unpatchify_head", L.ptr(h), L.ptr(weight), L.ptr(bias), L.ptr(out), channels, batch, height, width,
           patch, L.stream())
    return out


def timestep_features(t: torch.Tensor, freqs: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``[cos | sin](t * freqs)`` (src/iris3b/nn/embeddings.py:41-45); ``out``: FP32 ``[B, 2*len(freqs)]``."""
    check = _Check("timestep_features", t, freqs, out)
    check.fp32(t=t, freqs=freqs, out=out)
    check(out.shape == (t.numel(), 2 * freqs.numel()), "bad out")
    L.call("iris_timestep_features", L.ptr(t), L.ptr(freqs), t.numel(), freqs.numel(), L.ptr(out), L.stream())
    return out


def copy_rows(src, dst, batch: int, rows: int, src_offset: int, src_batch_rows: int, dst_offset: int,
              dst_batch_rows: int) -> None:
    """``dst[b*dst_batch_rows + dst_offset + r] = src[b*src_batch_rows + src_offset + r]`` for FP32 rows."""
    check = _Check("copy_rows", src, dst)
    check.fp32(src=src, dst=dst)
    width = src.shape[-1]
    check(dst.shape[-1] == width, "widths differ")
    check(src.numel() >= batch * src_batch_rows * width and dst.numel() >= batch * dst_batch_rows * width,
          "buffers too small")
    L.call("iris_copy_rows", L.ptr(src), L.ptr(dst), batch, rows, width, src_batch_rows, src_offset, dst_batch_rows,
           dst_offset, L.stream())


def silu_add_rows(x, t, rows_per_batch: int, out) -> None:
    """``out[r] = silu(x[r] + t[r // rows_per_batch])`` (src/iris_metal/model.py:207)."""
    check = _Check("silu_add_rows", x, t, out)
    check.fp32(x=x, t=t)
    check(out.shape == x.shape and out.is_contiguous(), "bad out")
    L.call("iris_silu_add_rows", L.ptr(x), L.ptr(t), x.shape[0], rows_per_batch, x.shape[1], L.ptr(out),
           L.dtype_code(out.dtype), L.stream())


def flow_euler(x, v, sigma: float, sigma_next: float | None, x_next, clean) -> None:
    """Turbo Euler step in the reference's FP32 operation order (src/iris3b/sampling.py:129-135)."""
    check = _Check("flow_euler", x, v, x_next, clean)
    L.call("iris_flow_euler", L.ptr(x), L.ptr(v), x.numel(), float(sigma), float(sigma_next or 0.0),
           L.ptr(x_next) if sigma_next is not None else None, L.ptr(clean), L.stream())


def dpm1_update(x, v, s: float, c_x: float, c_x0: float, out) -> None:
    check = _Check("dpm1_update", x, v, out)
    L.call("iris_dpm1_update", L.ptr(x), L.ptr(v), x.numel(), float(s), float(c_x), float(c_x0), L.ptr(out),
           L.stream())


def dpm_update(x, v, x0_prev, s: float, c_x: float, c_x0: float, c_d: float, r0: float, x_next, x0_out) -> None:
    """One FlowDPMSolver step (src/iris3b/flow/solver.py:90-109): first order when ``x0_prev``
    is None, else second order; ``x0_out`` receives this step's ``x0 = x - s*v``."""
    tensors = [t for t in (x, v, x0_prev, x_next, x0_out) if t is not None]
    check = _Check("dpm_update", *tensors)
    check(all(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == x.numel() for t in tensors),
          "needs contiguous FP32 tensors of one size")
    L.call("iris_dpm_update", L.ptr(x), L.ptr(v), L.ptr(x0_prev), x.numel(), float(s), float(c_x), float(c_x0),
           float(c_d), float(r0), L.ptr(x_next), L.ptr(x0_out), L.stream())


def cfg_combine(v_uncond, v_cond, scale: float, out) -> None:
    check = _Check("cfg_combine", v_uncond, v_cond, out)
    L.call("iris_cfg_combine", L.ptr(v_uncond), L.ptr(v_cond), v_cond.numel(), float(scale), L.ptr(out), L.stream())


def clamp(x, lo: float, hi: float, out) -> None:
    check = _Check("clamp", x, out)
    L.call("iris_clamp", L.ptr(x), x.numel(), float(lo), float(hi), L.ptr(out), L.stream())
