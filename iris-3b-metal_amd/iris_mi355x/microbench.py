"""Kernel microbenchmarks of libiris_hip.so (one GPU), also used as rocprofv3 drivers.

    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench fused-ops
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench gemm 4352 6400 2560 [--swiglu] [--rotate 6]
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench attention 1 20 5 4352 [--variant 4]
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench pixel-mlp [1048576]
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench copy 1
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench encode-text 1 200
    PYTHONPATH=iris-3b-metal_amd python -m iris_mi355x.microbench vendor

``vendor`` times the vendor libraries at the step's shapes for comparison (not the library of
this package): torch's BF16 ``linear`` (hipBLASLt) at the five GEMM shapes of the denoise step,
and torch's scaled-dot-product attention at the trunk attention shape (20 heads, K/V expanded).

``fused-ops`` is the bandwidth microbenchmark of the row kernels at the single-stream block
shape [1, 4352, 2560] BF16: RMSNorm + adaLN modulate, per-head qk-RMSNorm + 2-D RoPE for Q
(20 heads) and K (5 heads), and the post-norm gated residual. Inputs are N(0, 1), modulation
vectors N(0, 0.1), gains 1 + N(0, 0.02); each timed call uses the next of several buffer sets
whose total exceeds the 256 MB Infinity Cache, and GB/s counts the algorithmic bytes (every
input read once, every output written once). ``us`` is per call with the calls recorded in one
HIP graph and replayed (back to back, as in the denoise step's graph), ``us_eager`` per call of
eager launches (HIP events on the launch stream; includes the host's launch gaps).
"""

from __future__ import annotations

import argparse
import json

import torch

from . import _lib
from . import kernels as K
from . import tables

HBM_GBS = 8000.0
MFMA_TFLOPS = 2500.0


def _time(fn, iters: int, warmup: int = 3) -> float:
    """Average milliseconds per call of ``fn(i)`` over ``iters`` calls (HIP events)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def _time_graph(fn, iters: int, replays: int = 3) -> float:
    """Average milliseconds per call of ``fn(i)`` with ``iters`` calls recorded in one HIP graph
    and the graph replayed (HIP events around each replay, the fastest replay kept): back-to-back
    kernels as the denoise step runs them, without the host's launch gaps between eager calls."""
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            fn(i)
    best = None
    for _ in range(replays):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / iters
        best = ms if best is None else min(best, ms)
    del graph
    return best


def _sets(nbytes_per_set: int, floor: int = 4, cache_bytes: int = 256 << 20) -> int:
    return max(floor, -(-2 * cache_bytes // nbytes_per_set))


def fused_ops(iters: int = 50) -> list[dict]:
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    n, d, heads, kv_heads, eps = 4352, 2560, 20, 5, 1e-6
    results = []

    def both(fn):
        return _time_graph(fn, iters), _time(fn, iters)

    def randn(*shape, scale=1.0, dtype=torch.bfloat16):
        return (scale * torch.randn(*shape, generator=g, device=dev)).to(dtype)

    # RMSNorm + adaLN modulate, BF16 -> BF16
    nbytes = 2 * n * d * 2
    sets = _sets(nbytes)
    xs = [randn(1, n, d) for _ in range(sets)]
    outs = [torch.empty(1, n, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    w = 1 + randn(d, scale=0.02, dtype=torch.float32)
    mods = randn(1, 1, 6 * d, scale=0.1, dtype=torch.float32)
    ms, ms_eager = both(lambda i: K.rms_norm_modulate(xs[i % sets], w, mods[..., :d], mods[..., d:2 * d], eps,
                                                      torch.bfloat16, out=outs[i % sets]))
    results.append({"kernel": "rms_norm_modulate", "shape": [1, n, d], "bytes": nbytes, "sets": sets, "us": ms * 1e3,
                    "us_eager": ms_eager * 1e3})
    del xs, outs

    # qk-RMSNorm + RoPE of Q (20 heads) and K (5 heads)
    img = tables.rope_2d_angles(128, 64, 64, 10000.0, 16.0, "isotropic")
    txt = tables.rope_1d_angles(128, 256, 10000.0)
    cos, sin = tables.cos_sin(txt, img, device=dev)
    nbytes = 2 * (n * heads * 128 * 2) + 2 * (n * kv_heads * 128 * 2) + 2 * cos.numel() * 4
    sets = _sets(nbytes)
    qs = [randn(1, n, heads * 128) for _ in range(sets)]
    ks = [randn(1, n, kv_heads * 128) for _ in range(sets)]
    qo = [torch.empty(1, heads, n, 128, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ko = [torch.empty(1, kv_heads, n, 128, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    qw, kw = 1 + randn(128, scale=0.02, dtype=torch.float32), 1 + randn(128, scale=0.02, dtype=torch.float32)

    def qk(i):
        j = i % sets
        K.qk_norm_rope(qs[j], qw, cos, sin, eps, heads, out=qo[j])
        K.qk_norm_rope(ks[j], kw, cos, sin, eps, kv_heads, out=ko[j])

    ms, ms_eager = both(qk)
    results.append({"kernel": "qk_norm_rope (Q + K)", "shape": [1, n, (heads + kv_heads) * 128], "bytes": nbytes,
                    "sets": sets, "us": ms * 1e3, "us_eager": ms_eager * 1e3})
    del qs, ks, qo, ko

    # post-norm gated residual, FP32 residual in place, BF16 branch
    nbytes = 2 * n * d * 4 + n * d * 2
    sets = _sets(nbytes)
    res = [randn(1, n, d, dtype=torch.float32) for _ in range(sets)]
    br = [randn(1, n, d) for _ in range(sets)]
    ms, ms_eager = both(lambda i: K.gated_residual_rms_norm_(res[i % sets], br[i % sets], w, mods[..., 2 * d:3 * d],
                                                             eps))
    results.append({"kernel": "gated_residual_rms_norm_", "shape": [1, n, d], "bytes": nbytes, "sets": sets,
                    "us": ms * 1e3, "us_eager": ms_eager * 1e3})
    outs = [torch.empty(1, n, d, device=dev, dtype=torch.bfloat16) for _ in range(sets)]
    ms, ms_eager = both(lambda i: K.gated_residual_norm_modulate_(res[i % sets], br[i % sets], w,
                                                                  mods[..., 2 * d:3 * d], eps, w, mods[..., 3 * d:4 * d],
                                                                  mods[..., 4 * d:5 * d], outs[i % sets]))
    results.append({"kernel": "gated_residual_norm_modulate_ (fused pair)", "shape": [1, n, d],
                    "bytes": nbytes + n * d * 2, "sets": sets, "us": ms * 1e3, "us_eager": ms_eager * 1e3})
    del res, br, outs

    # reference point: a plain device copy of the same size class (44.6 MB in, 44.6 MB out)
    nbytes = 2 * n * d * 4
    sets = _sets(nbytes)
    src = [randn(n * d, dtype=torch.float32) for _ in range(sets)]
    dst = [torch.empty(n * d, device=dev) for _ in range(sets)]
    ms, ms_eager = both(lambda i: dst[i % sets].copy_(src[i % sets]))
    results.append({"kernel": "copy (torch, reference)", "shape": [n * d], "bytes": nbytes, "sets": sets,
                    "us": ms * 1e3, "us_eager": ms_eager * 1e3})
    for r in results:
        r["GB/s"] = r["bytes"] / (r["us"] * 1e-6) / 1e9
        r["hbm_frac"] = r["GB/s"] / HBM_GBS
    return results


def gemm(m: int, n: int, k: int, tile: int = -1, iters: int = 20, swiglu: bool = False, rotate: int = 1) -> dict:
    """``K.linear`` at M x N x K (BF16 in, BF16 out; with ``swiglu`` the N columns are interleaved
    w1 | w3 pairs and the output has N / 2). With ``rotate`` > 1 each call takes the next of that
    many weight copies, so with six copies of a large weight (more than the 256 MB Infinity Cache)
    every call reads its weight from HBM, as the denoise step does; one copy stays cache-resident."""
    a = torch.randn(m, k, device="cuda").to(torch.bfloat16)
    ws = [(0.02 * torch.randn(n, k, device="cuda")).to(torch.bfloat16) for _ in range(max(rotate, 1))]
    out = torch.empty(m, n // 2 if swiglu else n, device="cuda", dtype=torch.bfloat16)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        ms = _time(lambda i: K.linear(a, ws[i % len(ws)], out=out, swiglu=swiglu), iters)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"kernel": "gemm_bf16_swiglu" if swiglu else "gemm_bf16", "m": m, "n": n, "k": k, "tile": tile,
            "weight_copies": len(ws), "us": ms * 1e3, "TFLOP/s": tflops, "mfma_frac": tflops / MFMA_TFLOPS}


def pixel_mlp(n: int = 1 << 20, iters: int = 20) -> dict:
    """``K.pixel_mlp_`` over ``n`` pixels (the FP32 pixel stream of a 1024x1024 image by default):
    320 algorithmic bytes per pixel (stream read and written, branch, modulation, next input)."""
    g = torch.Generator(device="cuda").manual_seed(0)

    def randn(*shape, scale=1.0, dtype=torch.float32):
        return (scale * torch.randn(*shape, generator=g, device="cuda")).to(dtype)

    pixels = randn(n, 16)
    branch, mods = randn(n, 16, dtype=torch.bfloat16), randn(n, 64, scale=0.3, dtype=torch.bfloat16)
    gain = 1 + randn(16, scale=0.02)
    fc1 = (randn(64, 16, scale=0.3), randn(64, scale=0.1))
    fc2 = (randn(16, 64, scale=0.3), randn(16, scale=0.1))
    nxt = torch.empty(n, 16, device="cuda", dtype=torch.bfloat16)
    ms = _time(lambda i: K.pixel_mlp_(pixels, branch, mods, gain, fc1, fc2, gain, 1e-6, next_input=nxt), iters)
    nbytes = n * 320
    return {"kernel": "pixel_mlp_", "pixels": n, "bytes": nbytes, "us": ms * 1e3,
            "GB/s": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_GBS}


def attention(b: int, h: int, hkv: int, n: int, iters: int = 20, variant: int = -1) -> dict:
    """``K.flash_attention`` over ``n`` tokens; ``variant`` >= 0 forces that kernel variant (an index
    of the library's variant table, as ``iris_flash_attn_force_variant`` takes), -1 the automatic one."""
    n_pad = (n + 63) // 64 * 64
    q = torch.randn(b, h, n_pad, 128, device="cuda").to(torch.bfloat16)
    k = torch.randn(b, hkv, n_pad, 128, device="cuda").to(torch.bfloat16)
    vt = torch.randn(b, hkv, 128, n_pad, device="cuda").to(torch.bfloat16)
    out = torch.empty(b * n, h * 128, device="cuda", dtype=torch.bfloat16)
    _lib.call("iris_flash_attn_force_variant", variant)
    try:
        ms = _time(lambda i: K.flash_attention(q, k, vt, n, None, out, 0), iters)
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    tflops = 4.0 * b * n * n * h * 128 / (ms * 1e-3) / 1e12
    return {"kernel": "flash_attn", "variant": variant, "b": b, "heads": h, "kv_heads": hkv, "n": n, "us": ms * 1e3,
            "TFLOP/s": tflops,
            "mfma_frac": tflops / MFMA_TFLOPS}


def encode_text(batch: int, real: int, iters: int = 10) -> dict:
    """``HipIris.encode_text`` at full Iris-3B width (12 encoder layers of 2560, 300 tokens, the
    first ``real`` of them unmasked) on seeded synthetic weights of a two-block model."""
    from dataclasses import replace

    from .config import IRIS_3B
    from .engine import HipIris
    from .weights import synthetic_state_dict

    cfg = replace(IRIS_3B, depth=2, dual_depth=1, pixel=replace(IRIS_3B.pixel, depth=1))
    engine = HipIris(cfg, synthetic_state_dict(cfg, device="cuda"), device="cuda")
    g = torch.Generator(device="cuda").manual_seed(0)
    states = torch.randn(batch, cfg.text_len, cfg.text_lap_num_layers, cfg.text_dim, generator=g, device="cuda")
    mask = torch.zeros(batch, cfg.text_len, dtype=torch.int64, device="cuda")
    mask[:, :real] = 1
    ms = _time(lambda i: engine.encode_text(states, mask), iters)
    return {"op": "encode_text", "batch": batch, "tokens": cfg.text_len, "real": real, "ms": ms}


STEP_GEMMS = [(4352, 13696, 2560, "SwiGLU w1|w3"), (4352, 6400, 2560, "q|k|v|gate"), (4352, 2560, 2560, "proj"),
              (4352, 2560, 6848, "w2"), (4096, 16384, 2560, "pixel adaLN")]


def vendor(iters: int = 20) -> list[dict]:
    """hipBLASLt (torch BF16 ``linear``) at the step's GEMM shapes and torch SDPA at the trunk
    attention shape, HIP events on the launch stream."""
    import torch.nn.functional as F

    out = []
    for m, n, k, name in STEP_GEMMS:
        a = torch.randn(m, k, device="cuda").to(torch.bfloat16)
        w = (0.02 * torch.randn(n, k, device="cuda")).to(torch.bfloat16)
        ms = _time(lambda i: F.linear(a, w), iters)
        out.append({"op": f"torch linear ({name})", "m": m, "n": n, "k": k, "us": ms * 1e3,
                    "TFLOP/s": 2.0 * m * n * k / (ms * 1e-3) / 1e12})
    b, h, n, d = 1, 20, 4352, 128
    q, k_, v = (torch.randn(b, h, n, d, device="cuda").to(torch.bfloat16) for _ in range(3))
    ms = _time(lambda i: F.scaled_dot_product_attention(q, k_, v), iters)
    out.append({"op": "torch scaled_dot_product_attention", "b": b, "heads": h, "n": n, "us": ms * 1e3,
                "TFLOP/s": 4.0 * b * n * n * h * d / (ms * 1e-3) / 1e12})
    return out


def copy(gib: float, iters: int = 5) -> dict:
    src = torch.ones(int(gib * (1 << 28)), device="cuda", dtype=torch.float32)
    dst = torch.empty_like(src)
    ms = _time(lambda i: dst.copy_(src), iters)
    nbytes = 2 * src.numel() * 4
    return {"kernel": "copy", "bytes": nbytes, "us": ms * 1e3, "GB/s": nbytes / (ms * 1e-3) / 1e9}


def qkvg(n: int = 4352, iters: int = 20, rotate: int = 6) -> dict:
    """A single-stream block's packed q | k | v | gate projection as the step runs it
    (``K.linear_qk_rope``: the Q / K norm + RoPE and the V^T layout in the q | k | v store, the gate
    columns beside it in the same launch) over ``n`` tokens of one batch item (a multiple of 256),
    each call on the next of ``rotate`` weight copies so that every call reads its weight from HBM."""
    heads, kv_heads, d = 20, 5, 2560
    cols = (2 * heads + 2 * kv_heads) * 128
    n_pad = (n + 63) // 64 * 64
    bf16 = torch.bfloat16
    h = (0.5 * torch.randn(n, d, device="cuda")).to(bf16)
    ws = [(0.02 * torch.randn(cols, d, device="cuda")).to(bf16) for _ in range(rotate)]
    qw, kw = 1 + 0.1 * torch.randn(128, device="cuda"), 1 + 0.1 * torch.randn(128, device="cuda")
    cos, sin = torch.randn(n_pad, 64, device="cuda"), torch.randn(n_pad, 64, device="cuda")
    q = torch.empty(1, heads, n_pad, 128, device="cuda", dtype=bf16)
    k = torch.empty(1, kv_heads, n_pad, 128, device="cuda", dtype=bf16)
    vt = torch.zeros(1, kv_heads, 128, n_pad, device="cuda", dtype=bf16)
    out = torch.empty(n, cols, device="cuda", dtype=bf16)
    ms = _time(lambda i: K.linear_qk_rope([h], [ws[i % rotate]], [out], [qw], [kw], cos, sin, 1e-6, heads, kv_heads,
                                          q, k, [n], [0], vt=vt), iters)
    tflops = 2.0 * n * cols * d / (ms * 1e-3) / 1e12
    return {"kernel": "gemm_bf16_qk_rope (q|k|v|gate)", "n": n, "cols": cols, "k": d, "us": ms * 1e3,
            "TFLOP/s": tflops, "mfma_frac": tflops / MFMA_TFLOPS}


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("fused-ops")
    p = sub.add_parser("gemm")
    p.add_argument("m", type=int)
    p.add_argument("n", type=int)
    p.add_argument("k", type=int)
    p.add_argument("--tile", type=int, default=-1)
    p.add_argument("--tiles", type=str, default=None, help="comma-separated tiles, each measured in turn")
    p.add_argument("--swiglu", action="store_true")
    p.add_argument("--rotate", type=int, default=1)
    p = sub.add_parser("attention")
    for name in ("b", "h", "hkv", "n"):
        p.add_argument(name, type=int)
    p.add_argument("--variant", type=int, default=-1)
    p = sub.add_parser("qkvg")
    p.add_argument("n", type=int, nargs="?", default=4352)
    p = sub.add_parser("pixel-mlp")
    p.add_argument("pixels", type=int, nargs="?", default=1 << 20)
    p = sub.add_parser("copy")
    p.add_argument("gib", type=float, nargs="?", default=1.0)
    sub.add_parser("vendor")
    p = sub.add_parser("encode-text")
    p.add_argument("batch", type=int, nargs="?", default=1)
    p.add_argument("real", type=int, nargs="?", default=200)
    args = ap.parse_args()
    _lib.load()
    if args.cmd == "fused-ops":
        out = fused_ops()
    elif args.cmd == "gemm":
        tiles = [int(t) for t in args.tiles.split(",")] if args.tiles else [args.tile]
        out = [gemm(args.m, args.n, args.k, t, swiglu=args.swiglu, rotate=args.rotate) for t in tiles]
        out = out[0] if len(out) == 1 else out
    elif args.cmd == "attention":
        out = attention(args.b, args.h, args.hkv, args.n, variant=args.variant)
    elif args.cmd == "qkvg":
        out = qkvg(args.n)
    elif args.cmd == "pixel-mlp":
        out = pixel_mlp(args.pixels)
    elif args.cmd == "encode-text":
        out = encode_text(args.batch, args.real)
    elif args.cmd == "vendor":
        out = vendor()
    else:
        out = copy(args.gib)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
