"""Benchmark: Iris-3B denoise steps/s at 1024x1024, BF16, batch 1, on one MI355X.

A step is one Turbo denoise step: the full velocity forward (24 trunk blocks + 4 pixel
blocks) plus the FP32 flow-Euler update, with inputs resident in HBM. Weights are the
seeded synthetic Iris-3B weights (drawn on the device), noise N(0, 1) from seed 0, and 256
N(0, 1) prepared text tokens (the text adapter is outside the step, as in the reference).
``value`` times the engine's default path: the forward replayed from its recorded HIP graph
(recorded during the warm-up steps), the Euler update launched after it.

Prints one JSON line. Besides the driver's fields it carries:
- ``roofline``: the MFMA GEMM kernel's achieved TFLOP/s (algorithmic 2*M*N*K of each
  launch, unpadded, over its HIP-event time on the launch stream) against the 2.5 PFLOP/s
  dense BF16 peak, from a second timed pass of the same steps launched eagerly, so that every
  GEMM launch can be bracketed by events (``eager_ms_per_step``);
- ``cpu_baseline``: the FP32 CPU oracle timed on this host on one dual, one single and one
  pixel block of the same 1024x1024 workload, composed into steps/s;
- ``turbo_4step_s``: wall seconds of a whole 4-step Turbo sample (finiteness check included);
- ``encode_text``: the once-per-prompt text adapter (12 encoder layers of 2560 per token,
  300 tokens of which 200 are real, batch 1) on the GPU, and the FP32 CPU oracle of the same
  prompt beside it (unless ``--no-cpu-baseline``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "iris-3b-metal_amd"))
sys.path.insert(0, str(ROOT))

BF16_PEAK_TFLOPS = 2500.0
HBM_PEAK_GBS = 8000.0


def step_flops(cfg, height: int, width: int, n_text: int, batch: int = 1) -> dict:
    """Algorithmic FLOPs of one forward as this engine computes it (Linear 2*M*K*N,
    attention 4*N_q*N_k*H*d; norms and elementwise not counted)."""
    p = cfg.patch_size
    L = (height // p) * (width // p)
    T, N, D = n_text, n_text + L, cfg.hidden_size
    hid = cfg.mlp_hidden
    qkvg = D + 2 * cfg.kv_heads * cfg.head_dim + D
    def lin(m, k, n):
        return 2.0 * m * k * n
    gemm = lin(L, 3 * p * p, D)
    attn = 0.0
    for i in range(cfg.depth):
        last = i == cfg.depth - 1
        if cfg.block_kind(i) == "mmdit":
            rows = [L, T]
            attn += 4.0 * N * N * D
            for m in rows:
                gemm += lin(m, D, qkvg) + lin(m, D, D) + lin(m, D, 2 * hid) + lin(m, hid, D)
        else:
            gemm += lin(N, D, qkvg)
            attn += 4.0 * N * N * D
            m = L if last else N
            gemm += lin(m, D, D) + lin(m, D, 2 * hid) + lin(m, hid, D)
    px = cfg.pixel
    pp = p * p
    for _ in range(px.depth):
        gemm += lin(L, D, 4 * pp * px.hidden_size) + lin(L, pp * px.hidden_size, px.attn_hidden_size)
        gemm += lin(L, px.attn_hidden_size, 3 * px.attn_hidden_size) + lin(L, px.attn_hidden_size, px.attn_hidden_size)
        gemm += lin(L, px.attn_hidden_size, pp * px.hidden_size)
        attn += 4.0 * L * L * px.attn_hidden_size
    return {"gemm": gemm * batch, "attention": attn * batch, "total": (gemm + attn) * batch}


class LaunchTimer:
    """Brackets every GEMM launch with HIP events on the current stream."""

    def __init__(self, cfg, hidden_pad: int):
        import torch

        self.torch = torch
        self.cfg = cfg
        self.hidden_pad = hidden_pad
        self.records: list = []
        self.enabled = False

    def flops(self, m: int, n: int, k: int, swiglu: bool) -> float:
        hid = self.cfg.mlp_hidden
        if k == self.hidden_pad:
            k = hid
        if swiglu:
            n = 2 * hid
        elif n == 3 * self.cfg.patch_size ** 2:
            pass
        return 2.0 * m * n * k

    def wrap(self, K):
        torch = self.torch
        orig_linear, orig_grouped = K.linear, K.linear_grouped
        timer = self

        def linear(x, weight, bias=None, out=None, out_dtype=torch.bfloat16, swiglu=False, silu=False):
            if not timer.enabled:
                return orig_linear(x, weight, bias, out, out_dtype, swiglu, silu)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            res = orig_linear(x, weight, bias, out, out_dtype, swiglu, silu)
            e.record()
            m = x.numel() // x.shape[-1]
            k = x.shape[-1] if x.shape[-1] != timer.patch_k else 3 * timer.cfg.patch_size ** 2
            timer.records.append((s, e, timer.flops(m, weight.shape[0], k, swiglu)))
            return res

        def linear_grouped(xs, weights, biases, outs, swiglu=False):
            if not timer.enabled:
                return orig_grouped(xs, weights, biases, outs, swiglu)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            orig_grouped(xs, weights, biases, outs, swiglu)
            e.record()
            fl = sum(timer.flops(x.numel() // x.shape[-1], w.shape[0], x.shape[-1], swiglu) for x, w in zip(xs, weights))
            timer.records.append((s, e, fl))

        K.linear, K.linear_grouped = linear, linear_grouped

    def summary(self) -> tuple[float, float, int]:
        ms = sum(s.elapsed_time(e) for s, e, _ in self.records)
        fl = sum(f for _, _, f in self.records)
        return fl, ms, len(self.records)


def cpu_baseline(height: int, width: int, n_text: int, seed: int = 0) -> dict:
    """FP32 CPU oracle on one dual, one single and one pixel block of the workload."""
    import torch
    from dataclasses import replace

    from iris_mi355x.config import IRIS_3B
    from iris_mi355x.weights import synthetic_state_dict
    from oracle import iris_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = replace(IRIS_3B, depth=2, dual_depth=1, pixel=replace(IRIS_3B.pixel, depth=1))
    sd = synthetic_state_dict(cfg, seed=seed)
    p = cfg.patch_size
    grid = (height // p, width // p)
    L, D = grid[0] * grid[1], cfg.hidden_size
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(1, L, D, generator=g)
    text = torch.randn(1, n_text, D, generator=g)
    cond = torch.randn(1, 1, D, generator=g)
    img, txt, pix = O.rope_tables(cfg, grid, n_text)
    tokens = torch.cat([text, s], dim=1)
    pixels = torch.randn(L, p * p, cfg.pixel.hidden_size, generator=g)
    cpix = torch.randn(L, D, generator=g)
    blocks = {
        "dual": lambda: O.mmdit_block(sd, cfg, 0, s, text, cond, img, txt),
        "single": lambda: O.single_block(sd, cfg, 1, tokens, n_text, cond, img, txt),
        "pixel": lambda: O.pit_block(sd, cfg, 0, pixels, cpix, pix, grid),
    }
    times = {}
    with torch.no_grad():
        for name, fn in blocks.items():  # median of 3 runs per block kind
            runs = []
            for _ in range(3):
                t0 = time.perf_counter()
                fn()
                runs.append(time.perf_counter() - t0)
            times[name] = sorted(runs)[1]
    full = IRIS_3B
    n_dual = full.dual_depth
    step_s = n_dual * times["dual"] + (full.depth - n_dual) * times["single"] + full.pixel.depth * times["pixel"]
    return {
        "value": 1.0 / step_s,
        "unit": "steps/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"FP32 oracle (torch CPU), median of 3 runs of one dual ({times['dual']:.2f}s), one single "
                   f"({times['single']:.2f}s) and one pixel block ({times['pixel']:.2f}s) at {height}x{width}, "
                   f"{n_text} text tokens, composed as {n_dual} dual + {full.depth - n_dual} single + "
                   f"{full.pixel.depth} pixel blocks per step (embedders and head not counted)"),
    }


def text_prompt(cfg, real: int = 200, seed: int = 2):
    import torch

    g = torch.Generator().manual_seed(seed)
    states = torch.randn(1, cfg.text_len, cfg.text_lap_num_layers, cfg.text_dim, generator=g)
    mask = torch.zeros(1, cfg.text_len, dtype=torch.int64)
    mask[0, :real] = 1
    return states, mask


def cpu_encode_text(cfg, text_sd: dict) -> dict:
    """The FP32 CPU oracle of the text adapter on the prompt ``text_prompt`` draws, median of 3."""
    import torch

    from oracle import iris_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    states, mask = text_prompt(cfg)
    runs = []
    with torch.no_grad():
        for _ in range(3):
            t0 = time.perf_counter()
            O.embed_text(text_sd, cfg, states, mask)
            runs.append(time.perf_counter() - t0)
    return {"ms_per_prompt": 1000.0 * sorted(runs)[1], "cores": threads, "kind": "port"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--size", type=int, default=1024)
    ap.add_argument("--text", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-turbo", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus above 1 is not supported",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from iris_mi355x import _lib
    from iris_mi355x import kernels as K
    from iris_mi355x.config import IRIS_3B
    from iris_mi355x.engine import HipIris
    from iris_mi355x.sampling import TURBO_SIGMAS, turbo_sample
    from iris_mi355x.weights import synthetic_state_dict

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = IRIS_3B
    print(f"[bench] drawing Iris-3B weights on {torch.cuda.get_device_name(dev)}", file=sys.stderr, flush=True)
    sd = synthetic_state_dict(cfg, seed=0, device=dev)
    engine = HipIris(cfg, sd, device=dev)  # graphs=True: the default path
    text_sd = None
    if not args.no_cpu_baseline:  # the adapter's weights, for its CPU oracle
        text_sd = {k: v.cpu() for k, v in sd.items() if k.startswith(("y_embedder.", "y_pos_embedding"))}
    del sd
    torch.cuda.empty_cache()

    size, n_text = args.size, args.text
    noise = torch.randn(1, 3, size, size, generator=torch.Generator().manual_seed(0)).to(dev)
    text = torch.randn(1, n_text, cfg.hidden_size, generator=torch.Generator().manual_seed(1)).to(dev)
    sig = [float(torch.tensor(s, dtype=torch.float32)) for s in TURBO_SIGMAS]
    times = [torch.full((1,), s, dtype=torch.float32).mul(1000).to(dev) for s in TURBO_SIGMAS]
    x = noise.clone()
    x_next, clean, v = torch.empty_like(x), torch.empty_like(x), torch.empty_like(x)

    timer = LaunchTimer(cfg, engine.hidden_pad)
    timer.patch_k = engine.patch_k
    timer.wrap(K)

    def step(i: int):
        nonlocal x, x_next
        j = i % len(sig)
        engine(x, times[j], text, out=v)
        nxt = sig[j + 1] if j + 1 < len(sig) else sig[0]
        K.flow_euler(x, v, sig[j], nxt, x_next, clean)
        x, x_next = x_next, x

    warmup = max(args.warmup, 1)  # the first step records the forward's HIP graph
    print("[bench] warmup", file=sys.stderr, flush=True)
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms_per_step = 1000.0 * (time.perf_counter() - t0) / args.steps
    flops = step_flops(cfg, size, size, n_text)

    # the same steps launched eagerly, every GEMM launch between HIP events (the roofline)
    engine.graphs = False
    for i in range(2):
        step(i)
    torch.cuda.synchronize()
    timer.enabled = True
    print(f"[bench] timing {args.steps} eager steps (GEMM launch events)", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    eager_ms = 1000.0 * (time.perf_counter() - t0) / args.steps
    timer.enabled = False
    engine.graphs = True
    gemm_flops, gemm_ms, gemm_launches = timer.summary()
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else 0.0

    turbo_s = None
    if not args.no_turbo:
        turbo_sample(engine, noise, text)  # first call allocates the sampler's buffers
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        turbo_sample(engine, noise, text)
        torch.cuda.synchronize()
        turbo_s = time.perf_counter() - t0

    # the once-per-prompt text adapter
    states, mask = text_prompt(cfg)
    states_d, mask_d = states.to(dev), mask.to(dev)
    engine.encode_text(states_d, mask_d)
    torch.cuda.synchronize()
    reps = 5
    t0 = time.perf_counter()
    for _ in range(reps):
        engine.encode_text(states_d, mask_d)
    torch.cuda.synchronize()
    encode = {"ms_per_prompt": 1000.0 * (time.perf_counter() - t0) / reps, "batch": 1, "tokens": cfg.text_len,
              "real_tokens": int(mask.sum()), "encoder_layers": cfg.text_lap_num_layers, "text_dim": cfg.text_dim,
              "cpu_oracle": None}
    del states_d, mask_d

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU oracle of the text adapter", file=sys.stderr, flush=True)
        encode["cpu_oracle"] = cpu_encode_text(cfg, text_sd)
        del text_sd
        print("[bench] CPU baseline (oracle, one block of each kind)", file=sys.stderr, flush=True)
        cpu = cpu_baseline(size, size, n_text)

    result = {
        "metric": "denoise steps/sec @1024^2 bf16 b=1 on 1 MI355X",
        "value": 1000.0 / ms_per_step,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) noise and text tokens, seeded N(0,0.02) weights)",
        "config": {"workload": f"Iris-3B Turbo denoise step, {size}x{size}, batch 1, {n_text} text tokens",
                   "height": size, "width": size, "batch": 1, "text_tokens": n_text, "trunk_blocks": cfg.depth,
                   "pixel_blocks": cfg.pixel.depth, "parallelism": "single GPU"},
        "step_tflop": flops["total"] / 1e12,
        "mfma_frac_end_to_end": flops["total"] / (ms_per_step * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "roofline": {"bound": "mfma", "kernel": "gemm_kernel (all GEMM launches of the step)",
                     "achieved": gemm_tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": gemm_tflops / BF16_PEAK_TFLOPS, "traffic": None,
                     "launches": gemm_launches, "avg_launch_us": 1000.0 * gemm_ms / max(gemm_launches, 1)},
        "turbo_4step_s": turbo_s,
        "eager_ms_per_step": eager_ms,
        "encode_text": encode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
