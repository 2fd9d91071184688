"""Benchmark: Iris-3B denoise steps/s at 1024x1024, BF16, batch 1, on one MI355X.

A step is one Turbo denoise step: the full velocity forward (24 trunk blocks + 4 pixel
blocks) plus the FP32 flow-Euler update, with inputs resident in HBM. Weights are the
seeded synthetic Iris-3B weights (drawn on the device), noise N(0, 1) from seed 0, and 256
N(0, 1) prepared text tokens (the text adapter is outside the step, as in the reference).
``value`` times the engine's default path: the forward replayed from its recorded HIP graph
(recorded during the warm-up steps), the Euler update launched after it.

Prints one JSON line. Besides the driver's fields it carries:
- ``roofline``: the dominant kernel, the trunk's SwiGLU w1/w3 GEMM (``gemm_w4h_kernel`` with the
  SwiGLU epilogue, M x 2*6826 x 2560 per block), from a second timed pass of the same steps
  launched eagerly so that every GEMM launch can be bracketed by HIP events on its stream
  (``eager_ms_per_step``): ``achieved`` = algorithmic 2*M*N*K (unpadded) over the launches'
  event time, against the 2.5 PFLOP/s dense BF16 peak; ``traffic`` = HBM bytes per launch of
  that kernel from the committed counter summary
  ``profiles/gemm_swiglu_4352x13696x2560_traffic.txt`` (null when it is absent);
  ``gemm_all`` the same figures over every GEMM launch of the step, ``attention`` and
  ``attention_pixel`` over the trunk's and the pixel stage's attention launches (4*N^2*H*128),
  each with its HBM bytes per launch from ``profiles/attention_traffic_4352_4096.txt``;
- ``cpu_baseline``: the FP32 CPU oracle timed on this host on one whole 4-step Turbo sample of
  the same workload (four full forwards and Euler updates, ~100 s on 16 cores), each forward
  timed inside it; ``value`` is one step at the median of the four forwards
  (``--cpu-step-only``: one forward plus its update instead);
- ``turbo_4step_s``: wall seconds of a whole 4-step Turbo sample (finiteness check included),
  and ``cpu_turbo_4step_s`` beside it (the CPU sample's own wall time; with
  ``--cpu-step-only`` four times the timed step, marked as not measured);
- ``fused_ops``: the row kernels' bandwidth microbenchmark at [1, 4352, 2560] BF16 (achieved
  GB/s on algorithmic bytes, buffers rotated past the Infinity Cache, calls back to back in a
  replayed HIP graph as in the step; ``us_eager``: eager launches with their host gaps);
- ``single_block``: one single-stream block at 1024x1024 (4352 joint tokens) on its own,
  algorithmic TFLOP over its HIP-event time against the BF16 peak;
- ``guided``: 20 first-order guided steps (scale 3.0) over two prompts, a batch of four
  forwards per step (conditional N(0,1) tokens, zero unconditional tokens);
- ``pcie_inclusive``: the forward with the image and text tokens in pinned host memory, copied in
  and the velocity copied out around each call (never ``value``, which starts in HBM);
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
        # q | k | v, then the attention's output projection folded into expand (one GEMM)
        gemm += lin(L, px.attn_hidden_size, 3 * px.attn_hidden_size)
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
        self.attention: list = []  # (start, end, flop, query heads) per attention launch
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

        def linear(x, weight, bias=None, out=None, out_dtype=torch.bfloat16, swiglu=False, silu=False, **kw):
            if not timer.enabled:
                return orig_linear(x, weight, bias, out, out_dtype, swiglu, silu, **kw)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            res = orig_linear(x, weight, bias, out, out_dtype, swiglu, silu, **kw)
            e.record()
            m = x.numel() // x.shape[-1]
            k = x.shape[-1] if x.shape[-1] != timer.patch_k else 3 * timer.cfg.patch_size ** 2
            timer.records.append((s, e, timer.flops(m, weight.shape[0], k, swiglu), swiglu))
            return res

        def linear_grouped(xs, weights, biases, outs, swiglu=False, **kw):
            if not timer.enabled:
                return orig_grouped(xs, weights, biases, outs, swiglu, **kw)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            orig_grouped(xs, weights, biases, outs, swiglu, **kw)
            e.record()
            fl = sum(timer.flops(x.numel() // x.shape[-1], w.shape[0], x.shape[-1], swiglu) for x, w in zip(xs, weights))
            timer.records.append((s, e, fl, swiglu))

        orig_qk = K.linear_qk_rope

        def linear_qk_rope(xs, weights, outs, *args, **kwargs):
            if not timer.enabled:
                return orig_qk(xs, weights, outs, *args, **kwargs)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            orig_qk(xs, weights, outs, *args, **kwargs)
            e.record()
            fl = sum(timer.flops(x.numel() // x.shape[-1], w.shape[0], x.shape[-1], False) for x, w in zip(xs, weights))
            timer.records.append((s, e, fl, False))

        orig_attn = K.flash_attention

        def flash_attention(q, k, vt, n, out0, out1, *args, **kwargs):
            if not timer.enabled:
                return orig_attn(q, k, vt, n, out0, out1, *args, **kwargs)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            orig_attn(q, k, vt, n, out0, out1, *args, **kwargs)
            e.record()
            timer.attention.append((s, e, 4.0 * q.shape[0] * q.shape[1] * n * n * q.shape[3], q.shape[1]))

        K.linear, K.linear_grouped, K.flash_attention = linear, linear_grouped, flash_attention
        K.linear_qk_rope = linear_qk_rope

    def summary(self, swiglu_only: bool = False) -> tuple[float, float, int]:
        rows = [r for r in self.records if r[3] or not swiglu_only]
        ms = sum(s.elapsed_time(e) for s, e, _, _ in rows)
        fl = sum(f for _, _, f, _ in rows)
        return fl, ms, len(rows)


    def attention_summary(self, heads: int) -> dict:
        rows = [r for r in self.attention if r[3] == heads]
        ms = sum(s.elapsed_time(e) for s, e, _, _ in rows)
        fl = sum(f for _, _, f, _ in rows)
        tflops = fl / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
        return {"achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tflops / BF16_PEAK_TFLOPS,
                "launches": len(rows), "avg_launch_us": 1000.0 * ms / max(len(rows), 1),
                "flop_per_launch": fl / max(len(rows), 1)}


TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_swiglu_4352x13696x2560_traffic.txt"
ATTENTION_TRAFFIC_PROFILE = ROOT / "profiles" / "attention_traffic_4352_4096.txt"


def profiled_traffic(path: Path = TRAFFIC_PROFILE, key: str = "traffic_bytes_per_launch") -> float | None:
    """HBM bytes per launch recorded by a counter summary (its ``<key>:`` line), or None
    without one."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith(key + ":"):
            return float(line.split(":", 1)[1].strip().strip("`"))
    return None


def cpu_baseline(sd_cpu: dict, noise, text, turbo: bool) -> dict:
    """The FP32 CPU oracle on this host's cores. With ``turbo`` (the default): one whole 4-step
    Turbo sample of the benchmarked workload (four full forwards and their Euler updates), timed
    as a whole, each forward timed inside it; ``value`` is one step at the median of the four
    forwards. Without: one forward plus its Euler update."""
    import statistics

    import torch

    from iris_mi355x.config import IRIS_3B
    from oracle import iris_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = IRIS_3B
    noise, text = noise.float().cpu(), text.float().cpu()
    with torch.no_grad():  # warm the thread pool and allocator on a small input
        O.forward(sd_cpu, cfg, noise[:, :, :64, :64], torch.tensor([1000.0]), prepared_text=text)
        if turbo:
            forwards = []

            def model_fn(x, t):
                t1 = time.perf_counter()
                v = O.forward(sd_cpu, cfg, x, t, prepared_text=text)
                forwards.append(time.perf_counter() - t1)
                return v

            t0 = time.perf_counter()
            O.turbo_sample(model_fn, noise)
            total = time.perf_counter() - t0
            step = statistics.median(forwards) + (total - sum(forwards)) / len(forwards)
            return {"value": 1.0 / step, "unit": "steps/s", "cores": threads, "kind": "port",
                    "sample": f"one 4-step Turbo sample of the FP32 oracle (4 full forwards, 24 trunk + 4 "
                              f"pixel blocks, and their Euler updates) at {noise.shape[-2]}x{noise.shape[-1]}, "
                              f"{text.shape[1]} text tokens; value = one step at the median forward",
                    "forward_s": [round(f, 3) for f in forwards], "forward_median_s": statistics.median(forwards),
                    "turbo_4step_s": total, "turbo_measured": True}
        t0 = time.perf_counter()
        v = O.forward(sd_cpu, cfg, noise, torch.tensor([1000.0]), prepared_text=text)
        sigma, sigma_next = 1.0, 0.938
        clean = noise - sigma * v
        _ = (1 - sigma_next) * clean + sigma_next * (noise - (1 - sigma) * clean) / sigma
        step_s = time.perf_counter() - t0
    return {"value": 1.0 / step_s, "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"one Turbo step of the FP32 oracle (full forward, 24 trunk + 4 pixel blocks, and "
                      f"the Euler update) at {noise.shape[-2]}x{noise.shape[-1]}, {text.shape[1]} text tokens",
            "forward_s": [round(step_s, 3)], "forward_median_s": step_s,
            "turbo_4step_s": 4.0 * step_s, "turbo_measured": False}


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


def single_block_leg(engine, cfg, text, dev, reps: int = 10) -> dict:
    """One single-stream block (the first, index ``dual_depth``) at 1024x1024 on its own: the
    block's kernels re-run in place on the engine's workspace, timed by HIP events."""
    import torch

    from iris_mi355x import kernels as K

    g = torch.Generator(device=dev).manual_seed(3)
    grid = (64, 64)
    x = torch.randn(1, grid[0] * grid[1], cfg.hidden_size, generator=g, device=dev)
    t = torch.full((1,), 700.0, device=dev)
    index = cfg.dual_depth
    engine.block_forward(index, x, text, t, grid)
    for _ in range(2):
        engine.run_block()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        engine.run_block()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    n, d, hid = text.shape[1] + x.shape[1], cfg.hidden_size, cfg.mlp_hidden
    qkvg = 2 * d + 2 * cfg.kv_heads * cfg.head_dim
    flop = 2.0 * n * d * (qkvg + d + 2 * hid) + 2.0 * n * hid * d + 4.0 * n * n * d
    del K
    return {"block": index, "tokens": n, "ms": ms, "tflop": flop / 1e12,
            "achieved_tflops": flop / (ms * 1e-3) / 1e12, "mfma_frac": flop / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}


def guided_leg(engine, cfg, dev, size: int, n_text: int) -> dict:
    """20 first-order guided steps, scale 3.0, two prompts: a batch of four forwards per step."""
    import torch

    from iris_mi355x.sampling import dpm1_sample

    g = torch.Generator(device=dev).manual_seed(5)
    z = torch.randn(2, 3, size, size, generator=g, device=dev)
    cond = torch.randn(2, n_text, cfg.hidden_size, generator=g, device=dev)
    uncond = torch.zeros_like(cond)
    dpm1_sample(engine, z, cond, uncond, steps=2, cfg_scale=3.0)  # records the batch-4 graph
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dpm1_sample(engine, z, cond, uncond, steps=20, cfg_scale=3.0)
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    step_tflop = step_flops(cfg, size, size, n_text, batch=4)["total"] / 1e12
    return {"steps": 20, "prompts": 2, "batch": 4, "cfg_scale": 3.0, "s": total, "steps_per_s": 20 / total,
            "step_tflop": step_tflop, "mfma_frac": step_tflop * 20 / total / BF16_PEAK_TFLOPS}


def host_buffer_leg(engine, noise, text, t, reps: int = 20) -> dict:
    """The forward with the caller's tensors in host memory: the image and text tokens copied in
    and the velocity copied out over PCIe (pinned buffers) around each call. Not the headline
    value, which starts from inputs resident in HBM (as the reference's engine takes tensors that
    are already on its device)."""
    import torch

    dev = noise.device
    x_h, text_h = noise.cpu().pin_memory(), text.cpu().pin_memory()
    v_h = torch.empty_like(x_h).pin_memory()

    def call():
        v = engine(x_h.to(dev, non_blocking=True), t, text_h.to(dev, non_blocking=True))
        v_h.copy_(v, non_blocking=True)

    call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        call()
    torch.cuda.synchronize()
    ms = 1000.0 * (time.perf_counter() - t0) / reps
    return {"ms_per_forward": ms, "forwards_per_s": 1000.0 / ms, "reps": reps,
            "bytes_in": x_h.numel() * 4 + text_h.numel() * 4, "bytes_out": v_h.numel() * 4}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--size", type=int, default=1024)
    ap.add_argument("--text", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-step-only", action="store_true",
                    help="time one CPU forward step instead of a whole 4-step Turbo sample")
    ap.add_argument("--no-turbo", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip the fused-op, single-block and guided legs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; --gpus above 1 is not supported",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from iris_mi355x import _lib
    from iris_mi355x import kernels as K
    from iris_mi355x.config import IRIS_3B
    from iris_mi355x.engine import HipIris
    from iris_mi355x.sampling import TURBO_SIGMAS, turbo_sample
    from iris_mi355x.weights import synthetic_state_dict

    def say(msg: str) -> None:
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = IRIS_3B
    say(f"drawing Iris-3B weights on {torch.cuda.get_device_name(dev)}")
    sd = synthetic_state_dict(cfg, seed=0, device=dev)
    engine = HipIris(cfg, sd, device=dev)  # graphs=True: the default path
    sd_cpu = None
    if not args.no_cpu_baseline:  # the same weights for the CPU oracle (12 GB of host memory)
        sd_cpu = {k: v.cpu() for k, v in sd.items()}
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
    say("warmup")
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    say(f"timing {args.steps} steps")
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
    say(f"timing {args.steps} eager steps (GEMM launch events)")
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    eager_ms = 1000.0 * (time.perf_counter() - t0) / args.steps
    timer.enabled = False
    engine.graphs = True

    def rate(swiglu_only: bool) -> dict:
        fl, ms, launches = timer.summary(swiglu_only)
        tflops = fl / (ms * 1e-3) / 1e12 if ms > 0 else 0.0
        return {"achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": tflops / BF16_PEAK_TFLOPS,
                "launches": launches, "avg_launch_us": 1000.0 * ms / max(launches, 1),
                "flop_per_launch": fl / max(launches, 1)}

    roofline = {"bound": "mfma",
                "kernel": "gemm_w4h_pair_kernel<256, 256, SwiGLU, 192, 256, SwiGLU> (trunk w1/w3, M x 13652 x 2560)",
                **rate(True), "traffic": profiled_traffic(),
                "traffic_source": TRAFFIC_PROFILE.relative_to(ROOT).as_posix() if TRAFFIC_PROFILE.exists() else None}
    gemm_all = {"kernel": "every GEMM launch of the step (gemm_w4h_kernel / _pair_kernel, incl. the q|k|v store)", **rate(False)}
    att_source = ATTENTION_TRAFFIC_PROFILE.relative_to(ROOT).as_posix() if ATTENTION_TRAFFIC_PROFILE.exists() else None
    attention = {"kernel": "flash_attn_kernel, trunk joint attention (20 query / 5 K/V heads)",
                 **timer.attention_summary(cfg.num_heads),
                 "traffic": profiled_traffic(ATTENTION_TRAFFIC_PROFILE, "traffic_bytes_per_launch_trunk"),
                 "traffic_source": att_source}
    attention_pixel = {"kernel": "flash_attn_kernel, pixel-stage attention (10 heads)",
                       **timer.attention_summary(cfg.pixel.num_heads),
                       "traffic": profiled_traffic(ATTENTION_TRAFFIC_PROFILE, "traffic_bytes_per_launch_pixel"),
                       "traffic_source": att_source}

    turbo_s = None
    if not args.no_turbo:
        turbo_sample(engine, noise, text)  # first call allocates the sampler's buffers
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        turbo_sample(engine, noise, text)
        torch.cuda.synchronize()
        turbo_s = time.perf_counter() - t0

    extras = {}
    if not args.no_extras:
        from iris_mi355x import microbench

        say("fused-op bandwidth microbenchmark")
        extras["fused_ops"] = {r["kernel"]: {"GB/s": r["GB/s"], "hbm_frac": r["hbm_frac"], "us": r["us"],
                                             "us_eager": r["us_eager"], "bytes": r["bytes"]}
                               for r in microbench.fused_ops()}
        say("single-stream block at 1024x1024")
        extras["single_block"] = single_block_leg(engine, cfg, text, dev)
        say("guided sampling, 20 steps, batch 4")
        extras["guided"] = guided_leg(engine, cfg, dev, size, n_text)
        say("forward with host-resident inputs and output (PCIe-inclusive)")
        extras["pcie_inclusive"] = host_buffer_leg(engine, noise, text, times[0])

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
    if sd_cpu is not None:
        say("CPU oracle of the text adapter")
        encode["cpu_oracle"] = cpu_encode_text(cfg, sd_cpu)
        say("CPU baseline: the FP32 oracle " + ("Turbo step" if args.cpu_step_only else "4-step Turbo sample"))
        cpu = cpu_baseline(sd_cpu, noise, text, not args.cpu_step_only)

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
        "roofline": roofline,
        "gemm_all": gemm_all,
        "attention": attention,
        "attention_pixel": attention_pixel,
        "turbo_4step_s": turbo_s,
        "cpu_turbo_4step_s": None if cpu is None else cpu["turbo_4step_s"],
        "cpu_turbo_4step_measured": None if cpu is None else cpu["turbo_measured"],
        "eager_ms_per_step": eager_ms,
        **extras,
        "encode_text": encode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
