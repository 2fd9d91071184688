"""Samplers around the velocity predictor, with their updates on the GPU.

- ``turbo_sample``: the deterministic few-step flow-Euler loop of Iris-3B Turbo
  (src/iris3b/sampling.py:98-138, sigmas of src/iris_metal/turbo.py:12). The update runs as
  one FP32 kernel per step in the reference's operation order, the time values are staged
  on the device before the loop, and the only host synchronisation is the finiteness check
  of the final sample.
- ``dpm_sample``: the multistep ``FlowDPMSolver`` of the original route (order 2 by default,
  order 1 = flow-Euler in log-SNR form) with classifier-free guidance and its interval
  (src/iris3b/flow/solver.py:36-141); ``dpm1_sample`` is its first-order form.
"""

from __future__ import annotations

import math

import torch

from . import kernels as K
from .engine import require_finite

TURBO_SIGMAS = (1.0, 0.938, 0.833, 0.625)


@torch.no_grad()
def turbo_sample(model, noise: torch.Tensor, text: torch.Tensor, sigmas=TURBO_SIGMAS,
                 num_train_timesteps: int = 1000, check=require_finite) -> torch.Tensor:
    """``model(x, t_model, text) -> v``; returns ``clean.clamp(-1, 1)`` after ``len(sigmas)`` steps."""
    dev = text.device
    x = torch.empty(noise.shape, device=dev, dtype=torch.float32)
    x.copy_(noise)  # the loop writes its two latent buffers; the caller's noise stays untouched
    batch = x.shape[0]
    # t = float32(sigma) * num_train_timesteps in FP32, as the reference's sigma tensor
    times = [torch.full((batch,), s, dtype=torch.float32) * num_train_timesteps for s in sigmas]
    times = [t.to(dev) for t in times]
    sig32 = [float(torch.tensor(s, dtype=torch.float32)) for s in sigmas]
    clean = torch.empty_like(x)
    x_next = torch.empty_like(x)
    v = torch.empty_like(x)
    for i in range(len(sigmas)):
        model(x, times[i], text, out=v)
        last = i + 1 == len(sigmas)
        K.flow_euler(x, v, sig32[i], None if last else sig32[i + 1], None if last else x_next, clean)
        if not last:
            x, x_next = x_next, x
    if check is not None:
        check(clean)
    out = torch.empty_like(clean)
    K.clamp(clean, -1.0, 1.0, out)
    return out


def time_grid(steps: int, shift: float) -> list[float]:
    """src/iris3b/flow/schedule.py:24-25 and solver.py:84-88."""
    sigma = 1.0 - torch.linspace(1.0, 0.001, steps + 1, dtype=torch.float64)
    return (shift * sigma / (1 + (shift - 1) * sigma)).flip(0).tolist()


def _lam(t: float) -> float:
    return math.inf if t <= 0.0 else math.log((1.0 - t) / t)


@torch.no_grad()
def dpm_sample(model, z: torch.Tensor, cond: torch.Tensor, uncond: torch.Tensor | None = None, steps: int = 50,
               order: int = 2, shift: float = 1.0, cfg_scale: float = 1.0,
               cfg_interval: tuple[float, float] = (0.0, 1.0), num_timesteps: int = 1000,
               check=require_finite) -> torch.Tensor:
    """``FlowDPMSolver.sample`` (src/iris3b/flow/solver.py:111-141) with v-prediction: multistep
    DPM-Solver++ of order 1 or 2 (the order ramps up over the first steps and back to 1 at the
    end), classifier-free guidance over the batch ``cat([uncond, cond])`` for the steps whose
    start time lies inside ``cfg_interval`` (solver.py:58-74). Every update is one FP32 kernel
    (``iris_dpm_update``) that also keeps the step's ``x0`` for the next one. ``check`` sees the
    final sample (the original route's ``require_finite``, src/iris_metal/pipeline.py:328)."""
    if order not in (1, 2):
        raise ValueError(f"order must be 1 or 2, got {order}")
    grid = time_grid(steps, shift)
    x = torch.empty(z.shape, device=cond.device, dtype=torch.float32)
    x.copy_(z)  # the loop writes its two latent buffers; the caller's z stays untouched
    batch = x.shape[0]
    x2 = torch.empty((2 * batch, *x.shape[1:]), device=x.device, dtype=torch.float32)
    text2 = torch.cat([uncond, cond]) if uncond is not None else None
    v = torch.empty_like(x)
    v2 = torch.empty_like(x2)
    x_next = torch.empty_like(x)
    x0s = [torch.empty_like(x), torch.empty_like(x)]  # this step's x0 and the previous one
    flat = x.numel()
    s_prev = None
    for i in range(1, steps + 1):
        s, t = grid[i - 1], grid[i]
        lo, hi = cfg_interval
        use_cfg = uncond is not None and cfg_scale != 1.0 and lo < s < hi
        rows = 2 * batch if use_cfg else batch
        t_model = torch.full((rows,), s * num_timesteps, dtype=torch.float32, device=x.device)
        if use_cfg:
            for half in (0, 1):  # x2 = cat([x, x])
                K.copy_rows(x.reshape(1, flat), x2.reshape(2, flat), 1, 1, 0, 1, half, 2)
            model(x2, t_model, text2, out=v2)
            K.cfg_combine(v2[:batch], v2[batch:], cfg_scale, v)
        else:
            model(x, t_model, cond, out=v)
        x0, x0_prev = x0s[i % 2], x0s[(i + 1) % 2]
        if min(i, order, steps + 1 - i) == 1:
            phi1 = math.expm1(-(_lam(t) - _lam(s)))
            K.dpm_update(x, v, None, s, t / s, (1.0 - t) * phi1, 0.0, 1.0, x_next, x0)
        else:  # solver.py:96-109 with (s1, x0_1) the previous step and (s0, x0_0) this one
            lam_t, lam_0, lam_1 = _lam(t), _lam(s), _lam(s_prev)
            h, h0 = lam_t - lam_0, lam_0 - lam_1
            phi1 = math.expm1(-h)
            K.dpm_update(x, v, x0_prev, s, t / s, (1.0 - t) * phi1, 0.5 * (1.0 - t) * phi1, h0 / h, x_next, x0)
        s_prev = s
        x, x_next = x_next, x
    if check is not None:
        check(x)
    return x


def dpm1_sample(model, z: torch.Tensor, cond: torch.Tensor, uncond: torch.Tensor | None = None, steps: int = 20,
                shift: float = 4.0, cfg_scale: float = 3.0, cfg_interval: tuple[float, float] = (0.0, 1.0),
                num_timesteps: int = 1000, check=require_finite) -> torch.Tensor:
    """First-order ``FlowDPMSolver.sample`` (``dpm_sample`` with ``order=1``)."""
    return dpm_sample(model, z, cond, uncond, steps=steps, order=1, shift=shift, cfg_scale=cfg_scale,
                      cfg_interval=cfg_interval, num_timesteps=num_timesteps, check=check)
