"""The end-to-end parity bar shared by the GPU forward tests.

Predicted flow against the FP32 oracle: cosine similarity >= 0.999 and max relative error
(max |got - want| / max |want|) <= 2e-2. Both are evaluated in float64: in FP32 the cosine
of two 10^7-element tensors carries rounding errors of order 1e-3, the size of the bar.
"""

import torch

COS_MIN, MAX_REL = 0.999, 2e-2


def metrics(got: torch.Tensor, want: torch.Tensor) -> tuple[float, float]:
    got = got.detach().cpu().double().flatten()
    want = want.detach().cpu().double().flatten()
    cos = (got @ want / (got.norm() * want.norm())).item()
    max_rel = ((got - want).abs().max() / want.abs().max()).item()
    return cos, max_rel


def check(got: torch.Tensor, want: torch.Tensor, label: str = "") -> tuple[float, float]:
    cos, max_rel = metrics(got, want)
    print(f"{label}: cosine {cos:.7f} max-rel {max_rel:.3e}", flush=True)
    assert cos >= COS_MIN and max_rel <= MAX_REL, (label, cos, max_rel)
    return cos, max_rel
