"""End-to-end parity of the HIP forward against the FP32 CPU oracle.

Bar (from the north-star spec): predicted-flow cosine >= 0.999 and max relative error
(max |got - want| / max |want|) <= 2e-2, BF16 MFMA path versus FP32 reference."""

import pytest
import torch

from iris_mi355x.config import IRIS_3B, RELEASED_TOPOLOGY
from iris_mi355x.engine import HipIris
from iris_mi355x.sampling import turbo_sample
from iris_mi355x.weights import synthetic_state_dict
from oracle import iris_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
COS_MIN, MAX_REL = 0.999, 2e-2


def metrics(got, want):
    got, want = got.float().cpu().flatten(), want.float().cpu().flatten()
    cos = torch.nn.functional.cosine_similarity(got, want, dim=0).item()
    max_rel = ((got - want).abs().max() / want.abs().max()).item()
    return cos, max_rel


def check(got, want, label=""):
    cos, max_rel = metrics(got, want)
    print(f"{label}: cosine {cos:.6f} max-rel {max_rel:.3e}", flush=True)
    assert cos >= COS_MIN and max_rel <= MAX_REL, (cos, max_rel)


@pytest.fixture(scope="module")
def released():
    cfg = RELEASED_TOPOLOGY
    sd = synthetic_state_dict(cfg)
    return cfg, sd, HipIris(cfg, sd, device=DEV)


@pytest.mark.parametrize("batch,hw", [(1, (32, 32)), (2, (32, 48)), (1, (64, 40))])
def test_released_topology_forward_matches_oracle(released, batch, hw):
    cfg, sd, engine = released
    g = torch.Generator().manual_seed(batch + hw[1])
    x = torch.randn(batch, 3, *hw, generator=g)
    t = torch.tensor([125.0, 850.0][:batch])
    text = torch.randn(batch, cfg.text_len, cfg.hidden_size, generator=g)
    want = O.forward(sd, cfg, x, t, prepared_text=text)
    xd, td, textd = x.to(DEV), t.to(DEV), text.to(DEV)
    got = engine(xd, td, textd)
    check(got, want, f"released B={batch} {hw}")
    assert torch.equal(xd.cpu(), x) and torch.equal(textd.cpu(), text)  # inputs untouched
    again = engine(xd, td, textd)
    assert torch.equal(again, got)  # deterministic


def test_released_turbo_matches_oracle_sampler(released):
    cfg, sd, engine = released
    g = torch.Generator().manual_seed(0)
    noise = torch.randn(1, 3, 32, 32, generator=g)
    text = torch.randn(1, cfg.text_len, cfg.hidden_size, generator=g)
    want = O.turbo_sample(lambda x, t: O.forward(sd, cfg, x, t, prepared_text=text), noise)
    got = turbo_sample(engine, noise.to(DEV), text.to(DEV))
    check(got, want, "released turbo")


def test_upstream_dit_surface_matches_engine(released):
    """``as_dit()`` answers the upstream ``IrisDiT`` call of the Turbo route with ``.x``."""
    cfg, sd, engine = released
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 3, 32, 32, generator=g).to(DEV)
    t = torch.tensor([938.0]).to(DEV)
    text = torch.randn(1, cfg.text_len, cfg.hidden_size, generator=g).to(DEV)
    out = engine.as_dit()(x, t, None, y_mask=None, prepared_text=text, precompute_modulation=True)
    assert torch.equal(out.x, engine(x, t, text))
    with pytest.raises(NotImplementedError):
        engine.as_dit()(x, t, torch.zeros(1, 16, 3, 64, device=DEV), y_mask=torch.ones(1, 16, device=DEV))


def test_unsupported_topology_is_rejected():
    from iris_mi355x.config import TINY

    with pytest.raises(ValueError, match="released Iris-3B topology"):
        HipIris(TINY, synthetic_state_dict(TINY), device=DEV)


@pytest.fixture(scope="module")
def iris3b_blocks():
    """Iris-3B weights for one dual block, one single block and one pixel block (full width)."""
    from dataclasses import replace

    cfg = replace(IRIS_3B, depth=2, dual_depth=1, pixel=replace(IRIS_3B.pixel, depth=1))
    sd = synthetic_state_dict(cfg, device=DEV)
    return cfg, {k: v.cpu() for k, v in sd.items()}


def test_iris3b_shallow_forward_at_256px_matches_oracle(iris3b_blocks):
    """Full-width Iris-3B (D=2560, 20/5 heads, SwiGLU 6826, PiT 1280/10) with 1 dual + 1 single
    + 1 pixel block, 256x256 input, 256 text tokens."""
    cfg, sd = iris3b_blocks
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, 3, 256, 256, generator=g)
    t = torch.tensor([500.0])
    text = torch.randn(1, 256, cfg.hidden_size, generator=g)
    torch.set_num_threads(max(1, torch.get_num_threads()))
    want = O.forward(sd, cfg, x, t, prepared_text=text)
    engine = HipIris(cfg, sd, device=DEV)
    got = engine(x.to(DEV), t.to(DEV), text.to(DEV))
    check(got, want, "iris3b shallow 256px")
