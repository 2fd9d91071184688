"""Pins the oracle's block composition against the reference's own transformer blocks.

``tests/golden/block_golden.*`` holds the outputs of the unmodified reference
``MMDiTBlock.forward`` (src/iris3b/models/blocks/mmdit.py:84-128),
``SingleStreamBlock.forward`` / ``forward_joint``
(blocks/single_stream.py:69-143) and ``PiTBlock.forward`` (blocks/pit.py:74-93)
on seeded inputs, with this repository's synthetic weights loaded into them by
name (``tests/golden/make_block_golden.py``). The cases cover GQA with the
sigmoid gate, sandwich norm and qk-norm under ``shared_bias`` modulation (with
and without the precomputed shared cores), MHA with fused QKV under per-block
adaLN, the low-rank shared core, blocks built without a text output, a
single-stream block without text RoPE, and both PiT modulation layouts (the
"post" chunk order (scale, shift) is the one the reference warns about).
"""

import json
from dataclasses import replace
from pathlib import Path

import pytest
import torch

from iris_mi355x.config import RELEASED_TOPOLOGY, TINY
from iris_mi355x.weights import parameter_schema, synthetic_state_dict
from oracle import iris_oracle as O

GOLDEN = Path(__file__).parent / "golden"
BASES = {"released": RELEASED_TOPOLOGY, "tiny": TINY}
META = json.loads((GOLDEN / "block_golden.json").read_text())
CASES = {c["case"]: c for c in META["cases"]}


@pytest.fixture(scope="module")
def golden():
    from safetensors.torch import load_file

    return load_file(str(GOLDEN / "block_golden.safetensors"))


def _setup(case):
    cfg = replace(BASES[case["base"]], **case["overrides"])
    return cfg, synthetic_state_dict(cfg)


def _close(got, want):
    torch.testing.assert_close(got, want, rtol=2e-5, atol=2e-5)


def test_every_kind_of_block_is_covered():
    kinds = {(c["kind"], c["base"]) for c in META["cases"]}
    assert kinds == {(k, b) for k in ("mmdit", "single", "pit") for b in ("released", "tiny")}
    assert {c["case"] for c in META["cases"] if "drop" in c["case"]} == {
        "mmdit_released_drop", "mmdit_tiny_drop", "single_released_drop"}


@pytest.mark.parametrize("name", sorted(CASES))
def test_recipe_and_schema_are_the_golden_blocks_weights(name):
    """The weights the goldens were made with are regenerated bit for bit, and the
    schema's keys for the block are exactly the reference module's state_dict keys
    (which the generator loaded with ``strict=True``)."""
    import hashlib

    case = CASES[name]
    cfg, sd = _setup(case)
    recorded = case["weights"]
    for key, (shape, dig) in recorded.items():
        assert list(sd[key].shape) == shape
        assert hashlib.sha256(sd[key].contiguous().numpy().tobytes()).hexdigest() == dig, key
    prefix = (f"pixel_blocks.{case['index']}." if case["kind"] == "pit" else f"blocks.{case['index']}.")
    schema_block = {k for k in parameter_schema(cfg) if k.startswith(prefix)}
    assert schema_block == {k for k in recorded if k.startswith(prefix)}


@pytest.mark.parametrize("name", sorted(n for n, c in CASES.items() if c["kind"] == "mmdit"))
def test_oracle_mmdit_block_matches_reference(golden, name):
    case = CASES[name]
    cfg, p = _setup(case)
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith(name + "/")}
    img, txt, _ = O.rope_tables(cfg, tuple(case["grid"]), case["n_text"])
    ox, oy = O.mmdit_block(p, cfg, case["index"], g["x"], g["y"], g["cond"], img, txt)
    _close(ox, g["out_x"])
    _close(oy, g["out_y"])
    if "shared_out_x" in g:
        _close(ox, g["shared_out_x"])
        _close(oy, g["shared_out_y"])
    if not cfg.text_out(case["index"]):
        assert torch.equal(oy, g["y"])


@pytest.mark.parametrize("name", sorted(n for n, c in CASES.items() if c["kind"] == "single"))
def test_oracle_single_block_matches_reference(golden, name):
    case = CASES[name]
    cfg, p = _setup(case)
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith(name + "/")}
    n_txt = case["n_text"]
    img, txt, _ = O.rope_tables(cfg, tuple(case["grid"]), n_txt)
    tokens = torch.cat([g["y"], g["x"]], dim=1)
    out = O.single_block(p, cfg, case["index"], tokens, n_txt, g["cond"], img, txt)
    _close(out, g["out"])
    if "shared_out" in g:
        _close(out, g["shared_out"])
    if cfg.text_out(case["index"]):
        _close(out[:, n_txt:], g["out_x"])
        _close(out[:, :n_txt], g["out_y"])
    else:
        assert out.shape[1] == g["x"].shape[1]
        _close(out, g["out_x"])


@pytest.mark.parametrize("name", sorted(n for n, c in CASES.items() if c["kind"] == "pit"))
def test_oracle_pit_block_matches_reference(golden, name):
    case = CASES[name]
    cfg, p = _setup(case)
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith(name + "/")}
    grid = tuple(case["grid"])
    _, _, pix = O.rope_tables(cfg, grid, case["n_text"])
    out = O.pit_block(p, cfg, case["index"], g["x"], g["cond"], pix, grid)
    _close(out, g["out"])


def test_a_swapped_modulation_pair_fails_the_pit_golden(golden):
    """The golden separates the two chunk orders: reading the "post" tuples in the
    "pre" naming order (shift before scale) moves the output far off tolerance."""
    case = CASES["pit_released_post"]
    cfg, p = _setup(case)
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith("pit_released_post/")}
    name = f"pixel_blocks.{case['index']}.adaln"
    hp, pp = cfg.pixel.hidden_size, cfg.pixels_per_patch
    for suffix in ("weight", "bias"):
        t = p[f"{name}.{suffix}"].reshape(pp, 4, hp, *p[f"{name}.{suffix}"].shape[1:])
        p[f"{name}.{suffix}"] = t[:, [1, 0, 3, 2]].reshape(p[f"{name}.{suffix}"].shape)
    grid = tuple(case["grid"])
    _, _, pix = O.rope_tables(cfg, grid, case["n_text"])
    out = O.pit_block(p, cfg, case["index"], g["x"], g["cond"], pix, grid)
    assert (out - g["out"]).abs().max() > 1e-2


@pytest.mark.parametrize("name,prefixes", [
    ("mmdit_released", ("modulation_cores.adaln_img", "blocks.0.adaln_img")),
    ("single_released", ("modulation_cores.adaln_img", "blocks.1.adaln")),
    ("mmdit_tiny", ("blocks.0.adaln_img",)),
])
def test_a_swapped_shift_scale_pair_fails_the_trunk_golden(golden, name, prefixes):
    """Reading the MLP branch's (shift2, scale2) in swapped order, one of the
    plausible mistakes the block goldens must catch, moves the output far off tolerance
    (per-block adaLN at the tiny width has the smallest effect, 2.3e-3)."""
    case = CASES[name]
    cfg, p = _setup(case)
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith(name + "/")}
    for prefix in prefixes:
        for suffix in ("weight", "bias"):
            key = f"{prefix}.{suffix}"
            if key in p:
                t = p[key]
                p[key] = t.reshape(6, -1, *t.shape[1:])[[0, 1, 2, 4, 3, 5]].reshape(t.shape)
    img, txt, _ = O.rope_tables(cfg, tuple(case["grid"]), case["n_text"])
    if case["kind"] == "mmdit":
        got, _ = O.mmdit_block(p, cfg, case["index"], g["x"], g["y"], g["cond"], img, txt)
        want = g["out_x"]
    else:
        got = O.single_block(p, cfg, case["index"], torch.cat([g["y"], g["x"]], 1), case["n_text"], g["cond"], img, txt)
        want = g["out"]
    assert (got - want).abs().max() > 50 * 2e-5  # fifty times the golden tolerance
