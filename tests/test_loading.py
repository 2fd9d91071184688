"""Checkpoint-directory loading: config.yaml model section, lazily read and schema-checked
model.safetensors, and the Turbo distill.yaml recipe check (src/iris_metal/loading.py:15-77,
src/iris_metal/turbo.py:16-35)."""

import dataclasses

import pytest
import torch
import yaml

from iris_mi355x import loading
from iris_mi355x.config import RELEASED_TOPOLOGY
from iris_mi355x.weights import save_state_dict, synthetic_state_dict


def _checkpoint(tmp_path, cfg=RELEASED_TOPOLOGY, state=None, model_extra=None):
    model = dataclasses.asdict(cfg)
    model.update(model_extra or {})
    raw = {"name": "exported", "model": model, "train": {"batch_size": 8}, "sample": {"steps": 50}}
    (tmp_path / "config.yaml").write_text(yaml.safe_dump(raw))
    state = synthetic_state_dict(cfg) if state is None else state
    save_state_dict(state, tmp_path / "model.safetensors")
    return state


def test_config_section_round_trips(tmp_path):
    _checkpoint(tmp_path, model_extra={"not_a_model_key": 3})
    assert loading.load_config(tmp_path) == RELEASED_TOPOLOGY
    cfg = loading.load_config(tmp_path, overrides={"norm_eps": 1e-5, "pixel": {"depth": 1}})
    assert cfg.norm_eps == 1e-5 and cfg.pixel.depth == 1
    assert cfg.pixel.hidden_size == RELEASED_TOPOLOGY.pixel.hidden_size


def test_weights_are_read_lazily_and_match(tmp_path):
    state = _checkpoint(tmp_path)
    weights = loading.open_weights(tmp_path, RELEASED_TOPOLOGY)
    assert set(weights) == set(state) and len(weights) == len(state)
    for name in list(state)[:20]:
        assert weights.shape(name) == tuple(state[name].shape)
        assert torch.equal(weights[name], state[name])
    with pytest.raises(KeyError):
        weights["no.such.key"]


def test_mismatched_checkpoints_are_rejected(tmp_path):
    state = synthetic_state_dict(RELEASED_TOPOLOGY)
    name = sorted(state)[3]
    missing = {k: v for k, v in state.items() if k != name}
    _checkpoint(tmp_path, state=missing)
    with pytest.raises(ValueError, match="missing"):
        loading.open_weights(tmp_path, RELEASED_TOPOLOGY)
    extra = dict(state, **{"extra.weight": torch.zeros(2)})
    _checkpoint(tmp_path, state=extra)
    with pytest.raises(ValueError, match="unexpected"):
        loading.open_weights(tmp_path, RELEASED_TOPOLOGY)
    assert "extra.weight" in loading.open_weights(tmp_path, RELEASED_TOPOLOGY, strict=False)
    reshaped = dict(state, **{name: state[name].reshape(-1)[: state[name].numel() - 1].clone()})
    _checkpoint(tmp_path, state=reshaped)
    with pytest.raises(ValueError, match="shape"):
        loading.open_weights(tmp_path, RELEASED_TOPOLOGY)


def test_turbo_recipe_check(tmp_path):
    assert loading.load_turbo_sigmas(tmp_path) is None
    official = {"dmd": {"method": "tdm", "deterministic": True, "sigmas": [1.0, 0.938, 0.833, 0.625]}}
    (tmp_path / "distill.yaml").write_text(yaml.safe_dump(official))
    assert loading.load_turbo_sigmas(tmp_path) == (1.0, 0.938, 0.833, 0.625)
    for bad in (
        {"dmd": {**official["dmd"], "sigmas": [1.0, 0.9, 0.8, 0.6]}},
        {"dmd": {**official["dmd"], "sigmas": [True, 0.938, 0.833, 0.625]}},
        {"dmd": {**official["dmd"], "deterministic": False}},
        {"dmd": {**official["dmd"], "method": "dmd2"}},
        {"dmd": [1, 2]},
        {"other": 1},
    ):
        (tmp_path / "distill.yaml").write_text(yaml.safe_dump(bad))
        with pytest.raises(ValueError, match="official"):
            loading.load_turbo_sigmas(tmp_path)


@pytest.mark.gpu
def test_engine_from_checkpoint_matches_engine_from_state_dict(tmp_path):
    from iris_mi355x.engine import HipIris

    state = _checkpoint(tmp_path)
    engine = loading.load_engine(tmp_path, device="cuda")
    direct = HipIris(RELEASED_TOPOLOGY, state, device="cuda")
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, 3, 32, 32, generator=g).cuda()
    t = torch.tensor([500.0]).cuda()
    text = torch.randn(1, RELEASED_TOPOLOGY.text_len, RELEASED_TOPOLOGY.hidden_size, generator=g).cuda()
    assert torch.equal(engine(x, t, text), direct(x, t, text))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_engine_from_checkpoint_matches_oracle(tmp_path, dtype):
    """``load_engine`` on an FP32 and on a BF16 ``model.safetensors`` (the released Turbo
    checkpoint is BF16) against the FP32 oracle over that file's own tensors, text through the
    adapter (src/iris_metal/loading.py:20-77: Linear weights at the engine's BF16, every other
    tensor widened to FP32)."""
    from parity import check
    from safetensors.torch import load_file

    from oracle import iris_oracle as O

    cfg = RELEASED_TOPOLOGY
    state = {k: v.to(dtype) for k, v in synthetic_state_dict(cfg, seed=9).items()}
    _checkpoint(tmp_path, state=state)
    engine = loading.load_engine(tmp_path, device="cuda")
    file_tensors = {k: v.float() for k, v in load_file(str(tmp_path / "model.safetensors")).items()}
    assert all(v.dtype == dtype for v in load_file(str(tmp_path / "model.safetensors")).values())
    g = torch.Generator().manual_seed(10)
    x = torch.randn(2, 3, 32, 48, generator=g)
    t = torch.tensor([1000.0, 625.0])
    states = torch.randn(2, cfg.text_len, cfg.text_lap_num_layers, cfg.text_dim, generator=g)
    mask = torch.zeros(2, cfg.text_len, dtype=torch.int64)
    mask[0, :9], mask[1, :] = 1, 1
    want = O.forward(file_tensors, cfg, x, t, y=states, y_mask=mask)
    got = engine(x.cuda(), t.cuda(), engine.encode_text(states.cuda(), mask.cuda())).cpu()
    check(got, want, f"checkpoint {dtype}")
