"""Downstream task engines: the oracle's depth / restoration wrappers pinned by invariants, the
task export reader, and (GPU) the HIP task engines against the oracle
(src/iris3b/downstream/depth.py:26-48, restoration.py:135-142, src/iris_metal/tasks.py:69-150)."""

import dataclasses

import pytest
import torch
import torch.nn.functional as F
import yaml

from iris_mi355x import tasks
from iris_mi355x.config import RELEASED_TOPOLOGY
from iris_mi355x.weights import save_state_dict, synthetic_state_dict
from oracle import iris_oracle as O

CFG = RELEASED_TOPOLOGY


def depth_weights(seed=0):
    return synthetic_state_dict(CFG, seed=seed, schema=tasks.task_schema(CFG, "depth"))


def empty_prompt(real=4, seed=1):
    g = torch.Generator().manual_seed(seed)
    emb = torch.randn(1, CFG.text_len, CFG.text_lap_num_layers, CFG.text_dim, generator=g)
    mask = torch.zeros(1, CFG.text_len, dtype=torch.bool)
    mask[0, :real] = True
    return {"embeddings": emb, "mask": mask}


def test_depth_schema_widens_the_embedders_and_adds_the_reducer():
    schema = tasks.task_schema(CFG, "depth")
    pp, d = CFG.patch_size ** 2, CFG.hidden_size
    assert schema["pixel.s_embedder.proj.weight"].shape == (d, 4 * pp)
    assert schema["pixel.pixel_embedder.proj.weight"].shape == (CFG.pixel.hidden_size, 4)
    assert schema["depth_reducer.weight"].shape == (1, 3, 1, 1)
    base = tasks.task_schema(CFG, "restoration")  # the plain denoiser
    assert base == tasks.parameter_schema(CFG)
    widened = {"s_embedder.proj.weight", "pixel_embedder.proj.weight"}
    assert {k for k in schema if k.startswith("pixel.")} == {f"pixel.{k}" for k in base}
    assert all(schema[f"pixel.{k}"] == spec for k, spec in base.items() if k not in widened)
    with pytest.raises(ValueError):
        tasks.task_schema(CFG, "segmentation")


def test_oracle_depth_zero_channel_is_the_sliced_three_channel_model():
    """The fourth (zero) channel sits after RGB: depth_forward with the widened embedders equals
    the reducer over the 3-channel forward with the embedders' RGB columns."""
    p = depth_weights()
    pp = CFG.patch_size ** 2
    sub = {k[6:]: v for k, v in p.items() if k.startswith("pixel.")}
    sub["s_embedder.proj.weight"] = sub["s_embedder.proj.weight"][:, : 3 * pp].contiguous()
    sub["pixel_embedder.proj.weight"] = sub["pixel_embedder.proj.weight"][:, :3].contiguous()
    g = torch.Generator().manual_seed(2)
    rgb = torch.rand(2, 3, 32, 32, generator=g) * 2 - 1
    prompt = empty_prompt()
    got = O.depth_forward(p, CFG, rgb, prompt["embeddings"], prompt["mask"])
    t = torch.full((2,), 1000.0)
    v = O.forward(sub, CFG, rgb, t, prompt["embeddings"].expand(2, -1, -1, -1), y_mask=prompt["mask"].expand(2, -1))
    want = F.conv2d(v, p["depth_reducer.weight"], p["depth_reducer.bias"])
    assert got.shape == (2, 1, 32, 32)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
    # and the zero channel really is the last one: weights on it change nothing
    p2 = dict(p)
    w = p["pixel.s_embedder.proj.weight"].clone()
    w[:, 3 * pp:] = 5.0
    p2["pixel.s_embedder.proj.weight"] = w
    torch.testing.assert_close(O.depth_forward(p2, CFG, rgb, prompt["embeddings"], prompt["mask"]), got,
                               rtol=1e-5, atol=1e-6)


def test_oracle_restore_tile_moves_by_minus_sigma_times_a_constant_flow():
    """With the pixel head zeroed and a bias b, v = b everywhere, so the restored tile is
    exactly x - sigma * b per channel (and x itself for b = 0)."""
    p = synthetic_state_dict(CFG, seed=3)
    p["final_layer.linear.weight"] = torch.zeros_like(p["final_layer.linear.weight"])
    p["final_layer.linear.bias"] = torch.tensor([0.25, -1.5, 3.0])
    g = torch.Generator().manual_seed(4)
    x = torch.rand(1, 3, 32, 32, generator=g) * 2 - 1
    prompt = empty_prompt()
    got = O.restore_tile(p, CFG, x, prompt["embeddings"], prompt["mask"], 0.5)
    assert torch.equal(got, x - 0.5 * p["final_layer.linear.bias"].view(1, 3, 1, 1).expand_as(x))
    p["final_layer.linear.bias"] = torch.zeros(3)
    assert torch.equal(O.restore_tile(p, CFG, x, prompt["embeddings"], prompt["mask"], 0.5), x)


def write_export(path, task, state, settings=None):
    raw = {"model": dataclasses.asdict(CFG), "flow": {"num_train_timesteps": 1000, "prediction": "v"},
           "task": {"name": task, **(settings or {})}}
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.yaml").write_text(yaml.safe_dump(raw))
    save_state_dict(state, path / "model.safetensors")
    prompt = empty_prompt()
    from safetensors.torch import save_file

    save_file(prompt, str(path / "empty_prompt.safetensors"))
    return prompt


def test_read_export_checks_task_name_keys_and_shapes(tmp_path):
    state = depth_weights()
    write_export(tmp_path / "depth", "depth", state)
    e = tasks.read_export(tmp_path / "depth", "depth")
    assert e.cfg == CFG and e.num_train_timesteps == 1000 and e.prediction == "v"
    assert set(e.weights) == set(state) and torch.equal(e.weights["depth_reducer.bias"], state["depth_reducer.bias"])
    assert set(e.prompt) >= {"embeddings", "mask"}
    with pytest.raises(ValueError, match="not 'restoration'"):
        tasks.read_export(tmp_path / "depth", "restoration")
    bad = dict(state)
    bad.pop("depth_reducer.weight")
    write_export(tmp_path / "bad", "depth", bad)
    with pytest.raises(ValueError, match="missing"):
        tasks.read_export(tmp_path / "bad", "depth")
    narrow = dict(state, **{"pixel.pixel_embedder.proj.weight": torch.zeros(CFG.pixel.hidden_size, 3)})
    write_export(tmp_path / "narrow", "depth", narrow)
    with pytest.raises(ValueError, match="shape"):
        tasks.read_export(tmp_path / "narrow", "depth")


def test_prefixed_view():
    view = tasks.Prefixed({"pixel.a": torch.ones(1), "b": torch.zeros(1)}, "pixel.")
    assert list(view) == ["a"] and "a" in view and "b" not in view and len(view) == 1
    assert torch.equal(view["a"], torch.ones(1))


# -- GPU: the HIP task engines against the oracle ----------------------------------------------
def _check(got, want, label):
    from parity import check

    check(got, want, label)


@pytest.mark.gpu
def test_hip_depth_matches_oracle(tmp_path):
    state = depth_weights()
    prompt = write_export(tmp_path, "depth", state)
    depth = tasks.HipDepth.from_export(tmp_path, device="cuda")
    g = torch.Generator().manual_seed(5)
    rgb = torch.rand(2, 3, 32, 48, generator=g) * 2 - 1
    want = O.depth_forward(state, CFG, rgb, prompt["embeddings"], prompt["mask"])
    rgb_d = rgb.to("cuda")
    got = depth(rgb_d, None, None)
    assert got.shape == (2, 1, 32, 48)
    _check(got, want, "depth")
    assert torch.equal(rgb_d.cpu(), rgb)
    assert torch.equal(depth(rgb_d), got)  # the recorded graph replays the same result


@pytest.mark.gpu
def test_hip_restorer_matches_oracle(tmp_path):
    state = synthetic_state_dict(CFG, seed=6)
    prompt = write_export(tmp_path, "restoration", state, {"tile": 32, "sigma": 0.5})
    restorer = tasks.HipRestorer.from_export(tmp_path, device="cuda")
    assert restorer.tile == 32 and restorer.time == 500.0
    g = torch.Generator().manual_seed(7)
    x = torch.rand(1, 3, 32, 32, generator=g) * 2 - 1
    want = O.restore_tile(state, CFG, x, prompt["embeddings"], prompt["mask"], 0.5)
    xd = x.to("cuda")
    got = restorer.restore_tile(xd)
    _check(got - x.to("cuda"), want - x, "restore (update)")
    _check(got, want, "restore")
    assert torch.equal(xd.cpu(), x)
