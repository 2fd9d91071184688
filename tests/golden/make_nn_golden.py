"""Write layer-level golden vectors by running the reference's own ``iris3b.nn`` package.

Run in the development container only (it reads the reference checkout):

    python tests/golden/make_nn_golden.py [--reference /root/reference]

``iris3b.nn`` imports with torch alone, unmodified; nothing is stubbed. The
model-level modules (``iris3b.models``) need omegaconf, which is not installed,
so they are not imported. Weights come from this repository's own seeded
recipe (N(0, 0.02) weights, 1 + N(0, 0.02) gains) and are loaded into the
reference modules with ``load_state_dict``; inputs are seeded N(0, 1). Output:
``nn_golden.safetensors`` beside this script, holding for each case its
weights, inputs and the reference's outputs, plus ``nn_golden.json`` with the
case list and provenance.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent


def _seeded_state(module: torch.nn.Module, gen: torch.Generator) -> dict[str, torch.Tensor]:
    """Sorted keys; 1-D RMSNorm gains get 1 + N(0, 0.02), everything else N(0, 0.02)."""
    gains = {
        f"{prefix}.weight".lstrip(".")
        for prefix, sub in module.named_modules()
        if type(sub).__name__ == "RMSNorm"
    }
    state = {}
    for name, value in sorted(module.state_dict().items()):
        t = torch.randn(value.shape, generator=gen)
        state[name] = 1.0 + 0.02 * t if name in gains else 0.02 * t
    return state


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, str(Path(args.reference) / "src"))
    from iris3b.nn import attention as ref_attention
    from iris3b.nn import embeddings as ref_emb
    from iris3b.nn import mlp as ref_mlp
    from iris3b.nn import modulation as ref_mod
    from iris3b.nn import rope as ref_rope
    from iris3b.nn.norms import RMSNorm

    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(1234)
    out: dict[str, torch.Tensor] = {}
    cases = []

    def put(case: str, **tensors: torch.Tensor) -> None:
        for k, v in tensors.items():
            out[f"{case}/{k}"] = v.detach().contiguous().clone()

    def put_state(case: str, module: torch.nn.Module) -> None:
        state = _seeded_state(module, gen)
        module.load_state_dict(state)
        for k, v in state.items():
            out[f"{case}/w/{k}"] = v.contiguous()

    with torch.no_grad():
        # rotary tables
        for name, kw in {
            "rope2d_iso": dict(head_dim=128, height=6, width=4, aspect="isotropic"),
            "rope2d_square": dict(head_dim=64, height=4, width=6, aspect="square"),
            "rope2d_frame": dict(head_dim=64, height=4, width=6, frame_pairs=2, frame_index=1),
        }.items():
            cis = ref_rope.rope_2d(**kw)
            put(name, real=cis.real, imag=cis.imag)
            cases.append({"case": name, "fn": "rope_2d", "kwargs": kw})
        cis = ref_rope.rope_1d(128, 9)
        put("rope1d", real=cis.real, imag=cis.imag)
        cases.append({"case": "rope1d", "fn": "rope_1d", "kwargs": {"head_dim": 128, "length": 9}})
        q, k = torch.randn(2, 24, 3, 128, generator=gen), torch.randn(2, 24, 3, 128, generator=gen)
        qr, kr = ref_rope.apply_rope(q, k, ref_rope.rope_2d(128, 6, 4, aspect="isotropic"))
        put("apply_rope", q=q, k=k, q_out=qr, k_out=kr)
        cases.append({"case": "apply_rope", "fn": "apply_rope", "table": "rope2d_iso"})

        # norms and adaLN helpers (CPU eager expressions)
        normm = RMSNorm(48)
        put_state("rmsnorm", normm)
        x = torch.randn(3, 5, 48, generator=gen) * 3
        put("rmsnorm", x=x, y=normm(x))
        cases.append({"case": "rmsnorm", "fn": "RMSNorm", "eps": 1e-6})
        shift, scale, gate = (torch.randn(3, 1, 48, generator=gen) * 0.3 for _ in range(3))
        branch = torch.randn(3, 5, 48, generator=gen)
        put(
            "adaln_tails",
            x=x, shift=shift, scale=scale, gate=gate, branch=branch,
            norm_modulate=ref_mod.norm_modulate(normm, x, shift, scale),
            gated_norm_residual=ref_mod.gated_norm_residual(x, gate, normm, branch),
            modulated_residual=ref_mod.modulated_residual(x, branch, shift, scale),
        )
        cases.append({"case": "adaln_tails", "fn": "norm_modulate/gated_norm_residual/modulated_residual", "norm": "rmsnorm"})

        # MLPs
        sw = ref_mlp.SwiGLU(48, 4.0)
        put_state("swiglu", sw)
        xs = torch.randn(2, 7, 48, generator=gen)
        put("swiglu", x=xs, y=sw(xs))
        cases.append({"case": "swiglu", "fn": "SwiGLU", "dim": 48})
        ge = ref_mlp.GeluMLP(16, 4.0)
        put_state("gelu_mlp", ge)
        xg = torch.randn(2, 7, 16, generator=gen)
        put("gelu_mlp", x=xg, y=ge(xg))
        cases.append({"case": "gelu_mlp", "fn": "GeluMLP", "dim": 16})

        # attention modules
        sa = ref_attention.SelfAttention(128, 1, qk_norm=True)
        put_state("self_attention", sa)
        xa = torch.randn(2, 24, 128, generator=gen)
        rope = ref_rope.rope_2d(128, 6, 4, aspect="isotropic")
        put("self_attention", x=xa, y=sa(xa, rope=rope))
        cases.append({"case": "self_attention", "fn": "SelfAttention", "dim": 128, "heads": 1, "table": "rope2d_iso"})

        ja = ref_attention.JointAttention(64, 4, qk_norm=True, num_kv_heads=2)
        put_state("joint_attention", ja)
        xj = torch.randn(2, 24, 64, generator=gen)
        yj = torch.randn(2, 9, 64, generator=gen)
        gx = torch.sigmoid(torch.randn(2, 24, 64, generator=gen))
        gy = torch.sigmoid(torch.randn(2, 9, 64, generator=gen))
        ox, oy = ja(xj, yj, ref_rope.rope_2d(16, 6, 4, aspect="isotropic"), ref_rope.rope_1d(16, 9), gate_x=gx, gate_y=gy)
        put("joint_attention", x=xj, y=yj, gate_x=gx, gate_y=gy, out_x=ox, out_y=oy)
        cases.append({"case": "joint_attention", "fn": "JointAttention", "dim": 64, "heads": 4, "kv_heads": 2,
                      "tables": ["rope_2d(16, 6, 4, isotropic)", "rope_1d(16, 9)"]})

        # embedders
        te = ref_emb.TimestepEmbedder(64, max_period=10.0)
        put_state("timestep", te)
        t = torch.tensor([0.0, 125.0, 500.0, 1000.0])
        put("timestep", t=t, y=te(t))
        cases.append({"case": "timestep", "fn": "TimestepEmbedder", "hidden": 64})

        pe = ref_emb.PixelEmbedder(3, 16, 4)
        put_state("pixel_embed", pe)
        xp = torch.randn(2, 3, 8, 12, generator=gen)
        put("pixel_embed", x=xp, y=pe(xp))
        cases.append({"case": "pixel_embed", "fn": "PixelEmbedder", "hidden": 16, "patch": 4})
        put("sincos", y=ref_emb.sincos_pos_embed_2d(16, 8, 12))
        cases.append({"case": "sincos", "fn": "sincos_pos_embed_2d", "dim": 16, "height": 8, "width": 12})

        lin = ref_emb.TextEmbedder(32, 64)
        put_state("text_linear", lin)
        yl = torch.randn(2, 16, 32, generator=gen)
        put("text_linear", y_in=yl, y=lin(yl))
        cases.append({"case": "text_linear", "fn": "TextEmbedder", "text_dim": 32, "hidden": 64})

        mask = torch.zeros(2, 16, dtype=torch.long)
        mask[0, :5] = 1
        mask[1, :11] = 1
        tt = ref_emb.TransformerTextEmbedder(32, 128, num_heads=1, qk_norm=True)
        put_state("text_blocks2", tt)
        yt = torch.randn(2, 16, 32, generator=gen)
        put("text_blocks2", y_in=yt, mask=mask, y=tt(yt, mask))
        cases.append({"case": "text_blocks2", "fn": "TransformerTextEmbedder", "text_dim": 32, "hidden": 128, "heads": 1})

        lw = ref_emb.LayerwiseTextEmbedder(32, 128, num_layers=3, layer_num_heads=4, refiner_num_heads=1)
        put_state("text_lap", lw)
        yw = torch.randn(2, 16, 3, 32, generator=gen) * mask[:, :, None, None]
        put("text_lap", y_in=yw, mask=mask, y=lw(yw, mask))
        cases.append({"case": "text_lap", "fn": "LayerwiseTextEmbedder", "text_dim": 32, "hidden": 128,
                      "layers": 3, "layer_heads": 4, "heads": 1})

        core = torch.nn.Linear(64, 384)
        sb = ref_mod.SharedCoreBias(64, core)
        sl = ref_mod.SharedCoreModulation(64, 8, core)
        put_state("shared_core", core)
        put_state("shared_bias", sb)
        put_state("shared_lowrank", sl)
        c = torch.randn(2, 1, 64, generator=gen)
        put("shared_core", cond=c, bias_out=sb(c), lowrank_out=sl(c))
        cases.append({"case": "shared_core", "fn": "SharedCoreBias/SharedCoreModulation", "dim": 64, "rank": 8})

    from safetensors.torch import save_file

    save_file(out, str(HERE / "nn_golden.safetensors"))
    (HERE / "nn_golden.json").write_text(
        json.dumps(
            {
                "source": "iris3b.nn (reference src/iris3b/nn/*.py), imported unmodified",
                "torch": torch.__version__,
                "weights": "seeded N(0,0.02); norm gains 1+N(0,0.02); generator seed 1234",
                "cases": cases,
            },
            indent=1,
        )
    )
    print(f"wrote {len(out)} tensors, {len(cases)} cases")


if __name__ == "__main__":
    main()
