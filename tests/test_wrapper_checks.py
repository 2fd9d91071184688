"""Host-side argument checks of the kernel wrappers (the reference's ValueError contract,
tests/test_metal_engine.py:249-256, 296-320, 383-392): bad arguments raise before anything is
launched, with the messages the reference's tests match."""

import pytest
import torch

from iris_mi355x import kernels as K


@pytest.mark.parametrize("options", [{"col_offset": -1}, {"offset": -1}, {"heads": 0}])
def test_qk_norm_rope_rejects_invalid_pointer_offsets(options):
    """Checked before the device: the CPU tensors of the reference's test never get that far."""
    x = torch.ones(1, 2, 128)
    weight = torch.ones(128)
    cos = torch.ones(2, 64)
    kwargs = {"heads": 1, **options}
    with pytest.raises(ValueError, match="positive.*nonnegative"):
        K.qk_norm_rope(x, weight, cos, torch.zeros_like(cos), 1e-6, **kwargs)


def test_cpu_tensors_are_refused():
    with pytest.raises(ValueError, match="GPU"):
        K.pixel_rms_norm(torch.zeros(1, 1, 16), torch.ones(16), 1e-6)


@pytest.mark.gpu
def test_kernels_reject_non_fp32_gains():
    x = torch.randn(1, 4, 128, device="cuda")
    gain = torch.ones(128, device="cuda", dtype=torch.bfloat16)
    zeros = torch.zeros(1, 1, 128, device="cuda")
    with pytest.raises(ValueError, match="FP32"):
        K.rms_norm_modulate(x, gain, zeros, zeros, 1e-6, torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("parameter", ["rms_gain", "norm_gain", "next_gain", "fc1_bias", "fc2_bias"])
def test_pixel_kernels_reject_short_parameter_buffers(parameter):
    bf16 = torch.bfloat16
    pixels = torch.zeros(1, 1, 16, device="cuda", dtype=bf16)
    gain = torch.ones(16, device="cuda")
    if parameter == "rms_gain":
        with pytest.raises(ValueError, match="gain width"):
            K.pixel_rms_norm(pixels, gain[:1], 1e-6)
        return
    mods = torch.zeros(1, 1, 64, device="cuda", dtype=bf16)
    fc1 = (torch.zeros(64, 16, device="cuda"), torch.zeros(64, device="cuda"))
    fc2 = (torch.zeros(16, 64, device="cuda"), torch.zeros(16, device="cuda"))
    if parameter == "fc1_bias":
        fc1 = (fc1[0], fc1[1][:1])
    if parameter == "fc2_bias":
        fc2 = (fc2[0], fc2[1][:1])
    with pytest.raises(ValueError, match="gain width|pixel-stage widths"):
        K.pixel_mlp_(pixels, pixels.clone(), mods, gain[:1] if parameter == "norm_gain" else gain, fc1, fc2,
                     gain[:1] if parameter == "next_gain" else gain, 1e-6)
