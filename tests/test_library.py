"""CPU checks of the C ABI library: it is built, loads, and exports every declared symbol.

No kernel is launched here (there is no GPU in the build container)."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "iris_hip.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(iris_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from iris_mi355x import _lib

    if not _lib.LIBRARY.exists():
        pytest.fail("libiris_hip.so is not built: run __graft_entry__.build()")
    return _lib.load()


def test_header_declares_the_hot_path():
    names = declared()
    for required in ("iris_rms_norm_modulate", "iris_gated_residual_rms_norm", "iris_qk_norm_rope",
                     "iris_flash_attn", "iris_gemm_bf16", "iris_pixel_mlp", "iris_patchify_embed",
                     "iris_unpatchify_head", "iris_flow_euler", "iris_cfg_combine"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    from iris_mi355x import _lib

    assert sorted(_lib.exported_symbols()) == declared()


def test_abi_version(lib):
    from iris_mi355x import _lib

    assert lib.iris_abi_version() == _lib.ABI_VERSION == 3


def test_build_recipe_targets_gfx950_without_packed_fp32():
    from iris_mi355x import build

    flags = " ".join(build.HIPCC_FLAGS)
    assert "--offload-arch=gfx950" in flags
    assert "-Xclang -target-feature -Xclang -packed-fp32-ops" in flags
    assert {p.name for p in build.sources()} >= {"gemm.hip", "attention.hip", "rowops.hip", "pixel.hip"}


def test_invalid_arguments_are_rejected_before_launch(lib):
    """Host-side validation runs without touching the device (reference ValueError contract)."""
    from iris_mi355x import _lib

    with pytest.raises(ValueError, match="width"):
        _lib.call("iris_rms_norm_modulate", 1 << 20, _lib.F32, 1 << 20, _lib.BF16, 1 << 20, 1 << 20, 1 << 20,
                  4, 4, 100, 100, 1e-6, None)
    with pytest.raises(ValueError, match="k % 64"):
        _lib.call("iris_gemm_bf16", 1 << 20, 1 << 20, None, 1 << 20, _lib.BF16, 8, 8, 48, 48, 48, 8, 0, None)
    with pytest.raises(ValueError, match="power of two"):
        _lib.call("iris_flash_attn", 1 << 20, 1 << 20, 1 << 20, 1, 6, 2, 64, 64, 0, 0.1, None, 1 << 20, 768, 0,
                  64, None, None, 0, 0, 0, None)
    with pytest.raises(ValueError, match="not divisible"):
        _lib.call("iris_patchify_embed", 1 << 20, 1, 3, 30, 32, 16, 1 << 20, 768, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                  1 << 20, 1e-6, 1 << 20, _lib.F32, 1 << 20, None)
    with pytest.raises(ValueError, match="3 or 4 input channels"):
        _lib.call("iris_patchify_embed", 1 << 20, 1, 5, 32, 32, 16, 1 << 20, 1280, 1 << 20, 1 << 20, 1 << 20, 1 << 20,
                  1 << 20, 1e-6, 1 << 20, _lib.F32, 1 << 20, None)
    with pytest.raises(ValueError, match="3 or 1 output channels"):
        _lib.call("iris_unpatchify_head", 1 << 20, 1 << 20, 1 << 20, 1 << 20, 2, 1, 32, 32, 16, None)
    # the kernels address operands by 32-bit byte offsets: 2 GiB per operand is refused
    k = 8192
    with pytest.raises(ValueError, match="weight above 2 GiB"):
        _lib.call("iris_gemm_bf16", 1 << 20, 1 << 20, None, 1 << 20, _lib.BF16, 8, (1 << 30) // k, k, k, k,
                  (1 << 30) // k, 0, None)
    with pytest.raises(ValueError, match="activation above 2 GiB"):
        _lib.call("iris_gemm_bf16", 1 << 20, 1 << 20, None, 1 << 20, _lib.BF16, (1 << 30) // k, 64, k, k, k, 64, 0,
                  None)
    with pytest.raises(ValueError, match="below 2\\^23"):
        _lib.call("iris_flash_attn", 1 << 20, 1 << 20, 1 << 20, 1, 4, 1, 1 << 23, 1 << 23, 0, 0.1, None, 1 << 20,
                  512, 0, 1 << 23, None, None, 0, 0, 0, None)
