"""The BF16 GELU table of the pixel MLP kernel (csrc/gelu_bf16_table.inc): regenerated
byte for byte from its generator, and every entry checked as the BF16 nearest to a Phi(a)
with Phi from scipy's float64 ndtr (Cephes: an evaluation independent of the generator's
math.erfc, and accurate in the far negative tail, where torch's ndtr cancels); the rule the
kernel applies outside the table checked over every finite BF16."""

import importlib.util
from pathlib import Path

import torch
from scipy.special import ndtr

CSRC = Path(__file__).resolve().parents[1] / "iris-3b-metal_amd" / "iris_mi355x" / "csrc"


def _generator():
    spec = importlib.util.spec_from_file_location("gen_gelu_table", CSRC / "gen_gelu_table.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _values(bits):
    """float64 values of int BF16 bit patterns."""
    return (bits & 0xFFFF).to(torch.int16).view(torch.bfloat16).double()


def _exact_gelu(a):
    return a * torch.from_numpy(ndtr(a.numpy()))


def _nearest(result_bits, exact):
    """True where no same-sign finite BF16 neighbour of the result is closer to exact."""
    got = _values(result_bits)
    ok = torch.ones_like(exact, dtype=torch.bool)
    for step in (-1, 1):
        nb_bits = result_bits + step
        valid = ((nb_bits & 0x7F80) != 0x7F80) & ((nb_bits & 0x8000) == (result_bits & 0x8000))
        valid &= (nb_bits & 0x7FFF) != 0x7FFF  # no wrap across zero from the largest pattern
        ok &= ~(valid & ((_values(nb_bits) - exact).abs() < (got - exact).abs()))
    return ok


def test_committed_table_is_the_generator_output():
    gen = _generator()
    assert (CSRC / "gelu_bf16_table.inc").read_text() == gen.render()


def test_every_entry_is_the_nearest_bf16_of_the_exact_gelu():
    gen = _generator()
    table = torch.tensor(gen.table(), dtype=torch.int64)
    assert table.numel() == 2 * gen.PER_SIGN == 6144
    t = torch.arange(gen.PER_SIGN)
    arg_bits = torch.cat([(gen.LOW_EXPONENT << 7) + t, 0x8000 | ((gen.LOW_EXPONENT << 7) + t)])
    a = _values(arg_bits)
    assert a[0] == 2.0 ** -16 and a[gen.PER_SIGN - 1] == 256 - 1 and a[-1] == -(256 - 1)
    exact = _exact_gelu(a)
    assert torch.all(_nearest(table, exact))
    # closed forms: GELU(1) = Phi(1) = 0.8413447..., GELU(-1) = -0.1586552...; a Phi(a) -> a for a >> 0
    lookup = dict(zip(a.tolist(), _values(table).tolist()))
    assert lookup[1.0] == 0.83984375 and lookup[-1.0] == -0.158203125
    assert lookup[16.0] == 16.0 and lookup[-16.0] == 0.0  # -16 Phi(-16) ~ -1e-56 underflows
    assert lookup[2.0 ** -10] == 2.0 ** -11 and lookup[2.0 ** -16] == 2.0 ** -17  # a / 2 near zero
    assert lookup[200.0] == 200.0 and lookup[-200.0] == 0.0


def test_rule_outside_the_table_is_the_nearest_bf16():
    """|a| < 2^-16: the BF16 nearest to a / 2; |a| >= 256: a for a > 0, zero for a < 0. (The
    a / 2 rule holds up to 2^-10, the other from 16 on: checked over those wider ranges.)"""
    gen = _generator()
    bits = torch.arange(0x10000, dtype=torch.int64)
    finite = (bits & 0x7F80) != 0x7F80
    mag = bits & 0x7FFF
    outside = finite & ((mag < (117 << 7)) | (mag >= (131 << 7)))
    assert torch.all(outside | ~finite | ((mag >= (gen.LOW_EXPONENT << 7)) & (mag < (gen.LOW_EXPONENT << 7) + gen.PER_SIGN)))
    bits = bits[outside]
    a = _values(bits)
    below = (bits & 0x7FFF) < (117 << 7)
    rule = torch.where(below, a / 2, a.clamp(min=0.0))
    # the kernel rounds a / 2 (exact in FP32) to BF16 to nearest-even; float64 -> FP32 is exact here
    rule_bits = rule.float().to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
    exact = _exact_gelu(a)
    assert torch.all(_nearest(rule_bits, exact))
    assert int(outside.sum()) == 0xFF00 - 2 * 14 * 128
