"""Each HIP kernel against the FP32 CPU oracle (or an FP32 PyTorch expression of the same op)
on seeded inputs. Tolerances: FP32 outputs to FP32 rounding (summation order differs);
BF16 outputs to one BF16 rounding of the FP32 result; MFMA products to the BF16 operand
rounding they are specified with (FP32 accumulation)."""

import math

import pytest
import torch
import torch.nn.functional as F
from scipy.special import ndtr

from iris_mi355x import _lib
from iris_mi355x import kernels as K
from oracle import iris_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def gen(seed=0):
    return torch.Generator().manual_seed(seed)


def close_bf16(got, want, scale=None, floor=1e-3):
    """|got - want| within ~1.5 BF16 ulps of the magnitude (plus a floor)."""
    got, want = got.float().cpu(), want.float().cpu()
    tol = 6e-3 * want.abs() + floor * (scale if scale is not None else want.abs().max().item())
    err = (got - want).abs()
    assert torch.all(err <= tol), f"max err {err.max().item():.3e}, worst rel {(err / tol).max().item():.2f}x tol"


def close_attention(got, want, rel_l2=4e-3):
    """Attention to its BF16 rounding points: the output's relative L2 error (one BF16 rounding
    of the output is ~2^-9 / sqrt(3) = 1.1e-3; the BF16 probabilities in the P.V product add
    less, averaged over the keys) and, per element, ~1.5 BF16 ulps plus 1% of the largest
    output. A dropped or doubled 32-key tile at 4352 keys moves the output by ~9% in L2."""
    got, want = got.float().cpu(), want.float().cpu()
    err = ((got - want).norm() / want.norm()).item()
    print(f"attention rel-L2 {err:.3e}", flush=True)
    assert err <= rel_l2, f"relative L2 error {err:.3e} > {rel_l2:.1e}"
    close_bf16(got, want, floor=1e-2)


# -- rows ------------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(1, 4352, 2560), (2, 37, 256), (3, 7, 384), (2, 64, 384)])
@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
def test_rms_norm_modulate(shape, x_dtype):
    b, n, d = shape
    g = gen(1)
    x = torch.randn(shape, generator=g).to(x_dtype)
    w = 1 + 0.02 * torch.randn(d, generator=g)
    mods = 0.1 * torch.randn(b, 1, 6 * d, generator=g)
    shift, scale = mods[..., :d], mods[..., d:2 * d]  # strided chunks of one modulation vector
    want = O.modulate(O.rms_norm(x.float(), w, 1e-6), shift, scale)
    got = K.rms_norm_modulate(x.to(DEV), w.to(DEV), mods.to(DEV)[..., :d], mods.to(DEV)[..., d:2 * d], 1e-6,
                              torch.bfloat16)
    close_bf16(got, want)
    got32 = K.rms_norm_modulate(x.to(DEV), w.to(DEV), shift.to(DEV), scale.to(DEV), 1e-6, torch.float32)
    torch.testing.assert_close(got32.cpu(), want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("branch_dtype", [torch.bfloat16, torch.float32])
def test_gated_residual_rms_norm(branch_dtype):
    b, n, d = 2, 300, 2560
    g = gen(2)
    res = torch.randn(b, n, d, generator=g)
    branch = torch.randn(b, n, d, generator=g).to(branch_dtype)
    w = 1 + 0.02 * torch.randn(d, generator=g)
    gate = 0.1 * torch.randn(b, 1, d, generator=g)
    want = res + gate * O.rms_norm(branch.float(), w, 1e-6)
    r = res.to(DEV)
    out = K.gated_residual_rms_norm_(r, branch.to(DEV), w.to(DEV), gate.to(DEV), 1e-6)
    assert out.data_ptr() == r.data_ptr()
    torch.testing.assert_close(r.cpu(), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("shape", [(1, 4352, 2560), (2, 37, 256), (2, 64, 384)])
def test_gated_residual_fused_with_next_norm_modulate(shape):
    b, n, d = shape
    g = gen(22)
    res = torch.randn(b, n, d, generator=g)
    branch = torch.randn(b, n, d, generator=g).to(torch.bfloat16)
    w, w2 = 1 + 0.02 * torch.randn(d, generator=g), 1 + 0.02 * torch.randn(d, generator=g)
    mods = 0.1 * torch.randn(b, 1, 6 * d, generator=g)
    gate, shift, scale = mods[..., :d], mods[..., d:2 * d], mods[..., 2 * d:3 * d]
    new_res = res + gate * O.rms_norm(branch.float(), w, 1e-6)
    want = O.modulate(O.rms_norm(new_res, w2, 1e-6), shift, scale)
    r, md = res.to(DEV), mods.to(DEV)
    out = torch.empty(b, n, d, device=DEV, dtype=torch.bfloat16)
    K.gated_residual_norm_modulate_(r, branch.to(DEV), w.to(DEV), md[..., :d], 1e-6, w2.to(DEV), md[..., d:2 * d],
                                    md[..., 2 * d:3 * d], out)
    torch.testing.assert_close(r.cpu(), new_res, rtol=1e-5, atol=1e-5)
    close_bf16(out, want)


def _qk_reference(x, weight, cos, sin, heads, col_offset, eps=1e-6):
    b, n, _ = x.shape
    h = x[..., col_offset:col_offset + heads * 128].reshape(b, n, heads, 128).float()
    normed = O.rms_norm(h, weight, eps)
    cis = torch.complex(cos, sin)
    rotated, _ = O.apply_rope(normed, normed, cis)
    return rotated.transpose(1, 2)


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_qk_norm_rope_offsets_and_layout(src_dtype):
    """A text and an image projection land in one [B, H, N, 128] buffer at their offsets; rows
    outside the written range stay untouched (tests/test_metal_engine.py:159-176)."""
    b, t, l, heads = 2, 16, 48, 3
    width = heads * 128 + 256
    g = gen(3)
    yt = torch.randn(b, t, width, generator=g).to(src_dtype)
    xi = torch.randn(b, l, width, generator=g).to(src_dtype)
    w = 1 + 0.1 * torch.randn(128, generator=g)
    cis = torch.cat([O.rope_1d(128, t), O.rope_2d(128, 6, 8, aspect="isotropic")])
    cos, sin = cis.real.contiguous(), cis.imag.contiguous()
    n_out = t + l + 8
    out = torch.zeros(b, heads, n_out, 128, device=DEV, dtype=torch.bfloat16)
    cos_d, sin_d = torch.cat([cos, torch.zeros(8, 64)]).to(DEV), torch.cat([sin, torch.zeros(8, 64)]).to(DEV)
    K.qk_norm_rope(yt.to(DEV), w.to(DEV), cos_d, sin_d, 1e-6, heads, col_offset=128, out=out, offset=0)
    K.qk_norm_rope(xi.to(DEV), w.to(DEV), cos_d, sin_d, 1e-6, heads, col_offset=128, out=out, offset=t)
    got = out.float().cpu()
    want_t = _qk_reference(yt, w, cos[:t], sin[:t], heads, 128)
    want_i = _qk_reference(xi, w, cos[t:], sin[t:], heads, 128)
    close_bf16(got[:, :, :t], want_t, scale=4.0)
    close_bf16(got[:, :, t:t + l], want_i, scale=4.0)
    assert torch.all(got[:, :, t + l:] == 0)


@pytest.mark.parametrize("heads,kv_heads,n_text,n_image", [(20, 5, 256, 4096), (3, 3, 16, 48), (4, 1, 7, 90)])
def test_qkv_prepare_is_the_three_calls(heads, kv_heads, n_text, n_image):
    """One launch for Q / K norm + RoPE and the V transpose of a text and an image projection
    (offsets 0 and n_text) gives bit for bit what qk_norm_rope, qk_norm_rope and v_heads_t write,
    and leaves every other row and position as it was."""
    b = 1 if n_image > 1000 else 2
    g = torch.Generator(device=DEV).manual_seed(30)
    width = (heads + 2 * kv_heads) * 128 + 256  # q | k | v | a gate-like tail
    n = n_text + n_image
    n_pad = (n + 63) // 64 * 64 + 64
    cos = torch.randn(n_pad, 64, generator=g, device=DEV)
    sin = torch.randn(n_pad, 64, generator=g, device=DEV)
    wq = 1 + 0.1 * torch.randn(128, generator=g, device=DEV)
    wk = 1 + 0.1 * torch.randn(128, generator=g, device=DEV)
    projs = [torch.randn(b, rows, width, generator=g, device=DEV).to(torch.bfloat16) for rows in (n_text, n_image)]
    bufs = [[torch.full(shape, 3.0, device=DEV, dtype=torch.bfloat16)
             for shape in ((b, heads, n_pad, 128), (b, kv_heads, n_pad, 128), (b, kv_heads, 128, n_pad))]
            for _ in range(2)]
    k_col, v_col = heads * 128, (heads + kv_heads) * 128
    for proj, off in zip(projs, (0, n_text)):
        q1, k1, vt1 = bufs[0]
        K.qk_norm_rope(proj, wq, cos, sin, 1e-6, heads, 0, out=q1, offset=off)
        K.qk_norm_rope(proj, wk, cos, sin, 1e-6, kv_heads, k_col, out=k1, offset=off)
        K.v_heads_t(proj, kv_heads, vt1, v_col, off)
        K.qkv_prepare(proj, wq, wk, cos, sin, 1e-6, heads, kv_heads, *bufs[1], 0, k_col, v_col, off)
    for one, fused in zip(*bufs):
        assert torch.equal(one, fused)
    assert torch.all(bufs[1][0][:, :, n:] == 3.0) and torch.all(bufs[1][1][:, :, n:] == 3.0)


@pytest.mark.parametrize("gate", [False, True])
@pytest.mark.parametrize("heads,kv_heads,rows,batch,kdim",
                         [(20, 5, (4352,), 1, 2560), (20, 5, (4096, 256), 1, 2560), (3, 1, (400, 112), 2, 192)])
def test_linear_qk_rope_is_linear_then_qkv_prepare(heads, kv_heads, rows, batch, kdim, gate):
    """The q | k | v GEMM with the Q / K norm + RoPE in its store writes bit for bit what the plain
    GEMM followed by qkv_prepare writes (Q, K, and the V columns of the output): one group (the
    single-stream block, 4352 tokens), two groups with the second's tokens first (a dual block's
    image and text rows), and two batch items per group with tokens not a multiple of the tile.
    Other q / k rows and the Q / K columns of the output are left as they were. With a gate tail
    (a q | k | v | gate weight: the gate columns run beside the store, in the same launch at the
    step's shapes) the gate columns are bit for bit the plain GEMM's, with and without V^T."""
    g = torch.Generator(device=DEV).manual_seed(31)
    n_qkv = (heads + 2 * kv_heads) * 128
    n = n_qkv + (heads * 128 if gate else 0)
    v_col = (heads + kv_heads) * 128
    tokens = [r // batch for r in rows]
    offsets = [tokens[1], 0] if len(rows) == 2 else [0]
    n_pad = (sum(tokens) + 63) // 64 * 64 + 64
    cos = torch.randn(n_pad, 64, generator=g, device=DEV)
    sin = torch.randn(n_pad, 64, generator=g, device=DEV)
    xs = [(0.5 * torch.randn(r, kdim, generator=g, device=DEV)).to(torch.bfloat16) for r in rows]
    ws = [(0.05 * torch.randn(n, kdim, generator=g, device=DEV)).to(torch.bfloat16) for _ in rows]
    qws = [1 + 0.1 * torch.randn(128, generator=g, device=DEV) for _ in rows]
    kws = [1 + 0.1 * torch.randn(128, generator=g, device=DEV) for _ in rows]

    def buffers():
        return (torch.full((batch, heads, n_pad, 128), 3.0, device=DEV, dtype=torch.bfloat16),
                torch.full((batch, kv_heads, n_pad, 128), 3.0, device=DEV, dtype=torch.bfloat16))

    q_ref, k_ref = buffers()
    vt = torch.zeros(batch, kv_heads, 128, n_pad, device=DEV, dtype=torch.bfloat16)
    outs_ref = [K.linear(x, w) for x, w in zip(xs, ws)]  # (whatever tile the plain GEMM picks)
    for out, qw, kw, tok, off in zip(outs_ref, qws, kws, tokens, offsets):
        K.qkv_prepare(out.view(batch, tok, n), qw, kw, cos, sin, 1e-6, heads, kv_heads, q_ref, k_ref, vt, 0,
                      heads * 128, v_col, off)
    q, k = buffers()
    outs = [torch.full((r, n), 5.0, device=DEV, dtype=torch.bfloat16) for r in rows]
    K.linear_qk_rope(xs, ws, outs, qws, kws, cos, sin, 1e-6, heads, kv_heads, q, k, tokens, offsets)
    torch.cuda.synchronize()
    assert torch.equal(q, q_ref) and torch.equal(k, k_ref)
    for out, ref in zip(outs, outs_ref):
        assert torch.equal(out[:, v_col:], ref[:, v_col:])
        assert torch.all(out[:, :v_col] == 5.0)
    if all(t % 256 == 0 for t in tokens):  # the V heads straight into the V^T layout as well
        q, k = buffers()
        vt2 = torch.zeros_like(vt)
        outs = [torch.full((r, n), 5.0, device=DEV, dtype=torch.bfloat16) for r in rows]
        K.linear_qk_rope(xs, ws, outs, qws, kws, cos, sin, 1e-6, heads, kv_heads, q, k, tokens, offsets, vt=vt2)
        torch.cuda.synchronize()
        assert torch.equal(q, q_ref) and torch.equal(k, k_ref) and torch.equal(vt2, vt)
        for out, ref in zip(outs, outs_ref):
            assert torch.all(out[:, :n_qkv] == 5.0)
            assert torch.equal(out[:, n_qkv:], ref[:, n_qkv:])


def test_linear_qk_rope_rejects_bad_layouts():
    """Host checks before any launch: rows that are not whole batch items, positions past q / k."""
    x = torch.zeros(100, 128, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(3 * 128, 128, device=DEV, dtype=torch.bfloat16)
    out = torch.zeros(100, 3 * 128, device=DEV, dtype=torch.bfloat16)
    gain = torch.ones(128, device=DEV)
    cos = torch.zeros(128, 64, device=DEV)
    q = torch.zeros(1, 1, 128, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="whole batch items"):
        K.linear_qk_rope([x], [w], [out], [gain], [gain], cos, cos, 1e-6, 1, 1, q, q.clone(), [30], [0])
    with pytest.raises(ValueError, match="outside q/k"):
        K.linear_qk_rope([x], [w], [out], [gain], [gain], cos, cos, 1e-6, 1, 1, q, q.clone(), [100], [40])
    # with vt the weight must hold all kv_heads V heads: one of Q and K heads only (one head of
    # each) would leave vt's V head unwritten
    x = torch.zeros(256, 128, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(2 * 128, 128, device=DEV, dtype=torch.bfloat16)
    out = torch.zeros(256, 2 * 128, device=DEV, dtype=torch.bfloat16)
    cos = torch.zeros(256, 64, device=DEV)
    q = torch.zeros(1, 1, 256, 128, device=DEV, dtype=torch.bfloat16)
    vt = torch.zeros(1, 1, 128, 256, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="V heads"):
        K.linear_qk_rope([x], [w], [out], [gain], [gain], cos, cos, 1e-6, 1, 1, q, q.clone(), [256], [0], vt=vt)
    # the C entry point refuses it on its own (IRIS_E_INVALID), whatever the caller checked
    with pytest.raises(ValueError, match="V heads"):
        _lib.call("iris_gemm_bf16_qk_rope", 1, _lib.pointer_array([x.data_ptr()]), _lib.pointer_array([w.data_ptr()]),
                  _lib.pointer_array([out.data_ptr()]), _lib.int_array([256]), 2 * 128, 128, 128, 128, 2 * 128,
                  _lib.pointer_array([gain.data_ptr()]), _lib.pointer_array([gain.data_ptr()]),
                  _lib.int_array([256]), _lib.int_array([0]), cos.data_ptr(), cos.data_ptr(), 256, q.data_ptr(),
                  q.clone().data_ptr(), 1, 1, 256, vt.data_ptr(), 256, 1e-6, _lib.stream())


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_qk_norm_rope_trunk_shape_matches_oracle(src_dtype):
    """The single-stream block's Q (20 heads) and K (5 heads) of 256 text + 4096 image tokens,
    read from the packed q | k | v | gate projection, with the Iris-3B rotary table (text 1-D,
    64x64 isotropic 2-D), against the oracle's RMSNorm and ``apply_rope``; both the standalone
    kernel and the engine's fused ``qkv_prepare``."""
    from iris_mi355x import tables

    b, t, l, heads, kv = 1, 256, 4096, 20, 5
    n = t + l
    n_pad = (n + 63) // 64 * 64
    width = (heads + 2 * kv) * 128 + heads * 128
    g = torch.Generator(device=DEV).manual_seed(33)
    proj = torch.randn(b, n, width, generator=g, device=DEV).to(src_dtype)
    wq = 1 + 0.02 * torch.randn(128, generator=g, device=DEV)
    wk = 1 + 0.02 * torch.randn(128, generator=g, device=DEV)
    img = tables.rope_2d_angles(128, 64, 64, 10000.0, 16.0, "isotropic")
    txt = tables.rope_1d_angles(128, t, 10000.0)
    cos, sin = tables.cos_sin(txt, img, device=DEV)
    cis = torch.cat([O.rope_1d(128, t), O.rope_2d(128, 64, 64, aspect="isotropic")])
    torch.testing.assert_close(cos[:n].cpu(), cis.real, rtol=0, atol=2e-6)
    torch.testing.assert_close(sin[:n].cpu(), cis.imag, rtol=0, atol=2e-6)
    q = K.qk_norm_rope(proj, wq, cos, sin, 1e-6, heads, 0, out_dtype=torch.bfloat16)
    k = K.qk_norm_rope(proj, wk, cos, sin, 1e-6, kv, heads * 128, out_dtype=torch.bfloat16)
    cpu = proj.float().cpu()
    want_q = _qk_reference(cpu, wq.cpu(), cis.real, cis.imag, heads, 0)
    want_k = _qk_reference(cpu, wk.cpu(), cis.real, cis.imag, kv, heads * 128)
    close_bf16(q, want_q, scale=4.0)
    close_bf16(k, want_k, scale=4.0)
    if src_dtype != torch.bfloat16:
        return  # the engine's fused launch reads the BF16 projection only
    qf = torch.zeros(b, heads, n_pad, 128, device=DEV, dtype=torch.bfloat16)
    kf = torch.zeros(b, kv, n_pad, 128, device=DEV, dtype=torch.bfloat16)
    vt = torch.zeros(b, kv, 128, n_pad, device=DEV, dtype=torch.bfloat16)
    K.qkv_prepare(proj, wq, wk, cos, sin, 1e-6, heads, kv, qf, kf, vt, 0, heads * 128, (heads + kv) * 128)
    assert torch.equal(qf[:, :, :n], q) and torch.equal(kf[:, :, :n], k)


def test_qk_norm_rope_rejects_uncovered_rows():
    x = torch.randn(1, 10, 256, device=DEV)
    w = torch.ones(128, device=DEV)
    cos = torch.ones(8, 64, device=DEV)
    with pytest.raises(ValueError, match="do not cover"):
        K.qk_norm_rope(x, w, cos, cos, 1e-6, 2)


def test_vt_positions_is_the_quad_swap_involution():
    pos = K.vt_positions(64)
    assert pos[:16].tolist() == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]
    assert torch.equal(pos[pos], torch.arange(64))


@pytest.mark.parametrize("offset,n", [(16, 77), (0, 256), (37, 90)])
def test_v_heads_t_writes_the_permuted_transpose(offset, n):
    """Two projections (text rows, then image rows at an offset) land in one V^T buffer; every
    position outside the written tokens keeps its previous value."""
    b, heads, n_pad = 2, 5, 448
    x = torch.randn(b, n, 6400, generator=gen(4)).to(torch.bfloat16).to(DEV)
    out = torch.full((b, heads, 128, n_pad), 3.0, device=DEV, dtype=torch.bfloat16)
    K.v_heads_t(x, heads, out, col_offset=3200, offset=offset)
    v = x[..., 3200:3200 + heads * 128].reshape(b, n, heads, 128).permute(0, 2, 3, 1).cpu()
    token = K.vt_positions(n_pad) - offset  # token held by each position
    got = out.cpu()
    inside = (token >= 0) & (token < n)
    assert torch.equal(got[..., inside], v[..., token[inside]])
    assert torch.all(got[..., ~inside] == 3.0)


@pytest.mark.parametrize("with_next", [False, True])
def test_gated_residual_grouped_is_the_two_calls(with_next):
    """The image and text rows of a dual-stream block in one launch: bit for bit the two
    separate calls, each group on its own residual, branch, gain, gate and next-norm tensors."""
    g = torch.Generator(device=DEV).manual_seed(31)
    b, d = 2, 2560
    shapes = [(b, 1024, d), (b, 37, d)]
    res = [torch.randn(s, generator=g, device=DEV) for s in shapes]
    br = [torch.randn(s, generator=g, device=DEV).to(torch.bfloat16) for s in shapes]
    w = [1 + 0.1 * torch.randn(d, generator=g, device=DEV) for _ in shapes]
    mods = [0.1 * torch.randn(b, 1, 6 * d, generator=g, device=DEV) for _ in shapes]
    gate = [m[..., :d] for m in mods]
    nw = [1 + 0.1 * torch.randn(d, generator=g, device=DEV) for _ in shapes]
    shift = [m[..., d:2 * d] for m in mods]
    scale = [m[..., 2 * d:3 * d] for m in mods]
    one = [r.clone() for r in res]
    grouped = [r.clone() for r in res]
    outs1 = [torch.empty(s, device=DEV, dtype=torch.bfloat16) for s in shapes]
    outs2 = [torch.empty(s, device=DEV, dtype=torch.bfloat16) for s in shapes]
    for i in range(2):
        if with_next:
            K.gated_residual_norm_modulate_(one[i], br[i], w[i], gate[i], 1e-6, nw[i], shift[i], scale[i], outs1[i])
        else:
            K.gated_residual_rms_norm_(one[i], br[i], w[i], gate[i], 1e-6)
    if with_next:
        K.gated_residual_grouped_(grouped, br, w, gate, 1e-6, nw, shift, scale, outs2)
    else:
        K.gated_residual_grouped_(grouped, br, w, gate, 1e-6)
    for i in range(2):
        assert torch.equal(one[i], grouped[i])
        if with_next:
            assert torch.equal(outs1[i], outs2[i])


# -- GEMM --------------------------------------------------------------------------------
def _gemm_ref(a, w, bias=None):
    out = a.float().cpu() @ w.float().cpu().T
    return out if bias is None else out + bias.cpu()


@pytest.mark.parametrize("tile", list(range(-1, 18)))
@pytest.mark.parametrize("mnk", [(300, 320, 128), (4096, 1280, 256), (1, 64, 64), (513, 260, 192)])
def test_gemm_matches_fp32_reference(tile, mnk):
    m, n, k = mnk
    g = gen(5)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    bias = torch.randn(n, generator=g)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        out32 = K.linear(a.to(DEV), w.to(DEV), bias.to(DEV), out_dtype=torch.float32)
        out16 = K.linear(a.to(DEV), w.to(DEV), None)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    want = _gemm_ref(a, w, bias)
    torch.testing.assert_close(out32.cpu(), want, rtol=1e-4, atol=1e-4)
    close_bf16(out16, want - bias)


@pytest.mark.parametrize("tile", [-1, 11, 12, 1, 16, 17])
@pytest.mark.parametrize("shape,swiglu", [((4352, 6400, 2560), False), ((4352, 13696, 2560), True),
                                          ((4096, 16384, 2560), False)])
def test_gemm_bf16_output_over_several_rounds(tile, shape, swiglu):
    """BF16 output at trunk shapes of 425 to 1024 tiles of 256 x 256, more than one per CU: the
    four-wave kernel runs persistently over its rounds for plain output (the next tile's first
    K tile loaded while the current tile's output goes out), one tile per workgroup for SwiGLU;
    checked on sampled rows against an FP32 product of the same BF16 operands."""
    m, n, k = shape
    g = torch.Generator(device=DEV).manual_seed(16)
    a = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        out = K.linear(a, w, swiglu=swiglu)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    rows = torch.cat([torch.arange(0, m, 61), torch.tensor([m - 1])])
    prod = a[rows].float().cpu() @ w.float().cpu().T
    if swiglu:
        pairs = prod.reshape(len(rows), n // 64, 2, 32)
        want = (F.silu(pairs[:, :, 0]) * pairs[:, :, 1]).reshape(len(rows), n // 2)
    else:
        want = prod
    close_bf16(out[rows], want)


@pytest.mark.parametrize("tile", [13, 14, 15])
@pytest.mark.parametrize("shape", [(4352, 2560, 6848), (4096, 1280, 4096), (4096, 16384, 2560)])
def test_gemm_16x16_tiles_over_several_rounds(tile, shape):
    """The four-wave tiles on the 16 x 16 x 32 MFMA (288 x 160, 256 x 160, 128 x 160) at step
    shapes, persistent over one to thirteen rounds of 256 tiles for BF16 output (with and without
    bias) and one tile per workgroup for FP32 output; against an FP32 product on sampled rows."""
    m, n, k = shape
    g = torch.Generator(device=DEV).manual_seed(19)
    a = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16)
    bias = torch.randn(n, generator=g, device=DEV)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        out16 = K.linear(a, w)
        out16b = K.linear(a, w, bias)
        out32 = K.linear(a, w, bias, out_dtype=torch.float32)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    rows = torch.cat([torch.arange(0, m, 53), torch.tensor([m - 1])])
    prod = a[rows].float().cpu() @ w.float().cpu().T
    close_bf16(out16[rows], prod)
    close_bf16(out16b[rows], prod + bias.cpu())
    torch.testing.assert_close(out32[rows].cpu(), prod + bias.cpu(), rtol=1e-4, atol=2e-4)


@pytest.mark.parametrize("rows,n,k,bias", [((4352,), 2560, 6848, False), ((4096, 256), 2560, 6848, False),
                                            ((4096,), 16384, 2560, True), ((4096,), 1280, 4096, True),
                                            ((4096,), 3840, 1280, False), ((4096,), 1280, 1280, True),
                                            ((4096,), 4096, 1280, True), ((17408,), 2560, 6848, False)])
def test_gemm_plain_step_shapes_eager_and_graph_replays(rows, n, k, bias):
    """The step's plain GEMMs (BF16 output, optional FP32 bias): the single-stream w2, the dual
    blocks' grouped image + text w2, the pixel stage's adaLN, compress, q|k|v, proj and expand,
    and a guided batch of four images' w2. Against an FP32 product on sampled rows; every row
    bit for bit the same as the same rows computed alone (the summation order does not depend on
    the row count or the tile); and bit for bit the same when recorded in a HIP graph and replayed
    several times with eager work and synchronisation between the replays."""
    g = torch.Generator(device=DEV).manual_seed(41)
    xs = [torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16) for m in rows]
    ws = [(0.02 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16) for _ in rows]
    bs = [torch.randn(n, generator=g, device=DEV) for _ in rows] if bias else None

    def run(outs=None):
        outs = outs or [torch.empty(m, n, device=DEV, dtype=torch.bfloat16) for m in rows]
        if len(rows) == 1:
            K.linear(xs[0], ws[0], bs[0] if bias else None, out=outs[0])
        else:
            K.linear_grouped(xs, ws, bs, outs)
        return outs

    got = run()
    for i, m in enumerate(rows):
        sel = torch.cat([torch.arange(0, m, 37), torch.tensor([m - 1])])
        want = _gemm_ref(xs[i][sel].cpu(), ws[i].cpu(), bs[i].cpu() if bias else None)
        close_bf16(got[i][sel], want)
        part = K.linear(xs[i][:300].contiguous(), ws[i], bs[i] if bias else None)
        assert torch.equal(part, got[i][:300])
    outs = [torch.empty_like(o) for o in got]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(outs)
    for _ in range(3):
        for o in outs:
            o.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, e) for o, e in zip(outs, got))
        run()  # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("shape", [(4352, 6400, 2560), (4096, 16384, 2560)])
def test_gemm_trunk_shapes(shape):
    m, n, k = shape
    g = torch.Generator(device=DEV).manual_seed(6)
    a = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16)
    out = K.linear(a, w, out_dtype=torch.float32)
    rows = torch.arange(0, m, 97)
    want = a[rows].float().cpu() @ w.float().cpu().T
    torch.testing.assert_close(out[rows].cpu(), want, rtol=1e-4, atol=2e-4)


@pytest.mark.parametrize("rows", [(4352,), (4096, 256), (4096,), (17408,)])
def test_gemm_swiglu_column_split_in_one_launch(rows):
    """SwiGLU w1 | w3 at the step's shapes (the single-stream block, a dual block's grouped image +
    text rows, the last block's image rows, a guided batch of four): the automatic choice runs
    the first columns on 256 x 256 tiles and the rest on 192 x 256 tiles in one launch. Bit for
    bit what a single 256 x 256 tile launch over all columns writes (every tile sums k in order),
    close to an FP32 product on sampled rows, and the same again when replayed from a HIP graph
    with eager work and synchronisation between the replays."""
    n, k = 13696, 2560
    g = torch.Generator(device=DEV).manual_seed(47)
    xs = [torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16) for m in rows]
    ws = [(0.02 * torch.randn(n, k, generator=g, device=DEV)).to(torch.bfloat16) for _ in rows]

    def run(outs=None):
        outs = outs or [torch.full((m, n // 2), 7.0, device=DEV, dtype=torch.bfloat16) for m in rows]
        if len(rows) == 1:
            K.linear(xs[0], ws[0], out=outs[0], swiglu=True)
        else:
            K.linear_grouped(xs, ws, None, outs, swiglu=True)
        return outs

    got = run()
    _lib.call("iris_gemm_force_tile", 16)
    try:
        whole = run()
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    for o, w, x, m in zip(got, whole, xs, rows):
        assert torch.equal(o, w)
        sel = torch.cat([torch.arange(0, m, 211), torch.tensor([m - 1])])
        a = x[sel].float().cpu() @ ws[0].float().cpu().T if len(rows) == 1 else None
        if a is not None:  # interleaved 32-column groups: w1 rows 64p..64p+31, w3 rows 64p+32..
            a = a.view(-1, n // 64, 2, 32)
            close_bf16(o[sel].view(-1, n // 64, 32), F.silu(a[:, :, 0]) * a[:, :, 1])
    outs = [torch.empty_like(o) for o in got]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(outs)
    for _ in range(3):
        for o in outs:
            o.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(o, e) for o, e in zip(outs, got))
        run()  # eager work between the replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("tile", [-1, 0, 1, 4, 5, 6, 7, 8, 9, 10, 11, 12, 16, 17])
def test_gemm_swiglu_epilogue_and_grouped_streams(tile):
    d, hidden = 256, 682
    hp = 704
    g = gen(7)
    w1, w3 = 0.05 * torch.randn(hidden, d, generator=g), 0.05 * torch.randn(hidden, d, generator=g)
    packed = K.pack_swiglu(w1, w3, hp).to(torch.bfloat16)
    xs = [torch.randn(m, d, generator=g).to(torch.bfloat16) for m in (200, 33)]
    outs = [torch.full((m, hp), 7.0, device=DEV, dtype=torch.bfloat16) for m in (200, 33)]
    _lib.call("iris_gemm_force_tile", tile)
    try:
        K.linear_grouped([x.to(DEV) for x in xs], [packed.to(DEV)] * 2, None, outs, swiglu=True)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    for x, o in zip(xs, outs):
        a = x.float() @ w1.to(torch.bfloat16).float().T
        b = x.float() @ w3.to(torch.bfloat16).float().T
        want = F.silu(a) * b
        close_bf16(o[:, :hidden], want)
        assert torch.all(o[:, hidden:].float() == 0)  # zero-padded hidden columns


# -- attention -----------------------------------------------------------------------------
def _attn_inputs(b, h, hkv, n, seed):
    g = gen(seed)
    n_pad = (n + 63) // 64 * 64
    q = torch.randn(b, h, n, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(b, hkv, n, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(b, hkv, n, 128, generator=g).to(torch.bfloat16)
    qd = torch.zeros(b, h, n_pad, 128, dtype=torch.bfloat16)
    kd = torch.zeros(b, hkv, n_pad, 128, dtype=torch.bfloat16)
    vt = torch.zeros(b, hkv, 128, n_pad, dtype=torch.bfloat16)
    qd[:, :, :n], kd[:, :, :n], vt[..., :n] = q, k, v.transpose(-1, -2)
    vt = vt[..., K.vt_positions(n_pad)].contiguous()  # the kernel's V^T position order
    return q, k, v, qd.to(DEV), kd.to(DEV), vt.to(DEV)


@pytest.mark.parametrize("n", [333, 352])
@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5, 6])
def test_flash_attention_variants(variant, n):
    b, h, hkv = 1, 8, 2
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 16)
    want = O.attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(b, n, h * 128)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    _lib.call("iris_flash_attn_force_variant", variant)
    try:
        K.flash_attention(qd, kd, vt, n, None, out, n_split=0)
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    close_attention(out.view(b, n, -1), want)


@pytest.mark.parametrize("n", [77, 4352])
def test_flash_attention_32_key_variants_agree_bitwise(n):
    """The variants with 32-key tiles (register-staged, 3-stage ring, twelve-wave shared ring)
    differ only in how K/V reach LDS: the same products and sums in the same order (each
    exponent a single-rounding fma), so the same bits; the automatic choice between them (by
    grid size) keeps batched and single runs equal."""
    b, h, hkv = 1, 20, 5
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 19)
    outs = []
    try:
        for variant in (1, 3, 4):
            _lib.call("iris_flash_attn_force_variant", variant)
            out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
            K.flash_attention(qd, kd, vt, n, None, out, n_split=0)
            outs.append(out)
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    for i in range(1, len(outs)):
        assert torch.equal(outs[0], outs[i]), f"variant {(1, 3, 4)[i]} differs from variant 1"


@pytest.mark.parametrize("n", [1000, 4352])
def test_flash_attention_batch_rows_do_not_depend_on_the_batch(n):
    """20 query / 5 K/V heads: a batch of four gives each item the bits it gets alone (the
    automatic variant follows one item's shape: at 1000 tokens a batch-sized grid would have
    chosen the 16 x 16 x 32 form, which rounds differently from the single item's)."""
    b, h, hkv = 4, 20, 5
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 23)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    K.flash_attention(qd, kd, vt, n, None, out, n_split=0)
    for i in range(b):
        one = torch.zeros(n, h * 128, device=DEV, dtype=torch.bfloat16)
        K.flash_attention(qd[i:i + 1].contiguous(), kd[i:i + 1].contiguous(), vt[i:i + 1].contiguous(), n, None, one,
                          n_split=0)
        assert torch.equal(one, out[i * n:(i + 1) * n])


@pytest.mark.parametrize("b,h,hkv,n", [(1, 2, 1, 52), (2, 4, 1, 200), (1, 8, 2, 130), (1, 2, 2, 300)])
def test_flash_attention_small(b, h, hkv, n):
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 8)
    want = O.attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(b, n, h * 128)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    K.flash_attention(qd, kd, vt, n, None, out, n_split=0)
    close_attention(out.view(b, n, -1), want)


@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5, 6])
def test_flash_attention_rows_do_not_depend_on_padding_rows(variant):
    """A query row's output is bit-identical whatever the padding query rows (>= n) hold: the
    lazy max raise is decided per column, not per wave."""
    b, h, hkv, n = 1, 8, 2, 77
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 17)
    outs = []
    _lib.call("iris_flash_attn_force_variant", variant)
    try:
        for fill in (0.0, 300.0, float("nan")):
            qf = qd.clone()
            qf[:, :, n:] = fill
            out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
            K.flash_attention(qf, kd, vt, n, None, out, n_split=0)
            outs.append(out.cpu())
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("variant", [-1, 4, 5])
def test_flash_attention_trunk_shape_with_gate_and_split(variant):
    """20 query / 5 K/V heads over 256 text + 4096 image tokens, gate fused, rows split; the
    automatic choice and both twelve-wave forms (32 x 32 x 16 and 16 x 16 x 32 MFMAs)."""
    b, h, hkv, t, l = 1, 20, 5, 256, 4096
    n = t + l
    q, k, v, qd, kd, vt = _attn_inputs(b, h, hkv, n, 9)
    gate = torch.randn(n, h * 128, generator=gen(10)).to(torch.bfloat16)
    oy = torch.zeros(t, h * 128, device=DEV, dtype=torch.bfloat16)
    ox = torch.zeros(l, h * 128, device=DEV, dtype=torch.bfloat16)
    gd = gate.to(DEV)
    _lib.call("iris_flash_attn_force_variant", variant)
    try:
        K.flash_attention(qd, kd, vt, n, oy, ox, n_split=t, gate0=gd[:t], gate1=gd[t:])
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    heads = [0, 3, 4, 7, 18, 19]  # both ends of the first, second and last K/V head's group
    got = torch.cat([oy, ox]).float().cpu().view(n, h, 128)
    sel = torch.cat([torch.arange(0, t, 3), torch.arange(t, n, 7)])  # text and image rows
    for hh in heads:
        qh = q[:, hh:hh + 1, sel].float()
        kk = k[:, hh // 4:hh // 4 + 1].float()
        vv = v[:, hh // 4:hh // 4 + 1].float()
        plain = O.attention(qh, kk, vv)[0, 0]
        gates = torch.sigmoid(gate[sel, hh * 128:(hh + 1) * 128].float())
        close_attention(got[sel, hh], plain * gates)
        close_attention(got[sel, hh] / gates, plain)  # the gate does not hide an error


# -- attention at the magnitudes of the trained model -----------------------------------------
# Late single-stream blocks of the released model carry QK-norm gains up to ~27, so their
# attention logits reach hundreds of nats. The kernels' softmax keeps a lazy running max per
# query column that moves only when a probability would exceed 2^8 (a score ~5.5 nats above it);
# these inputs drive that path in most tiles, each in a different way:
# - "gainG": Q and K as the per-head RMSNorm leaves them (unit RMS) times a gain G: logits of
#   standard deviation G^2 (4, 27^2); the larger ones make the softmax nearly one-hot;
# - "ramp": every query along one direction with its own length, key j along it in proportion
#   to j: each query's logits climb 2-10 nats per 32 keys, so its max moves in nearly every tile
#   and the earlier tiles' output must be rescaled each time;
# - "last_key_peak": N(0,1)-scale logits except the last key, ~ln(n) + 2 above the rest for
#   every query: a raise in the very last tile that rescales the ~12% of the weight
#   accumulated before it.
LOGIT_MODES = ["gain2", "gain27", "ramp", "last_key_peak"]


def _logit_inputs(b, h, hkv, n, seed, mode):
    g = gen(seed)
    q = torch.randn(b, h, n, 128, generator=g)
    k = torch.randn(b, hkv, n, 128, generator=g)
    v = torch.randn(b, hkv, n, 128, generator=g)
    e = F.normalize(torch.randn(128, generator=g), dim=0)
    if mode.startswith("gain"):
        gain = float(mode[4:])
        q, k = q * gain, k * gain
    elif mode == "ramp":
        length = 2.0 + 8.0 * torch.rand(b, h, n, 1, generator=g)
        q = length * e + 0.02 * q
        k = 0.354 * torch.arange(n, dtype=torch.float32)[:, None] * e + 0.5 * k
    elif mode == "last_key_peak":
        q = 0.7 * q + 3.0 * e
        k[:, :, n - 1] = (math.log(n) + 2.0) * math.sqrt(128) / 3.0 * e
    else:
        raise ValueError(mode)
    q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
    n_pad = (n + 63) // 64 * 64
    qd = torch.zeros(b, h, n_pad, 128, dtype=torch.bfloat16)
    kd = torch.zeros(b, hkv, n_pad, 128, dtype=torch.bfloat16)
    vt = torch.zeros(b, hkv, 128, n_pad, dtype=torch.bfloat16)
    qd[:, :, :n], kd[:, :, :n], vt[..., :n] = q, k, v.transpose(-1, -2)
    vt = vt[..., K.vt_positions(n_pad)].contiguous()
    return q, k, v, qd.to(DEV), kd.to(DEV), vt.to(DEV)


def _peak_weight(q, k, hh, hkv_per):
    """Largest softmax weight per query row of head hh (how one-hot the inputs make it)."""
    s = q[0, hh].float() @ k[0, hh // hkv_per].float().T / math.sqrt(128)
    return torch.softmax(s, -1).max(-1).values


@pytest.mark.parametrize("mode", LOGIT_MODES)
@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5, 6])
def test_flash_attention_large_logits(variant, mode):
    """Every variant (64-key register-staged, 32-key register-staged, 64-key ring, 32-key ring,
    twelve-wave ring) against the FP32 oracle on the same BF16 inputs at large logits."""
    b, h, hkv, n = 2, 8, 2, 333
    q, k, v, qd, kd, vt = _logit_inputs(b, h, hkv, n, 40 + LOGIT_MODES.index(mode), mode)
    want = O.attention(q.float(), k.float(), v.float()).transpose(1, 2).reshape(b, n, h * 128)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    _lib.call("iris_flash_attn_force_variant", variant)
    try:
        K.flash_attention(qd, kd, vt, n, None, out, n_split=0)
    finally:
        _lib.call("iris_flash_attn_force_variant", -1)
    got = out.view(b, n, -1)
    assert torch.isfinite(got.float()).all()
    close_attention(got, want)
    if mode == "gain27":  # nearly one-hot: most rows are one value row, to BF16 rounding
        assert _peak_weight(q, k, 0, h // hkv).median() > 0.99


@pytest.mark.parametrize("mode", LOGIT_MODES)
def test_flash_attention_trunk_shape_large_logits(mode):
    """The trunk shape (20 query / 5 K/V heads over 256 text + 4096 image tokens, gate fused, rows
    split) at large logits, on the automatic variant choice."""
    b, h, hkv, t, l = 1, 20, 5, 256, 4096
    n = t + l
    q, k, v, qd, kd, vt = _logit_inputs(b, h, hkv, n, 50 + LOGIT_MODES.index(mode), mode)
    gate = torch.randn(n, h * 128, generator=gen(10)).to(torch.bfloat16)
    oy = torch.zeros(t, h * 128, device=DEV, dtype=torch.bfloat16)
    ox = torch.zeros(l, h * 128, device=DEV, dtype=torch.bfloat16)
    gd = gate.to(DEV)
    K.flash_attention(qd, kd, vt, n, oy, ox, n_split=t, gate0=gd[:t], gate1=gd[t:])
    got = torch.cat([oy, ox]).float().cpu().view(n, h, 128)
    assert torch.isfinite(got).all()
    sel = torch.cat([torch.arange(0, t, 5), torch.arange(t, n, 11)])
    for hh in (0, 7, 19):
        qh = q[:, hh:hh + 1, sel].float()
        plain = O.attention(qh, k[:, hh // 4:hh // 4 + 1].float(), v[:, hh // 4:hh // 4 + 1].float())[0, 0]
        gates = torch.sigmoid(gate[sel, hh * 128:(hh + 1) * 128].float())
        close_attention(got[sel, hh] / gates, plain)


@pytest.mark.parametrize("mode", ["gain27", "ramp"])
def test_flash_attention_masked_large_logits(mode):
    """The text refiner's masked attention (pad keys dropped, each query keeps its own key) at large
    logits, including an all-pad prompt and padding keys at the start."""
    b, h, n = 3, 4, 130
    q, k, v, qd, kd, vt = _logit_inputs(b, h, h, n, 60, mode)
    n_pad = qd.shape[2]
    mask = _text_mask(b, n + 5, n, 12, torch.int64)
    keep = mask[:, :n].bool()[:, None, None, :] | torch.eye(n, dtype=torch.bool)
    want = O.attention(q.float(), k.float(), v.float(), keep).transpose(1, 2).reshape(b, n, h * 128)
    km = torch.zeros(b, n_pad, device=DEV, dtype=torch.uint8)
    K.text_key_mask(mask.to(DEV), n, km)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    K.flash_attention_masked(qd, kd, vt, n, km, out)
    got = out.view(b, n, -1)
    assert torch.isfinite(got.float()).all()
    close_bf16(got, want, scale=1.0, floor=4e-3)


# -- text adapter ---------------------------------------------------------------------------
@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
def test_gemm_silu_epilogue(tile):
    """Linear + SiLU of the layer-wise blocks' MLP (hidden 83 zero-padded to 128 at the released
    width, 3328 at full width)."""
    g = gen(21)
    for m, n, k in ((300, 128, 64), (97, 3328, 128)):
        a = torch.randn(m, k, generator=g).to(torch.bfloat16)
        w = (0.1 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
        bias = torch.randn(n, generator=g)
        _lib.call("iris_gemm_force_tile", tile)
        try:
            out16 = K.linear(a.to(DEV), w.to(DEV), bias.to(DEV), silu=True)
            out32 = K.linear(a.to(DEV), w.to(DEV), bias.to(DEV), out_dtype=torch.float32, silu=True)
        finally:
            _lib.call("iris_gemm_force_tile", -1)
        want = F.silu(_gemm_ref(a, w, bias))
        torch.testing.assert_close(out32.cpu(), want, rtol=1e-4, atol=1e-4)
        close_bf16(out16, want)


@pytest.mark.parametrize("m", [6144, 6912, 12288])
def test_gemm_silu_epilogue_at_batched_adapter_shapes(m):
    """Linear + SiLU of the layer-wise blocks' MLP at full width for batched prompts (2 x 256,
    2 x 288 and 4 x 256 tokens x 12 layers): shapes whose automatic tile choice weighs a column
    split, which must not put the SiLU epilogue on a tile that lacks it."""
    g = gen(22)
    n, k = 3328, 2560
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    bias = 0.1 * torch.randn(n, generator=g)
    out16 = K.linear(a.to(DEV), w.to(DEV), bias.to(DEV), silu=True)
    want = F.silu(_gemm_ref(a, w, bias))
    close_bf16(out16, want)


@pytest.mark.parametrize("tile", [-1, 16, 17, 11])
def test_gemm_swiglu_fp32_output(tile):
    """SwiGLU into an FP32 output (stored straight from the accumulators, no LDS staging), one
    tile per workgroup; rows and hidden units not multiples of the tile."""
    d, hidden, hp = 192, 300, 320
    g = gen(13)
    w1, w3 = 0.05 * torch.randn(hidden, d, generator=g), 0.05 * torch.randn(hidden, d, generator=g)
    packed = K.pack_swiglu(w1, w3, hp).to(torch.bfloat16)
    x = torch.randn(333, d, generator=g).to(torch.bfloat16)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        out = K.linear(x.to(DEV), packed.to(DEV), swiglu=True, out_dtype=torch.float32)
    finally:
        _lib.call("iris_gemm_force_tile", -1)
    a = x.float() @ w1.to(torch.bfloat16).float().T
    b = x.float() @ w3.to(torch.bfloat16).float().T
    torch.testing.assert_close(out[:, :hidden].cpu(), F.silu(a) * b, rtol=1e-4, atol=1e-4)
    assert torch.all(out[:, hidden:].cpu() == 0)


@pytest.mark.parametrize("tile", [11, 16, 13])
def test_gemm_silu_is_refused_by_the_four_wave_tile(tile):
    a = torch.zeros(64, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(64, 64, device=DEV, dtype=torch.bfloat16)
    _lib.call("iris_gemm_force_tile", tile)
    try:
        with pytest.raises(_lib.IrisKernelError, match="SiLU"):
            K.linear(a, w, silu=True)
    finally:
        _lib.call("iris_gemm_force_tile", -1)


def _text_mask(b, n_in, n, seed, dtype):
    """Batch 0: pad keys first (so early key tiles hold no key of later queries), then random real
    tokens, then padding; batch 1: an all-pad prompt (identity attention); batch 2: all real."""
    g = gen(seed)
    mask = torch.zeros(b, n_in)
    lead = min(40, n // 4)
    mask[0, lead:int(0.8 * n)] = (torch.rand(int(0.8 * n) - lead, generator=g) < 0.7).float()
    if b > 2:
        mask[2] = 1.0
    return mask.to(dtype)


@pytest.mark.parametrize("b,h,n,mask_dtype", [(2, 2, 16, torch.int64), (1, 20, 300, torch.bool),
                                               (3, 4, 77, torch.float32), (2, 2, 130, torch.int32)])
def test_flash_attention_masked_text_refiner(b, h, n, mask_dtype):
    q, k, v, qd, kd, vt = _attn_inputs(b, h, h, n, 11)
    n_pad = qd.shape[2]
    mask = _text_mask(b, n + 5, n, 12, mask_dtype)
    keep = mask[:, :n].bool()[:, None, None, :] | torch.eye(n, dtype=torch.bool)
    want = O.attention(q.float(), k.float(), v.float(), keep).transpose(1, 2).reshape(b, n, h * 128)
    km = torch.full((b, n_pad), 9, device=DEV, dtype=torch.uint8)
    K.text_key_mask(mask.to(DEV), n, km)
    want_km = torch.zeros(b, n_pad, dtype=torch.uint8)
    want_km[:, :n] = mask[:, :n].bool().to(torch.uint8)
    assert torch.equal(km.cpu(), want_km)
    out = torch.zeros(b * n, h * 128, device=DEV, dtype=torch.bfloat16)
    K.flash_attention_masked(qd, kd, vt, n, km, out)
    got = out.view(b, n, -1)
    assert torch.isfinite(got.float()).all()
    close_bf16(got, want, scale=1.0, floor=4e-3)
    if b > 1:  # the all-pad prompt attends only to itself: out = v, to BF16 rounding
        # (its one probability enters P.V rounded to BF16 and the normaliser unrounded, so the
        # output is v to one BF16 step: relative 2^-7)
        torch.testing.assert_close(got[1].float().cpu(), v[1].transpose(0, 1).reshape(n, h * 128).float(),
                                   rtol=2.0**-7, atol=0.0)


@pytest.mark.parametrize("seqs,L,heads,d", [(37, 12, 32, 80), (50, 3, 4, 16), (5, 16, 1, 128)])
def test_layer_attention_matches_sdpa(seqs, L, heads, d):
    g = gen(13)
    qkv = torch.randn(seqs * L, 3 * heads * d, generator=g).to(torch.bfloat16)
    q, k, v = (t.transpose(1, 2) for t in qkv.float().view(seqs, L, 3, heads, d).unbind(2))
    want = O.attention(q, k, v).transpose(1, 2).reshape(seqs * L, heads * d)
    out = torch.zeros(seqs * L, heads * d, device=DEV, dtype=torch.bfloat16)
    K.layer_attention(qkv.to(DEV), out, L, heads)
    close_bf16(out, want)


@pytest.mark.parametrize("width", [64, 2560])
def test_layer_pool_with_fused_residual(width):
    rows, L = 45, 12
    g = gen(14)
    h = torch.randn(rows * L, width, generator=g)
    br = torch.randn(rows * L, width, generator=g).to(torch.bfloat16)
    w, b = 0.3 * torch.randn(1, L, generator=g), torch.randn(1, generator=g)
    want = F.linear((h + br.float()).view(rows, L, width).transpose(1, 2), w, b).squeeze(-1)
    out = torch.empty(rows, width, device=DEV)
    K.layer_pool(h.to(DEV), br.to(DEV), w.to(DEV), b.to(DEV), L, out)
    torch.testing.assert_close(out.cpu(), want, rtol=1e-5, atol=1e-5)
    out16 = torch.empty(rows, width, device=DEV, dtype=torch.bfloat16)
    K.layer_pool(h[:rows].to(DEV), None, torch.ones(1, device=DEV), None, 1, out16)
    assert torch.equal(out16.cpu(), h[:rows].to(torch.bfloat16))  # one layer, weight 1: the BF16 cast


@pytest.mark.parametrize("branch_dtype", [None, torch.bfloat16, torch.float32])
def test_residual_rms_norm_with_position_rows(branch_dtype):
    b, n, width = 2, 300, 2560
    g = gen(15)
    res = torch.randn(b * n, width, generator=g)
    br = None if branch_dtype is None else torch.randn(b * n, width, generator=g).to(branch_dtype)
    w = 1 + 0.02 * torch.randn(width, generator=g)
    pos = torch.randn(n, width, generator=g)
    want_res = res if br is None else res + br.float()
    want = O.rms_norm(want_res, w, 1e-6)
    r = res.to(DEV)
    out = torch.empty(b * n, width, device=DEV)
    K.residual_rms_norm(r, None if br is None else br.to(DEV), w.to(DEV), 1e-6, out, add_rows=pos.to(DEV))
    assert torch.equal(r.cpu(), want_res)  # one FP32 add, as torch does it
    torch.testing.assert_close(out.cpu(), want + pos.repeat(b, 1), rtol=2e-5, atol=2e-5)
    out16 = torch.empty(b * n, width, device=DEV, dtype=torch.bfloat16)
    K.residual_rms_norm(r, None, w.to(DEV), 1e-6, out16)
    close_bf16(out16, want)


# -- conditioning, pixel stage, sampler ----------------------------------------------------
@pytest.mark.parametrize("j", [3, 24, 70])
def test_gemv_with_core_biases(j):
    """The shared adaLN core plus one bias row per block (24 in Iris-3B; 70 > one wave of lanes)."""
    n, k, b = 1536, 256, 2
    g = gen(11)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    x = torch.randn(b, k, generator=g)
    bias, extra = torch.randn(n, generator=g), torch.randn(j, n, generator=g)
    out = torch.empty(j, b, n, device=DEV)
    K.gemv(w.to(DEV), x.to(DEV), bias.to(DEV), out, extra_bias=extra.to(DEV), in_silu=True)
    y = F.silu(x) @ w.float().T + bias
    torch.testing.assert_close(out.cpu(), y[None] + extra[:, None], rtol=1e-5, atol=1e-5)
    out2 = torch.empty(b, n, device=DEV)
    K.gemv(w.to(DEV), x.to(DEV), bias.to(DEV), out2, out_silu=True)
    torch.testing.assert_close(out2.cpu(), F.silu(x @ w.float().T + bias), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n,k,b", [(15360, 2560, 1), (100, 4096, 5), (13, 8, 3), (7, 520, 4)])
def test_gemv_shapes(n, k, b):
    """The adaLN-core shape (15360 x 2560), the largest K (4096: eight 16-byte chunks per lane),
    batches past four (two launches), row counts that leave a workgroup's last rows empty and a
    K that leaves some lanes without a chunk."""
    g = gen(12)
    w = (0.05 * torch.randn(n, k, generator=g)).to(torch.bfloat16)
    x = torch.randn(b, k, generator=g)
    bias = torch.randn(n, generator=g)
    out = torch.empty(b, n, device=DEV)
    K.gemv(w.to(DEV), x.to(DEV), bias.to(DEV), out)
    want = x.double() @ w.double().T + bias.double()
    torch.testing.assert_close(out.cpu().double(), want, rtol=1e-5, atol=1e-4)


def test_timestep_features():
    from iris_mi355x import tables

    t = torch.tensor([0.0, 125.0, 625.0, 1000.0])
    freqs = tables.timestep_freqs(256, 10.0, "cpu")
    out = torch.empty(4, 256, device=DEV)
    K.timestep_features(t.to(DEV), freqs.to(DEV), out)
    torch.testing.assert_close(out.cpu(), O.timestep_features(t, 256, 10.0), rtol=0, atol=2e-6)


@pytest.mark.parametrize("hw,patch,channels,out_channels", [((32, 48), 4, 3, 3), ((64, 64), 16, 3, 3),
                                                             ((32, 48), 16, 4, 1), ((64, 32), 4, 4, 3)])
def test_patchify_embed_and_head(hw, patch, channels, out_channels):
    """3-channel RGB and the depth fine-tune's 4-channel input; the 3-channel flow head and the
    1-channel depth head."""
    from iris_mi355x import tables

    b = 2
    h, w = hw
    g = gen(12)
    x = torch.randn(b, channels, h, w, generator=g)
    p = {"pixel_embedder.proj.weight": 0.5 * torch.randn(16, channels, generator=g),
         "pixel_embedder.proj.bias": 0.1 * torch.randn(16, generator=g)}
    nw = 1 + 0.02 * torch.randn(16, generator=g)
    n_patches = (h // patch) * (w // patch)
    k = channels * patch * patch
    kp = (k + 63) // 64 * 64
    patches = torch.zeros(b * n_patches, kp, device=DEV, dtype=torch.bfloat16)
    pixels = torch.empty(b * n_patches, patch * patch, 16, device=DEV)
    normed = torch.empty_like(pixels, dtype=torch.bfloat16)
    pos_x, pos_y = tables.sincos_halves(16, h, w, DEV)
    K.patchify_embed(x.to(DEV), patch, p["pixel_embedder.proj.weight"].to(DEV), p["pixel_embedder.proj.bias"].to(DEV),
                     pos_x, pos_y, nw.to(DEV), 1e-6, patches, pixels, normed)
    want_patches = O.patchify(x, patch).reshape(b * n_patches, -1)
    assert torch.equal(patches[:, :k].cpu(), want_patches.to(torch.bfloat16))
    assert torch.all(patches[:, k:] == 0)
    want_pix = O.pixel_embed(p, x, patch, True)
    torch.testing.assert_close(pixels.cpu(), want_pix, rtol=1e-5, atol=1e-5)
    close_bf16(normed, O.rms_norm(want_pix, nw, 1e-6))

    hw_ = 0.3 * torch.randn(out_channels, 16, generator=g)
    hb = 0.1 * torch.randn(out_channels, generator=g)
    out = torch.empty(b, out_channels, h, w, device=DEV)
    K.unpatchify_head(normed, hw_.to(DEV), hb.to(DEV), out, patch)
    want = O.unpatchify(normed.float().cpu() @ hw_.T + hb, b, h, w, patch)
    torch.testing.assert_close(out.cpu(), want, rtol=1e-5, atol=1e-5)


def _bf16(t):
    return t.to(torch.bfloat16).float()


def _gelu_exact(a):
    """a Phi(a) in float64 with scipy's ndtr for Phi, which keeps full relative precision for
    a << 0 (torch's float64 ndtr cancels below a ~ -7.5)."""
    a = a.double()
    return a * torch.from_numpy(ndtr(a.numpy()))


def _pixel_mlp_at_bf16_points(pixels, branch, mods, nw, fc1, fc2, nnw, eps):
    """The PiT tail at the kernel's BF16 rounding points, which are the reference's
    (src/iris_metal/kernels.py:256-287): h, both weights, the pre-activation and the GELU output
    in BF16; products summed exactly (float64) and the stream in FP32."""
    m = mods.float()
    scale1, shift1, scale2, shift2 = m.chunk(4, dim=-1)
    x = pixels + O.modulate(branch.float(), shift1, scale1)
    h = _bf16(O.rms_norm(x, nw, eps))
    a = _bf16((h.double() @ _bf16(fc1[0]).double().T + fc1[1].double()).float())
    g = _bf16(_gelu_exact(a).float())
    y = (g.double() @ _bf16(fc2[0]).double().T + fc2[1].double()).float()
    x = x + O.modulate(y, shift2, scale2)
    return x, g, m


def test_pixel_mlp_matches_post_modulated_tail():
    """In-place stream and next-block input against the tail at the BF16 rounding points, and
    the MLP branch against the FP32 oracle. Where the kernel's FP32 sum of a pre-activation and
    the exact one round to neighbouring BF16 values (a sum within an FP32 ulp or so of a BF16
    midpoint, about one pre-activation in 10^5), that pixel moves by up to one BF16 step of one
    GELU output times its fc2 weight: such pixels are bounded by that step and must be rare."""
    n = 4096 * 3 + 17
    g = gen(13)
    pixels = torch.randn(n, 16, generator=g)
    branch = torch.randn(n, 16, generator=g).to(torch.bfloat16)
    mods = (0.3 * torch.randn(n, 64, generator=g)).to(torch.bfloat16)
    nw, nnw = 1 + 0.1 * torch.randn(16, generator=g), 1 + 0.1 * torch.randn(16, generator=g)
    fc1 = (0.3 * torch.randn(64, 16, generator=g), 0.1 * torch.randn(64, generator=g))
    fc2 = (0.3 * torch.randn(16, 64, generator=g), 0.1 * torch.randn(16, generator=g))
    want, gel, m = _pixel_mlp_at_bf16_points(pixels, branch, mods, nw, fc1, fc2, nnw, 1e-6)
    pd = pixels.to(DEV)
    nxt = K.pixel_mlp_(pd, branch.to(DEV), mods.to(DEV), nw.to(DEV), fc1, fc2, nnw.to(DEV), 1e-6)
    got = pd.cpu()
    err = (got - want).abs()
    tight = 2e-5 + 2e-5 * want.abs()
    flip = 2 * 2.0 ** -8 * gel.abs().max() * _bf16(fc2[0]).abs().max() * (1 + m[:, 32:48].abs().max())
    print(f"pixel MLP: {int((err > tight).sum())} of {err.numel()} values beyond FP32 rounding, max err "
          f"{err.max().item():.2e} (one-flip bound {flip.item():.2e})", flush=True)
    assert (err > tight).float().mean().item() < 1e-3
    assert torch.all(err <= tight + flip)
    close_bf16(nxt, O.rms_norm(want, nnw, 1e-6), floor=2e-3)

    # the MLP branch against the FP32 oracle: within the BF16 rounding of h, the weights and G
    p = {"m.fc1.weight": fc1[0], "m.fc1.bias": fc1[1], "m.fc2.weight": fc2[0], "m.fc2.bias": fc2[1]}
    scale1, shift1, scale2, shift2 = m.chunk(4, dim=-1)
    x1 = pixels + O.modulate(branch.float(), shift1, scale1)
    ref = O.modulate(O.gelu_mlp(p, "m", O.rms_norm(x1, nw, 1e-6)), shift2, scale2)
    rel = ((got - x1) - ref).norm() / ref.norm()
    assert rel.item() < 8e-3, rel.item()


def test_pixel_mlp_bf16_stream_and_ragged_counts():
    """The BF16 pixel stream (the reference kernel's storage type) against the same tail at the
    BF16 rounding points with the stream read from and rounded back to BF16, at pixel counts that
    leave a partial 32-pixel wave step (1, 31, 33, 100) and none (0): lanes past the last pixel
    store nothing, and the pixels after the range stay untouched."""
    g = gen(21)
    fc1 = (0.3 * torch.randn(64, 16, generator=g), 0.1 * torch.randn(64, generator=g))
    fc2 = (0.3 * torch.randn(16, 64, generator=g), 0.1 * torch.randn(16, generator=g))
    nw, nnw = 1 + 0.1 * torch.randn(16, generator=g), 1 + 0.1 * torch.randn(16, generator=g)
    for n in (0, 1, 31, 33, 100):
        pixels = torch.randn(n + 7, 16, generator=g).to(torch.bfloat16)
        branch = torch.randn(n, 16, generator=g).to(torch.bfloat16)
        mods = (0.3 * torch.randn(n, 64, generator=g)).to(torch.bfloat16)
        pd = pixels.to(DEV)
        nxt = K.pixel_mlp_(pd[:n], branch.to(DEV), mods.to(DEV), nw.to(DEV), fc1, fc2, nnw.to(DEV), 1e-6)
        got = pd.cpu()
        assert torch.equal(got[n:], pixels[n:]), "pixels past the range were written"
        if n == 0:
            assert nxt.numel() == 0
            continue
        want, _, _ = _pixel_mlp_at_bf16_points(pixels[:n].float(), branch, mods, nw, fc1, fc2, nnw, 1e-6)
        close_bf16(got[:n], want, floor=2e-3)
        close_bf16(nxt, O.rms_norm(got[:n].float(), nnw, 1e-6), floor=2e-3)


def test_pixel_mlp_gelu_is_correctly_rounded_erf():
    """The GELU of the pixel MLP at every BF16 argument of its table (2^-16 <= |a| < 256) and at
    arguments on both sides of it: the exact-erf GELU correctly rounded to BF16, checked as the
    nearest BF16 to a Phi(a) in float64 (a zero norm gain makes every hidden pre-activation equal
    its bias, and an identity fc2 routes hidden units 0..15 to the 16 output channels of a zero
    pixel stream)."""
    table_bits = torch.cat([torch.arange(117 << 7, 132 << 7), torch.arange(117 << 7, 132 << 7) | 0x8000])
    edge = torch.tensor([0.0, -0.0, 2.0 ** -11, -(2.0 ** -11), 3.0 * 2.0 ** -12, 1e-30, -1e-30,
                         2.0 ** -10 * 0.99, 31.9, -31.9, 32.0, -32.0, 100.0, -100.0, 1e30, -1e30, 7.0, -7.0,
                         -5.5, -9.0, -13.0, -13.5, -14.0, 0.5, -0.5, 1.0, -1.0, 3.0, -3.0, 4.0])
    args = torch.cat([table_bits.to(torch.int16).view(torch.bfloat16).float(), _bf16(edge)])
    args = torch.cat([args, torch.zeros((-args.numel()) % 16)])
    zeros16 = torch.zeros(16, device=DEV)
    fc2 = (torch.eye(16, 64), torch.zeros(16))
    got = []
    for chunk in args.split(16):
        pixels = torch.zeros(64, 16, device=DEV)
        fc1_b = torch.zeros(64)
        fc1_b[:16] = chunk
        K.pixel_mlp_(pixels, torch.zeros(64, 16, device=DEV, dtype=torch.bfloat16),
                     torch.zeros(64, 64, device=DEV, dtype=torch.bfloat16), zeros16,
                     (torch.zeros(64, 16), fc1_b), fc2, torch.ones(16, device=DEV), 1e-6)
        got.append(pixels[0].cpu())
    got = torch.cat(got)
    assert torch.equal(got, _bf16(got)), "outputs are BF16 values"
    exact = _gelu_exact(args)
    bits = got.to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    for step in (-1, 1):  # both BF16 neighbours (same sign) are no closer than the result
        nb_bits = bits + step
        nb = (nb_bits & 0xFFFF).to(torch.int16).view(torch.bfloat16).double()
        valid = ((nb_bits & 0x7F80) != 0x7F80) & ((nb_bits & 0x8000) == (bits & 0x8000)) & (got != 0)
        closer = (nb - exact).abs() < (got.double() - exact).abs()
        assert not torch.any(closer & valid), args[closer & valid][:8]
    # zero results only where a Phi(a) is below half the smallest BF16 subnormal
    zero = got == 0
    assert torch.all(exact[zero].abs() <= 2.0 ** -134), args[zero & (exact.abs() > 2.0 ** -134)]
    # the textbook FP32 formula a (1 + erf(a / sqrt 2)) / 2 agrees where it does not cancel (a > -3)
    ok = args > -3
    close_bf16(got[ok], F.gelu(args[ok]), floor=0.0)


def test_flow_euler_is_bitwise_the_reference_update():
    g = gen(14)
    x, v = torch.randn(3, 64, 64, generator=g), torch.randn(3, 64, 64, generator=g)
    for s, s_next in ((1.0, 0.938), (0.938, 0.833), (0.833, 0.625)):
        sigma = torch.full((1,), s, dtype=torch.float32)
        clean = x - sigma * v
        implied = (x - (1 - sigma) * clean) / sigma
        sn = torch.full((1,), s_next, dtype=torch.float32)
        want = (1 - sn) * clean + sn * implied
        xn, cl = torch.empty(3, 64, 64, device=DEV), torch.empty(3, 64, 64, device=DEV)
        K.flow_euler(x.to(DEV), v.to(DEV), float(sigma), float(sn), xn, cl)
        assert torch.equal(cl.cpu(), clean)
        assert torch.equal(xn.cpu(), want)


def test_dpm_update_follows_the_solver_expressions():
    """Both orders of the FlowDPMSolver update against the reference's tensor expressions
    evaluated in FP32 on the CPU (solver.py:90-109): first order bit for bit; the second-order
    divide by r0 may round differently from a multiply by its reciprocal (one ulp)."""
    import math

    g = gen(16)
    x, v, x0_1 = (torch.randn(3, 64, 64, generator=g) for _ in range(3))
    lam = lambda u: math.log((1.0 - u) / u)
    s1, s0, t = 0.92, 0.80, 0.57
    # first order
    x0 = x - s0 * v
    phi1 = math.expm1(-(lam(t) - lam(s0)))
    want1 = (t / s0) * x - (1.0 - t) * phi1 * x0
    xd, vd = x.to(DEV), v.to(DEV)
    xn, x0o = torch.empty_like(xd), torch.empty_like(xd)
    K.dpm_update(xd, vd, None, s0, t / s0, (1.0 - t) * phi1, 0.0, 1.0, xn, x0o)
    assert torch.equal(x0o.cpu(), x0)
    assert torch.equal(xn.cpu(), want1)
    # second order
    h, h0 = lam(t) - lam(s0), lam(s0) - lam(s1)
    r0 = h0 / h
    d = (x0 - x0_1) / r0
    phi1 = math.expm1(-h)
    want2 = (t / s0) * x - (1.0 - t) * phi1 * x0 - 0.5 * (1.0 - t) * phi1 * d
    K.dpm_update(xd, vd, x0_1.to(DEV), s0, t / s0, (1.0 - t) * phi1, 0.5 * (1.0 - t) * phi1, r0, xn, x0o)
    assert torch.equal(x0o.cpu(), x0)
    torch.testing.assert_close(xn.cpu(), want2, rtol=2e-7, atol=1e-7)
    with pytest.raises(ValueError, match="alias"):
        K.dpm_update(xd, vd, None, s0, 1.0, 1.0, 0.0, 1.0, xd, x0o)


def test_cfg_combine_and_clamp():
    g = gen(15)
    u, c = torch.randn(1000, generator=g), torch.randn(1000, generator=g)
    out = torch.empty(1000, device=DEV)
    K.cfg_combine(u.to(DEV), c.to(DEV), 3.0, out)
    assert torch.equal(out.cpu(), u + 3.0 * (c - u))
    K.clamp(out, -1.0, 1.0, out)
    assert torch.equal(out.cpu(), (u + 3.0 * (c - u)).clamp(-1, 1))


def test_cpu_tensors_are_rejected():
    with pytest.raises(ValueError, match="GPU"):
        K.rms_norm_modulate(torch.randn(1, 2, 128), torch.ones(128), torch.zeros(1, 1, 128),
                            torch.zeros(1, 1, 128), 1e-6, torch.bfloat16)
