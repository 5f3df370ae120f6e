"""Pins the QK-norm + RoPE and sigmoid-gate oracles (CPU only): closed forms of the rotation and
the norm, agreement of the reference's two restated variants within the tolerance of the
reference's own test (kernels/qknorm_rope.py:86-110), and planted mistakes."""
import math

import pytest
import torch

from oracle.ref_torch import ref_qknorm_rope, ref_qknorm_rope_fp32, ref_sigmoid_mul


def _inputs(t=5, h=3, d=128, rd=64, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(t, h, d, generator=g).to(dtype)
    w = (0.1 * torch.randn(d, generator=g)).to(dtype)
    cos = torch.randn(t, rd, generator=g).to(dtype)
    sin = torch.randn(t, rd, generator=g).to(dtype)
    return x, w, cos, sin


def test_norm_closed_form():
    """w = 0, no rotation: rows come out with unit RMS (up to bf16 rounding) and keep direction."""
    x, w, _, _ = _inputs(rd=0)
    w.zero_()
    empty = torch.zeros(5, 0, dtype=torch.bfloat16)
    y = ref_qknorm_rope(x, w, empty, empty).float()
    rms = y.pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), atol=1e-2, rtol=0)
    cosang = (y * x.float()).sum(-1) / (y.norm(dim=-1) * x.float().norm(dim=-1))
    assert bool((cosang > 0.9999).all())


def test_rotation_closed_forms():
    """cos 1 / sin 0 is the identity; cos 0 / sin 1 maps (y1, y2) -> (-y2, y1) exactly."""
    x, w, cos, sin = _inputs()
    base = ref_qknorm_rope(x, w, torch.zeros(5, 0, dtype=x.dtype), torch.zeros(5, 0, dtype=x.dtype))
    one, zero = torch.ones_like(cos), torch.zeros_like(cos)
    assert torch.equal(ref_qknorm_rope(x, w, one, zero), base)
    rot = ref_qknorm_rope(x, w, zero, one)
    assert torch.equal(rot[..., :32], -base[..., 32:64])
    assert torch.equal(rot[..., 32:64], base[..., :32])
    assert torch.equal(rot[..., 64:], base[..., 64:])


def test_rotation_preserves_pair_norms():
    """With cos = cos(theta), sin = sin(theta), every rotated pair keeps its length."""
    x, w, _, _ = _inputs(d=256, rd=64, t=4)
    theta = torch.linspace(0, 3, 32)
    cos = torch.cat([theta.cos(), theta.cos()]).expand(4, 64).to(torch.bfloat16)
    sin = torch.cat([theta.sin(), theta.sin()]).expand(4, 64).to(torch.bfloat16)
    base = ref_qknorm_rope(x, w, cos[:, :0], sin[:, :0]).float()
    out = ref_qknorm_rope(x, w, cos, sin).float()
    n0 = base[..., :32].pow(2) + base[..., 32:64].pow(2)
    n1 = out[..., :32].pow(2) + out[..., 32:64].pow(2)
    torch.testing.assert_close(n1, n0, rtol=3e-2, atol=3e-2)


def _angles(n, rd, base=10000.0, dtype=torch.bfloat16):
    inv = 1.0 / base ** (torch.arange(0, rd, 2).float() / rd)
    f = torch.arange(n).float()[:, None] * inv[None, :]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def test_fused_variant_matches_reference_fp32_check():
    """The reference's own test shape (B 4, H 8, D 128, rotary 64) with real rotary angles, at the
    reference test's tolerance (kernels/qknorm_rope.py:99)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    cos, sin = _angles(4, 64)
    fused = ref_qknorm_rope(x.view(4, 8, 128), w, cos, sin).view(4, 8, 1, 128)
    ref = ref_qknorm_rope_fp32(x, w, cos.view(4, 1, 64), sin.view(4, 1, 64))
    torch.testing.assert_close(fused, ref, rtol=1e-2, atol=1e-2)


def test_fused_variant_with_random_cos_sin():
    """The reference test's randn cos/sin: the fused kernel rounds the normalised row to bf16
    before rotating, an error that |c| + |s| amplifies; bounded here by that rounding."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    cos = torch.randn(64, generator=g).to(torch.bfloat16)
    sin = torch.randn(64, generator=g).to(torch.bfloat16)
    fused = ref_qknorm_rope(x.view(4, 8, 128), w, cos, sin).view(4, 8, 1, 128).float()
    ref = ref_qknorm_rope_fp32(x, w, cos.expand(4, 1, 64), sin.expand(4, 1, 64)).float()
    y = ref_qknorm_rope(x.view(4, 8, 128), w, cos[:0], sin[:0]).view(4, 8, 1, 128).float()
    amp = torch.cat([cos[:32].float().abs() + sin[:32].float().abs()] * 2 + [torch.ones(64)])
    bound = 2.0 ** -8 * y.abs().amax(-1, keepdim=True) * amp + 2.0 ** -8 * ref.abs() + 1e-6
    assert bool(((fused - ref).abs() <= bound).all())


def _mutant_no_one_plus(x, w, cos, sin, eps=1e-5):
    return ref_qknorm_rope(x, w - 1.0, cos, sin, eps)   # scale by w instead of (1 + w)


def _mutant_wrong_pairing(x, w, cos, sin, eps=1e-5):
    out = ref_qknorm_rope(x, w, cos, sin, eps).float()  # rotate adjacent pairs instead
    return out[..., [i ^ 1 if i < 64 else i for i in range(x.shape[-1])]].to(x.dtype)


@pytest.mark.parametrize("mutant", [_mutant_no_one_plus, _mutant_wrong_pairing])
def test_checks_catch_planted_mistakes(mutant):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 8, 1, 128, generator=g).to(torch.bfloat16)
    w = (0.5 * torch.randn(128, generator=g)).to(torch.bfloat16)
    cos, sin = _angles(4, 64)
    ref = ref_qknorm_rope_fp32(x, w, cos.view(4, 1, 64), sin.view(4, 1, 64))
    bad = mutant(x.view(4, 8, 128), w, cos, sin).view(4, 8, 1, 128)
    with pytest.raises(AssertionError):
        torch.testing.assert_close(bad, ref, rtol=1e-2, atol=1e-2)


def test_sigmoid_mul_closed_forms():
    a = torch.tensor([1.0, -2.0, 3.5, 0.0], dtype=torch.bfloat16)
    b = torch.tensor([0.0, 100.0, -100.0, 5.0], dtype=torch.bfloat16)
    out = ref_sigmoid_mul(a, b)
    assert out.tolist() == [0.5, -2.0, 0.0, 0.0]
    x = torch.tensor([1.0], dtype=torch.bfloat16)
    assert math.isclose(ref_sigmoid_mul(x, x).item(), 1 / (1 + math.exp(-1)), rel_tol=1e-2)
