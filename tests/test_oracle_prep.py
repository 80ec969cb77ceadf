"""Pins of the decode-step preparation oracle (oracle/prep.py) on the CPU.

Each restatement is checked against something other than itself: a float64
per-element loop written in the kernel's partner/sign form, closed forms of
RMSNorm and of rotations built from real RoPE tables, and planted mistakes
that must fail.  The reference's own kernel tests (tests/test_cuda.py:34-38
and 104-118) fix the shapes and the allclose(atol=1e-5) bar used here.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import prep as orp


def _close64(a, b):
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


# ----------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("shape", [(2, 3, 256), (5, 64), (1, 512), (4, 128)])
def test_rms_norm_matches_f64_loop(shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g)
    w = torch.randn(shape[-1], generator=g)
    got = orp.torch_rms_norm(x, w, 1e-6)
    ref = orp.brute_rms_norm_f64(x.numpy(), w.numpy(), 1e-6)
    assert _close64(got.numpy(), ref) < 2e-6


def test_rms_norm_closed_forms():
    w = torch.linspace(-2.0, 2.0, 256)
    # a constant row c normalises to c / sqrt(c^2 + eps) * w
    for c in (3.0, -0.5, 1e-2):
        x = torch.full((1, 256), c)
        expect = c / math.sqrt(c * c + 1e-6) * w
        assert (orp.torch_rms_norm(x, w, 1e-6)[0] - expect).abs().max().item() < 1e-6
    # with eps = 0 the norm is scale invariant
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(1))
    a = orp.torch_rms_norm(x, w, 0.0)
    b = orp.torch_rms_norm(x * 37.5, w, 0.0)
    assert (a - b).abs().max().item() < 1e-5


def test_planted_rms_norm_mistakes_are_caught():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 256, generator=g)
    w = torch.randn(256, generator=g)
    ref = orp.brute_rms_norm_f64(x.numpy(), w.numpy(), 1e-6)
    summed = x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + 1e-6) * w  # sum instead of mean
    assert _close64(summed.numpy(), ref) > 1e-2
    no_weight = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    assert _close64(no_weight.numpy(), ref) > 1e-2
    tiny = torch.full((1, 256), 1e-4)
    no_eps = tiny * torch.rsqrt(tiny.pow(2).mean(-1, keepdim=True)) * w  # eps dropped
    assert _close64(no_eps.numpy(), orp.brute_rms_norm_f64(tiny.numpy(), w.numpy(), 1e-6)) > 1e-2


# --------------------------------------------------------------------- RoPE
def test_rope_matches_partner_form_on_reference_test_shapes():
    """tests/test_cuda.py:104-118: rows 8, dim 256, rope_dim 64, cap 128,
    pos 17, random (not rotation) tables -- so the sign and partner of every
    term matter."""
    torch.manual_seed(4)
    x = torch.randn(8, 256)
    cos = torch.randn(128, 64)
    sin = torch.randn(128, 64)
    got = orp.torch_rope(x, cos, sin, 17, 64)
    ref = orp.brute_rope_f64(x.numpy(), cos.numpy(), sin.numpy(), 17, 64)
    assert _close64(got.numpy(), ref) < 1e-5
    assert torch.equal(got[:, 64:], x[:, 64:])  # dims past rope_dim pass through


def test_rope_tables_closed_form():
    cos, sin = orp.rope_tables(64, 64, 1.0e7)
    for p in (0, 1, 17, 63):
        for i in (0, 1, 5, 31):
            ang = p * (1.0e7 ** (-i / 32))
            assert abs(cos[p, i].item() - math.cos(ang)) < 1e-5
            assert abs(sin[p, i + 32].item() - math.sin(ang)) < 1e-5


def test_rope_rotation_properties_with_real_tables():
    cos, sin = orp.rope_tables(64, 64, 1.0e4)
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(5))
    # position 0 is the identity
    assert (orp.torch_rope(x, cos, sin, 0, 64) - x).abs().max().item() < 1e-6
    # every (d, d + half) pair keeps its length
    y = orp.torch_rope(x, cos, sin, 29, 64)
    n0 = x[:, :32] ** 2 + x[:, 32:64] ** 2
    n1 = y[:, :32] ** 2 + y[:, 32:64] ** 2
    assert (n0 - n1).abs().max().item() < 1e-4
    # rotations compose: rope(rope(x, 3), 5) == rope(x, 8)
    z = orp.torch_rope(orp.torch_rope(x, cos, sin, 3, 64), cos, sin, 5, 64)
    assert (z - orp.torch_rope(x, cos, sin, 8, 64)).abs().max().item() < 1e-5


def test_planted_rope_mistakes_are_caught():
    torch.manual_seed(4)
    x = torch.randn(8, 256)
    cos = torch.randn(128, 64)
    sin = torch.randn(128, 64)
    ref = orp.brute_rope_f64(x.numpy(), cos.numpy(), sin.numpy(), 17, 64)
    rot = x[:, :64]
    flipped = rot * cos[17] + torch.cat((rot[:, 32:], -rot[:, :32]), dim=-1) * sin[17]  # wrong sign
    assert _close64(flipped.numpy(), ref[:, :64]) > 1e-2
    pairs = rot.reshape(8, 32, 2)
    inter = torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).reshape(8, 64)  # interleaved pairs
    assert _close64((rot * cos[17] + inter * sin[17]).numpy(), ref[:, :64]) > 1e-2
    off_by_one = orp.torch_rope(x, cos, sin, 18, 64)  # wrong table row
    assert _close64(off_by_one.numpy(), ref) > 1e-2


# ------------------------------------------------------------ attention prep
def test_attn_prep_slices_the_fused_projection_like_the_layer():
    """layers.py:58-64: [H x (q | gate) | Hkv x k | Hkv x v]."""
    H, Hkv, D = 4, 2, 64
    qkv = torch.cat([
        torch.cat([torch.full((D,), 10.0 + h), torch.full((D,), 20.0 + h)]) for h in range(H)
    ] + [torch.full((D,), 30.0 + g) for g in range(Hkv)] + [torch.full((D,), 40.0 + g) for g in range(Hkv)])
    ones = torch.ones(D)
    cos = torch.ones(8, D)
    sin = torch.zeros(8, D)
    q, gate, k, v = orp.attn_prep(qkv, ones, ones, 0.0, cos, sin, 3, D, H, Hkv, D)
    for h in range(H):
        assert torch.allclose(q[h], torch.ones(D))        # rms_norm of a constant row = 1
        assert torch.all(gate[h] == 20.0 + h)
    assert torch.allclose(k, torch.ones(Hkv, D))
    for g in range(Hkv):
        assert torch.all(v[g] == 40.0 + g)


def test_attn_prep_is_the_composition_of_the_pinned_parts():
    H, Hkv, D, rd = 8, 2, 256, 64
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(H * 2 * D + 2 * Hkv * D, generator=g)
    qn, kn = torch.randn(D, generator=g), torch.randn(D, generator=g)
    cos, sin = orp.rope_tables(256, rd, 1.0e7)
    q, gate, k, v = orp.attn_prep(qkv, qn, kn, 1e-6, cos, sin, 100, rd, H, Hkv, D)
    qraw = qkv[: H * 2 * D].view(H, 2 * D)[:, :D]
    ref_q = orp.brute_rope_f64(orp.brute_rms_norm_f64(qraw.numpy(), qn.numpy(), 1e-6), cos.numpy(),
                               sin.numpy(), 100, rd)
    assert _close64(q.numpy(), ref_q) < 1e-5
    kraw = qkv[H * 2 * D: H * 2 * D + Hkv * D].view(Hkv, D)
    ref_k = orp.brute_rope_f64(orp.brute_rms_norm_f64(kraw.numpy(), kn.numpy(), 1e-6), cos.numpy(),
                               sin.numpy(), 100, rd)
    assert _close64(k.numpy(), ref_k) < 1e-5
