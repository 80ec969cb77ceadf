"""GPU parity of the q/k RMSNorm, RoPE and fused decode-step preparation
kernels against the CPU oracle (oracle/prep.py).

Bar: the reference's own kernel tests compare with allclose(atol=1e-5)
(tests/test_cuda.py:34-38, 104-118); f32 outputs are held to that.  The bf16
cache rows are the f32 results rounded to nearest even: they must equal the
oracle's rounding except where the two f32 values straddle a rounding
boundary, and then differ by one bf16 unit at most.  v is a pure conversion
and must match bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from oracle import prep as orp

pytestmark = pytest.mark.gpu

ATOL = 1e-5


def _bf16_units_apart(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    ai = a.view(torch.int16).to(torch.int32)
    bi = b.view(torch.int16).to(torch.int32)
    return (ai - bi).abs()


@pytest.mark.parametrize("shape", [(2, 3, 256), (8, 64), (16, 128), (3, 512), (1, 256)])
def test_rms_norm_matches_oracle(hip_backend, shape):
    """The shapes of tests/test_cuda.py:34-38 and the other served row lengths."""
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g)
    gamma = torch.randn(shape[-1], generator=g)
    ref = orp.torch_rms_norm(x, gamma, 1e-6)
    got = hip_backend.rms_norm(x.cuda(), gamma.cuda(), 1e-6)
    assert got.shape == x.shape and got.dtype == torch.float32
    assert torch.allclose(got.cpu(), ref, atol=ATOL)


def test_rope_matches_reference_kernel_test(hip_backend):
    """tests/test_cuda.py:104-118: rows 8, dim 256, rope_dim 64, cap 128,
    device pos 17, random tables."""
    torch.manual_seed(4)
    x = torch.randn(8, 256)
    cos = torch.randn(128, 64)
    sin = torch.randn(128, 64)
    pos = torch.tensor([17], dtype=torch.int32, device="cuda")
    ref = orp.torch_rope(x, cos, sin, 17, 64)
    got = hip_backend.rope(x.cuda(), cos.cuda(), sin.cuda(), pos, 64)
    assert torch.allclose(got.cpu(), ref, atol=ATOL)
    assert torch.equal(got.cpu()[:, 64:], x[:, 64:])


@pytest.mark.parametrize("dim,rope_dim,pos", [(256, 256, 4095), (128, 32, 0), (64, 64, 1), (512, 128, 2000)])
def test_rope_real_tables(hip_backend, dim, rope_dim, pos):
    cos, sin = orp.rope_tables(4096, rope_dim, 1.0e7)
    x = torch.randn(5, dim, generator=torch.Generator().manual_seed(dim + pos))
    ref = orp.torch_rope(x, cos, sin, pos, rope_dim)
    got = hip_backend.rope(x.cuda(), cos.cuda(), sin.cuda(), torch.tensor([pos], dtype=torch.int32,
                                                                         device="cuda"), rope_dim)
    assert torch.allclose(got.cpu(), ref, atol=ATOL)


def _prep_case(H=8, Hkv=2, D=256, rd=64, cap=4096, seed=11):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(H * 2 * D + 2 * Hkv * D, generator=g) * 2.0
    qn = torch.randn(D, generator=g)
    kn = torch.randn(D, generator=g)
    cos, sin = orp.rope_tables(cap, rd, 1.0e7)
    return qkv, qn, kn, cos, sin


@pytest.mark.parametrize("H,Hkv,D,rd", [(8, 2, 256, 64), (16, 2, 256, 64), (8, 8, 128, 128), (4, 1, 64, 32)])
@pytest.mark.parametrize("layout", ["token-major", "head-major"])
def test_attn_prep_matches_layer_oracle(hip_backend, H, Hkv, D, rd, layout):
    """The decode-step preparation of layers.py:58-73: q f32, bf16 k/v written
    at the device position only."""
    cap, pos = 4096, 1234
    qkv, qn, kn, cos, sin = _prep_case(H, Hkv, D, rd, cap, seed=H * D + rd)
    q_ref, gate_ref, k_ref, v_ref = orp.attn_prep(qkv, qn, kn, 1e-6, cos, sin, pos, rd, H, Hkv, D)
    if layout == "token-major":
        kc = torch.full((cap, Hkv * D), 7.0, dtype=torch.bfloat16, device="cuda")
        vc = torch.full((cap, Hkv * D), 7.0, dtype=torch.bfloat16, device="cuda")
        kview, vview = kc, vc
        row = lambda c: c[pos].view(Hkv, D)  # noqa: E731
    else:
        kc = torch.full((Hkv, cap, D), 7.0, dtype=torch.bfloat16, device="cuda")
        vc = torch.full((Hkv, cap, D), 7.0, dtype=torch.bfloat16, device="cuda")
        kview, vview = kc.transpose(0, 1), vc.transpose(0, 1)
        row = lambda c: c[:, pos]  # noqa: E731
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q, gate = hip_backend.attn_prep(qkv.cuda(), qn.cuda(), kn.cuda(), 1e-6, cos.cuda(), sin.cuda(), p, rd,
                                    kview, vview, H, Hkv, D)
    assert torch.allclose(q.cpu(), q_ref, atol=ATOL)
    assert torch.equal(gate.cpu(), gate_ref)
    k_got, v_got = row(kc).cpu(), row(vc).cpu()
    units = _bf16_units_apart(k_got, k_ref.to(torch.bfloat16))
    assert units.max().item() <= 1 and (units == 0).float().mean().item() > 0.99
    assert torch.equal(v_got, v_ref.to(torch.bfloat16))
    # every other slot is untouched
    kc_cpu = kc.float().cpu()
    untouched = (kc_cpu == 7.0).sum().item()
    assert untouched == kc_cpu.numel() - Hkv * D


def test_attn_prep_bf16_q_and_positions_outside_the_cache(hip_backend):
    H, Hkv, D, rd, cap = 8, 2, 256, 64, 64
    qkv, qn, kn, cos, sin = _prep_case(H, Hkv, D, rd, 128, seed=3)
    q_ref, _, _, _ = orp.attn_prep(qkv, qn, kn, 1e-6, cos, sin, 100, rd, H, Hkv, D)
    kc = torch.zeros((cap, Hkv * D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    p = torch.tensor([100], dtype=torch.int32, device="cuda")  # past the 64-slot cache
    q, _ = hip_backend.attn_prep(qkv.cuda(), qn.cuda(), kn.cuda(), 1e-6, cos.cuda(), sin.cuda(), p, rd, kc, vc,
                                 H, Hkv, D, q_dtype=torch.bfloat16)
    assert q.dtype == torch.bfloat16
    assert (q.float().cpu() - q_ref).abs().max().item() <= q_ref.abs().max().item() * 2.0**-8
    assert kc.abs().sum().item() == 0 and vc.abs().sum().item() == 0  # nothing written


def test_attn_prep_in_a_graph_follows_the_device_position(hip_backend):
    """graph.py:41-53: one captured step, replayed with the position advanced
    on the device between replays, writes one slot per replay."""
    H, Hkv, D, rd, cap = 8, 2, 256, 64, 256
    qkv, qn, kn, cos, sin = _prep_case(H, Hkv, D, rd, cap, seed=21)
    dq, dqn, dkn, dcos, dsin = (t.cuda() for t in (qkv, qn, kn, cos, sin))
    kc = torch.zeros((cap, Hkv * D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    qbuf = torch.empty((H, D), device="cuda")

    def step():
        q, _ = hip_backend.attn_prep(dq, dqn, dkn, 1e-6, dcos, dsin, pos, rd, kc, vc, H, Hkv, D)
        qbuf.copy_(q)

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for p in (5, 6, 7):
        pos.fill_(p)
        g.replay()
        torch.cuda.synchronize()
        q_ref, _, k_ref, _ = orp.attn_prep(qkv, qn, kn, 1e-6, cos, sin, p, rd, H, Hkv, D)
        assert torch.allclose(qbuf.cpu(), q_ref, atol=ATOL)
        units = _bf16_units_apart(kc[p].view(Hkv, D).cpu(), k_ref.to(torch.bfloat16))
        assert units.max().item() <= 1
    assert kc.float().abs().sum(dim=1).nonzero().flatten().tolist() == [0, 5, 6, 7]


def test_prep_then_fixed_decode_equals_the_layer_oracle(hip_backend):
    """One decode step end to end: attn_prep writes slot pos, attention_fixed
    reads slots 0..pos -- against the oracle's prep + f32 attention over the
    same bf16 cache."""
    from oracle import attention as orc

    H, Hkv, D, rd, cap, pos = 8, 2, 256, 64, 2048, 777
    qkv, qn, kn, cos, sin = _prep_case(H, Hkv, D, rd, cap, seed=31)
    g = torch.Generator().manual_seed(32)
    kc = (torch.randn(cap, Hkv * D, generator=g)).to(torch.bfloat16)
    vc = (torch.randn(cap, Hkv * D, generator=g)).to(torch.bfloat16)
    q_ref, _, k_ref, v_ref = orp.attn_prep(qkv, qn, kn, 1e-6, cos, sin, pos, rd, H, Hkv, D)
    kd, vd = kc.cuda(), vc.cuda()
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q, _ = hip_backend.attn_prep(qkv.cuda(), qn.cuda(), kn.cuda(), 1e-6, cos.cuda(), sin.cuda(), p, rd, kd, vd,
                                 H, Hkv, D)
    out = hip_backend.attention_fixed(q, kd.view(cap, Hkv, D), vd.view(cap, Hkv, D), p, D**-0.5)
    kc[pos] = k_ref.reshape(-1).to(torch.bfloat16)
    vc[pos] = v_ref.reshape(-1).to(torch.bfloat16)
    ref = orc.torch_attention(q_ref, kc[: pos + 1].view(-1, Hkv, D).float(), vc[: pos + 1].view(-1, Hkv, D).float(),
                              D**-0.5)
    err = (out.cpu() - ref).abs().max().item()
    assert err <= 2e-3, err


def test_unserved_prep_shapes_raise(hip_backend):
    with pytest.raises(RuntimeError):
        hip_backend.rms_norm(torch.randn(4, 96, device="cuda"), torch.ones(96, device="cuda"), 1e-6)
    with pytest.raises(RuntimeError):
        hip_backend.rms_norm(torch.randn(4, 256, device="cuda", dtype=torch.bfloat16),
                             torch.ones(256, device="cuda"), 1e-6)
    with pytest.raises(ValueError):
        hip_backend.rope(torch.randn(4, 256, device="cuda"), torch.ones(8, 64, device="cuda"),
                         torch.zeros(8, 64, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"), 63)
