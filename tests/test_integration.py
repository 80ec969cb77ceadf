"""The reference-side adapter (breezetoken_amd.integration): eager decode falls
back for unserved shapes as TilelangBackend.attention does
(breezetoken/backends.py:657-680), attention_fixed raises (backends.py:682-706,
the graph path's fallback signal, graph.py:127-133).  The oracle stands in for
the reference's _torch_attention / SDPA, which the integrating code binds."""

from __future__ import annotations

import pytest
import torch

from breezetoken_amd import backend as bk
from breezetoken_amd import integration
from oracle import attention as orc


def _decode_inputs(H=8, HKV=2, D=256, S=40, kv_dtype=torch.bfloat16, q_dtype=torch.float32, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, D, generator=g).to(q_dtype)
    k = torch.randn(S, HKV, D, generator=g).to(kv_dtype)
    v = torch.randn(S, HKV, D, generator=g).to(kv_dtype)
    return q, k, v


def _oracle_fallback(q, k, v, scale):
    return orc.torch_attention(q.float(), k.float(), v.float(), scale)


def _oracle_prefill_fallback(qq, kk, vv, scale, q_offset):
    out = orc.torch_prefill_banded(qq[0].transpose(0, 1).float(), kk[0].transpose(0, 1).float(),
                                   vv[0].transpose(0, 1).float(), q_offset, scale)
    return out.transpose(0, 1).unsqueeze(0)


class _CpuBackend(integration.RocmAttentionMixin):
    attention_fallback = staticmethod(_oracle_fallback)
    prefill_fallback = staticmethod(_oracle_prefill_fallback)

    def __init__(self, device="cpu"):
        self.device = device


class _StubHip:
    def __init__(self):
        self.calls = []

    def attention(self, q, k, v, scale):
        self.calls.append("attention")
        return torch.full((q.shape[0], q.shape[1]), 7.0)

    def attention_fixed(self, q, k, v, pos, scale):
        self.calls.append("attention_fixed")
        return torch.full((q.shape[0], q.shape[1]), 9.0)


UNSERVED = {
    "f32 cache (reference dtype before the cache edit)": dict(kv_dtype=torch.float32),
    "head_dim 96": dict(D=96),
    "group 16": dict(H=32, HKV=2),
    "f16 q": dict(q_dtype=torch.float16),
}


def test_served_shape_fails_only_on_the_device():
    q, k, v = _decode_inputs()
    reason = bk.decode_unserved(q, k, v, torch.device("cpu"))
    assert reason is not None and "GPU" in reason


@pytest.mark.parametrize("case", list(UNSERVED))
def test_unserved_shapes_name_their_reason(case):
    q, k, v = _decode_inputs(**UNSERVED[case])
    reason = bk.decode_unserved(q, k, v, torch.device("cpu"))
    assert reason is not None and "GPU" not in reason, reason


def test_strided_and_mismatched_inputs_are_unserved():
    q, k, v = _decode_inputs()
    assert "identical strides" in bk.decode_unserved(q, k, v.transpose(0, 1).contiguous().transpose(0, 1))
    assert "equal shapes" in bk.decode_unserved(q, k, v[:-1])
    assert "at least one key" in bk.decode_unserved(q, k[:0], v[:0])
    assert "GQA group" in bk.decode_unserved(q[:5], k, v)


@pytest.mark.parametrize("case", list(UNSERVED) + ["served shape on a CPU backend"])
def test_eager_attention_falls_back_instead_of_raising(case):
    q, k, v = _decode_inputs(**UNSERVED.get(case, {}))
    be = _CpuBackend()
    got = be.attention(q, k, v, 0.0625)
    want = _oracle_fallback(q, k, v, 0.0625)
    assert torch.equal(got, want)


def test_attention_fixed_raises_for_unserved_calls():
    be = _CpuBackend()
    q, k, v = _decode_inputs(D=96)
    pos = torch.tensor([10], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="fixed attention"):
        be.attention_fixed(q, k, v, pos, 0.1)


def test_no_bound_fallback_raises():
    class Bare(integration.RocmAttentionMixin):
        def __init__(self):
            self.device = "cpu"

    q, k, v = _decode_inputs(D=96)
    with pytest.raises(RuntimeError, match="no fallback is bound"):
        Bare().attention(q, k, v, 0.1)


def test_served_calls_go_to_the_hip_backend(monkeypatch):
    """With the predicate satisfied the adapter never touches the fallback."""

    class Routed(_CpuBackend):
        def _gpu(self):
            return torch.device("cuda", 0)

    def boom(*a):
        raise AssertionError("fallback used for a served call")

    be = Routed()
    stub = _StubHip()
    be._hip_backend = stub
    be.attention_fallback = boom
    monkeypatch.setattr(integration, "decode_unserved", lambda q, k, v, dev: None)
    q, k, v = _decode_inputs()
    assert torch.equal(be.attention(q, k, v, 0.1), torch.full((8, 256), 7.0))
    assert torch.equal(be.attention_fixed(q, k, v, torch.tensor([3]), 0.1), torch.full((8, 256), 9.0))
    assert stub.calls == ["attention", "attention_fixed"]


def test_prefill_predicate_and_fallback():
    g = torch.Generator().manual_seed(3)
    S, H, HKV, D = 20, 8, 2, 96
    q = torch.randn(S, H, D, generator=g)
    k = torch.randn(S, HKV, D, generator=g).to(torch.bfloat16)
    v = torch.randn(S, HKV, D, generator=g).to(torch.bfloat16)
    assert "not served" in bk.prefill_unserved(q, k, v, 0)
    q3 = torch.randn(S, 6, 128, generator=g)
    k3 = torch.randn(S, 2, 128, generator=g).to(torch.bfloat16)
    assert "GPU" in bk.prefill_unserved(q3, k3, k3.clone(), 0)
    assert "GPU" in bk.prefill_unserved(q3.to(torch.bfloat16), k3, k3.clone(), 0)
    assert "f32 or bf16 q" in bk.prefill_unserved(q3.half(), k3, k3.clone(), 0)
    be = _CpuBackend()
    qq, kk, vv = q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0), v.transpose(0, 1).unsqueeze(0)
    got = be.prefill_sdpa(qq, kk, vv, D ** -0.5)
    assert got.shape == (1, H, S, D)
    assert torch.equal(got, _oracle_prefill_fallback(qq, kk, vv, D ** -0.5, 0))


@pytest.mark.gpu
def test_adapter_on_the_gpu_serves_and_falls_back(hip_backend):
    """Served shape: the HIP kernels (checked against the oracle); D = 96: the fallback."""

    class Gpu(integration.RocmAttentionMixin):
        attention_fallback = staticmethod(_oracle_fallback)

        def __init__(self):
            self.device = hip_backend.device
            self._hip_backend = hip_backend

    be = Gpu()
    q, k, v = _decode_inputs(S=1000, seed=5)
    got = be.attention(q.cuda(), k.cuda(), v.cuda(), 0.0625)
    err, cos = orc.compare(got.cpu().numpy(), _oracle_fallback(q, k, v, 0.0625).numpy())
    assert err <= 2e-3 and cos >= 0.99999
    q, k, v = _decode_inputs(D=96, S=50, seed=6)
    got = be.attention(q.cuda(), k.cuda(), v.cuda(), 0.1)
    want = _oracle_fallback(q.cuda(), k.cuda(), v.cuda(), 0.1)
    assert torch.equal(got, want)
    with pytest.raises(RuntimeError):
        be.attention_fixed(q.cuda(), k.cuda(), v.cuda(), torch.tensor([49], dtype=torch.int32, device="cuda"), 0.1)
