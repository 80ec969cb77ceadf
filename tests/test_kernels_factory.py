"""The reference-signature kernel factories ``gqa_decode`` / ``gqa_decode_fixed``
(breezetoken/kernels/cuda/attention.py:54-66, 208-232) and the launch wrappers
that call them (breezetoken/backends.py:523-568), with only the import swapped.

CPU: build-time ValueErrors, caching, and how the returned callable maps the
reference's (Q, K, V[, Pos], Lse, Part, Out) onto the C ABI (a recording
stand-in for the library; no GPU call).  GPU: the same wrappers against the
oracle and against HipBackend.
"""

from __future__ import annotations

import pytest
import torch

from breezetoken_amd import kernels
from breezetoken_amd._lib import BT_DTYPE_BF16, BT_DTYPE_F32
from oracle import attention as orc


def _build_attention(heads, groups, dim, scale, device):
    """backends.py:523-544 with ``from breezetoken_amd.kernels import gqa_decode``."""
    from breezetoken_amd.kernels import gqa_decode

    num_split = 16
    kernel = gqa_decode(heads, groups, dim, scale, num_split=num_split)

    def run(q, k, v):
        seq = k.shape[0]
        lse = torch.empty((1, heads, num_split), dtype=torch.float32, device=device)
        part = torch.empty((1, heads, num_split, dim), dtype=torch.float32, device=device)
        out = torch.empty((1, heads, dim), dtype=torch.float32, device=device)
        kernel(q.contiguous().view(1, heads, dim), k.contiguous().view(1, seq, groups, dim),
               v.contiguous().view(1, seq, groups, dim), lse, part, out)
        return out.view(heads, dim)

    return run


def _build_attention_fixed(heads, groups, dim, cap, scale, device):
    """backends.py:547-568 with ``from breezetoken_amd.kernels import gqa_decode_fixed``."""
    from breezetoken_amd.kernels import gqa_decode_fixed

    num_split = 16
    kernel = gqa_decode_fixed(heads, groups, dim, cap, scale, num_split=num_split)

    def run(q, k, v, pos):
        lse = torch.empty((1, heads, num_split), dtype=torch.float32, device=device)
        part = torch.empty((1, heads, num_split, dim), dtype=torch.float32, device=device)
        out = torch.empty((1, heads, dim), dtype=torch.float32, device=device)
        kernel(q.contiguous().view(1, heads, dim), k.view(1, cap, groups, dim), v.view(1, cap, groups, dim),
               pos.reshape(1).to(torch.int32), lse, part, out)
        return out.view(heads, dim)

    return run


# ------------------------------------------------------------------------ CPU
@pytest.mark.parametrize("args,match", [
    ((8, 3, 256, 0.0625), "divisible"),                 # attention.py:67-68
    ((32, 1, 256, 0.0625), "padded query tile"),        # group 32 > block_h 16 (attention.py:69-70)
    ((16, 1, 256, 0.0625), "not served"),               # group 16: this build serves <= 8
    ((8, 2, 96, 0.0625), "not served"),
])
def test_build_time_errors(args, match):
    with pytest.raises(ValueError, match=match):
        kernels.gqa_decode(*args)


def test_fixed_capacity_must_be_whole_tiles():
    with pytest.raises(ValueError, match="multiple of the K/V tile"):  # attention.py:227-228
        kernels.gqa_decode_fixed(8, 2, 256, 1000, 0.0625)
    assert kernels.gqa_decode_fixed(8, 2, 256, 1024, 0.0625) is kernels.gqa_decode_fixed(8, 2, 256, 1024, 0.0625)


class _Recorder:
    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def fn(*args):
            self.calls.append((name, args))
            return 0
        return fn


@pytest.fixture
def recorder(monkeypatch):
    rec = _Recorder()
    monkeypatch.setattr(kernels._lib, "lib", lambda: rec)
    monkeypatch.setattr(kernels, "_stream", lambda dev: 1234)
    return rec


def test_decode_wrapper_maps_onto_the_c_abi(recorder):
    H, G, D, S = 8, 2, 256, 100
    q = torch.randn(H, D)
    k = torch.randn(S, G, D).to(torch.bfloat16)
    v = torch.randn(S, G, D).to(torch.bfloat16)
    out = _build_attention(H, G, D, 0.0625, "cpu")(q, k, v)
    assert out.shape == (H, D)
    (n1, split), (n2, comb) = recorder.calls
    assert n1 == "bt_gqa_decode_split" and n2 == "bt_gqa_decode_combine"
    assert split[0] == q.data_ptr() and split[1] == BT_DTYPE_F32 and split[2] == H * D
    assert split[3] == k.data_ptr() and split[4] == v.data_ptr()
    assert split[5:7] == (G * D, D)                     # token and kv-head strides of (1, S, Hkv, D)
    assert split[7:10] == (None, None, None) and split[10] == S
    assert split[11:16] == (1, H, G, D, 16) and split[16] == 0.0625
    assert split[19] == 1234
    lse_ptr, part_ptr = split[17], split[18]
    assert comb[:9] == (lse_ptr, part_ptr, 1, H, D, 16, None, None, 16)
    assert comb[9] == out.data_ptr() and comb[10] == BT_DTYPE_F32 and comb[11] == H * D and comb[12] == 1234


def test_fixed_wrapper_passes_pos_and_capacity(recorder):
    H, G, D, cap = 16, 2, 128, 512
    q = torch.randn(H, D).to(torch.bfloat16)
    k = torch.zeros(cap, G, D, dtype=torch.bfloat16)
    v = torch.zeros(cap, G, D, dtype=torch.bfloat16)
    pos = torch.tensor([40], dtype=torch.int32)
    _build_attention_fixed(H, G, D, cap, 0.1, "cpu")(q, k, v, pos)
    (_, split), _ = recorder.calls
    assert split[1] == BT_DTYPE_BF16 and split[8] == pos.data_ptr() and split[10] == cap


def test_call_checks_shapes(recorder):
    kern = kernels.gqa_decode(8, 2, 256, 0.0625)
    q = torch.randn(1, 8, 256)
    k = torch.zeros(1, 10, 2, 256, dtype=torch.bfloat16)
    lse, part, out = torch.empty(1, 8, 16), torch.empty(1, 8, 16, 256), torch.empty(1, 8, 256)
    with pytest.raises(ValueError, match="Part"):
        kern(q, k, k, lse, torch.empty(1, 8, 8, 256), out)
    with pytest.raises(ValueError, match="bf16 cache"):
        kern(q, k.float(), k.float(), lse, part, out)
    kern(q, k, k, lse, part, out)
    assert [c[0] for c in recorder.calls] == ["bt_gqa_decode_split", "bt_gqa_decode_combine"]


# ------------------------------------------------------------------------ GPU
@pytest.mark.gpu
@pytest.mark.parametrize("heads,groups,dim,seq", [(8, 2, 256, 1), (8, 2, 256, 17), (8, 2, 256, 1000),
                                                  (16, 2, 256, 3000), (4, 4, 128, 64)])
def test_reference_wrappers_on_the_gpu(hip_backend, heads, groups, dim, seq):
    g = torch.Generator().manual_seed(seq + heads)
    q = torch.randn(heads, dim, generator=g)
    k = torch.randn(seq, groups, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(seq, groups, dim, generator=g).to(torch.bfloat16)
    scale = dim**-0.5
    print(f"[factory] H={heads} Hkv={groups} D={dim} S={seq}", flush=True)
    ref = orc.torch_attention(q, k.float(), v.float(), scale)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = _build_attention(heads, groups, dim, scale, "cuda")(qd, kd, vd)
    err, cos = orc.compare(out.cpu().numpy(), ref.numpy())
    assert err <= 2e-3 and cos >= 0.99999
    assert (out - hip_backend.attention(qd, kd, vd, scale)).abs().max().item() <= 1e-5
    cap = -(-seq // 32) * 32 + 32
    kc = torch.zeros(cap, groups, dim, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros(cap, groups, dim, dtype=torch.bfloat16, device="cuda")
    kc[:seq], vc[:seq] = kd, vd
    pos = torch.tensor([seq - 1], dtype=torch.int32, device="cuda")
    fixed = _build_attention_fixed(heads, groups, dim, cap, scale, "cuda")(qd, kc, vc, pos)
    err, cos = orc.compare(fixed.cpu().numpy(), ref.numpy())
    assert err <= 2e-3 and cos >= 0.99999
