"""bt_gqa_decode_noalloc: the decode entry point that allocates nothing (its
split workspace is the library's own per-GPU device array) must give exactly
what bt_gqa_decode gives with a caller workspace, call after call."""

from __future__ import annotations

import ctypes

import pytest
import torch

from breezetoken_amd import _lib
from breezetoken_amd import workloads as wl
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _both(lib, case, cap: int, ns: int):
    """(out of bt_gqa_decode with a workspace, out of bt_gqa_decode_noalloc) on the
    device-position path over a (cap, Hkv, D) cache."""
    heads, dim = case.q.shape
    kv_heads = case.k.shape[1]
    q = case.q.float().cuda()
    k, v = case.k.cuda(), case.v.cuda()
    pos = torch.tensor([case.pos], dtype=torch.int32, device="cuda")
    nbytes = int(lib.bt_decode_workspace_bytes(heads, dim, ns))
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ref = torch.empty(heads, dim, dtype=torch.float32, device="cuda")
    got = torch.full((heads, dim), float("nan"), dtype=torch.float32, device="cuda")
    args = (q.data_ptr(), _lib.BT_DTYPE_F32, heads * dim, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            None, pos.data_ptr(), None, cap, 1, heads, kv_heads, dim, ns, case.scale)
    _lib.check("bt_gqa_decode", lib.bt_gqa_decode(*args, ws.data_ptr(), nbytes, ref.data_ptr(),
                                                  _lib.BT_DTYPE_F32, heads * dim, _stream()))
    _lib.check("bt_gqa_decode_noalloc", lib.bt_gqa_decode_noalloc(*args, got.data_ptr(), _lib.BT_DTYPE_F32,
                                                                  heads * dim, _stream()))
    torch.cuda.synchronize()
    return ref.cpu(), got.cpu()


def test_noalloc_matches_workspace_entry_point_on_consecutive_calls(hip_backend):
    lib = _lib.lib()
    # A large call, then a smaller one on a different shape: the second reuses
    # the scratch the first filled and must not see any of it.
    for name, case, cap, ns in (
        ("C2 32k of 65536", wl.c2_inputs(32768, cap=65536), 65536, 128),
        ("H=16 D=128 1000 of 4096", wl.decode_inputs(41, 16, 2, 128, 4096, 1000), 4096, 37),
    ):
        print(f"[no-alloc] {name}", flush=True)
        ref, got = _both(lib, case, cap, ns)
        assert torch.equal(got, ref), f"{name}: differs from bt_gqa_decode by {(got - ref).abs().max():.3e}"
        want = orc.fixed_decode(case.q.float(), case.k.float(), case.v.float(), case.pos, case.scale)
        err, cos = orc.compare(got.numpy(), want.numpy())
        assert err <= 2e-3 and cos >= 0.99999, f"{name}: max-abs {err:.3e}, cosine {cos:.8f}"


def test_noalloc_refuses_shapes_beyond_its_scratch(hip_backend):
    lib = _lib.lib()
    heads, dim, ns = 64, 256, 256  # 64 * 256 * 257 * 4 B > 8 MiB
    assert lib.bt_decode_workspace_bytes(heads, dim, ns) > _lib.BT_NOALLOC_SCRATCH_BYTES
    q = torch.zeros(heads, dim, device="cuda")
    k = torch.zeros(1024, 8, dim, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(heads, dim, device="cuda")
    rc = lib.bt_gqa_decode_noalloc(q.data_ptr(), _lib.BT_DTYPE_F32, heads * dim, k.data_ptr(), k.data_ptr(),
                                   k.stride(0), k.stride(1), None, None, None, 1024, 1, heads, 8, dim, ns, 0.0625,
                                   out.data_ptr(), _lib.BT_DTYPE_F32, heads * dim, _stream())
    assert rc == _lib.BT_ENOSPC
