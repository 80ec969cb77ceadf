"""Graph safety of the backend's device buffers: a workspace a captured graph
points at stays allocated after a larger call replaces it (until close()), and
eager decode keeps one partials buffer per (heads, head_dim)."""

from __future__ import annotations

import pytest
import torch

from breezetoken_amd import workloads as wl
from breezetoken_amd.backend import HipBackend
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def test_prefill_workspace_growth_keeps_captured_graph_valid():
    be = HipBackend("cuda")
    try:
        q, k, v, scale = (t.cuda() if hasattr(t, "cuda") else t for t in wl.c4_inputs(128, q_f32=True))
        ref = orc.torch_prefill_attention(q.cpu(), k.cpu().float(), v.cpu().float(), scale)
        be.attention_prefill(q, k, v, scale)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = be.attention_prefill(q, k, v, scale)
        small_ws = be._ws["prefill"]
        # a longer prompt grows the workspace: the graph's buffer is retired, not freed
        q2, k2, v2, _ = (t.cuda() if hasattr(t, "cuda") else t for t in wl.c4_inputs(4096, q_f32=True))
        be.attention_prefill(q2, k2, v2, scale)
        assert be._ws["prefill"].data_ptr() != small_ws.data_ptr()
        assert any(t.data_ptr() == small_ws.data_ptr() for t in be._retired)
        del small_ws
        # allocations after the growth must not land in the retired buffer
        junk = [torch.full((1 << 20,), 7.0, device="cuda") for _ in range(8)]
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            err, cos = orc.compare(out.cpu().numpy(), ref.numpy())
            assert err <= 2e-3 and cos >= 0.99999
        del junk
    finally:
        be.close()


def test_eager_decode_keeps_one_workspace_per_shape():
    be = HipBackend("cuda")
    try:
        for valid in (40, 1000, 4096, 30000):
            case = wl.c2_inputs(valid, cap=valid)
            out = be.attention(case.q.float().cuda(), case.k.cuda(), case.v.cuda(), case.scale)
            ref = orc.torch_attention(case.q.float(), case.k.float(), case.v.float(), case.scale)
            err, cos = orc.compare(out.cpu().numpy(), ref.numpy())
            assert err <= 2e-3 and cos >= 0.99999
        decode_keys = [key for key in be._ws if isinstance(key, tuple) and key[0] == "decode"]
        assert decode_keys == [("decode", 8, 256)]
        assert not be._retired
    finally:
        be.close()


def test_host_plan_cache_is_bounded():
    be = HipBackend("cuda")
    try:
        for i in range(be.MAX_HOST_PLANS + 10):
            be.ragged_plan([100 + i, 300], 2, 64)
        assert len(be._plans) == be.MAX_HOST_PLANS
    finally:
        be.close()
