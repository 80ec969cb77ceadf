"""GPU parity of the Gated DeltaNet decode step against the CPU oracle
(oracle/gdn.py), at the bar of the reference's own kernel tests:
allclose(atol=1e-5) on the output and on the in-place updated state
(tests/test_cuda.py:56-77, 170-191)."""

from __future__ import annotations

import pytest
import torch

from oracle import gdn as org

pytestmark = pytest.mark.gpu

ATOL = 1e-5


def _case(hk, hv, dim, seed):
    torch.manual_seed(seed)
    q = torch.randn(hk, dim)
    k = torch.randn(hk, dim)
    v = torch.randn(hv, dim)
    g = torch.randn(hv) * 0.1
    beta = torch.randn(hv)
    state = torch.randn(hv, dim, dim)
    return q, k, v, g, beta, state


@pytest.mark.parametrize("hk,hv,dim,seed", [(16, 16, 128, 3), (8, 16, 128, 5), (16, 32, 128, 7),
                                            (16, 16, 64, 9), (4, 12, 64, 11)])
def test_gdn_decode_matches_oracle(hip_backend, hk, hv, dim, seed):
    """(16, 16, 128) and (8, 16, 128) are the reference's kernel test cases;
    (16, 32, 128) the 35B-A3B grouping."""
    q, k, v, g, beta, state = _case(hk, hv, dim, seed)
    st_ref = state.clone()
    ref = org.torch_gdn_decode(q, k, v, g, beta, st_ref, dim**-0.5)
    st = state.cuda()
    out = hip_backend.gdn_decode(q.cuda(), k.cuda(), v.cuda(), g.cuda(), beta.cuda(), st, dim**-0.5)
    assert torch.allclose(out.cpu(), ref, atol=ATOL)
    assert torch.allclose(st.cpu(), st_ref, atol=ATOL)


def test_gdn_decode_many_steps_carry_the_state(hip_backend):
    """32 consecutive tokens through one layer's state, compared every step."""
    hk, hv, dim = 16, 16, 128
    torch.manual_seed(13)
    st_ref = torch.randn(hv, dim, dim) * 0.1
    st = st_ref.cuda()
    for step in range(32):
        q, k, v = torch.randn(hk, dim), torch.randn(hk, dim), torch.randn(hv, dim)
        g, beta = -torch.rand(hv) * 0.5, torch.randn(hv)
        ref = org.torch_gdn_decode(q, k, v, g, beta, st_ref, dim**-0.5)
        out = hip_backend.gdn_decode(q.cuda(), k.cuda(), v.cuda(), g.cuda(), beta.cuda(), st, dim**-0.5)
        assert torch.allclose(out.cpu(), ref, atol=ATOL), step
    assert torch.allclose(st.cpu(), st_ref, atol=ATOL)


def test_gdn_decode_in_a_graph(hip_backend):
    """Captured once and replayed: each replay advances the in-place state by
    one step, like the graph decode loop (graph.py:65-136)."""
    hk, hv, dim = 16, 16, 128
    q, k, v, g, beta, state = _case(hk, hv, dim, 17)
    state *= 0.1
    dq, dk, dv, dg, db = (t.cuda() for t in (q, k, v, g, beta))
    st = state.cuda()
    obuf = torch.empty(hv, dim, device="cuda")

    def step():
        obuf.copy_(hip_backend.gdn_decode(dq, dk, dv, dg, db, st, dim**-0.5))

    st_ref = state.clone()
    step()
    org.torch_gdn_decode(q, k, v, g, beta, st_ref, dim**-0.5)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    st.copy_(st_ref.cuda())  # replays continue from the oracle's state after the eager step
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        ref = org.torch_gdn_decode(q, k, v, g, beta, st_ref, dim**-0.5)
        assert torch.allclose(obuf.cpu(), ref, atol=ATOL)
        assert torch.allclose(st.cpu(), st_ref, atol=ATOL)


def test_gdn_unserved_shapes_raise(hip_backend):
    q = torch.randn(4, 96, device="cuda")
    with pytest.raises(RuntimeError):
        hip_backend.gdn_decode(q, q, q, torch.zeros(4, device="cuda"), torch.zeros(4, device="cuda"),
                               torch.zeros(4, 96, 96, device="cuda"), 0.1)
    q = torch.randn(3, 64, device="cuda")
    with pytest.raises(ValueError):
        hip_backend.gdn_decode(q, q, torch.randn(4, 64, device="cuda"), torch.zeros(4, device="cuda"),
                               torch.zeros(4, device="cuda"), torch.zeros(4, 64, 64, device="cuda"), 0.1)
