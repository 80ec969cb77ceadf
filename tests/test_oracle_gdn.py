"""Pins of the Gated DeltaNet decode oracle (oracle/gdn.py) on the CPU.

The einsum restatement of backends.py:242-271 is checked against a float64
loop written from the update rule, against closed forms of the delta rule,
and against planted mistakes that must fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn as org


def _case(hk, hv, dim, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(hk, dim, generator=g)
    k = torch.randn(hk, dim, generator=g)
    v = torch.randn(hv, dim, generator=g)
    gl = torch.randn(hv, generator=g) * 0.1
    beta = torch.randn(hv, generator=g)
    state = torch.randn(hv, dim, dim, generator=g)
    return q, k, v, gl, beta, state


@pytest.mark.parametrize("hk,hv,dim", [(2, 2, 16), (2, 4, 8), (1, 3, 12), (3, 3, 32)])
def test_gdn_matches_f64_loop(hk, hv, dim):
    q, k, v, gl, beta, state = _case(hk, hv, dim, seed=hk * 100 + hv * 10 + dim)
    ref_out, ref_state = org.brute_gdn_decode_f64(q, k, v, gl, beta, state, dim**-0.5)
    st = state.clone()
    out = org.torch_gdn_decode(q, k, v, gl, beta, st, dim**-0.5)
    assert np.abs(out.numpy() - ref_out).max() < 1e-4
    assert np.abs(st.numpy() - ref_state).max() < 1e-5


def test_gdn_closed_forms():
    q, k, v, gl, beta, state = _case(2, 2, 16, seed=1)
    scale = 0.25
    # beta -> -inf: nothing is written, the state only decays
    st = state.clone()
    out = org.torch_gdn_decode(q, k, v, gl, torch.full((2,), -1e4), st, scale)
    decayed = state * torch.exp(gl).view(2, 1, 1)
    assert (st - decayed).abs().max().item() < 1e-6
    qn = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6) * scale
    assert (out - torch.einsum("hdv,hd->hv", decayed, qn)).abs().max().item() < 1e-5
    # zero state: out = (qn . kn) * sigmoid(beta) * v
    st = torch.zeros_like(state)
    out = org.torch_gdn_decode(q, k, v, gl, beta, st, scale)
    kn = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    expect = (qn * kn).sum(-1, keepdim=True) * torch.sigmoid(beta).unsqueeze(-1) * v
    assert (out - expect).abs().max().item() < 1e-5
    # full write strength, no decay: the new state maps kn to v (the delta rule)
    st = state.clone()
    org.torch_gdn_decode(q, k, v, torch.zeros(2), torch.full((2,), 40.0), st, scale)
    recalled = torch.einsum("hdv,hd->hv", st, kn)
    assert (recalled - v).abs().max().item() < 1e-3


def test_gdn_value_head_reads_key_head_modulo():
    """Value head h uses key head h % Hk (backends.py:266, gdn.py:13-18)."""
    q, k, v, gl, beta, state = _case(2, 4, 8, seed=2)
    st = state.clone()
    out = org.torch_gdn_decode(q, k, v, gl, beta, st, 0.3)
    for h in range(4):
        st1 = state[h:h + 1].clone()
        kh = h % 2
        o1 = org.torch_gdn_decode(q[kh:kh + 1], k[kh:kh + 1], v[h:h + 1], gl[h:h + 1], beta[h:h + 1], st1, 0.3)
        assert (o1[0] - out[h]).abs().max().item() < 1e-5


def test_planted_gdn_mistakes_are_caught():
    q, k, v, gl, beta, state = _case(2, 4, 16, seed=3)
    scale = 16**-0.5
    ref_out, ref_state = org.brute_gdn_decode_f64(q, k, v, gl, beta, state, scale)

    def variant(decay_fn, index_fn, sig=True):
        qn = q * torch.rsqrt(q.pow(2).sum(-1, keepdim=True) + 1e-6) * scale
        kn = k * torch.rsqrt(k.pow(2).sum(-1, keepdim=True) + 1e-6)
        idx = index_fn(torch.arange(4))
        decayed = state * decay_fn(gl).view(4, 1, 1)
        rec = torch.einsum("hdv,hd->hv", decayed, kn[idx])
        delta = (v - rec) * (torch.sigmoid(beta) if sig else beta).unsqueeze(-1)
        st = decayed + kn[idx].unsqueeze(-1) * delta.unsqueeze(-2)
        return torch.einsum("hdv,hd->hv", st, qn[idx]).numpy()

    assert np.abs(variant(torch.exp, lambda h: h % 2) - ref_out).max() < 1e-4  # the variant harness is right
    assert np.abs(variant(lambda x: x, lambda h: h % 2) - ref_out).max() > 1e-2  # g used without exp
    assert np.abs(variant(torch.exp, lambda h: h // 2) - ref_out).max() > 1e-2  # blocked instead of modulo heads
    assert np.abs(variant(torch.exp, lambda h: h % 2, sig=False) - ref_out).max() > 1e-2  # raw beta
