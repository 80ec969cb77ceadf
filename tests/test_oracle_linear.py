"""Pins of the decode matvec oracle (oracle/linear.py) on the CPU."""

from __future__ import annotations

import numpy as np
import torch

from oracle import linear as orl


def _case(K, N, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(K, generator=g), torch.randn(K, N, generator=g).to(torch.bfloat16)


def test_linear_matches_f64_for_any_share_count():
    x, w = _case(1024, 384, 1)
    got = orl.torch_linear(x, w).numpy()
    for sk in (1, 3, 8, 32):
        ref = orl.split_k_linear(x, w, sk)
        assert np.abs(got - ref).max() < 1e-4 * np.abs(ref).max()


def test_linear_one_hot_picks_a_row_and_is_linear():
    x, w = _case(512, 64, 2)
    e = torch.zeros(512)
    e[137] = 1.0
    assert torch.equal(orl.torch_linear(e, w), w[137].float())
    x2, _ = _case(512, 64, 3)
    lhs = orl.torch_linear(2.0 * x - 0.5 * x2, w)
    rhs = 2.0 * orl.torch_linear(x, w) - 0.5 * orl.torch_linear(x2, w)
    assert (lhs - rhs).abs().max().item() < 1e-4


def test_planted_linear_mistakes_are_caught():
    x, w = _case(256, 256, 4)
    ref = orl.split_k_linear(x, w, 1)
    transposed = (x @ w.float().t()).numpy()
    assert np.abs(transposed - ref).max() > 1e-1
    dropped = orl.split_k_linear(x[:192], w[:192], 1)  # the last of four shares lost
    assert np.abs(dropped - ref).max() > 1e-1
