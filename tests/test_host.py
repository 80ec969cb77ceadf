"""Host-side logic that runs without a GPU: the KV cache view contract, the
synthetic workloads and the backend's refusal to run anywhere but a GPU."""

from __future__ import annotations

import pytest
import torch

from breezetoken_amd import workloads as wl
from breezetoken_amd.kvcache import SLOT_ALIGN, KVCache, padded_slots


def test_kvcache_keeps_the_reference_views():
    cap, n_kv, dim = 1000, 2, 256
    c = KVCache(cap, n_kv, dim, "cpu")
    assert c.k.shape == (cap, n_kv * dim) and c.k.dtype == torch.bfloat16
    assert c.k.is_contiguous() and c.v.is_contiguous()
    # layers.py:71-78
    row = torch.randn(n_kv * dim)
    c.k[17] = row
    assert torch.equal(c.k[:18].view(18, n_kv, dim)[17].reshape(-1), row.to(torch.bfloat16))
    # graph.py:52-58
    idx = torch.tensor([42])
    c.v.index_copy_(0, idx, row.reshape(1, -1).to(torch.bfloat16))
    kv, vv = c.views()
    assert vv.shape == (cap, n_kv, dim) and torch.equal(vv[42].reshape(-1), row.to(torch.bfloat16))
    # prefill.py:54-55
    c.k[:5] = torch.ones(5, n_kv * dim)
    assert c.k[:5].float().sum().item() == 5 * n_kv * dim
    # padding stays inside one allocation, past the views
    assert c._store.shape[1] == padded_slots(cap) and padded_slots(cap) % SLOT_ALIGN == 0
    assert padded_slots(cap) >= cap + SLOT_ALIGN
    assert c.v.data_ptr() - c.k.data_ptr() == padded_slots(cap) * n_kv * dim * 2


def test_kvcache_rejects_other_dtypes():
    with pytest.raises(ValueError):
        KVCache(16, 2, 256, "cpu", dtype=torch.float32)


def test_c5_ragged_lengths_are_the_documented_draw():
    assert wl.ragged_lengths() == [2591, 8912, 338, 24869, 25539, 3714, 1872, 10204, 432, 2306, 602,
                                   16534, 1872, 261, 3672, 1332, 1813, 7569, 2162, 763, 775, 2974,
                                   1430, 557, 5790, 2822, 1215, 264, 27327, 2799, 549, 521]
    assert sum(wl.ragged_lengths()) == 164380


def test_c5_regions_are_tile_aligned():
    case = wl.c5_inputs(lens=[1, 40, 64])
    assert case.offsets == [0, 32, 96]
    assert case.k.shape == (160, 2, 256)


def test_c3_outlier_rows():
    case = wl.decode_inputs(2, 16, 2, 256, 2048, 1000, outlier_frac=0.01)
    norms = case.k[:1000].float().norm(dim=-1)  # (1000, 2)
    assert int((norms > 4 * 16).sum()) == 20  # round(0.01 * 1000 * 2) rows scaled by 8


def test_algorithmic_work_formulas():
    assert wl.decode_bytes(32768, 8, 2, 256) == 67_125_248
    assert wl.decode_bytes(1024, 8, 2, 256) == 2_113_536
    assert wl.prefill_flops(8192, 8, 256) == 274_911_461_376


def test_backend_needs_a_gpu_device():
    from breezetoken_amd.backend import HipBackend

    with pytest.raises((ValueError, RuntimeError)):
        HipBackend("cpu")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            HipBackend("cuda")
