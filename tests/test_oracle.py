"""Pin the CPU oracle before trusting it (no GPU needed).

Each oracle function is checked against something it does not share code with:
the other torch branch the reference ships, an independent float64 brute force,
closed forms, invariants and split/combine identities.  Planted mistakes (a
wrong GQA head mapping, a dropped scale, a wrong causal diagonal, a skipped
rescale in the combine) are shown to fail the same checks, so the checks
discriminate.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as orc

H, HKV, D = 8, 2, 256
SCALE = D**-0.5


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16).float()


def _decode_inputs(seq, seed=0, heads=H, kv=HKV, dim=D):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(heads, dim, generator=g).to(torch.bfloat16).float()
    k = torch.randn(seq, kv, dim, generator=g).to(torch.bfloat16).float()
    v = torch.randn(seq, kv, dim, generator=g).to(torch.bfloat16).float()
    return q, k, v


# ----------------------------------------------------------------- decode
@pytest.mark.parametrize("seq", [1, 17, 128, 300])
def test_sdpa_branch_matches_einsum_branch(seq):
    q, k, v = _decode_inputs(seq, seed=seq)
    a = orc.torch_attention(q, k, v, SCALE)
    b = orc.torch_attention_einsum(q, k, v, SCALE)
    assert (a - b).abs().max().item() < 2e-6


@pytest.mark.parametrize("seq,heads,kv", [(1, 8, 2), (33, 8, 2), (128, 16, 2), (77, 4, 4), (50, 8, 1)])
def test_torch_oracle_matches_f64_brute_force(seq, heads, kv):
    q, k, v = _decode_inputs(seq, seed=seq + heads, heads=heads, kv=kv)
    got = orc.torch_attention(q, k, v, SCALE).numpy()
    ref = orc.brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    err, cos = orc.compare(got, ref)
    assert err < 1e-5 and cos > 1 - 1e-9


def test_planted_wrong_head_mapping_is_caught():
    """An oracle that maps head h to kv head h % Hkv (instead of h // group) fails the f64 check."""
    q, k, v = _decode_inputs(64, seed=3)
    group = H // HKV
    wrong = torch.stack(
        [orc.torch_attention(q[h : h + 1], k[:, h % HKV : h % HKV + 1], v[:, h % HKV : h % HKV + 1], SCALE)[0]
         for h in range(H)]
    )
    right = torch.stack(
        [orc.torch_attention(q[h : h + 1], k[:, h // group : h // group + 1], v[:, h // group : h // group + 1], SCALE)[0]
         for h in range(H)]
    )
    ref = orc.brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    assert orc.compare(right.numpy(), ref)[0] < 1e-5
    assert orc.compare(wrong.numpy(), ref)[0] > 1e-2


def test_planted_dropped_scale_is_caught():
    q, k, v = _decode_inputs(64, seed=4)
    ref = orc.brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    bad = orc.torch_attention(q, k, v, 1.0).numpy()
    assert orc.compare(bad, ref)[0] > 1e-2


def test_closed_form_single_key():
    """S = 1: softmax of one score is 1, so out[h] = V[0, h // group]."""
    q, k, v = _decode_inputs(1, seed=5)
    out = orc.torch_attention(q, k, v, SCALE)
    for h in range(H):
        assert torch.allclose(out[h], v[0, h // (H // HKV)], atol=1e-6)


def test_closed_form_equal_keys_give_mean_of_v():
    q, _, v = _decode_inputs(40, seed=6)
    k = _rand((1, HKV, D), 7).expand(40, HKV, D).contiguous()
    out = orc.torch_attention(q, k, v, SCALE)
    mean = v.mean(dim=0)  # (Hkv, D)
    for h in range(H):
        assert torch.allclose(out[h], mean[h // (H // HKV)], atol=1e-5)


def test_closed_form_dominant_key():
    """A key aligned with q and scaled far above the rest takes all the weight."""
    q, k, v = _decode_inputs(50, seed=8)
    group = H // HKV
    for g in range(HKV):
        k[23, g] = q[g * group] * 40.0  # only head g*group is dominated
    out = orc.torch_attention(q, k, v, SCALE)
    for g in range(HKV):
        assert torch.allclose(out[g * group], v[23, g], atol=1e-5)


def test_closed_form_constant_v():
    q, k, _ = _decode_inputs(70, seed=9)
    v = torch.full((70, HKV, D), 0.375)
    out = orc.torch_attention(q, k, v, SCALE)
    assert torch.allclose(out, torch.full_like(out, 0.375), atol=1e-6)


def test_permutation_invariance():
    q, k, v = _decode_inputs(90, seed=10)
    perm = torch.randperm(90, generator=torch.Generator().manual_seed(1))
    a = orc.torch_attention(q, k, v, SCALE)
    b = orc.torch_attention(q, k[perm], v[perm], SCALE)
    assert (a - b).abs().max().item() < 1e-6


def test_fixed_decode_ignores_slots_past_pos():
    q, k, v = _decode_inputs(256, seed=11)
    pos = 99
    a = orc.fixed_decode(q, k, v, pos, SCALE)
    k2, v2 = k.clone(), v.clone()
    k2[pos + 1 :] = 1e4
    v2[pos + 1 :] = float("nan")
    b = orc.fixed_decode(q, k2, v2, pos, SCALE)
    assert torch.equal(a, b)
    assert torch.allclose(a, orc.torch_attention(q, k[: pos + 1], v[: pos + 1], SCALE))


# ----------------------------------------------------------- split + combine
@pytest.mark.parametrize("seq,tiles_per", [(1, 1), (31, 1), (32, 1), (33, 1), (1000, 32), (4096, 32)])
@pytest.mark.parametrize("ns", [1, 2, 3, 16, 64])
def test_split_partition_covers_context(seq, tiles_per, ns):
    parts = orc.split_partition(seq, ns, 32)
    assert len(parts) == ns
    full = [(b, e) for b, e in parts if e > b]
    # non-empty splits tile [0, seq) contiguously, in split order
    assert full[0][0] == 0 and full[-1][1] == seq
    for (_, e0), (b1, _) in zip(full, full[1:]):
        assert e0 == b1
    assert all(e == b for b, e in parts[len(full):])  # empty splits come last
    tiles = [-(-(e - b) // 32) for b, e in parts]
    # the first `extra` splits carry the extra tile (attention.py:106-112)
    total = -(-seq // 32)
    base, extra = divmod(total, ns)
    assert tiles == [base + (1 if s < extra else 0) for s in range(ns)]


@pytest.mark.parametrize("seq,ns,block", [(1, 4, 32), (100, 3, 16), (1000, 16, 32), (1000, 7, 16), (33, 2, 32)])
def test_round_robin_partition_covers_every_token_once(seq, ns, block):
    parts = orc.round_robin_partition(seq, ns, block)
    allidx = np.sort(np.concatenate(parts))
    assert np.array_equal(allidx, np.arange(seq))
    for s, r in enumerate(parts):
        assert np.all((r // block) % ns == s)


@pytest.mark.parametrize("partition", ["contiguous", "round_robin"])
@pytest.mark.parametrize("seq", [1, 17, 100, 128, 1000])
@pytest.mark.parametrize("ns", [1, 2, 3, 5, 16, 64])
def test_combine_of_splits_equals_unsplit(seq, ns, partition):
    q, k, v = _decode_inputs(seq, seed=seq * 7 + ns)
    lse, part = orc.split_decode(q.numpy(), k.numpy(), v.numpy(), SCALE, ns, partition=partition)
    out = orc.combine_lse(lse, part)
    ref = orc.brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    assert orc.compare(out, ref)[0] < 1e-12


@pytest.mark.parametrize("partition", ["contiguous", "round_robin"])
def test_empty_split_rule(partition):
    q, k, v = _decode_inputs(40, seed=12)  # 2 tiles, 16 splits -> 14 empty
    lse, part = orc.split_decode(q.numpy(), k.numpy(), v.numpy(), SCALE, 16, partition=partition)
    assert np.isneginf(lse[:, 2:]).all()
    assert np.all(part[:, 2:] == 0)
    assert np.isfinite(lse[:, :2]).all()


def test_lse_closed_form():
    """One split: lse = log2 sum_j 2^(q.k_j * scale * log2e) (the log2-domain convention)."""
    q, k, v = _decode_inputs(20, seed=13)
    lse, _ = orc.split_decode(q.numpy(), k.numpy(), v.numpy(), SCALE, 1)
    qd, kd = q.double().numpy(), k.double().numpy()
    for h in range(H):
        x = kd[:, h // (H // HKV)] @ qd[h] * SCALE * math.log2(math.e)
        assert abs(lse[h, 0] - math.log2(sum(2.0**xi for xi in x))) < 1e-9


def test_planted_combine_without_rescale_is_caught():
    """A combine that averages partials without the LSE weights disagrees with the unsplit result."""
    q, k, v = _decode_inputs(500, seed=14)
    lse, part = orc.split_decode(q.numpy(), k.numpy(), v.numpy(), SCALE, 8)
    bad = part.mean(axis=1)
    ref = orc.brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    assert orc.compare(bad, ref)[0] > 1e-3
    assert orc.compare(orc.combine_lse(lse, part), ref)[0] < 1e-12


# ----------------------------------------------------------------- prefill
def _prefill_inputs(steps, seed=0, heads=H, kv=HKV, dim=D):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(steps, heads, dim, generator=g).to(torch.bfloat16).float()
    k = torch.randn(steps, kv, dim, generator=g).to(torch.bfloat16).float()
    v = torch.randn(steps, kv, dim, generator=g).to(torch.bfloat16).float()
    return q, k, v


@pytest.mark.parametrize("steps", [1, 7, 64, 130])
def test_prefill_branches_agree_and_match_f64(steps):
    q, k, v = _prefill_inputs(steps, seed=steps)
    a = orc.torch_prefill_attention(q, k, v, SCALE)
    b = orc.torch_prefill_einsum(q, k, v, SCALE)
    ref = orc.brute_force_prefill_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    assert (a - b).abs().max().item() < 2e-6
    assert orc.compare(a.numpy(), ref)[0] < 1e-5


def test_prefill_row_i_is_decode_over_prefix():
    q, k, v = _prefill_inputs(48, seed=15)
    out = orc.torch_prefill_attention(q, k, v, SCALE)
    for i in (0, 1, 17, 31, 32, 47):
        dec = orc.torch_attention(q[i], k[: i + 1], v[: i + 1], SCALE)
        assert (out[i] - dec).abs().max().item() < 2e-6
    group = H // HKV
    for h in range(H):
        assert torch.allclose(out[0, h], v[0, h // group], atol=1e-6)


# ----------------------------------------------------------- chunked prefill
@pytest.mark.parametrize("pos0,steps", [(0, 40), (5, 1), (17, 23), (64, 64), (100, 7)])
def test_banded_prefill_matches_f64_with_offset(pos0, steps):
    q, k, v = _prefill_inputs(pos0 + steps, seed=pos0 * 7 + steps)
    out = orc.torch_prefill_banded(q[pos0:], k, v, pos0, SCALE)
    ref = orc.brute_force_prefill_f64(q[pos0:].numpy(), k.numpy(), v.numpy(), SCALE, pos0=pos0)
    assert out.shape == (steps, H, D)
    assert orc.compare(out.numpy(), ref)[0] < 1e-5


def test_banded_prefill_zero_offset_is_causal_prefill():
    q, k, v = _prefill_inputs(50, seed=21)
    a = orc.torch_prefill_banded(q, k, v, 0, SCALE)
    b = orc.torch_prefill_attention(q, k, v, SCALE)
    assert (a - b).abs().max().item() < 2e-6


def test_chunked_prefill_equals_full_prefill_rows():
    """Prefilling [0, 96) at once and prefilling [40, 96) after [0, 40) give the
    same rows for positions 40..95 (qwen36_moe.py:394-428 vs prefill.py:56-68)."""
    q, k, v = _prefill_inputs(96, seed=22)
    full = orc.torch_prefill_attention(q, k, v, SCALE)
    chunk = orc.torch_prefill_banded(q[40:], k, v, 40, SCALE)
    assert (full[40:] - chunk).abs().max().item() < 2e-6


def test_planted_top_left_mask_for_chunk_is_caught():
    """``is_causal=True`` with S < seq aligns the mask top-left (row j sees keys
    0..j), which is what the reference's explicit band avoids
    (qwen36_moe.py:412-413); that mistake fails the f64 check."""
    q, k, v = _prefill_inputs(60, seed=23)
    pos0 = 36
    ref = orc.brute_force_prefill_f64(q[pos0:].numpy(), k.numpy(), v.numpy(), SCALE, pos0=pos0)
    qq = q[pos0:].transpose(0, 1).unsqueeze(0)
    kk = k.transpose(0, 1).unsqueeze(0)
    vv = v.transpose(0, 1).unsqueeze(0)
    bad = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True, scale=SCALE,
                                                           enable_gqa=True)
    assert orc.compare(bad[0].transpose(0, 1).numpy(), ref)[0] > 1e-2


def test_planted_wrong_causal_diagonal_is_caught():
    """Masking j < i (excluding the diagonal) instead of j <= i fails the f64 check."""
    q, k, v = _prefill_inputs(24, seed=16)
    ref = orc.brute_force_prefill_f64(q.numpy(), k.numpy(), v.numpy(), SCALE)
    qq = q.transpose(0, 1).unsqueeze(0)
    kk = k.repeat_interleave(H // HKV, dim=1).transpose(0, 1).unsqueeze(0)
    vv = v.repeat_interleave(H // HKV, dim=1).transpose(0, 1).unsqueeze(0)
    mask = torch.ones(24, 24, dtype=torch.bool).tril(diagonal=-1)
    mask[0, 0] = True  # keep row 0 defined
    bad = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=SCALE)
    bad = bad[0].transpose(0, 1).numpy()
    assert orc.compare(bad, ref)[0] > 1e-2
