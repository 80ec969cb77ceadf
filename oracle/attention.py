"""CPU restatement of the reference's GQA attention math (test infrastructure only).

Nothing here is on the product path: ``breezetoken_amd`` never imports this
module.  Every function cites the reference file:line it restates.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

LOG2E = 1.4426950408889634  # breezetoken/kernels/cuda/attention.py:18


# --------------------------------------------------------------------------- #
# torch f32 oracle (the reference's own numerical reference)
# --------------------------------------------------------------------------- #


def torch_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Decode attention, SDPA branch of ``_torch_attention`` (backends.py:196-209).

    q (H, D), k/v (S, Hkv, D) -> (H, D); non-causal, GQA head h reads KV head
    h // (H // Hkv).  Computed in f32 on whatever values the inputs hold.
    """
    if q.ndim != 2 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("attention expects q (H, D), k/v (S, Hkv, D)")
    heads, dim = q.shape
    qq = q.float().reshape(1, heads, 1, dim)
    kk = k.float().permute(1, 0, 2).unsqueeze(0)
    vv = v.float().permute(1, 0, 2).unsqueeze(0)
    out = F.scaled_dot_product_attention(
        qq, kk, vv, dropout_p=0.0, is_causal=False, scale=scale, enable_gqa=True
    )
    return out.reshape(heads, dim)


def torch_attention_einsum(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float
) -> torch.Tensor:
    """Decode attention, einsum fallback branch of ``_torch_attention`` (backends.py:210-215).

    The reference subscripts ``k``/``v`` as ``"ksd"`` (kv head first) although its
    callers pass ``(S, Hkv, D)``; that branch only runs when SDPA raises, which
    torch >= 2.5 with ``enable_gqa`` does not.  This restatement keeps the
    branch's math (grouped einsum + softmax) on the callers' layout, i.e. with
    ``k.permute(1, 0, 2)``, which is what the SDPA branch computes.
    """
    heads, dim = q.shape
    groups = k.shape[1]
    group = heads // groups
    qg = q.float().reshape(groups, group, dim)
    kk = k.float().permute(1, 0, 2)
    vv = v.float().permute(1, 0, 2)
    scores = torch.einsum("kgd,ksd->kgs", qg, kk) * scale
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("kgs,ksd->kgd", probs, vv).reshape(heads, dim)


def torch_prefill_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float
) -> torch.Tensor:
    """Causal GQA prefill attention, SDPA branch of ``_prefill_attn`` (prefill.py:56-68, 78).

    q (S, H, D), k/v (S, Hkv, D) -> (S, H, D) in f32.  Top-left causal (query i
    sees keys 0..i; the prompt starts at position 0, prefill.py:54-55).  The
    sigmoid gate and o-proj that follow (prefill.py:78-79) are outside this path.
    """
    qq = q.float().transpose(0, 1).unsqueeze(0)
    kk = k.float().transpose(0, 1).unsqueeze(0)
    vv = v.float().transpose(0, 1).unsqueeze(0)
    out = F.scaled_dot_product_attention(
        qq, kk, vv, dropout_p=0.0, is_causal=True, scale=scale, enable_gqa=True
    )
    return out[0].transpose(0, 1).contiguous()


def torch_prefill_einsum(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float
) -> torch.Tensor:
    """Causal prefill, einsum + tril fallback branch (prefill.py:69-77); returns (S, H, D).

    As in the decode fallback, the reference subscripts ``k``/``v`` (S, Hkv, D)
    as ``"ksd"``; the restatement applies the branch's math to the callers'
    layout (``k.permute(1, 0, 2)``).
    """
    steps, heads, dim = q.shape
    groups = k.shape[1]
    group = heads // groups
    qg = q.float().reshape(steps, groups, group, dim).permute(1, 2, 0, 3)
    kk = k.float().permute(1, 0, 2)
    vv = v.float().permute(1, 0, 2)
    scores = torch.einsum("kgtd,ksd->kgts", qg, kk) * scale
    mask = torch.ones(steps, steps, dtype=torch.bool).tril()
    scores = scores.masked_fill(~mask, float("-inf"))
    out = torch.einsum("kgts,ksd->kgtd", torch.softmax(scores, dim=-1), vv)
    return out.permute(2, 0, 1, 3).reshape(steps, heads, dim)


def torch_prefill_banded(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos0: int, scale: float
) -> torch.Tensor:
    """Chunked prefill with an explicit causal band, ``Qwen36MoE._attn_batch``
    (qwen36_moe.py:412-428): q (S, H, D) are new tokens at absolute positions
    pos0 .. pos0 + S - 1; k/v (pos0 + S, Hkv, D) the cache up to and including
    them (token-major here; the reference reads the head-major view
    ``k_cache[:, :seq]``, the same values).  Query row j sees keys 0 .. pos0 + j
    (``k_idx <= q_idx``, qwen36_moe.py:414-417).  Returns (S, H, D) in f32.
    """
    steps = q.shape[0]
    seq = pos0 + steps
    k_idx = torch.arange(seq)
    q_idx = pos0 + torch.arange(steps)
    mask = k_idx.unsqueeze(0) <= q_idx.unsqueeze(1)  # (S, seq)
    qq = q.float().transpose(0, 1).unsqueeze(0)
    kk = k.float().transpose(0, 1).unsqueeze(0)
    vv = v.float().transpose(0, 1).unsqueeze(0)
    out = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=scale, enable_gqa=True)
    return out[0].transpose(0, 1).contiguous()


def fixed_decode(
    q: torch.Tensor, k_cap: torch.Tensor, v_cap: torch.Tensor, pos: int, scale: float
) -> torch.Tensor:
    """Fixed-capacity decode contract of ``gqa_decode_fixed`` (attention.py:296-301).

    ``pos`` is the 0-based index of the token being decoded; keys ``j <= pos``
    are valid (valid length = pos + 1, graph.py:52-61, layers.py:71-80).
    Slots past ``pos`` must not influence the result.
    """
    return torch_attention(q, k_cap[: pos + 1], v_cap[: pos + 1], scale)


# --------------------------------------------------------------------------- #
# float64 brute force (independent of torch's SDPA kernels)
# --------------------------------------------------------------------------- #


def brute_force_decode_f64(q, k, v, scale: float) -> np.ndarray:
    """softmax(q_h . K_g^T * scale) V_g for every head h, g = h // (H/Hkv), in float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    heads, dim = q.shape
    groups = k.shape[1]
    group = heads // groups
    out = np.empty((heads, dim), dtype=np.float64)
    for h in range(heads):
        g = h // group
        s = k[:, g, :] @ q[h] * scale
        s = s - s.max()
        p = np.exp(s)
        out[h] = (p @ v[:, g, :]) / p.sum()
    return out


def brute_force_prefill_f64(q, k, v, scale: float, pos0: int = 0) -> np.ndarray:
    """Causal prefill in float64: row i (position pos0 + i) is decode over keys
    0..pos0+i.  q (S, H, D), k/v (pos0 + S, Hkv, D) -> (S, H, D)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    steps, heads, dim = q.shape
    groups = k.shape[1]
    group = heads // groups
    seq = k.shape[0]
    assert seq == pos0 + steps
    band = np.arange(seq)[None, :] <= (pos0 + np.arange(steps))[:, None]
    out = np.empty((steps, heads, dim), dtype=np.float64)
    for h in range(heads):
        g = h // group
        s = (q[:, h, :] @ k[:, g, :].T) * scale  # (S, seq)
        s = np.where(band, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h, :] = (p @ v[:, g, :]) / p.sum(axis=1, keepdims=True)
    return out


# --------------------------------------------------------------------------- #
# split-KV partition, per-split LSE/partials and the LSE combine
# --------------------------------------------------------------------------- #


def split_partition(seqlen: int, num_split: int, block_n: int = 32) -> list[tuple[int, int]]:
    """Token range [begin, end) of every split (attention.py:106-112).

    ``tiles = ceil(seqlen / block_n)``; split s gets ``tiles // num_split +
    (s < tiles % num_split)`` consecutive tiles starting at ``s * base +
    min(s, extra)``; the last tile is clipped to ``seqlen``.
    """
    tiles = -(-seqlen // block_n)
    base, extra = divmod(tiles, num_split)
    out = []
    for s in range(num_split):
        n = base + (1 if s < extra else 0)
        begin = (s * base + min(s, extra)) * block_n
        end = min(seqlen, begin + n * block_n)
        out.append((begin, max(begin, end)))
    return out


def round_robin_partition(seqlen: int, num_split: int, block_n: int) -> list[np.ndarray]:
    """Token indices of every split when tile t (tokens [t*block_n, (t+1)*block_n))
    goes to split t % num_split -- the MI355X kernel's dealing, which replaces the
    contiguous ranges of attention.py:106-112 (the combined output is the same)."""
    idx = np.arange(seqlen)
    tile = idx // block_n
    return [idx[tile % num_split == s] for s in range(num_split)]


def split_decode(q, k, v, scale: float, num_split: int, block_n: int = 32,
                 partition: str = "contiguous"):
    """Per-split (Lse, Part) of ``gqa_decode``'s split kernel (attention.py:114-166), float64.

    Returns ``lse`` (H, NS) in the log2 domain, ``lse = log2(l) + m * scale *
    log2e`` with ``l = sum exp2((s - m) * scale * log2e)``, and ``part`` (H, NS,
    D) = the split's normalised output.  An empty split has lse = -inf and a
    zero partial (attention.py:153-160).  ``partition`` is ``"contiguous"`` (the
    reference, ``split_partition``) or ``"round_robin"`` (``round_robin_partition``).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    heads, dim = q.shape
    groups = k.shape[1]
    group = heads // groups
    c = scale * LOG2E
    lse = np.full((heads, num_split), -np.inf)
    part = np.zeros((heads, num_split, dim))
    if partition == "contiguous":
        rows = [np.arange(b, e) for b, e in split_partition(k.shape[0], num_split, block_n)]
    elif partition == "round_robin":
        rows = round_robin_partition(k.shape[0], num_split, block_n)
    else:
        raise ValueError(f"unknown partition {partition!r}")
    for s, r in enumerate(rows):
        if r.size == 0:
            continue
        for h in range(heads):
            g = h // group
            x = (k[r, g, :] @ q[h]) * c  # log2-domain scores
            m = x.max()
            p = np.exp2(x - m)
            l_sum = p.sum()
            part[h, s] = (p @ v[r, g, :]) / l_sum
            lse[h, s] = math.log2(l_sum) + m
    return lse, part


def combine_lse(lse, part) -> np.ndarray:
    """LSE combine of the second kernel (attention.py:168-189), float64.

    ``tot = log2 sum_s 2^(lse_s - max) + max``; ``out = sum_s 2^(lse_s - tot) part_s``.
    """
    lse = np.asarray(lse, dtype=np.float64)
    part = np.asarray(part, dtype=np.float64)
    mx = lse.max(axis=1, keepdims=True)
    tot = np.log2(np.exp2(lse - mx).sum(axis=1, keepdims=True)) + mx
    w = np.exp2(lse - tot)  # (H, NS); exp2(-inf) = 0 for empty splits
    return np.einsum("hs,hsd->hd", w, part)


# --------------------------------------------------------------------------- #
# helpers shared by tests
# --------------------------------------------------------------------------- #


def compare(got, ref) -> tuple[float, float]:
    """(max-abs error, cosine similarity) of two arrays, in float64."""
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    err = float(np.abs(g - r).max()) if g.size else 0.0
    den = float(np.linalg.norm(g) * np.linalg.norm(r))
    cos = float(g @ r / den) if den > 0 else 1.0
    return err, cos
