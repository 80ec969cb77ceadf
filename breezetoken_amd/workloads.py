"""Seeded synthetic inputs for the benchmark configurations.

All draws use ``torch.Generator().manual_seed(seed)`` on the CPU, in the order
q, K, V, values ~ N(0, 1), rounded to bf16 (the KV cache dtype).  Softmax
scale is ``1 / sqrt(head_dim)`` (``attn_scale``, breezetoken/model/config.py:41-43).
The position convention is the reference's: ``pos`` is the 0-based index of the
token being decoded and the valid length is ``pos + 1`` (graph.py:52-61).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

# C5: 32 ragged sequences, lengths log-uniform over [256, 32768].
RAGGED_BATCH = 32
RAGGED_MIN, RAGGED_MAX = 256, 32768


@dataclass
class DecodeCase:
    q: torch.Tensor          # (H, D) bf16
    k: torch.Tensor          # (cap, Hkv, D) bf16
    v: torch.Tensor          # (cap, Hkv, D) bf16
    valid: int               # valid length (pos + 1)
    scale: float

    @property
    def pos(self) -> int:
        return self.valid - 1


def c1_inputs() -> DecodeCase:
    """Config 1: B=1, H=8, Hkv=2, D=256, S=128, seed 0 (the CPU oracle case)."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(8, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(128, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(128, 2, 256, generator=g).to(torch.bfloat16)
    return DecodeCase(q, k, v, 128, 256**-0.5)


def decode_inputs(
    seed: int, heads: int, kv_heads: int, dim: int, cap: int, valid: int,
    outlier_frac: float = 0.0, outlier_scale: float = 8.0,
) -> DecodeCase:
    """q (H, D), K/V (cap, Hkv, D) ~ N(0, 1) bf16; the whole capacity is drawn so
    slots past ``valid`` hold random data that must not affect the result.

    ``outlier_frac`` > 0 (config 3): after drawing q, K, V, ``round(frac * valid *
    Hkv)`` distinct (slot, kv_head) rows among the valid slots are chosen with
    ``torch.randperm`` on the same generator and multiplied by ``outlier_scale``
    before the bf16 rounding.
    """
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(heads, dim, generator=g)
    k = torch.randn(cap, kv_heads, dim, generator=g)
    v = torch.randn(cap, kv_heads, dim, generator=g)
    if outlier_frac > 0:
        n = int(round(outlier_frac * valid * kv_heads))
        rows = torch.randperm(valid * kv_heads, generator=g)[:n]
        kf = k[:valid].reshape(valid * kv_heads, dim)
        kf[rows] *= outlier_scale
    return DecodeCase(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16), valid, dim**-0.5)


def c2_inputs(valid: int, cap: int = 65536) -> DecodeCase:
    """Config 2: Qwen3.5-0.8B-like decode, H=8, Hkv=2, D=256, cap 65536, seed 1."""
    return decode_inputs(1, 8, 2, 256, cap, valid)


def c3_inputs(valid: int, cap: int | None = None) -> DecodeCase:
    """Config 3: 35B-A3B-like decode, H=16, Hkv=2, D=256, 1% of K rows x8, seed 2."""
    return decode_inputs(2, 16, 2, 256, cap or valid, valid, outlier_frac=0.01)


def c4_inputs(steps: int, q_f32: bool = False):
    """Config 4: causal prefill, H=8, Hkv=2, D=256, seed 3: q (S, 8, 256) bf16
    (or the same draws unrounded in f32, as the reference's prefill keeps q),
    k/v (S, 2, 256) bf16."""
    g = torch.Generator().manual_seed(3)
    q = torch.randn(steps, 8, 256, generator=g)
    if not q_f32:
        q = q.to(torch.bfloat16)
    k = torch.randn(steps, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(steps, 2, 256, generator=g).to(torch.bfloat16)
    return q, k, v, 256**-0.5


def ragged_lengths(batch: int = RAGGED_BATCH, seed: int = 4) -> list[int]:
    """Config 5 lengths: floor(exp(ln 256 + u (ln 32768 - ln 256))), u ~ U[0, 1) f64, seed 4."""
    u = torch.rand(batch, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    lo, hi = math.log(RAGGED_MIN), math.log(RAGGED_MAX)
    return [int(math.floor(math.exp(lo + float(x) * (hi - lo)))) for x in u]


@dataclass
class RaggedCase:
    q: torch.Tensor            # (B, H, D) bf16
    k: torch.Tensor            # (slots, Hkv, D) bf16, shared cache
    v: torch.Tensor
    lens: list[int]
    offsets: list[int]         # first slot of each sequence (32-slot aligned regions)
    scale: float


def c5_inputs(lens: list[int] | None = None, heads: int = 8, kv_heads: int = 2, dim: int = 256) -> RaggedCase:
    """Config 5: ragged decode in one shared bf16 cache; each sequence's region is
    padded to a multiple of 32 slots.  q, K, V drawn from a generator seeded 4
    after the lengths."""
    lens = ragged_lengths() if lens is None else list(lens)
    offsets, total = [], 0
    for n in lens:
        offsets.append(total)
        total += -(-n // 32) * 32
    g = torch.Generator().manual_seed(4)
    torch.rand(len(lens), generator=g, dtype=torch.float64)  # the lengths' draw
    q = torch.randn(len(lens), heads, dim, generator=g).to(torch.bfloat16)
    k = torch.randn(total, kv_heads, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(total, kv_heads, dim, generator=g).to(torch.bfloat16)
    return RaggedCase(q, k, v, lens, offsets, dim**-0.5)


def decode_bytes(valid: int, heads: int, kv_heads: int, dim: int) -> int:
    """Algorithmic HBM bytes of one decode call: K+V bf16 of the valid prefix,
    q (f32) read once and the f32 output written once."""
    return 2 * valid * kv_heads * dim * 2 + heads * dim * 4 * 2


def prefill_flops(steps: int, heads: int, dim: int) -> int:
    """Causal prefill flops: 4 * H * D * sum_{i=1..S} i = 2 H D S (S + 1)."""
    return 2 * heads * dim * steps * (steps + 1)
