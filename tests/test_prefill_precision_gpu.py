"""Prefill precision on the GPU: f32 q as the reference computes it, and V of
any bf16 magnitude.

* The reference keeps q in f32 through RMSNorm/RoPE into SDPA
  (breezetoken/model/prefill.py:49-68).  bt_gqa_prefill takes that f32 q as
  two fp16 terms after a power-of-two scale per row (hi + lo, ~22 significant
  bits) and is held to the parity gate (max-abs 2e-3, cosine 0.99999) against
  the oracle's f32 SDPA on the same unrounded q, at unit scores and at score
  standard deviations of 2 to 16 on every prefill path.
* V enters P.V as fp16 scaled by a power of two per 64-key block, so bf16 V
  beyond fp16's range (|v| > 65504) or deep in its subnormals (|v| ~ 1e-5 and
  below) must still match.  Each prefill kernel path is run on V patterns with
  uniform, outlier-row, alternating-block, zero-block and falling magnitudes.
  The gate scales with the data: |got - ref| <= 2e-3 * A(|V|) elementwise,
  A(|V|) the oracle's attention over |V| (the magnitude each output averages;
  for unit-variance V it is ~0.8, i.e. the usual 2e-3 gate), plus cosine
  0.99999.  Magnitude changes fall on 64-key block boundaries: inside one
  block the image keeps values down to 2^-25 of the block's largest (fp16's
  normal range), so a row whose keys mix 1e-20 and 1e3 within one block
  loses the small ones -- the one limit of the per-block scale.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from breezetoken_amd import workloads as wl
from oracle import attention as orc

pytestmark = pytest.mark.gpu

ATOL = 2e-3
COS = 0.99999


@pytest.mark.parametrize("steps", [128, 2048])
def test_c4_prefill_f32_q_matches_reference_arithmetic(hip_backend, steps):
    q, k, v, scale = wl.c4_inputs(steps, q_f32=True)
    assert q.dtype == torch.float32
    ref = orc.torch_prefill_attention(q, k.float(), v.float(), scale)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    err, cos = orc.compare(out.numpy(), ref.numpy())
    print(f"[c4 f32 q] S={steps}: max-abs {err:.3e} cosine {cos:.9f}", flush=True)
    assert err <= ATOL and cos >= COS


def test_c4_prefill_8192_f32_q_full_output(hip_backend):
    """The benchmark shape with f32 q: every row against the oracle's f32 SDPA."""
    q, k, v, scale = wl.c4_inputs(8192, q_f32=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    ref = orc.torch_prefill_attention(q, k.float(), v.float(), scale)
    err, cos = orc.compare(out.numpy(), ref.numpy())
    print(f"[c4 f32 q] S=8192: max-abs {err:.3e} cosine {cos:.9f}", flush=True)
    assert err <= ATOL and cos >= COS


def test_c4_prefill_8192_f32_q_sampled_rows(hip_backend):
    """The benchmark shape with f32 q: sampled rows against decode attention
    over keys 0..i in f32."""
    q, k, v, scale = wl.c4_inputs(8192, q_f32=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    for i in [0, 1, 31, 32, 63, 64, 1000, 4095, 4096, 8000, 8190, 8191]:
        ref = orc.torch_attention(q[i], k[: i + 1].float(), v[: i + 1].float(), scale)
        err, cos = orc.compare(out[i].numpy(), ref.numpy())
        assert err <= ATOL and cos >= COS, (i, err, cos)


def test_c4_prefill_f32_q_error_below_bf16_q(hip_backend):
    """Taking q as scaled fp16 must beat rounding it to bf16 (which alone misses the gate)."""
    q, k, v, scale = wl.c4_inputs(512, q_f32=True)
    ref = orc.torch_prefill_attention(q, k.float(), v.float(), scale).numpy()
    e32, _ = orc.compare(hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu().numpy(), ref)
    qb = q.to(torch.bfloat16)
    e16, _ = orc.compare(hip_backend.attention_prefill(qb.cuda(), k.cuda(), v.cuda(), scale).cpu().numpy(), ref)
    print(f"[c4 S=512] max-abs vs f32-q reference: f32 q {e32:.3e}, bf16 q {e16:.3e}", flush=True)
    assert e32 < e16


def _v_pattern(name: str, kv_len: int, kv: int, dim: int, g: torch.Generator) -> torch.Tensor:
    v = torch.randn(kv_len, kv, dim, generator=g)
    blk = torch.arange(kv_len) // 64
    if name.startswith("uniform_"):
        v = v * float(name.split("_")[1])
    elif name == "outlier_rows_1e5":
        v[::37] *= 1e5
    elif name == "alternating_blocks":
        v = v * torch.where(blk % 2 == 0, 1e3, 1e-3).view(-1, 1, 1)
    elif name == "zero_blocks":
        v[(blk == 0) | (blk == 2)] = 0.0
    elif name == "big_then_tiny":
        v = v * torch.where(blk < 2, 1e4, 1e-4).view(-1, 1, 1)
    elif name == "tiny_then_big":
        v = v * torch.where(blk < 2, 1e-20, 1e3).view(-1, 1, 1)
    else:
        raise ValueError(name)
    return v.to(torch.bfloat16)


V_PATTERNS = ["uniform_3e4", "uniform_1e5", "uniform_1e-5", "uniform_1e-30", "outlier_rows_1e5",
              "alternating_blocks", "zero_blocks", "big_then_tiny", "tiny_then_big"]
# (name, heads, kv, dim, steps, q_offset, q dtype, split_keys): the pair kernel
# (its grid fills 256 CUs: 16 kv heads x 1024 / 64 query-block pairs), the
# two-waves-per-SIMD kernel alone and with split keys (short prompts), and a
# group of 3 (run as three single-head subsets).
PATHS = [
    ("pair_f32q", 64, 16, 128, 1024, 0, torch.float32, True),
    ("pair_bf16q", 64, 16, 128, 1024, 0, torch.bfloat16, True),
    ("prefill8_f32q", 8, 2, 256, 320, 0, torch.float32, False),
    ("prefill8_split_bf16q", 8, 2, 128, 96, 640, torch.bfloat16, True),
    ("group3_f32q", 6, 2, 128, 200, 0, torch.float32, True),
]


@pytest.mark.parametrize("pattern", V_PATTERNS)
@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
def test_prefill_v_magnitudes(hip_backend, path, pattern):
    name, heads, kv, dim, steps, pos0, qdt, split = path
    print(f"[v-range] {name} {pattern}", flush=True)
    g = torch.Generator().manual_seed(11)
    q = torch.randn(steps, heads, dim, generator=g).to(qdt)
    k = torch.randn(pos0 + steps, kv, dim, generator=g).to(torch.bfloat16)
    v = _v_pattern(pattern, pos0 + steps, kv, dim, g)
    scale = dim**-0.5
    ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), pos0, scale)
    mag = orc.torch_prefill_banded(q.float(), k.float(), v.float().abs(), pos0, scale)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=pos0, split_keys=split).cpu()
    assert torch.isfinite(out).all(), "non-finite output"
    excess = ((out - ref).abs() / (ATOL * mag).clamp_min(1e-38)).max().item()
    _, cos = orc.compare(out.numpy().astype(np.float64), ref.numpy().astype(np.float64))
    print(f"    error / (2e-3 * A(|V|)) max {excess:.3f}, cosine {cos:.9f}", flush=True)
    assert excess <= 1.0 and cos >= COS


# ------------------------------------- f32 q at the score scales of a real model
# q/k RMSNorm weights of 2-3 give scores (logits) with a standard deviation of
# 4-9; taken as a single fp16 term, f32 q's rounding error in the scores grows
# with |q|.|k| and crosses the 2e-3 gate from a standard deviation of about 2.
# Every prefill path takes f32 q as two fp16 terms (hi + lo), which keeps the
# scores at f32 q's precision at any scale.  Inputs: q ~ N(0, 1) f32 and K ~
# N(0, 1) bf16, both scaled by sqrt(std), so q.k * D^-0.5 has standard deviation
# `std`; "blockwise" also scales every 64-key block of K by 1, 2 or 4.
SCALE_PATHS = [
    # (name, heads, kv, dim, steps, q_offset, split_keys)
    ("prefill8", 8, 2, 256, 300, 0, False),
    ("split_keys", 8, 2, 256, 300, 0, True),
    ("direct_tiles", 8, 2, 256, 100, 0, True),
    ("paired_split", 8, 2, 256, 3000, 0, True),
    ("chunked", 16, 2, 256, 300, 1000, True),
    ("group6_subsets", 12, 2, 256, 500, 0, True),
    ("group3_d128", 6, 2, 128, 400, 37, True),
    ("pair_d128", 64, 16, 128, 1024, 0, True),
]


def _scaled(steps, heads, kv, dim, q_offset, std, blockwise=False, seed=7):
    g = torch.Generator().manual_seed(seed + steps + 13 * heads + q_offset)
    a = math.sqrt(std)
    q = torch.randn(steps, heads, dim, generator=g) * a
    k = torch.randn(q_offset + steps, kv, dim, generator=g) * a
    if blockwise:
        k = k * (2.0 ** (torch.arange(q_offset + steps) // 64 % 3)).view(-1, 1, 1) / 2.0
    v = torch.randn(q_offset + steps, kv, dim, generator=g)
    return q, k.to(torch.bfloat16), v.to(torch.bfloat16), dim**-0.5


def _check_scaled(hip_backend, path, std, blockwise=False):
    name, heads, kv, dim, steps, pos0, split = path
    q, k, v, scale = _scaled(steps, heads, kv, dim, pos0, std, blockwise)
    print(f"[f32 q, score std {std}{' blockwise' if blockwise else ''}] {name}", flush=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=pos0, split_keys=split).cpu()
    ref = orc.torch_prefill_banded(q, k.float(), v.float(), pos0, scale)
    err, cos = orc.compare(out.numpy(), ref.numpy())
    print(f"    max-abs {err:.3e} cosine {cos:.9f}", flush=True)
    assert err <= ATOL and cos >= COS


@pytest.mark.parametrize("std", [2, 4, 8, 16])
@pytest.mark.parametrize("path", SCALE_PATHS, ids=[p[0] for p in SCALE_PATHS])
def test_f32_q_score_scales(hip_backend, path, std):
    _check_scaled(hip_backend, path, std)


@pytest.mark.parametrize("path", SCALE_PATHS[:2], ids=[p[0] for p in SCALE_PATHS[:2]])
def test_f32_q_blockwise_key_scales(hip_backend, path):
    """K blocks at 1x, 2x and 4x one another (the per-block K scale moves with them)."""
    _check_scaled(hip_backend, path, 8, blockwise=True)


@pytest.mark.parametrize("std", [4, 16])
def test_f32_q_score_scales_c4_8192(hip_backend, std):
    """Config 4's longest prompt on the pair kernel with f32 q at large score
    scales: every row against the oracle."""
    _check_scaled(hip_backend, ("pair_c4_8192", 8, 2, 256, 8192, 0, True), std)


def test_f32_q_lo_term_matters(hip_backend):
    """The lo term is what carries the precision: dropping it from the oracle's
    q (q rounded to one fp16 term per row scale, as the hi term alone would
    compute) misses the gate at score std 8, while the kernel meets it."""
    steps, heads, kv, dim = 300, 8, 2, 256
    q, k, v, scale = _scaled(steps, heads, kv, dim, 0, 8)
    e = torch.floor(torch.log2(q.abs().amax(-1, keepdim=True))) - 14
    q_hi = (q * torch.exp2(-e)).half().float() * torch.exp2(e)
    ref = orc.torch_prefill_attention(q, k.float(), v.float(), scale).numpy()
    hi_only, _ = orc.compare(orc.torch_prefill_attention(q_hi, k.float(), v.float(), scale).numpy(), ref)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu().numpy()
    err, _ = orc.compare(out, ref)
    print(f"[lo term] score std 8: hi only {hi_only:.3e}, kernel {err:.3e}", flush=True)
    assert hi_only > ATOL and err <= ATOL
