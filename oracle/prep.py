"""CPU restatement of the decode-step preparation ahead of attention (test
infrastructure only: ``breezetoken_amd`` never imports this module).

Restated reference pieces:

* ``rope_tables`` -- the cos/sin tables of ``LayerMixin._rope_tables``
  (breezetoken/model/layers.py:26-32);
* ``torch_rms_norm`` -- ``_torch_rms_norm`` (breezetoken/backends.py:187-189);
* ``torch_rope`` -- ``_torch_rope`` (breezetoken/backends.py:218-226), with the
  position as a Python int instead of a device tensor read by ``.item()``;
* ``attn_prep`` -- the q/k norm + RoPE and cache writes of ``LayerMixin._attn``
  (breezetoken/model/layers.py:58-73), the cache stored bf16;
* ``brute_rms_norm_f64`` / ``brute_rope_f64`` -- per-element float64 loops of
  the same definitions, the rotation written in the partner/sign form of the
  reference's kernel (breezetoken/kernels/cuda/rope.py:31-37) rather than the
  concatenation form of the torch path, so the two formulations check each
  other.
"""

from __future__ import annotations

import numpy as np
import torch


def rope_tables(cap: int, rope_dim: int, theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin (cap, rope_dim) f32 tables (layers.py:26-32): inverse frequencies
    theta^(-i/half) for i < half, phases p * inv, both halves equal."""
    half = rope_dim // 2
    inv = theta ** (-torch.arange(0, half, dtype=torch.float32) / half)
    phases = torch.outer(torch.arange(cap, dtype=torch.float32), inv)
    freqs = torch.cat((phases, phases), dim=-1)
    return freqs.cos(), freqs.sin()


def torch_rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * w over the last dim, in f32 (backends.py:187-189)."""
    xf = x.float()
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def torch_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pos: int, rope_dim: int) -> torch.Tensor:
    """Partial rotate-half RoPE at position ``pos`` (backends.py:218-226)."""
    rot = x[..., :rope_dim].float()
    tail = x[..., rope_dim:].float()
    half = rope_dim // 2
    turned = rot * cos[pos] + torch.cat((-rot[..., half:], rot[..., :half]), dim=-1) * sin[pos]
    return torch.cat((turned, tail), dim=-1).to(x.dtype)


def attn_prep(
    qkv: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, eps: float,
    cos: torch.Tensor, sin: torch.Tensor, pos: int, rope_dim: int,
    heads: int, kv_heads: int, head_dim: int,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The decode-step preparation of layers.py:58-73 on a flat f32 ``qkv``.

    Returns (q (H, D) f32, gate (H, D) f32, k (Hkv, D) f32, v (Hkv, D) f32):
    the values the reference writes into ``cache.k[pos]`` / ``cache.v[pos]``
    before rounding to the cache dtype.
    """
    D = head_dim
    q_size = heads * 2 * D
    kv_size = kv_heads * D
    qg = qkv[:q_size].view(1, heads, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    k = qkv[q_size:q_size + kv_size].view(1, kv_heads, D)
    v = qkv[q_size + kv_size:].view(1, kv_heads, D)
    q = torch_rope(torch_rms_norm(q, q_norm, eps), cos, sin, pos, rope_dim)
    k = torch_rope(torch_rms_norm(k, k_norm, eps), cos, sin, pos, rope_dim)
    return q.reshape(heads, D), gate.reshape(heads, D), k.reshape(kv_heads, D), v.reshape(kv_heads, D)


def brute_rms_norm_f64(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Row by row in float64: x_d / sqrt(sum_j x_j^2 / N + eps) * w_d."""
    x = np.asarray(x, dtype=np.float64)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    n = rows.shape[1]
    for r in range(rows.shape[0]):
        ms = sum(float(v) * float(v) for v in rows[r]) / n
        inv = 1.0 / np.sqrt(ms + eps)
        for d in range(n):
            out[r, d] = rows[r, d] * inv * float(w[d])
    return out.reshape(x.shape)


def brute_rope_f64(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, pos: int, rope_dim: int) -> np.ndarray:
    """Per element in float64, partner/sign form (kernels/cuda/rope.py:31-37):
    y[d] = x[d] cos[pos][d] + sign * x[partner] sin[pos][d] for d < rope_dim."""
    x = np.asarray(x, dtype=np.float64)
    rows = x.reshape(-1, x.shape[-1])
    out = rows.copy()
    half = rope_dim // 2
    for r in range(rows.shape[0]):
        for d in range(rope_dim):
            partner = d + half if d < half else d - half
            sign = -1.0 if d < half else 1.0
            out[r, d] = rows[r, d] * float(cos[pos, d]) + sign * rows[r, partner] * float(sin[pos, d])
    return out.reshape(x.shape)

