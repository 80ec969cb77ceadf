"""Kernel factories with the reference's call signature: ``gqa_decode`` and
``gqa_decode_fixed`` (breezetoken/kernels/cuda/attention.py:54-205, 208-366).

The reference builds one tilelang kernel per shape and returns it; its launch
wrappers (breezetoken/backends.py:523-568) call it with views and freshly
allocated outputs::

    kernel = gqa_decode(heads, groups, dim, scale, num_split=16)
    kernel(Q (1, H, D), K (1, S, Hkv, D), V, Lse (1, H, NS), Part (1, H, NS, D), Out (1, H, D))

    kernel = gqa_decode_fixed(heads, groups, dim, cap, scale, num_split=16)
    kernel(Q, K (1, cap, Hkv, D), V, Pos (1,) int32, Lse, Part, Out)

The factories here return callables of the same shape that run the split and
combine HIP kernels of libbreezetoken_amd.so on torch's current stream, so the
reference's ``_build_attention`` / ``_build_attention_fixed`` need only an
import swap.  The arguments keep their meaning:

* ``Lse`` receives the per-split log2-domain LSE and ``Part`` the normalised
  per-split partials (attention.py:153-166), ``Out`` the combined output
  (attention.py:168-189);
* ``Pos`` holds the 0-based index of the token being decoded: keys
  ``0 .. Pos[0]`` are valid (attention.py:296-301);
* build-time ``ValueError`` for the reference's invalid shapes
  (attention.py:67-70, 227-232) and for shapes these kernels do not serve.

Differences (the combined ``Out`` is the same either way):

* K and V are the bf16 cache (the reference's cache is f32); Q is f32 or bf16,
  ``Out`` f32 or bf16, ``Lse`` and ``Part`` f32;
* tile t of 16 tokens goes to split ``t % num_split`` (round-robin) instead of
  contiguous ranges, so the per-split ``Lse`` / ``Part`` hold a different
  partition of the keys; a split without keys writes ``Lse = -inf`` and leaves
  its ``Part`` row as it was (the combine skips it);
* ``block_h``, ``block_n``, ``threads`` and ``dtype`` are the tilelang tiling
  and element type: they are accepted for the signature and checked where they
  constrain the shape (``heads // groups <= block_h``, ``cap % block_n == 0``).
"""

from __future__ import annotations

from functools import cache

import torch

from . import _lib
from ._lib import BT_DTYPE_BF16, BT_DTYPE_F32, check

SERVED_DIMS = (64, 128, 256)
MAX_GROUP = 8
MAX_SPLITS = 4096


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _code(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float32:
        return BT_DTYPE_F32
    if t.dtype == torch.bfloat16:
        return BT_DTYPE_BF16
    raise ValueError(f"{what} must be float32 or bfloat16, got {t.dtype}")


def _check_build(heads: int, groups: int, dim: int, num_split: int, block_h: int) -> None:
    if heads % groups:
        raise ValueError("heads must be divisible by groups")
    if heads // groups > block_h:
        raise ValueError("the query group must fit in one padded query tile")
    if heads // groups > MAX_GROUP or dim not in SERVED_DIMS:
        raise ValueError(f"heads={heads} groups={groups} dim={dim} is not served (group <= {MAX_GROUP}, "
                         f"dim in {SERVED_DIMS})")
    if not 1 <= num_split <= MAX_SPLITS:
        raise ValueError(f"num_split must be in 1..{MAX_SPLITS}")


class _SplitDecode:
    """The callable ``gqa_decode`` / ``gqa_decode_fixed`` return."""

    def __init__(self, heads: int, groups: int, dim: int, scale: float, num_split: int, cap: int | None):
        self.heads, self.groups, self.dim = heads, groups, dim
        self.scale, self.num_split, self.cap = float(scale), num_split, cap

    def _expect(self, t: torch.Tensor, shape: tuple, what: str) -> None:
        if tuple(t.shape) != shape:
            raise ValueError(f"{what} must have shape {shape}, got {tuple(t.shape)}")

    def __call__(self, *args: torch.Tensor) -> None:
        fixed = self.cap is not None
        if len(args) != (7 if fixed else 6):
            raise TypeError("expected (Q, K, V, Pos, Lse, Part, Out)" if fixed else "expected (Q, K, V, Lse, Part, Out)")
        if fixed:
            q, k, v, pos, lse, part, out = args
        else:
            (q, k, v, lse, part, out), pos = args, None
        H, G, D, NS = self.heads, self.groups, self.dim, self.num_split
        seq = self.cap if fixed else k.shape[1]
        self._expect(q, (1, H, D), "Q")
        self._expect(k, (1, seq, G, D), "K")
        self._expect(v, (1, seq, G, D), "V")
        self._expect(lse, (1, H, NS), "Lse")
        self._expect(part, (1, H, NS, D), "Part")
        self._expect(out, (1, H, D), "Out")
        if seq < 1:
            raise ValueError("K must hold at least one key")
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise ValueError("K and V must be the bf16 cache")
        if lse.dtype != torch.float32 or part.dtype != torch.float32:
            raise ValueError("Lse and Part must be float32")
        q_code, out_code = _code(q, "Q"), _code(out, "Out")
        if k.stride() != v.stride() or k.stride(3) != 1:
            raise ValueError("K and V need identical strides and a unit head_dim stride")
        if not (q.is_contiguous() and lse.is_contiguous() and part.is_contiguous() and out.is_contiguous()):
            raise ValueError("Q, Lse, Part and Out must be contiguous")
        dev = q.device
        tensors = (k, v, lse, part, out) + ((pos,) if fixed else ())
        if any(t.device != dev for t in tensors):
            raise ValueError("all tensors must be on one device")
        if fixed and (pos.dtype != torch.int32 or pos.numel() != 1):
            raise ValueError("Pos must be a device int32 tensor of one element")
        lib = _lib.lib()
        stream = _stream(dev)
        rc = lib.bt_gqa_decode_split(
            q.data_ptr(), q_code, H * D, k.data_ptr(), v.data_ptr(), k.stride(1), k.stride(2),
            None, pos.data_ptr() if fixed else None, None, seq,
            1, H, G, D, NS, self.scale, lse.data_ptr(), part.data_ptr(), stream)
        check("bt_gqa_decode_split", rc)
        rc = lib.bt_gqa_decode_combine(
            lse.data_ptr(), part.data_ptr(), 1, H, D, NS, None, None, NS,
            out.data_ptr(), out_code, H * D, stream)
        check("bt_gqa_decode_combine", rc)


@cache
def gqa_decode(heads: int, groups: int, dim: int, scale: float, num_split: int = 16, block_h: int = 16,
               block_n: int = 32, threads: int = 128, dtype: str = "float32") -> _SplitDecode:
    """Split attention for one batch item (attention.py:54-205):
    ``kernel(Q, K, V, Lse, Part, Out)`` with K/V ``(1, S, Hkv, D)``."""
    _check_build(heads, groups, dim, num_split, block_h)
    return _SplitDecode(heads, groups, dim, scale, num_split, None)


@cache
def gqa_decode_fixed(heads: int, groups: int, dim: int, cap: int, scale: float, num_split: int = 16,
                     block_h: int = 16, block_n: int = 32, threads: int = 128,
                     dtype: str = "float32") -> _SplitDecode:
    """Fixed-capacity variant used by the graph decode path (attention.py:208-366):
    ``kernel(Q, K, V, Pos, Lse, Part, Out)`` with K/V the whole ``(1, cap, Hkv, D)``
    cache and ``Pos`` a device int32; keys past ``Pos[0]`` are masked."""
    if cap % block_n:
        raise ValueError("cap must be a multiple of the K/V tile")
    _check_build(heads, groups, dim, num_split, block_h)
    return _SplitDecode(heads, groups, dim, scale, num_split, cap)
