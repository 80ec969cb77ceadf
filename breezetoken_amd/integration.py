"""Reference-side adapter: ``HipBackend`` behind the reference backend's
``attention`` / ``attention_fixed`` contract, eager fallback included.

The reference's ``TilelangBackend.attention`` (breezetoken/backends.py:657-680)
never raises for a shape: what its kernel does not serve goes to the module's
``_torch_attention`` (backends.py:196-215).  ``attention_fixed``
(backends.py:682-706) does raise ``RuntimeError`` for an unserved shape, and
the graph path takes that as the signal to decode eagerly (graph.py:127-133).

``RocmAttentionMixin`` keeps both rules on top of the HIP kernels:

* ``attention`` runs the decode kernels when ``decode_unserved`` finds nothing
  wrong, and otherwise calls ``attention_fallback`` -- the reference binds its
  own ``_torch_attention`` there.  The decision depends only on shapes, dtypes,
  layout and device, never on whether the library loads: on a GPU a served
  shape with a missing library raises rather than falling back;
* ``attention_fixed`` always goes to ``HipBackend.attention_fixed`` for served
  shapes and raises ``RuntimeError`` otherwise, as the reference does;
* ``prefill_sdpa`` is the drop-in for the prefill SDPA call
  (model/prefill.py:60-68, (1, H, S, D) layout) with ``prefill_fallback``
  (the reference's ``F.scaled_dot_product_attention`` call) for what the
  prefill kernels do not serve.

No fallback is bound here: this package ships no CPU or torch attention.  With
``attention_fallback`` (or ``prefill_fallback``) left ``None`` an unserved call
raises ``RuntimeError`` naming the reason.
"""

from __future__ import annotations

from typing import Callable

import torch

from .backend import HipBackend, decode_unserved, prefill_unserved


class RocmAttentionMixin:
    """Mix into the reference backend class (it provides ``self.device``).

    ``attention_fallback(q, k, v, scale) -> (H, D)`` and
    ``prefill_fallback(qq, kk, vv, scale, q_offset) -> (1, H, S, D)`` are
    class or instance attributes the integrating code sets."""

    attention_fallback: Callable | None = None
    prefill_fallback: Callable | None = None

    def _hip(self) -> HipBackend:
        hip = getattr(self, "_hip_backend", None)
        if hip is None:
            hip = HipBackend(self.device)
            self._hip_backend = hip
        return hip

    def _gpu(self) -> torch.device | None:
        """The backend's GPU, or None on a CPU backend (then nothing is served)."""
        dev = torch.device(self.device)
        if dev.type != "cuda":
            return None
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        return dev

    def _fallback(self, fn: Callable | None, what: str, reason: str):
        if fn is None:
            raise RuntimeError(f"{what} is not served here ({reason}) and no fallback is bound")
        return fn

    def attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
        """Eager decode (backends.py:657-680): q (H, D), k/v (S, Hkv, D) -> (H, D)."""
        gpu = self._gpu()
        reason = "the backend device is not a GPU" if gpu is None else decode_unserved(q, k, v, gpu)
        if reason is None:
            return self._hip().attention(q, k, v, scale)
        return self._fallback(self.attention_fallback, "attention", reason)(q, k, v, scale)

    def attention_fixed(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                        scale: float) -> torch.Tensor:
        """Graph-path decode (backends.py:682-706); unserved shapes raise."""
        gpu = self._gpu()
        reason = "the backend device is not a GPU" if gpu is None else decode_unserved(q, k, v, gpu)
        if reason is not None:
            raise RuntimeError(f"fixed attention is not served for this call: {reason}")
        return self._hip().attention_fixed(q, k, v, pos, scale)

    def prefill_sdpa(self, qq: torch.Tensor, kk: torch.Tensor, vv: torch.Tensor, scale: float,
                     out_dtype: torch.dtype = torch.float32, q_offset: int = 0) -> torch.Tensor:
        """Causal prefill SDPA (prefill.py:60-68; qwen36_moe.py:415-423 with
        q_offset > 0): qq (1, H, S, D), kk/vv (1, Hkv, q_offset + S, D) ->
        (1, H, S, D) in ``out_dtype``."""
        gpu = self._gpu()
        if gpu is None:
            reason = "the backend device is not a GPU"
        elif qq.ndim != 4 or kk.ndim != 4 or qq.shape[0] != 1 or kk.shape[0] != 1 or vv.shape != kk.shape:
            reason = "prefill expects qq (1, H, S, D), kk/vv (1, Hkv, q_offset + S, D)"
        else:
            reason = prefill_unserved(qq[0].transpose(0, 1), kk[0].transpose(0, 1), vv[0].transpose(0, 1),
                                      int(q_offset), gpu)
        if reason is None:
            return self._hip().sdpa_prefill(qq, kk, vv, scale, out_dtype, q_offset=q_offset)
        out = self._fallback(self.prefill_fallback, "prefill", reason)(qq, kk, vv, scale, q_offset)
        return out.to(out_dtype)
