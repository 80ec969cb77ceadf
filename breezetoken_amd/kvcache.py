"""Fixed-capacity bf16 KV cache laid out for gfx950 HBM3E.

Mirrors the reference ``KVCache`` (breezetoken/model/config.py:100-111): one
layer's ``k`` and ``v`` are ``(max_context, n_kv * head_dim)`` tensors, token
major, so every caller view keeps working unchanged:

* ``cache.k[pos] = k.reshape(-1)``                  (layers.py:71-73)
* ``cache.k[:seq].view(seq, n_kv, head_dim)``       (layers.py:77-78)
* ``cache.k.index_copy_(0, index, k.reshape(1, -1))`` (graph.py:52-53)
* ``cache.k.view(cap, n_kv, head_dim)``             (graph.py:57-58)
* ``cache.k[:steps] = k.reshape(steps, -1)``        (prefill.py:54-55)

Differences from the reference, all below the view contract:

* dtype is bf16 (the reference stores f32, config.py:104-106 with
  qwen35.py:118-121); writers must cast, e.g. ``index_copy_`` needs
  ``k.to(torch.bfloat16)``;
* ``k`` and ``v`` are prefix views of one allocation whose slot count is padded
  up to a multiple of ``SLOT_ALIGN`` (whole 32-token tiles) plus one spare tile,
  and whose base is 256-byte aligned, so the decode kernel's 16-byte loads of a
  partial last tile stay inside the allocation;
* K and V of one layer sit in one allocation (K first), so a layer's cache is a
  single HBM extent.
"""

from __future__ import annotations

import torch

SLOT_ALIGN = 32  # the reference's K/V tile (cap % block_n == 0, attention.py:227-228): two 16-token decode tiles


def padded_slots(capacity: int) -> int:
    return -(-capacity // SLOT_ALIGN) * SLOT_ALIGN + SLOT_ALIGN


class KVCache:
    """One attention layer's bf16 KV cache: ``k``/``v`` are ``(capacity, n_kv*head_dim)``."""

    def __init__(
        self,
        capacity: int,
        n_kv: int,
        head_dim: int,
        device: str | torch.device,
        dtype: torch.dtype = torch.bfloat16,
    ) -> None:
        if capacity <= 0 or n_kv <= 0 or head_dim <= 0:
            raise ValueError("capacity, n_kv and head_dim must be positive")
        if dtype != torch.bfloat16:
            raise ValueError("the MI355X cache is bf16")
        self.capacity = capacity
        self.n_kv = n_kv
        self.head_dim = head_dim
        row = n_kv * head_dim
        slots = padded_slots(capacity)
        self._store = torch.zeros((2, slots, row), device=device, dtype=dtype)
        if self._store.is_cuda and self._store.data_ptr() % 256:
            raise RuntimeError("cache allocation is not 256-byte aligned")
        self.k = self._store[0, :capacity]
        self.v = self._store[1, :capacity]

    @property
    def device(self) -> torch.device:
        return self._store.device

    def views(self) -> tuple[torch.Tensor, torch.Tensor]:
        """``(capacity, n_kv, head_dim)`` views, as the graph path passes them (graph.py:57-58)."""
        shape = (self.capacity, self.n_kv, self.head_dim)
        return self.k.view(shape), self.v.view(shape)

    def reset(self) -> None:
        # Slots are written before they are read (config.py:108-111); nothing to clear.
        pass

    def nbytes(self) -> int:
        return self._store.numel() * self._store.element_size()
