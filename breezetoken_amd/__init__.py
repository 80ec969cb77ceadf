"""MI355X-native (gfx950) GQA attention for breezetoken's Qwen3.5 attention layers.

The compute lives in hand-written HIP kernels (``csrc/``) behind the C ABI of
``include/breezetoken_amd.h``; this package is the Python host side:

* ``backend.HipBackend`` -- ``attention`` / ``attention_fixed`` /
  ``attention_prefill`` / ``attention_ragged`` with the reference call
  signatures (breezetoken/backends.py:47-51, 657-706; model/prefill.py:56-68);
* ``kvcache.KVCache`` -- the fixed-capacity bf16 cache with the reference's
  ``(max_context, n_kv * head_dim)`` views (breezetoken/model/config.py:100-111);
* ``workloads`` -- seeded synthetic inputs for the benchmark configurations;
* ``build`` -- compiles ``libbreezetoken_amd.so`` for gfx950.
"""

from .kvcache import KVCache

__all__ = ["KVCache", "HipBackend", "make_backend"]
__version__ = "0.1.0"


def __getattr__(name):
    if name in ("HipBackend", "make_backend"):
        from . import backend

        return getattr(backend, name)
    raise AttributeError(name)
