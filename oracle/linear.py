"""CPU restatement of the decode matvec (test infrastructure only:
``breezetoken_amd`` never imports this module).

* ``torch_linear`` -- ``_torch_linear`` (breezetoken/backends.py:182-184),
  x.float() @ w.float() flattened: the definition the reference's split-K bf16
  GEMV (kernels/cuda/gemv.py:18-40) is tested against (tests/test_cuda.py:28-32).
* ``split_k_linear`` -- the same product as per-share partial sums added in
  share order (gemv.py:18-40 + backends.py:327-331), in float64.
"""

from __future__ import annotations

import numpy as np
import torch


def torch_linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x (..., K) times w (K, N) in f32 -> (N,) (backends.py:182-184)."""
    return (x.reshape(-1).float() @ w.float()).reshape(-1)


def split_k_linear(x, w, splits: int) -> np.ndarray:
    """sum over s of x[ks] . w[ks, :] for the ``splits`` consecutive shares of
    K, in float64; any share count gives the same product."""
    x = np.asarray(x.float() if isinstance(x, torch.Tensor) else x, dtype=np.float64).reshape(-1)
    w = np.asarray(w.float() if isinstance(w, torch.Tensor) else w, dtype=np.float64)
    K = x.shape[0]
    per = -(-K // splits)
    parts = [x[s * per:(s + 1) * per] @ w[s * per:(s + 1) * per] for s in range(splits)]
    out = np.zeros(w.shape[1])
    for p in parts:
        out += p
    return out
