"""CPU restatement of the Gated DeltaNet decode step (test infrastructure only:
``breezetoken_amd`` never imports this module).

* ``torch_gdn_decode`` -- ``_torch_gdn_decode`` (breezetoken/backends.py:242-271),
  the contract of ``Backend.gdn_decode`` (backends.py:79-92) that the
  reference's kernel (kernels/cuda/gdn.py:31-139) is tested against;
* ``brute_gdn_decode_f64`` -- the same step as float64 loops over heads, key
  rows and value columns, written from the update rule rather than from the
  einsum form, so the two check each other.
"""

from __future__ import annotations

import numpy as np
import torch

def torch_gdn_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                     state: torch.Tensor, scale: float, eps: float = 1e-6) -> torch.Tensor:
    """One gated-delta-rule step, ``state`` (Hv, D, D) f32 updated in place
    (``_torch_gdn_decode``, breezetoken/backends.py:242-271): q/k L2-normalised
    (q also scaled), state decayed by exp(g), recall kn.S, delta (v - recall)
    sigmoid(beta), S += kn (x) delta, output qn.S; value head h reads key head
    h % Hk."""
    heads_k, dim = q.shape
    heads_v = v.shape[0]
    qf, kf, vf = q.float(), k.float(), v.float()
    qn = qf * torch.rsqrt(qf.pow(2).sum(dim=-1, keepdim=True) + eps) * scale
    kn = kf * torch.rsqrt(kf.pow(2).sum(dim=-1, keepdim=True) + eps)
    index = torch.arange(heads_v) % heads_k
    decayed = state * torch.exp(g.float()).view(heads_v, 1, 1)
    recalled = torch.einsum("hdv,hd->hv", decayed, kn[index])
    delta = (vf - recalled) * torch.sigmoid(beta.float()).unsqueeze(-1)
    state.copy_(decayed + kn[index].unsqueeze(-1) * delta.unsqueeze(-2))
    return torch.einsum("hdv,hd->hv", state, qn[index])


def brute_gdn_decode_f64(q, k, v, g, beta, state, scale: float, eps: float = 1e-6):
    """The same step in float64 with explicit loops over heads, key rows and
    value columns; returns (out, new_state) and leaves ``state`` unchanged."""
    def f64(x):
        return (x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)).astype(np.float64)

    q, k, v, g, beta = f64(q), f64(k), f64(v), f64(g), f64(beta)
    st = f64(state).copy()
    heads_k, dim = q.shape
    heads_v = v.shape[0]
    out = np.zeros((heads_v, dim))
    for h in range(heads_v):
        kh = h % heads_k
        qn = q[kh] / np.sqrt(np.dot(q[kh], q[kh]) + eps) * scale
        kn = k[kh] / np.sqrt(np.dot(k[kh], k[kh]) + eps)
        decay = np.exp(g[h])
        b = 1.0 / (1.0 + np.exp(-beta[h]))
        s = st[h] * decay
        for j in range(dim):
            recall = sum(s[i, j] * kn[i] for i in range(dim))
            delta = (v[h, j] - recall) * b
            for i in range(dim):
                s[i, j] += kn[i] * delta
            out[h, j] = sum(s[i, j] * qn[i] for i in range(dim))
        st[h] = s
    return out, st
