"""GPU parity of ragged multi-sequence decode (config 5) against the CPU oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from breezetoken_amd import workloads as wl
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _run(backend, case, target=None):
    dev = "cuda"
    seq_off = torch.tensor(case.offsets, dtype=torch.int64, device=dev)
    seq_len = torch.tensor(case.lens, dtype=torch.int32, device=dev)
    return backend.attention_ragged(case.q.float().to(dev), case.k.to(dev), case.v.to(dev), seq_off,
                                    seq_len, case.lens, case.scale, target_groups=target)


def _check(out, case):
    out = out.cpu()
    for b, (n, o) in enumerate(zip(case.lens, case.offsets)):
        ref = orc.torch_attention(case.q[b].float(), case.k[o : o + n].float(), case.v[o : o + n].float(),
                                  case.scale)
        err, cos = orc.compare(out[b].numpy(), ref.numpy())
        assert err <= 2e-3 and cos >= 0.99999, (b, n, err, cos)


def test_c5_ragged_decode(hip_backend):
    case = wl.c5_inputs()
    print(f"[c5] batch={len(case.lens)} tokens={sum(case.lens)}", flush=True)
    _check(_run(hip_backend, case), case)


@pytest.mark.parametrize("target", [1, 7, 64, 512])
def test_ragged_any_split_plan(hip_backend, target):
    case = wl.c5_inputs(lens=[1, 31, 32, 33, 500, 4097, 1234, 64])
    _check(_run(hip_backend, case, target), case)
