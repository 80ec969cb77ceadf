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


def test_ragged_three_kv_heads(hip_backend):
    # A kv head count that is not a power of two: the kernel splits the
    # work-group index by a division instead of a shift.
    case = wl.c5_inputs(lens=[1, 33, 500, 4097, 64], heads=6, kv_heads=3, dim=128)
    _check(_run(hip_backend, case), case)


def _host_plan_tables(lens, target):
    import ctypes

    from breezetoken_amd import _lib

    lib = _lib.lib()
    b = len(lens)
    cap = sum(max(1, -(-n // 32)) for n in lens)
    L = (ctypes.c_int32 * b)(*lens)
    work = (ctypes.c_int32 * (4 * cap))()
    base = (ctypes.c_int32 * b)()
    cnt = (ctypes.c_int32 * b)()
    tot = ctypes.c_int32()
    n = lib.bt_ragged_plan(ctypes.addressof(L), b, target, ctypes.addressof(work), cap,
                           ctypes.addressof(base), ctypes.addressof(cnt), ctypes.addressof(tot))
    assert n >= 0
    return list(work)[: 4 * n], list(base), list(cnt), tot.value


PLAN_CASES = {
    "c5": (wl.ragged_lengths(), 128),
    "c5_target_256": (wl.ragged_lengths(), 256),
    "c5_more_seqs_than_groups": (wl.ragged_lengths(), 8),
    "one_long_sequence": ([32768, 300, 17], 256),
    "edge_lengths": ([0, 1, 31, 32, 33, 500, 4097, 1234, 64], 64),
    "single": ([70000], 256),
    "many": ([(i * 7919) % 20000 for i in range(1500)], 256),
}


@pytest.mark.parametrize("name", list(PLAN_CASES))
def test_device_plan_equals_host_plan(hip_backend, name):
    """bt_ragged_plan_device builds the host planner's tables bit for bit, then pads."""
    lens, target = PLAN_CASES[name]
    print(f"[plan] {name}: batch {len(lens)}, target {target}", flush=True)
    work_h, base_h, cnt_h, tot_h = _host_plan_tables(lens, target)
    seq_len = torch.tensor(lens, dtype=torch.int32, device="cuda")
    work, cap, base, cnt, _ = hip_backend.ragged_plan_device(seq_len, target)
    total = hip_backend._dev_plans[(len(lens), target)][3]
    torch.cuda.synchronize()
    assert int(total.item()) == tot_h
    assert base.cpu().tolist() == base_h and cnt.cpu().tolist() == cnt_h
    w = work.cpu().reshape(-1).tolist()
    assert w[: 4 * tot_h] == work_h
    assert all(w[4 * i] == -1 for i in range(tot_h, cap))


def test_ragged_decode_device_plan_matches_host_plan(hip_backend):
    case = wl.c5_inputs()
    dev = "cuda"
    seq_off = torch.tensor(case.offsets, dtype=torch.int64, device=dev)
    seq_len = torch.tensor(case.lens, dtype=torch.int32, device=dev)
    args = (case.q.float().to(dev), case.k.to(dev), case.v.to(dev), seq_off, seq_len)
    host = hip_backend.attention_ragged(*args, case.lens, case.scale)
    device = hip_backend.attention_ragged(*args, None, case.scale)
    assert torch.equal(host, device)
    _check(device, case)


def test_ragged_decode_graph_with_growing_lengths(hip_backend):
    """A multi-sequence decode step with the device plan, captured once: every
    replay re-plans from the device lengths, which grow by one per step."""
    dev = "cuda"
    lens0 = [300, 4000, 17, 1025, 9000, 64, 2048, 33]
    final = [n + 5 for n in lens0]
    case = wl.c5_inputs(lens=final)
    seq_off = torch.tensor(case.offsets, dtype=torch.int64, device=dev)
    seq_len = torch.tensor(lens0, dtype=torch.int32, device=dev)
    q, k, v = case.q.float().to(dev), case.k.to(dev), case.v.to(dev)
    out = hip_backend.attention_ragged(q, k, v, seq_off, seq_len, None, case.scale)  # allocates
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = hip_backend.attention_ragged(q, k, v, seq_off, seq_len, None, case.scale)
    for step in range(5):
        g.replay()
        torch.cuda.synchronize()
        lens = [n + step for n in lens0]
        eager = hip_backend.attention_ragged(q, k, v, seq_off, seq_len, lens, case.scale)
        assert torch.equal(out, eager), step
        got = out.cpu()
        for b, (n, o) in enumerate(zip(lens, case.offsets)):
            ref = orc.torch_attention(case.q[b].float(), case.k[o : o + n].float(), case.v[o : o + n].float(),
                                      case.scale)
            err, cos = orc.compare(got[b].numpy(), ref.numpy())
            assert err <= 2e-3 and cos >= 0.99999, (step, b, err, cos)
        seq_len.add_(1)
