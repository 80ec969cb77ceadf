#!/usr/bin/env python3
"""Benchmark of the MI355X GQA attention path (one GPU).

Headline (decode µs per call and HBM GB/s, config 2): split-KV GQA flash-decode,
Qwen3.5-0.8B-like H=8 / Hkv=2 / D=256, bf16 fixed-capacity cache of 65,536
slots, valid length 32,768 given by a device position tensor, q/K/V ~ N(0, 1)
bf16 (seed 1).  One step = one decode call (split + LSE combine).  The calls
are captured in a hipGraph (``torch.cuda.graph``) the way the model's decode
step holds them: one graph per decode step with one call per attention layer
(the 0.8B model has 6), each on its own layer cache, so a replay streams 6
distinct 64 MiB prefixes (384 MiB, more than the 256 MB Infinity Cache) from
HBM.  ``ms_per_step`` = replay time / 6; ``value`` = algorithmic bytes of a
call / ``ms_per_step``, in GB/s.  A graph holding a single call replayed
``--steps`` times is reported as ``extra.single_call_graph``.

Also reported (``extra``): 1k/4k/32k decode, config 3, config 5 (ragged), all
timed the same way (one call per distinct layer cache inside one graph), a
MALL-hot variant of config 2 (one cache, 6 calls per graph) for contrast, and
causal prefill TFLOP/s (config 4) when the prefill kernel is served.

``roofline`` times the split kernel alone (the dominant kernel) with HIP events
on the stream it is launched on; ``cpu_baseline`` times the CPU torch f32
reference attention (the restated ``_torch_attention``) on this host.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
METRIC = "decode-attn µs/call + achieved HBM GB/s (% peak) at 4k/32k ctx; prefill TFLOP/s"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_graph(torch, fn, steps: int, warmup: int, calls_per_graph: int = 1) -> float:
    """Capture ``fn`` (calls_per_graph calls) in one graph; return ms per call over
    ``steps`` calls timed with HIP events on the current stream."""
    stream = torch.cuda.current_stream()
    fn()  # eager preflight: allocates workspaces outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls_per_graph):
            fn()
    replays = max(1, steps // calls_per_graph)
    for _ in range(max(1, warmup // calls_per_graph)):
        graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * calls_per_graph)


def pmc_mode(torch, backend, dev) -> int:
    """Launches for counter collection: a plain copy of known size (to scale
    FETCH_SIZE / WRITE_SIZE) and the config-2 split kernel on 6 layer caches."""
    import ctypes

    from breezetoken_amd import _lib
    from breezetoken_amd import workloads as wl
    from breezetoken_amd.kvcache import KVCache

    H, HKV, D, CAP, L = 8, 2, 256, 65536, 32768
    src = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device=dev).normal_()
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.mul(src, 2.0, out=dst)  # MulFunctor kernel: 256 MiB read + 256 MiB written
    case = wl.c2_inputs(L, cap=CAP)
    ns = backend.pick_splits(HKV, CAP)
    lse = torch.empty((H, ns), dtype=torch.float32, device=dev)
    part = torch.empty((H, ns, D), dtype=torch.float32, device=dev)
    q = case.q.float().to(dev)
    pos = torch.tensor([case.pos], dtype=torch.int32, device=dev)
    caches = []
    for _ in range(6):
        c = KVCache(CAP, HKV, D, dev)
        c.k.copy_(case.k.reshape(CAP, -1))
        c.v.copy_(case.v.reshape(CAP, -1))
        caches.append(c.views() + (c,))
    lib = _lib.lib()
    for _ in range(5):
        for kv, vv, _c in caches:
            rc = lib.bt_gqa_decode_split(
                q.data_ptr(), _lib.BT_DTYPE_F32, H * D, kv.data_ptr(), vv.data_ptr(), kv.stride(0),
                kv.stride(1), None, pos.data_ptr(), None, CAP, 1, H, HKV, D, ns, case.scale,
                lse.data_ptr(), part.data_ptr(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            _lib.check("bt_gqa_decode_split", rc)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "pmc", "copy_kernel": "MulFunctor", "copy_bytes_each_way": src.numel() * 2,
                      "split_algorithmic_bytes": 2 * L * HKV * D * 2 + H * D * 4}), flush=True)
    return 0


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's description."""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.lower().startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def time_cpu(fn, seconds: float, min_calls: int = 20, max_calls: int = 2000) -> tuple[float, int]:
    """Median seconds per call of ``fn`` after 3 warm-up calls: at least
    ``min_calls`` calls, more while ``seconds`` last."""
    for _ in range(3):
        fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_calls or (time.perf_counter() < t_end and len(times) < max_calls):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baselines(torch, head_case, L: int, nbytes: int, seconds: float, headline_only: bool):
    """The reference's torch f32 CPU attention (restated in oracle/, as the
    reference computes it: backends.py:196-215 for decode, prefill.py:56-68 for
    prefill) on the host cores: the config-2 headline row, then one row per
    further config (C3 at 32k, C4 causal prefill, C5 looping over its 32
    sequences).  Returns (headline dict, rows)."""
    from breezetoken_amd import workloads as wl
    from oracle.attention import torch_attention, torch_prefill_attention

    threads = torch.get_num_threads()
    host = f"cpu={os.cpu_count()} logical ({cpu_model()}), torch threads={threads}"
    qc, kc, vc = head_case.q.float(), head_case.k[:L].float(), head_case.v[:L].float()
    med, n = time_cpu(lambda: torch_attention(qc, kc, vc, head_case.scale), seconds)
    head = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "us_per_call": round(med * 1e6, 1), "cpu_model": cpu_model(),
            "sample": f"{n} calls of config-2 decode (valid 32768, H=8, Hkv=2, D=256) in torch f32 SDPA "
                      f"on the host CPU, median after 3 warm-ups; {host}"}
    log(f"cpu baseline: {med * 1e6:.0f} us/call on {threads} threads ({cpu_model()})")
    rows = []
    if headline_only:
        return head, rows
    c3 = wl.c3_inputs(32768)
    q3, k3, v3 = c3.q.float(), c3.k.float(), c3.v.float()
    med, n = time_cpu(lambda: torch_attention(q3, k3, v3, c3.scale), seconds / 3)
    b3 = wl.decode_bytes(32768, 16, 2, 256)
    rows.append({"config": "C3 decode, H=16 Hkv=2 D=256, valid 32768", "us_per_call": round(med * 1e6, 1),
                 "GBps": round(b3 / med / 1e9, 3), "calls": n})
    for steps, min_calls in ((512, 20), (2048, 20), (8192, 3)):
        q4, k4, v4, sc4 = wl.c4_inputs(steps)
        q4, k4, v4 = q4.float(), k4.float(), v4.float()
        med, n = time_cpu(lambda: torch_prefill_attention(q4, k4, v4, sc4), seconds / 3, min_calls=min_calls)
        fl = wl.prefill_flops(steps, 8, 256)
        rows.append({"config": f"C4 causal prefill, H=8 Hkv=2 D=256, S={steps}", "us_per_call": round(med * 1e6, 1),
                     "TFLOPs": round(fl / med / 1e12, 4), "calls": n})
    c5 = wl.c5_inputs()
    seqs = [(c5.q[b].float(), c5.k[o:o + n_].float(), c5.v[o:o + n_].float())
            for b, (o, n_) in enumerate(zip(c5.offsets, c5.lens))]

    def c5_loop():
        for qq, kk, vv in seqs:
            torch_attention(qq, kk, vv, c5.scale)

    med, n = time_cpu(c5_loop, seconds / 3)
    b5 = 2 * sum(c5.lens) * 2 * 256 * 2 + len(c5.lens) * 8 * 256 * 4 * 2
    rows.append({"config": "C5 ragged decode, 32 sequences looped, H=8 Hkv=2 D=256", "us_per_call": round(med * 1e6, 1),
                 "GBps": round(b5 / med / 1e9, 3), "calls": n})
    for r in rows:
        r["host"] = host
    log("cpu rows: " + json.dumps(rows))
    return head, rows


def prefill_mode(torch, backend, dev, calls: int, q_f32: bool = False, warmup: int = 2) -> int:
    """Config-4 prefill at S=8192 only (for rocprofv3 kernel traces): ``calls``
    calls after ``warmup`` warm-up calls, timed with HIP events on the current
    stream.  q is bf16 as config 4 draws it, or its f32 draws (``q_f32``).
    MFMA-heavy work runs ~10% slower for its first ~10 ms in a process (clock
    ramp), so a trace meant to match the warmed bench number wants ~50
    warm-up calls."""
    from breezetoken_amd import workloads as wl

    q, k, v, scale = wl.c4_inputs(8192, q_f32=q_f32)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    for _ in range(max(0, warmup)):
        backend.attention_prefill(q, k, v, scale, torch.bfloat16)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(torch.cuda.current_stream())
    for _ in range(calls):
        backend.attention_prefill(q, k, v, scale, torch.bfloat16)
    end.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / calls
    fl = wl.prefill_flops(8192, 8, 256)
    print(json.dumps({"mode": "prefill", "steps": 8192, "q_dtype": "f32" if q_f32 else "bf16", "calls": calls,
                      "us_per_call": round(us, 2),
                      "TFLOPs": round(fl / us / 1e6, 1)}), flush=True)
    return 0


def floor_mode(torch, backend, dev, steps: int, warmup: int) -> int:
    """Machine floors beside the config-2 decode kernels, in one process (the
    probes are libbt_floor.so, built from breezetoken_amd/probes/floor.hip):

    * an empty kernel as a graph node, alone in its graph and 24 in a chain;
    * a plain streaming read of 64 MiB (config 2's K and V at 32k): 16-byte
      non-temporal buffer loads, LPT loads per thread issued before any is
      used, rotating over six 64 MiB buffers per graph (384 MiB, past the
      256 MB MALL) as the decode rows rotate six layer caches, and MALL-hot
      (one buffer six times);
    * that read followed by a one-wave dependent kernel (the two-node shape of
      a split + combine call);
    * the config-2 split kernel alone and the whole call at 32k, six layer
      caches per graph, as the headline measures them.
    """
    import ctypes

    from breezetoken_amd import _lib
    from breezetoken_amd import workloads as wl
    from breezetoken_amd.kvcache import KVCache

    fl = ctypes.CDLL(str(ROOT / "breezetoken_amd" / "libbt_floor.so"))
    vp = ctypes.c_void_p
    fl.bt_floor_empty.argtypes = [vp]
    fl.bt_floor_read.argtypes = [vp, ctypes.c_int64, ctypes.c_int32, vp, vp]
    fl.bt_floor_tiny.argtypes = [vp, vp, vp]
    fl.bt_floor_read_lds.argtypes = [vp, ctypes.c_int64, vp, vp]
    fl.bt_floor_read_rows.argtypes = [vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, vp, vp]
    for f in (fl.bt_floor_empty, fl.bt_floor_read, fl.bt_floor_tiny, fl.bt_floor_read_lds, fl.bt_floor_read_rows):
        f.restype = ctypes.c_int

    def st():
        return vp(torch.cuda.current_stream().cuda_stream)

    def ok(rc):
        if rc != 0:
            raise RuntimeError(f"floor probe launch failed: {rc}")

    nbytes = 64 << 20
    res: dict = {"mode": "floor", "read_bytes": nbytes, "layers_per_graph": 6}
    res["empty_node_us_alone"] = round(1e3 * time_graph(torch, lambda: ok(fl.bt_floor_empty(st())), steps, warmup), 3)
    res["empty_node_us_chain24"] = round(1e3 * time_graph(
        torch, lambda: [ok(fl.bt_floor_empty(st())) for _ in range(24)], steps, warmup) / 24, 3)
    g = torch.Generator(device=dev).manual_seed(5)
    bufs = [torch.randint(0, 1 << 30, (nbytes // 4,), dtype=torch.int32, device=dev, generator=g) for _ in range(6)]
    out = torch.empty(nbytes // 4096, dtype=torch.int32, device=dev)
    out2 = torch.empty(1, dtype=torch.int32, device=dev)
    reads = {}
    for lpt in (8, 16, 32):
        cold = time_graph(torch, lambda: [ok(fl.bt_floor_read(b.data_ptr(), nbytes, lpt, out.data_ptr(), st()))
                                          for b in bufs], steps, warmup) / 6
        hot = time_graph(torch, lambda: [ok(fl.bt_floor_read(bufs[0].data_ptr(), nbytes, lpt, out.data_ptr(), st()))
                                         for _ in bufs], steps, warmup) / 6
        reads[lpt] = {"work_groups": nbytes // (4096 * lpt), "cold_us": round(cold * 1e3, 3),
                      "cold_GBps": round(nbytes / (cold * 1e-3) / 1e9, 1), "mall_hot_us": round(hot * 1e3, 3)}
    res["read_64MiB"] = reads
    # through LDS (HBM -> LDS copies), and along token rows the way the decode
    # kernel reads one kv head of K (two 32 MiB halves of each 64 MiB buffer:
    # 512 of every 1,024 bytes), both cold
    lds_us = time_graph(torch, lambda: [ok(fl.bt_floor_read_lds(b.data_ptr(), nbytes, out.data_ptr(), st()))
                                        for b in bufs], steps, warmup) / 6
    res["read_64MiB_via_lds"] = {"cold_us": round(lds_us * 1e3, 3),
                                 "cold_GBps": round(nbytes / (lds_us * 1e-3) / 1e9, 1)}
    rows = nbytes // 1024
    for mode, key, nb_ in ((0, "read_half_rows_32MiB", nbytes // 2), (1, "read_rows_halves_adjacent_groups", nbytes),
                           (2, "read_rows_halves_one_group", nbytes),
                           (3, "read_rows_halves_adjacent_groups_row_loads", nbytes),
                           (4, "read_rows_halves_adjacent_groups_quarter_row_loads", nbytes),
                           (5, "read_rows_halves_adjacent_groups_quarter_row_loads_row_minor_lanes", nbytes)):
        us = time_graph(torch, lambda: [ok(fl.bt_floor_read_rows(b.data_ptr(), rows, 1024, mode, out.data_ptr(), st()))
                                        for b in bufs], steps, warmup) / 6
        res[key] = {"cold_us": round(us * 1e3, 3), "cold_GBps": round(nb_ / (us * 1e-3) / 1e9, 1)}
    best = min(reads, key=lambda k: reads[k]["cold_us"])
    res["read_plus_dependent_node_us"] = round(1e3 * time_graph(
        torch, lambda: [(ok(fl.bt_floor_read(b.data_ptr(), nbytes, best, out.data_ptr(), st())),
                         ok(fl.bt_floor_tiny(out.data_ptr(), out2.data_ptr(), st()))) for b in bufs],
        steps, warmup) / 6, 3)
    res["read_plus_dependent_node_lpt"] = best
    del bufs
    torch.cuda.empty_cache()
    # the decode kernels, as the headline times them
    H, HKV, D, CAP, L = 8, 2, 256, 65536, 32768
    case = wl.c2_inputs(L, cap=CAP)
    layers = []
    for _ in range(6):
        cache = KVCache(CAP, HKV, D, dev)
        cache.k.copy_(case.k.reshape(CAP, -1))
        cache.v.copy_(case.v.reshape(CAP, -1))
        kv, vv = cache.views()
        layers.append((cache, case.q.float().to(dev), kv, vv,
                       torch.tensor([case.pos], dtype=torch.int32, device=dev)))
    lib = _lib.lib()
    ns = backend.pick_splits(HKV, CAP)
    lse = torch.empty((H, ns), dtype=torch.float32, device=dev)
    part = torch.empty((H, ns, D), dtype=torch.float32, device=dev)

    def split_only():
        for _, lq, lk, lv, lp in layers:
            _lib.check("bt_gqa_decode_split", lib.bt_gqa_decode_split(
                lq.data_ptr(), _lib.BT_DTYPE_F32, H * D, lk.data_ptr(), lv.data_ptr(), lk.stride(0), lk.stride(1),
                None, lp.data_ptr(), None, CAP, 1, H, HKV, D, ns, case.scale, lse.data_ptr(), part.data_ptr(), st()))

    res["c2_32k_split_us"] = round(1e3 * time_graph(torch, split_only, steps, warmup) / 6, 3)
    res["c2_32k_call_us"] = round(1e3 * time_graph(
        torch, lambda: [backend.attention_fixed(lq, lk, lv, lp, case.scale) for _, lq, lk, lv, lp in layers],
        steps, warmup) / 6, 3)
    res["c2_32k_algorithmic_bytes"] = wl.decode_bytes(L, H, HKV, D)
    print(json.dumps(res), flush=True)
    return 0


CHUNKED_CASES = ((16, 128, 8192), (16, 512, 16384), (8, 256, 4096), (8, 512, 0), (8, 2048, 0))


def chunked_inputs(torch, dev, heads: int, steps: int, pos0: int):
    """Seeded q (S, H, 256) and k/v (pos0 + S, 2, 256) bf16 on ``dev``."""
    g = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(steps, heads, 256, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(pos0 + steps, 2, 256, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(pos0 + steps, 2, 256, generator=g, device=dev).to(torch.bfloat16)
    return q, k, v


def chunked_mode(torch, backend, dev, calls: int) -> int:
    """Split-key prefill only (for rocprofv3 kernel traces): ``calls`` eager
    calls of each CHUNKED_CASES shape after two warm-up calls, in that order."""
    for heads, steps, pos0 in CHUNKED_CASES:
        q, k, v = chunked_inputs(torch, dev, heads, steps, pos0)
        for _ in range(2):
            backend.attention_prefill(q, k, v, 256**-0.5, torch.bfloat16, q_offset=pos0)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(torch.cuda.current_stream())
        for _ in range(calls):
            backend.attention_prefill(q, k, v, 256**-0.5, torch.bfloat16, q_offset=pos0)
        end.record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        print(json.dumps({"mode": "chunked", "heads": heads, "steps": steps, "q_offset": pos0, "calls": calls,
                          "us_per_call_eager": round(start.elapsed_time(end) * 1e3 / calls, 2)}), flush=True)
    return 0


def decode_mode(torch, backend, dev, calls: int, valid: int, graph: bool = False) -> int:
    """Config-2 fixed-capacity decode at one valid length only (for rocprofv3
    kernel traces of split vs combine): ``calls`` calls rotating over six layer
    caches (384 MiB, past the MALL) after two warm-up rounds, timed with HIP
    events on the current stream.  Eager launches by default (the host's launch
    gaps leave the GPU idle between calls); ``graph``: the six calls captured in
    one hipGraph and replayed, as the headline times them."""
    from breezetoken_amd import workloads as wl
    from breezetoken_amd.kvcache import KVCache

    cap = 65536
    case = wl.c2_inputs(valid, cap=cap)
    layers = []
    for _ in range(6):
        cache = KVCache(cap, case.k.shape[1], case.k.shape[2], dev)
        cache.k.copy_(case.k.reshape(cap, -1))
        cache.v.copy_(case.v.reshape(cap, -1))
        layers.append((cache,) + cache.views())
    q = case.q.float().to(dev)
    pos = torch.tensor([case.pos], dtype=torch.int32, device=dev)
    for i in range(12):
        _, k, v = layers[i % 6]
        backend.attention_fixed(q, k, v, pos, case.scale)
    torch.cuda.synchronize()
    if graph:
        six = lambda: [backend.attention_fixed(q, k, v, pos, case.scale) for _, k, v in layers]  # noqa: E731
        us = time_graph(torch, six, max(1, calls // 6), 2) * 1e3 / 6  # one replay = six calls
        print(json.dumps({"mode": "decode", "valid": valid, "calls": 6 * max(1, calls // 6), "us_per_call_graph": round(us, 2),
                          "num_split": backend.pick_splits(case.k.shape[1], cap)}), flush=True)
        return 0
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(torch.cuda.current_stream())
    for i in range(calls):
        _, k, v = layers[i % 6]
        backend.attention_fixed(q, k, v, pos, case.scale)
    end.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / calls
    print(json.dumps({"mode": "decode", "valid": valid, "calls": calls, "us_per_call_eager": round(us, 2),
                      "num_split": backend.pick_splits(case.k.shape[1], cap)}), flush=True)
    return 0


def ragged_mode(torch, backend, dev, calls: int) -> int:
    """Config-5 ragged decode only (for rocprofv3 kernel traces): ``calls`` calls
    over three copies of the cache after two warm-up calls, timed with HIP events
    on the current stream."""
    from breezetoken_amd import workloads as wl

    rc5 = wl.c5_inputs()
    rq = rc5.q.float().to(dev)
    rkv = [(rc5.k.to(dev), rc5.v.to(dev)) for _ in range(3)]  # ~1 GB: the calls do not hit the MALL
    roff = torch.tensor(rc5.offsets, dtype=torch.int64, device=dev)
    rlen = torch.tensor(rc5.lens, dtype=torch.int32, device=dev)

    def call(i):
        rk, rv = rkv[i % len(rkv)]
        backend.attention_ragged(rq, rk, rv, roff, rlen, rc5.lens, rc5.scale)

    for i in range(2):
        call(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(torch.cuda.current_stream())
    for i in range(calls):
        call(i)
    end.record(torch.cuda.current_stream())
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / calls
    nbytes = 2 * sum(rc5.lens) * rc5.k.shape[1] * rc5.k.shape[2] * 2 + len(rc5.lens) * rq.shape[1] * rq.shape[2] * 4 * 2
    print(json.dumps({"mode": "ragged", "sequences": len(rc5.lens), "tokens": sum(rc5.lens), "calls": calls,
                      "us_per_call": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--q-f32", action="store_true", help="prefill mode: f32 q (the reference's prefill arithmetic)")
    ap.add_argument("--valid", type=int, default=32768, help="decode mode: valid length (config 2)")
    ap.add_argument("--graph", action="store_true", help="decode mode: replay the calls in a hipGraph")
    ap.add_argument("--mode", choices=["bench", "pmc", "prefill", "decode", "ragged", "chunked", "floor"],
                    default="bench",
                    help="pmc: only a 256 MiB device copy and the config-2 split kernel, "
                         "5 launches each, for rocprofv3 --pmc runs; prefill: only config-4 "
                         "prefill at S=8192 (--steps calls), for kernel traces; decode: only "
                         "config-2 decode at --valid (--steps calls), for kernel traces; ragged: only "
                         "config-5 ragged decode (--steps calls), for kernel traces; chunked: "
                         "only the split-key prefill shapes (--steps calls each), for kernel traces; "
                         "floor: the machine-floor probes (empty node, plain 64 MiB read, read + dependent "
                         "node) beside the config-2 split kernel and call")
    args = ap.parse_args()
    if args.gpus != 1:
        print("this build measures one GPU only: the decode/prefill kernels run on a single "
              "MI355X and no multi-GPU path is built (the kernels shard by kv head or by "
              "context, with an all-gather of split partials before the same combine); "
              "run with --gpus 1",
              file=sys.stderr)
        return 2

    import ctypes

    import torch

    from breezetoken_amd import _lib
    from breezetoken_amd import workloads as wl
    from breezetoken_amd.backend import HipBackend
    from breezetoken_amd.kvcache import KVCache

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    backend = HipBackend(dev)
    log(f"{backend!r}")
    H, HKV, D, CAP = 8, 2, 256, 65536
    if args.mode == "pmc":
        return pmc_mode(torch, backend, dev)
    if args.mode == "prefill":
        return prefill_mode(torch, backend, dev, max(1, min(args.steps, 200)), args.q_f32, min(args.warmup, 200))
    if args.mode == "decode":
        return decode_mode(torch, backend, dev, max(1, min(args.steps, 2000)), args.valid, args.graph)
    if args.mode == "ragged":
        return ragged_mode(torch, backend, dev, max(1, min(args.steps, 500)))
    if args.mode == "chunked":
        return chunked_mode(torch, backend, dev, max(1, min(args.steps, 200)))
    if args.mode == "floor":
        return floor_mode(torch, backend, dev, max(10, min(args.steps, 2000)), max(1, min(args.warmup, 200)))

    def fixed_case(case, cap):
        cache = KVCache(cap, case.k.shape[1], case.k.shape[2], dev)
        cache.k.copy_(case.k.reshape(cap, -1))
        cache.v.copy_(case.v.reshape(cap, -1))
        kv, vv = cache.views()
        q = case.q.float().to(dev)
        pos = torch.tensor([case.pos], dtype=torch.int32, device=dev)
        return cache, q, kv, vv, pos

    def decode_point(case, cap, steps, warmup, n_layers=6):
        """µs per call with one graph holding one call per distinct layer cache."""
        lay = [fixed_case(case, cap) for _ in range(n_layers)]
        heads = case.q.shape[0]

        def run():
            for _, lq, lk, lv, lp in lay:
                backend.attention_fixed(lq, lk, lv, lp, case.scale)

        ms = time_graph(torch, run, steps, warmup) / n_layers
        nbytes = wl.decode_bytes(case.valid, heads, case.k.shape[1], case.k.shape[2])
        res = {"valid": case.valid, "us_per_call": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9,
               "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes": nbytes,
               "layer_caches": n_layers}
        del lay
        torch.cuda.empty_cache()
        return res

    # ---------------------------------------------------------------- headline
    L = 32768
    LAYERS = 6  # attention layers of the 0.8B decoder: (i + 1) % 4 == 0 of 24 (config.py:37-39)
    log(f"config 2 headline: H={H} Hkv={HKV} D={D} cap={CAP} valid={L}, {LAYERS} layer caches")
    head_case = wl.c2_inputs(L, cap=CAP)
    layers = [fixed_case(head_case, CAP) for _ in range(LAYERS)]
    q, kv, vv, pos = layers[0][1], layers[0][2], layers[0][3], layers[0][4]

    def decode_step():
        for _, lq, lk, lv, lp in layers:
            backend.attention_fixed(lq, lk, lv, lp, head_case.scale)

    ms_per_step = time_graph(torch, decode_step, args.steps, args.warmup, calls_per_graph=1) / LAYERS
    nbytes = wl.decode_bytes(L, H, HKV, D)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    log(f"headline: {ms_per_step * 1e3:.2f} us/call, {value:.0f} GB/s")
    single_ms = time_graph(torch, lambda: backend.attention_fixed(q, kv, vv, pos, head_case.scale),
                           args.steps, args.warmup)

    # ---- roofline: the split kernel alone, HIP events on its stream ----------
    lib = _lib.lib()
    ns = backend.pick_splits(HKV, CAP)
    lse = torch.empty((H, ns), dtype=torch.float32, device=dev)
    part = torch.empty((H, ns, D), dtype=torch.float32, device=dev)

    def split_only():
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for _, lq, lk, lv, lp in layers:
            rc = lib.bt_gqa_decode_split(
                lq.data_ptr(), _lib.BT_DTYPE_F32, H * D, lk.data_ptr(), lv.data_ptr(), lk.stride(0),
                lk.stride(1), None, lp.data_ptr(), None, CAP, 1, H, HKV, D, ns, head_case.scale,
                lse.data_ptr(), part.data_ptr(), stream,
            )
            _lib.check("bt_gqa_decode_split", rc)

    split_ms = time_graph(torch, split_only, args.steps, args.warmup, calls_per_graph=1) / LAYERS
    split_bytes = 2 * L * HKV * D * 2 + H * D * 4  # K + V of the valid prefix, q once
    achieved = split_bytes / (split_ms * 1e-3) / 1e9
    log(f"split kernel: {split_ms * 1e3:.2f} us, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%})")
    traffic = None
    tfile = ROOT / "profiles" / "decode_split_c2_32k_traffic.json"
    if tfile.is_file():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": "gqa_decode_split_kernel<4,256>", "kernel_us": round(split_ms * 1e3, 3),
                "algorithmic_bytes": split_bytes, "num_split": ns}

    extra: dict = {"headline_us_per_call": round(ms_per_step * 1e3, 3), "num_split": ns,
                   "single_call_graph": {"us_per_call": round(single_ms * 1e3, 3),
                                         "GBps": round(nbytes / (single_ms * 1e-3) / 1e9, 1)},
                   "num_cus": backend.num_cus, "arch": backend.arch}
    # --------------------------------------------------------------- extras
    if not args.no_extra:
        esteps, ewarm = max(100, args.steps // 2), max(10, args.warmup // 2)
        extra["c2"] = [decode_point(wl.c2_inputs(v, cap=CAP), CAP, esteps, ewarm)
                       for v in (1024, 4096, 32768)]
        log("c2 sweep: " + ", ".join(f"{r['valid']}: {r['us_per_call']:.2f}us {r['GBps']:.0f}GB/s"
                                     for r in extra["c2"]))
        # hot: the same cache 6 times per graph, so the 64 MiB prefix stays in the Infinity Cache
        hot_ms = time_graph(torch, lambda: [backend.attention_fixed(q, kv, vv, pos, head_case.scale)
                                            for _ in range(LAYERS)], esteps, ewarm) / LAYERS
        extra["c2_mall_hot_32k"] = {"us_per_call": hot_ms * 1e3, "GBps": nbytes / (hot_ms * 1e-3) / 1e9}
        log(f"c2 MALL-hot 32k: {hot_ms * 1e3:.2f} us/call")
        del layers
        torch.cuda.empty_cache()
        c3 = []
        for v in (8192, 32768, 131072):
            c3.append(decode_point(wl.c3_inputs(v, cap=131072), 131072, esteps, ewarm))
        extra["c3"] = c3
        log("c3: " + ", ".join(f"{r['valid']}: {r['us_per_call']:.2f}us {r['GBps']:.0f}GB/s" for r in c3))
        # ragged (config 5)
        rc5 = wl.c5_inputs()
        rq = rc5.q.float().to(dev)
        rkv = [(rc5.k.to(dev), rc5.v.to(dev)) for _ in range(3)]  # 3 layer caches, ~1 GB
        roff = torch.tensor(rc5.offsets, dtype=torch.int64, device=dev)
        rlen = torch.tensor(rc5.lens, dtype=torch.int32, device=dev)
        rms = time_graph(torch, lambda: [backend.attention_ragged(rq, rk, rv, roff, rlen, rc5.lens, rc5.scale)
                                         for rk, rv in rkv], esteps, ewarm) / len(rkv)
        rbytes = 2 * sum(rc5.lens) * HKV * D * 2 + len(rc5.lens) * H * D * 4 * 2
        extra["c5_ragged"] = {"us_per_call": rms * 1e3, "GBps": rbytes / (rms * 1e-3) / 1e9,
                              "frac_hbm_peak": rbytes / (rms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                              "tokens": sum(rc5.lens), "bytes": rbytes}
        log(f"c5 ragged: {rms * 1e3:.2f} us/call")
        del rkv
        torch.cuda.empty_cache()
        # prefill (config 4: bf16 q/k/v, bf16 output), and at S = 8192 also with the
        # same q draws in f32, as the reference's prefill computes it (prefill.py:49-68).
        # Like the decode rows, one graph holds LAYERS calls on LAYERS separate copies of
        # the inputs (a model's layers), so a short prompt's figure is not the host's
        # graph-launch rate.
        pre = []
        for s, qf32 in ((128, False), (512, False), (2048, False), (8192, False), (8192, True)):
            base = [t.to(dev) if hasattr(t, "to") else t for t in wl.c4_inputs(s, q_f32=qf32)]
            sets = [(base[0].clone(), base[1].clone(), base[2].clone(), base[3]) for _ in range(LAYERS)]
            del base
            try:
                # MFMA-heavy work runs ~10% slower for its first ~10 ms in a process (clock
                # ramp; measured 334 -> 287 us at S = 8192), so the long rows warm up ~30 ms
                pms = time_graph(torch, lambda: [backend.attention_prefill(qp, kp, vp, sc, torch.bfloat16)
                                                 for qp, kp, vp, sc in sets],
                                 max(20, esteps // 10), 20 if s >= 8192 else 5) / LAYERS
            except RuntimeError as exc:
                pre.append({"steps": s, "error": str(exc)[:120]})
                break
            fl = wl.prefill_flops(s, 8, 256)
            pre.append({"steps": s, "q_dtype": "f32" if qf32 else "bf16", "us_per_call": pms * 1e3,
                        "TFLOPs": fl / (pms * 1e-3) / 1e12,
                        "frac_bf16_peak": fl / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS})
        extra["c4_prefill"] = pre
        big = next((r for r in pre if r.get("steps") == 8192 and r.get("q_dtype") == "bf16" and "TFLOPs" in r), None)
        if big:
            # the call = K/V^T image pre-pass + MFMA kernel; both inside the timed region
            extra["c4_prefill_roofline"] = {
                "bound": "mfma", "achieved": round(big["TFLOPs"], 1), "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(big["frac_bf16_peak"], 4), "steps": big["steps"],
                "kernels": "prefill_vts_kernel<256,0> + gqa_prefill_pair_kernel<256>",
                "algorithmic_flops": wl.prefill_flops(big["steps"], 8, 256)}
        log("c4: " + json.dumps(pre))
        # chunked prefill at a cached prefix (qwen36_moe.py:394-428) and a short prompt:
        # the split-key schedule against one work-group per query block, same process
        chunked = []
        for heads, steps, pos0 in CHUNKED_CASES:
            base = chunked_inputs(torch, dev, heads, steps, pos0)
            sets = [tuple(t.clone() for t in base) for _ in range(LAYERS)]  # LAYERS calls per graph
            del base
            row = {"heads": heads, "kv_heads": 2, "steps": steps, "q_offset": pos0}
            for key, split in (("us_split", True), ("us_unsplit", False)):
                row[key] = 1e3 * time_graph(
                    torch, lambda: [backend.attention_prefill(qc, kc, vc, 256**-0.5, torch.bfloat16,
                                                              q_offset=pos0, split_keys=split)
                                    for qc, kc, vc in sets],
                    max(20, esteps // 10), 5) / LAYERS
            if pos0 > 0:
                # steady state of a chunk loop with the images kept (only this chunk's blocks converted)
                imgs = [backend.prefill_images(pos0 + steps, 2, 256) for _ in sets]
                row["us_split_kept_images"] = 1e3 * time_graph(
                    torch, lambda: [backend.attention_prefill(qc, kc, vc, 256**-0.5, torch.bfloat16,
                                                              q_offset=pos0, images=im)
                                    for (qc, kc, vc), im in zip(sets, imgs)],
                    max(20, esteps // 10), 5) / LAYERS
                del imgs
            del sets
            fl = 2 * heads * 256 * steps * (steps + 2 * pos0 + 1)
            row["TFLOPs_split"] = fl / (row["us_split"] * 1e-6) / 1e12
            chunked.append(row)
        extra["chunked_prefill"] = chunked
        log("chunked prefill: " + json.dumps(chunked))
        # decode-step preparation (q/k RMSNorm + RoPE + bf16 cache writes, layers.py:58-73)
        # for six layers: one fused launch each vs the reference's six-launch decomposition
        # (rms_norm x2, rope x2, index_copy_ x2) on the same HIP operators.
        from breezetoken_amd.backend import rope_tables

        RD, PCAP = 64, 65536
        tcos, tsin = rope_tables(PCAP, RD, 1.0e7, dev)
        gp = torch.Generator().manual_seed(7)
        qkvs = [torch.randn(H * 2 * D + 2 * HKV * D, generator=gp).to(dev) for _ in range(LAYERS)]
        qn = torch.randn(D, generator=gp).to(dev)
        kn = torch.randn(D, generator=gp).to(dev)
        pcaches = [(torch.zeros(PCAP, HKV * D, dtype=torch.bfloat16, device=dev),
                    torch.zeros(PCAP, HKV * D, dtype=torch.bfloat16, device=dev)) for _ in range(LAYERS)]
        ppos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
        pidx = ppos.long()

        def prep_fused():
            for x, (kc_, vc_) in zip(qkvs, pcaches):
                backend.attn_prep(x, qn, kn, 1e-6, tcos, tsin, ppos, RD, kc_, vc_, H, HKV, D)

        def prep_split():
            for x, (kc_, vc_) in zip(qkvs, pcaches):
                q_ = x[: H * 2 * D].view(H, 2 * D)[:, :D]
                k_ = x[H * 2 * D: H * 2 * D + HKV * D].view(HKV, D)
                v_ = x[H * 2 * D + HKV * D:].view(1, HKV * D)
                q_ = backend.rope(backend.rms_norm(q_, qn, 1e-6), tcos, tsin, ppos, RD)
                k_ = backend.rope(backend.rms_norm(k_, kn, 1e-6), tcos, tsin, ppos, RD)
                kc_.index_copy_(0, pidx, k_.reshape(1, -1).to(torch.bfloat16))
                vc_.index_copy_(0, pidx, v_.to(torch.bfloat16))

        fused_ms = time_graph(torch, prep_fused, esteps, ewarm) / LAYERS
        split_ms_p = time_graph(torch, prep_split, esteps, ewarm) / LAYERS
        pbytes = (H * D + 2 * HKV * D) * 4 + 2 * D * 4 + 2 * RD * 4 + H * D * 4 + 2 * HKV * D * 2
        extra["decode_prep"] = {
            "fused_us_per_layer": round(fused_ms * 1e3, 3), "unfused_us_per_layer": round(split_ms_p * 1e3, 3),
            "launches_fused": 1, "launches_unfused": 6, "speedup": round(split_ms_p / fused_ms, 2),
            "bytes_per_layer": pbytes, "shape": {"heads": H, "kv_heads": HKV, "head_dim": D, "rope_dim": RD}}
        log(f"decode prep: fused {fused_ms * 1e3:.2f} us/layer, unfused {split_ms_p * 1e3:.2f} us/layer")
        del pcaches
        torch.cuda.empty_cache()
        # Gated DeltaNet decode step (backends.py:79-92): one launch per layer vs the
        # reference's torch formulation (backends.py:242-271) on the same GPU.
        gdn = {}
        for name, hk_, hv_, nl in (("0.8B", 16, 16, 18), ("35B-A3B", 16, 32, 30)):
            dg = 128
            gg = torch.Generator().manual_seed(hv_)
            gq = torch.randn(hk_, dg, generator=gg).to(dev)
            gk = torch.randn(hk_, dg, generator=gg).to(dev)
            gv = torch.randn(hv_, dg, generator=gg).to(dev)
            glog = (-torch.rand(hv_, generator=gg) * 0.5).to(dev)
            gbeta = torch.randn(hv_, generator=gg).to(dev)
            states = [(torch.randn(hv_, dg, dg, generator=gg) * 0.1).to(dev) for _ in range(nl)]
            sc = dg ** -0.5
            kmap = torch.arange(hv_, device=dev) % hk_

            def gdn_hip():
                for st_ in states:
                    backend.gdn_decode(gq, gk, gv, glog, gbeta, st_, sc)

            def gdn_torch():
                for st_ in states:
                    qn_ = gq * torch.rsqrt(gq.pow(2).sum(-1, keepdim=True) + 1e-6) * sc
                    kn_ = gk * torch.rsqrt(gk.pow(2).sum(-1, keepdim=True) + 1e-6)
                    dec = st_ * torch.exp(glog).view(hv_, 1, 1)
                    rec = torch.einsum("hdv,hd->hv", dec, kn_[kmap])
                    dl = (gv - rec) * torch.sigmoid(gbeta).unsqueeze(-1)
                    st_.copy_(dec + kn_[kmap].unsqueeze(-1) * dl.unsqueeze(-2))
                    torch.einsum("hdv,hd->hv", st_, qn_[kmap])

            hip_ms = time_graph(torch, gdn_hip, esteps, ewarm) / nl
            torch_ms = time_graph(torch, gdn_torch, max(20, esteps // 5), 5) / nl
            gbytes = 2 * hv_ * dg * dg * 4 + 2 * hk_ * dg * 4 + 2 * hv_ * dg * 4 + 2 * hv_ * 4
            gdn[name] = {"heads_k": hk_, "heads_v": hv_, "dim": dg, "layers_per_graph": nl,
                         "us_per_layer": round(hip_ms * 1e3, 3), "GBps": round(gbytes / (hip_ms * 1e-3) / 1e9, 1),
                         "frac_hbm_peak": round(gbytes / (hip_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "bytes_per_layer": gbytes, "torch_gpu_us_per_layer": round(torch_ms * 1e3, 3)}
            log(f"gdn {name}: {hip_ms * 1e3:.2f} us/layer ({gbytes / (hip_ms * 1e-3) / 1e9:.0f} GB/s), "
                f"torch on GPU {torch_ms * 1e3:.2f} us/layer")
            del states
        extra["gdn_decode"] = gdn
        torch.cuda.empty_cache()
        # decode matvec (backends.py:36-37): the vocabulary head and the 0.8B projections, with
        # enough distinct weight copies per graph to stream from HBM (> 256 MB MALL), against
        # torch's bf16 matmul (vendor BLAS) on the same weights.
        gemv = {}
        for name, K, N in (("head", 1024, 248320), ("attn_qkv", 1024, 5120), ("mlp_gate_up", 1024, 7168),
                           ("mlp_down", 3584, 1024)):
            copies = max(1, -(-384 * 2**20 // (K * N * 2)))
            gw = torch.Generator().manual_seed(K + N)
            xs_ = torch.randn(K, generator=gw).to(dev)
            wts = [torch.randn(K, N, generator=gw).to(torch.bfloat16).to(dev) for _ in range(copies)]
            xb = xs_.to(torch.bfloat16).reshape(1, K)
            hip_ms = time_graph(torch, lambda: [backend.linear(xs_, w_) for w_ in wts],
                                max(20, esteps // 5), 5) / copies
            blas_ms = time_graph(torch, lambda: [torch.matmul(xb, w_) for w_ in wts],
                                 max(20, esteps // 5), 5) / copies
            wbytes = K * N * 2 + K * 4 + N * 4
            gemv[name] = {"K": K, "N": N, "copies_per_graph": copies, "us_per_call": round(hip_ms * 1e3, 3),
                          "GBps": round(wbytes / (hip_ms * 1e-3) / 1e9, 1),
                          "frac_hbm_peak": round(wbytes / (hip_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                          "torch_bf16_matmul_us": round(blas_ms * 1e3, 3)}
            log(f"gemv {name} {K}x{N}: {hip_ms * 1e3:.2f} us ({wbytes / (hip_ms * 1e-3) / 1e9:.0f} GB/s), "
                f"torch bf16 matmul {blas_ms * 1e3:.2f} us")
            del wts
            torch.cuda.empty_cache()
        extra["gemv"] = gemv

    # ------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    if not args.no_cpu:
        cpu_baseline, cpu_rows = cpu_baselines(torch, head_case, L, nbytes, args.cpu_seconds, args.no_extra)
        if cpu_rows:
            extra["cpu_rows"] = cpu_rows

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), bf16 KV cache)",
        "config": {"workload": "C2 split-KV GQA decode, H=8 Hkv=2 D=256, cap 65536, valid 32768 "
                               "(device pos), hipGraph replay", "batch": 1, "heads": H, "kv_heads": HKV,
                   "head_dim": D, "capacity": CAP, "valid": L, "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu_baseline, "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
