#!/usr/bin/env python3
"""Benchmark of the MI355X GQA attention path (one GPU).

Headline (BASELINE.json ``metric``, config 2): split-KV GQA flash-decode,
Qwen3.5-0.8B-like H=8 / Hkv=2 / D=256, bf16 fixed-capacity cache of 65,536
slots, valid length 32,768 given by a device position tensor, q/K/V ~ N(0, 1)
bf16 (seed 1).  One step = one decode call (split + LSE combine) captured in a
hipGraph (``torch.cuda.graph``) and replayed; inputs are resident in HBM.
``value`` = algorithmic bytes of a call / time per call, in GB/s.

Also reported (``extra``): 1k/4k/32k decode, config 3, config 5 (ragged), a
cold-cache variant of config 2 (5 rotating caches > the 256 MB Infinity Cache)
and causal prefill TFLOP/s (config 4) when the prefill kernel is served.

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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    args = ap.parse_args()
    if args.gpus != 1:
        print("this build measures one GPU only: the decode/prefill kernels run on a single "
              "MI355X and no multi-GPU path is built (see DESIGN.md); run with --gpus 1",
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

    def fixed_case(case, cap):
        cache = KVCache(cap, case.k.shape[1], case.k.shape[2], dev)
        cache.k.copy_(case.k.reshape(cap, -1))
        cache.v.copy_(case.v.reshape(cap, -1))
        kv, vv = cache.views()
        q = case.q.float().to(dev)
        pos = torch.tensor([case.pos], dtype=torch.int32, device=dev)
        return cache, q, kv, vv, pos

    def decode_point(case, cap, steps, warmup, check=False):
        cache, q, kv, vv, pos = fixed_case(case, cap)
        heads = case.q.shape[0]
        ms = time_graph(torch, lambda: backend.attention_fixed(q, kv, vv, pos, case.scale), steps, warmup)
        nbytes = wl.decode_bytes(case.valid, heads, kv.shape[1], kv.shape[2])
        res = {"valid": case.valid, "us_per_call": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9,
               "frac_hbm_peak": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes": nbytes}
        if check:
            from oracle.attention import compare, fixed_decode  # checker only

            out = backend.attention_fixed(q, kv, vv, pos, case.scale).cpu()
            ref = fixed_decode(case.q.float(), case.k.float(), case.v.float(), case.pos, case.scale)
            err, cos = compare(out.numpy(), ref.numpy())
            res["parity"] = {"max_abs": err, "cosine": cos}
        del cache
        return res

    # ---------------------------------------------------------------- headline
    L = 32768
    log(f"config 2 headline: H={H} Hkv={HKV} D={D} cap={CAP} valid={L}")
    head_case = wl.c2_inputs(L, cap=CAP)
    cache, q, kv, vv, pos = fixed_case(head_case, CAP)
    step = lambda: backend.attention_fixed(q, kv, vv, pos, head_case.scale)  # noqa: E731
    ms_per_step = time_graph(torch, step, args.steps, args.warmup)
    nbytes = wl.decode_bytes(L, H, HKV, D)
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    log(f"headline: {ms_per_step * 1e3:.2f} us/call, {value:.0f} GB/s")

    # ---- roofline: the split kernel alone, HIP events on its stream ----------
    lib = _lib.lib()
    ns = backend.pick_splits(HKV, CAP)
    lse = torch.empty((H, ns), dtype=torch.float32, device=dev)
    part = torch.empty((H, ns, D), dtype=torch.float32, device=dev)

    def split_only():
        rc = lib.bt_gqa_decode_split(
            q.data_ptr(), _lib.BT_DTYPE_F32, H * D, kv.data_ptr(), vv.data_ptr(), kv.stride(0),
            kv.stride(1), None, pos.data_ptr(), None, 0, 1, H, HKV, D, ns, head_case.scale,
            lse.data_ptr(), part.data_ptr(), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
        )
        _lib.check("bt_gqa_decode_split", rc)

    split_ms = time_graph(torch, split_only, args.steps, args.warmup, calls_per_graph=20)
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
                   "num_cus": backend.num_cus, "arch": backend.arch}
    # --------------------------------------------------------------- extras
    if not args.no_extra:
        esteps, ewarm = max(100, args.steps // 2), max(10, args.warmup // 2)
        extra["c2"] = [decode_point(wl.c2_inputs(v, cap=CAP), CAP, esteps, ewarm, check=True)
                       for v in (1024, 4096, 32768)]
        log("c2 sweep: " + ", ".join(f"{r['valid']}: {r['us_per_call']:.2f}us {r['GBps']:.0f}GB/s"
                                     for r in extra["c2"]))
        # cold: 5 distinct caches (>256 MB Infinity Cache), one call each per replay
        caches = [fixed_case(head_case, CAP) for _ in range(5)]
        def cold():
            for c in caches:
                backend.attention_fixed(c[1], c[2], c[3], c[4], head_case.scale)
        cold_ms = time_graph(torch, cold, esteps, ewarm) / 5
        extra["c2_cold_32k"] = {"us_per_call": cold_ms * 1e3, "GBps": nbytes / (cold_ms * 1e-3) / 1e9,
                                "frac_hbm_peak": nbytes / (cold_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                                "caches": 5}
        log(f"c2 cold 32k: {cold_ms * 1e3:.2f} us/call")
        del caches
        c3 = []
        for v in (8192, 32768, 131072):
            c3.append(decode_point(wl.c3_inputs(v, cap=131072), 131072, esteps, ewarm))
        extra["c3"] = c3
        log("c3: " + ", ".join(f"{r['valid']}: {r['us_per_call']:.2f}us {r['GBps']:.0f}GB/s" for r in c3))
        # ragged (config 5)
        rc5 = wl.c5_inputs()
        rq = rc5.q.float().to(dev)
        rk, rv = rc5.k.to(dev), rc5.v.to(dev)
        roff = torch.tensor(rc5.offsets, dtype=torch.int64, device=dev)
        rlen = torch.tensor(rc5.lens, dtype=torch.int32, device=dev)
        rms = time_graph(torch, lambda: backend.attention_ragged(rq, rk, rv, roff, rlen, rc5.lens, rc5.scale),
                         esteps, ewarm)
        rbytes = 2 * sum(rc5.lens) * HKV * D * 2 + len(rc5.lens) * H * D * 4 * 2
        extra["c5_ragged"] = {"us_per_call": rms * 1e3, "GBps": rbytes / (rms * 1e-3) / 1e9,
                              "frac_hbm_peak": rbytes / (rms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                              "tokens": sum(rc5.lens), "bytes": rbytes}
        log(f"c5 ragged: {rms * 1e3:.2f} us/call")
        del rk, rv
        # prefill (config 4), if served
        pre = []
        for s in (128, 512, 2048, 8192):
            qp, kp, vp, sc = (t.to(dev) if hasattr(t, "to") else t for t in wl.c4_inputs(s))
            try:
                pms = time_graph(torch, lambda: backend.attention_prefill(qp, kp, vp, sc, torch.bfloat16),
                                 max(20, esteps // 10), 5)
            except RuntimeError as exc:
                pre.append({"steps": s, "error": str(exc)[:120]})
                break
            fl = wl.prefill_flops(s, 8, 256)
            pre.append({"steps": s, "us_per_call": pms * 1e3, "TFLOPs": fl / (pms * 1e-3) / 1e12,
                        "frac_bf16_peak": fl / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS})
        extra["c4_prefill"] = pre
        log("c4: " + json.dumps(pre))

    # ------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    if not args.no_cpu:
        from oracle.attention import torch_attention  # the reference CPU path, restated

        threads = torch.get_num_threads()
        qc = head_case.q.float()
        kc = head_case.k[:L].float()
        vc = head_case.v[:L].float()
        for _ in range(3):
            torch_attention(qc, kc, vc, head_case.scale)
        times = []
        t_end = time.perf_counter() + args.cpu_seconds
        while len(times) < 20 or (time.perf_counter() < t_end and len(times) < 2000):
            t0 = time.perf_counter()
            torch_attention(qc, kc, vc, head_case.scale)
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        cpu_baseline = {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
                        "kind": "port", "us_per_call": round(med * 1e6, 1),
                        "sample": f"{len(times)} calls of config-2 decode (valid 32768, H=8, Hkv=2, "
                                  f"D=256) in torch f32 SDPA on the host CPU, median; "
                                  f"cpu={os.cpu_count()} logical, torch threads={threads}"}
        log(f"cpu baseline: {med * 1e6:.0f} us/call on {threads} threads")

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
