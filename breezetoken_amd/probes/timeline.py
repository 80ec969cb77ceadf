"""Per-work-group timeline of the short-prompt prefill kernel (gqa_prefill8).

Loads ``libbt_timeline.so`` -- the product library with gqa_prefill8.hip built
under BT_TIMELINE, made by ``breezetoken_amd.build.build()`` -- in place of the
product library, times config-4 prefill calls (bf16 q/k/v, H = 8, Hkv = 2,
D = 256) in a hipGraph of six calls, then records one eager call and prints,
for waves 0 and 4, the minimum / median / maximum over work-groups of each of
the kernel's eight timestamps (microseconds from the first work-group's start;
the device clock runs at 100 MHz) and each work-group's span.

usage: python -m breezetoken_amd.probes.timeline 128,512,2048
"""

from __future__ import annotations

import ctypes
import sys

import numpy as np

POINTS = ["start", "q ready", "tiles ready", "block 0 done", "loop done", "last P.V", "stores issued",
          "stores done"]
SLOTS = 4096 * 16


def main(argv: list[str]) -> int:
    import torch

    from breezetoken_amd import _lib, build, workloads as wl
    from breezetoken_amd.backend import HipBackend

    if not build.TIMELINE_LIB.exists():
        raise SystemExit(f"{build.TIMELINE_LIB} is missing: run breezetoken_amd.build.build() first")
    _lib.LIB_PATH = build.TIMELINE_LIB
    _lib._lib = None
    be = HipBackend("cuda:0")
    lib = _lib.lib()
    lib.bt_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.bt_timeline_read.restype = ctypes.c_int
    lib.bt_timeline_clear.restype = ctypes.c_int
    for S in [int(x) for x in argv[0].split(",")]:
        q, k, v, sc = wl.c4_inputs(S)
        base = (q.cuda(), k.cuda(), v.cuda())
        sets = [tuple(t.clone() for t in base) for _ in range(6)]
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            for a, b, c in sets:  # warm-up outside the capture: workspaces are allocated here
                be.attention_prefill(a, b, c, sc, torch.bfloat16)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                for a, b, c in sets:
                    be.attention_prefill(a, b, c, sc, torch.bfloat16)
        for _ in range(20):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(60):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us_call = e0.elapsed_time(e1) * 1e3 / 60 / 6
        if lib.bt_timeline_clear() != 0:
            raise RuntimeError("bt_timeline_clear failed")
        be.attention_prefill(*base, sc, torch.bfloat16)
        torch.cuda.synchronize()
        buf = np.zeros(SLOTS, dtype=np.uint64)
        if lib.bt_timeline_read(buf.ctypes.data, SLOTS) != 0:
            raise RuntimeError("bt_timeline_read failed")
        t = buf.reshape(4096, 2, 8).astype(np.int64)
        t = t[t[:, 0, 0] > 0]
        t0 = t[:, 0, 0].min()
        print(f"S {S}: {us_call:.2f} us per call (hipGraph of 6); eager call: {len(t)} work-groups recorded",
              flush=True)
        for w in (0, 1):
            print(f"  wave {4 * w}:")
            for kk, name in enumerate(POINTS):
                x = (t[:, w, kk] - t0) / 100.0
                print(f"    {name:14s} min {x.min():7.2f}  med {np.median(x):7.2f}  max {x.max():7.2f}")
        span = (t[:, 1, 7] - t[:, 0, 0]) / 100.0
        print(f"  work-group span (wave 0 start -> wave 4 stores done): min {span.min():.2f} "
              f"med {np.median(span):.2f} max {span.max():.2f}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
