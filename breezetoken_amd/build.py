"""Build libbreezetoken_amd.so for gfx950 with hipcc (no torch headers involved).

``python -m breezetoken_amd.build`` compiles every ``csrc/*.hip`` to an object in
parallel and links the shared library in-tree, next to this file.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libbreezetoken_amd.so"
# Machine-floor probes for bench.py --mode floor (not part of the attention ABI).
PROBE_SRC = PKG / "probes" / "floor.hip"
PROBE_LIB = PKG / "libbt_floor.so"
# The product library with gqa_prefill8.hip built under BT_TIMELINE: the
# prefill timeline probe (probes/timeline.py) loads it in place of LIB.
TIMELINE_SRC = CSRC / "gqa_prefill8.hip"
TIMELINE_LIB = PKG / "libbt_timeline.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-warning-option",
    # Keep hipcc from emitting packed-FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; install ROCm or set HIPCC")


def _compile(src: Path, obj: Path, extra: tuple[str, ...] = ()) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def _link(objs: list[Path], lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> Path:
    """Compile all kernels and link ``libbreezetoken_amd.so`` (and the floor
    probes' ``libbt_floor.so``); returns the attention library's path."""
    srcs = sorted(CSRC.glob("*.hip"))
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in srcs]
    probe_obj = objdir / "floor_probe.o"
    tl_obj = objdir / "prefill8_timeline.o"
    jobs = [(s, o, ()) for s, o in zip(srcs, objs)]
    jobs += [(PROBE_SRC, probe_obj, ()), (TIMELINE_SRC, tl_obj, ("-DBT_TIMELINE",))]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        list(ex.map(lambda job: _compile(*job), jobs))
    _link(objs, LIB)
    _link([probe_obj], PROBE_LIB)
    _link([o for o in objs if o.stem != TIMELINE_SRC.stem] + [tl_obj], TIMELINE_LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, {PROBE_LIB.name} and {TIMELINE_LIB.name}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
