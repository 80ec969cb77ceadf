"""Write the config-1 golden vector (tests/golden/c1_decode.npz).

Config 1: one GQA decode call, B=1, H=8, Hkv=2, D=256, S=128; q, K, V drawn
N(0, 1) from torch.Generator seed 0 in that order, stored bf16 and upcast to
f32; softmax scale 1/16.  The expected output is the restated reference torch
f32 oracle (``oracle.attention.torch_attention``, backends.py:196-209); the
float64 brute force is stored beside it.  Inputs are kept as raw bf16 bit
patterns (uint16) so the fixture does not depend on the generator.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from breezetoken_amd.workloads import c1_inputs  # noqa: E402
from oracle.attention import brute_force_decode_f64, torch_attention  # noqa: E402

OUT = Path(__file__).resolve().parent / "c1_decode.npz"


def bits(t):
    return t.contiguous().view(__import__("torch").int16).numpy().view(np.uint16)


def main() -> None:
    case = c1_inputs()
    q, k, v = case.q.float(), case.k.float(), case.v.float()
    out = torch_attention(q, k, v, case.scale).numpy().astype(np.float32)
    out64 = brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), case.scale)
    np.savez_compressed(
        OUT, q_bf16=bits(case.q), k_bf16=bits(case.k), v_bf16=bits(case.v),
        scale=np.float64(case.scale), out_f32=out, out_f64=out64,
    )
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
