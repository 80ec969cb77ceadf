"""Config-1 golden vector: inputs, oracle output and its float64 counterpart."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from breezetoken_amd.workloads import c1_inputs
from oracle.attention import brute_force_decode_f64, compare, torch_attention

FIXTURE = Path(__file__).resolve().parent / "golden" / "c1_decode.npz"


def _load():
    with np.load(FIXTURE, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _from_bits(a):
    return torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def test_fixture_inputs_match_seeded_generator():
    g = _load()
    case = c1_inputs()
    assert np.array_equal(case.q.view(torch.int16).numpy().view(np.uint16), g["q_bf16"])
    assert np.array_equal(case.k.view(torch.int16).numpy().view(np.uint16), g["k_bf16"])
    assert np.array_equal(case.v.view(torch.int16).numpy().view(np.uint16), g["v_bf16"])
    assert g["q_bf16"].shape == (8, 256) and g["k_bf16"].shape == (128, 2, 256)


def test_oracle_reproduces_golden_output():
    g = _load()
    q, k, v = (_from_bits(g[n]).float() for n in ("q_bf16", "k_bf16", "v_bf16"))
    out = torch_attention(q, k, v, float(g["scale"])).numpy()
    assert np.abs(out - g["out_f32"]).max() < 1e-6
    err, cos = compare(g["out_f32"], g["out_f64"])
    assert err < 1e-5 and cos > 1 - 1e-9
    f64 = brute_force_decode_f64(q.numpy(), k.numpy(), v.numpy(), float(g["scale"]))
    assert np.abs(f64 - g["out_f64"]).max() < 1e-12
