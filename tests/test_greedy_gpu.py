"""64-token greedy decode: identical token ids with the HIP attention and with
the torch f32 reference attention.

A small seeded decoder with the Qwen3.5 attention layer's shape (8 query heads
with a sigmoid output gate, 2 kv heads, head_dim 256, q/k RMSNorm, RoPE, bf16
fixed-capacity KV cache written before it is read; breezetoken/model/layers.py:
55-82, graph.py:35-63, prefill.py:36-80) runs twice on the GPU with every
operation identical except attention:

* HIP path: ``HipBackend.attention_prefill`` for the prompt and
  ``attention_fixed`` (device position tensor, the graph-decode operator) for
  every generated token;
* reference path: the restated ``_torch_attention`` / causal SDPA of the oracle
  in f32 on the CPU, fed the same bf16 cache contents (backends.py:196-215,
  prefill.py:56-68).

Both paths must produce the same 64 token ids.  The smallest top-1/top-2 logit
margin of the reference run is printed so a near-tie would be visible.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as orc

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN, LAYERS, FFN = 4096, 1024, 4, 2048
H, HKV, D = 8, 2, 256
PROMPT, NEW = 16, 64
CAP = 256  # KV cache slots


def _params(device):
    g = torch.Generator().manual_seed(1234)

    def w(*shape, fan_in):
        return (torch.randn(*shape, generator=g) / math.sqrt(fan_in)).to(device)

    layers = []
    for _ in range(LAYERS):
        layers.append({
            "norm": torch.ones(HIDDEN, device=device),
            "w_qkv": w(H * 2 * D + 2 * HKV * D, HIDDEN, fan_in=HIDDEN),
            "q_norm": (1.0 + 0.1 * torch.randn(D, generator=g)).to(device),
            "k_norm": (1.0 + 0.1 * torch.randn(D, generator=g)).to(device),
            "w_o": w(HIDDEN, H * D, fan_in=H * D),
            "norm2": torch.ones(HIDDEN, device=device),
            "w_gate": w(FFN, HIDDEN, fan_in=HIDDEN),
            "w_up": w(FFN, HIDDEN, fan_in=HIDDEN),
            "w_down": w(HIDDEN, FFN, fan_in=FFN),
        })
    emb = w(VOCAB, HIDDEN, fan_in=1) * 0.5
    head = w(VOCAB, HIDDEN, fan_in=HIDDEN) * 4.0  # sharper logits: clear top-1 margins
    prompt = torch.randint(0, VOCAB, (PROMPT,), generator=g)
    return layers, emb, head, prompt


def _rms(x, w, eps=1e-6):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x, pos):
    """x (T, heads, D), pos (T,) int -> rotary embedding over the full head dim."""
    half = D // 2
    inv = 1.0 / (10000.0 ** (torch.arange(half, device=x.device, dtype=torch.float32) / half))
    ang = pos.to(torch.float32)[:, None] * inv[None, :]
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)


def _rope_tab(x, positions, cos, sin):
    """The same rotation from (CAP, D) tables (layers.py:26-32, backends.py:218-226)."""
    half = D // 2
    c, s_ = cos[positions][:, None, :], sin[positions][:, None, :]
    return x * c + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * s_


class _Decoder:
    def __init__(self, params, attn_prefill, attn_decode, device, tables=None, prep_decode=None):
        self.layers, self.emb, self.head, _ = params
        self.attn_prefill, self.attn_decode = attn_prefill, attn_decode
        self.tables, self.prep_decode = tables, prep_decode
        self.device = device
        self.k = [torch.zeros(CAP, HKV * D, dtype=torch.bfloat16, device=device) for _ in range(LAYERS)]
        self.v = [torch.zeros(CAP, HKV * D, dtype=torch.bfloat16, device=device) for _ in range(LAYERS)]
        self.pos = torch.zeros(1, dtype=torch.int32, device=device)

    def _block(self, i, x, positions, decode: bool):
        p = self.layers[i]
        t = x.shape[0]
        qkv = _rms(x, p["norm"]) @ p["w_qkv"].T
        if decode and self.prep_decode is not None:
            # q/k norm + RoPE + cache writes at the device position in one call
            q, gate = self.prep_decode(qkv.reshape(-1), p, self.k[i], self.v[i], self.pos)
            q, gate = q.reshape(1, H, D), gate.reshape(1, H, D)
        else:
            qg = qkv[:, : H * 2 * D].reshape(t, H, 2 * D)
            q, gate = qg[..., :D], qg[..., D:]
            k = qkv[:, H * 2 * D : H * 2 * D + HKV * D].reshape(t, HKV, D)
            v = qkv[:, H * 2 * D + HKV * D :].reshape(t, HKV, D)
            if self.tables is not None:
                q = _rope_tab(_rms(q, p["q_norm"]), positions, *self.tables)
                k = _rope_tab(_rms(k, p["k_norm"]), positions, *self.tables)
            else:
                q = _rope(_rms(q, p["q_norm"]), positions)
                k = _rope(_rms(k, p["k_norm"]), positions)
            self.k[i][positions] = k.reshape(t, -1).to(torch.bfloat16)  # write before read
            self.v[i][positions] = v.reshape(t, -1).to(torch.bfloat16)
        kc = self.k[i].view(CAP, HKV, D)
        vc = self.v[i].view(CAP, HKV, D)
        if decode:
            out = self.attn_decode(q.reshape(H, D), kc, vc, self.pos, D**-0.5).reshape(1, H, D)
        else:
            out = self.attn_prefill(q, kc[:t], vc[:t], D**-0.5)
        out = out * torch.sigmoid(gate)
        x = x + out.reshape(t, H * D) @ p["w_o"].T
        h = _rms(x, p["norm2"])
        return x + (torch.nn.functional.silu(h @ p["w_gate"].T) * (h @ p["w_up"].T)) @ p["w_down"].T

    def _logits(self, x):
        return _rms(x, torch.ones(HIDDEN, device=self.device)) @ self.head.T

    def generate(self, prompt):
        ids = prompt.to(self.device)
        x = self.emb[ids]
        positions = torch.arange(PROMPT, device=self.device)
        for i in range(LAYERS):
            x = self._block(i, x, positions, decode=False)
        logits = self._logits(x[-1:])
        out, margins = [], []
        for step in range(NEW):
            top = torch.topk(logits[0], 2)
            margins.append(float(top.values[0] - top.values[1]))
            tok = int(top.indices[0])
            out.append(tok)
            if step == NEW - 1:
                break
            pos = PROMPT + step
            self.pos.fill_(pos)
            x = self.emb[torch.tensor([tok], device=self.device)]
            for i in range(LAYERS):
                x = self._block(i, x, torch.tensor([pos], device=self.device), decode=True)
            logits = self._logits(x)
        return out, margins


def _ref_prefill(q, k, v, scale):
    # the kernel's inputs: bf16 q, the bf16 cache; reference arithmetic in f32 on the CPU
    qb = q.to(torch.bfloat16).float().cpu()
    return orc.torch_prefill_attention(qb, k.float().cpu(), v.float().cpu(), scale).to(q.device)


def _ref_decode(q, k, v, pos, scale):
    valid = int(pos.item()) + 1
    return orc.torch_attention(q.float().cpu(), k[:valid].float().cpu(), v[:valid].float().cpu(),
                               scale).to(q.device)


def test_greedy_64_tokens_identical(hip_backend):
    dev = torch.device("cuda")
    params = _params(dev)
    prompt = params[3]

    def hip_prefill(q, k, v, scale):
        return hip_backend.attention_prefill(q.to(torch.bfloat16), k, v, scale, torch.float32)

    def hip_decode(q, k, v, pos, scale):
        return hip_backend.attention_fixed(q.float().contiguous(), k, v, pos, scale)

    print("[greedy] reference path", flush=True)
    ref_ids, margins = _Decoder(params, _ref_prefill, _ref_decode, dev).generate(prompt)
    print("[greedy] HIP path", flush=True)
    hip_ids, _ = _Decoder(params, hip_prefill, hip_decode, dev).generate(prompt)
    print(f"[greedy] min top-1 margin {min(margins):.4f}, distinct ids {len(set(ref_ids))}", flush=True)
    assert len(hip_ids) == NEW
    assert hip_ids == ref_ids, f"first divergence at step {next(i for i, (a, b) in enumerate(zip(hip_ids, ref_ids)) if a != b)}"


def test_greedy_64_tokens_identical_with_fused_decode_prep(hip_backend):
    """As above, and the HIP path also runs each decode step's q/k RMSNorm,
    RoPE and bf16 cache writes as one ``attn_prep`` launch (layers.py:58-73)
    instead of the torch operators; both paths rotate with the same tables."""
    from oracle import prep as orp

    dev = torch.device("cuda")
    params = _params(dev)
    prompt = params[3]
    cos, sin = (t.to(dev) for t in orp.rope_tables(CAP, D, 10000.0))

    def hip_prefill(q, k, v, scale):
        return hip_backend.attention_prefill(q.to(torch.bfloat16), k, v, scale, torch.float32)

    def hip_decode(q, k, v, pos, scale):
        return hip_backend.attention_fixed(q.float().contiguous(), k, v, pos, scale)

    def hip_prep(qkv, p, kc, vc, pos):
        return hip_backend.attn_prep(qkv.contiguous(), p["q_norm"], p["k_norm"], 1e-6, cos, sin, pos, D,
                                     kc, vc, H, HKV, D)

    print("[greedy+prep] reference path", flush=True)
    ref_ids, margins = _Decoder(params, _ref_prefill, _ref_decode, dev, tables=(cos, sin)).generate(prompt)
    print("[greedy+prep] HIP path", flush=True)
    hip_ids, _ = _Decoder(params, hip_prefill, hip_decode, dev, tables=(cos, sin),
                          prep_decode=hip_prep).generate(prompt)
    print(f"[greedy+prep] min top-1 margin {min(margins):.4f}, distinct ids {len(set(ref_ids))}", flush=True)
    assert hip_ids == ref_ids, f"first divergence at step {next(i for i, (a, b) in enumerate(zip(hip_ids, ref_ids)) if a != b)}"
