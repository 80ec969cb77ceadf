"""GPU parity of the causal GQA prefill kernel against the CPU oracle.

The f32-output mode is held to the decode gate (max-abs <= 2e-3, cosine >=
0.99999) against the restated causal SDPA (prefill.py:56-68) in f32 on the same
bf16 inputs.  The bf16-output mode is compared with that reference rounded to
bf16: one bf16 rounding of |o| ~ 2-4 alone is up to 2^-8 * 4 = 1.6e-2, so the
bound there is 2e-3 plus one bf16 half-ulp of the reference value.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from breezetoken_amd import workloads as wl
from oracle import attention as orc

pytestmark = pytest.mark.gpu

ATOL = 2e-3
COS = 0.99999


def _close(got, ref, atol=ATOL, cos_min=COS):
    g = got.detach().float().cpu().numpy()
    r = ref.detach().float().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    assert np.isfinite(g).all(), "non-finite output"
    err, cos = orc.compare(g, r)
    assert err <= atol and cos >= cos_min, f"max-abs {err:.3e}, cosine {cos:.8f}"


def _inputs(steps, heads=8, kv=2, dim=256, seed=3):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(steps, heads, dim, generator=g).to(torch.bfloat16)
    k = torch.randn(steps, kv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(steps, kv, dim, generator=g).to(torch.bfloat16)
    return q, k, v, dim**-0.5


@pytest.mark.parametrize("steps", [128, 512, 2048])
def test_c4_prefill_f32_output(hip_backend, steps):
    q, k, v, scale = wl.c4_inputs(steps)
    print(f"[c4] S={steps}", flush=True)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale)
    assert out.shape == (steps, 8, 256) and out.dtype == torch.float32
    _close(out, ref)


def test_c4_prefill_8192_full_output(hip_backend):
    """S = 8192, every row against the restated causal SDPA in f32 (pair kernel)."""
    q, k, v, scale = wl.c4_inputs(8192)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(out, ref)


def test_c4_prefill_8192_sampled_rows(hip_backend):
    """S = 8192: every sampled row i must equal decode attention over keys 0..i."""
    q, k, v, scale = wl.c4_inputs(8192)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    rows = [0, 1, 31, 32, 63, 64, 1000, 4095, 4096, 8000, 8190, 8191]
    for i in rows:
        ref = orc.torch_attention(q[i].float(), k[: i + 1].float(), v[: i + 1].float(), scale)
        _close(out[i], ref)


@pytest.mark.parametrize("steps", [128, 512, 2048, 8192])
def test_c4_prefill_bf16_output(hip_backend, steps):
    """Config 4's output format (bf16), on every path the benchmark times: the
    direct-tile kernel (S = 128), the split-key schedule (512, 2048) and the
    pair kernel (8192)."""
    q, k, v, scale = wl.c4_inputs(steps)
    print(f"[c4 bf16 out] S={steps}", flush=True)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    g = out.float().cpu()
    half_ulp = ref.abs().clamp_min(2.0**-126).log2().floor().exp2() * 2.0**-8
    assert ((g - ref).abs() <= ATOL + half_ulp).all()
    _close(g, ref.to(torch.bfloat16).float(), atol=4e-3 + 2.0**-7)


@pytest.mark.parametrize("steps", [1, 2, 7, 33, 65, 100, 257, 1000])
def test_ragged_prompt_lengths(hip_backend, steps):
    q, k, v, scale = _inputs(steps, seed=steps)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale), ref)


@pytest.mark.parametrize("heads,kv,dim", [(8, 2, 128), (4, 4, 256), (8, 4, 256), (16, 2, 256), (8, 8, 128),
                                          (16, 2, 128), (4, 2, 128),
                                          (6, 2, 256), (12, 2, 128), (10, 2, 256), (3, 1, 128)])
def test_other_group_sizes(hip_backend, heads, kv, dim):
    """Group sizes 1, 2, 4, 8 at D = 128 / 256 run the two-waves-per-SIMD kernel
    directly; 3, 5, 6 run it as subsets of 1 or 2 heads."""
    q, k, v, scale = _inputs(300, heads, kv, dim, seed=heads * 100 + kv)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale), ref)


def test_sdpa_shaped_shim(hip_backend):
    """The (1, H, S, D) call of prefill.py:60-68, including transposed views."""
    q, k, v, scale = _inputs(200)
    qq = q.cuda().transpose(0, 1).unsqueeze(0)
    kk = k.cuda().transpose(0, 1).unsqueeze(0)
    vv = v.cuda().transpose(0, 1).unsqueeze(0)
    out = hip_backend.sdpa_prefill(qq, kk, vv, scale)
    assert out.shape == (1, 8, 200, 256)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(out[0].transpose(0, 1), ref)


def test_prefill_rows_match_decode_kernel(hip_backend):
    """Row i of prefill equals the decode kernel over keys 0..i (test_model.py:92-98's
    batched == token-wise property, at the attention level)."""
    q, k, v, scale = _inputs(300, seed=11)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale)
    kd, vd = k.cuda(), v.cuda()
    for i in (0, 5, 63, 64, 199, 299):
        dec = hip_backend.attention(q[i].float().cuda(), kd[: i + 1], vd[: i + 1], scale)
        _close(out[i], dec, atol=1e-3)


def test_prefill_deterministic(hip_backend):
    q, k, v, scale = _inputs(500, seed=12)
    a = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).clone()
    b = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale)
    assert torch.equal(a, b)


def test_prefill_unserved_raises(hip_backend):
    q, k, v, scale = _inputs(16, dim=64)
    with pytest.raises(RuntimeError):
        hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale)


# ---------------------------------------------- chunked prefill (query offset)
@pytest.mark.parametrize("steps,pos0", [(128, 17), (300, 1000), (64, 64), (1, 5000), (65, 63), (257, 4096)])
def test_chunked_prefill_query_offset(hip_backend, steps, pos0):
    """The banded-mask chunk of qwen36_moe.py:394-428: queries at positions
    pos0 .. pos0 + S - 1 over keys 0 .. pos0 + S - 1."""
    g = torch.Generator().manual_seed(steps * 31 + pos0)
    q = torch.randn(steps, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(pos0 + steps, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(pos0 + steps, 2, 256, generator=g).to(torch.bfloat16)
    scale = 256**-0.5
    print(f"[chunk] S={steps} pos0={pos0}", flush=True)
    ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), pos0, scale)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=pos0)
    assert out.shape == (steps, 16, 256)
    _close(out, ref)


@pytest.mark.parametrize("heads,kv,dim,steps,pos0", [(8, 2, 256, 100, 37), (4, 4, 256, 70, 129), (8, 4, 128, 200, 64),
                                                     (6, 2, 256, 90, 300)])
def test_chunked_prefill_other_group_sizes(hip_backend, heads, kv, dim, steps, pos0):
    """Query offsets for group sizes 4, 1, 2 and 3 (three single-head subsets)."""
    g = torch.Generator().manual_seed(heads * 1000 + kv * 100 + pos0)
    q = torch.randn(steps, heads, dim, generator=g).to(torch.bfloat16)
    k = torch.randn(pos0 + steps, kv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(pos0 + steps, kv, dim, generator=g).to(torch.bfloat16)
    scale = dim**-0.5
    print(f"[chunk] H={heads} Hkv={kv} D={dim} S={steps} pos0={pos0}", flush=True)
    ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), pos0, scale)
    _close(hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=pos0), ref)


def _prefill_with_workspace(q, k, v, scale, q_offset, ws_bytes):
    """bt_gqa_prefill with a workspace of exactly ``ws_bytes`` (f32 output)."""
    import ctypes

    from breezetoken_amd import _lib

    steps, heads, dim = q.shape
    out = torch.empty((steps, heads, dim), dtype=torch.float32, device="cuda")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    rc = _lib.lib().bt_gqa_prefill(
        q.data_ptr(), _lib.BT_DTYPE_BF16, k.data_ptr(), v.data_ptr(), q.stride(0), q.stride(1), k.stride(0),
        k.stride(1),
        steps, q_offset, heads, k.shape[1], dim, float(scale), ws.data_ptr(), ws_bytes, out.data_ptr(),
        _lib.BT_DTYPE_F32, out.stride(0), out.stride(1),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check("bt_gqa_prefill", rc)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("heads,kv,steps,pos0", [(8, 2, 512, 0), (8, 2, 2048, 0), (8, 2, 256, 4096),
                                                 (16, 2, 128, 5000), (8, 2, 300, 1000), (4, 4, 200, 0)])
def test_split_key_schedule_matches_unsplit(hip_backend, heads, kv, steps, pos0):
    """Short prompts and long cached prefixes split the key range over several
    work-groups when the workspace holds the partials; the LSE merge of the
    chunks equals the one-work-group-per-query-block schedule and the oracle."""
    from breezetoken_amd import _lib

    lib = _lib.lib()
    g = torch.Generator().manual_seed(steps + pos0 + heads)
    q = torch.randn(steps, heads, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(pos0 + steps, kv, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(pos0 + steps, kv, 256, generator=g).to(torch.bfloat16)
    scale = 256**-0.5
    vt_only = lib.bt_prefill_workspace_bytes(pos0 + steps, kv, 256)
    split = lib.bt_prefill_split_workspace_bytes(steps, pos0, heads, kv, 256)
    print(f"[split] H={heads} Hkv={kv} S={steps} pos0={pos0} ws {vt_only} -> {split}", flush=True)
    assert split > vt_only  # these shapes leave CUs idle with one work-group per query block
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    unsplit = _prefill_with_workspace(qd, kd, vd, scale, pos0, vt_only)
    chunked = _prefill_with_workspace(qd, kd, vd, scale, pos0, split)
    ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), pos0, scale)
    _close(unsplit, ref)
    _close(chunked, ref)
    assert (chunked - unsplit).abs().max().item() <= 1e-3


def test_backend_split_keys_switch(hip_backend):
    """HipBackend.attention_prefill splits by default where the plan does, and
    split_keys=False keeps one work-group per query block; both match the oracle."""
    steps, pos0 = 64, 3000
    g = torch.Generator().manual_seed(41)
    q = torch.randn(steps, 16, 256, generator=g).to(torch.bfloat16)
    k = torch.randn(pos0 + steps, 2, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(pos0 + steps, 2, 256, generator=g).to(torch.bfloat16)
    scale = 256**-0.5
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    split = hip_backend.attention_prefill(qd, kd, vd, scale, q_offset=pos0)
    one = hip_backend.attention_prefill(qd, kd, vd, scale, q_offset=pos0, split_keys=False)
    torch.cuda.synchronize()
    ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), pos0, scale)
    _close(split, ref)
    _close(one, ref)
    assert (split - one).abs().max().item() <= 1e-3


def test_long_prompt_needs_no_split(hip_backend):
    """Config 4 at S = 8192 runs the pair kernel: no split and no extra workspace."""
    from breezetoken_amd import _lib

    lib = _lib.lib()
    assert lib.bt_prefill_split_workspace_bytes(8192, 0, 8, 2, 256) == lib.bt_prefill_workspace_bytes(8192, 2, 256)


def test_chunked_prefill_head_major_cache(hip_backend):
    """The SDPA call of qwen36_moe.py:415-423 on views of a head-major
    (Hkv, capacity, D) cache, and the chunks together equal one full prefill."""
    cap, total, split = 4096, 900, 333
    g = torch.Generator().manual_seed(40)
    kc = torch.zeros(2, cap, 256, dtype=torch.bfloat16)
    vc = torch.zeros(2, cap, 256, dtype=torch.bfloat16)
    kc[:, :total] = torch.randn(2, total, 256, generator=g).to(torch.bfloat16)
    vc[:, :total] = torch.randn(2, total, 256, generator=g).to(torch.bfloat16)
    q = torch.randn(total, 8, 256, generator=g).to(torch.bfloat16)
    scale = 256**-0.5
    kd, vd, qd = kc.cuda(), vc.cuda(), q.cuda()
    full = hip_backend.attention_prefill(qd, kd[:, :total].transpose(0, 1), vd[:, :total].transpose(0, 1), scale)
    parts = []
    for lo, hi in ((0, split), (split, total)):
        qq = qd[lo:hi].transpose(0, 1).unsqueeze(0)
        out = hip_backend.sdpa_prefill(qq, kd[:, :hi].unsqueeze(0), vd[:, :hi].unsqueeze(0), scale, q_offset=lo)
        assert out.shape == (1, 8, hi - lo, 256)
        parts.append(out[0].transpose(0, 1))
    chunked = torch.cat(parts)
    ref = orc.torch_prefill_attention(q.float(), kc[:, :total].transpose(0, 1).float(),
                                      vc[:, :total].transpose(0, 1).float(), scale)
    _close(chunked, ref)
    _close(full, ref)
    assert (chunked - full).abs().max().item() <= 1e-3


def test_chunked_prefill_bad_offset_raises(hip_backend):
    q, k, v, scale = _inputs(16)
    with pytest.raises(RuntimeError):
        hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=3)


@pytest.mark.parametrize("heads,kv,dim", [(8, 2, 256), (6, 2, 128), (16, 2, 256)])
def test_chunked_prefill_with_kept_images_equals_fresh_images(hip_backend, heads, kv, dim):
    """Chunked prefill over one cache with PrefillImages: every chunk converts
    only its own blocks, and equals (bit for bit) the call that rebuilds the
    images from the whole prefix; a rewound chunk and another cache rebuild."""
    cap = 2048
    g = torch.Generator().manual_seed(heads + dim)
    k = torch.randn(cap, kv, dim, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(cap, kv, dim, generator=g).to(torch.bfloat16).cuda()
    q_all = torch.randn(cap, heads, dim, generator=g).cuda()
    scale = dim**-0.5
    images = hip_backend.prefill_images(cap, kv, dim)
    chunks = [(0, 300), (300, 401), (701, 64), (765, 1), (766, 500), (1266, 700)]
    for pos0, s in chunks:
        q = q_all[pos0 : pos0 + s]
        kk, vv = k[: pos0 + s], v[: pos0 + s]
        got = hip_backend.attention_prefill(q, kk, vv, scale, q_offset=pos0, images=images)
        want = hip_backend.attention_prefill(q, kk, vv, scale, q_offset=pos0)
        assert torch.equal(got, want), (pos0, s)
        assert images.valid_keys == pos0 + s
    # the last chunk again (cached keys only up to its own start)
    pos0, s = chunks[-1]
    got = hip_backend.attention_prefill(q_all[pos0 : pos0 + s], k[: pos0 + s], v[: pos0 + s], scale,
                                        q_offset=pos0, images=images)
    ref = orc.torch_prefill_banded(q_all[pos0 : pos0 + s].cpu(), k[: pos0 + s].float().cpu(),
                                   v[: pos0 + s].float().cpu(), pos0, scale)
    _close(got, ref)
    # another cache through the same images object: rebuilt from key 0
    k2, v2 = (k * 0.5).contiguous(), (v * 2).contiguous()
    got = hip_backend.attention_prefill(q_all[500:600], k2[:600], v2[:600], scale, q_offset=500, images=images)
    want = hip_backend.attention_prefill(q_all[500:600], k2[:600], v2[:600], scale, q_offset=500)
    assert torch.equal(got, want)


@pytest.mark.parametrize("steps,q_offset,heads,kv,dim", [
    (1, 0, 8, 2, 256), (64, 0, 8, 2, 256), (100, 0, 8, 2, 256), (128, 0, 8, 2, 256), (128, 0, 16, 2, 256),
    (300, 0, 8, 2, 256), (512, 0, 8, 2, 256), (512, 0, 4, 4, 128), (128, 0, 2, 2, 128), (40, 17, 8, 2, 256),
    (100, 28, 8, 1, 256),
])
@pytest.mark.parametrize("pattern", ["normal", "large_v_tiny_k", "blockwise"])
def test_short_prompt_direct_tiles_equal_images(hip_backend, steps, q_offset, heads, kv, dim, pattern):
    """Short prompts (at most two 64-key blocks per work-group) convert K and V
    inside the main kernel instead of through the image pre-pass: the result
    equals, bit for bit, the image path (the kept-image entry point always
    takes it), and both match the oracle."""
    total = q_offset + steps
    g = torch.Generator().manual_seed(steps * 7 + heads + dim + q_offset)
    q = torch.randn(steps, heads, dim, generator=g)
    k = torch.randn(total, kv, dim, generator=g)
    v = torch.randn(total, kv, dim, generator=g)
    if pattern == "large_v_tiny_k":
        v, k = v * 3e4, k * 1e-3
    elif pattern == "blockwise":  # a different magnitude in every 64-key block
        for b in range(0, total, 64):
            v[b : b + 64] *= 10.0 ** (b // 64 % 5 - 2)
            k[b : b + 64] *= 2.0 ** (b // 64 % 3)
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    scale = dim**-0.5
    print(f"[direct] S={steps} off={q_offset} H={heads} Hkv={kv} D={dim} {pattern}", flush=True)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    direct = hip_backend.attention_prefill(qd, kd, vd, scale, q_offset=q_offset)
    images = hip_backend.prefill_images(total, kv, dim)
    via_images = hip_backend.attention_prefill(qd, kd, vd, scale, q_offset=q_offset, images=images)
    assert torch.equal(direct, via_images)
    ref = orc.torch_prefill_banded(q, k.float(), v.float(), q_offset, scale)
    amax = orc.torch_prefill_banded(q, k.float(), v.float().abs(), q_offset, scale).abs()
    err = (direct.cpu() - ref).abs()
    assert bool((err <= 2e-3 * torch.clamp(amax, min=1.0)).all()), float(err.max())


@pytest.mark.parametrize("steps,heads,kv,dim", [
    (1500, 8, 2, 256), (2048, 8, 2, 256), (3000, 8, 2, 256), (4096, 8, 2, 256), (2048, 16, 2, 128),
    (2500, 4, 2, 256), (3333, 8, 1, 128),
])
def test_paired_split_prefill(hip_backend, steps, heads, kv, dim):
    """Mid-length prompts take the paired split (query blocks nqb-1-r and r
    share the work-groups of pair r, ranges cut evenly, partials merged by the
    combine: S = 3000 and 4096 at H = 8, 2048 at H = 16, 3333 at Hkv = 1) or the
    uniform one (the others): every row matches the oracle; sampled rows are
    checked against decode attention over their prefix."""
    q, k, v, scale = _inputs(steps, heads, kv, dim, seed=steps + heads)
    print(f"[paired] S={steps} H={heads} Hkv={kv} D={dim}", flush=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale).cpu()
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(out, ref)
    for i in (0, 1, 63, 64, steps // 2, steps - 2, steps - 1):
        _close(out[i], orc.torch_attention(q[i].float(), k[: i + 1].float(), v[: i + 1].float(), scale))


@pytest.mark.parametrize("steps,q_offset,heads,kv", [(3000, 500, 8, 2), (2600, 64, 8, 2)])
def test_paired_split_chunked_prefill(hip_backend, steps, q_offset, heads, kv):
    """The paired split behind a cached prefix (each pair's ranges then start
    inside the prefix blocks): matches the banded oracle."""
    total = q_offset + steps
    g = torch.Generator().manual_seed(total)
    q = torch.randn(steps, heads, 256, generator=g)
    k = torch.randn(total, kv, 256, generator=g).to(torch.bfloat16)
    v = torch.randn(total, kv, 256, generator=g).to(torch.bfloat16)
    print(f"[paired chunk] S={steps} off={q_offset}", flush=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), 1 / 16, q_offset=q_offset)
    _close(out, orc.torch_prefill_banded(q, k.float(), v.float(), q_offset, 1 / 16))


# ------------------------------------------- long prompts: the pair kernel
def _pair_grid(steps, heads, kv):
    """Work-groups of the pair kernel (query blocks of 128 / min(G, 8) positions,
    two per work-group); bt_gqa_prefill runs it when this fills the device."""
    group = heads // kv
    hg = min(group, 8)
    nqb = -(-steps // (128 // hg))
    return (nqb + 1) // 2 * kv * (group // hg)


@pytest.mark.parametrize("steps,heads,kv,dim,q_offset,q_f32", [
    (4096, 16, 2, 256, 0, False),    # G = 8: the 35B-A3B attention shape
    (4100, 16, 2, 256, 0, True),     # odd block count (one work-group runs the middle block alone), f32 q
    (4096, 16, 2, 256, 1000, False),  # behind a cached prefix
    (8192, 8, 2, 128, 0, False),     # G = 4 at D = 128
    (8192, 8, 4, 256, 0, False),     # G = 2
    (8192, 8, 8, 128, 0, True),      # G = 1
    (8200, 8, 2, 256, 0, False),     # config-4 shape, ragged last block
])
def test_pair_kernel_shapes(hip_backend, steps, heads, kv, dim, q_offset, q_f32):
    """Every group size and head dim the pair kernel serves, at prompt lengths
    where its grid fills the device: every row against the oracle."""
    assert _pair_grid(steps, heads, kv) >= hip_backend.num_cus
    g = torch.Generator().manual_seed(steps + 10 * heads + kv + q_offset)
    q = torch.randn(steps, heads, dim, generator=g)
    q = q if q_f32 else q.to(torch.bfloat16)
    k = torch.randn(q_offset + steps, kv, dim, generator=g).to(torch.bfloat16)
    v = torch.randn(q_offset + steps, kv, dim, generator=g).to(torch.bfloat16)
    scale = dim**-0.5
    print(f"[pair] S={steps} H={heads} Hkv={kv} D={dim} off={q_offset} f32q={q_f32}", flush=True)
    out = hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale, q_offset=q_offset).cpu()
    if q_offset:
        ref = orc.torch_prefill_banded(q.float(), k.float(), v.float(), q_offset, scale)
    else:
        ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(out, ref)


@pytest.mark.parametrize("steps,heads,kv,dim,q_f32", [(2048, 6, 2, 256, False), (1500, 10, 2, 128, True),
                                                      (4096, 14, 2, 128, False), (3001, 12, 2, 256, True)])
def test_head_subset_group_sizes_long_prompts(hip_backend, steps, heads, kv, dim, q_f32):
    """Group sizes 3, 5, 6, 7 (subsets of 1 or 2 heads, each with its own
    split plan) on long prompts: every row against the oracle."""
    q, k, v, scale = _inputs(steps, heads, kv, dim, seed=steps + heads)
    if q_f32:
        q = q.float() + 1e-3 * torch.randn(q.shape, generator=torch.Generator().manual_seed(steps))
    print(f"[head subsets] S={steps} H={heads} Hkv={kv} D={dim} f32q={q_f32}", flush=True)
    ref = orc.torch_prefill_attention(q.float(), k.float(), v.float(), scale)
    _close(hip_backend.attention_prefill(q.cuda(), k.cuda(), v.cuda(), scale), ref)


@pytest.mark.parametrize("q_f32", [False, True])
def test_kept_images_chunk_on_the_pair_kernel(hip_backend, q_f32):
    """A chunk long enough for the pair kernel (4,096 queries at G = 8) behind a
    1,000-key prefix, through images laid out for an 8,192-slot cache (more
    blocks than the call's keys, conversion from block 15 on): equal bit for
    bit to the call that builds fresh images, and to the banded oracle."""
    cap, heads, kv, dim = 8192, 16, 2, 256
    chunks = [(0, 1000), (1000, 4096)]
    assert _pair_grid(4096, heads, kv) >= hip_backend.num_cus
    g = torch.Generator().manual_seed(8192 + q_f32)
    k = torch.randn(cap, kv, dim, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(cap, kv, dim, generator=g).to(torch.bfloat16).cuda()
    q_all = torch.randn(5096, heads, dim, generator=g)
    q_all = (q_all if q_f32 else q_all.to(torch.bfloat16)).cuda()
    scale = dim**-0.5
    images = hip_backend.prefill_images(cap, kv, dim)
    for pos0, s in chunks:
        print(f"[kept images] chunk {pos0}+{s} f32q={q_f32}", flush=True)
        q = q_all[pos0 : pos0 + s]
        kk, vv = k[: pos0 + s], v[: pos0 + s]
        got = hip_backend.attention_prefill(q, kk, vv, scale, q_offset=pos0, images=images)
        want = hip_backend.attention_prefill(q, kk, vv, scale, q_offset=pos0)
        assert torch.equal(got, want), (pos0, s)
        assert images.valid_keys == pos0 + s
    ref = orc.torch_prefill_banded(q.float().cpu(), kk.float().cpu(), vv.float().cpu(), pos0, scale)
    _close(got, ref)
