"""The C ABI library: it loads, exports every declared entry point, and its
host-only functions (no device work) behave.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from breezetoken_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "breezetoken_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(bt_\w+)\s*\(", text, re.M)))


def test_header_declares_the_python_binding_set():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert _lib.LIB_PATH.is_file(), "build with `python -m breezetoken_amd.build`"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (bt_\w+)", out))
    missing = set(declared_symbols()) - exported
    assert not missing, missing
    lib = _lib.lib()
    for name in declared_symbols():
        assert getattr(lib, name) is not None


def test_library_holds_gfx950_code():
    out = subprocess.run(["strings", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    assert "gfx950" in out


def test_version_and_strerror():
    lib = _lib.lib()
    assert lib.bt_version() >= 100
    assert b"invalid" in lib.bt_strerror(_lib.BT_EINVAL)
    assert b"not served" in lib.bt_strerror(_lib.BT_ENOTSUP)
    assert b"workspace" in lib.bt_strerror(_lib.BT_ENOSPC)


def test_workspace_bytes():
    lib = _lib.lib()
    # lse (8 x 128 f32, padded to 256 B) + part (8 x 128 x 256 f32)
    assert lib.bt_decode_workspace_bytes(8, 256, 128) == 4096 + 8 * 128 * 256 * 4
    assert lib.bt_decode_workspace_bytes(8, 256, 1) == 256 + 8 * 256 * 4
    assert lib.bt_decode_workspace_bytes(0, 256, 1) == 0
    # prefill: the fp16 V^T image (one per kv head, whole 64-key blocks), one
    # int32 scale exponent per kv head and block, then the fp16 K image and its
    # exponents (each part 256-byte aligned)
    assert lib.bt_prefill_workspace_bytes(8192, 2, 256) == 2 * (2 * 8192 * 256 * 2 + 1024)
    assert lib.bt_prefill_workspace_bytes(65, 1, 128) == 2 * (128 * 128 * 2 + 256)
    assert lib.bt_prefill_workspace_bytes(0, 1, 128) == 0
    # the split-key size refuses the same malformed shapes (before any device query)
    assert lib.bt_prefill_split_workspace_bytes(0, 0, 8, 2, 256) == 0
    assert lib.bt_prefill_split_workspace_bytes(16, -1, 8, 2, 256) == 0
    assert lib.bt_prefill_split_workspace_bytes(16, 0, 6, 4, 256) == 0


@pytest.mark.parametrize(
    "kv,ctx,cus,expect",
    [(2, 65536, 256, 128), (2, 1024, 256, 32), (2, 1, 256, 1), (1, 32768, 256, 256), (2, 32768, 304, 152)],
)
def test_pick_splits(kv, ctx, cus, expect):
    assert _lib.lib().bt_decode_pick_splits(kv, ctx, cus) == expect


def _plan(lens, target):
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
    return n, list(work)[: 4 * max(n, 0)], list(base), list(cnt), tot.value


def _tokens_per_split(L, ns):
    return -(-L // ns)


def test_ragged_plan_is_proportional_and_consistent():
    lens = [2591, 8912, 338, 24869, 0, 31, 32768]
    n, work, base, cnt, tot = _plan(lens, 128)
    assert n == tot == sum(cnt) <= 128
    for b, L in enumerate(lens):
        assert 1 <= cnt[b] <= max(1, -(-L // 32))
        assert base[b] == sum(cnt[:b])
    assert cnt[6] > cnt[3] > cnt[1] > cnt[0] > cnt[2]
    entries = [tuple(work[4 * i : 4 * i + 4]) for i in range(n)]
    # every split index base_b + s appears exactly once, with its sequence's count and base
    assert sorted(bs + s for b, s, ns, bs in entries) == list(range(n))
    for b, s, ns, bs in entries:
        assert ns == cnt[b] and bs == base[b] and 0 <= s < ns
    # longest splits first
    sizes = [_tokens_per_split(lens[b], cnt[b]) for b, *_ in entries]
    assert all(x >= y for x, y in zip(sizes, sizes[1:]))


def test_ragged_plan_cap_is_the_smallest_that_fits():
    """ns_b = ceil(len_b / T) for the smallest T with sum_b ns_b <= target: one round of
    work-groups, and no smaller per-split token cap would fit (config-5 lengths)."""
    from breezetoken_amd import workloads as wl

    lens = wl.ragged_lengths()
    for target in (128, 256, 40):
        n, work, base, cnt, tot = _plan(lens, target)
        assert tot <= target
        cap = max(_tokens_per_split(L, c) for L, c in zip(lens, cnt))
        assert all(c == max(1, min(-(-L // cap), -(-L // 32))) for L, c in zip(lens, cnt))
        smaller = sum(max(1, min(-(-L // (cap - 1)), -(-L // 32))) for L in lens)
        assert smaller > target
    # more sequences than work-groups: one split each
    n, work, base, cnt, tot = _plan(lens, 8)
    assert cnt == [1] * len(lens) and tot == len(lens)


def test_ragged_plan_rejects_bad_input():
    lib = _lib.lib()
    assert lib.bt_ragged_plan(None, 1, 1, None, 0, None, None, None) == _lib.BT_EINVAL
    n, *_ = _plan([-1], 4)
    assert n == _lib.BT_EINVAL


def test_entry_points_refuse_bad_arguments_before_launching():
    """Validation happens on the host; these calls never reach the GPU."""
    lib = _lib.lib()
    fake = 1 << 20  # aligned, never dereferenced
    # null q
    rc = lib.bt_gqa_decode(None, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 8, 2, 256,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_EINVAL
    # heads not a multiple of kv_heads
    rc = lib.bt_gqa_decode(fake, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 7, 2, 256,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_EINVAL
    # unserved head_dim and group size
    rc = lib.bt_gqa_decode(fake, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 8, 2, 96,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_ENOTSUP
    rc = lib.bt_gqa_decode(fake, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 32, 2, 256,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_ENOTSUP
    # misaligned k, odd stride
    rc = lib.bt_gqa_decode(fake, 0, 0, fake + 2, fake, 512, 256, None, None, None, 16, 1, 8, 2, 256,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_EINVAL
    rc = lib.bt_gqa_decode(fake, 0, 0, fake, fake, 511, 256, None, None, None, 16, 1, 8, 2, 256,
                           16, 0.0625, fake, 1 << 30, fake, 0, 0, None)
    assert rc == _lib.BT_EINVAL
    # workspace too small
    rc = lib.bt_gqa_decode(fake, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 8, 2, 256,
                           16, 0.0625, fake, 100, fake, 0, 0, None)
    assert rc == _lib.BT_ENOSPC
    # too many splits
    rc = lib.bt_gqa_decode_split(fake, 0, 0, fake, fake, 512, 256, None, None, None, 16, 1, 8, 2,
                                 256, 5000, 0.0625, fake, fake, None)
    assert rc == _lib.BT_ENOTSUP
    # prefill: unserved head dim, bad strides or offset, missing or short workspace
    big = 1 << 30
    rc = lib.bt_gqa_prefill(fake, 1, fake, fake, 2048, 256, 512, 256, 16, 0, 8, 2, 64, 0.125, fake, big,
                            fake, 0, 2048, 256, None)
    assert rc == _lib.BT_ENOTSUP
    rc = lib.bt_gqa_prefill(fake, 1, fake, fake, 2048, 256, 512, 256, 0, 0, 8, 2, 256, 0.0625, fake, big,
                            fake, 0, 2048, 256, None)
    assert rc == _lib.BT_EINVAL
    rc = lib.bt_gqa_prefill(fake, 1, fake, fake, 2048, 256, 512, 256, 16, -1, 8, 2, 256, 0.0625, fake, big,
                            fake, 0, 2048, 256, None)
    assert rc == _lib.BT_EINVAL
    rc = lib.bt_gqa_prefill(fake, 1, fake, fake, 2048, 256, 512, 256, 16, 0, 8, 2, 256, 0.0625, None, big,
                            fake, 0, 2048, 256, None)
    assert rc == _lib.BT_EINVAL
    # the V^T workspace covers q_offset + seqlen keys
    need = lib.bt_prefill_workspace_bytes(16 + 100, 2, 256)
    rc = lib.bt_gqa_prefill(fake, 1, fake, fake, 2048, 256, 512, 256, 16, 100, 8, 2, 256, 0.0625, fake,
                            need - 1, fake, 0, 2048, 256, None)
    assert rc == _lib.BT_ENOSPC


def test_norm_rope_and_prep_refuse_bad_arguments_before_launching():
    """bt_rms_norm_rope / bt_attn_prep validation happens on the host."""
    lib = _lib.lib()
    fake = 1 << 20
    # rms_norm_rope: null x, nothing to do, odd or oversized rope_dim, cos without sin, unserved dim
    assert lib.bt_rms_norm_rope(None, 256, 4, 256, fake, 1e-6, None, None, None, 0, 1, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 256, 4, 256, None, 1e-6, None, None, None, 0, 1, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 256, 4, 256, None, 0.0, fake, fake, fake, 63, 16, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 256, 4, 256, None, 0.0, fake, fake, fake, 258, 16, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 256, 4, 256, None, 0.0, fake, None, fake, 64, 16, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 256, 4, 256, fake, -1.0, None, None, None, 0, 1, fake, 256,
                                None) == _lib.BT_EINVAL
    assert lib.bt_rms_norm_rope(fake, 96, 4, 96, fake, 1e-6, None, None, None, 0, 1, fake, 96,
                                None) == _lib.BT_ENOTSUP
    # attn_prep: null pos, one norm weight only, bad q dtype, unserved head_dim
    args = [fake, 8, 2, 256, fake, fake, 1e-6, fake, fake, fake, 64, 4096, fake, 0, fake, fake, 512,
            256, 65536, None]
    bad = list(args); bad[9] = None
    assert lib.bt_attn_prep(*bad) == _lib.BT_EINVAL
    bad = list(args); bad[5] = None
    assert lib.bt_attn_prep(*bad) == _lib.BT_EINVAL
    bad = list(args); bad[13] = 7
    assert lib.bt_attn_prep(*bad) == _lib.BT_EINVAL
    bad = list(args); bad[10] = 65
    assert lib.bt_attn_prep(*bad) == _lib.BT_EINVAL
    bad = list(args); bad[3] = 80; bad[10] = 64
    assert lib.bt_attn_prep(*bad) == _lib.BT_ENOTSUP


def test_gdn_decode_refuses_bad_arguments_before_launching():
    lib = _lib.lib()
    fake = 1 << 20
    ok = [fake, fake, fake, fake, fake, fake, 16, 16, 128, 0.088, 1e-6, fake, None]
    bad = list(ok); bad[5] = None                  # null state
    assert lib.bt_gdn_decode(*bad) == _lib.BT_EINVAL
    bad = list(ok); bad[7] = 12                    # value heads not a multiple of key heads
    assert lib.bt_gdn_decode(*bad) == _lib.BT_EINVAL
    bad = list(ok); bad[5] = fake + 4              # misaligned state
    assert lib.bt_gdn_decode(*bad) == _lib.BT_EINVAL
    bad = list(ok); bad[8] = 96                    # unserved dim
    assert lib.bt_gdn_decode(*bad) == _lib.BT_ENOTSUP


def test_gemv_refuses_bad_arguments_and_sizes_its_workspace():
    lib = _lib.lib()
    fake = 1 << 20
    assert lib.bt_gemv_workspace_bytes(0, 8) == 0
    assert lib.bt_gemv_workspace_bytes(1024, 1024) > 0          # small N: K is split
    assert lib.bt_gemv_bf16(None, fake, 1024, 1024, 1024, fake, fake, 1 << 30, None) == _lib.BT_EINVAL
    assert lib.bt_gemv_bf16(fake, fake, 1024, 1024, 1020, fake, fake, 1 << 30, None) == _lib.BT_EINVAL
    assert lib.bt_gemv_bf16(fake, fake + 8, 1024, 1024, 1024, fake, fake, 1 << 30, None) == _lib.BT_EINVAL
    assert lib.bt_gemv_bf16(fake, fake, 1024, 1024, 1024, fake, None, 0, None) == _lib.BT_ENOSPC
    assert lib.bt_gemv_bf16(fake, fake, 1 << 20, 4096, 1024, fake, fake, 1 << 30, None) == _lib.BT_ENOTSUP


@pytest.mark.parametrize(
    "steps,q_offset,heads,max_chunks",
    [
        # grid z of the split launches in the committed kernel trace of these shapes
        (128, 8192, 16, 15),
        (512, 16384, 16, 4),
        (256, 4096, 8, 14),
        (512, 0, 8, 8),  # one-block chunks
        (2048, 0, 8, 3),  # 12-block chunks: 240 work-groups in the compact grid
        (1024, 0, 8, 4),
        # the paired split (pairs of query blocks r and nqb-1-r, each cut into
        # 2 equal ranges): at most 2 ranges reach a query block
        (4096, 0, 8, 2),
        (3000, 0, 8, 2),
        # S = 8192 runs the pair kernel
        (8192, 0, 8, 0),
    ],
)
def test_prefill_split_plan_sizes(steps, q_offset, heads, max_chunks):
    """The split-key plan on a 256-CU device (the count assumed without a GPU):
    the workspace is the V^T and K images and their block scales plus f32 partials and
    LSEs of kv_heads x query blocks x max_chunks x 128 rows (max_chunks: the most
    ranges of the uniform or paired split that reach one query block).  S = 8192
    runs the pair kernel, which needs no partials."""
    from breezetoken_amd import _lib

    lib = _lib.lib()
    kv, dim = 2, 256
    vt = lib.bt_prefill_workspace_bytes(q_offset + steps, kv, dim)
    nblk = -(-(q_offset + steps) // 64)
    assert vt == 2 * (kv * nblk * 64 * dim * 2 + -(-(kv * nblk * 4) // 256) * 256)
    got = lib.bt_prefill_split_workspace_bytes(steps, q_offset, heads, kv, dim)
    if max_chunks == 0:
        assert got == vt
        return
    positions_per_group = 16 * 8 // (heads // kv)
    query_blocks = -(-steps // positions_per_group)
    rows = kv * query_blocks * max_chunks * 128
    assert got == -(-vt // 256) * 256 + rows * dim * 4 + rows * 4
