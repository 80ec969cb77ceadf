"""Host-side checks of the paired split-key schedule of the prefill kernel.

The device code (gqa_prefill8.hip: the work-group's segments in
gqa_prefill8_kernel, pair_chunks for the combine) cuts pair r = (query blocks
nqb-1-r and r) into `parts` equal ranges of its key blocks.  This test restates
that index arithmetic and checks what the schedule must guarantee: every (query
block, key block) is covered exactly once, every chunk index of a query block
is written exactly once and lies below its chunk count, and each work-group has
at most two segments.  The restated chunk counts are tied to the library's own
plan through the partial-buffer size it reports.
"""

from __future__ import annotations

import itertools

import pytest

ROWS, KB = 128, 64


def _blocks(steps, q_offset, group):
    pos = 16 * (8 // group)
    nqb = -(-steps // pos)
    return nqb, (lambda qb: (q_offset + min(steps, (qb + 1) * pos) + KB - 1) // KB)


def _segments(nqb, n_blocks, parts):
    """(work-group, [(query block, first, end, chunk, chunks)]) of the paired split."""
    out = []
    for x in range((nqb + 1) // 2 * parts):
        r, k = divmod(x, parts)
        qhi, qlo = nqb - 1 - r, r
        nhi = n_blocks(qhi)
        nlo = n_blocks(qlo) if qlo != qhi else 0
        size = -(-(nhi + nlo) // parts)
        r0, r1 = k * size, min(nhi + nlo, k * size + size)
        segs = []
        if r0 < r1:
            if r0 < nhi:
                segs.append((qhi, r0, min(nhi, r1), k, -(-nhi // size)))
            if r1 > nhi:
                kf = nhi // size
                segs.append((qlo, max(0, r0 - nhi), r1 - nhi, k - kf, (nhi + nlo - 1) // size - kf + 1))
        out.append((x, segs))
    return out


@pytest.mark.parametrize(
    "steps,q_offset,group,parts",
    list(itertools.product([1, 7, 100, 512, 1000, 2048, 3000, 4096], [0, 17, 4096], [1, 2, 4, 8], [1, 2, 3, 4, 8])),
)
def test_paired_ranges_cover_every_block_once(steps, q_offset, group, parts):
    nqb, n_blocks = _blocks(steps, q_offset, group)
    covered, chunks = {}, {}
    for _, segs in _segments(nqb, n_blocks, parts):
        assert len(segs) <= 2
        for qb, a, b, c, n in segs:
            assert 0 <= c < n and (qb, c) not in chunks
            chunks[(qb, c)] = n
            for blk in range(a, b):
                assert (qb, blk) not in covered
                covered[(qb, blk)] = True
    for qb in range(nqb):
        assert all((qb, blk) in covered for blk in range(n_blocks(qb)))
        counts = {n for (q, _), n in chunks.items() if q == qb}
        assert len(counts) == 1
        assert all((qb, c) in chunks for c in range(counts.pop()))


@pytest.mark.parametrize("steps,heads,kv,dim", [(3000, 8, 2, 256), (4096, 8, 2, 256), (6000, 4, 2, 128)])
def test_library_plan_matches_paired_chunk_counts(steps, heads, kv, dim):
    """The library's plan (256 CUs without a GPU) for these shapes is the paired
    split with parts = 256 / (pairs x kv heads); its partial buffer holds
    kv x query blocks x (most chunks of any query block) x 128 rows."""
    from breezetoken_amd import _lib

    lib = _lib.lib()
    group = heads // kv
    nqb, n_blocks = _blocks(steps, 0, group)
    parts = max(1, min(256 // ((nqb + 1) // 2 * kv), 64))
    most = max(n for _, segs in _segments(nqb, n_blocks, parts) for *_, n in segs)
    rows = kv * nqb * most * ROWS
    assert lib.bt_prefill_partials_bytes(steps, 0, heads, kv, dim) == rows * (dim * 4 + 4)
