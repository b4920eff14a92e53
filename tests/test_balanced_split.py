"""Index arithmetic of the decode kernel's balanced split, on the CPU.

paged_decode_fast_bal gives wave w of each head group the blocks
[w*Wb, (w+1)*Wb) of the concatenated block list of all sequences,
Wb = max(min_blocks, ceil(total / waves)); a sequence whose blocks span
several waves gets its j-th partial (j = w - floor(cb / Wb)) from wave w, in
that wave's slot 2*w (the sequence began at or before the wave's first block)
or 2*w + 1 (it began inside the wave), and paged_decode_merge combines
n_b = floor((ce - 1) / Wb) - floor(cb / Wb) + 1 partials. This test restates
that arithmetic and checks, over random context lengths, that every block of
every sequence is folded exactly once, that no two waves write the same slot,
and that the merge reads exactly the slots the waves wrote. It also checks
the library's workspace sizes for both modes.
"""
from __future__ import annotations

import math
import random

import pytest

from minivllm import _native


def pieces(ctx, S, M, waves, min_blocks):
    """{(b, j): (first block, end block, slot)} written by the waves, and n_b
    per b, following paged_decode_fast_bal / paged_decode_merge. Slots are
    per head: 2*w + (0 if the sequence began at or before the wave's first
    block else 1)."""
    nb = [min(max(c, 0), M * S) for c in ctx]
    nb = [-(-c // S) for c in nb]
    cinc, run = [], 0
    for n in nb:
        run += n
        cinc.append(run)
    total = run
    wb = max(min_blocks, -(-total // waves))
    written, slots_used = {}, set()
    for w in range(waves):
        pos, end = w * wb, min(total, (w + 1) * wb)
        if pos >= end:
            continue
        b = next(i for i, c in enumerate(cinc) if c > pos)
        while pos < end:
            cb = cinc[b - 1] if b else 0
            ce = cinc[b]
            pe = min(end, ce)
            n_b = (ce - 1) // wb - cb // wb + 1
            j = w - cb // wb
            assert (b, j) not in written
            slot = 2 * w + (0 if w * wb >= cb else 1)
            if n_b > 1:
                assert slot not in slots_used        # one writer per slot
                slots_used.add(slot)
            written[(b, j)] = (pos - cb, pe - cb, slot)
            pos = pe
            while b < len(ctx) - 1 and cinc[b] <= pos:
                b += 1
    n, merge_slots = {}, {}
    for b in range(len(ctx)):
        cb = cinc[b - 1] if b else 0
        ce = cinc[b]
        n[b] = 0 if ce <= cb else (ce - 1) // wb - cb // wb + 1
        merge_slots[b] = [2 * (cb // wb + j) + (0 if (cb // wb + j) * wb >= cb else 1) for j in range(n[b])]
    return written, n, nb, merge_slots


@pytest.mark.parametrize("seed", range(40))
def test_every_block_is_folded_once_and_indices_fit(seed):
    rng = random.Random(seed)
    S = rng.choice([1, 4, 8, 16, 32])
    M = rng.randint(1, 300)
    B = rng.choice([1, 3, 64, 65, 200, 1000])
    waves = rng.choice([1, 2, 7, 128, 512])
    min_blocks = max(1, -(-rng.choice([16, 64, 256]) // S))
    ctx = [rng.choice([0, 1, S, M * S, rng.randint(0, M * S + 5)]) for _ in range(B)]
    written, n, nb, merge_slots = pieces(ctx, S, M, waves, min_blocks)
    for b in range(B):
        got = sorted(v[:2] for (bb, _), v in written.items() if bb == b)
        js = sorted(j for (bb, j) in written if bb == b)
        assert js == list(range(n[b])), (b, js, n[b])          # the merge reads exactly these
        if n[b] > 1:                                           # ... from the slots they were written to
            assert merge_slots[b] == [written[(b, j)][2] for j in range(n[b])]
            assert all(0 <= sl < 2 * waves for sl in merge_slots[b])
        covered = [x for lo, hi in got for x in range(lo, hi)]
        assert covered == list(range(nb[b]))                   # each block once, in order


def test_workspace_sizes_of_both_modes():
    lib = _native.lib()
    B, H, D, S, M = 64, 32, 128, 16, 256

    def layout(n_parts, cinc):
        n = B * H * n_parts
        acc = n * D * 4
        ml = math.ceil(acc / 256) * 256
        if not cinc:
            return ml + n * 8
        return math.ceil((ml + n * 8) / 256) * 256 + B * 4

    # automatic split: balanced mode, two partial slots per (head, wave)
    waves = lib.mgi_paged_decode_balanced_waves(B, H, D, S, M, 0)
    assert waves > 0
    n = H * waves * 2
    ml = math.ceil(n * D * 4 / 256) * 256
    assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) == math.ceil((ml + n * 8) / 256) * 256 + B * 4
    # an explicit partition size keeps partition mode: 8 partitions of 512
    assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 512) == layout(8, False)
    # a table that fits one partition needs no workspace
    assert lib.mgi_paged_decode_workspace_bytes(4, 8, 32, 16, 4, 0) == 0
    # past the balanced mode's batch limit: partition mode
    P = lib.mgi_paged_decode_split_tokens(5000, 1, 32, 16, 256, 0)
    n = 5000 * 1 * -(-256 * 16 // P)
    assert lib.mgi_paged_decode_workspace_bytes(5000, 1, 32, 16, 256, 0) == (
        math.ceil(n * 32 * 4 / 256) * 256 + n * 8)


def test_balanced_waves_query():
    lib = _native.lib()
    waves = lib.mgi_paged_decode_balanced_waves(64, 32, 128, 16, 256, 0)
    assert waves > 0 and waves * 8 <= 3 * 256        # three per CU over 8 head groups (256 CUs, or none visible)
    assert lib.mgi_paged_decode_balanced_waves(64, 32, 128, 16, 256, 512) == 0   # explicit partitions
    assert lib.mgi_paged_decode_balanced_waves(5000, 1, 32, 16, 256, 0) == 0     # past the batch limit
    assert lib.mgi_paged_decode_balanced_waves(4, 8, 32, 16, 4, 0) == 0          # one partition: no split
