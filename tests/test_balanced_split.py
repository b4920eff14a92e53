"""Index arithmetic and ticket protocol of the decode kernel's balanced split, on the CPU.

paged_decode_fast_bal cuts the concatenated block list of all sequences
(total blocks) into P segments of Lw = max(min_blocks, ceil(total / P))
blocks, and each segment into claims numbered in list order: the segment's
own claim of A blocks (streamed by its wave) and R ticket claims of a blocks
(a = floor(Lw * (16 - t1) / 16 / R), R = min(R_max, that share // min_blocks),
A = Lw - R * a). Ticket t is claim 1 + t // P of segment t % P. A sequence
whose blocks span several claims gets its j-th partial from claim
claim_of(cb) + j, in slot 2*c (the sequence began at or before the claim's
first block) or 2*c + 1 (it began inside the claim) of its head, and
paged_decode_merge combines claim_of(ce - 1) - claim_of(cb) + 1 partials.

This test restates that arithmetic and checks, over random context lengths
and tier settings, that the own claims and the tickets name every claim
once, that no claim inside the list is empty, that every block of every
sequence is folded exactly once, that no two claims write the same slot, and
that the merge reads exactly the slots the claims wrote. A step-by-step model
of the ticket protocol (counter zeroed by wave 0 when it starts, tickets drawn
by every wave after its own claim, counters starting from stale values)
checks that every claim is streamed at least once and every wave stops. It
also checks the library's workspace sizes for both modes.
"""
from __future__ import annotations

import math
import random

import pytest

from minivllm import _native


class Claims:
    """make_claims / claim_of / claim_begin / claim_end of paged_decode.hip."""

    def __init__(self, total, P, min_blocks, t1_16ths, r_max):
        self.P, self.total = P, total
        self.Lw = max(min_blocks, -(-total // P))
        small = self.Lw * (16 - t1_16ths) // 16
        R = min(small // min_blocks, r_max)
        self.a = small // R if R > 0 else 0
        self.K = 1 + R
        self.A = self.Lw - R * self.a
        assert self.A >= 1
        self.count = P * (1 + r_max)          # claim slots per head in the workspace

    def of(self, pos):
        seg = pos // self.Lw
        off = pos - seg * self.Lw
        return seg * self.K + (0 if off < self.A else 1 + (off - self.A) // self.a)

    def begin(self, i):
        seg, k = divmod(i, self.K)
        return min(seg * self.Lw + (0 if k == 0 else self.A + (k - 1) * self.a), self.total)

    def end(self, i):
        seg, k = divmod(i, self.K)
        return min(seg * self.Lw + self.A + k * self.a, self.total)

    def slot(self, i, cb):
        return 2 * i + (0 if self.begin(i) >= cb else 1)

    def streamed(self):
        """Own claims, then the claims the tickets 0 .. P*(K-1)-1 name."""
        n_tickets = self.P * (self.K - 1)
        return [w * self.K for w in range(self.P)] + [
            (t % self.P) * self.K + 1 + t // self.P for t in range(n_tickets)]


def pieces(ctx, S, M, P, min_blocks, t1_16ths, r_max):
    """{(b, j): (first block, end block, slot)} written by the claims, and n_b
    per b, following paged_decode_fast_bal / paged_decode_merge."""
    nb = [-(-min(max(c, 0), M * S) // S) for c in ctx]
    cinc, run = [], 0
    for n in nb:
        run += n
        cinc.append(run)
    cl = Claims(run, P, min_blocks, t1_16ths, r_max)
    order = cl.streamed()
    assert sorted(order) == list(range(P * cl.K))             # every claim named once
    if run:
        last = cl.of(run - 1)
        assert all(cl.end(c) > cl.begin(c) for c in range(last + 1))   # none empty inside the list
        assert all(cl.end(c) == cl.begin(c) for c in range(last + 1, P * cl.K))
        assert [cl.of(x) for x in range(run)] == sorted(cl.of(x) for x in range(run))
    written, slots_used = {}, set()
    for c in order:
        pos, end = cl.begin(c), cl.end(c)
        if pos >= end:
            continue
        b = next(i for i, x in enumerate(cinc) if x > pos)
        while pos < end:
            cb = cinc[b - 1] if b else 0
            ce = cinc[b]
            pe = min(end, ce)
            n_b = cl.of(ce - 1) - cl.of(cb) + 1
            j = c - cl.of(cb)
            assert (b, j) not in written
            if n_b > 1:
                sl = cl.slot(c, cb)
                assert sl not in slots_used        # one writer per slot
                slots_used.add(sl)
                written[(b, j)] = (pos - cb, pe - cb, sl)
            else:
                written[(b, j)] = (pos - cb, pe - cb, None)
            pos = pe
            while b < len(ctx) - 1 and cinc[b] <= pos:
                b += 1
    n, merge_slots = {}, {}
    for b in range(len(ctx)):
        cb = cinc[b - 1] if b else 0
        ce = cinc[b]
        n[b] = 0 if ce <= cb else cl.of(ce - 1) - cl.of(cb) + 1
        merge_slots[b] = [cl.slot(cl.of(cb) + j, cb) for j in range(n[b])]
    return written, n, nb, merge_slots, cl


@pytest.mark.parametrize("seed", range(60))
def test_every_block_is_folded_once_and_indices_fit(seed):
    rng = random.Random(seed)
    S = rng.choice([1, 4, 8, 16, 32])
    M = rng.randint(1, 300)
    B = rng.choice([1, 3, 64, 65, 200, 1000])
    P = rng.choice([1, 2, 7, 96, 128, 512])
    min_blocks = max(1, -(-rng.choice([16, 64, 256]) // S))
    t1 = rng.choice([1, 8, 14, 16])
    r_max = rng.choice([0, 1, 3, 16])
    ctx = [rng.choice([0, 1, S, M * S, rng.randint(0, M * S + 5)]) for _ in range(B)]
    written, n, nb, merge_slots, cl = pieces(ctx, S, M, P, min_blocks, t1, r_max)
    for b in range(B):
        got = sorted(v[:2] for (bb, _), v in written.items() if bb == b)
        js = sorted(j for (bb, j) in written if bb == b)
        assert js == list(range(n[b])), (b, js, n[b])          # the merge reads exactly these
        if n[b] > 1:                                           # ... from the slots they were written to
            assert merge_slots[b] == [written[(b, j)][2] for j in range(n[b])]
            assert all(0 <= sl < 2 * cl.count for sl in merge_slots[b])
        covered = [x for lo, hi in got for x in range(lo, hi)]
        assert covered == list(range(nb[b]))                   # each block once, in order


def test_claims_without_second_tier_match_an_even_split():
    # no ticket claims: wave w takes [w*Wb, (w+1)*Wb), Wb = max(min_blocks, ceil(total / P))
    for total, P, mb, t1, r in [(10240, 96, 4, 14, 0), (5, 96, 4, 14, 3), (1000, 7, 1, 16, 3), (0, 3, 2, 14, 3)]:
        cl = Claims(total, P, mb, t1, r)
        wb = max(mb, -(-total // P))
        assert cl.K == 1
        for w in range(P):
            assert (cl.begin(w), cl.end(w)) == (min(w * wb, total), min((w + 1) * wb, total))


def test_claims_of_the_headline_workload():
    # B=64 x U[512, 4096] at S=16 is about 9200 blocks over 96 waves: own
    # claims of 84 blocks and three ticket claims of 4 blocks per segment
    cl = Claims(9216, 96, 4, 14, 3)
    assert (cl.Lw, cl.A, cl.a, cl.K) == (96, 84, 4, 4)


def run_ticket_protocol(P, n_claims, n2, start_value, rng, zero_first=False):
    """Random interleaving of paged_decode_fast_bal's ticket steps for one
    head group. Wave 0 zeroes the counter as its first step; every wave runs
    its own claim (a random number of steps), then draws tickets until one is
    past n2, streaming claim P + t for each ticket t < n2 (unsigned compare,
    as in the kernel). Returns how often each claim was streamed."""
    counter = [start_value]
    streamed = [0] * n_claims
    # per wave: program counter state
    state = [{"phase": "start", "work": rng.randint(0, 6)} for _ in range(P)]
    live = list(range(P))
    first = zero_first
    while live:
        w = 0 if first else rng.choice(live)
        first = False
        st = state[w]
        if st["phase"] == "start":
            if w == 0 and n2 > 0:
                counter[0] = 0
            streamed[w] += 1 if w < n_claims else 0
            st["phase"] = "own"
        elif st["phase"] == "own":
            if st["work"] > 0:
                st["work"] -= 1
            else:
                st["phase"] = "ticket" if n2 > 0 else "done"
        elif st["phase"] == "ticket":
            t = counter[0]
            counter[0] = (counter[0] + 1) & 0xFFFFFFFF
            tu = t & 0xFFFFFFFF
            if tu >= n2:
                st["phase"] = "done"
            else:
                streamed[P + tu] += 1
                st["work"] = rng.randint(0, 3)
                st["phase"] = "own"
        if st["phase"] == "done":
            live.remove(w)
    return streamed


@pytest.mark.parametrize("seed", range(200))
def test_ticket_protocol_streams_every_claim(seed):
    rng = random.Random(seed)
    P = rng.choice([1, 2, 3, 8, 24])
    n2 = rng.choice([0, 1, 2, P, 3 * P, 7 * P])
    # a stale counter: zero, small, around n2, huge, or negative as int32
    start = rng.choice([0, 1, n2 // 2, n2, n2 + 1, 0x7FFFFFFF, 0xFFFFFFFF, rng.randint(0, 1 << 32)])
    streamed = run_ticket_protocol(P, P + n2, n2, start & 0xFFFFFFFF, rng)
    assert all(x >= 1 for x in streamed), (P, n2, start, streamed)


def test_ticket_protocol_streams_each_claim_once_when_wave0_starts_first():
    rng = random.Random(5)
    for _ in range(50):
        P = rng.randint(1, 30)
        n2 = rng.randint(0, 4 * P)
        start = rng.choice([0, 3, 0xFFFFFFFF])
        # wave 0 zeroes before anyone draws: no stale tickets, no second streaming
        streamed = run_ticket_protocol(P, P + n2, n2, start, rng, zero_first=True)
        assert streamed == [1] * (P + n2)


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

    # automatic split: balanced mode, two partial slots per (head, claim):
    # one own claim per wave plus three ticket claims per wave; then the block
    # list (B int32) and one ticket counter per head group of four heads
    waves = lib.mgi_paged_decode_balanced_waves(B, H, D, S, M, 0)
    assert waves > 0
    n = H * waves * (1 + 3) * 2
    ml = math.ceil(n * D * 4 / 256) * 256
    assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) == (
        math.ceil((ml + n * 8) / 256) * 256 + B * 4 + (H // 4) * 4)
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


def wave_of_workgroup(i, ngroups, P):
    """paged_decode_fast_bal's map from workgroup id to (head group, wave)."""
    full = ngroups * 8 * (P // 8)
    if i < full:
        r, q = i % (ngroups * 8), i // (ngroups * 8)
        return r // 8, q * 8 + r % 8
    return (i - full) % ngroups, 8 * (P // 8) + (i - full) // ngroups


@pytest.mark.parametrize("ngroups,P", [(8, 96), (4, 192), (1, 768), (3, 7), (8, 13), (16, 48), (5, 1)])
def test_workgroup_map_is_a_bijection_spreading_head_groups_over_xcds(ngroups, P):
    seen = [wave_of_workgroup(i, ngroups, P) for i in range(ngroups * P)]
    assert sorted(seen) == [(g, w) for g in range(ngroups) for w in range(P)]
    # with round-robin dispatch (XCD = workgroup id mod 8), the waves of every
    # head group below the last multiple of 8 sit on all eight XCDs equally
    for g in range(ngroups):
        xcds = [i % 8 for i in range(ngroups * P) if seen[i][0] == g and seen[i][1] < 8 * (P // 8)]
        assert all(xcds.count(x) == P // 8 for x in range(8))


def test_tier_overrides_are_clamped_and_size_the_workspace(monkeypatch):
    lib = _native.lib()
    B, H, D, S, M = 64, 32, 128, 16, 256
    waves = lib.mgi_paged_decode_balanced_waves(B, H, D, S, M, 0)

    def expected(r):
        n = H * waves * (1 + r) * 2
        ml = math.ceil(n * D * 4 / 256) * 256
        return math.ceil((ml + n * 8) / 256) * 256 + B * 4 + (H // 4) * 4

    for r_env, r in (("0", 0), ("3", 3), ("100", 64), ("-5", 0)):
        monkeypatch.setenv("MINIVLLM_HIP_BAL_TIER2", r_env)
        assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) == expected(r), r_env
    monkeypatch.delenv("MINIVLLM_HIP_BAL_TIER2")
    assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) == expected(3)   # the default
    # the own-claim share only changes how segments are cut, not the workspace
    for t1 in ("0", "16", "99"):
        monkeypatch.setenv("MINIVLLM_HIP_BAL_TIER1", t1)
        assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) == expected(3)
