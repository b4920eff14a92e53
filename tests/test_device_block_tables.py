"""Device-resident block tables (minivllm.device_block_tables), on the CPU
and (the churn test, marked gpu) on the GPU the runtime keeps them on.

Each step's gather must equal the -1 padded tables the reference builds on the
host (minivllm/model_runner.py:176-201), through appends, preemption rewrites
(shorter and longer), sequences leaving and rejoining, row eviction and
growth in both directions.
"""
from __future__ import annotations

import random

import pytest
import torch

from minivllm.decode_graphs import pack_decode_step, step_metadata
from minivllm.device_block_tables import DeviceBlockTables


def padded(tables, M):
    return [t + [-1] * (M - len(t)) for t in tables]


def run_step(dt, ids, tables):
    rows, upd = dt.stage(ids, tables)
    B = len(ids)
    step = pack_decode_step([0] * B, [1] * B, [0] * B, rows, upd, B).to(dt.table.device)
    dt.apply(step[5 * B:])
    M = max(len(t) for t in tables)
    _, meta = step_metadata(step, B, dt, M)
    return meta.block_tables, len(upd) // 3


@pytest.mark.parametrize("device", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
@pytest.mark.parametrize("seed", range(4))
def test_random_churn_matches_host_tables(seed, device):
    rng = random.Random(seed)
    dt = DeviceBlockTables(device, rows=3, cols=2)
    live: dict[str, list[int]] = {}
    events = {"append": 0, "shrink": 0, "rewrite": 0, "evict": 0, "grow_rows": 0, "grow_cols": 0}
    next_id = 0
    for _ in range(300):
        # sequences join, leave, gain blocks, or are preempted and recomputed
        if len(live) < 6 and rng.random() < 0.3:
            live[f"s{next_id}"] = [rng.randrange(1000) for _ in range(rng.randint(1, 3))]
            next_id += 1
        if live and rng.random() < 0.1:
            live.pop(rng.choice(sorted(live)))
        for sid, t in live.items():
            r = rng.random()
            if r < 0.2:
                t.append(rng.randrange(1000))
                events["append"] += 1
            elif r < 0.25:
                n = rng.randint(1, max(1, len(t) - 1))
                events["shrink" if n < len(t) else "rewrite"] += 1
                t[:] = [rng.randrange(1000) for _ in range(n)]
            elif r < 0.28:
                t[rng.randrange(len(t))] = rng.randrange(1000)   # same length, edited in place
                events["rewrite"] += 1
        if not live:
            continue
        batch = rng.sample(sorted(live), rng.randint(1, len(live)))
        tables = [live[s] for s in batch]
        rows0, cols0, owners0 = dt.rows, dt.cols, dict(dt._owner)
        got, _ = run_step(dt, batch, tables)
        M = max(len(t) for t in tables)
        assert got.tolist() == padded(tables, M)
        assert got.is_contiguous() and got.dtype == torch.int64
        events["grow_rows"] += dt.rows > rows0
        events["grow_cols"] += dt.cols > cols0
        events["evict"] += any(o not in dt._owner.values() for o in owners0.values())
        # row 0 is the padding row and never changes
        assert dt.table[0].tolist() == [-1] * dt.cols
    for name, n in events.items():
        assert n > 0, (name, events)


def test_unchanged_tables_send_no_updates_and_appends_send_one_entry():
    dt = DeviceBlockTables("cpu", rows=4, cols=8)
    a, b = [5, 9], [7]
    _, n = run_step(dt, ["a", "b"], [a, b])
    assert n == 3
    _, n = run_step(dt, ["a", "b"], [a, b])
    assert n == 0
    a.append(11)
    got, n = run_step(dt, ["b", "a"], [b, a])
    assert n == 1
    assert got.tolist() == [[7, -1, -1], [5, 9, 11]]


def test_a_shorter_rewrite_clears_the_old_tail():
    dt = DeviceBlockTables("cpu", rows=2, cols=4)
    t = [1, 2, 3, 4]
    run_step(dt, ["x"], [t])
    t[:] = [8]                                   # preempted, recomputed into one new block
    got, n = run_step(dt, ["x", "y"], [t, [6, 6, 6]])
    assert got.tolist() == [[8, -1, -1], [6, 6, 6]]
    assert n == 1 + 3 + 3                         # new entry, three -1s, y's three entries
    assert dt.table[dt._row["x"]].tolist() == [8, -1, -1, -1]


def test_padding_rows_gather_the_all_minus_one_row():
    dt = DeviceBlockTables("cpu", rows=2, cols=4)
    rows, upd = dt.stage(["a"], [[3, 4]])
    step = pack_decode_step([1], [20], [99], rows, upd, 4)
    dt.apply(step[20:])
    out = torch.empty(4, 4, dtype=torch.int64)
    dt.gather_into(step[16:20], out)
    assert out.tolist() == [[3, 4, -1, -1]] + [[-1] * 4] * 3
    assert step[:16].tolist() == [1, 0, 0, 0, 20, 0, 0, 0, 21, 0, 0, 0, 99, -1, -1, -1]


def test_gather_wider_than_the_table_grows_columns():
    dt = DeviceBlockTables("cpu", rows=1, cols=2)
    rows, upd = dt.stage(["a"], [[3, 4]])
    dt.apply(torch.tensor(upd, dtype=torch.int64))
    out = torch.empty(1, 16, dtype=torch.int64)
    dt.gather_into(torch.tensor(rows), out)
    assert out.tolist() == [[3, 4] + [-1] * 14]
