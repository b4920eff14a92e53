"""Captured decode steps: the whole batched decode step (embeddings, every
layer's projections, KV append and paged decode attention, MLP, final norm,
LM head and the greedy argmax) recorded once per batch-size bucket as a HIP
graph and replayed each step.

A step's metadata (input ids, positions, context lengths, slot mapping and
block tables) lives in one static int64 device buffer per graph. The runtime
fills it from one host-to-device copy of the step's scalars and table
updates (``pack_decode_step``), gathering the tables from the device-resident
``DeviceBlockTables``; ``run`` fills it from a host-built buffer instead. Graphs are keyed by
(batch bucket, table-width bucket): the width is the smallest power of two
(at least 16) or the position limit in blocks that holds the batch's
longest table, so the attention grid is sized for the contexts actually
present. Rows past the real batch are padding: slot -1 (the KV append skips
them), context length 0 (attention writes zeros), token and position 0; their
logits are discarded. All graphs of one DecodeGraphs share one memory pool
(they never run concurrently).

Capture needs the HIP decode backend: the PyTorch reference backend reads
device data on the host while filtering padding slots, which a graph cannot
record.
"""
from __future__ import annotations

import numpy as np
import torch

from .decode_batch_metadata import DecodeBatchMetadata
from .kv_block_pool import KVBlockPool

# Batch buckets captured by default. On MI355X a replayed step of the
# dim-2048, 12-layer model at context 512 takes 1.3 ms against 2.1-2.2 ms of
# eager launches up to 16 rows and 1.86 against 2.16 ms at 64 rows; at 256
# rows the step is bound by the GPU (4.27 vs 4.24 ms). In the full preemption
# runtime (decode tokens/s): eager 40.0-41.1 k, buckets up to 64 rows 42.9 k,
# up to 128 rows 43.6-43.8 k, up to 256 rows 42.4-42.5 k (padding 129-256
# rows to 256 doubles the GEMM and elementwise work of those steps; padding
# rows cost the attention nothing), so 129+ row batches run eagerly.
DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128)


def pack_decode_metadata(tokens, positions, slots, tables, B_pad: int, M: int) -> torch.Tensor:
    """Host int64 buffer [ids | positions | context_lengths | slots | tables]
    for B_pad rows (rows past len(tokens) are padding) and table width M."""
    B = len(tokens)
    host = np.full(4 * B_pad + B_pad * M, -1, dtype=np.int64)
    host[:3 * B_pad] = 0
    if B:
        host[:B] = tokens
        host[B_pad:B_pad + B] = positions
        host[2 * B_pad:2 * B_pad + B] = host[B_pad:B_pad + B] + 1
        host[3 * B_pad:3 * B_pad + B] = slots
        lens = np.fromiter((len(t) for t in tables), dtype=np.int64, count=B)
        n = int(lens.sum())
        flat = np.fromiter((x for t in tables for x in t), dtype=np.int64, count=n)
        starts = np.repeat(np.cumsum(lens) - lens, lens)
        rows = np.repeat(np.arange(B, dtype=np.int64), lens)
        host[4 * B_pad + rows * M + (np.arange(n, dtype=np.int64) - starts)] = flat
    return torch.from_numpy(host)


def metadata_views(buf: torch.Tensor, B_pad: int, M: int):
    """(input_ids [B,1], DecodeBatchMetadata) as views of a packed buffer."""
    meta = DecodeBatchMetadata(
        positions=buf[B_pad:2 * B_pad],
        context_lengths=buf[2 * B_pad:3 * B_pad],
        block_tables=buf[4 * B_pad:].view(B_pad, M),
        slot_mapping=buf[3 * B_pad:4 * B_pad],
    )
    return buf[0:B_pad].view(B_pad, 1), meta


def pack_decode_step(tokens, positions, slots, rows, updates, B_pad: int) -> torch.Tensor:
    """Host int64 buffer [ids | positions | context_lengths | slots | table rows |
    table updates] of one decode step for B_pad rows. ``rows`` and ``updates``
    come from DeviceBlockTables.stage; padding rows get token and position 0,
    context 0, slot -1 and table row 0 (all -1)."""
    B = len(tokens)
    host = np.empty(5 * B_pad + len(updates), dtype=np.int64)
    host[:3 * B_pad] = 0
    host[3 * B_pad:4 * B_pad] = -1
    host[4 * B_pad:5 * B_pad] = 0
    if B:
        host[:B] = tokens
        host[B_pad:B_pad + B] = positions
        host[2 * B_pad:2 * B_pad + B] = host[B_pad:B_pad + B] + 1
        host[3 * B_pad:3 * B_pad + B] = slots
        host[4 * B_pad:4 * B_pad + B] = rows
    host[5 * B_pad:] = updates
    return torch.from_numpy(host)


def step_metadata(buf: torch.Tensor, B: int, tables, M: int):
    """(input_ids [B,1], DecodeBatchMetadata) of a device copy of
    pack_decode_step(..., B_pad=B) after tables.apply(buf[5B:]); the block
    tables are a fresh [B, M] gather of the device-resident rows."""
    meta = DecodeBatchMetadata(
        positions=buf[B:2 * B],
        context_lengths=buf[2 * B:3 * B],
        block_tables=tables.gather(buf[4 * B:5 * B], M),
        slot_mapping=buf[3 * B:4 * B],
    )
    return buf[0:B].view(B, 1), meta


def width_buckets(max_blocks: int) -> tuple[int, ...]:
    """Table widths graphs are captured for: powers of two from 16 below
    max_blocks, then max_blocks."""
    out, w = [], 16
    while w < max_blocks:
        out.append(w)
        w *= 2
    return tuple(out) + (max_blocks,)


class _Captured:
    def __init__(self, model, pool: KVBlockPool, B_pad: int, M: int, mempool):
        dev = pool.k.device
        self.B_pad, self.M = B_pad, M
        self.buf = pack_decode_metadata([], [], [], [], B_pad, M).to(dev)
        ids, meta = metadata_views(self.buf, B_pad, M)
        with torch.inference_mode():
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                for _ in range(2):  # padding rows only: nothing is written to the pool
                    model.decode_batch(input_ids=ids, metadata=meta, kv_pool=pool)
            torch.cuda.current_stream(dev).wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, pool=mempool):
                logits = model.decode_batch(input_ids=ids, metadata=meta, kv_pool=pool)
                self.logits = logits[:, -1, :]
                self.tokens = torch.argmax(self.logits, dim=-1)

    def replay(self, host: torch.Tensor, B: int):
        self.buf.copy_(host)
        self.graph.replay()
        return self.logits[:B].clone(), self.tokens[:B].tolist()

    def replay_staged(self, step: torch.Tensor, B: int, tables):
        """Replays from a device copy of pack_decode_step(..., B_pad) whose
        table updates are applied."""
        n = 4 * self.B_pad
        self.buf[:n].copy_(step[:n])
        tables.gather_into(step[n:n + self.B_pad], self.buf[n:].view(self.B_pad, self.M))
        self.graph.replay()
        return self.logits[:B].clone(), self.tokens[:B].tolist()


class DecodeGraphs:
    """Per-bucket captured decode steps of one (model, pool) pair."""

    def __init__(self, model, pool: KVBlockPool, max_blocks_per_seq: int,
                 buckets: tuple[int, ...] = DEFAULT_BUCKETS):
        from .attention import HIP_BACKENDS

        if not pool.k.is_cuda:
            raise ValueError("decode graphs need the KV pool on a GPU")
        backends = {blk.attn.decode_attention_backend for blk in model.blocks}
        if not backends <= set(HIP_BACKENDS):
            raise ValueError("decode graphs need the hip decode backend")
        if max_blocks_per_seq < 1:
            raise ValueError("max_blocks_per_seq must be positive")
        self.model, self.pool, self.M = model, pool, int(max_blocks_per_seq)
        self.buckets = tuple(sorted(buckets))
        self.widths = width_buckets(self.M)
        self._graphs: dict[tuple[int, int], _Captured] = {}
        self._mempool = torch.cuda.graph_pool_handle()

    def bucket(self, B: int) -> int | None:
        return next((b for b in self.buckets if b >= B), None)

    def width(self, max_len: int) -> int | None:
        return next((w for w in self.widths if w >= max_len), None)

    def capture(self, B_pad: int, width: int | None = None) -> None:
        """Captures the graph of batch bucket B_pad at one table width (default:
        every width bucket)."""
        for w in (self.widths if width is None else (width,)):
            if (B_pad, w) not in self._graphs:
                self._graphs[(B_pad, w)] = _Captured(self.model, self.pool, B_pad, w, self._mempool)

    def target(self, B: int, max_len: int) -> tuple[int, int] | None:
        """(batch bucket, width bucket) of a step, or None if none fits."""
        B_pad, W = self.bucket(B), self.width(max_len)
        return None if B_pad is None or W is None else (B_pad, W)

    def replay_staged(self, key: tuple[int, int], step: torch.Tensor, B: int, tables):
        """One decode step of B rows from a device copy of pack_decode_step
        (padded to key[0] rows, table updates applied)."""
        self.capture(*key)
        return self._graphs[key].replay_staged(step, B, tables)

    def run(self, tokens, positions, slots, tables):
        """One decode step for len(tokens) rows; None if no bucket fits."""
        B = len(tokens)
        B_pad = self.bucket(B)
        W = self.width(max(len(t) for t in tables))
        if B_pad is None or W is None:
            return None
        self.capture(B_pad, W)
        host = pack_decode_metadata(tokens, positions, slots, tables, B_pad, W)
        return self._graphs[(B_pad, W)].replay(host, B)
