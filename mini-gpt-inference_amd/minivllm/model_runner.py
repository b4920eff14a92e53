"""Runtime state -> device tensors (minivllm/model_runner.py:10-304).

``decode_batch`` reserves one KV slot per sequence (possibly allocating a
block), builds DecodeBatchMetadata, runs one batched decode step, commits
``length += 1`` and returns ``(logits[:, -1, :], greedy next tokens)``.

The metadata of a step (input ids, positions, context lengths and slot
mapping) is packed into one int64 host buffer together with the block-table
entries that changed since the last step, and moved with a single
host-to-device copy. Block tables stay resident on the device, one row per
sequence (minivllm.device_block_tables): the copy applies the changed entries
and one gather builds the batch's -1 padded [B, M] table. The reference
rebuilds every table on the host and issues about B + 5 separate copies (one
per block-table row, minivllm/model_runner.py:176-214). With
``enable_decode_graphs`` the step replays a captured HIP graph instead
(minivllm.decode_graphs).
"""
from __future__ import annotations

import torch

from .block_manager import BlockManager
from .decode_graphs import DEFAULT_BUCKETS, DecodeGraphs, pack_decode_step, step_metadata
from .device_block_tables import DeviceBlockTables
from .kv_block_pool import KVBlockPool
from .kv_runtime import KVRuntimeContext, PrefillChunkContext, PrefillRuntimeContext
from .model import MiniGPT
from .sequence import SequenceState


class ModelRunner:
    def __init__(self, model: MiniGPT, kv_pool: KVBlockPool, block_manager: BlockManager):
        self.model = model
        self.kv_pool = kv_pool
        self.block_manager = block_manager

    @property
    def device(self) -> torch.device:
        return next(self.model.parameters()).device

    # ------------------------------------------------------------- prefill

    def prefill(self, seq: SequenceState) -> int:
        """Whole-prompt prefill; returns the greedy first token."""
        T = len(seq.prompt_tokens)
        start = seq.length
        input_ids = torch.tensor([seq.prompt_tokens], device=self.device, dtype=torch.long)
        slots = self.block_manager.reserve_slots(seq, T)
        slots, table = self._chunk_index_tensors(seq, slots, start + T)
        contexts = [PrefillRuntimeContext(seq_state=seq, kv_pool=self.kv_pool, layer_idx=i,
                                          start_pos=start, context_length=start + T, slot_mapping=slots,
                                          block_table=table)
                    for i in range(self.model.n_layer)]
        logits = self.model.prefill(input_ids, contexts)
        seq.length += T
        return int(torch.argmax(logits[:, -1], dim=-1).item())

    def prefill_chunk(self, seq: SequenceState, start_pos: int, num_tokens: int) -> torch.Tensor:
        assert start_pos == seq.prompt_pos
        assert start_pos == seq.length
        # A resumed request recomputes its cached prefix (prompt +
        # generated[:-1]); the pending last token stays for decode.
        tokens = seq.prefill_input_tokens[start_pos:start_pos + num_tokens]
        assert len(tokens) == num_tokens, "prefill chunk exceeds input prefix"
        input_ids = torch.tensor([tokens], device=self.device, dtype=torch.long)
        slots = self.block_manager.reserve_slots(seq=seq, num_tokens=num_tokens)
        slots, table = self._chunk_index_tensors(seq, slots, start_pos + num_tokens)
        contexts = [PrefillChunkContext(seq_state=seq, kv_pool=self.kv_pool, layer_idx=i,
                                        start_pos=start_pos, num_tokens=num_tokens, slot_mapping=slots,
                                        block_table=table)
                    for i in range(self.model.n_layer)]
        logits = self.model.prefill_chunk(input_ids=input_ids, contexts=contexts)
        seq.length += num_tokens
        return logits

    def _chunk_index_tensors(self, seq: SequenceState, slots: list[int], context_length: int):
        """With the KV pool on a GPU: the chunk's slots and the sequence's first
        ceil(context_length / S) table entries in one host-to-device copy,
        shared by every layer. On the CPU: (slots, None)."""
        if not self.kv_pool.k.is_cuda:
            return slots, None
        n_blocks = -(-context_length // self.kv_pool.block_size)
        buf = torch.tensor(list(slots) + list(seq.block_table[:n_blocks]), dtype=torch.long)
        buf = buf.to(self.kv_pool.k.device, non_blocking=False)
        return buf[:len(slots)], buf[len(slots):]

    # -------------------------------------------------------------- decode

    def _reserve_decode_rows(self, sequences: list[SequenceState]):
        """Reserves this step's slot per sequence; returns the metadata rows."""
        slots = [self.block_manager.reserve_append_slot(seq)[2] for seq in sequences]
        return ([seq.last_token for seq in sequences], [seq.length for seq in sequences], slots,
                [seq.block_table for seq in sequences])

    def _device_tables(self) -> DeviceBlockTables:
        tables = getattr(self, "_block_tables", None)
        if tables is None:
            cols = -(-self.model.block_size // self.kv_pool.block_size)
            tables = self._block_tables = DeviceBlockTables(self.device, cols=cols)
        return tables

    def _stage_decode_step(self, sequences, rows, B_pad: int) -> torch.Tensor:
        """Device copy of this step's packed metadata for B_pad rows, with the
        block-table updates applied to the device-resident tables."""
        tokens, positions, slots, tables = rows
        dt = self._device_tables()
        table_rows, updates = dt.stage([seq.seq_id for seq in sequences], tables)
        step = pack_decode_step(tokens, positions, slots, table_rows, updates, B_pad).to(self.device)
        dt.apply(step[5 * B_pad:])
        return step

    def _prepare_decode_batch(self, sequences: list[SequenceState]):
        B = len(sequences)
        assert B > 0
        rows = self._reserve_decode_rows(sequences)
        M = max(len(t) for t in rows[3])
        step = self._stage_decode_step(sequences, rows, B)
        return step_metadata(step, B, self._device_tables(), M)

    def enable_decode_graphs(self, max_blocks_per_seq: int | None = None,
                             buckets: tuple[int, ...] | None = None) -> None:
        """Replays decode steps from HIP graphs captured per (batch-size bucket,
        block-table width bucket), capturing each on first use.

        Needs the model on a GPU with the hip decode backend. Widths go up to
        ``max_blocks_per_seq`` (default: the model's position limit in
        blocks); steps that fit no bucket run eagerly.
        """
        M = max_blocks_per_seq or -(-self.model.block_size // self.kv_pool.block_size)
        self._decode_graphs = DecodeGraphs(self.model, self.kv_pool, M,
                                           buckets if buckets is not None else DEFAULT_BUCKETS)

    def capture_decode_graphs(self, batch_sizes) -> None:
        """Captures the buckets for these batch sizes at every table width now
        (e.g. before timing)."""
        for B in batch_sizes:
            b = self._decode_graphs.bucket(B)
            if b is not None:
                self._decode_graphs.capture(b)

    def decode_one(self, seq: SequenceState) -> int:
        """Serial one-sequence decode; returns the greedy next token."""
        block, offset, slot = self.block_manager.reserve_append_slot(seq)
        contexts = [KVRuntimeContext(seq_state=seq, block_manager=self.block_manager, kv_pool=self.kv_pool,
                                     layer_idx=i, logical_pos=seq.length, context_length=seq.length + 1,
                                     physical_block=block, block_offset=offset, physical_slot=slot)
                    for i in range(self.model.n_layer)]
        input_ids = torch.tensor([[seq.last_token]], device=self.device, dtype=torch.long)
        logits = self.model.decode(input_ids=input_ids, contexts=contexts)
        seq.length += 1
        return int(torch.argmax(logits[:, -1], dim=-1).item())

    def decode_batch(self, sequences: list[SequenceState]):
        if not sequences:
            return []
        B = len(sequences)
        rows = self._reserve_decode_rows(sequences)
        M = max(len(t) for t in rows[3])
        graphs = getattr(self, "_decode_graphs", None)
        key = graphs.target(B, M) if graphs is not None else None
        step = self._stage_decode_step(sequences, rows, key[0] if key else B)
        if key is not None:
            out = graphs.replay_staged(key, step, B, self._device_tables())
        else:  # eager (also when no graph bucket fits)
            input_ids, metadata = step_metadata(step, B, self._device_tables(), M)
            logits = self.model.decode_batch(input_ids=input_ids, metadata=metadata, kv_pool=self.kv_pool)
            last = logits[:, -1, :]
            out = (last, torch.argmax(last, dim=-1).tolist())
        for seq in sequences:
            seq.length += 1
        return out
