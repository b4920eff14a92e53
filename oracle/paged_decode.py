"""numpy restatement of the paged-KV decode hot path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, to verify results. Arrays follow the reference layouts:
  q            [B, H, D]
  k_pool/v_pool[L, N, S, H, D]
  block_tables [B, M]   (-1 padding in the tail)
  context_lens [B]
bfloat16 data is carried as uint16 bit patterns (numpy has no bf16 type);
``as_float`` widens it exactly.

Functions and the reference code they restate:
  kv_append                  minivllm/attention.py:370-392 (+ skip of slot < 0)
  paged_attention_online_v1  minivllm/paged_attention_batch.py:121-278
  paged_attention_reference  minivllm/paged_attention_batch.py:7-118
  dense_gold                 experiments/gpu_day6_fused_decode_ab.py:80-97
  partition_partials /
  merge_partials             the split-context merge (no reference function;
                             the per-block merge of paged_attention_batch.py:217-254
                             applied across partitions)
  paged_prefill              the per-token prefill loop of
                             minivllm/attention.py:269-299 (query i of a chunk
                             starting at start_pos runs paged_attention_online,
                             minivllm/paged_attention_v1_reference.py, with
                             context_length = start_pos + i + 1), computed as one
                             dense causal softmax over the gathered tokens
"""
from __future__ import annotations

import math

import numpy as np

BF16_NAN = np.uint16(0x7FC0)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns (uint16) to float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even; NaN -> 0x7FC0."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    return np.where(nan, BF16_NAN, rounded).astype(np.uint16)


def as_float(x: np.ndarray, dtype=np.float64) -> np.ndarray:
    """Widens f32/f16 arrays or bf16 bit patterns (uint16) to `dtype`."""
    x = np.asarray(x)
    if x.dtype == np.uint16:
        return bf16_bits_to_f32(x).astype(dtype)
    return x.astype(dtype)


# --------------------------------------------------------------- KV append

def kv_append(k_pool: np.ndarray, v_pool: np.ndarray, layer: int, k_new: np.ndarray,
              v_new: np.ndarray, slots: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Returns copies of the pools after writing row t to slot slots[t].

    Restates the decode KV write of minivllm/attention.py:370-392
    (blk = slot // S, off = slot % S, pool[layer, blk, off] = row) with the
    build's padding rule: rows whose slot is negative or past the pool are
    skipped. Same-dtype rows are copied bit for bit; float32 rows written to a
    bfloat16 (uint16) pool are rounded to nearest even.
    """
    k_out = np.array(k_pool, copy=True)
    v_out = np.array(v_pool, copy=True)
    N, S = k_pool.shape[1], k_pool.shape[2]
    for t, slot in enumerate(np.asarray(slots).tolist()):
        if slot < 0 or slot >= N * S:
            continue
        blk, off = divmod(int(slot), S)
        for dst, src in ((k_out, np.asarray(k_new[t])), (v_out, np.asarray(v_new[t]))):
            if dst.dtype == src.dtype:
                _bits(dst)[layer, blk, off] = _bits(src)
            elif dst.dtype == np.uint16 and src.dtype == np.float32:
                dst[layer, blk, off] = f32_to_bf16_bits(src)
            else:
                raise ValueError(f"unsupported conversion {src.dtype} -> {dst.dtype}")
    return k_out, v_out


def _bits(a: np.ndarray) -> np.ndarray:
    """Unsigned-integer view of `a` (same memory), for bit-exact copies."""
    return a.view({2: np.uint16, 4: np.uint32, 8: np.uint64}[a.dtype.itemsize])


# ------------------------------------------------------- decode attention

def _scale(D: int, scale: float | None) -> float:
    return 1.0 / math.sqrt(D) if scale is None else scale


def paged_attention_online_v1(q, k_pool, v_pool, block_tables, context_lens, layer: int,
                              scale: float | None = None, acc=np.float64) -> np.ndarray:
    """Batched online softmax over block-table columns, arithmetic in `acc`.

    Restates paged_attention_batch_online_v1 (paged_attention_batch.py:121-278):
    for each column j, gather block max(table[:, j], 0) for every row, mask
    slots >= ctx - j*S to -inf (and their values to 0) before arithmetic, fold
    with O = (alpha*l*O + sum p v) / l_new, and keep the previous state for
    rows whose context ended before column j.
    """
    q = as_float(q, acc)
    B, H, D = q.shape
    S = k_pool.shape[2]
    M = np.asarray(block_tables).shape[1]
    sc = _scale(D, scale)
    ctx = np.asarray(context_lens, dtype=np.int64)
    tables = np.asarray(block_tables, dtype=np.int64)
    m = np.full((B, H), -np.inf, dtype=acc)
    l = np.zeros((B, H), dtype=acc)
    O = np.zeros((B, H, D), dtype=acc)
    offs = np.arange(S)
    with np.errstate(invalid="ignore", divide="ignore"):
        for j in range(M):
            blocks = np.maximum(tables[:, j], 0)
            n_valid = np.clip(ctx - j * S, 0, S)
            valid = offs[None, :] < n_valid[:, None]                    # [B, S]
            keys = as_float(k_pool[layer, blocks], acc)                 # [B, S, H, D]
            vals = as_float(v_pool[layer, blocks], acc)
            keys = np.where(valid[:, :, None, None], keys, 0.0)
            vals = np.where(valid[:, :, None, None], vals, 0.0)
            scores = np.einsum("bhd,bshd->bhs", q, keys)
            scores = np.where(valid[:, None, :], scores, -np.inf) * sc
            m_new = np.maximum(m, scores.max(axis=-1))
            alpha = np.exp(m - m_new)
            p = np.where(valid[:, None, :], np.exp(scores - m_new[..., None]), 0.0)
            l_new = alpha * l + p.sum(axis=-1)
            blk_O = np.einsum("bhs,bshd->bhd", p, vals)
            O_new = (alpha[..., None] * l[..., None] * O + blk_O) / l_new[..., None]
            active = n_valid > 0
            m = np.where(active[:, None], m_new, m)
            l = np.where(active[:, None], l_new, l)
            O = np.where(active[:, None, None], O_new, O)
    return O


def paged_attention_reference(q, k_pool, v_pool, block_tables, context_lens, layer: int,
                              scale: float | None = None, acc=np.float64) -> np.ndarray:
    """Per-sequence, per-block online softmax (paged_attention_batch.py:7-118)."""
    q = as_float(q, acc)
    B, H, D = q.shape
    S = k_pool.shape[2]
    sc = _scale(D, scale)
    out = np.zeros((B, H, D), dtype=acc)
    for b in range(B):
        ctx = int(context_lens[b])
        assert ctx > 0
        m = np.full(H, -np.inf, dtype=acc)
        l = np.zeros(H, dtype=acc)
        O = np.zeros((H, D), dtype=acc)
        for j in range((ctx + S - 1) // S):
            phys = int(block_tables[b][j])
            assert phys >= 0
            n = min(S, ctx - j * S)
            keys = as_float(k_pool[layer, phys, :n], acc)               # [n, H, D]
            vals = as_float(v_pool[layer, phys, :n], acc)
            scores = np.einsum("hd,thd->ht", q[b], keys) * sc
            m_new = np.maximum(m, scores.max(axis=-1))
            alpha = np.exp(m - m_new)
            p = np.exp(scores - m_new[:, None])
            l_new = alpha * l + p.sum(axis=-1)
            O = (alpha[:, None] * l[:, None] * O + np.einsum("ht,thd->hd", p, vals)) / l_new[:, None]
            m, l = m_new, l_new
        out[b] = O
    return out


def gather_tokens(k_pool, v_pool, block_tables, ctx: int, b: int, layer: int, acc=np.float64):
    """Logical K and V ([ctx, H, D]) of sequence b through its block table."""
    S = k_pool.shape[2]
    ks, vs = [], []
    for j in range((ctx + S - 1) // S):
        phys = int(block_tables[b][j])
        n = min(S, ctx - j * S)
        ks.append(as_float(k_pool[layer, phys, :n], acc))
        vs.append(as_float(v_pool[layer, phys, :n], acc))
    return np.concatenate(ks, axis=0), np.concatenate(vs, axis=0)


def dense_gold(q, k_pool, v_pool, block_tables, context_lens, layer: int,
               scale: float | None = None, acc=np.float64) -> np.ndarray:
    """Independent dense softmax over the gathered tokens (no online recurrence).

    Restates dense_gold of experiments/gpu_day6_fused_decode_ab.py:80-97.
    """
    q = as_float(q, acc)
    B, H, D = q.shape
    sc = _scale(D, scale)
    out = np.zeros((B, H, D), dtype=acc)
    for b in range(B):
        keys, vals = gather_tokens(k_pool, v_pool, block_tables, int(context_lens[b]), b, layer, acc)
        scores = np.einsum("hd,thd->ht", q[b], keys) * sc
        scores -= scores.max(axis=-1, keepdims=True)
        w = np.exp(scores)
        w /= w.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("ht,thd->hd", w, vals)
    return out


# -------------------------------------------------- split-context partials

def partition_partials(q, k_pool, v_pool, block_tables, context_lens, layer: int,
                       part_tokens: int, scale: float | None = None, acc=np.float64):
    """Per-partition (max, sum, unnormalised output) of each (b, h).

    Partition p of sequence b covers logical tokens [p*P, min(ctx, (p+1)*P)).
    Returns a list over b of (m [np, H], l [np, H], O [np, H, D]) with natural
    exponentials: l = sum_t e^(s_t - m), O = sum_t e^(s_t - m) v_t.
    """
    q = as_float(q, acc)
    B, H, D = q.shape
    sc = _scale(D, scale)
    result = []
    for b in range(B):
        ctx = int(context_lens[b])
        keys, vals = gather_tokens(k_pool, v_pool, block_tables, ctx, b, layer, acc)
        n_parts = (ctx + part_tokens - 1) // part_tokens
        ms = np.zeros((n_parts, H), acc)
        ls = np.zeros((n_parts, H), acc)
        Os = np.zeros((n_parts, H, D), acc)
        for p in range(n_parts):
            lo, hi = p * part_tokens, min(ctx, (p + 1) * part_tokens)
            s = np.einsum("hd,thd->ht", q[b], keys[lo:hi]) * sc
            mp = s.max(axis=-1)
            w = np.exp(s - mp[:, None])
            ms[p], ls[p] = mp, w.sum(axis=-1)
            Os[p] = np.einsum("ht,thd->hd", w, vals[lo:hi])
        result.append((ms, ls, Os))
    return result


def merge_partials(ms: np.ndarray, ls: np.ndarray, Os: np.ndarray) -> np.ndarray:
    """M = max_p m_p; L = sum_p l_p e^(m_p - M); O = sum_p O_p e^(m_p - M) / L."""
    M = ms.max(axis=0)
    w = np.exp(ms - M[None, :])
    L = (w * ls).sum(axis=0)
    return (w[..., None] * Os).sum(axis=0) / L[:, None]


# ------------------------------------------------------- prefill attention

def paged_prefill(q, k_pool, v_pool, block_table, start: int, layer: int,
                  scale: float | None = None, acc=np.float64) -> np.ndarray:
    """Causal attention of chunk queries q [T, H, D] through one block table.

    Query row i sits at absolute position start + i and attends logical
    tokens 0 .. start + i of the sequence (token j in physical block
    block_table[j // S], offset j % S of `layer`): the result of the
    reference's per-token prefill loop (minivllm/attention.py:269-299), which
    calls paged_attention_online with context_length = start + i + 1. Tokens
    past start + T - 1 are never read. Tokens whose table entry lies outside
    [0, N) are masked, and a row left with no visible token is zero.
    """
    q = as_float(q, acc)
    T, H, D = q.shape
    N, S = k_pool.shape[1], k_pool.shape[2]
    sc = _scale(D, scale)
    ctx = start + T
    # Token j lives in block table[j // S]; an entry outside [0, N) masks its
    # tokens (the library's contract; the reference asserts it never happens).
    pos = np.arange(ctx)
    blk = np.asarray(block_table, dtype=np.int64)[pos // S]
    valid = (blk >= 0) & (blk < N)
    safe = np.where(valid, blk, 0)
    keys = as_float(k_pool[layer, safe, pos % S], acc)                      # [ctx, H, D]
    vals = np.where(valid[:, None, None], as_float(v_pool[layer, safe, pos % S], acc), 0.0)
    # Batched over heads: [H, T, D] x [H, D, ctx] -> [H, T, ctx] scores.
    scores = np.matmul(q.transpose(1, 0, 2), keys.transpose(1, 2, 0)) * sc
    visible = (pos[None, :] <= (start + np.arange(T))[:, None]) & valid[None, :]  # [T, ctx]
    scores = np.where(visible[None], scores, -np.inf)
    rowmax = scores.max(axis=-1, keepdims=True)
    w = np.where(visible[None], np.exp(scores - np.where(np.isfinite(rowmax), rowmax, 0.0)), 0.0)
    den = w.sum(axis=-1, keepdims=True)
    w = np.divide(w, den, out=np.zeros_like(w), where=den > 0)              # no visible key: zeros
    return np.matmul(w, vals.transpose(1, 0, 2)).transpose(1, 0, 2)       # [T, H, D]
