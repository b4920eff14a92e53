"""Parity of the HIP paged prefill attention (mgi_paged_prefill) on the MI355X.

Kernel level: every element against the prefill oracle, evaluated in double
on the same inputs. Tolerances are those of the reference's prefix test
(tests/test_prefill_prefix_sdpa_v2.py:58-63) for fp32 -- atol 2e-5, rtol 2e-4
-- 2e-2 for bf16 and 2e-3 for f16 (whose softmax weights and output round
to 11 significant bits). Pools hold NaN in every slot no chunk row may see,
tables are scattered permutations, and q is a strided view of a fused QKV
row as in the model. Shapes cover the matrix-core buckets (head_dim 32, 64,
128, 256), partial tiles, chunks after a long prefix, block sizes that are
not powers of two, and the generic path (head dims off the 16-byte grid,
non-unit head-dim strides).

Model level: the reference's prefix test recast for the "hip" prefill mode,
the golden Mini-GPT token streams with HIP prefill and decode, and a bf16
preemption runtime against the sdpa_v2 prefill.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import _e2e
import _fixtures as fx
from minivllm import hip_paged_decode as hpd
from minivllm.block_manager import BlockManager
from minivllm.kv_block_pool import KVBlockPool
from minivllm.model import MiniGPT
from minivllm.model_runner import ModelRunner
from minivllm.sequence import SequenceState
from oracle import paged_decode as ora

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
F32_TOL = dict(rtol=2e-4, atol=2e-5)
BF16_TOL = dict(rtol=2e-2, atol=2e-2)
F16_TOL = dict(rtol=2e-3, atol=2e-3)
TOL = {torch.float32: F32_TOL, torch.bfloat16: BF16_TOL, torch.float16: F16_TOL}
DTYPES = dict(argvalues=[torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])


def prefill_case(start, T, H, D, S, dtype, seed=0, L=2, layer=1, spare=3):
    """Pool with positions 0..start+T-1 of one sequence written through a
    scattered table and NaN elsewhere; q [T, H, D] a strided view."""
    total = start + T
    n_used = -(-total // S)
    N = 2 * n_used + spare
    g = torch.Generator().manual_seed(seed)
    table = torch.randperm(N, generator=g)[:n_used]
    k = torch.full((L, N, S, H, D), float("nan"))
    v = torch.full((L, N, S, H, D), float("nan"))
    pos = torch.arange(total)
    k[layer, table[pos // S], pos % S] = torch.randn((total, H, D), generator=g)
    v[layer, table[pos // S], pos % S] = torch.randn((total, H, D), generator=g)
    pool = KVBlockPool(L, N, S, H, D, device=DEV, dtype=dtype)
    pool.k.copy_(k.to(dtype))
    pool.v.copy_(v.to(dtype))
    qkv = torch.randn((T, 3, H, D), generator=g).to(dtype)
    return qkv, pool, table, layer


def run_hip(q, pool, table, start, layer):
    print(f"  hip prefill start={start} T={q.shape[0]} H={q.shape[1]} D={q.shape[2]} "
          f"S={pool.block_size} dtype={q.dtype} table={table.dtype}", flush=True)
    with torch.inference_mode():
        out = hpd.paged_prefill_hip(q, pool, table.to(DEV), start, layer)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype and tuple(out.shape) == tuple(q.shape)
    return out


def check(out, q, pool, table, start, layer):
    want = ora.paged_prefill(fx.to_numpy(q), fx.to_numpy(pool.k), fx.to_numpy(pool.v),
                             table.numpy(), start, layer)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, **TOL[q.dtype])


CASES = [
    # start, T, H, D, S
    (0, 1, 4, 128, 16),
    (0, 7, 4, 128, 16),
    (5, 7, 4, 128, 16),
    (63, 65, 4, 128, 16),
    (0, 406, 16, 128, 16),
    (1000, 200, 16, 128, 16),
    (0, 128, 8, 32, 16),
    (100, 64, 8, 64, 16),
    (30, 33, 2, 256, 16),
    (20, 11, 4, 8, 4),
    (17, 40, 3, 24, 5),
]


@pytest.mark.parametrize("dtype", **DTYPES)
@pytest.mark.parametrize("start,T,H,D,S", CASES)
def test_matches_oracle(start, T, H, D, S, dtype):
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, dtype)
    q = qkv.to(DEV)[:, 0]
    out = run_hip(q, pool, table, start, layer)
    check(out, q, pool, table, start, layer)


SPLIT_CASES = [
    # start, T, H, D, S, keys per partition
    (0, 406, 4, 128, 16, 64),
    (1000, 200, 4, 128, 16, 192),
    (511, 130, 2, 64, 16, 128),
    (100, 20, 4, 256, 16, 64),
    (64, 64, 8, 32, 16, 64),
    (77, 150, 3, 128, 5, 128),
    (300, 100, 4, 96, 16, 64),
    (250, 90, 2, 48, 16, 128),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("start,T,H,D,S,keys", SPLIT_CASES)
def test_forced_key_split_matches_oracle(monkeypatch, start, T, H, D, S, keys, dtype):
    """Keys split into partitions of `keys` keys (partials merged by the
    decode merge) against the oracle, with a NaN-filled workspace."""
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", str(keys))
    lib = hpd._native.lib()
    code = hpd._native.DTYPE_CODES[dtype]
    assert lib.mgi_paged_prefill_workspace_bytes(start, T, H, D, code) > 0
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, dtype, seed=13)
    q = qkv.to(DEV)[:, 0]
    torch.cuda.empty_cache()
    torch.empty(1 << 24, device=DEV).fill_(float("nan"))  # freed: the workspace may reuse it
    out = run_hip(q, pool, table, start, layer)
    check(out, q, pool, table, start, layer)


# Every configuration of the matrix-core prefill, selected through
# MINIVLLM_HIP_PREFILL_TR: 0 is paged_prefill_mfma; the others are
# paged_prefill_tr's (groups - 1, wavefronts per group, 16-row blocks per
# wavefront, tiles in flight; 11422 is 1422 with paired rows, each
# workgroup taking a short and a long half tile). Cases: block sizes 16 ..
# 256 (one to sixteen 16-key granules per block), head dims 48 to 128 (below
# and at the kernels' padded widths of 64 and 128), partial tiles, odd and
# even half-tile counts, and contexts past 16384 keys, where the workgroup's
# block-table window moves.
TR_CONFIGS = ["0", "412", "422", "812", "1412", "1422", "11422"]
TR_CASES = [
    # start, T, H, D, S
    (0, 406, 8, 128, 16),
    (300, 1000, 8, 128, 16),
    (1000, 200, 4, 128, 16),
    (63, 65, 4, 128, 32),
    (100, 130, 4, 64, 64),
    (5, 300, 2, 128, 256),
    (16200, 300, 2, 128, 16),
    (16300, 200, 1, 64, 16),
    # head dims below the kernel's padded width (96 and 80 in the 128-wide
    # kernels, 48 in the 64-wide ones): the chunks past D read zeros
    (100, 130, 4, 96, 16),
    (63, 65, 4, 80, 32),
    (200, 150, 2, 48, 16),
]
_TR_EXPECTED: dict = {}


def _tr_case(start, T, H, D, S, dtype):
    key = (start, T, H, D, S, dtype)
    if key not in _TR_EXPECTED:
        qkv, pool, table, layer = prefill_case(start, T, H, D, S, dtype, seed=23)
        q = qkv.to(DEV)[:, 0]
        want = ora.paged_prefill(fx.to_numpy(q), fx.to_numpy(pool.k), fx.to_numpy(pool.v),
                                 table.numpy(), start, layer)
        _TR_EXPECTED.clear()  # one case's pools at a time
        _TR_EXPECTED[key] = (q, pool, table, layer, want)
    return _TR_EXPECTED[key]


@pytest.mark.parametrize("config", TR_CONFIGS)
@pytest.mark.parametrize("start,T,H,D,S", TR_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_prefill_kernel_configs_match_oracle(monkeypatch, dtype, start, T, H, D, S, config):
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_TR", config)
    q, pool, table, layer, want = _tr_case(start, T, H, D, S, dtype)
    print(f"  config {config}", flush=True)
    got = run_hip(q, pool, table, start, layer).float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, **TOL[dtype])


def test_paired_rows_automatic_choice_is_bit_identical_to_1422(monkeypatch):
    """A 2048-row chunk after 2048 cached tokens with one head per 16 CUs:
    the launcher takes the paired-row configuration, whose 64-row half-tile
    pairs fill the chip in one round. Each row's 16-row block and key-tile
    order are those of 1422, so the outputs are bit-identical to it; sampled
    rows (the ends of half tiles included) are checked against the oracle."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus % 16 != 0:
        pytest.skip("needs a CU count divisible by 16")
    start, T, H, D, S = 2048, 2048, cus // 16, 128, 16
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, torch.bfloat16, seed=37, spare=1)
    q = qkv.to(DEV)[:, 0]
    monkeypatch.delenv("MINIVLLM_HIP_PREFILL_TR", raising=False)
    auto = run_hip(q, pool, table, start, layer)
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_TR", "11422")
    paired = run_hip(q, pool, table, start, layer)
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_TR", "1422")
    plain = run_hip(q, pool, table, start, layer)
    assert torch.equal(auto, paired)
    assert torch.equal(paired, plain)
    rows = sorted({0, 15, 16, 63, 64, 1023, 1024, 1983, 1984, T - 1} |
                  set(np.random.default_rng(5).integers(0, T, 22).tolist()))
    kp, vp = fx.to_numpy(pool.k), fx.to_numpy(pool.v)
    qn = fx.to_numpy(q)
    got = paired.float().cpu().numpy()
    for i in rows:
        want = ora.paged_prefill(qn[i:i + 1], kp, vp, table.numpy(), start + i, layer)
        np.testing.assert_allclose(got[i:i + 1], want, **BF16_TOL)


@pytest.mark.parametrize("config", TR_CONFIGS[1:])
@pytest.mark.parametrize("split_keys", ["0", "128"], ids=["whole", "split128"])
def test_prefill_kernel_configs_f16_masked_and_split(monkeypatch, config, split_keys):
    """Each paged_prefill_tr configuration in f16, with invalid table entries
    (masked keys, a row with none visible) and with its keys split over
    workgroups."""
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_TR", config)
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", split_keys)
    start, T, H, D, S = 200, 180, 4, 128, 16
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, torch.float16, seed=29)
    q = qkv.to(DEV)[:, 0]
    bad = table.clone()
    bad[3] = -1
    bad[15] = pool.num_blocks + 1
    print(f"  config {config} split {split_keys}", flush=True)
    out = run_hip(q, pool, bad, start, layer)
    check(out, q, pool, bad, start, layer)
    first = table.clone()
    first[0] = -1
    out0 = run_hip(q[:40], pool, first, 0, layer)
    check(out0, q[:40], pool, first, 0, layer)
    assert torch.count_nonzero(out0[:16]) == 0


@pytest.mark.parametrize("start,T,H", [(3000, 256, 8), (8192, 256, 32)], ids=["412_split", "1422_split"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_key_split_agrees_with_unsplit(monkeypatch, dtype, start, T, H):
    """The automatic split (a small chunk after a long prefix) against the
    same call with the split turned off: same softmax, summed in another
    order. After 8192 keys with 32 heads the partitions hold 33 key tiles
    and the split runs on 128-row workgroups; after 3000, on 64-row ones."""
    D, S = 128, 16
    lib = hpd._native.lib()
    assert lib.mgi_paged_prefill_workspace_bytes(start, T, H, D, hpd._native.DTYPE_CODES[dtype]) > 0
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, dtype, seed=17)
    q = qkv.to(DEV)[:, 0]
    split = run_hip(q, pool, table, start, layer)
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", "-1")
    assert lib.mgi_paged_prefill_workspace_bytes(start, T, H, D, hpd._native.DTYPE_CODES[dtype]) == 0
    whole = run_hip(q, pool, table, start, layer)
    check(split, q, pool, table, start, layer)
    torch.testing.assert_close(split.float(), whole.float(), **TOL[dtype])


@pytest.mark.parametrize("split_keys", ["0", "64"], ids=["auto", "split64"])
@pytest.mark.parametrize("dtype", **DTYPES)
def test_invalid_table_entries_are_masked(monkeypatch, dtype, split_keys):
    """Entries outside [0, N) mask their block's keys; a row with no visible key is zero."""
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", split_keys)
    qkv, pool, table, layer = prefill_case(40, 60, 4, 128, 16, dtype, seed=11)
    q = qkv.to(DEV)[:, 0]
    bad = table.clone()
    bad[1] = -1
    bad[4] = pool.num_blocks + 7
    out = run_hip(q, pool, bad, 40, layer)
    check(out, q, pool, bad, 40, layer)
    first = table.clone()
    first[0] = -1
    out0 = run_hip(q, pool, first, 0, layer)
    check(out0, q, pool, first, 0, layer)
    assert torch.count_nonzero(out0[:16]) == 0


def test_zero_block_size_pool_is_refused():
    """A pool whose blocks hold no tokens is refused on the host, before any launch."""
    pool = KVBlockPool(1, 4, 0, 2, 64, device=DEV, dtype=torch.bfloat16)
    q = torch.zeros((3, 2, 64), device=DEV, dtype=torch.bfloat16)
    table = torch.zeros(4, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError, match="block_size must be positive"):
        hpd.paged_prefill_hip(q, pool, table, 0, 0)
    with pytest.raises(ValueError, match="block_size must be positive"):
        hpd.kv_append(pool, 0, q, q, torch.zeros(3, dtype=torch.long, device=DEV))
    with pytest.raises(ValueError, match="block_size must be positive"):
        hpd.paged_attention_batch_hip(q, pool, table.view(3 + 1, 1)[:3], torch.ones(3, dtype=torch.long,
                                                                                   device=DEV), 0)


def test_int32_table_and_contiguous_q_match_int64_and_view():
    qkv, pool, table, layer = prefill_case(37, 50, 4, 128, 16, torch.bfloat16, seed=3)
    q = qkv.to(DEV)[:, 0]
    a = run_hip(q, pool, table, 37, layer)
    b = run_hip(q.contiguous(), pool, table.to(torch.int32), 37, layer)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("dtype,D,strided", [(torch.float16, 20, False), (torch.bfloat16, 12, False),
                                             (torch.float32, 64, True)],
                         ids=["f16_d20", "bf16_d12", "f32_dstride2"])
def test_generic_path(dtype, D, strided):
    start, T, H, S = 21, 30, 3, 16
    qkv, pool, table, layer = prefill_case(start, T, H, D, S, dtype, seed=5)
    q = qkv.to(DEV)[:, 0]
    if strided:
        q = torch.randn((T, H, 2 * D), generator=torch.Generator().manual_seed(9)).to(DEV)[..., ::2]
    out = run_hip(q, pool, table, start, layer)
    want = ora.paged_prefill(fx.to_numpy(q.float()), fx.to_numpy(pool.k.float()),
                             fx.to_numpy(pool.v.float()), table.numpy(), start, layer)
    np.testing.assert_allclose(out.float().cpu().numpy(), want, **TOL[dtype])


def test_one_row_chunk_equals_the_decode_kernel():
    qkv, pool, table, layer = prefill_case(299, 1, 8, 128, 16, torch.float32, seed=7)
    q = qkv.to(DEV)[:, 0]
    pre = run_hip(q, pool, table, 299, layer)
    with torch.inference_mode():
        dec = hpd.paged_attention_batch_hip(q, pool, table[None].to(DEV),
                                            torch.tensor([300], device=DEV), layer)
    torch.cuda.synchronize()
    torch.testing.assert_close(pre, dec, rtol=2e-6, atol=2e-6)


def test_validation_errors():
    qkv, pool, table, layer = prefill_case(16, 16, 2, 64, 16, torch.float32)
    q = qkv.to(DEV)[:, 0]
    with pytest.raises(ValueError, match="shorter"):
        hpd.paged_prefill_hip(q, pool, table[:1].to(DEV), 16, layer)
    with pytest.raises(ValueError, match="GPU"):
        hpd.paged_prefill_hip(q.cpu(), pool, table.to(DEV), 16, layer)
    with pytest.raises(ValueError, match="dtype"):
        hpd.paged_prefill_hip(q.to(torch.bfloat16), pool, table.to(DEV), 16, layer)
    with pytest.raises(ValueError, match="layer_idx"):
        hpd.paged_prefill_hip(q, pool, table.to(DEV), 16, 5)


# ------------------------------------------------------------ model level

def run_chunks(model, pieces, mode, block_size=4):
    """tests/test_prefill_prefix_sdpa_v2.py:13-38 on the GPU: chunked prefill
    of one prompt with an interleaved physical allocation and a NaN pool."""
    model.set_prefill_fastpath_mode(mode)
    n_blocks = 64
    bm = BlockManager(n_blocks, block_size)
    perm = list(range(n_blocks))[::2] + list(range(n_blocks))[1::2]
    bm.free_blocks = list(reversed(perm))
    attn = model.blocks[0].attn
    pool = KVBlockPool(model.n_layer, n_blocks, block_size, attn.n_head, attn.head_size, device=DEV)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    runner = ModelRunner(model, pool, bm)
    prompt = [1 + i * 7 % (model.vocab_size - 1) for i in range(sum(pieces))]
    seq = SequenceState(seq_id="seq", prompt_tokens=prompt, max_tokens=len(prompt) + 3)
    outputs = []
    with torch.inference_mode():
        for length in pieces:
            outputs.append(runner.prefill_chunk(seq, seq.prompt_pos, length).clone())
            seq.prompt_pos += length
    bm.check_invariants([seq])
    k, v = pool.gather_sequence(seq)
    return torch.cat(outputs, dim=1), k, v, list(seq.block_table)


@pytest.fixture(scope="module")
def prefix_model():
    torch.manual_seed(2026)
    m = MiniGPT(n_embd=32, n_head=4, vocab_size=64, block_size=192, dropout=0.0, n_layer=2)
    return m.eval().to(DEV)


@pytest.mark.parametrize("pieces", [[5, 7, 19], [1, 1, 9], [16, 1, 15], [8, 8, 8, 8],
                                    [3, 5, 4, 16, 11], [16, 16, 16, 16], [64, 32, 32]],
                         ids=lambda p: "-".join(map(str, p)))
def test_reference_prefix_cases_with_hip_prefill(prefix_model, pieces):
    print(f"  prefix case {pieces}", flush=True)
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = run_chunks(prefix_model, pieces, "reference")
    got = run_chunks(prefix_model, pieces, "hip")
    assert got[3] == ref[3]
    for a, b in zip(got[:3], ref[:3]):
        torch.testing.assert_close(a, b, **F32_TOL)
    assert torch.equal(got[0].argmax(-1), ref[0].argmax(-1))


@pytest.mark.parametrize("case", _e2e.GOLDEN_C1["cases"], ids=lambda c: f"B{c['batch']}_P{c['prompt_len']}")
def test_golden_tokens_with_hip_prefill_and_decode(case):
    torch.backends.cuda.matmul.allow_tf32 = False
    print(f"  C1 hip prefill + decode B{case['batch']}_P{case['prompt_len']}", flush=True)
    tokens, rt = _e2e.run_c1(case, "cuda", "hip", prefill_mode="hip")
    assert tokens == case["outputs"]
    assert rt.iteration == case["iterations"]


def test_bf16_runtime_hip_prefill_matches_sdpa_v2():
    """bf16 preemption runtime, HIP decode, prefill 'hip' vs 'sdpa_v2': the
    schedule is identical and token streams may differ only where the sdpa_v2
    run's top-2 logit margin at the first divergence is a near tie (< 0.1)."""
    spec = _e2e.RuntimeSpec(n_requests=12, prompt_mean=96, prompt_cap=320, output_len=12, n_embd=512,
                            n_head=4, n_layer=2, vocab=2048, max_running=12, token_budget=256, seed=3)
    prompts = _e2e.make_prompts(spec)
    model = _e2e.make_model(spec, DEV, torch.bfloat16)
    model.set_decode_attention_backend("hip")
    out, margins = {}, {}
    for mode in ("sdpa_v2", "hip"):
        model.set_prefill_fastpath_mode(mode)
        rt, seqs = _e2e.make_runtime(spec, model, prompts, DEV, torch.bfloat16)
        if mode == "sdpa_v2":
            margins = _e2e.record_margins(rt)
        stats = _e2e.run_to_completion(rt, seqs)
        out[mode] = ({s.seq_id: (len(s.prompt_tokens), s.generated_tokens) for s in seqs}, stats)
    assert out["sdpa_v2"][1]["preemptions"] > 0
    for key in ("steps", "preemptions", "repeated_kv_tokens", "output_tokens"):
        assert out["sdpa_v2"][1][key] == out["hip"][1][key], key
    diverged = _e2e.first_divergences(out["sdpa_v2"][0], out["hip"][0], margins)
    print(f"  hip prefill vs sdpa_v2, bf16: diverged {diverged}", flush=True)
    assert all(m < 0.1 for _, _, m in diverged), diverged


# ------------------------------------------------------------ any finite scale

def run_hip_scaled(q, pool, table, start, layer, scale, out=None):
    """mgi_paged_prefill through the C ABI with an explicit scale (the torch
    binding always passes 1/sqrt(D)), into `out` (any strides) if given."""
    lib = hpd._native.lib()
    T, H, D = q.shape
    L, N, S = pool.k.shape[:3]
    code = hpd._native.DTYPE_CODES[q.dtype]
    tbl = table.to(DEV)
    ws_bytes = int(lib.mgi_paged_prefill_workspace_bytes(start, T, H, D, code))
    ws = torch.full((max(ws_bytes, 4) // 4,), float("nan"), device=DEV)
    if out is None:
        out = torch.full_like(q, float("nan"))
    print(f"  hip prefill scale={scale} start={start} T={T} H={H} D={D} dtype={q.dtype} "
          f"out strides={tuple(out.stride())}", flush=True)
    hpd._native.check(lib.mgi_paged_prefill(
        out.data_ptr(), hpd._native.strides(out), q.data_ptr(), hpd._native.strides(q),
        pool.k.data_ptr(), pool.v.data_ptr(), hpd._native.strides(pool.k), hpd._native.strides(pool.v),
        code, tbl.data_ptr(), tbl.stride(0), hpd._native.ITYPE_CODES[tbl.dtype], tbl.shape[0],
        start, T, H, D, S, N, L, layer, float(scale), ws.data_ptr(), ws_bytes,
        hpd._native.stream_handle(DEV)))
    torch.cuda.synchronize()
    return out


SCALE_CASES = [
    # dtype, start, T, H, D, kernel configuration, keys per partition (0: whole)
    (torch.bfloat16, 100, 130, 4, 128, "1422", "0"),
    (torch.bfloat16, 100, 130, 4, 128, "11422", "0"),
    (torch.bfloat16, 100, 130, 4, 128, "412", "0"),
    (torch.bfloat16, 100, 130, 4, 128, "0", "0"),
    (torch.float16, 100, 130, 4, 128, "-1", "0"),
    (torch.float32, 37, 50, 4, 64, "-1", "0"),
    (torch.bfloat16, 1000, 200, 4, 128, "-1", "128"),
]


@pytest.mark.parametrize("scale", [-1 / math.sqrt(128), -0.3, 0.0, 0.3, 4.0],
                         ids=["neg_rsqrt", "neg", "zero", "pos", "large"])
@pytest.mark.parametrize("dtype,start,T,H,D,config,split", SCALE_CASES,
                         ids=["bf16_1422", "bf16_paired", "bf16_412", "bf16_mfma", "f16", "f32", "bf16_split"])
def test_any_finite_scale_matches_oracle(monkeypatch, dtype, start, T, H, D, config, split, scale):
    """softmax(scale * q.k) for negative, zero and positive scales: the kernels
    take maxima over raw scores, so a negative scale is carried by the query's
    sign; the oracle scales before its maximum."""
    if config != "-1":
        monkeypatch.setenv("MINIVLLM_HIP_PREFILL_TR", config)
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", split)
    qkv, pool, table, layer = prefill_case(start, T, H, D, 16, dtype, seed=31)
    q = qkv.to(DEV)[:, 0]
    got = run_hip_scaled(q, pool, table, start, layer, scale).float().cpu().numpy()
    want = ora.paged_prefill(fx.to_numpy(q), fx.to_numpy(pool.k), fx.to_numpy(pool.v), table.numpy(),
                             start, layer, scale=scale)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_strided_outputs(dtype):
    """The output through any strides: a head-major view keeps the matrix-core
    kernels (16-byte strides) and matches the contiguous output bit for bit;
    an odd row stride takes the generic path and matches the oracle."""
    start, T, H, D = 60, 90, 4, 128
    qkv, pool, table, layer = prefill_case(start, T, H, D, 16, dtype, seed=37)
    q = qkv.to(DEV)[:, 0]
    scale = 1 / math.sqrt(D)
    base = run_hip_scaled(q, pool, table, start, layer, scale)
    head_major = torch.full((H, T, D), float("nan"), device=DEV, dtype=dtype).permute(1, 0, 2)
    got = run_hip_scaled(q, pool, table, start, layer, scale, out=head_major)
    assert torch.equal(got.contiguous().view(torch.int16 if dtype != torch.float32 else torch.int32),
                       base.view(torch.int16 if dtype != torch.float32 else torch.int32))
    wide = torch.full((T, H, D + 3), float("nan"), device=DEV, dtype=dtype)
    odd = wide[..., :D]
    got = run_hip_scaled(q, pool, table, start, layer, scale, out=odd).float().cpu().numpy()
    want = ora.paged_prefill(fx.to_numpy(q), fx.to_numpy(pool.k), fx.to_numpy(pool.v), table.numpy(),
                             start, layer)
    np.testing.assert_allclose(got, want, **TOL[dtype])
    assert torch.isnan(wide[..., D:]).all(), "the padding columns must stay untouched"
