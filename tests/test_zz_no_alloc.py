"""mgi_paged_decode_noalloc, the decode entry point that allocates nothing
(its split workspace is the library's per-device scratch array), against
mgi_paged_decode with a workspace from the caller: both through the C ABI,
on calls in a row with shrinking inputs (the later calls find the earlier
calls' partials, ticket counters and block sums in the scratch). The outputs
must be bit-identical: same kernels, same split, only the workspace address
differs (and mgi_paged_decode is itself checked against the oracle in
test_paged_decode_gpu.py).
"""
from __future__ import annotations

import math

import pytest
import torch

import _fixtures as fx
from minivllm import _native

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SCRATCH_BYTES = 32 << 20

# (B, ctx low, ctx high, pool blocks, seed): the first call splits over a
# 4096-token table, the second over a 1024-token one, the third fits one
# partition and does not split.
CALLS = [(64, 512, 4096, 20000, 0), (16, 128, 1024, 2000, 1), (5, 1, 100, 64, 2)]


def _args(w, out, split):
    B, H, D = w.q.shape
    L, N, S = w.pool.k.shape[:3]
    M = w.tables.shape[1]
    return [out.data_ptr(), _native.strides(out), w.q.data_ptr(), _native.strides(w.q),
            w.pool.k.data_ptr(), w.pool.v.data_ptr(), _native.strides(w.pool.k), _native.strides(w.pool.v),
            _native.DTYPE_CODES[w.q.dtype], w.tables.data_ptr(), _native.strides(w.tables),
            _native.ITYPE_CODES[w.tables.dtype], w.ctx.data_ptr(), w.ctx.stride(0),
            _native.ITYPE_CODES[w.ctx.dtype], B, H, D, S, N, M, L, int(w.layer), 1.0 / math.sqrt(D), split]


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("dtype,split", [(torch.bfloat16, 0), (torch.float32, 0), (torch.bfloat16, 256)],
                         ids=["bf16-auto", "f32-auto", "bf16-partitions"])
def test_noalloc_matches_the_workspace_entry_on_calls_in_a_row(dtype, split):
    lib = _native.lib()
    stream = _native.stream_handle(DEV)
    for B, lo, hi, N, seed in CALLS:
        print(f"  noalloc vs workspace entry: B={B} ctx U[{lo},{hi}] {dtype} split={split}", flush=True)
        w = fx.make_decode_workload(B, 32, 128, 16, N, lo, hi, dtype, DEV, seed=seed, poison=True)
        L, N_, S = w.pool.k.shape[:3]
        ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(B, 32, 128, S, w.tables.shape[1], split))
        assert ws_bytes <= SCRATCH_BYTES
        if (lo, hi) != (1, 100):
            assert ws_bytes > 0, "the call must split, so the scratch is used"
        ref = torch.full_like(w.q, float("nan"))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        _native.check(lib.mgi_paged_decode(*_args(w, ref, split), ws.data_ptr(), ws_bytes, stream))
        got = torch.full_like(w.q, float("nan"))
        _native.check(lib.mgi_paged_decode_noalloc(*_args(w, got, split), stream))
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(_bits(got), _bits(ref))
