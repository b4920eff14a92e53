"""libminivllm_hip.so loads, exports every symbol include/minivllm_hip.h declares,
and rejects bad arguments on the host (no device work is issued by these
calls: validation returns before any HIP call)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from minivllm import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "minivllm_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mgi_\w+)\s*\(", text)))


def test_header_declares_the_binding_table():
    assert declared_symbols() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.mgi_abi_version() == 104


def test_torch_binding_loads_and_validates_on_the_host():
    """The _hip_ops extension (csrc/torch_ops.cpp) loads next to the library
    and raises the wrappers' ValueErrors before any device work: CPU tensors
    are refused first."""
    ops = _native.ops()
    for name in ("kv_append", "paged_decode", "paged_decode_append", "paged_prefill"):
        assert callable(getattr(ops, name)), name
    from minivllm import hip_paged_decode as hpd
    from minivllm.kv_block_pool import KVBlockPool

    pool = KVBlockPool(1, 4, 16, 2, 64)
    q = torch.zeros(1, 2, 64)
    with pytest.raises(ValueError, match="q must be on a GPU device"):
        hpd.paged_attention_batch_hip(q, pool, torch.zeros(1, 1, dtype=torch.long),
                                      torch.ones(1, dtype=torch.long), 0)
    with pytest.raises(ValueError, match="KV pool must be on a GPU device"):
        hpd.kv_append(pool, 0, q, q, torch.zeros(1, dtype=torch.long))
    with pytest.raises(ValueError, match="q must be on a GPU device"):
        hpd.paged_prefill_hip(q, pool, torch.zeros(1, dtype=torch.long), 0, 0)
    with pytest.raises(ValueError, match="q must be on a GPU device"):
        hpd.paged_attention_batch_append_hip(q, pool, torch.zeros(1, 1, dtype=torch.long),
                                             torch.ones(1, dtype=torch.long), 0, q, q,
                                             torch.zeros(1, dtype=torch.long))


def test_ctypes_path_when_the_extension_cannot_load(monkeypatch, tmp_path):
    """With the library present but the _hip_ops extension missing, the eager
    calls go through ctypes (minivllm._ctypes_ops), with a warning, and
    refuse CPU tensors with the extension's messages."""
    from minivllm import _ctypes_ops
    from minivllm import hip_paged_decode as hpd
    from minivllm.kv_block_pool import KVBlockPool

    monkeypatch.setattr(_native, "_ops", None)
    monkeypatch.setattr(_native, "ops_path", lambda: tmp_path / "_hip_ops_missing.so")
    with pytest.warns(RuntimeWarning, match="through ctypes"):
        assert _native.ops() is _ctypes_ops
    assert _native.ops() is _ctypes_ops  # chosen once
    pool = KVBlockPool(1, 4, 16, 2, 64)
    q = torch.zeros(1, 2, 64)
    with pytest.raises(ValueError, match="^q must be on a GPU device for the HIP backend$"):
        hpd.paged_attention_batch_hip(q, pool, torch.zeros(1, 1, dtype=torch.long),
                                      torch.ones(1, dtype=torch.long), 0)
    with pytest.raises(ValueError, match="^KV pool must be on a GPU device for the HIP backend$"):
        hpd.kv_append(pool, 0, q, q, torch.zeros(1, dtype=torch.long))
    with pytest.raises(ValueError, match="^q must be on a GPU device for the HIP backend$"):
        hpd.paged_prefill_hip(q, pool, torch.zeros(1, dtype=torch.long), 0, 0)
    with pytest.raises(ValueError, match="^q must be on a GPU device for the HIP backend$"):
        hpd.paged_attention_batch_append_hip(q, pool, torch.zeros(1, 1, dtype=torch.long),
                                             torch.ones(1, dtype=torch.long), 0, q, q,
                                             torch.zeros(1, dtype=torch.long))


def test_missing_library_is_an_error_not_a_fallback(monkeypatch, tmp_path):
    """Without libminivllm_hip.so there is no path at all: RuntimeError."""
    monkeypatch.setattr(_native, "_ops", None)
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "library_path", lambda: tmp_path / "libminivllm_hip_missing.so")
    with pytest.raises(RuntimeError, match="HIP extension not built"):
        _native.ops()


def test_split_tokens_and_workspace_sizes():
    lib = _native.lib()
    # decode microbench shape: M = 256 columns of S = 16 -> 8 partitions of 512
    # (partition mode; the automatic split's workspace is checked in
    # test_balanced_split.py)
    assert lib.mgi_paged_decode_split_tokens(64, 32, 128, 16, 256, 0) == 512
    n = 64 * 32 * 8
    acc = n * 128 * 4
    assert lib.mgi_paged_decode_workspace_bytes(64, 32, 128, 16, 256, 512) == ((acc + 255) // 256) * 256 + n * 8
    # a table that fits one partition needs no workspace
    assert lib.mgi_paged_decode_workspace_bytes(4, 8, 32, 16, 4, 0) == 0
    for S, M, req in [(16, 8192, 0), (8, 100, 0), (12, 77, 100), (16, 256, 1), (16, 256, 5000),
                      (1, 10**6, 0), (16, 3, 0)]:
        P = lib.mgi_paged_decode_split_tokens(1, 1, 128, S, M, req)
        assert P % S == 0                     # partitions start on block boundaries
        assert 0 < P <= min(M * S, 128 * S)   # at most 128 blocks per partition
        assert (M * S + P - 1) // P <= 65535
    assert lib.mgi_paged_decode_split_tokens(1, 1, 128, 16, 256, 5000) == 2048


def _prefill_ws(monkeypatch, split_keys, start, T, H, D, dtype=1):
    monkeypatch.setenv("MINIVLLM_HIP_PREFILL_SPLIT_KEYS", str(split_keys))
    return _native.lib().mgi_paged_prefill_workspace_bytes(start, T, H, D, dtype)


def test_prefill_split_workspace_sizes(monkeypatch):
    """The key split's workspace: [T*H*parts*D f32, 256-aligned | T*H*parts
    float2], parts = ceil((start + T) / keys per partition)."""
    start, T, H, D, keys = 1000, 200, 4, 128, 192
    parts = -(-(start + T) // keys)
    n = T * H * parts
    assert _prefill_ws(monkeypatch, keys, start, T, H, D) == ((n * D * 4 + 255) // 256) * 256 + n * 8
    # forced sizes round up to whole 64-key tiles
    assert _prefill_ws(monkeypatch, 130, start, T, H, D) == _prefill_ws(monkeypatch, 192, start, T, H, D)
    # no split: turned off, fp32, a partition as long as the longest query tile,
    # head dims the merge cannot take, more partitions than a grid dimension holds
    assert _prefill_ws(monkeypatch, -1, start, T, H, D) == 0
    assert _prefill_ws(monkeypatch, keys, start, T, H, D, dtype=0) == 0
    assert _prefill_ws(monkeypatch, 1280, start, T, H, D) == 0
    assert _prefill_ws(monkeypatch, keys, start, T, H, 20) == 0
    assert _prefill_ws(monkeypatch, 64, 64 * 70000, 64, H, D) == 0
    assert _prefill_ws(monkeypatch, 64, 64 * 60000, 64, H, D) > 0
    # automatic: a short chunk after a long prefix splits, a first chunk does not
    assert _prefill_ws(monkeypatch, 0, 3000, 256, 32, 128) > 0
    assert _prefill_ws(monkeypatch, 0, 0, 512, 32, 128) == 0
    assert _prefill_ws(monkeypatch, 0, 0, 1024, 16, 128) == 0
    assert _prefill_ws(monkeypatch, 0, 0, 4096, 32, 128) == 0
    assert _prefill_ws(monkeypatch, 0, 512, 256, 16, 128) > 0


def _i64(*xs):
    return (ctypes.c_int64 * len(xs))(*xs)


def test_paged_decode_rejects_bad_arguments_on_host():
    lib = _native.lib()
    st3, st5, st2 = _i64(1, 1, 1), _i64(1, 1, 1, 1, 1), _i64(1, 1)
    fake = 0x1000  # never dereferenced: every call below fails validation first

    def call(**kw):
        a = dict(out=fake, q=fake, k=fake, v=fake, dtype=_native.MGI_F32, bt=fake, bt_it=1, cl=fake,
                 cl_it=1, B=1, H=1, D=8, S=16, N=4, M=1, L=1, layer=0, scale=0.5)
        a.update(kw)
        return lib.mgi_paged_decode(a["out"], st3, a["q"], st3, a["k"], a["v"], st5, st5, a["dtype"],
                                    a["bt"], st2, a["bt_it"], a["cl"], 1, a["cl_it"], a["B"], a["H"],
                                    a["D"], a["S"], a["N"], a["M"], a["L"], a["layer"], a["scale"], 0,
                                    None, 0, None)

    cases = [
        (dict(q=None), "null tensor pointer"),
        (dict(B=0), "q dimensions must be nonzero"),
        (dict(M=0), "at least one block column"),
        (dict(layer=1), "layer_idx outside KV pool"),
        (dict(dtype=7), "unknown dtype"),
        (dict(bt_it=5), "int32 or int64"),
        (dict(scale=float("nan")), "scale must be finite"),
        (dict(D=1024), "head_dim larger than 512"),
    ]
    for kw, msg in cases:
        assert call(**kw) == _native.MGI_EINVAL or call(**kw) == _native.MGI_EUNSUPPORTED, kw
        assert msg in lib.mgi_last_error().decode(), (kw, lib.mgi_last_error())


def test_paged_decode_append_rejects_bad_arguments_on_host():
    """The fused append + decode entry checks both calls' arguments before any
    launch (the pointers are never dereferenced)."""
    lib = _native.lib()
    st3, st5, st2 = _i64(1, 1, 1), _i64(1, 1, 1, 1, 1), _i64(1, 1)
    fake = 0x1000

    def call(**kw):
        a = dict(out=fake, q=fake, k=fake, v=fake, dtype=_native.MGI_BF16, kn=fake, vn=fake,
                 new_dtype=_native.MGI_BF16, slots=fake, sl_it=1, sl_s=1, bt=fake, cl=fake, B=1, H=1, D=8,
                 S=16, N=4, M=1, L=1, layer=0)
        a.update(kw)
        return lib.mgi_paged_decode_append(
            a["out"], st3, a["q"], st3, a["k"], a["v"], st5, st5, a["dtype"], a["kn"], a["vn"], st3, st3,
            a["new_dtype"], a["slots"], a["sl_s"], a["sl_it"], a["bt"], st2, 1, a["cl"], 1, 1, a["B"], a["H"],
            a["D"], a["S"], a["N"], a["M"], a["L"], a["layer"], 0.5, 0, None, 0, None)

    cases = [
        (dict(q=None), "null tensor pointer"),
        (dict(kn=None), "null tensor pointer"),
        (dict(slots=None), "null tensor pointer"),
        (dict(B=0), "q dimensions must be nonzero"),
        (dict(layer=1), "layer_idx outside KV pool"),
        (dict(sl_it=4), "slot_mapping must be int32 or int64"),
        (dict(sl_s=-1), "strides must be non-negative"),
        (dict(new_dtype=5), "unknown dtype"),
        (dict(new_dtype=_native.MGI_F16), "only same-dtype copies and conversions to/from f32"),
    ]
    for kw, msg in cases:
        assert call(**kw) in (_native.MGI_EINVAL, _native.MGI_EUNSUPPORTED), kw
        assert msg in lib.mgi_last_error().decode(), (kw, lib.mgi_last_error())


def test_paged_decode_rejects_too_many_partitions_on_host():
    """A small split_tokens over a wide table would need more partitions than a
    grid dimension holds: refused before any launch (the pointers are never
    dereferenced)."""
    lib = _native.lib()
    B, H, D, S, N, M = 1, 1, 128, 16, 8, 70000
    pool = _i64(N * S * H * D, S * H * D, H * D, D, 1)
    st3, st2 = _i64(H * D, D, 1), _i64(M, 1)
    fake = 0x10000

    def call(split):
        return lib.mgi_paged_decode(fake, st3, fake, st3, fake, fake, pool, pool, _native.MGI_BF16,
                                    fake, st2, 1, fake, 1, 1, B, H, D, S, N, M, 1, 0, 0.1, split,
                                    fake, 1 << 40, None)

    assert call(S) == _native.MGI_EUNSUPPORTED
    assert "65535 partitions" in lib.mgi_last_error().decode()
    assert lib.mgi_paged_decode_split_tokens(B, H, D, S, M, S) == S   # 70000 partitions of S tokens


def test_paged_prefill_rejects_bad_arguments_on_host():
    lib = _native.lib()
    st3, st5 = _i64(1, 1, 1), _i64(1, 1, 1, 1, 1)
    fake = 0x1000  # never dereferenced: every call below fails validation first

    def call(**kw):
        a = dict(out=fake, q=fake, dtype=_native.MGI_BF16, bt=fake, bt_it=1, n_blocks=2, start=16, T=8,
                 H=2, D=64, S=16, N=4, L=1, layer=0, scale=0.125)
        a.update(kw)
        return lib.mgi_paged_prefill(a["out"], st3, a["q"], st3, fake, fake, st5, st5, a["dtype"],
                                     a["bt"], 1, a["bt_it"], a["n_blocks"], a["start"], a["T"], a["H"],
                                     a["D"], a["S"], a["N"], a["L"], a["layer"], a["scale"], None, 0, None)

    assert call(T=0) == _native.MGI_OK  # nothing to do: no launch
    cases = [
        (dict(T=-1), "row count must be non-negative"),
        (dict(q=None), "null tensor pointer"),
        (dict(H=0), "q dimensions must be nonzero"),
        (dict(layer=1), "layer_idx outside KV pool"),
        (dict(start=-1), "start_pos must be non-negative"),
        (dict(n_blocks=1), "block table shorter"),
        (dict(dtype=9), "unknown dtype"),
        (dict(bt_it=3), "int32 or int64"),
        (dict(scale=float("inf")), "scale must be finite"),
        (dict(D=1024), "head_dim larger than 512"),
    ]
    for kw, msg in cases:
        assert call(**kw) in (_native.MGI_EINVAL, _native.MGI_EUNSUPPORTED), kw
        assert msg in lib.mgi_last_error().decode(), (kw, lib.mgi_last_error())


def test_kv_append_rejects_bad_arguments_on_host():
    lib = _native.lib()
    st3, st5 = _i64(1, 1, 1), _i64(1, 1, 1, 1, 1)
    fake = 0x1000

    def call(T=1, layer=0, pool_dtype=_native.MGI_BF16, new_dtype=_native.MGI_BF16, k_pool=fake):
        return lib.mgi_kv_append(k_pool, fake, st5, st5, pool_dtype, fake, fake, st3, st3, new_dtype,
                                 fake, 1, _native.MGI_I64, T, 2, 8, 16, 4, 1, layer, None)

    assert call(T=0) == _native.MGI_OK  # nothing to do: no launch
    assert call(T=-1) == _native.MGI_EINVAL
    assert call(layer=3) == _native.MGI_EINVAL
    assert call(k_pool=None) == _native.MGI_EINVAL
    assert call(pool_dtype=_native.MGI_BF16, new_dtype=_native.MGI_F16) == _native.MGI_EUNSUPPORTED
    assert "f32" in lib.mgi_last_error().decode()


def test_status_mapping_to_python_exceptions():
    lib = _native.lib()
    st3, st5 = _i64(1, 1, 1), _i64(1, 1, 1, 1, 1)
    lib.mgi_kv_append(None, None, st5, st5, 0, None, None, st3, st3, 0, None, 1, 1, 1, 1, 1, 1, 1, 1,
                      0, None)
    with pytest.raises(ValueError, match="null tensor pointer"):
        _native.check(_native.MGI_EINVAL)
    with pytest.raises(RuntimeError):
        _native.check(_native.MGI_ELAUNCH)


def test_dtype_codes_cover_supported_types():
    assert set(_native.DTYPE_CODES) == {torch.float32, torch.bfloat16, torch.float16}
    assert set(_native.ITYPE_CODES) == {torch.int32, torch.int64}


def test_missing_library_raises_runtime_error(monkeypatch, tmp_path):
    """No silent fallback: without the built library every entry point raises."""
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "library_path", lambda: tmp_path / "libminivllm_hip.so")
    with pytest.raises(RuntimeError, match="not built"):
        _native.lib()


def test_noalloc_decode_refuses_splits_beyond_its_scratch_on_host():
    """mgi_paged_decode_noalloc holds 32 MiB of split workspace per device: a
    call whose split needs more (here 256-token partitions of 64 x 32 heads x
    4096-token tables, 272 MB) is refused before anything is resolved or
    launched (the pointers are never dereferenced)."""
    lib = _native.lib()
    B, H, D, S, N, M = 64, 32, 128, 16, 20000, 256
    assert lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 16) > 32 << 20
    pool = _i64(N * S * H * D, S * H * D, H * D, D, 1)
    st3, st2 = _i64(H * D, D, 1), _i64(M, 1)
    fake = 0x10000
    st = lib.mgi_paged_decode_noalloc(fake, st3, fake, st3, fake, fake, pool, pool, _native.MGI_BF16,
                                      fake, st2, 1, fake, 1, 1, B, H, D, S, N, M, 1, 0, 0.1, 16, None)
    assert st == _native.MGI_EUNSUPPORTED
    msg = lib.mgi_last_error().decode()
    assert "scratch" in msg and str(32 << 20) in msg
