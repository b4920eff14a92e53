"""ctypes binding and build recipe of the C oracle -- TEST INFRASTRUCTURE ONLY.

``build()`` compiles paged_decode_oracle.c with gcc (-O3 -fopenmp, no
-march so the library runs on any x86-64 host) into
oracle/_build/libpaged_decode_oracle.so. ``paged_decode`` runs it on numpy
arrays (f32, or bfloat16 as uint16 bit patterns) and returns float32 [B,H,D].
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "paged_decode_oracle.c"
LIB = HERE / "_build" / "libpaged_decode_oracle.so"

_lib = None


def build(verbose: bool = False) -> Path:
    LIB.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_name(LIB.name + f".tmp{os.getpid()}")
    cmd = ["gcc", "-O3", "-fopenmp", "-fPIC", "-shared", "-std=c11", str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        p, i64 = ctypes.c_void_p, ctypes.c_int64
        lib.oracle_paged_decode.restype = ctypes.c_int
        lib.oracle_paged_decode.argtypes = [p, p, p, ctypes.c_int, p, p, i64, i64, i64, i64, i64,
                                            i64, i64, i64, ctypes.c_double, ctypes.c_int, p,
                                            ctypes.c_int]
        _lib = lib
    return _lib


def paged_decode(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray,
                 context_lens: np.ndarray, layer: int, scale: float | None = None,
                 acc_double: bool = True, threads: int = 1) -> np.ndarray:
    """C restatement of paged_attention_batch_online_v1; returns float32 [B, H, D]."""
    lib = _load()
    if q.dtype == np.uint16 and k_pool.dtype == np.uint16 and v_pool.dtype == np.uint16:
        dtype = 1
    elif q.dtype == np.float32 and k_pool.dtype == np.float32 and v_pool.dtype == np.float32:
        dtype = 0
    else:
        raise ValueError("q and pools must all be float32 or all bfloat16 bits (uint16)")
    q = np.ascontiguousarray(q)
    k_pool = np.ascontiguousarray(k_pool)
    v_pool = np.ascontiguousarray(v_pool)
    tables = np.ascontiguousarray(block_tables, dtype=np.int64)
    ctx = np.ascontiguousarray(context_lens, dtype=np.int64)
    B, H, D = q.shape
    L, N, S = k_pool.shape[:3]
    M = tables.shape[1]
    out = np.empty((B, H, D), dtype=np.float32)
    sc = 1.0 / np.sqrt(D) if scale is None else scale
    rc = lib.oracle_paged_decode(q.ctypes.data, k_pool.ctypes.data, v_pool.ctypes.data, dtype,
                                 tables.ctypes.data, ctx.ctypes.data, B, H, D, S, N, M, L, layer,
                                 float(sc), int(acc_double), out.ctypes.data, int(threads))
    if rc != 0:
        raise ValueError("C oracle rejected its arguments")
    return out
