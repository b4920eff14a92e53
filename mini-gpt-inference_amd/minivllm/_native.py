"""ctypes binding of libminivllm_hip.so (the C ABI in include/minivllm_hip.h).

The library is loaded lazily on first use. A missing or unloadable library is
a hard error (RuntimeError): nothing in this package falls back to another
implementation when the HIP extension is absent.
"""
from __future__ import annotations

import ctypes
import functools
import threading

import torch

from ._build import library_path, ops_path

MGI_OK = 0
MGI_EINVAL = -1
MGI_EUNSUPPORTED = -2
MGI_ELAUNCH = -3
MGI_EWORKSPACE = -4

MGI_F32, MGI_BF16, MGI_F16 = 0, 1, 2
MGI_I32, MGI_I64 = 0, 1

DTYPE_CODES = {torch.float32: MGI_F32, torch.bfloat16: MGI_BF16, torch.float16: MGI_F16}
ITYPE_CODES = {torch.int32: MGI_I32, torch.int64: MGI_I64}

# Every symbol include/minivllm_hip.h declares.
EXPORTED_SYMBOLS = (
    "mgi_last_error",
    "mgi_abi_version",
    "mgi_kv_append",
    "mgi_paged_decode",
    "mgi_paged_decode_append",
    "mgi_paged_decode_noalloc",
    "mgi_paged_decode_workspace_bytes",
    "mgi_paged_decode_split_tokens",
    "mgi_paged_decode_balanced_waves",
    "mgi_paged_prefill",
    "mgi_paged_prefill_workspace_bytes",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_ops = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_pi64 = ctypes.POINTER(ctypes.c_int64)


def _declare(lib: ctypes.CDLL) -> None:
    lib.mgi_last_error.restype = ctypes.c_char_p
    lib.mgi_last_error.argtypes = []
    lib.mgi_abi_version.restype = _i
    lib.mgi_abi_version.argtypes = []
    lib.mgi_kv_append.restype = _i
    lib.mgi_kv_append.argtypes = [
        _p, _p, _pi64, _pi64, _i,          # pools, strides, pool dtype
        _p, _p, _pi64, _pi64, _i,          # new k/v, strides, dtype
        _p, _i64, _i,                      # slot mapping, stride, itype
        _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # T H D S N L layer
        _p,                                # stream
    ]
    lib.mgi_paged_decode.restype = _i
    lib.mgi_paged_decode.argtypes = [
        _p, _pi64,                         # out, strides
        _p, _pi64,                         # q, strides
        _p, _p, _pi64, _pi64, _i,          # pools, strides, dtype
        _p, _pi64, _i,                     # block tables, strides, itype
        _p, _i64, _i,                      # context lengths, stride, itype
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # B H D S N M L layer
        ctypes.c_float, _i64,              # scale, split tokens
        _p, ctypes.c_size_t,               # workspace, bytes
        _p,                                # stream
    ]
    lib.mgi_paged_decode_append.restype = _i
    lib.mgi_paged_decode_append.argtypes = [
        _p, _pi64,                         # out, strides
        _p, _pi64,                         # q, strides
        _p, _p, _pi64, _pi64, _i,          # pools, strides, dtype
        _p, _p, _pi64, _pi64, _i,          # new k/v, strides, dtype
        _p, _i64, _i,                      # slot mapping, stride, itype
        _p, _pi64, _i,                     # block tables, strides, itype
        _p, _i64, _i,                      # context lengths, stride, itype
        _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # B H D S N M L layer
        ctypes.c_float, _i64,              # scale, split tokens
        _p, ctypes.c_size_t,               # workspace, bytes
        _p,                                # stream
    ]
    lib.mgi_paged_decode_noalloc.restype = _i
    lib.mgi_paged_decode_noalloc.argtypes = lib.mgi_paged_decode.argtypes[:-3] + [_p]
    lib.mgi_paged_decode_workspace_bytes.restype = ctypes.c_size_t
    lib.mgi_paged_decode_workspace_bytes.argtypes = [_i64] * 6
    lib.mgi_paged_decode_split_tokens.restype = _i64
    lib.mgi_paged_decode_split_tokens.argtypes = [_i64] * 6
    lib.mgi_paged_decode_balanced_waves.restype = _i64
    lib.mgi_paged_decode_balanced_waves.argtypes = [_i64] * 6
    lib.mgi_paged_prefill.restype = _i
    lib.mgi_paged_prefill.argtypes = [
        _p, _pi64,                         # out, strides
        _p, _pi64,                         # q, strides
        _p, _p, _pi64, _pi64, _i,          # pools, strides, dtype
        _p, _i64, _i, _i64,                # block table, stride, itype, entries
        _i64, _i64,                        # start_pos, T
        _i64, _i64, _i64, _i64, _i64, _i64,  # H D S N L layer
        ctypes.c_float,                    # scale
        _p, ctypes.c_size_t,               # workspace, bytes
        _p,                                # stream
    ]
    lib.mgi_paged_prefill_workspace_bytes.restype = ctypes.c_size_t
    lib.mgi_paged_prefill_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _i]


def lib() -> ctypes.CDLL:
    """Returns the loaded library; raises RuntimeError when it is unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise RuntimeError(
                    f"HIP extension not built: {path} is missing "
                    "(run `python -c 'import __graft_entry__ as g; g.build()'` at the repo root)")
            try:
                handle = ctypes.CDLL(str(path))
            except OSError as exc:
                raise RuntimeError(f"HIP extension failed to load: {exc}") from exc
            _declare(handle)
            _lib = handle
    return _lib


def ops():
    """The eager path's binding: kv_append, paged_decode, paged_decode_append
    and paged_prefill on tensors, validated, calling the C ABI on the current
    stream.

    Normally the PyTorch extension _hip_ops (csrc/torch_ops.cpp). When the
    library loads but the extension does not (missing, or built against
    another PyTorch), the same calls go through ctypes (minivllm._ctypes_ops:
    same checks and messages, same kernels and bits, more host time per
    call), with a warning. Raises RuntimeError when the library itself is
    unavailable."""
    global _ops
    if _ops is not None:
        return _ops
    lib()  # the library first: a clear error when it is the missing piece
    with _lock:
        if _ops is None:
            try:
                _ops = _load_extension()
            except RuntimeError as exc:
                import warnings

                from . import _ctypes_ops

                warnings.warn(f"{exc}; calling libminivllm_hip.so through ctypes instead", RuntimeWarning,
                              stacklevel=2)
                _ops = _ctypes_ops
    return _ops


def _load_extension():
    """Imports the _hip_ops extension module; RuntimeError when it cannot."""
    import importlib.util

    path = ops_path()
    if not path.exists():
        raise RuntimeError(f"PyTorch binding not built: {path} is missing")
    try:
        spec = importlib.util.spec_from_file_location("minivllm._hip_ops", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
    except (ImportError, OSError) as exc:
        raise RuntimeError(f"PyTorch binding failed to load: {exc}") from exc
    return mod


@functools.lru_cache(maxsize=1024)
def _stride_array(st: tuple):
    return (ctypes.c_int64 * len(st))(*st)


def strides(t: torch.Tensor):
    """The tensor's element strides as a ctypes int64 array (cached per stride
    tuple; the C side only reads it)."""
    return _stride_array(t.stride())


def check(status: int) -> None:
    """Maps a C status to the reference's exception types."""
    if status == MGI_OK:
        return
    msg = (lib().mgi_last_error() or b"").decode(errors="replace")
    if status in (MGI_EINVAL, MGI_EUNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"libminivllm_hip error {status}: {msg}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The HIP stream of torch's current stream on `device`."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream
