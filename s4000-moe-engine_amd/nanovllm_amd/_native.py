"""ctypes binding of libkvc.so, the C ABI declared in include/kvc.h.

The library is the only compute path: there is no torch or CPU fallback.  If
it is missing, every entry point raises RuntimeError naming the build command.
Status codes map to the exception types the engine's own Python raises for the
same conditions (ValueError for unsupported shapes, AssertionError for layout
preconditions, RuntimeError for backend failures).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

PKG_ROOT = pathlib.Path(__file__).resolve().parent.parent
LIB_PATH = pathlib.Path(os.environ.get("KVC_LIBRARY", PKG_ROOT / "lib" / "libkvc.so"))

KVC_KV_BF16 = 0
KVC_KV_INT8_TOKHEAD = 1
KVC_KV_INT8_CHAN = 2
# include/kvc.h KVC_STATIC_SCRATCH_BYTES
STATIC_SCRATCH_BYTES = 64 << 20

_ERRORS = {
    -1: ValueError,
    -2: AssertionError,
    -3: RuntimeError,
    -4: ValueError,
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes), mirroring include/kvc.h.
SIGNATURES = {
    "kvc_last_error": (ctypes.c_char_p, []),
    "kvc_abi_version": (_INT, []),
    "kvc_store_kv": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64, _P, _INT,
                            _I64, _I64, _I64, _INT, _P]),
    "kvc_store_int8_tokhead": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64,
                                      _P, _INT, _I64, _I64, _I64, _P]),
    "kvc_store_int8_chan": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P, _P,
                                   _I64, _P, _P, _I64, _P, _INT, _I64, _I64, _I64, _P]),
    "kvc_kv_calib_observe": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P,
                                    _P]),
    "kvc_kv_calib_freeze": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "kvc_paged_decode_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "kvc_paged_decode_layout": (_INT, [_I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "kvc_paged_decode": (_INT, [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _INT,
                                _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _P, _I64,
                                _I64, _F32, _P, _I64, _I64, _P, _SZ, _P]),
    "kvc_paged_decode_append": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _INT,
                                       _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P,
                                       _I64, _I64, _F32, _P, _I64, _I64, _P, _SZ, _P]),
    "kvc_paged_decode_append_int8": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                            _P, _INT, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                            _P, _I64, _I64, _P, _I64, _I64, _F32, _P, _I64,
                                            _I64, _P, _SZ, _P]),
    "kvc_paged_decode_append_int8_chan": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64,
                                                 _I64, _P, _INT, _P, _P, _P, _P, _P, _P, _P,
                                                 _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P,
                                                 _I64, _I64, _P, _I64, _I64, _F32, _P, _I64,
                                                 _I64, _P, _SZ, _P]),
    "kvc_paged_decode_append_static": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                              _P, _INT, _P, _P, _I64, _I64, _I64, _I64, _P,
                                              _I64, _I64, _P, _I64, _I64, _F32, _P, _I64, _I64,
                                              _P]),
    "kvc_decode_stamps": (_INT, [_P, _INT, _P, _P]),
    "kvc_varlen_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64]),
    "kvc_varlen_prefill_units": (_I64, [_P, _P, _I64, _I64, _I64, _I64]),
    "kvc_varlen_attention": (_INT, [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64,
                                    _I64, _INT, _P, _P, _P, _P, _P, _P, _I64, _P, _I64,
                                    _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64,
                                    _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _I64, _I64, _P,
                                    _SZ, _P]),
    "kvc_varlen_attention_append": (_INT, [_P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P,
                                           _I64, _I64, _P, _INT, _P, _P, _I64, _I64, _I64,
                                           _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64,
                                           _I64, _I64, _I64, _F32, _P, _I64, _I64, _P, _SZ,
                                           _P]),
    "kvc_varlen_decode_cus": (_INT, [_I64, _I64, _I64, _I64, _INT, _I64, _I64]),
    "kvc_dequant_chan": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]),
    "kvc_dequant_tokhead": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "kvc_gather_kv": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _INT, _P, _P, _P, _P, _P, _P,
                             _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _P]),
    "kvc_block_gather": (_INT, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _I64, _P]),
    "kvc_block_scatter": (_INT, [_P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "kvc_block_copy": (_INT, [_P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "kvc_block_d2h": (_INT, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "kvc_block_h2d": (_INT, [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "kvc_qk_norm_rope_store": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                                      _I64, _I64, _I64, _I64, _P, _INT, _P, _P, _F32,
                                      _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _P,
                                      _I64, _P, _INT, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_fns: dict = {}  # name -> bound ctypes function (looked up once)


def load() -> ctypes.CDLL:
    """Load libkvc.so once; RuntimeError (never a fallback) when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.is_file():
                raise RuntimeError(
                    f"libkvc.so not found at {LIB_PATH}; build it with "
                    f"`make -C {PKG_ROOT / 'csrc'}` (hipcc, gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
                _fns[name] = fn
            _lib = lib
    return _lib


def call(name: str, *args) -> int:
    """Invoke entry point `name`; raise the mapped exception on a nonzero status."""
    fn = _fns.get(name)
    if fn is None:
        fn = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        msg = _lib.kvc_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, RuntimeError)(msg or f"{name} failed with status {rc}")
    return rc


def query(name: str, *args):
    """Invoke a size/count query (no status code)."""
    fn = _fns.get(name)
    if fn is None:
        fn = getattr(load(), name)
    return fn(*args)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on t's device (all work is stream-ordered)."""
    if not t.is_cuda:
        raise RuntimeError(f"the HIP KV path needs device tensors, got {t.device}")
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"the HIP KV path needs device tensors, got {t.device}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    """Split-K scratch from torch's caching allocator (graph-capture safe)."""
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def exported_symbols() -> list[str]:
    return [name for name in SIGNATURES]
