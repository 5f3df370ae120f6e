"""ctypes binding of libtileinfer_amd.so (declarations: include/tileinfer_amd.h).

The library is loaded lazily on first use, after torch (torch's bundled HIP runtime has the same
soname as ROCm's, so the kernels and torch share one runtime and torch's stream handles are valid
here). There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported before the library: shared HIP runtime)

LIB_PATH = Path(__file__).resolve().parent / "libtileinfer_amd.so"

# Codes mirrored from include/tileinfer_amd.h.
TI_OK = 0
TI_EINVAL = 1
TI_ELAUNCH = 2
TI_EUNSUPPORTED = 3
TI_DTYPE_BF16 = 0
TI_DTYPE_F16 = 1
TI_DECODE_AUTO = 0
TI_DECODE_MFMA = 1
TI_DECODE_SCALAR = 2
TI_DECODE_REUSE_KV = 0x10
TI_DECODE_STREAM_KV = 0x20
ABI_VERSION = 7

# Every symbol declared in include/tileinfer_amd.h, with its ctypes signature.
_c_i32, _c_i64, _c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
_I32P, _I64P = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)
SIGNATURES = {
    "ti_kv_append": (ctypes.c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp,
                                    _c_i64, _c_i64, _c_i64, _c_i32, _c_vp]),
    "ti_gqa_decode_plan": (ctypes.c_int, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                          _I32P, _I32P, _I64P]),
    "ti_gqa_decode_paged": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64,
                                           _c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32, _c_i32,
                                           _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                           _c_vp]),
    "ti_copy_blocks": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_i64, _c_vp]),
    "ti_gqa_prefill_paged": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64,
                                            _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64,
                                            _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                            _c_i64, _c_i32, _c_i32, _c_i32, _c_vp]),
    "ti_gqa_prefill_paged_gated": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                                  _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                                  _c_vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                                  _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32,
                                                  _c_i32, _c_vp, _c_i64, _c_i64, _c_vp]),
    "ti_gqa_prefill_paged_partial": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                                    _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                                    _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                                    _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
                                                    _c_i32, _c_i32, _c_i32, _c_vp]),
    "ti_gqa_prefill_key_splits": (ctypes.c_int32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "ti_gqa_decode_paged_prefixed": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                                    _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_i32,
                                                    _c_i32, _c_i32, _c_i32, _c_i32, _c_i64,
                                                    _c_i32, _c_i32, _c_i32, _c_i32, _c_vp,
                                                    _c_i64, _c_i64, _c_vp, _c_vp, _c_i32,
                                                    _c_i32, _c_vp]),
    "ti_gqa_prefill_workspace_bytes": (ctypes.c_int, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                                      _c_i32, _c_i32, _I64P]),
    "ti_paged_metadata": (ctypes.c_int, [_c_vp, _c_i64, _c_i32, _c_i32, _c_vp, _c_vp, _c_vp,
                                         _c_vp, _c_vp, _c_vp, _c_vp, _c_i32, _c_i32, _c_vp, _c_vp,
                                         _c_vp, _c_i64, _c_i32, _c_i32, _c_vp]),
    "ti_qknorm_rope": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp,
                                      _c_vp, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                      ctypes.c_float, _c_i32, _c_vp]),
    "ti_qknorm_rope_append": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp,
                                             _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64,
                                             _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp,
                                             _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                             ctypes.c_float, _c_i32, _c_vp]),
    "ti_sigmoid_mul": (ctypes.c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_vp]),
    "ti_gqa_decode_paged_append": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                                  _c_i64, _c_vp, _c_vp, _c_vp, _c_i64, _c_i32,
                                                  _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32,
                                                  _c_i32, _c_i32, _c_i32, _c_vp, _c_vp, _c_i64,
                                                  _c_i64, _c_vp, _c_i64, _c_vp]),
    "ti_gqa_decode_paged_gated": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64,
                                                 _c_vp, _c_vp, _c_vp, _c_i64, _c_i32, _c_i32,
                                                 _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32,
                                                 _c_i32, _c_i32, _c_vp, _c_i64, _c_i64, _c_vp]),
    "ti_gqa_decode_paged_noalloc": (ctypes.c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp,
                                                   _c_i64, _c_vp, _c_vp, _c_i32, _c_i32, _c_i32,
                                                   _c_i32, _c_i32, _c_i64, _c_i32, _c_i32, _c_i32,
                                                   _c_i32, _c_vp]),
    "ti_gqa_decode_scratch_bytes": (ctypes.c_int64, []),
    "ti_last_error": (ctypes.c_char_p, []),
    "ti_abi_version": (ctypes.c_int32, []),
}

_lock = threading.Lock()
_lib = None


class TileInferError(RuntimeError):
    """A nonzero return code from the C ABI, with the library's error text."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[ti error {code}] {message}")
        self.code = code


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library, with argument/return types set."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p} is missing: build it with `python -m tileinfer_amd.build` "
                "(there is no non-HIP fallback)")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.ti_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{p}: ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(rc: int) -> None:
    if rc != TI_OK:
        msg = load().ti_last_error().decode(errors="replace")
        raise TileInferError(rc, msg)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return TI_DTYPE_BF16
    if dtype == torch.float16:
        return TI_DTYPE_F16
    raise TypeError(f"unsupported dtype {dtype}: the paged KV path handles bfloat16 and float16")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device` (torch's raw query when it has one:
    ~0.1 us against ~2 us for building a torch.cuda.Stream object)."""
    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream
