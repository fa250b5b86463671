"""ctypes binding of ``libinfrared_amd.so`` (declared in ``include/infrared_amd.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded (one runtime per process: torch's streams and device pointers
are then valid inside the library). There is no fallback: if the library is
missing or a call fails, a ``RuntimeError`` names the cause.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libinfrared_amd.so")

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
_DTYPE_CODES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

# err_flags bits (IR_ERR_*)
ERR_SLOT_RANGE = 1
ERR_BLOCK_RANGE = 2
ERR_CONTEXT_RANGE = 4
ERR_GATHER_RANGE = 8
ERR_PLAN = 16
ERR_WRITE_SLOT = 32

_c_i32, _c_i64, _c_f32, _c_p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/infrared_amd.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ir_last_error": (ctypes.c_char_p, []),
    "ir_version": (ctypes.c_char_p, []),
    "ir_kv_scatter": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64,
         _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p],
    ),
    "ir_gather_slots": (
        _c_i32,
        [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p,
         _c_p, _c_p],
    ),
    "ir_paged_gather": (
        _c_i32,
        [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i32, _c_p, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p],
    ),
    "ir_paged_decode_workspace_size": (
        _c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32],
    ),
    "ir_paged_decode_default_partition": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32]),
    "ir_paged_decode_num_counters": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "ir_paged_decode": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i32,
         _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_i32,
         _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p],
    ),
    "ir_paged_decode_noalloc": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i32,
         _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_i32,
         _c_p, _c_p],
    ),
    "ir_paged_decode_plan_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "ir_paged_decode_planned_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32]),
    "ir_paged_decode_plan": (
        _c_i32,
        [_c_p, _c_i64, _c_i32, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i64, _c_i64,
         _c_i32, _c_i32, _c_p, _c_i64, _c_p, _c_p],
    ),
    "ir_paged_decode_planned": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_i32, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p],
    ),
    "ir_paged_attention_masked": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64,
         _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_i32, _c_f32, _c_i32, _c_p, _c_p, _c_p],
    ),
    "ir_rope_kv_scatter": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64,
         _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_p, _c_p],
    ),
    "ir_paged_prefill": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64, _c_i32,
         _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_f32,
         _c_i32, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p],
    ),
    "ir_decode_form": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_p, _c_i64,
         _c_i32, _c_p, _c_p, _c_i32, _c_p, ctypes.c_uint32, _c_p],
    ),
    "ir_stream_capture_id": (_c_i32, [_c_p, ctypes.POINTER(ctypes.c_uint64)]),
    "ir_varlen_form_scan": (
        _c_i32,
        [_c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_p,
         _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_p],
    ),
    "ir_varlen_form_tables": (
        _c_i32,
        [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_p, _c_i64, _c_i32, _c_p],
    ),
    "ir_hbm_read_granule": (_c_i64, []),
    "ir_hbm_read": (_c_i32, [_c_p, _c_i64, _c_p, _c_i32, _c_p]),
    "ir_paged_prefill_plan_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "ir_paged_prefill_plan": (
        _c_i32,
        [_c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p,
         _c_i64, _c_p],
    ),
    "ir_paged_prefill_plan_xcds": (_c_i32, []),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (loads it on first use); raises if it was never built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build the HIP kernels first "
                        "(python -m infrared_amd.build); there is no non-HIP fallback"
                    )
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raises ``RuntimeError`` with the library's message when ``rc`` is an error."""
    if rc != 0:
        msg = lib().ir_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"dtype {dtype} is not supported (float32, float16, bfloat16)") from None


def stream_ptr(device: torch.device) -> int:
    """Raw handle of torch's current stream on ``device`` (the capturing stream
    under hipGraph capture): the same handle as
    ``torch.cuda.current_stream(device).cuda_stream``, read without building a
    stream object."""
    if _raw_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    index = device.index
    return _raw_stream(torch.cuda.current_device() if index is None else index)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on the same ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"infrared_amd runs on ROCm device tensors only; got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev
