"""ctypes binding of the gfx950 C ABI (``include/vsa_capi.h``).

The shared library is built in-tree by ``make -C simple-vsa_amd/csrc`` (or
``__graft_entry__.build()``).  Nothing here falls back to another
implementation: if the library is missing, or a kernel reports an error,
the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libvsa_mi355x.so")

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
GATE_NONE, GATE_FULL, GATE_PER_TOKEN, GATE_TOKEN_MAJOR = 0, 1, 2, 3
GATE_F32 = 4   # flag: an fp32 gate beside bf16 / fp16 inputs

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

# name -> argument types (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "vsa_status_string": [ctypes.c_int],
    "vsa_version": [],
    "vsa_pool_qkv": [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _P],
    "vsa_coarse_fwd": [_P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _F, _I32, _P],
    "vsa_topk": [_P, _P, _I64, _I32, _I32, _P],
    "vsa_csr_build": [_P, _P, _P, _P, _I64, _I32, _I32, _I32, _P],
    "vsa_sparse_fwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I64, _I64, _I64,
                       _I32, _I32, _I32, _F, _I32, _P],
    "vsa_bwd_prep": [_P, _P, _P, _P, _I32, _I32, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P],
    "vsa_coarse_bwd": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _F, _I32, _P],
    "vsa_sparse_bwd_dq": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I32,
                          _I32, _I32, _F, _I32, _P],
    "vsa_dkdv_tile_order": [_P, _P, _I64, _I64, _I64, _I32, _I32, _P],
    "vsa_sparse_bwd_dkdv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                            _I64, _I32, _I32, _I32, _F, _P, _I32, _P],
    "vsa_sparse_bwd_dkdv_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64,
                                    _I64, _I64, _I32, _I32, _I32, _F, _I32, _P],
    "vsa_tile_metadata": [_I32, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P],
    "vsa_rows_move": [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P,
                      _I64, _P],
    "vsa_rows_zero_unmarked": [_P, _I64, _I64, _I64, _P, _I64, _P, _P],
    # tiled sequences (tile / untile fused into the op)
    "vsa_tile_slot_rows": [_I32, _I32, _I32, _I32, _I32, _I32, _P, _P],
    "vsa_tile_pool_qkv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I32,
                          _I32, _I32, _I32, _I32, _P],
    "vsa_sparse_fwd_tiled": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _I64, _I32, _I64,
                             _I64, _I64, _I32, _I32, _I32, _F, _I32, _P],
    "vsa_bwd_prep_tiled": [_P, _P, _P, _P, _I32, _P, _I64, _I32, _P, _P, _P, _P, _I64, _I64, _I32,
                           _I32, _I32, _P],
    "vsa_sparse_bwd_dq_tiled": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I32, _I64,
                                _I64, _I64, _I32, _I32, _I32, _F, _I32, _P],
    "vsa_sparse_bwd_dkdv_tiled": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                  _I64, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _F, _P, _I32,
                                  _P],
}
_RESTYPES = {"vsa_status_string": ctypes.c_char_p, "vsa_version": ctypes.c_char_p}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load the library once (thread-safe) and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"MI355X VSA kernels are not built ({LIB_PATH} is missing); "
                    "run `make -C simple-vsa_amd/csrc` or __graft_entry__.build()")
            lib = ctypes.CDLL(LIB_PATH)
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def status_string(code: int) -> str:
    return load().vsa_status_string(code).decode()


def call(name: str, *args) -> None:
    """Invoke an entry point; a non-zero status becomes a RuntimeError."""
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed: {status_string(rc)} (status {rc})")


def ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current HIP stream of ``t``'s device, as the C ABI's ``void*``."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dt]
    except KeyError:
        raise ValueError("the MI355X path supports float16, bfloat16 and float32 tensors") from None
