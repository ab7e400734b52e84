"""ctypes binding of libkvtier.so (the C ABI declared in include/kvtier.h).

The library is the only compute path of this package: if it is missing, every op raises (there is no CPU or torch
fallback).  Arguments are plain device pointers, integer sizes/strides and the current HIP stream.
"""
from __future__ import annotations

import ctypes
import os
import re
from typing import Optional

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkvtier.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "kvtier.h")

KVT_OK, KVT_EINVAL, KVT_ELAUNCH, KVT_ERANGE = 0, -1, -2, -3
KVT_ENOTSUP, KVT_ENOMEM, KVT_EHIP = -4, -5, -6
DTYPE_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
_U = ctypes.c_uint64

# argument types per entry point, in declaration order (must match include/kvtier.h)
SIGNATURES = {
    "kvt_quant_store_tiered": [_P, _P, _I, _L, _L, _L, _L, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                               _P, _P, _L, _I, _P],
    "kvt_quant_store_int8": [_P, _P, _I, _L, _L, _L, _L, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P],
    "kvt_quant_store_int4": [_P, _P, _I, _L, _L, _L, _L, _P, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    "kvt_page_table_update": [_P, _L, _L, _P, _P, _P, _P],
    "kvt_append_plan": [_I, _P, _P, _P, _P, _P, _P, _L, _I, _P, _I, _P, _P, _P, _P, _P],
    "kvt_append_evict": [_P, _P, _I, _L, _L, _L, _L, _P, _P, _L, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                         _P, _L, _P, _P, _I, _P],
    "kvt_sparse_cu_seqlens": [_P, _P, _L, _P, _P, _I, _I, _I, _P],
    "kvt_compact_gather": [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _P, _I, _P, _L, _P, _P, _I,
                           _I, _I, _I, _I, _I, _P, _P, _P],
    "kvt_sparse_decode": [_I, _P, _L, _P, _P, _P, _P, _L, _P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _P, _I, _P, _L,
                          _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _P, _P, _P, _P, _L, _P],
    "kvt_sparse_prefill": [_I, _P, _L, _L, _P, _I, _P, _I, _I, _P, _L, _L, _L, _I, _P, _P, _P, _P, _L, _P, _P, _P,
                           _P, _P, _L, _P, _P, _P, _L, _P, _I, _I, _I, _I, _I, _F, _P, _I, _L, _L, _P],
    "kvt_prefix_gather": [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _P, _P, _P, _L, _P, _I, _P, _P, _I, _I, _L,
                          _I, _I, _I, _P, _P, _P],
    "kvt_decode_ref": [_I, _P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                       _L, _P, _L, _P, _P, _L, _F, _I, _I, _P, _P, _P],
    "kvt_decode_mfma": [_P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L, _L, _F,
                        _I, _P, _I, _P, _P, _I, _P, _P],
    "kvt_decode_plan": [_P, _P, _P, _P, _P, _L, _I, _I, _P, _I, _P, _P],
    "kvt_decode_mfma_noalloc": [_P, _L, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _L,
                                _L, _F, _I, _P, _I, _P, _I, _P, _P, _L, _P],
    "kvt_decode_combine": [_P, _P, _I, _I, _I, _I, _I, _L, _P, _P, _P, _P, _L, _P],
    "kvt_prefill_attn": [_P, _L, _L, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                         _P, _L, _L, _P, _P, _L, _L, _L, _L, _L, _F, _P, _I, _L, _L, _I, _P, _L, _P],
    "kvt_prefill_work_bytes": [_I, _I, _I, _I, _I, _P],
    "kvt_vmm_granularity": [_I, _P],
    "kvt_vmm_reserve": [_I, _U, _P, _P],
    "kvt_vmm_commit": [_P, _U],
    "kvt_vmm_release_beyond": [_P, _U, _P],
    "kvt_vmm_backed": [_P, _P, _P, _P],
    "kvt_vmm_destroy": [_P],
}

_lib: Optional[ctypes.CDLL] = None


def header_symbols():
    """Entry points declared in include/kvtier.h (used by the ABI test)."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"^int\s+(kvt_\w+)\(", text, flags=re.M)))


def lib() -> ctypes.CDLL:
    """Load libkvtier.so once; raise if it is absent (build it with __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: the HIP kernels are not built (run __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = handle
    return _lib


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def require_device(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise AssertionError("libkvtier operates on device tensors only (no CPU fallback)")


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status == KVT_OK:
        return
    if status == KVT_EINVAL:
        raise ValueError(f"{name}: unsupported shape, dtype or size (status {status})")
    if status == KVT_ERANGE:
        raise ValueError(f"{name}: size beyond the supported maximum (status {status})")
    if status == KVT_ENOTSUP:
        raise RuntimeError(f"{name}: the device does not support virtual memory management (status {status})")
    if status == KVT_ENOMEM:
        raise RuntimeError(f"{name}: out of device address space or physical memory (status {status})")
    if status == KVT_EHIP:
        raise RuntimeError(f"{name}: HIP runtime call failed (status {status})")
    raise RuntimeError(f"{name}: kernel launch failed (status {status})")
