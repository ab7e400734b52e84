"""Lazy backing of KV pool buffers on HIP virtual memory: reserve the whole pool as address space, back it on demand.

Follows the reference's lazy KV cache (patches/kv_lazy.py; docs/ELASTIC_MEMORY.md:46-53): the buffers of the full
context are reserved as address space, a floor of tokens (SGLANG_KV_LAZY_FLOOR, 4096) is backed at start, every page
hand-out backs the prefix up to the highest slot plus a margin (SGLANG_KV_LAZY_MARGIN, 2048 tokens, commits in
margin-sized steps), a headroom rule keeps SGLANG_KV_LAZY_HEADROOM_MB (1536) of device memory free, and when the pool
goes idle the backing beyond the floor is unmapped.

``VmmArena`` is one reserved range (the C ABI kvt_vmm_* of libkvtier.so: hipMemAddressReserve / hipMemCreate /
hipMemMap / hipMemSetAccess); ``LazyKVBacking`` holds the arenas of a pool's per-row buffers (one per tensor, rows
= token slots) and applies the policy.  Tensors over an arena span the whole reservation; only rows below
``backed_tokens`` are backed, and nothing may touch the rest (the pool's kernels read only slots that the
allocator handed out, and every hand-out backs its slots first).
"""
from __future__ import annotations

import ctypes
import logging
import os
import sys
import time
from typing import Callable, List, Optional, Tuple

import torch

from . import _lib

logger = logging.getLogger(__name__)

# --------------------------------------------------------------------------------------------- DLPack (ROCm device)
# A torch tensor over arena memory is made through the DLPack exchange structures (dlpack.h, DLPack 0.x ABI that
# torch.from_dlpack accepts as a "dltensor" capsule); kDLROCM marks a HIP device pointer.
_KDL_ROCM = 10
_DL_CODES = {torch.uint8: (1, 8), torch.int8: (0, 8), torch.int16: (0, 16), torch.int32: (0, 32),
             torch.int64: (0, 64), torch.float16: (2, 16), torch.float32: (2, 32), torch.bfloat16: (4, 16)}


class _DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int), ("device_id", ctypes.c_int)]


class _DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class _DLTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device", _DLDevice), ("ndim", ctypes.c_int), ("dtype", _DLDataType),
                ("shape", ctypes.POINTER(ctypes.c_int64)), ("strides", ctypes.POINTER(ctypes.c_int64)),
                ("byte_offset", ctypes.c_uint64)]


class _DLManagedTensor(ctypes.Structure):
    pass


_DELETER = ctypes.CFUNCTYPE(None, ctypes.POINTER(_DLManagedTensor))
_DLManagedTensor._fields_ = [("dl_tensor", _DLTensor), ("manager_ctx", ctypes.c_void_p), ("deleter", _DELETER)]

# The exchange struct lives in malloc'd memory and the deleter is never freed: torch keeps the struct's address and
# calls its deleter whenever the tensor goes, which can be during interpreter shutdown, after this module's objects
# are gone.  _live keeps the arena (the owner) alive while a tensor over it exists; the deleter's references are
# bound as default arguments so that it still works once the module's globals have been cleared.
_libc = ctypes.CDLL(None)
_libc.malloc.restype = ctypes.c_void_p
_libc.malloc.argtypes = [ctypes.c_size_t]
_libc.free.restype = None
_libc.free.argtypes = [ctypes.c_void_p]
_live = {}   # struct address -> owner


@_DELETER
def _dl_deleter(p, _live=_live, _free=_libc.free, _cast=ctypes.cast, _vp=ctypes.c_void_p):
    addr = _cast(p, _vp).value
    _live.pop(addr, None)
    _free(addr)


ctypes.pythonapi.Py_IncRef(ctypes.py_object(_dl_deleter))   # immortal: torch may call it at any time

_capsule_new = ctypes.pythonapi.PyCapsule_New
_capsule_new.restype = ctypes.py_object
_capsule_new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


def _tensor_at(ptr: int, shape: Tuple[int, ...], dtype: torch.dtype, device_index: int, owner) -> torch.Tensor:
    """A contiguous torch tensor aliasing device memory at ``ptr``; ``owner`` is kept alive as long as the tensor."""
    code, bits = _DL_CODES[dtype]
    nd = len(shape)
    head = ctypes.sizeof(_DLManagedTensor)
    addr = _libc.malloc(head + 8 * max(nd, 1))
    if not addr:
        raise MemoryError("malloc of a DLPack header failed")
    m = _DLManagedTensor.from_address(addr)
    shp = (ctypes.c_int64 * max(nd, 1)).from_address(addr + head)
    for i, x in enumerate(shape):
        shp[i] = int(x)
    m.dl_tensor.data = ptr
    m.dl_tensor.device = _DLDevice(_KDL_ROCM, device_index)
    m.dl_tensor.ndim = nd
    m.dl_tensor.dtype = _DLDataType(code, bits, 1)
    m.dl_tensor.shape = ctypes.cast(addr + head, ctypes.POINTER(ctypes.c_int64))
    m.dl_tensor.strides = None   # compact row-major
    m.dl_tensor.byte_offset = 0
    m.manager_ctx = None
    m.deleter = _dl_deleter
    _live[addr] = owner
    try:
        t = torch.from_dlpack(_capsule_new(addr, b"dltensor", None))
    except Exception:
        _live.pop(addr, None)
        _libc.free(addr)
        raise
    if t.data_ptr() != ptr or tuple(t.shape) != tuple(shape) or t.dtype != dtype:
        raise RuntimeError("torch.from_dlpack did not alias the arena memory as asked")
    return t


# ------------------------------------------------------------------------------------------------------ the arena
class VmmArena:
    """One reserved range of device address space with a backed prefix (kvt_vmm_reserve / commit /
    release_beyond / destroy).  Freed when the last reference (this object or a tensor over it) goes."""

    def __init__(self, nbytes: int, device: Optional[int] = None):
        self.device = torch.cuda.current_device() if device is None else int(device)
        h, base = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("kvt_vmm_reserve", self.device, int(nbytes), ctypes.byref(h), ctypes.byref(base))
        self._h = h
        self.base = int(base.value)
        g = ctypes.c_uint64()
        _lib.call("kvt_vmm_granularity", self.device, ctypes.byref(g))
        self.granularity = int(g.value)

    def _query(self) -> Tuple[int, int, int]:
        b, r, n = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _lib.call("kvt_vmm_backed", self._h, ctypes.byref(b), ctypes.byref(r), ctypes.byref(n))
        return int(b.value), int(r.value), int(n.value)

    @property
    def backed(self) -> int:
        return self._query()[0]

    @property
    def reserved(self) -> int:
        return self._query()[1]

    @property
    def n_mappings(self) -> int:
        return self._query()[2]

    def commit(self, nbytes: int) -> None:
        _lib.call("kvt_vmm_commit", self._h, int(nbytes))

    def release_beyond(self, keep_bytes: int) -> int:
        freed = ctypes.c_uint64()
        _lib.call("kvt_vmm_release_beyond", self._h, int(keep_bytes), ctypes.byref(freed))
        return int(freed.value)

    def tensor(self, shape: Tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
        """A contiguous tensor over the start of the reservation (only its backed prefix may be touched)."""
        n = 1
        for s in shape:
            n *= int(s)
        if n * torch.empty(0, dtype=dtype).element_size() > self.reserved:
            raise ValueError(f"tensor {tuple(shape)} {dtype} exceeds the arena's {self.reserved} reserved bytes")
        return _tensor_at(self.base, tuple(int(s) for s in shape), dtype, self.device, self)

    def close(self) -> None:
        if self._h is not None and self._h.value:
            _lib.call("kvt_vmm_destroy", self._h)
            self._h = None

    def __del__(self):
        if sys.is_finalizing():   # interpreter shutdown: the process exit gives everything back
            return
        try:
            self.close()
        except Exception:
            pass


# ------------------------------------------------------------------------------------------------------ the policy
def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name, str(default))
    try:
        return int(raw)
    except ValueError:
        raise ValueError(f"{name}={raw!r} is not an integer") from None


class LazyKVBacking:
    """The buffers of one pool (rows = token slots, ``rows`` of them) on arenas, with the reference's lazy policy
    (patches/kv_lazy.py:113-175 lazy_ensure / lazy_release; :70-88 ensure_prefix / release_beyond).

    ``arena_factory`` and ``free_memory`` are injection points (tests drive the policy on the CPU with stand-ins);
    by default they are VmmArena and torch.cuda.mem_get_info.
    """

    def __init__(self, rows: int, size: int, page_size: int, device=None, floor: Optional[int] = None,
                 margin: Optional[int] = None, headroom_mb: Optional[int] = None,
                 arena_factory: Optional[Callable] = None, free_memory: Optional[Callable[[], int]] = None):
        self.rows = int(rows)
        self.size = int(size)
        self.page_size = int(page_size)
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.floor = min(self.size, _env_int("SGLANG_KV_LAZY_FLOOR", 4096) if floor is None else int(floor))
        self.margin = _env_int("SGLANG_KV_LAZY_MARGIN", 2048) if margin is None else int(margin)
        if self.margin <= 0 or self.floor < 0:
            raise ValueError(f"lazy backing: margin {self.margin} must be > 0 and floor {self.floor} >= 0")
        self.headroom = (_env_int("SGLANG_KV_LAZY_HEADROOM_MB", 1536) if headroom_mb is None else int(headroom_mb)) << 20
        dev_index = self.device.index if self.device.index is not None else None
        self._arena_factory = arena_factory or (lambda nbytes: VmmArena(nbytes, dev_index))
        self._free_memory = free_memory or (lambda: torch.cuda.mem_get_info(self.device)[0])
        self.buffers: List[Tuple[object, torch.Tensor, int]] = []   # (arena, tensor, bytes per row)
        self.backed_tokens = 0
        self._last_empty = 0.0

    # -- layout
    def add(self, shape: Tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
        """Reserve a [rows, ...] buffer; returns the tensor over it (backed up to backed_tokens)."""
        if int(shape[0]) != self.rows:
            raise ValueError(f"lazy buffer rows {shape[0]} != pool rows {self.rows}")
        row_bytes = torch.empty(0, dtype=dtype).element_size()
        for s in shape[1:]:
            row_bytes *= int(s)
        arena = self._arena_factory(self.rows * row_bytes)
        t = arena.tensor(tuple(shape), dtype)
        self.buffers.append((arena, t, row_bytes))
        if self.backed_tokens:
            self._commit_rows(arena, t, row_bytes, 0, self.backed_tokens)
        return t

    def bytes_per_token(self) -> int:
        return sum(rb for _, _, rb in self.buffers)

    @property
    def backed_bytes(self) -> int:
        return sum(a.backed for a, _, _ in self.buffers)

    # -- mechanism
    def _commit_rows(self, arena, t: torch.Tensor, row_bytes: int, old: int, new: int) -> None:
        arena.commit(new * row_bytes)
        if new > old:
            t[old:new].zero_()   # fresh backing reads as zeros, like the eagerly allocated pool

    def ensure_prefix(self, num_tokens: int) -> None:
        """Back rows [0, num_tokens) of every buffer (patches/kv_lazy.py:70-75)."""
        want = min(int(num_tokens), self.rows)
        if want <= self.backed_tokens:
            return
        for arena, t, rb in self.buffers:
            self._commit_rows(arena, t, rb, self.backed_tokens, want)
        self.backed_tokens = want

    def release_beyond(self, num_tokens: int) -> int:
        """Unmap the backing beyond the first num_tokens rows of every buffer (patches/kv_lazy.py:77-88); the
        device is synchronized first (queued work may still read the rows)."""
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        freed = 0
        for arena, _, rb in self.buffers:
            freed += arena.release_beyond(int(num_tokens) * rb)
        self.backed_tokens = min(self.backed_tokens, int(num_tokens))
        return freed

    # -- policy
    def want_tokens(self, num_tokens: int) -> int:
        """Slots [0, want) are backed after ensure(num_tokens): the next multiple of the margin past
        num_tokens + margin, capped at size + page_size (the slot index == size exists), patches/kv_lazy.py:119-120."""
        m = self.margin
        return min(self.size + self.page_size, -(-(int(num_tokens) + m) // m) * m)

    def ensure(self, num_tokens: int) -> None:
        """Back slots [0, num_tokens + margin) in margin steps, keeping `headroom` bytes of device memory free
        (patches/kv_lazy.py:113-160; no elastic expert cache here to give memory back, so a commit that would leave
        less than half the headroom is refused with RuntimeError)."""
        want = self.want_tokens(num_tokens)
        if want <= self.backed_tokens:
            return
        delta = (want - self.backed_tokens) * self.bytes_per_token()
        if self._free_memory() - delta < self.headroom:
            now = time.time()
            if now - self._last_empty > 30.0:
                if self.device.type == "cuda":
                    torch.cuda.empty_cache()   # torch-cached blocks are not driver-free
                self._last_empty = now
            free = self._free_memory()
            if free - delta < self.headroom // 2:
                raise RuntimeError(f"KV lazy backing: no headroom for {want} tokens (free {free >> 20} MB, "
                                   f"need {(delta + self.headroom) >> 20} MB)")
        try:
            self.ensure_prefix(want)
        except RuntimeError:
            if self.device.type == "cuda":
                torch.cuda.empty_cache()
            self.ensure_prefix(want)
        logger.info("KV lazy commit: tokens %d -> %d (backed %.0f MB)", num_tokens, want, self.backed_bytes / 2 ** 20)

    def release(self) -> int:
        """Back to the floor (patches/kv_lazy.py:162-168)."""
        freed = self.release_beyond(self.floor)
        if freed:
            logger.info("KV lazy backing: released %.0f MB beyond the %d-token floor", freed / 2 ** 20, self.floor)
        return freed
