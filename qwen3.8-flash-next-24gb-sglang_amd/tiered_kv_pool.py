"""KV pools of the tiered path: INT4-G32 full-context rows + an INT8 ring of the last R written slots + owner table.

Mirrors the reference's pool classes (``MHATokenToKVPoolInt8`` patches/kv_int8.py:69-202,
``MHATokenToKVPoolInt4`` patches/kv_int4.py:81-227, ``MHATokenToKVPoolTiered`` patches/kv_tiers.py:103-229) with
the same attributes, accessors, guards and exceptions, standalone (no SGLang base class: the upstream
``MHATokenToKVPool`` parts they use -- buffer lists, size/page_size/layer bookkeeping -- are restated here).
Writes go through the HIP kernels (sparse_attn.quant_store_kv_*).  With lazy=True (or SGLANG_KV_LAZY=1, as the
reference's patches/kv_lazy.py:100-106) the per-slot buffers live on HIP virtual memory and are backed on demand
(lazy_kv.LazyKVBacking; the ring and owner table stay eagerly allocated); ``PagedTokenAllocator`` mirrors the
allocator hooks that drive it.  CPU offload is not provided (it raises NotImplementedError like the reference).
"""
from __future__ import annotations

import logging
import os
from typing import Optional, Tuple

import torch

from .lazy_kv import LazyKVBacking
from .sparse_attn import KV_INT4_GROUP, KV_INT8_GROUP, quant_store_kv_int4, quant_store_kv_int8, quant_store_kv_tiered

logger = logging.getLogger(__name__)


def _is_unit_scale(s) -> bool:
    """patches/kv_int4.py:77-78."""
    return s is None or (isinstance(s, (int, float)) and s == 1)


def unwrap_write_loc(loc_info):
    """The write location of a set_kv_buffer call: a tensor, or a tuple / object carrying it first (upstream
    memory_pool.unwrap_write_loc returns (loc, ...))."""
    if isinstance(loc_info, torch.Tensor):
        return loc_info, None, None
    if isinstance(loc_info, (tuple, list)):
        return loc_info[0], None, None
    return loc_info.loc, None, None


def _detect_oob(loc: torch.Tensor, lo: int, hi: int, what: str) -> None:
    """Optional bounds probe of write slots (reference maybe_detect_oob, patches/kv_tiers.py:192); a host-synchronous
    check enabled by KVT_DETECT_OOB=1, off by default like the reference's async probe."""
    if os.environ.get("KVT_DETECT_OOB") and loc.numel():
        mn, mx = int(loc.min()), int(loc.max())
        if mn < lo or mx >= hi:
            raise IndexError(f"{what}: slot range [{mn}, {mx}] outside [{lo}, {hi})")


class _QuantKVPool:
    """Shared bookkeeping of the quantized MHA pools (NHD layout, rows = size + page_size)."""

    kv_bits: Optional[int] = None
    GROUP = 1

    def __init__(self, size: int, page_size: int, dtype: torch.dtype, head_num: int, head_dim: int, layer_num: int,
                 device, enable_memory_saver: bool = False, start_layer: int = 0, v_head_dim: Optional[int] = None,
                 lazy: Optional[bool] = None, **unused):
        self.lazy = (os.environ.get("SGLANG_KV_LAZY") == "1") if lazy is None else bool(lazy)
        self._lazy = None
        self.size = size
        self.page_size = page_size
        self.dtype = dtype
        self.store_dtype = dtype
        self.head_num = head_num
        self.head_dim = head_dim
        self.v_head_dim = head_dim if v_head_dim is None else v_head_dim
        self.layer_num = layer_num
        self.device = device
        self.start_layer = start_layer
        self.end_layer = start_layer + layer_num - 1
        self.use_hnd = False
        self.kv_cache_layout = "nhd"
        self.k_scale_buffer = None
        self.v_scale_buffer = None
        self._create_buffers()
        L, H = self.layer_num, self.head_num
        # static per-channel smoothing constants, identity (patches/kv_int4.py:95-100)
        self.sm_k = torch.ones((L, H, self.head_dim), dtype=torch.float16, device=self.device)
        self.sm_v = torch.ones((L, H, self.v_head_dim), dtype=torch.float16, device=self.device)
        self.sm_k_inv = torch.ones_like(self.sm_k)
        self.sm_v_inv = torch.ones_like(self.sm_v)

    # -- layout
    @property
    def k_groups(self) -> int:
        if self.head_dim % self.GROUP:
            raise ValueError(f"head_dim {self.head_dim} not a multiple of GROUP {self.GROUP}")
        return self.head_dim // self.GROUP

    @property
    def v_groups(self) -> int:
        if self.v_head_dim % self.GROUP:
            raise ValueError(f"v_head_dim {self.v_head_dim} not a multiple of GROUP {self.GROUP}")
        return self.v_head_dim // self.GROUP

    def _rows(self) -> int:
        return self.size + self.page_size

    def _scale_shapes(self):
        rows = self._rows()
        return (rows, self.head_num, self.k_groups), (rows, self.head_num, self.v_groups)

    def _kv_buffer_shapes(self):
        raise NotImplementedError

    def _create_buffers(self):
        (ksh, vsh) = self._kv_buffer_shapes()
        ks_shape, vs_shape = self._scale_shapes()
        if self.lazy:
            # address space for every slot, the floor backed now (patches/kv_lazy.py:100-106)
            lz = LazyKVBacking(self._rows(), self.size, self.page_size, self.device)
            self.k_buffer = [lz.add(ksh, self.store_dtype) for _ in range(self.layer_num)]
            self.v_buffer = [lz.add(vsh, self.store_dtype) for _ in range(self.layer_num)]
            self.k_scale_buffer = [lz.add(ks_shape, torch.float16) for _ in range(self.layer_num)]
            self.v_scale_buffer = [lz.add(vs_shape, torch.float16) for _ in range(self.layer_num)]
            lz.ensure_prefix(lz.floor)
            self._lazy = lz
            logger.info("KV lazy backing: %d tokens reserved as VA, %d backed (floor), margin %d, %.1f KB/token",
                        self.size, lz.floor, lz.margin, lz.bytes_per_token() / 1024)
            return
        self.k_buffer = [torch.zeros(ksh, dtype=self.store_dtype, device=self.device) for _ in range(self.layer_num)]
        self.v_buffer = [torch.zeros(vsh, dtype=self.store_dtype, device=self.device) for _ in range(self.layer_num)]
        self.k_scale_buffer = [torch.zeros(ks_shape, dtype=torch.float16, device=self.device)
                               for _ in range(self.layer_num)]
        self.v_scale_buffer = [torch.zeros(vs_shape, dtype=torch.float16, device=self.device)
                               for _ in range(self.layer_num)]

    def _clear_buffers(self):
        self.k_buffer = self.v_buffer = self.k_scale_buffer = self.v_scale_buffer = None
        self._lazy = None

    # -- accessors
    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self.k_buffer[layer_id - self.start_layer]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self.v_buffer[layer_id - self.start_layer]

    def get_kv_buffer(self, layer_id: int):
        return self.get_key_buffer(layer_id), self.get_value_buffer(layer_id)

    def get_kv_scale_buffer(self, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        idx = layer_id - self.start_layer
        return self.k_scale_buffer[idx], self.v_scale_buffer[idx]

    def get_kv_smooth_buffer(self, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        idx = layer_id - self.start_layer
        return self.sm_k[idx], self.sm_v[idx]

    def get_kv_size_bytes(self):
        kb = sum(t.numel() * t.element_size() for t in self.k_buffer + self.k_scale_buffer)
        vb = sum(t.numel() * t.element_size() for t in self.v_buffer + self.v_scale_buffer)
        return kb, vb

    # -- write path
    def _write_prologue(self, loc_info, cache_k, cache_v, k_scale, v_scale, layer, layer_id_override, dcp_kv_mask,
                        name):
        if dcp_kv_mask is not None:
            raise NotImplementedError(f"{name} KV cache does not support DCP KV masks")
        if not (_is_unit_scale(k_scale) and _is_unit_scale(v_scale)):
            raise ValueError(f"{name} KV cache computes its own scales; got k_scale/v_scale")
        loc, _, _ = unwrap_write_loc(loc_info)
        _detect_oob(loc, 0, self.size + self.page_size, f"set_kv_buffer ({name})")
        layer_id = layer_id_override if layer_id_override is not None else layer.layer_id
        idx = layer_id - self.start_layer
        cache_k = cache_k.view(-1, self.head_num, self.head_dim)
        cache_v = cache_v.view(-1, self.head_num, self.v_head_dim)
        return loc, idx, cache_k, cache_v

    def set_kv_buffer_prefix_valid(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__}: prefix-valid commit is not supported")

    def get_cpu_copy(self, indices, mamba_indices=None):
        raise NotImplementedError(f"{type(self).__name__}: CPU offload is not supported")

    def load_cpu_copy(self, kv_cache_cpu, indices, mamba_indices=None):
        raise NotImplementedError(f"{type(self).__name__}: CPU offload is not supported")

    # -- lazy backing (patches/kv_lazy.py:113-175); no-ops on an eagerly allocated pool
    @property
    def lazy_backed_tokens(self) -> int:
        """Slots [0, n) are backed (every slot of an eager pool)."""
        return self._rows() if self._lazy is None else self._lazy.backed_tokens

    def lazy_ensure(self, num_tokens: int) -> None:
        """Back slots [0, num_tokens + margin) in margin steps (RuntimeError when the device cannot)."""
        if self._lazy is not None:
            self._lazy.ensure(num_tokens)

    def lazy_release(self) -> None:
        """Unmap the backing beyond the floor (the pool is idle: no slot in use)."""
        if self._lazy is not None:
            self._lazy.release()


class MHATokenToKVPoolInt8(_QuantKVPool):
    """int8 K/V [rows, H, D] + fp16 absmax/127 scales per (token, head, 64 channels) (patches/kv_int8.py:69-202)."""

    GROUP = KV_INT8_GROUP
    kv_bits = 8

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self.dtype != torch.int8 or self.store_dtype != torch.int8:
            raise ValueError(f"MHATokenToKVPoolInt8 needs dtype int8, got {self.dtype}/{self.store_dtype}")

    def _kv_buffer_shapes(self):
        rows = self._rows()
        return (rows, self.head_num, self.head_dim), (rows, self.head_num, self.v_head_dim)

    def set_kv_buffer(self, layer, loc_info, cache_k, cache_v, k_scale=None, v_scale=None, layer_id_override=None,
                      dcp_kv_mask=None):
        loc, idx, ck, cv = self._write_prologue(loc_info, cache_k, cache_v, k_scale, v_scale, layer,
                                                layer_id_override, dcp_kv_mask, "int8_g64")
        quant_store_kv_int8(ck, cv, loc, self.k_buffer[idx], self.v_buffer[idx], self.k_scale_buffer[idx],
                            self.v_scale_buffer[idx], self.sm_k_inv[idx], self.sm_v_inv[idx])


class MHATokenToKVPoolInt4(_QuantKVPool):
    """Nibble-packed int4 K/V [rows, H, D // 2] + fp16 absmax/7 scales per (token, head, 32 channels)
    (patches/kv_int4.py:81-227)."""

    GROUP = KV_INT4_GROUP
    kv_bits = 4

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self.dtype != torch.uint8 or self.store_dtype != torch.uint8:
            raise ValueError(f"MHATokenToKVPoolInt4 needs dtype uint8, got {self.dtype}/{self.store_dtype}")

    def _kv_buffer_shapes(self):
        if self.head_dim % 2 or self.v_head_dim % 2:
            raise ValueError("MHATokenToKVPoolInt4 needs even head dims")
        rows = self._rows()
        return (rows, self.head_num, self.head_dim // 2), (rows, self.head_num, self.v_head_dim // 2)

    def set_kv_buffer(self, layer, loc_info, cache_k, cache_v, k_scale=None, v_scale=None, layer_id_override=None,
                      dcp_kv_mask=None):
        loc, idx, ck, cv = self._write_prologue(loc_info, cache_k, cache_v, k_scale, v_scale, layer,
                                                layer_id_override, dcp_kv_mask, "int4_g32")
        quant_store_kv_int4(ck, cv, loc, self.k_buffer[idx], self.v_buffer[idx], self.k_scale_buffer[idx],
                            self.v_scale_buffer[idx], self.sm_k_inv[idx], self.sm_v_inv[idx])


def ring_slots_from_env() -> int:
    """SGLANG_KV_TIERS_W: ring slots R (default 8192), a positive power of two (patches/kv_tiers.py:91-100)."""
    raw = os.environ.get("SGLANG_KV_TIERS_W", "8192")
    try:
        r = int(raw)
    except ValueError:
        raise ValueError(f"SGLANG_KV_TIERS_W={raw!r} is not an integer") from None
    if r <= 0 or (r & (r - 1)):
        raise ValueError(f"SGLANG_KV_TIERS_W must be a positive power of two, got {r}")
    return r


class MHATokenToKVPoolTiered(MHATokenToKVPoolInt4):
    """INT4-G32 full-context rows (inherited) + an INT8-G64 ring of the last R written slots + owner table
    (patches/kv_tiers.py:103-229)."""

    RING_GROUP = KV_INT8_GROUP
    kv_tiered = True

    def __init__(self, *args, **kwargs):
        self.ring_k = self.ring_v = self.ring_ks = self.ring_vs = self.ring_owner = None
        super().__init__(*args, **kwargs)
        R = ring_slots_from_env()
        if R > self.size:
            raise ValueError(f"SGLANG_KV_TIERS_W={R} exceeds the KV pool size {self.size}")
        if self.head_dim % self.RING_GROUP or self.v_head_dim % self.RING_GROUP:
            raise ValueError(f"head dims {self.head_dim}/{self.v_head_dim} not multiples of RING_GROUP {self.RING_GROUP}")
        self.ring_slots = R
        L, H = self.layer_num, self.head_num
        ks_shape = (R, H, self.head_dim // self.RING_GROUP)
        vs_shape = (R, H, self.v_head_dim // self.RING_GROUP)
        self.ring_k = [torch.zeros((R, H, self.head_dim), dtype=torch.int8, device=self.device) for _ in range(L)]
        self.ring_v = [torch.zeros((R, H, self.v_head_dim), dtype=torch.int8, device=self.device) for _ in range(L)]
        self.ring_ks = [torch.zeros(ks_shape, dtype=torch.float16, device=self.device) for _ in range(L)]
        self.ring_vs = [torch.zeros(vs_shape, dtype=torch.float16, device=self.device) for _ in range(L)]
        self.ring_owner = torch.full((R,), -1, dtype=torch.int32, device=self.device)
        ring_bytes = sum(t.numel() * t.element_size() for t in self.ring_k + self.ring_v + self.ring_ks + self.ring_vs)
        logger.info("KV tiers: ring R=%d slots (int8_g%d over int4_g%d), %.0f MB, owner %d KB", R, self.RING_GROUP,
                    self.GROUP, ring_bytes / 2 ** 20, self.ring_owner.numel() * 4 // 1024)

    @property
    def ring_mask(self) -> int:
        return self.ring_slots - 1

    def _ring_bytes(self):
        kb = sum(t.numel() * t.element_size() for t in self.ring_k + self.ring_ks)
        vb = sum(t.numel() * t.element_size() for t in self.ring_v + self.ring_vs)
        return kb + self.ring_owner.numel() * self.ring_owner.element_size(), vb

    def get_kv_size_bytes(self):
        kb, vb = super().get_kv_size_bytes()
        if self.ring_k is not None:
            rk, rv = self._ring_bytes()
            kb += rk
            vb += rv
        return kb, vb

    def _clear_buffers(self):
        super()._clear_buffers()
        self.ring_k = self.ring_v = self.ring_ks = self.ring_vs = self.ring_owner = None

    def get_kv_ring_buffer(self, layer_id: int):
        idx = layer_id - self.start_layer
        return self.ring_k[idx], self.ring_v[idx], self.ring_ks[idx], self.ring_vs[idx]

    def get_kv_ring_owner(self) -> torch.Tensor:
        return self.ring_owner

    def set_kv_buffer(self, layer, loc_info, cache_k, cache_v, k_scale=None, v_scale=None, layer_id_override=None,
                      dcp_kv_mask=None):
        if dcp_kv_mask is not None:
            raise NotImplementedError("int8ring_int4 KV cache does not support DCP KV masks")
        if not (_is_unit_scale(k_scale) and _is_unit_scale(v_scale)):
            raise ValueError("int8ring_int4 KV cache computes its own scales; got k_scale/v_scale")
        loc, _, _ = unwrap_write_loc(loc_info)
        if loc.numel() > self.ring_slots:
            raise ValueError(f"int8ring_int4: {loc.numel()} tokens in one write exceed the ring of {self.ring_slots} slots")
        loc, idx, ck, cv = self._write_prologue(loc_info, cache_k, cache_v, None, None, layer, layer_id_override, None,
                                                "int8ring_int4")
        quant_store_kv_tiered(ck, cv, loc, self.k_buffer[idx], self.v_buffer[idx], self.k_scale_buffer[idx],
                              self.v_scale_buffer[idx], self.ring_k[idx], self.ring_v[idx], self.ring_ks[idx],
                              self.ring_vs[idx], self.ring_owner, self.sm_k_inv[idx], self.sm_v_inv[idx],
                              self.ring_mask)

    def lazy_release(self) -> None:
        """Release the lazy backing, and reset the owner table (patches/kv_tiers.py:224-229)."""
        super().lazy_release()
        if self.ring_owner is not None:
            self.ring_owner.fill_(-1)


class PagedTokenAllocator:
    """Page-granular slot allocator with the lazy-backing hooks of the reference (SGLang's
    PagedTokenToKVPoolAllocator as patched by patches/kv_lazy.py:207-283): pages 1 .. size // page_size in
    slot order; ``alloc`` backs the slots of the pages it is about to hand out (kvcache.lazy_ensure((max page + 1) *
    page_size)) and refuses (returns None, pages stay free) when that fails; when every page is free again the list
    returns to slot order and the pool's backing beyond the floor is released (kvcache.lazy_release())."""

    def __init__(self, size: int, page_size: int, kvcache, device="cpu"):
        if size % page_size:
            raise ValueError(f"size {size} is not a multiple of page_size {page_size}")
        self.size = size
        self.page_size = page_size
        self.num_pages = size // page_size
        self._kvcache = kvcache
        self.device = device
        self.clear()

    def clear(self) -> None:
        self.free_pages = torch.arange(1, self.num_pages + 1, dtype=torch.int64)

    def available_size(self) -> int:
        return int(self.free_pages.numel()) * self.page_size

    def _lazy_hook(self, pages: torch.Tensor) -> bool:
        ensure = getattr(self._kvcache, "lazy_ensure", None)
        if ensure is None or pages.numel() == 0:
            return True
        try:
            ensure((int(pages.max()) + 1) * self.page_size)
            return True
        except Exception as ex:
            logger.warning("KV lazy backing: commit failed, allocation refused (%s)", ex)
            return False

    def alloc(self, need_size: int) -> Optional[torch.Tensor]:
        """``need_size`` slots (a multiple of page_size) as int64 slot indices, or None when the pool is full or
        their backing cannot be committed."""
        if need_size % self.page_size:
            raise ValueError(f"need_size {need_size} is not a multiple of page_size {self.page_size}")
        n = need_size // self.page_size
        if n > self.free_pages.numel():
            return None
        out_pages = self.free_pages[:n]
        if not self._lazy_hook(out_pages):
            return None
        self.free_pages = self.free_pages[n:]
        idx = (out_pages[:, None] * self.page_size + torch.arange(self.page_size, dtype=torch.int64)).reshape(-1)
        return idx.to(self.device)

    def free(self, free_index: torch.Tensor) -> None:
        if free_index.numel() == 0:
            return
        pages = torch.unique(free_index.to("cpu", torch.int64) // self.page_size)
        self.free_pages = torch.cat((pages, self.free_pages))
        if self.free_pages.numel() >= self.num_pages:   # pool idle: slot order + give the memory back
            release = getattr(self._kvcache, "lazy_release", None)
            self.clear()
            if release is not None:
                release()
