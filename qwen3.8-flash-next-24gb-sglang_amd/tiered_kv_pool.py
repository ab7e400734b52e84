"""Quantized KV pools of the ``int8_g64`` / ``int4_g32`` / ``int8ring_int4`` modes, as SGLang's attention backend
sees them.

The drop-in contract (class names, constructor arguments, attribute and accessor names, the layouts of the buffers
they return and the exception types of the write guards) is that of the reference's pool classes
``MHATokenToKVPoolInt8`` (patches/kv_int8.py:69-202), ``MHATokenToKVPoolInt4`` (patches/kv_int4.py:81-227) and
``MHATokenToKVPoolTiered`` (patches/kv_tiers.py:103-229).  The implementation is organised differently:

* a pool is a set of per-layer *buffer families* keyed by name (``k``, ``v``, ``ks``, ``vs`` for the per-slot rows,
  ``rk``, ``rv``, ``rks``, ``rvs`` for the ring).  Each class only declares its family layout
  (``_slot_families``), and allocation, byte accounting, buffer descriptors and clearing are generic over the
  families;
* the per-slot families go either to torch memory or, in lazy mode, to HIP virtual-memory arenas
  (``lazy_kv.LazyKVBacking``); the ring of the tiered mode is a ``RingTier`` object that always lives in torch memory;
* ``set_kv_buffer`` is one method in the base class: guards, then ``_check_write`` (the tiered mode refuses writes
  larger than its ring), then ``_store`` (one HIP launch sequence per class, through ``sparse_attn``).

CPU offload and prefix-valid commits raise ``NotImplementedError``, as in the reference.
"""
from __future__ import annotations

import logging
import math
import os
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from .lazy_kv import LazyKVBacking
from .sparse_attn import KV_INT4_GROUP, KV_INT8_GROUP, quant_store_kv_int4, quant_store_kv_int8, quant_store_kv_tiered

logger = logging.getLogger(__name__)

_SLOT_FAMILIES = ("k", "v", "ks", "vs")      # descriptor order: payloads first, then scales


@dataclass(frozen=True)
class KvBufferDesc:
    """How the serving runtime's memory owner sees one per-slot buffer: name, shape, bytes per row, tokens per row
    (the fields of SGLang's ``KvBufferDesc`` that the reference's pools fill, patches/kv_int4.py:131-142)."""
    name: str
    shape: Tuple[int, ...]
    row_bytes: int
    tokens_per_row: int = 1


def _unit(scale) -> bool:
    """A write-time K/V scale the quantized pools accept: absent or the number 1 (they derive their own scales)."""
    return scale is None or (isinstance(scale, (int, float)) and not isinstance(scale, bool) and scale == 1)


def unwrap_write_loc(loc_info):
    """Slot tensor of a ``set_kv_buffer`` location argument: the tensor itself, the first item of a tuple / list,
    or the ``loc`` attribute of a location object (upstream ``memory_pool.unwrap_write_loc``).  Returns
    (loc, None, None) like the upstream helper."""
    if isinstance(loc_info, torch.Tensor):
        loc = loc_info
    elif isinstance(loc_info, (tuple, list)):
        loc = loc_info[0]
    else:
        loc = loc_info.loc
    return loc, None, None


def _bytes(tensors) -> int:
    return sum(t.numel() * t.element_size() for t in tensors)


def _probe_slots(loc: torch.Tensor, hi: int, where: str) -> None:
    """Bounds probe of write slots against [0, hi), the reference's ``maybe_detect_oob`` (patches/kv_tiers.py:192).
    It synchronizes the host, so it runs only with KVT_DETECT_OOB=1."""
    if not os.environ.get("KVT_DETECT_OOB") or loc.numel() == 0:
        return
    lo_seen, hi_seen = int(loc.min()), int(loc.max())
    if lo_seen < 0 or hi_seen >= hi:
        raise IndexError(f"{where}: write slots span [{lo_seen}, {hi_seen}], the pool has rows [0, {hi})")


class _QuantKVPool:
    """Per-slot quantized KV rows (NHD: [rows, heads, bytes]) with fp16 group scales; rows = size + page_size (the
    slot index ``size`` is the padding slot)."""

    MODE = "quantized"          # --kv-cache-dtype spelling, used in messages
    GROUP = 1                   # channels per stored scale
    CODE_DTYPE: Optional[torch.dtype] = None
    kv_bits: Optional[int] = None

    def __init__(self, size: int, page_size: int, dtype: torch.dtype, head_num: int, head_dim: int, layer_num: int,
                 device, enable_memory_saver: bool = False, start_layer: int = 0, v_head_dim: Optional[int] = None,
                 lazy: Optional[bool] = None, **unused):
        if dtype != self.CODE_DTYPE:
            raise ValueError(f"{type(self).__name__} stores {self.CODE_DTYPE} codes; dtype {dtype} was requested")
        self.size, self.page_size = int(size), int(page_size)
        self.dtype = self.store_dtype = dtype
        self.head_num, self.head_dim = int(head_num), int(head_dim)
        self.v_head_dim = self.head_dim if v_head_dim is None else int(v_head_dim)
        self.layer_num, self.start_layer = int(layer_num), int(start_layer)
        self.end_layer = self.start_layer + self.layer_num - 1
        self.device = device
        self.use_hnd = False
        self.kv_cache_layout = "nhd"
        self.lazy = (os.environ.get("SGLANG_KV_LAZY") == "1") if lazy is None else bool(lazy)
        self._lazy: Optional[LazyKVBacking] = None
        self._fam: Optional[Dict[str, List[torch.Tensor]]] = None
        self._allocate_slot_families()
        # per-channel smoothing constants and their inverses, fp16 [L, H, D]: identity, as served
        # (patches/kv_int4.py:95-100)
        one = lambda d: torch.ones((self.layer_num, self.head_num, d), dtype=torch.float16, device=self.device)
        self.sm_k, self.sm_v = one(self.head_dim), one(self.v_head_dim)
        self.sm_k_inv, self.sm_v_inv = one(self.head_dim), one(self.v_head_dim)

    # ------------------------------------------------------------------------------------------ layout
    def _codes_per_row(self, dim: int) -> int:
        """Bytes of codes per (slot, head) for `dim` channels."""
        raise NotImplementedError

    def _n_groups(self, dim: int, what: str) -> int:
        if dim % self.GROUP:
            raise ValueError(f"{self.MODE}: {what} {dim} does not split into {self.GROUP}-channel scale groups")
        return dim // self.GROUP

    @property
    def k_groups(self) -> int:
        return self._n_groups(self.head_dim, "head_dim")

    @property
    def v_groups(self) -> int:
        return self._n_groups(self.v_head_dim, "v_head_dim")

    def _rows(self) -> int:
        return self.size + self.page_size

    def _slot_families(self) -> Dict[str, Tuple[Tuple[int, ...], torch.dtype]]:
        """Shape and dtype of one layer's tensor of each per-slot family, in descriptor order."""
        rows, H = self._rows(), self.head_num
        return {"k": ((rows, H, self._codes_per_row(self.head_dim)), self.CODE_DTYPE),
                "v": ((rows, H, self._codes_per_row(self.v_head_dim)), self.CODE_DTYPE),
                "ks": ((rows, H, self.k_groups), torch.float16),
                "vs": ((rows, H, self.v_groups), torch.float16)}

    def _allocate_slot_families(self) -> None:
        layout = self._slot_families()
        if self.lazy:
            # the whole pool reserved as address space, the floor backed now (patches/kv_lazy.py:100-106)
            self._lazy = LazyKVBacking(self._rows(), self.size, self.page_size, self.device)
            make = self._lazy.add
        else:
            make = lambda shape, dt: torch.zeros(shape, dtype=dt, device=self.device)
        self._fam = {name: [make(*layout[name]) for _ in range(self.layer_num)] for name in _SLOT_FAMILIES}
        if self._lazy is not None:
            self._lazy.ensure_prefix(self._lazy.floor)
            logger.info("%s pool: %d slots of address space, %d backed now, commits of %d slots, %.1f KB per slot",
                        self.MODE, self.size, self._lazy.floor, self._lazy.margin,
                        self._lazy.bytes_per_token() / 1024)

    def _family(self, name: str) -> Optional[List[torch.Tensor]]:
        return None if self._fam is None else self._fam[name]

    k_buffer = property(lambda self: self._family("k"))
    v_buffer = property(lambda self: self._family("v"))
    k_scale_buffer = property(lambda self: self._family("ks"))
    v_scale_buffer = property(lambda self: self._family("vs"))

    @property
    def _kv_buffer_descs(self) -> List[KvBufferDesc]:
        """Descriptors of the per-slot buffers in registration order k0.., v0.., ks0.., vs0..: code rows as their
        own shape; scale rows as raw bytes (rows, heads * groups * 2), the way the memory owner registers them
        (names and row sizes: patches/kv_int4.py:131-142, gemv/test_kv_int4.py:311-313)."""
        out = []
        for name, (shape, dt) in self._slot_families().items():
            row_bytes = math.prod(shape[1:]) * torch.empty(0, dtype=dt).element_size()
            desc_shape = shape if dt == self.CODE_DTYPE else (shape[0], row_bytes)
            out += [KvBufferDesc(f"{name}{i}", desc_shape, row_bytes, 1) for i in range(self.layer_num)]
        return out

    def _clear_buffers(self) -> None:
        self._fam = None
        self._lazy = None

    # ------------------------------------------------------------------------------------------ accessors
    def _local(self, layer_id: int) -> int:
        return layer_id - self.start_layer

    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self._fam["k"][self._local(layer_id)]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self._fam["v"][self._local(layer_id)]

    def get_kv_buffer(self, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        i = self._local(layer_id)
        return self._fam["k"][i], self._fam["v"][i]

    def get_kv_scale_buffer(self, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        i = self._local(layer_id)
        return self._fam["ks"][i], self._fam["vs"][i]

    def get_kv_smooth_buffer(self, layer_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        i = self._local(layer_id)
        return self.sm_k[i], self.sm_v[i]

    def get_kv_size_bytes(self) -> Tuple[int, int]:
        """(K bytes, V bytes) over all layers: codes + scales."""
        f = self._fam
        return _bytes(f["k"] + f["ks"]), _bytes(f["v"] + f["vs"])

    # ------------------------------------------------------------------------------------------ write path
    def _check_write(self, loc: torch.Tensor) -> None:
        """Mode-specific refusal of a write before anything is launched."""

    def _store(self, i: int, loc, ck: torch.Tensor, cv: torch.Tensor) -> None:
        raise NotImplementedError

    def set_kv_buffer(self, layer, loc_info, cache_k: torch.Tensor, cache_v: torch.Tensor, k_scale=None,
                      v_scale=None, layer_id_override: Optional[int] = None,
                      dcp_kv_mask: Optional[torch.Tensor] = None) -> None:
        """Quantize K/V rows ([N, H, D] or [N, H * D], bf16 / fp16 / fp32) into slots `loc` of one layer
        (the layer object's layer_id, or layer_id_override as HybridLinearKVPool passes it)."""
        if dcp_kv_mask is not None:
            raise NotImplementedError(f"{self.MODE}: writes under a DCP KV mask are not supported")
        if not (_unit(k_scale) and _unit(v_scale)):
            raise ValueError(f"{self.MODE}: the pool derives its own scales; k_scale / v_scale must be 1 or None")
        loc = unwrap_write_loc(loc_info)[0]
        _probe_slots(loc, self._rows(), f"{self.MODE} set_kv_buffer")
        self._check_write(loc)
        i = self._local(layer.layer_id if layer_id_override is None else layer_id_override)
        self._store(i, loc, cache_k.view(-1, self.head_num, self.head_dim),
                    cache_v.view(-1, self.head_num, self.v_head_dim))

    def set_kv_buffer_prefix_valid(self, *args, **kwargs):
        raise NotImplementedError(f"{self.MODE}: prefix-valid commits are not supported by a quantized pool")

    def get_cpu_copy(self, indices, mamba_indices=None):
        raise NotImplementedError(f"{self.MODE}: no CPU offload for quantized pools")

    def load_cpu_copy(self, kv_cache_cpu, indices, mamba_indices=None):
        raise NotImplementedError(f"{self.MODE}: no CPU offload for quantized pools")

    # ------------------------------------------------------------------------------------------ lazy backing
    # (patches/kv_lazy.py:113-175); no-ops on an eagerly allocated pool
    @property
    def lazy_backed_tokens(self) -> int:
        """Slots [0, n) have memory behind them (all rows of an eager pool)."""
        return self._rows() if self._lazy is None else self._lazy.backed_tokens

    def lazy_ensure(self, num_tokens: int) -> None:
        """Back slots [0, num_tokens + margin) in margin steps (RuntimeError when the device cannot)."""
        if self._lazy is not None:
            self._lazy.ensure(num_tokens)

    def lazy_release(self) -> None:
        """Return the backing beyond the floor to the driver (call when no slot is in use)."""
        if self._lazy is not None:
            self._lazy.release()


class MHATokenToKVPoolInt8(_QuantKVPool):
    """``int8_g64``: int8 codes [rows, H, D] + fp16 absmax/127 scales per (slot, head, 64 channels)
    (patches/kv_int8.py:69-202)."""

    MODE = "int8_g64"
    GROUP = KV_INT8_GROUP
    CODE_DTYPE = torch.int8
    kv_bits = 8

    def _codes_per_row(self, dim: int) -> int:
        return dim

    def _store(self, i, loc, ck, cv):
        ks, vs = self.get_kv_scale_buffer(self.start_layer + i)
        quant_store_kv_int8(ck, cv, loc, self._fam["k"][i], self._fam["v"][i], ks, vs, self.sm_k_inv[i],
                            self.sm_v_inv[i])


class MHATokenToKVPoolInt4(_QuantKVPool):
    """``int4_g32``: two channels per byte [rows, H, D / 2] (even channel in the low nibble, code + 8) + fp16
    absmax/7 scales per (slot, head, 32 channels) (patches/kv_int4.py:81-227)."""

    MODE = "int4_g32"
    GROUP = KV_INT4_GROUP
    CODE_DTYPE = torch.uint8
    kv_bits = 4

    def _codes_per_row(self, dim: int) -> int:
        if dim % 2:
            raise ValueError(f"{self.MODE}: odd head dim {dim} cannot be packed two channels per byte")
        return dim // 2

    def _store(self, i, loc, ck, cv):
        ks, vs = self.get_kv_scale_buffer(self.start_layer + i)
        quant_store_kv_int4(ck, cv, loc, self._fam["k"][i], self._fam["v"][i], ks, vs, self.sm_k_inv[i],
                            self.sm_v_inv[i])


def ring_slots_from_env() -> int:
    """Ring rows R of the tiered mode from SGLANG_KV_TIERS_W (default 8192).  The ring row of a slot is
    slot & (R - 1), so R must be a power of two; anything else is a ValueError (patches/kv_tiers.py:91-100)."""
    text = os.environ.get("SGLANG_KV_TIERS_W", "8192").strip()
    if not text.lstrip("-").isdigit():
        raise ValueError(f"SGLANG_KV_TIERS_W: expected an integer ring size, got {text!r}")
    r = int(text)
    if r < 1 or bin(r).count("1") != 1:
        raise ValueError(f"SGLANG_KV_TIERS_W: the ring size must be a power of two >= 1, got {r}")
    return r


class RingTier:
    """The hot tier of ``int8ring_int4``: per layer, INT8-G codes int8 [R, H, D] and fp16 scales [R, H, D / G] of the
    slots most recently written into each ring row, plus the owner table int32 [R] shared by all layers
    (owner[r] = the slot whose row r holds, -1 for none).  Always plain device memory, allocated once: the decode
    graph captures its addresses (patches/kv_tiers.py:63-74)."""

    def __init__(self, rows: int, layers: int, heads: int, head_dim: int, v_head_dim: int, group: int, device):
        def fam(dim, dt, per):
            return [torch.zeros((rows, heads, dim // per), dtype=dt, device=device) for _ in range(layers)]
        self.rows, self.group = rows, group
        self.k, self.v = fam(head_dim, torch.int8, 1), fam(v_head_dim, torch.int8, 1)
        self.ks, self.vs = fam(head_dim, torch.float16, group), fam(v_head_dim, torch.float16, group)
        self.owner = torch.full((rows,), -1, dtype=torch.int32, device=device)

    def layer(self, i: int):
        return self.k[i], self.v[i], self.ks[i], self.vs[i]

    def nbytes(self) -> Tuple[int, int]:
        """(K side incl. the owner table, V side)."""
        return _bytes(self.k + self.ks + [self.owner]), _bytes(self.v + self.vs)


class MHATokenToKVPoolTiered(MHATokenToKVPoolInt4):
    """``int8ring_int4``: the INT4-G32 rows of every slot (inherited; written on every write) plus a ``RingTier``
    whose row slot & (R - 1) holds the INT8-G64 form of the last slot written there (patches/kv_tiers.py:103-229).
    Readers take the ring row when owner[slot & (R - 1)] == slot, else the INT4 row.  ``kv_bits`` stays 4 and
    ``kv_tiered`` is the backend's dispatch key; the ring is not a per-slot buffer, so it has no descriptor and
    stays out of the lazy backing."""

    MODE = "int8ring_int4"
    RING_GROUP = KV_INT8_GROUP
    kv_tiered = True

    def __init__(self, *args, **kwargs):
        self._ring: Optional[RingTier] = None
        super().__init__(*args, **kwargs)
        R = ring_slots_from_env()
        if R > self.size:
            raise ValueError(f"{self.MODE}: a ring of {R} rows needs a pool of at least {R} slots (pool: {self.size})")
        for d in (self.head_dim, self.v_head_dim):
            if d % self.RING_GROUP:
                raise ValueError(f"{self.MODE}: head dim {d} does not split into {self.RING_GROUP}-channel ring groups")
        self.ring_slots = R
        self._ring = RingTier(R, self.layer_num, self.head_num, self.head_dim, self.v_head_dim, self.RING_GROUP,
                              self.device)
        kb, vb = self._ring.nbytes()
        logger.info("%s pool: INT8-G%d ring of %d rows per layer over INT4-G%d rows; ring %.1f MiB incl. the %d-byte "
                    "owner table", self.MODE, self.RING_GROUP, R, self.GROUP, (kb + vb) / 2 ** 20,
                    self._ring.owner.numel() * 4)

    def _ring_family(self, name: str):
        return None if self._ring is None else getattr(self._ring, name)

    ring_k = property(lambda self: self._ring_family("k"))
    ring_v = property(lambda self: self._ring_family("v"))
    ring_ks = property(lambda self: self._ring_family("ks"))
    ring_vs = property(lambda self: self._ring_family("vs"))
    ring_owner = property(lambda self: self._ring_family("owner"))

    @property
    def ring_mask(self) -> int:
        return self.ring_slots - 1

    def get_kv_size_bytes(self) -> Tuple[int, int]:
        """Per-slot rows plus the ring (the owner table counts on the K side)."""
        kb, vb = super().get_kv_size_bytes()
        if self._ring is not None:
            rk, rv = self._ring.nbytes()
            kb, vb = kb + rk, vb + rv
        return kb, vb

    def _clear_buffers(self) -> None:
        super()._clear_buffers()
        self._ring = None

    def get_kv_ring_buffer(self, layer_id: int):
        """(ring_k, ring_v, ring_ks, ring_vs) of one layer."""
        return self._ring.layer(self._local(layer_id))

    def get_kv_ring_owner(self) -> torch.Tensor:
        return self._ring.owner

    def _check_write(self, loc: torch.Tensor) -> None:
        # a write of more tokens than ring rows would alias itself in the ring: refused as a misconfiguration
        if loc.numel() > self.ring_slots:
            raise ValueError(f"{self.MODE}: a write of {loc.numel()} tokens does not fit the {self.ring_slots}-row "
                             f"ring")

    def _store(self, i, loc, ck, cv):
        ks, vs = self.get_kv_scale_buffer(self.start_layer + i)
        rk, rv, rks, rvs = self._ring.layer(i)
        quant_store_kv_tiered(ck, cv, loc, self._fam["k"][i], self._fam["v"][i], ks, vs, rk, rv, rks, rvs,
                              self._ring.owner, self.sm_k_inv[i], self.sm_v_inv[i], self.ring_mask)

    def lazy_release(self) -> None:
        """Release the lazy backing and forget every ring owner (patches/kv_tiers.py:224-229): a reader then takes
        the INT4 row of any slot until it is written again."""
        super().lazy_release()
        if self._ring is not None:
            self._ring.owner.fill_(-1)


class HybridLinearKVPool:
    """The parts of SGLang's ``HybridLinearKVPool`` the quantized pools need: a model with linear-attention layers
    keeps its full-attention layers' KV in ``full_kv_pool`` under local layer ids, and the wrapper translates global
    layer ids and forwards the accessors, including the ring and smoothing ones the quantized modes add
    (patches/kv_tiers.py:787-808; smoothing forwarder: flat patch sglang/qwen4exp-serving-73a255206f.patch:4351-4355).
    """

    def __init__(self, full_kv_pool, full_attention_layer_ids):
        self.full_kv_pool = full_kv_pool
        self.full_attention_layer_id_mapping = {int(g): i + full_kv_pool.start_layer
                                                for i, g in enumerate(full_attention_layer_ids)}

    def _transfer_full_attention_id(self, layer_id: int) -> int:
        local = self.full_attention_layer_id_mapping.get(int(layer_id))
        if local is None:
            raise ValueError(f"layer {layer_id} is not a full-attention layer of this model")
        return local

    def _wait_for_layer(self, layer_id: int) -> None:
        """Layer-wise KV transfer hook of the upstream class; nothing is transferred here."""

    def _fwd(self, name: str, layer_id: int):
        self._wait_for_layer(layer_id)
        return getattr(self.full_kv_pool, name)(self._transfer_full_attention_id(layer_id))

    def get_key_buffer(self, layer_id: int):
        return self._fwd("get_key_buffer", layer_id)

    def get_value_buffer(self, layer_id: int):
        return self._fwd("get_value_buffer", layer_id)

    def get_kv_buffer(self, layer_id: int):
        return self._fwd("get_kv_buffer", layer_id)

    def get_kv_scale_buffer(self, layer_id: int):
        return self._fwd("get_kv_scale_buffer", layer_id)

    def get_kv_smooth_buffer(self, layer_id: int):
        return self._fwd("get_kv_smooth_buffer", layer_id)

    def get_kv_ring_buffer(self, layer_id: int):
        return self._fwd("get_kv_ring_buffer", layer_id)

    def get_kv_ring_owner(self):
        return self.full_kv_pool.get_kv_ring_owner()

    def set_kv_buffer(self, layer, loc_info, cache_k, cache_v, k_scale=None, v_scale=None, **kwargs):
        kwargs.pop("layer_id_override", None)
        local = self._transfer_full_attention_id(layer.layer_id)
        self.full_kv_pool.set_kv_buffer(None, loc_info, cache_k, cache_v, k_scale, v_scale,
                                        layer_id_override=local, **kwargs)


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
