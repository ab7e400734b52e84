"""Position-indexed tiered KV cache (evict mode) and the decode-attention entry points.

The reference writes every token twice (INT4 row + INT8 ring row, slot-indexed ring, patches/kv_tiers.py:4-16).
This module adds the mode the reference specifies but never built: the ring holds the newest R positions of each
sequence (row = ring_base + position mod R) and a token leaving the ring is requantized INT8 -> INT4-G32 into the
page of its position (docs/KV_TIERS_PLAN.md:53, :63-67, :82).  Pages come from a host free list in a seeded
random order and are recorded in a per-sequence page table (int32 [S, max_pages]) by a device kernel.

    cache = PosTieredCache(layers, H, D, n_pages, ring_total, max_seqs, max_pages, device)
    s = cache.add_seq(ring_len=8192)
    plan = cache.plan_append([s], [n])      # positions, new pages (page-table update launch)
    for layer: cache.append(layer, plan, k, v)
    cache.commit(plan)
    out = kvt_decode_attn(cache, layer, q)  # split-K over INT4 pages + INT8 ring
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib

PAGE = 64
G4 = 32


class PageAllocator:
    """Host free list of physical INT4 pages in a seeded random order ("physical pages randomly permuted from
    seed"): pop() hands them out in that order."""

    def __init__(self, n_pages: int, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        self.free: List[int] = torch.randperm(n_pages, generator=g).tolist()
        self.next = 0

    def pop(self) -> int:
        if self.next >= len(self.free):
            raise RuntimeError("INT4 page pool exhausted")
        p = self.free[self.next]
        self.next += 1
        return p

    @property
    def n_free(self) -> int:
        return len(self.free) - self.next


@dataclass
class AppendPlan:
    seq_ids: torch.Tensor      # int32 [N] device
    positions: torch.Tensor    # int64 [N] device
    counts: List[int]
    seqs: List[int]

    @property
    def n(self) -> int:
        return int(self.seq_ids.numel())


@dataclass
class DevicePlan(AppendPlan):
    """A fixed append layout (seqs[j] appends counts[j] tokens per call) whose positions, page pops and length
    updates are computed on the device by launch_plan: one kernel, no host work, capturable in a HIP graph.  The
    seq_ids / positions buffers are rewritten by every launch."""
    seqs_dev: Optional[torch.Tensor] = None    # int32 [n]
    cu_dev: Optional[torch.Tensor] = None      # int32 [n + 1]


class PosTieredCache:
    """Per layer: INT4 pool k4/v4 uint8 [n_pages * 64, H, D // 2] + fp16 scales [.., H, D // 32], INT8 ring rk/rv
    int8 [ring_total, H, D] + fp16 scales [ring_total, H, D // group8].  Shared by all layers: per-sequence ring
    placement (ring_base, ring_len, ring_start), lengths and the page table."""

    def __init__(self, layers: int, H: int, D: int, n_pages: int, ring_total: int, max_seqs: int, max_pages: int,
                 device="cuda", group8: int = 64, page_seed: int = 0, sm: bool = False):
        assert D == 256, "the kernels are built for head_dim 256"
        assert group8 in (64, D)
        self.L, self.H, self.D, self.group8 = layers, H, D, group8
        self.device = torch.device(device)
        rows = n_pages * PAGE
        z = dict(device=self.device)
        self.k4 = [torch.zeros(rows, H, D // 2, dtype=torch.uint8, **z) for _ in range(layers)]
        self.v4 = [torch.zeros(rows, H, D // 2, dtype=torch.uint8, **z) for _ in range(layers)]
        self.ks4 = [torch.zeros(rows, H, D // G4, dtype=torch.float16, **z) for _ in range(layers)]
        self.vs4 = [torch.zeros(rows, H, D // G4, dtype=torch.float16, **z) for _ in range(layers)]
        self.rk = [torch.zeros(ring_total, H, D, dtype=torch.int8, **z) for _ in range(layers)]
        self.rv = [torch.zeros(ring_total, H, D, dtype=torch.int8, **z) for _ in range(layers)]
        self.rks = [torch.zeros(ring_total, H, D // group8, dtype=torch.float16, **z) for _ in range(layers)]
        self.rvs = [torch.zeros(ring_total, H, D // group8, dtype=torch.float16, **z) for _ in range(layers)]
        self.sm_k = self.sm_v = self.sm_k_inv = self.sm_v_inv = None   # identity smoothing
        self.ring_total = ring_total
        self.max_seqs, self.max_pages = max_seqs, max_pages
        self.page_table = torch.full((max_seqs, max_pages), -1, dtype=torch.int32, **z)
        self.ring_base = torch.zeros(max_seqs, dtype=torch.int64, **z)
        self.ring_len = torch.ones(max_seqs, dtype=torch.int32, **z)
        self.ring_start = torch.zeros(max_seqs, dtype=torch.int64, **z)
        self.seq_lens = torch.zeros(max_seqs, dtype=torch.int32, **z)
        self.alloc = PageAllocator(n_pages, page_seed)
        # the same free list on the device, for plans computed there (kvt_append_plan): the permutation, the index of
        # the next free page (kept equal to alloc.next: host pops are pushed before a device plan runs) and a status
        # word the plan kernel raises when it could not give a page (1: pool exhausted, 2: page-table row full)
        self.free_list = torch.tensor(self.alloc.free, dtype=torch.int32, device=self.device)
        self.free_head = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.plan_status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._dev_head = 0
        self._ring_used = 0
        # bumped by every change of the sequence state (lengths, rings, page table); a decode plan records it
        self.version = 0
        # set once launch_plan has been captured into a graph: from then on replays may advance the device state past
        # the host mirror at any time, so host-side planning first reads the device state back (sync_host)
        self._device_may_advance = False
        # host mirror
        self.h_len: List[int] = []
        self.h_ring: List[tuple] = []       # (base, len, start)
        self.h_pages: List[List[int]] = []
        self.h_shared: List[int] = []       # shared prefix pages per sequence

    # -- sequences
    @property
    def n_seqs(self) -> int:
        return len(self.h_len)

    def add_seq(self, ring_len: int, ring_start: int = 0, shared_pages: Sequence[int] = ()) -> int:
        """New sequence with its own ring of ring_len rows (a power of two).  Positions below ring_start come from
        shared_pages (physical INT4 pages already holding a common prefix; paged-prefix reuse)."""
        assert ring_len > 0 and ring_len & (ring_len - 1) == 0, "ring_len must be a power of two"
        assert len(shared_pages) * PAGE >= ring_start and ring_start % PAGE == 0
        self._catch_up()
        self.version += 1
        s = self.n_seqs
        assert s < self.max_seqs
        if self._ring_used + ring_len > self.ring_total:
            raise RuntimeError("ring rows exhausted")
        base = self._ring_used
        self._ring_used += ring_len
        self.h_len.append(ring_start)
        self.h_ring.append((base, ring_len, ring_start))
        self.h_pages.append(list(shared_pages))
        self.h_shared.append(len(shared_pages))
        self.ring_base[s] = base
        self.ring_len[s] = ring_len
        self.ring_start[s] = ring_start
        self.seq_lens[s] = ring_start
        if shared_pages:
            self.page_table[s, :len(shared_pages)] = torch.tensor(list(shared_pages), dtype=torch.int32)
        return s

    def hot_start(self, s: int) -> int:
        base, R, start = self.h_ring[s]
        return max(start, self.h_len[s] - R)

    # -- write path
    def plan_append(self, seqs: Sequence[int], counts: Sequence[int]) -> AppendPlan:
        """Positions of the next counts[i] tokens of seqs[i]; pages the evictions of this append enter for the first
        time are popped from the allocator and written into the device page table (one small launch)."""
        if len(set(seqs)) != len(list(seqs)):
            raise ValueError("a plan lists each sequence once")
        self._catch_up()
        self.version += 1
        sid, pos, upd_s, upd_l, upd_p = [], [], [], [], []
        for s, n in zip(seqs, counts):
            base, R, start = self.h_ring[s]
            assert 0 <= n <= R, f"{n} tokens in one append exceed the ring of {R}"
            L0 = self.h_len[s]
            for p in range(L0, L0 + n):
                e = p - R
                if e >= start and e % PAGE == 0:
                    lp = e // PAGE
                    assert lp == len(self.h_pages[s]), "page table out of order"
                    if lp >= self.max_pages:
                        raise RuntimeError("page table row full")
                    phys = self.alloc.pop()
                    self.h_pages[s].append(phys)
                    upd_s.append(s)
                    upd_l.append(lp)
                    upd_p.append(phys)
            sid.extend([s] * n)
            pos.extend(range(L0, L0 + n))
        dev = self.device
        if upd_s:
            upd = torch.tensor([upd_s, upd_l, upd_p], dtype=torch.int32).to(dev)
            _lib.call("kvt_page_table_update", self.page_table.data_ptr(), self.page_table.stride(0), len(upd_s),
                      upd[0].data_ptr(), upd[1].data_ptr(), upd[2].data_ptr(), _lib.stream())
        self._push_free_head()
        return AppendPlan(torch.tensor(sid, dtype=torch.int32).to(dev), torch.tensor(pos, dtype=torch.int64).to(dev),
                          list(counts), list(seqs))

    def plan_device(self, seqs: Sequence[int], counts: Sequence[int]) -> DevicePlan:
        """A device plan of the append layout `seqs[j]` appends `counts[j]` tokens (distinct sequences, each count at
        most its ring): built once, then launched by launch_plan every step, e.g. one token per sequence for decode."""
        seqs, counts = list(seqs), list(counts)
        if len(set(seqs)) != len(seqs):
            raise ValueError("a plan lists each sequence once")
        if len(seqs) > 1024:
            raise ValueError("a device plan covers at most 1024 sequences")
        for s, n in zip(seqs, counts):
            assert 0 <= s < self.n_seqs, f"unknown sequence {s}"
            R = self.h_ring[s][1]
            assert 0 <= n <= R, f"{n} tokens in one append exceed the ring of {R}"
        cu = [0]
        for n in counts:
            cu.append(cu[-1] + n)
        dev = self.device
        self._push_free_head()   # (a plan is built eagerly, before any capture that launches it)
        return DevicePlan(torch.zeros(cu[-1], dtype=torch.int32, device=dev),
                          torch.zeros(cu[-1], dtype=torch.int64, device=dev), counts, seqs,
                          torch.tensor(seqs, dtype=torch.int32, device=dev), torch.tensor(cu, dtype=torch.int32, device=dev))

    def _new_pages(self, s: int, n: int) -> range:
        """Logical pages that appending n tokens to sequence s enters for the first time (closed form)."""
        base, R, start = self.h_ring[s]
        L0 = self.h_len[s]
        e0, e1 = max(start, L0 - R), L0 + n - R
        lp0 = (e0 + PAGE - 1) // PAGE
        return range(lp0, (e1 + PAGE - 1) // PAGE) if e1 > e0 else range(lp0, lp0)

    def _catch_up(self) -> None:
        """Before planning on the host: if graph replays of a captured device plan may have advanced the lengths, page
        table and free-list head, read them back first (the host mirror and allocator would otherwise hand out pages
        the device already gave away)."""
        if self._device_may_advance and not torch.cuda.is_current_stream_capturing():
            self.sync_host()

    def _push_free_head(self) -> None:
        """Make the device free-list head equal the host allocator's position (pages popped on the host)."""
        if self._dev_head != self.alloc.next:
            self.free_head.fill_(self.alloc.next)
            self._dev_head = self.alloc.next

    def launch_plan(self, plan: DevicePlan) -> None:
        """Enqueue the device plan (positions, page pops into the page table, seq_lens += counts); capturable.  Run
        eagerly, it first pushes host-side pops to the device free-list head, checks capacity (RuntimeError, as the
        host planner) and then advances the host mirror (lengths, pages) in closed form; under graph capture the
        mirror is left as it is -- sync_host() reads the device state back after replays."""
        capturing = torch.cuda.is_current_stream_capturing()
        self.version += 1
        if capturing:
            self._device_may_advance = True
        else:
            self._catch_up()
            need = sum(len(self._new_pages(s, n)) for s, n in zip(plan.seqs, plan.counts))
            if need > self.alloc.n_free:
                raise RuntimeError("INT4 page pool exhausted")
            for s, n in zip(plan.seqs, plan.counts):
                r = self._new_pages(s, n)
                if len(r) and r.stop > self.max_pages:
                    raise RuntimeError("page table row full")
            self._push_free_head()
        _lib.call("kvt_append_plan", len(plan.seqs), plan.seqs_dev.data_ptr(), plan.cu_dev.data_ptr(),
                  self.seq_lens.data_ptr(), self.ring_len.data_ptr(), self.ring_start.data_ptr(),
                  self.page_table.data_ptr(), self.page_table.stride(0), self.max_pages, self.free_list.data_ptr(),
                  self.free_list.numel(), self.free_head.data_ptr(), plan.seq_ids.data_ptr(),
                  plan.positions.data_ptr(), self.plan_status.data_ptr(), _lib.stream())
        if not capturing:
            for s, n in zip(plan.seqs, plan.counts):
                for lp in self._new_pages(s, n):
                    assert lp == len(self.h_pages[s]), "page table out of order"
                    self.h_pages[s].append(self.alloc.pop())
                self.h_len[s] += n
            self._dev_head = self.alloc.next

    def sync_host(self) -> None:
        """Rebuild the host mirror (lengths, page lists, allocator position) from the device after graph replays of
        launch_plan (synchronizes the device).  Raises RuntimeError if a device plan could not give a page."""
        status = int(self.plan_status.item())
        if status:
            raise RuntimeError(f"a device append plan could not give a page (status {status}: 1 = pool exhausted, "
                               "2 = page-table row full)")
        lens = self.seq_lens[:self.n_seqs].tolist()
        pt = self.page_table[:self.n_seqs].tolist()
        for s in range(self.n_seqs):
            self.h_len[s] = int(lens[s])
            self.h_pages[s] = [int(p) for p in pt[s][:self._page_count(s)]]
        self.alloc.next = int(self.free_head.item())
        self._dev_head = self.alloc.next
        self.version += 1

    def _page_count(self, s: int) -> int:
        """Entries of sequence s's page-table row: its shared prefix pages, or every page an evicted position has
        entered (positions below hot_start), whichever is more."""
        return max(self.h_shared[s], -(-self.hot_start(s) // PAGE))

    def append(self, layer: int, plan: AppendPlan, k: torch.Tensor, v: torch.Tensor) -> None:
        """Quantize-append the plan's tokens (k, v: [N, H, D] bf16/fp16/fp32) into layer `layer`."""
        N = plan.n
        assert k.shape == (N, self.H, self.D) and v.shape == k.shape and k.stride(2) == 1 and v.stride(2) == 1
        assert k.dtype == v.dtype and k.dtype in _lib.DTYPE_CODE
        if N == 0:
            return
        _lib.require_device(k, v)
        _lib.call("kvt_append_evict", k.data_ptr(), v.data_ptr(), _lib.DTYPE_CODE[k.dtype], k.stride(0), k.stride(1),
                  v.stride(0), v.stride(1), plan.seq_ids.data_ptr(), plan.positions.data_ptr(), N, self.H, self.D,
                  self.k4[layer].data_ptr(), self.v4[layer].data_ptr(), self.ks4[layer].data_ptr(),
                  self.vs4[layer].data_ptr(), self.rk[layer].data_ptr(), self.rv[layer].data_ptr(),
                  self.rks[layer].data_ptr(), self.rvs[layer].data_ptr(), self.ring_base.data_ptr(),
                  self.ring_len.data_ptr(), self.ring_start.data_ptr(), self.page_table.data_ptr(),
                  self.page_table.stride(0), None, None, self.group8, _lib.stream())

    def commit(self, plan: AppendPlan) -> None:
        """Advance the sequence lengths after every layer has been written (a device plan advanced them already)."""
        if isinstance(plan, DevicePlan):
            return
        for s, n in zip(plan.seqs, plan.counts):
            self.h_len[s] += n
        self.version += 1
        idx = torch.tensor(plan.seqs, dtype=torch.int64)
        add = torch.tensor(plan.counts, dtype=torch.int32)
        self.seq_lens.index_add_(0, idx.to(self.device), add.to(self.device))

    # -- byte accounting (algorithmic HBM bytes of one decode step over one layer)
    def kv_bytes(self, seqs: Optional[Sequence[int]] = None) -> int:
        """KV payload + scale bytes a decode step reads per layer: hot tokens x (2 D + 2 * 2 D / group8) and cold
        tokens x (D + 2 * 2 D / 32), per KV head (K and V)."""
        seqs = range(self.n_seqs) if seqs is None else seqs
        hot_b = self.H * 2 * (self.D + 2 * (self.D // self.group8))
        cold_b = self.H * 2 * (self.D // 2 + 2 * (self.D // G4))
        tot = 0
        for s in seqs:
            hs = self.hot_start(s)
            tot += (self.h_len[s] - hs) * hot_b + hs * cold_b
        return tot

    def append_bytes(self, n: int, n_evicted: int, in_bytes: int = 2) -> int:
        """HBM bytes one append of n tokens moves per layer when n_evicted of them overwrite a ring row that goes
        to an INT4 page: K and V inputs (in_bytes per element) read, INT8 rows + scales written, and per eviction
        the INT8 row + scales read and the INT4 row + scales written; plus the sequence id and position per token."""
        ring_row = self.H * 2 * (self.D + 2 * (self.D // self.group8))
        pool_row = self.H * 2 * (self.D // 2 + 2 * (self.D // G4))
        return n * (self.H * 2 * self.D * in_bytes + ring_row + 12) + n_evicted * (ring_row + pool_row)


def _choose_chunk(max_len: int, items: int, lo: int = 64, hi: int = 512) -> int:
    """Tokens per split for the reference-precision kernel: enough work items to fill the chip (>= 512 blocks),
    at most hi tokens each."""
    want = max(1, 512 // max(1, items))
    c = max(lo, min(hi, -(-max_len // want)))
    return int(min(hi, 1 << (c - 1).bit_length()))


ROWS_MIN_POS = 64   # positions per split of the full-row kernel at least (a block has 8 wavefronts)


def _rows_kernel(H: int, Hq: int) -> bool:
    """The full-row split-K kernel serves two KV heads with up to 8 q heads each (a wavefront computes both heads of a
    position); other shapes take the head-wise kernel."""
    return H == 2 and Hq % H == 0 and Hq // H <= 8


def _choose_splits_mfma(max_len: int, items: int, blocks: int = 256, min_pos: int = 256) -> int:
    """Splits per work item of the MFMA kernels (an item is a sequence for the full-row kernel, a (sequence, KV head)
    for the head-wise one): about `blocks` blocks in all (one 8-wavefront block per CU on 256 CUs), each with at least
    min_pos positions."""
    n = -(-blocks // max(1, items))
    return int(max(1, min(n, -(-max_len // min_pos))))


HOT_COST4 = 7   # a ring position's share of a split (the kernels' kHotCost4; a paged position costs 4)


def _split_counts_mfma(lens: Sequence[int], items_per_seq: int, blocks: int = 256, min_pos: int = 256,
                       hot: Optional[Sequence[int]] = None) -> List[int]:
    """Per-sequence split counts of the MFMA kernels for a ragged batch: at most blocks // items_per_seq splits per
    KV-head item in all (one block per CU: one block more than the CUs would run as a second wave), shared in
    proportion to each sequence's cost -- 4 per paged position, HOT_COST4 per ring position (hot[i] ring positions
    of sequence i; all paged if hot is None) -- by largest remainders; each sequence at least 1 split and at most one
    per min_pos positions."""
    S = len(lens)
    per = max(1, blocks // max(1, items_per_seq))
    hot = hot if hot is not None else [0] * S
    w = [4 * (L - h) + HOT_COST4 * h for L, h in zip(lens, hot)]
    caps = [max(1, -(-L // min_pos)) for L in lens]
    tot = sum(w)
    if tot <= 0:
        return [1] * S
    raw = [per * x / tot for x in w]
    counts = [max(1, min(cap, int(r))) for r, cap in zip(raw, caps)]
    left = per - sum(counts)
    while left > 0:
        open_ = [i for i in range(S) if counts[i] < caps[i]]
        if not open_:
            break
        open_.sort(key=lambda i: raw[i] - counts[i], reverse=True)
        for i in open_[:left]:
            counts[i] += 1
        left = per - sum(counts)
    return counts


def _hot_counts(cache: "PosTieredCache", S: int) -> List[int]:
    """Ring (INT8) positions of each of the first S sequences, from the host mirror."""
    return [cache.h_len[s] - min(cache.h_len[s], cache.hot_start(s)) for s in range(S)]


def _decode_grid(cache: "PosTieredCache", Hq: int, splits: Optional[int], ws: dict, device):
    """(n_chunks, split_map, split_counts, n_map, rows) of an MFMA decode: uniform splits, or for more than one
    sequence a split map with counts in proportion to the lengths; rows = the full-row kernel serves the shape."""
    S, H = cache.n_seqs, cache.H
    rows = _rows_kernel(H, Hq)
    items, min_pos = (1, ROWS_MIN_POS) if rows else (H, 256)
    if splits is None and S > 1:
        counts = _split_counts_mfma(cache.h_len[:S], items, min_pos=min_pos, hot=_hot_counts(cache, S))
        split_map, split_counts, counts = _split_map(counts, ws, device)
        return max(counts), split_map, split_counts, sum(counts), rows
    max_len = max(cache.h_len) if S else 0
    n = splits if splits is not None else _choose_splits_mfma(max_len, S * items, min_pos=min_pos)
    return int(n), None, None, 0, rows


def decode_split_counts(cache: "PosTieredCache", Hq: int) -> List[int]:
    """The per-sequence split counts kvt_decode_attn(impl="mfma") gives a ragged batch of the cache's current lengths
    (for callers that prepare a split map themselves, e.g. for the no-allocation entry point)."""
    rows = _rows_kernel(cache.H, Hq)
    items, min_pos = (1, ROWS_MIN_POS) if rows else (cache.H, 256)
    return _split_counts_mfma(cache.h_len[:cache.n_seqs], items, min_pos=min_pos, hot=_hot_counts(cache, cache.n_seqs))


@dataclass
class DecodePlan:
    """One decode step's plan for the full-row kernel (kvt_decode_plan): every block's position ranges and the pool
    rows of its first tiles, built on the device from the cache's current lengths, ring placement and page table, and
    shared by the step's layers.  Valid until the cache's sequence state changes (an append, a new sequence, a page
    table change): kvt_decode_attn refuses a plan older than the cache (ValueError), and a block whose plan entry does
    not match the sequence's current length or ring placement computes its ranges itself."""
    entries: torch.Tensor                  # int32 [blocks, 64]
    n_chunks: int                          # partial slots per (sequence, KV head)
    split_map: Optional[torch.Tensor]
    split_counts: Optional[torch.Tensor]
    n_map: int
    Hq: int
    version: int


def kvt_decode_plan(cache: "PosTieredCache", Hq: int, splits: Optional[int] = None,
                    workspace: Optional[dict] = None) -> DecodePlan:
    """Build the decode plan of the cache's current state for queries of Hq heads (one small launch; capturable: in a
    HIP graph the plan is rebuilt from the device state at every replay).  Plans exist for the full-row kernel's
    shapes (two KV heads, up to 8 q heads each)."""
    S = cache.n_seqs
    if not _rows_kernel(cache.H, Hq):
        raise ValueError(f"decode plans serve the full-row kernel (2 KV heads, <= 8 q heads each), not {Hq} / {cache.H}")
    if S == 0:
        raise ValueError("decode plan of an empty cache")
    ws = workspace if workspace is not None else {}
    n_chunks, split_map, split_counts, n_map, _ = _decode_grid(cache, Hq, splits, ws, cache.device)
    blocks = n_map if split_map is not None else S * n_chunks
    ent = ws.get("decode_plan")
    if ent is None or ent.numel() < blocks * 64 or ent.device != cache.device:
        ent = torch.empty(blocks * 64, dtype=torch.int32, device=cache.device)
        ws["decode_plan"] = ent
    _lib.call("kvt_decode_plan", cache.seq_lens.data_ptr(), cache.ring_len.data_ptr(), cache.ring_start.data_ptr(),
              cache.ring_base.data_ptr(), cache.page_table.data_ptr(), cache.page_table.stride(0), S, n_chunks,
              _lib.ptr(split_map), n_map, ent.data_ptr(), _lib.stream())
    return DecodePlan(ent, n_chunks, split_map, split_counts, n_map, Hq, cache.version)


def _split_map(counts: List[int], ws: dict, device) -> Tuple[torch.Tensor, torch.Tensor, List[int]]:
    """Device split map {sequence, index, count} per split, the per-sequence counts on the device and as a list,
    cached in the workspace while the counts stay the same (lengths grow by one per step; the counts change rarely).
    Under graph capture a cached map is kept even if the lengths now suggest other counts: the kernel reads the
    current lengths, so any split map gives the same result (the counts only steer the balance)."""
    key = ("split_map", tuple(counts))
    hit = ws.get("split_map_key")
    if hit is not None and hit != key and torch.cuda.is_current_stream_capturing():
        return ws["split_map"], ws["split_counts"], list(hit[1])
    if hit != key:
        rows = [(b, c, n) for b, n in enumerate(counts) for c in range(n)]
        ws["split_map"] = torch.tensor(rows, dtype=torch.int32).reshape(-1).to(device)
        ws["split_counts"] = torch.tensor(counts, dtype=torch.int32).to(device)
        ws["split_map_key"] = key
    return ws["split_map"], ws["split_counts"], list(counts)


def kvt_decode_attn(cache: PosTieredCache, layer: int, q: torch.Tensor, out: Optional[torch.Tensor] = None,
                    impl: str = "ref", chunk: Optional[int] = None, max_len: Optional[int] = None,
                    out_dtype: torch.dtype = torch.float32, workspace: Optional[dict] = None,
                    events: Optional[list] = None, splits: Optional[int] = None,
                    deterministic: bool = False, tile_order: Optional[str] = None,
                    plan: Optional[DecodePlan] = None, headwise: bool = False, check_q: bool = True,
                    partials_only: bool = False) -> Optional[torch.Tensor]:
    """Decode attention of one query token per sequence over the tiered cache of `layer`.

    q: bf16 [S, Hq, D] (S = cache.n_seqs); returns out [S, Hq, D] (fp32 or bf16) = softmax(q K^T / sqrt(D)) V over
    every position of each sequence, K/V dequantized from the INT4 pages (positions < hot_start) and the INT8 ring.
    impl "ref": splits of `chunk` positions; impl "mfma": `splits` equal-cost splits per sequence (full-row kernel:
    two KV heads with up to 8 q heads each, both heads per block) or per (sequence, KV head) (head-wise kernel: the
    other shapes, or headwise=True), or, by default for more than one sequence, split counts in proportion to each
    sequence's length.
    plan (impl "mfma", full-row kernel): the step's DecodePlan (kvt_decode_plan) -- its grid replaces `splits`, and
    every block starts from its plan entry instead of computing its ranges; a plan older than the cache's state raises
    ValueError.
    events: if a list, timing events (start, after the split-K kernel, after the combine) are appended.
    partials_only: launch the split-K kernel alone (its partials stay in the workspace; returns None) -- to time
    the kernel by itself.
    deterministic (impl "mfma"): bit-identical results from call to call: tiles go to the wavefronts of a block in
    a fixed order and the combine kernel merges the splits.  By default tiles go first come (the block's wavefronts
    finish together) and the fp32 summation order varies in the last bits.
    tile_order ("fixed" / "dynamic", impl "mfma"): overrides the tile order alone.
    check_q (impl "mfma"): the matrix-core kernels take Q in fp16; outside a graph capture a Q with an entry beyond the
    fp16 range (|q| > 65504) or not finite raises ValueError (one device reduction and synchronization).  Under
    capture the check is skipped and such a Q gives non-finite outputs.
    """
    S = cache.n_seqs
    assert q.dim() == 3 and q.shape[0] == S and q.shape[2] == cache.D and q.dtype == torch.bfloat16
    assert q.stride(2) == 1 and q.stride(1) == cache.D
    Hq = q.shape[1]
    H, D = cache.H, cache.D
    assert Hq % H == 0
    gs = Hq // H
    if max_len is None:
        max_len = max(cache.h_len) if S else 0
    ws = workspace if workspace is not None else {}
    split_map = split_counts = None
    n_map = 0
    flags = 0
    if impl == "mfma":
        chunk = 0   # every split holds a partial
        if plan is not None:
            if headwise or not _rows_kernel(H, Hq) or plan.Hq != Hq:
                raise ValueError("a decode plan serves the full-row kernel at the q head count it was made for")
            if plan.version != cache.version:
                raise ValueError("stale decode plan: the cache's sequence state changed after kvt_decode_plan")
            n_chunks, split_map, split_counts, n_map = plan.n_chunks, plan.split_map, plan.split_counts, plan.n_map
        elif headwise and _rows_kernel(H, Hq):
            # the head-wise kernel's grid (the A/B reference of the full-row kernel)
            if splits is None and S > 1:
                counts = _split_counts_mfma(cache.h_len[:S], H, hot=_hot_counts(cache, S))
                split_map, split_counts, counts = _split_map(counts, ws, q.device)
                n_chunks, n_map = max(counts), sum(counts)
            else:
                n_chunks = splits if splits is not None else _choose_splits_mfma(max_len, S * H)
        else:
            n_chunks, split_map, split_counts, n_map, _ = _decode_grid(cache, Hq, splits, ws, q.device)
        fixed_order = (tile_order or ("fixed" if deterministic else "dynamic")) == "fixed"
        flags = (0 if fixed_order else 1) | (2 if headwise else 0)
        if check_q and not torch.cuda.is_current_stream_capturing():
            if not bool(torch.isfinite(q).all()) or float(q.abs().max()) > 65504.0:
                raise ValueError("kvt_decode_attn (impl 'mfma'): q has entries beyond the fp16 range the matrix-core "
                                 "kernels take (|q| > 65504 or not finite)")
    else:
        if chunk is None:
            chunk = _choose_chunk(max_len, S * H)
        n_chunks = max(1, -(-max_len // chunk))
    n_slots = n_chunks   # partial slots per (sequence, KV head)
    need_o = S * H * n_slots * gs * D
    po = ws.get("part_o")
    if po is None or po.numel() < need_o:
        po = torch.empty(need_o, dtype=torch.float32, device=q.device)
        pml = torch.empty(S * H * n_slots * gs * 2, dtype=torch.float32, device=q.device)
        ws["part_o"], ws["part_ml"] = po, pml
    pml = ws["part_ml"]
    if out is None:
        out = torch.empty(S, Hq, D, dtype=out_dtype, device=q.device)
    assert out.shape == (S, Hq, D) and out.is_contiguous()
    scale = 1.0 / math.sqrt(D)
    _lib.require_device(q, out)
    if events is not None:
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
    if impl == "ref":
        _lib.call("kvt_decode_ref", 0, q.data_ptr(), q.stride(0), cache.seq_lens.data_ptr(), S, H, Hq, D, cache.group8,
                  cache.k4[layer].data_ptr(), cache.v4[layer].data_ptr(), cache.ks4[layer].data_ptr(),
                  cache.vs4[layer].data_ptr(), cache.rk[layer].data_ptr(), cache.rv[layer].data_ptr(),
                  cache.rks[layer].data_ptr(), cache.rvs[layer].data_ptr(), None, None, cache.ring_base.data_ptr(),
                  cache.ring_len.data_ptr(), cache.ring_start.data_ptr(), cache.page_table.data_ptr(),
                  cache.page_table.stride(0), None, 0, None, None, 0, scale, chunk, n_chunks, po.data_ptr(),
                  pml.data_ptr(), _lib.stream())
    elif impl == "mfma":
        if cache.rk[layer].numel() >= 2 ** 31:
            raise ValueError("kvt_decode_mfma: ring buffers beyond 2^31 bytes per layer are not supported")
        _lib.call("kvt_decode_mfma", q.data_ptr(), q.stride(0), cache.seq_lens.data_ptr(), S, H, Hq, D, cache.group8,
                  cache.k4[layer].data_ptr(), cache.v4[layer].data_ptr(), cache.ks4[layer].data_ptr(),
                  cache.vs4[layer].data_ptr(), cache.rk[layer].data_ptr(), cache.rv[layer].data_ptr(),
                  cache.rks[layer].data_ptr(), cache.rvs[layer].data_ptr(), cache.ring_base.data_ptr(),
                  cache.ring_len.data_ptr(), cache.ring_start.data_ptr(), cache.page_table.data_ptr(),
                  cache.page_table.stride(0), cache.k4[layer].shape[0], scale, n_chunks, _lib.ptr(split_map), n_map,
                  po.data_ptr(), pml.data_ptr(), flags, None if plan is None else plan.entries.data_ptr(),
                  _lib.stream())
    else:
        raise ValueError(f"unknown decode implementation {impl!r}")
    if events is not None:
        ev1.record()
    if partials_only:
        return None
    _lib.call("kvt_decode_combine", po.data_ptr(), pml.data_ptr(), S, H, Hq, D, n_chunks, chunk,
              cache.seq_lens.data_ptr(), _lib.ptr(split_counts), out.data_ptr() if out.dtype == torch.float32 else None,
              out.data_ptr() if out.dtype == torch.bfloat16 else None, out.stride(0), _lib.stream())
    if events is not None:
        ev2 = torch.cuda.Event(enable_timing=True)
        ev2.record()
        events.append((ev0, ev1, ev2))
    return out


def kvt_decode_attn_noalloc(cache: PosTieredCache, layer: int, q: torch.Tensor, out: torch.Tensor,
                            splits: Optional[int] = None, split_map: Optional[torch.Tensor] = None,
                            split_counts: Optional[torch.Tensor] = None, deterministic: bool = False) -> torch.Tensor:
    """kvt_decode_attn(impl="mfma") through the library's no-allocation entry point: the split partials live in the
    library's per-GPU scratch array, the caller passes q, out and (for ragged batches) the split map and per-sequence
    split counts it prepared beforehand; nothing is allocated by the call.  Calls on one GPU must not overlap (they
    share the scratch).  A workload whose partials exceed the scratch raises ValueError before any launch."""
    S = cache.n_seqs
    H, D = cache.H, cache.D
    assert q.dim() == 3 and q.shape[0] == S and q.shape[2] == D and q.dtype == torch.bfloat16
    assert q.stride(2) == 1 and q.stride(1) == D
    Hq = q.shape[1]
    assert out.shape == (S, Hq, D) and out.is_contiguous() and out.dtype in (torch.float32, torch.bfloat16)
    assert (split_map is None) == (split_counts is None), "split_map and split_counts go together"
    if split_map is not None:
        n_map = split_map.numel() // 3
        n_chunks = int(splits) if splits is not None else n_map
        assert split_counts.dtype == torch.int32 and split_counts.numel() >= S
    else:
        n_map = 0
        if splits is not None:
            n_chunks = splits
        elif _rows_kernel(H, Hq):
            n_chunks = _choose_splits_mfma(max(cache.h_len) if S else 0, S, min_pos=ROWS_MIN_POS)
        else:
            n_chunks = _choose_splits_mfma(max(cache.h_len) if S else 0, S * H)
    _lib.require_device(q, out)
    rows = S * H * n_chunks * (Hq // H)
    need = ((rows * D + 63) // 64 * 64 + rows * 2) * 4
    status = _lib.lib().kvt_decode_mfma_noalloc(
        q.data_ptr(), q.stride(0), cache.seq_lens.data_ptr(), S, H, Hq, D, cache.group8, cache.k4[layer].data_ptr(),
        cache.v4[layer].data_ptr(), cache.ks4[layer].data_ptr(), cache.vs4[layer].data_ptr(),
        cache.rk[layer].data_ptr(), cache.rv[layer].data_ptr(), cache.rks[layer].data_ptr(),
        cache.rvs[layer].data_ptr(), cache.ring_base.data_ptr(), cache.ring_len.data_ptr(),
        cache.ring_start.data_ptr(), cache.page_table.data_ptr(), cache.page_table.stride(0),
        cache.k4[layer].shape[0], 1.0 / math.sqrt(D), n_chunks, _lib.ptr(split_map), n_map, _lib.ptr(split_counts),
        0 if deterministic else 1, out.data_ptr() if out.dtype == torch.float32 else None,
        out.data_ptr() if out.dtype == torch.bfloat16 else None, out.stride(0), _lib.stream())
    if status == _lib.KVT_ERANGE:
        raise ValueError(f"kvt_decode_mfma_noalloc: the split partials need {need} bytes, more than the library's "
                         f"{8 << 20}-byte scratch (fewer splits or a smaller batch)")
    if status != _lib.KVT_OK:
        raise RuntimeError(f"kvt_decode_mfma_noalloc: status {status}")
    return out


def decode_attn_slots(q, seq_lens, req_to_token, req_indices, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, ring_mask,
                      sm_k=None, sm_v=None, out_dtype=torch.float32, chunk: Optional[int] = None,
                      max_len: Optional[int] = None, impl: str = "mfma",
                      workspace: Optional[dict] = None) -> torch.Tensor:
    """Decode attention over the slot-indexed (dual-write) tiered pool: position p of request b is slot
    req_to_token[req_indices[b], p], hot when owner[slot & ring_mask] == slot (patches/kv_tiers.py:500-504).
    q: bf16 [B, Hq, D]; seq_lens int32 [B]; req_indices int64 [B].  Returns [B, Hq, D].

    impl "mfma" (default): the fused sparse decode over the matrix cores with every position 0 .. seq_len - 1
    selected (one index row 0 .. max_len - 1 shared by all requests through a zero row stride), rows dequantized
    exactly as the gather writes them; within 2e-3 / 1e-3 of the oracle.  impl "ref": the scalar
    reference-precision kernel in splits of `chunk` positions (2e-5)."""
    B, Hq, D = q.shape
    H = k4.shape[1]
    assert k4.shape[2] * 2 == D and q.dtype == torch.bfloat16 and q.stride(2) == 1 and q.stride(1) == D
    assert req_to_token.dtype == torch.int32 and req_to_token.stride(1) == 1
    assert req_indices.dtype == torch.int64 and seq_lens.dtype == torch.int32
    g8 = D // rks.shape[-1]
    if max_len is None:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("decode_attn_slots: pass max_len (a host int >= every seq_len) under graph capture")
        max_len = int(seq_lens.max())   # one device reduction and synchronization
    if impl == "mfma":
        from .sparse_attn import qwen_sparse_decode_attn
        ws = workspace if workspace is not None else {}
        idx = ws.get("dense_idx")
        if idx is None or idx.shape[1] < max_len or idx.device != q.device:
            idx = torch.arange(max_len, dtype=torch.int32, device=q.device)[None]
            ws["dense_idx"] = idx
        cu = ws.get("dense_cu")
        if cu is None or cu.numel() != B + 1 or cu.device != q.device:
            cu = torch.zeros(B + 1, dtype=torch.int32, device=q.device)
            ws["dense_cu"] = cu
        torch.cumsum(seq_lens.clamp(max=max_len), 0, dtype=torch.int32, out=cu[1:])
        out = torch.empty(B, Hq, D, dtype=out_dtype, device=q.device)
        return qwen_sparse_decode_attn(q, k4, v4, req_to_token, req_indices, idx[:, :max_len].expand(B, max_len),
                                       seq_lens, cu, B, max_len, k_scale=ks4, v_scale=vs4, sm_k=sm_k, sm_v=sm_v,
                                       kv_bits=4, ring_k=rk, ring_v=rv, ring_ks=rks, ring_vs=rvs, owner=owner,
                                       ring_mask=ring_mask, out=out, workspace=ws)
    if impl != "ref":
        raise ValueError(f"unknown decode implementation {impl!r}")
    if chunk is None:
        chunk = _choose_chunk(max_len, B * H)
    n_chunks = max(1, -(-max_len // chunk))
    gs = Hq // H
    po = torch.empty(B * H * n_chunks * gs * D, dtype=torch.float32, device=q.device)
    pml = torch.empty(B * H * n_chunks * gs * 2, dtype=torch.float32, device=q.device)
    out = torch.empty(B, Hq, D, dtype=out_dtype, device=q.device)
    _lib.require_device(q, k4, owner)
    _lib.call("kvt_decode_ref", 1, q.data_ptr(), q.stride(0), seq_lens.data_ptr(), B, H, Hq, D, g8, k4.data_ptr(),
              v4.data_ptr(), ks4.data_ptr(), vs4.data_ptr(), rk.data_ptr(), rv.data_ptr(), rks.data_ptr(),
              rvs.data_ptr(), _lib.ptr(sm_k), _lib.ptr(sm_v), None, None, None, None, 0, req_to_token.data_ptr(),
              req_to_token.stride(0), req_indices.data_ptr(), owner.data_ptr(), int(ring_mask), 1.0 / math.sqrt(D),
              chunk, n_chunks, po.data_ptr(), pml.data_ptr(), _lib.stream())
    _lib.call("kvt_decode_combine", po.data_ptr(), pml.data_ptr(), B, H, Hq, D, n_chunks, chunk, seq_lens.data_ptr(),
              None, out.data_ptr() if out_dtype == torch.float32 else None,
              out.data_ptr() if out_dtype == torch.bfloat16 else None, out.stride(0), _lib.stream())
    return out


_prefill_ws: dict = {}   # (device index, stream) -> zeroed kvt_prefill_attn workspace (counters stay zero between calls)
_cu_count: dict = {}
PREFILL_MAX_ITEMS = 4096   # (sequence, KV head, query tile) items of a spread prefill launch


def prefill_spread_blocks(items: int, device: torch.device) -> int:
    """Blocks of a spread prefill launch: one per CU (a block fills a CU), for launches of at most
    PREFILL_MAX_ITEMS query tiles; 0 (one block per query tile) beyond."""
    if items > PREFILL_MAX_ITEMS:
        return 0
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_count:
        _cu_count[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_count[idx]


def prefill_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The cached prefill workspace of (device, current stream), at least nbytes, zeroed when (re)allocated.  Calls
    on one stream run one after another and share it (each call leaves its merge counters at zero); calls on other
    streams get their own, so launches that may overlap never share counters.  (Allocate it before a graph capture:
    capture records on a side stream, which then owns a workspace of its own.)"""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, torch.cuda.current_stream(idx).cuda_stream)
    ws = _prefill_ws.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
        _prefill_ws[key] = ws
    return ws


def kvt_prefill_attn(cache: PosTieredCache, layer: int, q: torch.Tensor, cu_q: torch.Tensor,
                     kv_lens: Optional[torch.Tensor] = None, max_q: Optional[int] = None,
                     k_src: Optional[torch.Tensor] = None, v_src: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16,
                     spread: Optional[int] = None, work: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal prefill attention of the chunk queries q (bf16 [total_q, Hq, D]; sequence b = cache sequence b owns
    rows cu_q[b] .. cu_q[b+1]) over the tiered cache of `layer`, which must already hold the chunk: the queries sit
    at positions kv_lens[b] - q_len .. kv_lens[b] - 1 (kv_lens defaults to the cache lengths) and each attends to
    every position up to its own (patches/kv_paged_prefix.py:200).  k_src / v_src (bf16 [positions, H, D], batch 1):
    read keys from these rows instead, as the reference does for a chunk without a prefix.  spread: blocks that
    share the launch's key tiles equally, splitting query tiles where a share ends and merging the pieces in the
    kernel (0: one block per query tile, the latest first; default prefill_spread_blocks); work: a zeroed uint8
    workspace of kvt_prefill_work_bytes (default: the device's cached one, allocated on first use -- call once
    before a graph capture).  Returns out ([total_q, Hq, D], bf16 like the reference or fp32)."""
    assert q.dim() == 3 and q.dtype == torch.bfloat16 and q.stride(2) == 1 and q.shape[2] == cache.D
    assert cu_q.dtype in (torch.int32, torch.int64) and cu_q.is_contiguous() and cu_q.is_cuda
    batch = cu_q.shape[0] - 1
    H, D = cache.H, cache.D
    Hq = q.shape[1]
    assert Hq % H == 0 and Hq // H <= 16
    if kv_lens is None:
        kv_lens = cache.seq_lens[:batch]
    assert kv_lens.dtype == torch.int32 and kv_lens.is_cuda and kv_lens.numel() >= batch
    if max_q is None:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("kvt_prefill_attn: pass max_q (the longest chunk, a host int) under graph capture")
        max_q = int((cu_q[1:] - cu_q[:-1]).max()) if batch else 0   # one device reduction and synchronization
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    assert out.shape == q.shape and out.dtype in (torch.bfloat16, torch.float32) and out.stride(2) == 1
    if (k_src is None) != (v_src is None):
        raise ValueError("k_src and v_src go together")
    if k_src is not None:
        assert batch == 1 and k_src.dtype == torch.bfloat16 and v_src.dtype == torch.bfloat16
        assert k_src.stride(2) == 1 and v_src.stride(2) == 1 and k_src.shape[1:] == (H, D) == v_src.shape[1:]
        # (a synchronization; skipped under capture, where keys past k_src's rows read as zero: the kernel's reads
        # of k_src / v_src are bounded by their row count)
        if not torch.cuda.is_current_stream_capturing() and min(k_src.shape[0], v_src.shape[0]) < int(kv_lens[0]):
            raise ValueError("k_src / v_src hold fewer rows than the context length")
    elif max((cache.hot_start(s) for s in range(batch)), default=0) > 8192 * 64:
        raise ValueError("kvt_prefill_attn: paged key ranges beyond 524,288 positions are not supported")
    _lib.require_device(q, out, k_src, v_src, work)
    if q.data_ptr() % 16 or q.stride(0) % 8 or q.stride(1) % 8:
        raise ValueError("kvt_prefill_attn: q rows must start at 16-byte boundaries (strides multiples of 8)")
    if batch == 0 or max_q == 0:
        return out
    if spread is None:
        spread = prefill_spread_blocks(-(-max_q // (8 * (16 // (Hq // H)))) * batch * H, q.device)
    need = ctypes.c_int64(0)
    _lib.call("kvt_prefill_work_bytes", batch, H, Hq, int(max_q), int(spread), ctypes.byref(need))
    if need.value and work is None:
        work = prefill_workspace(q.device, need.value)
    if work is not None and (work.dtype != torch.uint8 or not work.is_contiguous() or work.numel() < need.value):
        raise ValueError(f"kvt_prefill_attn: work must be a contiguous uint8 tensor of at least {need.value} bytes")
    _lib.call("kvt_prefill_attn", q.data_ptr(), q.stride(0), q.stride(1), cu_q.data_ptr(),
              int(cu_q.dtype == torch.int64), kv_lens.data_ptr(), batch, max_q, H, Hq, D, cache.group8,
              cache.k4[layer].data_ptr(), cache.v4[layer].data_ptr(), cache.ks4[layer].data_ptr(),
              cache.vs4[layer].data_ptr(), cache.rk[layer].data_ptr(), cache.rv[layer].data_ptr(),
              cache.rks[layer].data_ptr(), cache.rvs[layer].data_ptr(), cache.ring_base.data_ptr(),
              cache.ring_len.data_ptr(), cache.ring_start.data_ptr(), cache.page_table.data_ptr(),
              cache.page_table.stride(0), cache.k4[layer].shape[0], _lib.ptr(k_src), _lib.ptr(v_src),
              min(k_src.shape[0], v_src.shape[0]) if k_src is not None else 0,
              k_src.stride(0) if k_src is not None else 0, k_src.stride(1) if k_src is not None else 0,
              v_src.stride(0) if v_src is not None else 0, v_src.stride(1) if v_src is not None else 0,
              1.0 / math.sqrt(D), out.data_ptr(), int(out.dtype == torch.float32), out.stride(0), out.stride(1),
              int(spread), _lib.ptr(work), work.numel() if work is not None else 0, _lib.stream())
    return out
