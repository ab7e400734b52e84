"""CPU oracle for the tiered quantized KV cache (``int8ring_int4``): TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU with torch tensors, the arithmetic of the reference's tiered KV path so that
the HIP kernels can be checked against it.  It is test infrastructure, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it, and the package never
falls back to it.

Every function cites the reference lines it restates (paths relative to the reference repository).  The torch
forms follow the reference's own torch references (``gemv/test_kv_tiers.py:56-87``, ``gemv/test_kv_int4.py:44-65``,
``gemv/test_kv_int8.py:37-47``), which the reference's kernels are asserted equal to:

* fp32 scale math, IEEE fp32 division, ``torch.round`` (round-half-to-even), RNE conversions to fp16/bf16;
* the fp16-max clamp of every stored scale (``patches/kv_tiers.py:336-337``, ``patches/kv_int4.py:330-333``).

How each part is pinned (every function has a named check in ``tests/test_oracle.py``): the reference tests'
special cases and constants (0x88, 0x01|0xF0, 65504, 127*65504 and 7*65504 in bf16, the -7..7 row), an independent
scalar restatement in pure Python (``tests/golden/scalar_model.py``: golden vectors, per-slot tier loops), brute force
(all 225 nibble pairs, per-element valid counts, the token-by-token evict model against its closed form), invariants
of the owner table (last writer of each residue class, the s/s+R boundary flip, one winner per collision), the closed
form of softmax attention at a single position (returns exactly that V row) and a float64 softmax.
Parts with no such check: none.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

G4 = 32                 # channels per fp16 scale in the INT4 pool (patches/kv_int4.py:286)
G8 = 64                 # channels per fp16 scale in the INT8 ring (patches/kv_int8.py:278)
FP16_MAX = 65504.0      # fp16-max clamp of every stored scale (patches/kv_tiers.py:336-337)
PAGE = 64               # tokens per INT4 page (scripts/serve.sh page size 64; sglang/PATCH_NOTES.md:289)


# ----------------------------------------------------------------------------------------------- quantization
def _scaled(x: torch.Tensor, sm_inv: Optional[torch.Tensor]) -> torch.Tensor:
    """x = f32(k) * f32(sm_inv) (patches/kv_tiers.py:332-333, :362-363); sm_inv [H, D] broadcast over tokens."""
    xf = x.float()
    if sm_inv is not None:
        xf = xf * sm_inv.float()
    return xf if xf.is_contiguous() else xf.contiguous()


def quant_groups(x: torch.Tensor, group: int, qmax: float, sm_inv: Optional[torch.Tensor] = None):
    """Symmetric group quantization of the last dim.

    s = fp16(min(a > 0 ? a / qmax : 1, 65504)), q = clamp(rne(x / f32(s)), -qmax, qmax), with a = max|x| over
    the group (patches/kv_tiers.py:334-339 for qmax 127; :364-370 for qmax 7; torch form
    gemv/test_kv_tiers.py:65-83).  Returns (q float tensor shaped like x, s fp16 [..., D // group]).
    """
    xf = _scaled(x, sm_inv)
    if xf.data_ptr() == x.data_ptr():      # an fp32 input: work on a copy (the steps below are in place)
        xf = xf.clone()
    return _quant_fp32_inplace(xf, group, qmax)


def _quant_fp32_inplace(xf: torch.Tensor, group: int, qmax: float):
    """quant_groups' arithmetic on a contiguous fp32 tensor that it may overwrite with the codes."""
    xg = xf.view(*xf.shape[:-1], xf.shape[-1] // group, group)
    a = xg.abs().amax(-1)
    s = torch.where(a > 0, a / qmax, torch.ones_like(a)).clamp_(max=FP16_MAX).half()
    # q = clamp(rne(x / f32(s)), -qmax, qmax): the same IEEE division, rounding and clamp, in place over x's copy
    xg.div_(s.float()[..., None]).round_().clamp_(-qmax, qmax)
    return xf, s


def quant8(x: torch.Tensor, group: int = G8, sm_inv: Optional[torch.Tensor] = None):
    """INT8-G ring row: (q int8 [..., D], s fp16 [..., D // group]) (gemv/test_kv_tiers.py:77-83;
    patches/kv_tiers.py:325-351).  group=256 is the per-(token, head) form (patches/kv_fakeq.py:9)."""
    q, s = quant_groups(x, group, 127.0, sm_inv)
    return q.to(torch.int8), s


def pack4(q: torch.Tensor) -> torch.Tensor:
    """q int in [-7, 7] [..., D] -> uint8 [..., D // 2]: low nibble = even channel, high = odd, +8 offset
    (gemv/test_kv_int4.py:44-46; patches/kv_int4.py:337-339)."""
    q = q.to(torch.int32)
    return ((q[..., 0::2] + 8) | ((q[..., 1::2] + 8) << 4)).to(torch.uint8)


def unpack4(p: torch.Tensor) -> torch.Tensor:
    """uint8 [..., D // 2] -> int32 [..., D] (gemv/test_kv_int4.py:49-52)."""
    b = p.to(torch.int32)
    return torch.stack([(b & 15) - 8, (b >> 4) - 8], dim=-1).reshape(*p.shape[:-1], 2 * p.shape[-1])


def quant4(x: torch.Tensor, sm_inv: Optional[torch.Tensor] = None):
    """INT4-G32 pool row: (packed uint8 [..., D // 2], s fp16 [..., D // 32]) (gemv/test_kv_int4.py:55-61;
    patches/kv_int4.py:324-341, IEEE division as tl.div_rn)."""
    q, s = quant_groups(x, G4, 7.0, sm_inv)
    return pack4(q), s


def dequant8(q: torch.Tensor, s: torch.Tensor, sm: Optional[torch.Tensor] = None, group: int = G8) -> torch.Tensor:
    """bf16(f32(q) * f32(s) * f32(sm)) (patches/kv_tiers.py:524-525; torch form gemv/test_kv_tiers.py:86-87)."""
    x = q.float() * s.float().repeat_interleave(group, dim=-1)
    if sm is not None:
        x = x * sm.float()
    return x.to(torch.bfloat16)


def dequant4(p: torch.Tensor, s: torch.Tensor, sm: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(f32((b & 15) - 8 | (b >> 4) - 8) * f32(s) * f32(sm)) (patches/kv_tiers.py:516-523;
    gemv/test_kv_int4.py:64-65)."""
    x = unpack4(p).float() * s.float().repeat_interleave(G4, dim=-1)
    if sm is not None:
        x = x * sm.float()
    return x.to(torch.bfloat16)


def requant8to4(q8: torch.Tensor, s8: torch.Tensor, group8: int = G8):
    """Ring-eviction requantization: x = f32(q8) * f32(s8) (exact in fp32), then INT4-G32 with fresh 32-channel
    scales (docs/KV_TIERS_PLAN.md:53, torch reference at :82; "do NOT reuse s8*127/7")."""
    D = q8.shape[-1]
    x = (q8.float().view(*q8.shape[:-1], D // group8, group8) * s8.float()[..., None]).view(q8.shape)
    q, s = _quant_fp32_inplace(x, G4, 7.0)
    return pack4(q), s


# ----------------------------------------------------------------------------------------------- dual-write (slot ring)
def stamp_owner(owner: torch.Tensor, loc: torch.Tensor, ring_mask: int) -> None:
    """owner[slot & mask] = slot for every slot of the write (patches/kv_tiers.py:272-280).  Colliding slots of one
    write race on the GPU (one winner, arbitrary); the oracle resolves the race as the last writer in loc order,
    and tests of collisions check the invariant (one winner among the writers) rather than which one wins."""
    for s in loc.tolist():
        owner[int(s) & ring_mask] = int(s)


def quant_store_tiered(k, v, loc, k_buf, v_buf, k_scale, v_scale, rk, rv, rks, rvs, owner, sm_k_inv, sm_v_inv,
                       ring_mask, group8: int = G8) -> None:
    """Dual write (patches/kv_tiers.py:283-443): stamp the owner, INT8 ring row at slot & mask for the owner only,
    INT4 row at slot for every token.  In place on CPU tensors laid out as the reference pool."""
    N = k.shape[0]
    assert N <= ring_mask + 1
    if N == 0:
        return
    stamp_owner(owner, loc, ring_mask)
    sl = loc.long()
    r = sl & ring_mask
    hot = owner.long()[r] == sl
    q8k, s8k = quant8(k, group8, sm_k_inv)
    q8v, s8v = quant8(v, group8, sm_v_inv)
    rk[r[hot]] = q8k[hot]
    rks[r[hot]] = s8k[hot]
    rv[r[hot]] = q8v[hot]
    rvs[r[hot]] = s8v[hot]
    pk, sk = quant4(k, sm_k_inv)
    pv, sv = quant4(v, sm_v_inv)
    k_buf[sl] = pk
    k_scale[sl] = sk
    v_buf[sl] = pv
    v_scale[sl] = sv


def quant_store_int4(k, v, loc, k_buf, v_buf, k_scale, v_scale, sm_k_inv, sm_v_inv) -> None:
    """INT4-G32 quant + nibble pack + scatter at loc (patches/kv_int4.py:289-393)."""
    if k.shape[0] == 0:
        return
    sl = loc.long()
    p, s = quant4(k, sm_k_inv)
    k_buf[sl] = p
    k_scale[sl] = s
    p, s = quant4(v, sm_v_inv)
    v_buf[sl] = p
    v_scale[sl] = s


def is_hot(slots: torch.Tensor, owner: torch.Tensor, ring_mask: int) -> torch.Tensor:
    """Tier rule hot = owner[slot & mask] == slot (patches/kv_tiers.py:500-504)."""
    sl = slots.long()
    return owner.long()[sl & ring_mask] == sl


def dequant_slots_tiered(slots, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, ring_mask, sm_k=None, sm_v=None,
                         group8: int = G8):
    """bf16 K/V rows [n, H, D] of the given slots, each from its tier (patches/kv_tiers.py:500-538)."""
    sl = slots.long()
    hot = is_hot(sl, owner, ring_mask)
    r = sl & ring_mask
    dk4 = dequant4(k4[sl], ks4[sl], sm_k)
    dv4 = dequant4(v4[sl], vs4[sl], sm_v)
    dk8 = dequant8(rk[r], rks[r], sm_k, group8)
    dv8 = dequant8(rv[r], rvs[r], sm_v, group8)
    h = hot[:, None, None]
    return torch.where(h, dk8, dk4), torch.where(h, dv8, dv4)


def cu_seqlens_valid(seq_lens, indices, topk):
    """cu_k of the compact gather: per request the count of selected columns with 0 <= pos < seq_len, prefix
    summed (the counting the reference does in qwen_sparse_fa2_cu_seqlens_triton, used by
    gemv/test_kv_tiers.py:297-301)."""
    idx = indices[:, :topk].long()
    counts = ((idx >= 0) & (idx < seq_lens.long()[:, None])).sum(1)
    return torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32)


# ----------------------------------------------------------------------------------------------- attention
def attention_rows(q: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor, scale: float) -> torch.Tensor:
    """fp32 softmax attention of one query over bf16-dequantized rows (gemv/test_kv_paged_prefix.py:520-528).

    q: [Hq, D]; k_rows, v_rows: [n, H, D] (bf16); KV head of q head i is i // (Hq // H).  Returns fp32 [Hq, D];
    an empty selection returns NaN (0/0, gemv/test_kv_paged_prefix.py:524-526)."""
    Hq, D = q.shape
    H = k_rows.shape[1]
    gs = Hq // H
    out = torch.empty(Hq, D, dtype=torch.float32)
    qf = q.float() * scale
    for h in range(H):
        qh = qf[h * gs:(h + 1) * gs]
        if k_rows.shape[0] == 0:
            out[h * gs:(h + 1) * gs] = float("nan")
            continue
        kk = k_rows[:, h].float()
        vv = v_rows[:, h].float()
        out[h * gs:(h + 1) * gs] = torch.softmax(qh @ kk.T, dim=-1) @ vv
    return out


def prefill_selected_positions(idx_row: torch.Tensor, visible: int, kv_len: int, topk: int) -> torch.Tensor:
    """Positions a prefill query attends to (patches/kv_paged_prefix.py:200-229, test oracle
    gemv/test_kv_paged_prefix.py:515-519): the first min(topk, visible) entries of its index row with
    0 <= idx < kv_len; visible = j + kv_len - q_len + 1 for query j of its chunk."""
    n = max(0, min(topk, visible))          # a query with no visible position (kv_len < q_len) selects nothing
    pos = idx_row[:n].long()
    return pos[(pos >= 0) & (pos < kv_len)]


# ----------------------------------------------------------------------------------------------- position rings (evict)
class PageAllocator:
    """Free list of physical INT4 pages in a seeded random order (the physical placement the configurations ask
    for: "physical pages randomly permuted from seed").  pop() hands out pages in that order; the device page
    table must equal what this allocator assigns."""

    def __init__(self, n_pages: int, seed: int):
        g = torch.Generator().manual_seed(seed)
        self.free: List[int] = torch.randperm(n_pages, generator=g).tolist()
        self.next = 0

    def pop(self) -> int:
        if self.next >= len(self.free):
            raise RuntimeError("INT4 page pool exhausted")
        p = self.free[self.next]
        self.next += 1
        return p


@dataclass
class SeqState:
    """One sequence of the position-indexed tiered cache: ring rows [ring_base, ring_base + ring_len), positions
    below ring_start come from pages shared with another sequence, page_table maps logical -> physical page."""
    ring_base: int
    ring_len: int
    ring_start: int = 0
    length: int = 0
    pages: List[int] = field(default_factory=list)

    @property
    def hot_start(self) -> int:
        return max(self.ring_start, self.length - self.ring_len)


class PosTieredCache:
    """CPU model of the evict-mode tiered cache (one layer): per-sequence INT8 ring indexed by position mod R,
    INT4 pool in 64-token pages behind a page table.  Appending position p >= ring_start + R first requantizes the
    ring row it overwrites (position e = p - R) into the INT4 pool (docs/KV_TIERS_PLAN.md:53, :63-67, :82), then
    quantizes the new token into the ring row (patches/kv_tiers.py:325-351)."""

    def __init__(self, H, D, n_pages, ring_total, group8=G8):
        self.H, self.D, self.group8 = H, D, group8
        rows = n_pages * PAGE
        self.k4 = torch.zeros(rows, H, D // 2, dtype=torch.uint8)
        self.v4 = torch.zeros_like(self.k4)
        self.ks4 = torch.zeros(rows, H, D // G4, dtype=torch.float16)
        self.vs4 = torch.zeros_like(self.ks4)
        self.rk = torch.zeros(ring_total, H, D, dtype=torch.int8)
        self.rv = torch.zeros_like(self.rk)
        self.rks = torch.zeros(ring_total, H, D // group8, dtype=torch.float16)
        self.rvs = torch.zeros_like(self.rks)
        self.seqs: List[SeqState] = []

    def add_seq(self, ring_base, ring_len, ring_start=0, shared_pages: Sequence[int] = ()):
        assert ring_len > 0 and ring_len & (ring_len - 1) == 0
        st = SeqState(ring_base, ring_len, ring_start, ring_start, list(shared_pages))
        assert len(st.pages) * PAGE >= ring_start
        self.seqs.append(st)
        return len(self.seqs) - 1

    def plan_pages(self, seq: int, n_new: int, alloc: PageAllocator) -> List[Tuple[int, int]]:
        """Pages a coming append of n_new tokens evicts into for the first time: [(logical, physical)], popped from
        the allocator in increasing logical order (what the host allocator writes into the device page table)."""
        st = self.seqs[seq]
        out = []
        for p in range(st.length, st.length + n_new):
            e = p - st.ring_len
            if e >= st.ring_start and e % PAGE == 0:
                lp = e // PAGE
                assert lp == len(st.pages)
                phys = alloc.pop()
                st.pages.append(phys)
                out.append((lp, phys))
        return out

    def append(self, seq: int, k: torch.Tensor, v: torch.Tensor, sm_k_inv=None, sm_v_inv=None):
        """Append n tokens (k, v: [n, H, D]) at positions length..length+n-1 (n <= ring_len)."""
        st = self.seqs[seq]
        n = k.shape[0]
        assert n <= st.ring_len
        for i in range(n):
            p = st.length + i
            r = st.ring_base + (p & (st.ring_len - 1))
            e = p - st.ring_len
            if e >= st.ring_start:
                row = st.pages[e // PAGE] * PAGE + e % PAGE
                pk, sk = requant8to4(self.rk[r], self.rks[r], self.group8)
                pv, sv = requant8to4(self.rv[r], self.rvs[r], self.group8)
                self.k4[row], self.ks4[row], self.v4[row], self.vs4[row] = pk, sk, pv, sv
            q, s = quant8(k[i], self.group8, sm_k_inv)
            self.rk[r], self.rks[r] = q, s
            q, s = quant8(v[i], self.group8, sm_v_inv)
            self.rv[r], self.rvs[r] = q, s
        st.length += n

    def rows(self, seq: int, sm_k=None, sm_v=None):
        """bf16 K, V [length, H, D] of a sequence in position order, each position from its tier."""
        st = self.seqs[seq]
        L, hs = st.length, st.hot_start
        pos = torch.arange(L)
        cold = pos[:hs]
        hot = pos[hs:]
        pt = torch.tensor(st.pages, dtype=torch.long) if st.pages else torch.zeros(0, dtype=torch.long)
        crow = pt[cold // PAGE] * PAGE + cold % PAGE if cold.numel() else cold
        hrow = st.ring_base + (hot & (st.ring_len - 1))
        dk = torch.cat([dequant4(self.k4[crow], self.ks4[crow], sm_k), dequant8(self.rk[hrow], self.rks[hrow], sm_k, self.group8)])
        dv = torch.cat([dequant4(self.v4[crow], self.vs4[crow], sm_v), dequant8(self.rv[hrow], self.rvs[hrow], sm_v, self.group8)])
        return dk, dv

    def page_table(self, max_pages: int) -> torch.Tensor:
        pt = torch.full((len(self.seqs), max_pages), -1, dtype=torch.int32)
        for i, st in enumerate(self.seqs):
            if st.pages:
                pt[i, :len(st.pages)] = torch.tensor(st.pages, dtype=torch.int32)
        return pt


def evict_closed_form(xk: torch.Tensor, xv: torch.Tensor, ring_len: int, ring_start: int = 0, group8: int = G8,
                      sm_k_inv=None, sm_v_inv=None) -> dict:
    """State of one sequence of the evict-mode cache after positions ring_start .. ring_start + n - 1 were appended
    (in any chunking), as closed forms over all tokens at once: positions p >= hot_start = max(ring_start,
    length - R) hold quant8(x[p]) in ring row p & (R - 1) (patches/kv_tiers.py:325-351); every older appended
    position holds requant8to4 of its INT8 row (docs/KV_TIERS_PLAN.md:53, :82), in page order.  xk / xv: the
    appended rows [n, H, D] (row i = position ring_start + i).  Returns the hot codes / scales in position order
    with their ring rows, the cold INT4 codes / scales in position order and hot_start."""
    n = xk.shape[0]
    length = ring_start + n
    hs = max(ring_start, length - ring_len)
    q8k, s8k = quant8(xk, group8, sm_k_inv)
    q8v, s8v = quant8(xv, group8, sm_v_inv)
    c = hs - ring_start                       # appended rows that left the ring
    pk, sk = requant8to4(q8k[:c], s8k[:c], group8)
    pv, sv = requant8to4(q8v[:c], s8v[:c], group8)
    pos_hot = torch.arange(hs, length)
    return dict(hot_start=hs, ring_rows=pos_hot & (ring_len - 1), rk=q8k[c:], rks=s8k[c:], rv=q8v[c:], rvs=s8v[c:],
                k4=pk, ks4=sk, v4=pv, vs4=sv)


# ----------------------------------------------------------------------------------------------- synthetic inputs
def make_kv(n: int, H: int, D: int, gen: torch.Generator, outlier_ch: torch.Tensor, outlier_mul: float = 8.0):
    """K ~ N(0,1) with the given channels (per head) scaled x8 as outliers, V ~ N(0,1); bf16 on the CPU
    (the synthetic distribution of every configuration; outlier channels chosen from the seed)."""
    k = torch.randn(n, H, D, generator=gen)
    v = torch.randn(n, H, D, generator=gen)
    mul = torch.ones(H, D)
    for h in range(H):
        mul[h, outlier_ch[h]] = outlier_mul
    return (k * mul).to(torch.bfloat16), v.to(torch.bfloat16)


def outlier_channels(H: int, D: int, n_out: int, gen: torch.Generator) -> torch.Tensor:
    """n_out distinct outlier channels per KV head, drawn from the generator."""
    return torch.stack([torch.randperm(D, generator=gen)[:n_out] for _ in range(H)])


def make_q(Hq: int, D: int, gen: torch.Generator, n: int = 1) -> torch.Tensor:
    """Q ~ N(0,1) / 16 in bf16."""
    return (torch.randn(n, Hq, D, generator=gen) / 16).to(torch.bfloat16)
