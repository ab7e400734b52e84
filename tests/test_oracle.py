"""Pinning the CPU oracle (oracle/ref.py) before the HIP kernels are compared with it.

Each check is chosen so that a plausible mistake fails it: the reference tests' special cases and constants
(gemv/test_kv_int4.py, gemv/test_kv_int8.py, gemv/test_kv_tiers.py), the golden vectors of the independent scalar
model (tests/golden/), round-half-even ties, brute force over every nibble pair, the owner-table invariants, and
closed forms of attention.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import ref

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant_vectors.npz")


def _gold():
    return np.load(GOLD)


def _x_from_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


# ---------------------------------------------------------------------------------------------- nibble packing
def test_pack_unpack_all_pairs():
    """Every (even, odd) pair in [-7, 7]^2 round-trips; pack(-7, 7) = 0x01 | 0xF0, pack(0, 0) = 0x88
    (gemv/test_kv_int4.py:72-81)."""
    qa = torch.arange(-7, 8, dtype=torch.int32)
    qq = torch.cartesian_prod(qa, qa).reshape(-1)
    qq = torch.cat([qq, torch.zeros(256 - qq.numel() % 256, dtype=torch.int32)]).reshape(-1, 256)
    pp = ref.pack4(qq)
    assert pp.dtype == torch.uint8 and int(pp.min()) >= 0x11 and int(pp.max()) <= 0xFF
    assert torch.equal(ref.unpack4(pp), qq)
    assert int(ref.pack4(torch.tensor([[-7, 7]]))[0, 0]) == 0x01 | 0xF0
    assert int(ref.pack4(torch.tensor([[0, 0]]))[0, 0]) == 0x88
    # nibble order: low = even channel
    assert int(ref.pack4(torch.tensor([[1, -1]]))[0, 0]) == (9 | (7 << 4))


# ---------------------------------------------------------------------------------------------- golden vectors
def test_golden_vectors_quant8_quant4():
    g = _gold()
    x = _x_from_bits(g["x_bf16_bits"])
    q8, s8 = ref.quant8(x, 64)
    assert torch.equal(q8, torch.from_numpy(g["q8_g64"])) and torch.equal(s8, torch.from_numpy(g["s8_g64"]))
    q8b, s8b = ref.quant8(x, 256)
    assert torch.equal(q8b, torch.from_numpy(g["q8_g256"])) and torch.equal(s8b, torch.from_numpy(g["s8_g256"]))
    p4, s4 = ref.quant4(x)
    assert torch.equal(p4, torch.from_numpy(g["p4"])) and torch.equal(s4, torch.from_numpy(g["s4"]))
    d8 = ref.dequant8(q8, s8)
    assert torch.equal(d8.view(torch.int16), torch.from_numpy(g["d8_g64_bits"].astype(np.int16)))
    d4 = ref.dequant4(p4, s4)
    assert torch.equal(d4.view(torch.int16), torch.from_numpy(g["d4_bits"].astype(np.int16)))
    rp, rs = ref.requant8to4(q8, s8)
    assert torch.equal(rp, torch.from_numpy(g["requant_p4"])) and torch.equal(rs, torch.from_numpy(g["requant_s4"]))


def test_golden_vectors_fresh_scalar_model_with_smoothing():
    """Random rows with random smoothing factors sm_inv in [0.5, 2): oracle == scalar model element by element."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import scalar_model as sm
    gen = torch.Generator().manual_seed(7)
    x = (torch.randn(6, 256, generator=gen) * 2).to(torch.bfloat16)
    sm_inv = (0.5 + 1.5 * torch.rand(1, 256, generator=gen)).half()
    q8, s8 = ref.quant8(x, 64, sm_inv)
    p4, s4 = ref.quant4(x, sm_inv)
    for r in range(x.shape[0]):
        xs = [float(v) for v in x[r].float()]
        m = [float(v) for v in sm_inv[0].float()]
        c, s = sm.quant_row(xs, 64, 127.0, m)
        assert q8[r].tolist() == c and s8[r].float().tolist() == s
        c4, sc4 = sm.quant_row(xs, 32, 7.0, m)
        assert p4[r].tolist() == sm.pack_row(c4) and s4[r].float().tolist() == sc4


# ---------------------------------------------------------------------------------------------- special cases
def test_ties_round_half_to_even():
    """.5 ties at s = 1 go to the even neighbour (torch.round; patches/kv_int4.py:334-337)."""
    x = torch.tensor([[7.0, 2.5, -2.5, 0.5, -0.5, 1.5, 3.5, -6.5] * 4], dtype=torch.bfloat16)
    p, s = ref.quant4(x)
    assert float(s[0, 0]) == 1.0
    assert ref.unpack4(p)[0, :8].tolist() == [7, 2, -2, 0, 0, 2, 4, -6]
    x8 = torch.tensor([[127.0, 4.5, -4.5, 0.5, 100.5, -126.5, 63.5, 1.5] * 8], dtype=torch.bfloat16)
    q, s8 = ref.quant8(x8)
    assert float(s8[0, 0]) == 1.0
    assert q[0, :8].tolist() == [127, 4, -4, 0, 100, -126, 64, 2]


def test_int4_special_rows():
    """zero row -> s = 1, 0x88; zero group; the -7..7 row (gemv/test_kv_int4.py:86-115)."""
    x = torch.randn(3, 2, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16) * 3
    x[0] = 0
    x[1, 1, 64:96] = 0
    full = torch.tensor([-7, 7, -6, 6, -5, 5, -4, 4, -3, 3, -2, 2, -1, 1, 0, 7] * 16, dtype=torch.bfloat16)
    x[2, 0] = full
    p, s = ref.quant4(x)
    assert (s[0] == 1.0).all() and (p[0] == 0x88).all()
    assert float(s[1, 1, 2]) == 1.0 and (p[1, 1, 32:48] == 0x88).all()
    assert (s[2, 0] == 1.0).all()
    assert torch.equal(ref.unpack4(p[2, 0]).unique(), torch.arange(-7, 8, dtype=torch.int32))
    # scale index (slot * H + h) * 8 + g and shape
    assert s.shape == (3, 2, 8) and p.shape == (3, 2, 128)


def test_int8_special_rows():
    """zero row -> s = 1, q = 0; zero group; |q| reaches 127 (gemv/test_kv_int8.py:54-79)."""
    x = torch.randn(3, 2, 256, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16) * 3
    x[0] = 0
    x[1, 0, 64:128] = 0
    q, s = ref.quant8(x)
    assert (s[0] == 1.0).all() and (q[0] == 0).all()
    assert float(s[1, 0, 1]) == 1.0 and (q[1, 0, 64:128] == 0).all()
    assert int(q.abs().max()) == 127
    assert s.shape == (3, 2, 4)


def test_fp16_max_clamp():
    """1e6 / bf16-max groups -> s = 65504, dequant saturates to bf16(7 * 65504) / bf16(127 * 65504)
    (gemv/test_kv_int4.py:256-289, gemv/test_kv_tiers.py:412-436)."""
    big = torch.zeros(1, 2, 256, dtype=torch.bfloat16)
    big[0, 0, :32] = torch.tensor([1e6, -1e6, 5e5, -5e5, 4.6e5, -4.6e5, 1e5, -1e5] * 4).to(torch.bfloat16)
    big[0, 1, 64:96] = torch.finfo(torch.bfloat16).max
    p, s = ref.quant4(big)
    assert float(s[0, 0, 0]) == 65504.0 and float(s[0, 1, 2]) == 65504.0 and torch.isfinite(s).all()
    d = ref.dequant4(p, s)[0]
    sat = torch.tensor(7 * 65504.0).to(torch.bfloat16)
    assert float(d[0, 0]) == float(sat) and float(d[0, 1]) == -float(sat)
    assert (d[1, 64:96] == sat).all()
    q_b = ref.unpack4(p)
    assert int(q_b[0, 0, :32].abs().max()) == 7 and int(q_b[0, 0, 6].abs()) < 7
    q8, s8 = ref.quant8(big)
    assert float(s8[0, 1, 1]) == 65504.0 and torch.isfinite(s8).all()
    d8 = ref.dequant8(q8, s8)[0]
    assert float(d8[1, 64]) == float(torch.tensor(127 * 65504.0).to(torch.bfloat16))


def test_relative_rms_bands():
    """int8-g64 relative RMS < 1.2 % and int4-g32 in 8-11.5 % on N(0, 3) (gemv/test_kv_int8.py:165-170,
    gemv/test_kv_int4.py:249-254)."""
    x = (torch.randn(2000, 2, 256, generator=torch.Generator().manual_seed(2)) * 3).to(torch.bfloat16)

    def relerr(a, b):
        return float(((a.float() - b.float()).pow(2).mean() / b.float().pow(2).mean()).sqrt())

    e8 = relerr(ref.dequant8(*ref.quant8(x)), x)
    e4 = relerr(ref.dequant4(*ref.quant4(x)), x)
    assert e8 < 0.012 and 0.08 < e4 < 0.115, (e8, e4)


def test_requant_close_to_direct_int4():
    """INT8 -> INT4 requant vs INT4 from bf16: codes differ on < 2 % of the nibbles (docs/KV_TIERS_PLAN.md:82 plausibility
    bound), and x8 = q8 * s8 is exact in fp32."""
    x = (torch.randn(4000, 2, 256, generator=torch.Generator().manual_seed(3)) * 3).to(torch.bfloat16)
    q8, s8 = ref.quant8(x)
    rp, rs = ref.requant8to4(q8, s8)
    dp, ds = ref.quant4(x)
    mism = (ref.unpack4(rp) != ref.unpack4(dp)).float().mean()
    assert float(mism) < 0.02
    x8 = q8.double() * s8.double().repeat_interleave(64, -1)
    assert torch.equal(x8.float().double(), x8)


# ---------------------------------------------------------------------------------------------- owner / tiers
def test_owner_last_writer_and_boundary():
    """Ascending writes: owner[r] = last slot of class r; writing s + R flips the owner, s is then cold and its INT4
    row intact (gemv/test_kv_tiers.py:117-191)."""
    R, H, D, slots = 64, 2, 256, 4096
    gen = torch.Generator().manual_seed(0)
    sl = torch.randperm(slots, generator=gen)[:1000].sort().values
    bufs = _new_bufs(slots, R, H, D)
    k = (torch.randn(1000, H, D, generator=gen) * 3).to(torch.bfloat16)
    v = (torch.randn(1000, H, D, generator=gen) * 3).to(torch.bfloat16)
    ones = torch.ones(H, D, dtype=torch.float16)
    a = 0
    while a < 1000:                                  # alias-free chunks (span < R)
        e = a + 1
        while e < 1000 and int(sl[e]) - int(sl[a]) < R:
            e += 1
        ref.quant_store_tiered(k[a:e], v[a:e], sl[a:e], *bufs, ones, ones, R - 1)
        a = e
    k4, v4, ks4, vs4, rk, rv, rks, rvs, owner = bufs
    exp = torch.full((R,), -1, dtype=torch.int64)
    for s in sl.tolist():
        exp[s & (R - 1)] = s
    assert torch.equal(owner.long(), exp)
    pk, sk = ref.quant4(k)
    assert torch.equal(k4[sl], pk) and torch.equal(ks4[sl], sk)
    hot = ref.is_hot(sl, owner, R - 1)
    q8, s8 = ref.quant8(k)
    assert torch.equal(rk[sl[hot] & (R - 1)], q8[hot]) and torch.equal(rks[sl[hot] & (R - 1)], s8[hot])
    # boundary
    bufs = _new_bufs(slots, R, H, D)
    ref.quant_store_tiered(k[:1], v[:1], torch.tensor([100]), *bufs, ones, ones, R - 1)
    ref.quant_store_tiered(k[1:2], v[1:2], torch.tensor([100 + R]), *bufs, ones, ones, R - 1)
    assert int(bufs[8][100 & (R - 1)]) == 100 + R
    assert not bool(ref.is_hot(torch.tensor([100]), bufs[8], R - 1)[0])
    assert torch.equal(bufs[0][100], pk[0])


def _new_bufs(slots, R, H, D, g8=64):
    return (torch.full((slots, H, D // 2), 0x77, dtype=torch.uint8), torch.full((slots, H, D // 2), 0x99, dtype=torch.uint8),
            torch.full((slots, H, D // 32), 3.0, dtype=torch.float16), torch.full((slots, H, D // 32), 5.0, dtype=torch.float16),
            torch.full((R, H, D), 0x33, dtype=torch.int8), torch.full((R, H, D), 0x44, dtype=torch.int8),
            torch.full((R, H, D // g8), 7.0, dtype=torch.float16), torch.full((R, H, D // g8), 9.0, dtype=torch.float16),
            torch.full((R,), -1, dtype=torch.int32))


def test_collision_one_winner():
    """Slots congruent mod R in one write: exactly one owner per contested row, drawn from its writers
    (gemv/test_kv_tiers.py:193-235)."""
    R, H, D = 64, 2, 256
    bufs = _new_bufs(4096, R, H, D)
    gen = torch.Generator().manual_seed(4)
    classes = torch.randint(0, 8, (R,), generator=gen)
    members = torch.randperm(4096 // R, generator=gen)[:R]
    loc = members * R + classes
    x = torch.randn(R, H, D, generator=gen).to(torch.bfloat16)
    ones = torch.ones(H, D, dtype=torch.float16)
    ref.quant_store_tiered(x, x, loc, *bufs, ones, ones, R - 1)
    owner = bufs[8]
    for r in range(R):
        cand = loc[(loc & (R - 1)) == r]
        if cand.numel() == 0:
            assert int(owner[r]) == -1
        else:
            assert int(owner[r]) in set(cand.tolist())
    assert int(ref.is_hot(loc, owner, R - 1).sum()) == int((owner >= 0).sum()) <= 8


# ---------------------------------------------------------------------------------------------- position rings
def test_pos_cache_eviction_and_pages():
    """Evict mode: after L appends with ring R the newest R positions are INT8 (bit-exact quant8 of their input),
    every older position is the requant of its INT8 row into the page the allocator assigned, page order = allocator
    order; chunked appends give the same state as token-by-token appends."""
    H, D, R = 2, 256, 128
    gen = torch.Generator().manual_seed(5)
    x_k = (torch.randn(700, H, D, generator=gen) * 2).to(torch.bfloat16)
    x_v = (torch.randn(700, H, D, generator=gen) * 2).to(torch.bfloat16)
    caches = []
    for chunking in ([1] * 700, [100] * 7, [128, 128, 128, 128, 128, 60]):
        c = ref.PosTieredCache(H, D, n_pages=32, ring_total=R)
        alloc = ref.PageAllocator(32, seed=9)
        s = c.add_seq(0, R)
        a = 0
        for n in chunking:
            c.plan_pages(s, n, alloc)
            c.append(s, x_k[a:a + n], x_v[a:a + n])
            a += n
        caches.append(c)
    c0 = caches[0]
    for c in caches[1:]:
        for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
            assert torch.equal(getattr(c, name), getattr(c0, name)), name
    st = c0.seqs[0]
    assert st.length == 700 and st.hot_start == 700 - R
    assert st.pages == ref.PageAllocator(32, seed=9).free[:len(st.pages)]
    assert len(st.pages) == math.ceil((700 - R) / 64)
    dk, dv = c0.rows(0)
    q8, s8 = ref.quant8(x_k)
    rp, rs = ref.requant8to4(q8, s8)
    assert torch.equal(dk[700 - R:], ref.dequant8(q8[700 - R:], s8[700 - R:]))
    assert torch.equal(dk[:700 - R], ref.dequant4(rp[:700 - R], rs[:700 - R]))


# ---------------------------------------------------------------------------------------------- attention
def test_attention_single_position_and_empty():
    """One valid position: the output is exactly that V row; no position: NaN (gemv/test_kv_paged_prefix.py:436-457,
    :524-526)."""
    gen = torch.Generator().manual_seed(6)
    q = torch.randn(16, 256, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, 2, 256, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, 2, 256, generator=gen).to(torch.bfloat16)
    o = ref.attention_rows(q, k, v, 1 / 16)
    assert torch.equal(o[:8], v[0, 0].float().expand(8, 256)) and torch.equal(o[8:], v[0, 1].float().expand(8, 256))
    o = ref.attention_rows(q, k[:0], v[:0], 1 / 16)
    assert torch.isnan(o).all()


def test_attention_matches_float64():
    """fp32 attention == float64 softmax within 1e-5 (GQA mapping: q head i reads KV head i // 8)."""
    gen = torch.Generator().manual_seed(8)
    q = (torch.randn(16, 256, generator=gen) / 16).to(torch.bfloat16)
    k = torch.randn(300, 2, 256, generator=gen).to(torch.bfloat16)
    v = torch.randn(300, 2, 256, generator=gen).to(torch.bfloat16)
    o = ref.attention_rows(q, k, v, 1 / 16)
    for i in range(16):
        h = i // 8
        s = (q[i].double() @ k[:, h].double().T) / 16
        w = torch.softmax(s, 0)
        e = w @ v[:, h].double()
        assert float((o[i].double() - e).abs().max()) < 1e-5


def test_prefill_selection_rule():
    idx = torch.tensor([3, 0, 7, -1, 5, 9, 2])
    pos = ref.prefill_selected_positions(idx, visible=5, kv_len=8, topk=7)
    assert pos.tolist() == [3, 0, 7, 5]          # first min(topk, visible) = 5 entries, -1 dropped, < kv_len
    pos = ref.prefill_selected_positions(idx, visible=9, kv_len=8, topk=7)
    assert pos.tolist() == [3, 0, 7, 5, 2]       # 9 >= kv_len dropped
    pos = ref.prefill_selected_positions(idx, visible=9, kv_len=8, topk=3)
    assert pos.tolist() == [3, 0, 7]             # only the first topk entries
    for visible in (0, -5):                      # kv_len < q_len: the early queries see nothing
        assert ref.prefill_selected_positions(idx, visible=visible, kv_len=8, topk=7).numel() == 0


# ---------------------------------------------------------------------------------------------- gathers' building blocks
def test_cu_seqlens_valid_brute_force():
    """cu_k = prefix sum of the per-request counts of columns c < topk with 0 <= indices[b][c] < seq_lens[b], counted
    element by element (indices with -1 padding, entries >= seq_len and columns past topk that must not count)."""
    gen = torch.Generator().manual_seed(11)
    for batch, topk, width in ((1, 5, 5), (4, 37, 40), (7, 200, 260)):
        seq = torch.randint(0, 300, (batch,), generator=gen).to(torch.int32)
        idx = torch.randint(-2, 330, (batch, width), generator=gen).to(torch.int32)
        idx[0, : min(3, width)] = -1
        cu = ref.cu_seqlens_valid(seq, idx, topk)
        want = [0]
        for b in range(batch):
            n = 0
            for c in range(topk):
                v = int(idx[b, c])
                if 0 <= v < int(seq[b]):
                    n += 1
            want.append(want[-1] + n)
        assert cu.dtype == torch.int32 and cu.tolist() == want


def test_dequant_slots_tiered_scalar_loop():
    """Tiered rows of given slots against a per-slot scalar loop (tests/golden/scalar_model.py): the ring row
    r = slot & mask when owner[r] == slot, else the INT4 row; unowned ring rows are poisoned (NaN / inf scales,
    0x77 codes) and a stale owner (another slot of the class) must send its slot to INT4
    (gemv/test_kv_tiers.py:259-262, :320, :370-378)."""
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import scalar_model as sm
    gen = torch.Generator().manual_seed(12)
    H, D, R, slots = 2, 256, 16, 256
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    v4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    ks4 = (0.05 + torch.rand(slots, H, D // 32, generator=gen)).half()
    vs4 = (0.05 + torch.rand(slots, H, D // 32, generator=gen)).half()
    rk = torch.full((R, H, D), 0x77, dtype=torch.int8)
    rv = torch.full((R, H, D), 0x77, dtype=torch.int8)
    rks = torch.full((R, H, D // 64), float("nan"), dtype=torch.float16)
    rvs = torch.full((R, H, D // 64), float("inf"), dtype=torch.float16)
    owner = torch.full((R,), -1, dtype=torch.int32)
    owned = [0, 3, 5, 6, 9, 12, 15]
    for r in owned:
        owner[r] = r + R * int(torch.randint(0, slots // R, (1,), generator=gen))
        rk[r] = torch.randint(-127, 128, (H, D), dtype=torch.int8, generator=gen)
        rv[r] = torch.randint(-127, 128, (H, D), dtype=torch.int8, generator=gen)
        rks[r] = (0.001 + 0.01 * torch.rand(H, D // 64, generator=gen)).half()
        rvs[r] = (0.001 + 0.01 * torch.rand(H, D // 64, generator=gen)).half()
    smk = (0.5 + torch.rand(H, D, generator=gen)).half()
    smv = (0.5 + torch.rand(H, D, generator=gen)).half()
    # every owner slot, its stale neighbours of the same class, and random slots
    query = [int(owner[r]) for r in owned] + [int(owner[r]) + R for r in owned if int(owner[r]) + R < slots]
    query += torch.randint(0, slots, (40,), generator=gen).tolist()
    sl = torch.tensor(query)
    dk, dv = ref.dequant_slots_tiered(sl, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, R - 1, smk, smv)
    assert torch.isfinite(dk.float()).all() and torch.isfinite(dv.float()).all()
    n_hot = 0
    for i, s_ in enumerate(query):
        r = s_ & (R - 1)
        hot = int(owner[r]) == s_
        n_hot += hot
        for h in range(H):
            for got, cod8, sc8, cod4, sc4, smf in ((dk, rk, rks, k4, ks4, smk), (dv, rv, rvs, v4, vs4, smv)):
                if hot:
                    codes, scales, g = cod8[r, h].tolist(), sc8[r, h].float().tolist(), 64
                else:
                    codes, scales, g = sm.unpack_row(cod4[s_, h].tolist()), sc4[s_, h].float().tolist(), 32
                want = sm.dequant_row_bits(codes, scales, g, smf[h].float().tolist())
                assert got[i, h].view(torch.int16).tolist() == [w - 65536 if w >= 32768 else w for w in want]
    assert 0 < n_hot < len(query)


def test_quant_store_int4_scatter():
    """quant_store_int4 writes quant4(k) / quant4(v) at the given slots of the K and V tensors and nothing else."""
    gen = torch.Generator().manual_seed(13)
    H, D, slots = 2, 256, 64
    k = (torch.randn(10, H, D, generator=gen) * 3).to(torch.bfloat16)
    v = (torch.randn(10, H, D, generator=gen) * 3).to(torch.bfloat16)
    loc = torch.randperm(slots, generator=gen)[:10]
    kb = torch.full((slots, H, D // 2), 0x55, dtype=torch.uint8)
    vb = torch.full((slots, H, D // 2), 0x66, dtype=torch.uint8)
    ksb = torch.full((slots, H, 8), 3.0, dtype=torch.float16)
    vsb = torch.full((slots, H, 8), 5.0, dtype=torch.float16)
    ref.quant_store_int4(k, v, loc, kb, vb, ksb, vsb, None, None)
    pk, sk = ref.quant4(k)
    pv, sv = ref.quant4(v)
    assert torch.equal(kb[loc], pk) and torch.equal(ksb[loc], sk) and torch.equal(vb[loc], pv) and torch.equal(vsb[loc], sv)
    rest = torch.ones(slots, dtype=torch.bool)
    rest[loc] = False
    assert (kb[rest] == 0x55).all() and (vb[rest] == 0x66).all() and (ksb[rest] == 3).all() and (vsb[rest] == 5).all()


def test_evict_closed_form_matches_token_model():
    """The closed form of the evict-mode state (all tokens at once) equals the token-by-token model
    (PosTieredCache.append), for a ring of 64 over 500 positions and for a sequence that starts at a shared
    prefix (ring_start 128) with group 256."""
    gen = torch.Generator().manual_seed(14)
    H, D = 2, 256
    for R, start, n, g8 in ((64, 0, 500, 64), (128, 128, 300, 256), (64, 0, 40, 64)):
        xk = (torch.randn(n, H, D, generator=gen) * 2).to(torch.bfloat16)
        xv = (torch.randn(n, H, D, generator=gen) * 2).to(torch.bfloat16)
        c = ref.PosTieredCache(H, D, n_pages=16, ring_total=R, group8=g8)
        alloc = ref.PageAllocator(16, seed=3)
        shared = [alloc.pop() for _ in range(start // 64)]
        s = c.add_seq(0, R, start, shared)
        for a in range(0, n, 37):
            m = min(37, n - a)
            c.plan_pages(s, m, alloc)
            c.append(s, xk[a:a + m], xv[a:a + m])
        f = ref.evict_closed_form(xk, xv, R, start, g8)
        st = c.seqs[s]
        assert f["hot_start"] == st.hot_start
        assert torch.equal(c.rk[f["ring_rows"]], f["rk"]) and torch.equal(c.rks[f["ring_rows"]], f["rks"])
        assert torch.equal(c.rv[f["ring_rows"]], f["rv"]) and torch.equal(c.rvs[f["ring_rows"]], f["rvs"])
        cold = torch.arange(start, st.hot_start)
        pt = torch.tensor(st.pages, dtype=torch.long)
        rows = pt[cold // 64] * 64 + cold % 64 if cold.numel() else cold
        assert torch.equal(c.k4[rows], f["k4"]) and torch.equal(c.ks4[rows], f["ks4"])
        assert torch.equal(c.v4[rows], f["v4"]) and torch.equal(c.vs4[rows], f["vs4"])


def test_page_allocator_is_the_seeded_permutation():
    """The oracle's allocator hands out torch.randperm(n, seed) in order, each page once, then refuses."""
    a = ref.PageAllocator(50, seed=7)
    got = [a.pop() for _ in range(50)]
    assert got == torch.randperm(50, generator=torch.Generator().manual_seed(7)).tolist() and sorted(got) == list(range(50))
    with pytest.raises(RuntimeError):
        a.pop()


def test_synthetic_inputs():
    """make_kv: V ~ N(0, 1), K ~ N(0, 1) with the 8 outlier channels of each head scaled x8 (distinct channels per
    head from outlier_channels); make_q: N(0, 1) / 16; all bf16."""
    gen = torch.Generator().manual_seed(15)
    och = ref.outlier_channels(2, 256, 8, gen)
    assert och.shape == (2, 8) and all(len(set(r.tolist())) == 8 for r in och)
    k, v = ref.make_kv(20000, 2, 256, gen, och)
    assert k.dtype == v.dtype == torch.bfloat16
    std_k = k.float().std(0)
    for h in range(2):
        mask = torch.zeros(256, dtype=torch.bool)
        mask[och[h]] = True
        assert float((std_k[h, mask] - 8).abs().max()) < 0.3 and float((std_k[h, ~mask] - 1).abs().max()) < 0.05
    assert abs(float(v.float().std()) - 1) < 0.01 and abs(float(v.float().mean())) < 0.01
    q = ref.make_q(16, 256, gen, n=500)
    assert q.shape == (500, 16, 256) and abs(float(q.float().std()) - 1 / 16) < 0.002
