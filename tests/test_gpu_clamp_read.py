"""Read side of the reference's clamp regime (gemv/test_kv_tiers.py:412-456, gemv/test_kv_int4.py:256-289): a row
whose head-0 group 0 holds +-1e6 / 5e5 / 4.6e5 / 1e5 and whose head-1 group 2 (channels 64-95) is bf16 max is written
through the writers (scales clamp to 65504, never inf), then read back through every reader:

* the compact and prefix gathers: the row bit-exact against the oracle's dequant and every gathered row finite,
  first from the INT8 ring (the row's slot owns its ring row), then from the INT4 pool after the owner flips;
* the fused top-k decode (kvt_sparse_decode), the paged prefix-chunk attention (sparse_gqa_fwd_interface_paged)
  and the position-cache split-K decode (kvt_decode_mfma, the row in the ring and, after later appends, requantized
  into an INT4 page): all outputs finite and within 2e-3 + 2^-10 sum_i p_i |v_i| of the oracle's fp32 attention.

The queries are zero on the saturated channels, so the scores stay ordinary while K rows reach 127 * 65504 (beyond
fp16) and the saturated V rows reach every output.  The bound's second term is twice the error of the weights'
rounding: the gathers' readers round each weight once to 11 bits (2^-11 relative, bound 2^-10 sum p|v|); the split-K
decode kernels round it twice -- p to fp16, then p times the V scale to fp16, the scale folded into the weight of the
fp16 P.V product -- so theirs is 2^-9 sum p|v|."""
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ = 2, 256, 16
SLOTS, R, L, POS7 = 2048, 64, 512, 17
SCALE = D ** -0.5


def _big_row():
    big = torch.zeros(H, D)
    big[0, :32] = torch.tensor([1e6, -1e6, 5e5, -5e5, 4.6e5, -4.6e5, 1e5, -1e5] * 4)
    big[1, 64:96] = torch.finfo(torch.bfloat16).max
    return big.to(torch.bfloat16)


def _zero_big_channels(q):
    """q [..., HQ, D]: q heads 0-7 read KV head 0, 8-15 KV head 1; zero where the clamp row saturates."""
    q = q.clone()
    q[..., :8, :32] = 0
    q[..., 8:, 64:96] = 0
    return q


@pytest.fixture(scope="module")
def clamp_pool():
    """A tiered slot pool written by the dual writer (random rows, identity smoothing), one request of L positions on
    a permutation of the slots, the clamp row written last at the slot of position POS7 (so its slot owns its ring
    row).  Returns device buffers and the request."""
    import kvtier  # noqa: F401
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(77)
    k16 = (torch.randn(SLOTS, H, D, generator=gen) * 2).to(torch.bfloat16)
    v16 = (torch.randn(SLOTS, H, D, generator=gen) * 2).to(torch.bfloat16)
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    k4 = torch.zeros(SLOTS, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
    ks4 = torch.zeros(SLOTS, H, D // 32, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
    rk = torch.zeros(R, H, D, dtype=torch.int8, device=dev); rv = torch.zeros_like(rk)
    rks = torch.zeros(R, H, D // 64, dtype=torch.float16, device=dev); rvs = torch.zeros_like(rks)
    owner = torch.full((R,), -1, dtype=torch.int32, device=dev)
    bufs = (k4, v4, ks4, vs4, rk, rv, rks, rvs, owner)
    for a in range(0, SLOTS, R):
        sa.quant_store_kv_tiered(k16[a:a + R].to(dev), v16[a:a + R].to(dev),
                                 torch.arange(a, a + R, dtype=torch.int32, device=dev), *bufs, ones, ones, R - 1)
    r2t = torch.randperm(SLOTS, generator=gen)[:L].to(torch.int32)[None]
    slot7 = int(r2t[0, POS7])
    big = _big_row()
    sa.quant_store_kv_tiered(big[None].to(dev), (-big)[None].to(dev), torch.tensor([slot7], dtype=torch.int32,
                             device=dev), *bufs, ones, ones, R - 1)
    torch.cuda.synchronize()
    q8, s8 = ref.quant8(big[None])
    q8v, s8v = ref.quant8((-big)[None])
    p4, s4 = ref.quant4(big[None])
    p4v, s4v = ref.quant4((-big)[None])
    # the write side, as the reference asserts it: clamped scales, codes and scales bit-exact
    assert float(s8[0, 1, 1]) == 65504.0 and float(s4[0, 1, 2]) == 65504.0 and float(s4[0, 0, 0]) == 65504.0
    assert int(owner[slot7 & (R - 1)]) == slot7
    assert torch.equal(rk[slot7 & (R - 1)].cpu(), q8[0]) and torch.equal(rks[slot7 & (R - 1)].cpu(), s8[0])
    assert torch.equal(rv[slot7 & (R - 1)].cpu(), q8v[0]) and torch.equal(rvs[slot7 & (R - 1)].cpu(), s8v[0])
    assert torch.equal(k4[slot7].cpu(), p4[0]) and torch.equal(ks4[slot7].cpu(), s4[0])
    assert torch.equal(v4[slot7].cpu(), p4v[0]) and torch.equal(vs4[slot7].cpu(), s4v[0])
    d8 = (ref.dequant8(q8, s8)[0], ref.dequant8(q8v, s8v)[0])
    d4 = (ref.dequant4(p4, s4)[0], ref.dequant4(p4v, s4v)[0])
    assert float(d8[0][1, 64]) == float(torch.tensor(127 * 65504.0).to(torch.bfloat16))
    assert float(d4[0][0, 0]) == float(torch.tensor(7 * 65504.0).to(torch.bfloat16))
    return dict(bufs=bufs, ones=ones, r2t=r2t, slot7=slot7, d8=d8, d4=d4, gen=gen)


def _rows(st):
    """The oracle's dequantized K, V rows of the request's L positions from the pool's current device state."""
    k4, v4, ks4, vs4, rk, rv, rks, rvs, owner = (t.cpu() for t in st["bufs"])
    return ref.dequant_slots_tiered(st["r2t"][0], k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, R - 1)


def _tier_kw(st):
    k4, v4, ks4, vs4, rk, rv, rks, rvs, owner = st["bufs"]
    return dict(k_scale=ks4, v_scale=vs4, sm_k=st["ones"], sm_v=st["ones"], kv_bits=4, ring_k=rk, ring_v=rv,
                ring_ks=rks, ring_vs=rvs, owner=owner, ring_mask=R - 1)


def _within(out, exp, bound, what):
    assert torch.isfinite(out).all(), what
    assert float(exp.abs().max()) > 100, what                    # the saturated V rows reach the outputs
    excess = (out - exp).abs() - (2e-3 + bound)
    assert float(excess.max()) <= 0, (what, float(excess.max()))


def _gathers(st, want):
    """Compact gather of a top-k row holding POS7 and prefix gather of positions 0 .. POS7 + 7: the clamp row equals
    `want` bit for bit, every gathered row equals the oracle's and is finite."""
    from kvtier import sparse_attn as sa
    k4, v4 = st["bufs"][0], st["bufs"][1]
    kk, vv = _rows(st)
    g = torch.Generator().manual_seed(5)
    idx = torch.randperm(L, generator=g)[:64]
    idx[0] = POS7
    idx = idx.sort().values.to(torch.int32)[None]
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    counts = torch.empty(1, dtype=torch.int32, device=dev)
    cu = torch.empty(2, dtype=torch.int32, device=dev)
    sa.qwen_sparse_fa2_cu_seqlens_triton(seq, idx.to(dev), counts, cu, 1, 64)
    ok = torch.full((64, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
    ov = torch.full_like(ok, float("nan"))
    ridx = torch.zeros(1, dtype=torch.int64, device=dev)
    sa.qwen_sparse_kv_extraction_compact_triton(k4, v4, st["r2t"].to(dev), ridx, idx.to(dev), seq, cu, ok, ov, 1, 64,
                                                **_tier_kw(st))
    n = POS7 + 8
    pk = torch.full((n, H, D), float("nan"), dtype=torch.bfloat16, device=dev)
    pv = torch.full_like(pk, float("nan"))
    kw = _tier_kw(st)
    sa.qwen_sparse_prefix_gather_dequant_tiered(k4, v4, kw["k_scale"], kw["v_scale"], st["ones"], st["ones"],
                                                st["r2t"].to(dev), ridx, torch.tensor([n], dtype=torch.int32,
                                                device=dev), torch.tensor([0, n], dtype=torch.int32, device=dev),
                                                pk, pv, 1, n, ring_k=kw["ring_k"], ring_v=kw["ring_v"],
                                                ring_ks=kw["ring_ks"], ring_vs=kw["ring_vs"], owner=kw["owner"],
                                                ring_mask=R - 1)
    torch.cuda.synchronize()
    ok, ov, pk, pv = ok.cpu(), ov.cpu(), pk.cpu(), pv.cpu()
    sel = idx[0].long()
    assert all(bool(torch.isfinite(t).all()) for t in (ok, ov, pk, pv)), "a gather produced inf / NaN"
    assert torch.equal(ok, kk[sel]) and torch.equal(ov, vv[sel])
    assert torch.equal(pk, kk[:n]) and torch.equal(pv, vv[:n])
    r7 = int((sel == POS7).nonzero()[0, 0])
    assert torch.equal(ok[r7], want[0]) and torch.equal(ov[r7], want[1])
    assert torch.equal(pk[POS7], want[0]) and torch.equal(pv[POS7], want[1])


def _attention(st):
    """Top-k decode over all L positions and a 32-query prefix chunk (queries at L - 32 .. L - 1, each selecting every
    visible position), against the oracle with the clamp bound."""
    from kvtier import sparse_attn as sa
    k4, v4 = st["bufs"][0], st["bufs"][1]
    kk, vv = _rows(st)
    g = torch.Generator().manual_seed(9)
    # fused top-k decode, every position selected
    q = _zero_big_channels((torch.randn(1, HQ, D, generator=g) / 4).to(torch.bfloat16))
    idx = torch.arange(L, dtype=torch.int32)[None]
    seq = torch.tensor([L], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, L], dtype=torch.int32, device=dev)
    ridx = torch.zeros(1, dtype=torch.int64, device=dev)
    kw = _tier_kw(st)
    out = sa.qwen_sparse_decode_attn(q.to(dev), k4, v4, st["r2t"].to(dev), ridx, idx.to(dev), seq, cu, 1, L, **kw)
    torch.cuda.synchronize()
    exp = ref.attention_rows(q[0], kk, vv, SCALE)
    bound = 2.0 ** -10 * ref.attention_rows(q[0], kk, vv.abs(), SCALE)
    _within(out.cpu()[0].float(), exp, bound, "kvt_sparse_decode")
    # paged prefix-chunk attention: 32 queries, the clamp row visible to all
    nq = 32
    qc = _zero_big_channels((torch.randn(nq, HQ, D, generator=g) / 4).to(torch.bfloat16))
    idxc = torch.full((nq, L), -1, dtype=torch.int32)
    for j in range(nq):
        vis = L - nq + j + 1
        idxc[j, :vis] = torch.arange(vis, dtype=torch.int32)
    outc = torch.empty(nq, HQ, D, dtype=torch.float32, device=dev)
    sa.sparse_gqa_fwd_interface_paged(qc.to(dev), idxc.to(dev), torch.tensor([0, nq], dtype=torch.int64, device=dev),
                                      seq, st["r2t"].to(dev), ridx, scale=SCALE, max_q=nq, out=outc, k_buf=k4,
                                      v_buf=v4, **kw)
    torch.cuda.synchronize()
    for j in range(nq):
        vis = L - nq + j + 1
        e = ref.attention_rows(qc[j], kk[:vis], vv[:vis], SCALE)
        b = 2.0 ** -10 * ref.attention_rows(qc[j], kk[:vis], vv[:vis].abs(), SCALE)
        _within(outc.cpu()[j], e, b, ("sparse_gqa_fwd_interface_paged", j))


def test_clamp_rows_hot_then_int4(clamp_pool):
    """The clamp row from the INT8 ring (its slot owns the ring row), then -- the owner flipped to another slot of
    the same residue class -- from the INT4 pool: gathers bit-exact and finite, attention within the clamp bound."""
    st = clamp_pool
    owner = st["bufs"][8]
    slot7 = st["slot7"]
    _gathers(st, st["d8"])
    _attention(st)
    prev = int(owner[slot7 & (R - 1)])
    owner[slot7 & (R - 1)] = slot7 + R if slot7 + R < SLOTS else slot7 - R
    try:
        _gathers(st, st["d4"])
        _attention(st)
    finally:
        owner[slot7 & (R - 1)] = prev
        torch.cuda.synchronize()


def test_clamp_rows_position_cache_decode(kvt_pkg):
    """The position cache (ring 128): clamp rows appended at positions 5 / 40 / 150 / 250 / 300 through the quantize-
    append; after each chunk the early ones have been requantized into INT4 pages (scale 65504) and the late ones sit
    in the INT8 ring.  kvt_decode_attn (split-K matrix-core kernel, both kernels' grids) over the whole context:
    finite and within the clamp bound of the oracle's attention over the oracle cache's rows."""
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    gen = torch.Generator().manual_seed(21)
    och = ref.outlier_channels(H, D, 8, gen)
    ring, n_pages = 128, 64
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=ring, max_seqs=1, max_pages=n_pages, device=dev,
                        page_seed=21)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=ring)
    alloc = ref.PageAllocator(n_pages, seed=21)
    dc.add_seq(ring)
    oc.add_seq(0, ring)
    big = _big_row()
    a = 0
    for n in (96, 96, 96, 80):
        xk, xv = ref.make_kv(n, H, D, gen, och)
        for p in (5, 40, 150, 250, 300):
            if a <= p < a + n:
                xk[p - a] = big
                xv[p - a] = -big
        plan = dc.plan_append([0], [n])
        dc.append(0, plan, xk.to(dev), xv.to(dev))
        dc.commit(plan)
        oc.plan_pages(0, n, alloc)
        oc.append(0, xk, xv)
        a += n
        kk, vv = oc.rows(0)
        q = _zero_big_channels(ref.make_q(HQ, D, gen, n=1))
        exp = ref.attention_rows(q[0], kk, vv, SCALE)
        bound = 2.0 ** -9 * ref.attention_rows(q[0], kk, vv.abs(), SCALE)   # two roundings of each weight
        for headwise in (False, True):
            for splits in (None, 3):
                out = kvt_decode_attn(dc, 0, q.to(dev), impl="mfma", splits=splits, headwise=headwise)
                torch.cuda.synchronize()
                _within(out.cpu()[0], exp, bound, ("kvt_decode_mfma", a, headwise, splits))
