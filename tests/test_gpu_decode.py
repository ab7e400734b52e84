"""GPU parity of split-K decode attention over the tiered cache against the oracle (fp32 softmax over the
bf16-dequantized rows, gemv/test_kv_paged_prefix.py:520-528).

Tolerances: the reference-precision kernel dequantizes exactly like the oracle and accumulates in fp32, so it is
held to 2e-5 max-abs; the MFMA kernel (exact fp16 codes, scales folded in fp32 (K) or into fp16 P (V), fp32
accumulation) to the stated bound 2e-3 max-abs / 1e-3 mean-abs on the configurations' data.  On a single-position
context the MFMA output is exactly code * scale of that V row (checked bit-exact), which differs from the oracle's
bf16 row by at most half a bf16 ulp.
"""
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ = 2, 256, 16
SCALE = D ** -0.5


def _build(lens, rings, seed=0, n_pages=None, chunk=512, starts=None, hq=HQ):
    """Device and oracle caches with the same appended tokens (configuration-style K with outlier channels) and one
    query of hq heads per sequence."""
    from kvtier.kvt import PosTieredCache
    gen = torch.Generator().manual_seed(seed)
    n_pages = n_pages or sum(max(0, l - r) // 64 + 2 for l, r in zip(lens, rings))
    ring_total = sum(rings)
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=ring_total, max_seqs=len(lens),
                        max_pages=max(lens) // 64 + 2, device=dev, page_seed=seed + 1)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=ring_total)
    alloc = ref.PageAllocator(n_pages, seed=seed + 1)
    base = 0
    for r in rings:
        dc.add_seq(r)
        oc.add_seq(base, r)
        base += r
    och = ref.outlier_channels(H, D, 8, gen)
    done = [0] * len(lens)
    while any(d < l for d, l in zip(done, lens)):
        seqs = [s for s in range(len(lens)) if done[s] < lens[s]]
        cnt = [min(chunk, rings[s], lens[s] - done[s]) for s in seqs]
        plan = dc.plan_append(seqs, cnt)
        ks, vs = [], []
        for s, n in zip(seqs, cnt):
            xk, xv = ref.make_kv(n, H, D, gen, och)
            oc.plan_pages(s, n, alloc)
            oc.append(s, xk, xv)
            ks.append(xk); vs.append(xv)
        dc.append(0, plan, torch.cat(ks).to(dev), torch.cat(vs).to(dev))
        dc.commit(plan)
        for s, n in zip(seqs, cnt):
            done[s] += n
    q = ref.make_q(hq, D, gen, n=len(lens))
    oc.alloc = alloc   # the oracle's page allocator, for callers that keep appending
    return dc, oc, q


def _oracle_out(oc, q):
    outs = []
    for s in range(q.shape[0]):
        kk, vv = oc.rows(s)
        outs.append(ref.attention_rows(q[s], kk, vv, SCALE))
    return torch.stack(outs)


@pytest.mark.parametrize("impl,tol,mtol", [("ref", 2e-5, 1e-5), ("mfma", 2e-3, 1e-3)])
def test_decode_pos_rings(kvt_pkg, impl, tol, mtol):
    """4 sequences (3000 / 700 / 130 / 64 positions, rings 1024 / 512 / 256 / 128): hot/cold boundaries inside
    tiles and sub-chunks, partial last tiles, splits of 128 positions with idle wavefronts."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([3000, 700, 130, 64], [1024, 512, 256, 128], seed=1)
    torch.cuda.synchronize()
    out = kvt_decode_attn(dc, 0, q.to(dev), impl=impl).cpu()
    exp = _oracle_out(oc, q)
    err = (out - exp).abs()
    assert float(err.max()) < tol and float(err.mean()) < mtol, (float(err.max()), float(err.mean()))


@pytest.mark.parametrize("hq", [20, 24, 32])
def test_decode_mfma_wide_groups(kvt_pkg, hq):
    """Groups of more than 8 q heads per KV head (10, 12 -- the served model's 24 / 2 -- and 16): the head-wise kernel,
    one head per MFMA column, Q rows read by every wavefront.  Three sequences through the split map and at fixed
    split counts against the oracle; the scalar reference kernel too."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([5000, 2100, 700], [2048, 1024, 256], seed=51, hq=hq)
    qd = q.to(dev)
    exp = _oracle_out(oc, q)
    outs = {"map": kvt_decode_attn(dc, 0, qd, impl="mfma"),
            "splits17": kvt_decode_attn(dc, 0, qd, impl="mfma", splits=17, deterministic=True),
            "ref": kvt_decode_attn(dc, 0, qd, impl="ref")}
    for name, out in outs.items():
        assert out.shape == (3, hq, D), name
        err = (out.cpu() - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (hq, name, float(err.max()), float(err.mean()))


@pytest.mark.parametrize("splits", [1, 3, 17, 64])
def test_decode_mfma_splits(kvt_pkg, splits):
    """The MFMA kernel at several split counts (one to many tiles and ring sub-chunks per wavefront, wavefront
    ranges that straddle the paged / ring boundary, idle wavefronts) against the oracle."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([5000, 2100], [2048, 1024], seed=3)
    out = kvt_decode_attn(dc, 0, q.to(dev), impl="mfma", splits=splits).cpu()
    err = (out - _oracle_out(oc, q)).abs()
    assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (splits, float(err.max()), float(err.mean()))


@pytest.mark.parametrize("splits", [None, 1, 3, 17, 300])
def test_decode_rows_vs_headwise(kvt_pkg, splits):
    """The full-row kernel (both KV heads of a position per wavefront: 16 / 2 heads) against the head-wise kernel
    (headwise=True) and the oracle: three sequences through the split map (splits None) or at fixed split counts
    (one block for a whole sequence up to more blocks than 16-position tiles); both kernels within the oracle
    tolerance, and within 2e-4 of each other (the same products in another fp32 summation order)."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([5000, 2100, 700], [2048, 1024, 256], seed=41)
    qd = q.to(dev)
    exp = _oracle_out(oc, q)
    rows = kvt_decode_attn(dc, 0, qd, impl="mfma", splits=splits)
    head = kvt_decode_attn(dc, 0, qd, impl="mfma", splits=splits, headwise=True)
    for name, out in (("rows", rows), ("head", head)):
        err = (out.cpu() - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (splits, name, float(err.max()))
    assert float((rows - head).abs().max()) <= 2e-4, splits


@pytest.mark.parametrize("lens,rings,splits", [([3000], [512], None), ([20000], [256], 7), ([20000], [256], 300),
                                               ([5000, 2100, 700, 65], [2048, 1024, 256, 64], None), ([17], [16], None)])
def test_decode_plan(kvt_pkg, lens, rings, splits):
    """A decode plan (kvt_decode_plan: every block's ranges and first tile rows, built on the device) gives the same
    result as blocks that compute their ranges themselves -- bit for bit with the fixed tile order -- for one sequence
    at several split counts and a ragged batch through the split map; and within the oracle tolerance."""
    from kvtier.kvt import kvt_decode_attn, kvt_decode_plan
    dc, oc, q = _build(lens, rings, seed=43)
    qd = q.to(dev)
    ws = {}
    plan = kvt_decode_plan(dc, HQ, splits=splits, workspace=ws)
    with_plan = kvt_decode_attn(dc, 0, qd, impl="mfma", plan=plan, workspace=ws, deterministic=True)
    without = kvt_decode_attn(dc, 0, qd, impl="mfma", splits=splits, deterministic=True)
    assert torch.equal(with_plan, without)
    dyn = kvt_decode_attn(dc, 0, qd, impl="mfma", plan=plan, workspace=ws)
    assert float((dyn - without).abs().max()) <= 2e-4
    err = (with_plan.cpu() - _oracle_out(oc, q)).abs()
    assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, float(err.max())


def test_decode_plan_stale(kvt_pkg):
    """A plan older than the cache's sequence state is refused on the host (ValueError); a stale plan that reaches
    the kernel anyway (its version forged here) is caught there: every block whose entry was made for another length
    computes its ranges itself, so the result equals a decode without plan bit for bit (fixed tile order)."""
    from kvtier.kvt import kvt_decode_attn, kvt_decode_plan
    dc, oc, q = _build([6000], [1024], seed=45)
    qd = q.to(dev)
    ws = {}
    plan = kvt_decode_plan(dc, HQ, workspace=ws)
    g = torch.Generator().manual_seed(46)
    xk, xv = ref.make_kv(3, H, D, g, ref.outlier_channels(H, D, 8, g))
    ap = dc.plan_append([0], [3])
    dc.append(0, ap, xk.to(dev), xv.to(dev))
    dc.commit(ap)
    with pytest.raises(ValueError):
        kvt_decode_attn(dc, 0, qd, impl="mfma", plan=plan, workspace=ws)
    plan.version = dc.version
    got = kvt_decode_attn(dc, 0, qd, impl="mfma", plan=plan, workspace=ws, deterministic=True)
    want = kvt_decode_attn(dc, 0, qd, impl="mfma", splits=plan.n_chunks, deterministic=True)
    assert torch.equal(got, want)
    with pytest.raises(ValueError):   # a plan serves the full-row kernel's shapes only
        kvt_decode_plan(dc, 24)


def test_decode_q_range(kvt_pkg):
    """The matrix-core kernels take Q in fp16: a bf16 Q with an entry beyond 65504 or not finite raises ValueError
    outside graph capture; check_q=False skips the check (an even channel beyond the range becomes inf in fp16: the
    output is then not finite)."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([900], [256], seed=47)
    for bad in (7.0e4, float("inf"), float("nan")):
        qb = q.clone()
        qb[0, 3, 16] = bad
        with pytest.raises(ValueError):
            kvt_decode_attn(dc, 0, qb.to(dev), impl="mfma")
        with pytest.raises(ValueError):
            kvt_decode_attn(dc, 0, qb.to(dev), impl="mfma", headwise=True)
    qb = q.clone()
    qb[0, 3, 16] = 7.0e4
    out = kvt_decode_attn(dc, 0, qb.to(dev), impl="mfma", check_q=False)
    assert not bool(torch.isfinite(out[0, 3]).all())
    ok = q.clone()
    ok[0, 3, 17] = 6.5e4                      # within the fp16 range: accepted
    kvt_decode_attn(dc, 0, ok.to(dev), impl="mfma")


def test_combine_ignores_unused_slots(kvt_pkg):
    """Partial slots beyond the splits a sequence uses may hold anything (here NaN, left in a reused workspace): the
    combine kernel loads them with the others but must not let them into the sum (reference-precision path with
    more chunks than the context needs, and the MFMA path with a ragged split map)."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([3000, 700], [1024, 512], seed=41)
    qd = q.to(dev)
    exp = _oracle_out(oc, q)
    for kw in (dict(impl="ref", chunk=256, max_len=20000), dict(impl="mfma", deterministic=True)):
        ws = {}
        kvt_decode_attn(dc, 0, qd, workspace=ws, **kw)
        ws["part_o"].fill_(float("nan"))
        ws["part_ml"].fill_(float("nan"))
        out = kvt_decode_attn(dc, 0, qd, workspace=ws, **kw).cpu()
        assert not bool(torch.isnan(out).any()), kw
        err = (out - exp).abs()
        assert float(err.max()) < 2e-3, (kw, float(err.max()))


def test_decode_mfma_page_windows(kvt_pkg):
    """One split over 40,000 positions: each wavefront walks about 9,000 paged positions, i.e. several 64-page
    windows of page ids."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([40000], [1024], seed=5, chunk=1024)
    out = kvt_decode_attn(dc, 0, q.to(dev), impl="mfma", splits=1).cpu()
    err = (out - _oracle_out(oc, q)).abs()
    assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (float(err.max()), float(err.mean()))


@pytest.mark.parametrize("hq", [16, 24])
def test_decode_mfma_closed_forms(kvt_pkg, hq):
    """Hot: a single ring position gives out == code * scale of its V row in fp32 (P = 1; the scale enters the matrix
    product through P and the fp16 x fp16 products are exact).  Cold: 64 identical rows in a shared INT4 page
    (positions below ring_start) give uniform attention, out == code * scale of that row; the V row is k / 8 with
    integers k in -7..7 and +-7 in every group of 32 channels, so every scale is exactly 1/8 and every partial sum of
    the kernel (raw 1024 + n / 1024 + 16 n values times 1/8 or 1/128, the constant excess removed per tile) is a
    small multiple of 1/8: exact in fp32.  16 q heads (groups of 8) and 24 (groups of 12, one head per column)."""
    from kvtier import sparse_attn as sa
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    gen = torch.Generator().manual_seed(4)
    q = ref.make_q(hq, D, gen)
    gs = hq // H
    xk = (torch.randn(1, H, D, generator=gen) * 2).to(torch.bfloat16)
    xv = (torch.randn(1, H, D, generator=gen) * 2).to(torch.bfloat16)
    # hot
    dc = PosTieredCache(1, H, D, n_pages=2, ring_total=64, max_seqs=1, max_pages=2, device=dev)
    dc.add_seq(64)
    plan = dc.plan_append([0], [1])
    dc.append(0, plan, xk.to(dev), xv.to(dev))
    dc.commit(plan)
    out = kvt_decode_attn(dc, 0, q.to(dev), impl="mfma").cpu()
    vrow = dc.rv[0][0].cpu().float() * dc.rvs[0][0].cpu().float().repeat_interleave(64, -1)
    for i in range(hq):
        assert torch.equal(out[0, i], vrow[i // gs]), ("hot", i)
    # cold: page 1 holds 64 copies of the row, written by the INT4 writer; the sequence starts at position 64
    dc = PosTieredCache(1, H, D, n_pages=2, ring_total=64, max_seqs=1, max_pages=2, device=dev)
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    kv = torch.randint(-7, 8, (H, D), generator=gen)
    kv[:, ::32] = 7
    xv_c = (kv.float() / 8).to(torch.bfloat16).unsqueeze(0)
    sa.quant_store_kv_int4(xk.expand(64, H, D).contiguous().to(dev), xv_c.expand(64, H, D).contiguous().to(dev),
                           torch.arange(64, 128, device=dev), dc.k4[0], dc.v4[0], dc.ks4[0], dc.vs4[0], ones, ones)
    dc.add_seq(64, ring_start=64, shared_pages=[1])
    out = kvt_decode_attn(dc, 0, q.to(dev), impl="mfma").cpu()
    codes = ref.unpack4(dc.v4[0][64].cpu()).float()
    vrow = codes * dc.vs4[0][64].cpu().float().repeat_interleave(32, -1)
    assert torch.equal(dc.vs4[0][64].cpu().float(), torch.full((H, 8), 0.125)) and torch.equal(vrow, kv.float() / 8)
    for i in range(hq):
        assert torch.equal(out[0, i], vrow[i // gs]), ("cold", i)


def test_decode_mfma_group256(kvt_pkg):
    """Per-(token, head) INT8 ring scales (group 256) on the MFMA path."""
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    gen = torch.Generator().manual_seed(6)
    L, R = 1500, 512
    dc = PosTieredCache(1, H, D, n_pages=32, ring_total=R, max_seqs=1, max_pages=32, device=dev, group8=256)
    oc = ref.PosTieredCache(H, D, n_pages=32, ring_total=R, group8=256)
    alloc = ref.PageAllocator(32, seed=0)
    dc.add_seq(R)
    oc.add_seq(0, R)
    och = ref.outlier_channels(H, D, 8, gen)
    for a in range(0, L, 300):
        n = min(300, L - a)
        xk, xv = ref.make_kv(n, H, D, gen, och)
        plan = dc.plan_append([0], [n])
        dc.append(0, plan, xk.to(dev), xv.to(dev))
        dc.commit(plan)
        oc.plan_pages(0, n, alloc)
        oc.append(0, xk, xv)
    q = ref.make_q(HQ, D, gen)
    for impl, tol in (("ref", 2e-5), ("mfma", 2e-3)):
        out = kvt_decode_attn(dc, 0, q.to(dev), impl=impl).cpu()
        err = (out - _oracle_out(oc, q)).abs()
        assert float(err.max()) < tol, (impl, float(err.max()))


def test_decode_pos_single_and_empty(kvt_pkg):
    """A single-token context returns exactly its V row; an empty context is NaN (0/0)."""
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    dc, oc, q = _build([1, 5], [64, 64], seed=2)
    out = kvt_decode_attn(dc, 0, q.to(dev), impl="ref").cpu()
    kk, vv = oc.rows(0)
    assert torch.equal(out[0, :8], vv[0, 0].float().expand(8, D)) and torch.equal(out[0, 8:], vv[0, 1].float().expand(8, D))
    empty = PosTieredCache(1, H, D, n_pages=2, ring_total=64, max_seqs=1, max_pages=2, device=dev)
    empty.add_seq(64)
    o = kvt_decode_attn(empty, 0, q[:1].to(dev), impl="ref", max_len=1)
    assert torch.isnan(o).all()


def test_decode_slot_rings_config0(kvt_pkg):
    """The CPU-plumbing configuration on the GPU: 4,096 tokens appended one at a time through the dual-write path
    (R = 512, per-(token, head) INT8, identity slots), then one decode step; codes bit-exact, output vs oracle."""
    from kvtier import sparse_attn as sa
    from kvtier.kvt import decode_attn_slots
    gen = torch.Generator().manual_seed(0)
    N, R = 4096, 512
    och = ref.outlier_channels(H, D, 8, gen)
    xk, xv = ref.make_kv(N, H, D, gen, och)
    q = ref.make_q(HQ, D, gen)
    k4 = torch.zeros(N, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
    ks4 = torch.zeros(N, H, 8, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
    rk = torch.zeros(R, H, D, dtype=torch.int8, device=dev); rv = torch.zeros_like(rk)
    rks = torch.zeros(R, H, 1, dtype=torch.float16, device=dev); rvs = torch.zeros_like(rks)
    owner = torch.full((R,), -1, dtype=torch.int32, device=dev)
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    xk_d, xv_d = xk.to(dev), xv.to(dev)
    locs = torch.arange(N, dtype=torch.int32, device=dev)
    for t in range(N):
        sa.quant_store_kv_tiered(xk_d[t:t + 1], xv_d[t:t + 1], locs[t:t + 1], k4, v4, ks4, vs4, rk, rv, rks, rvs, owner,
                                 ones, ones, R - 1)
    torch.cuda.synchronize()
    e = [torch.zeros(N, H, D // 2, dtype=torch.uint8), torch.zeros(N, H, D // 2, dtype=torch.uint8),
         torch.zeros(N, H, 8, dtype=torch.float16), torch.zeros(N, H, 8, dtype=torch.float16),
         torch.zeros(R, H, D, dtype=torch.int8), torch.zeros(R, H, D, dtype=torch.int8),
         torch.zeros(R, H, 1, dtype=torch.float16), torch.zeros(R, H, 1, dtype=torch.float16),
         torch.full((R,), -1, dtype=torch.int32)]
    for a in range(0, N, R):
        ref.quant_store_tiered(xk[a:a + R], xv[a:a + R], torch.arange(a, a + R), *e, None, None, R - 1, group8=256)
    got = [t.cpu() for t in (k4, v4, ks4, vs4, rk, rv, rks, rvs, owner)]
    for i in range(9):
        assert torch.equal(got[i], e[i]), i
    rtt = torch.arange(N, dtype=torch.int32, device=dev)[None]
    kk, vv = ref.dequant_slots_tiered(torch.arange(N), *e, R - 1, group8=256)
    exp = ref.attention_rows(q[0], kk, vv, SCALE)
    for impl, tol, mtol in (("ref", 2e-5, 2e-5), ("mfma", 2e-3, 1e-3)):
        out = decode_attn_slots(q.to(dev), torch.tensor([N], dtype=torch.int32, device=dev), rtt,
                                torch.zeros(1, dtype=torch.int64, device=dev), k4, v4, ks4, vs4, rk, rv, rks, rvs,
                                owner, R - 1, impl=impl).cpu()
        err = (out[0] - exp).abs()
        assert float(err.max()) < tol and float(err.mean()) < mtol, (impl, float(err.max()))


@pytest.mark.parametrize("hq,lens", [(16, [5000, 1300, 64]), (24, [5000, 1300, 64]), (16, [20000, 9000, 300, 17])])
def test_decode_slots_mfma_ragged(kvt_pkg, hq, lens):
    """Dense decode over the slot-indexed tiered pool through the matrix cores: requests of 5,000 / 1,300 / 64
    positions (one 16-column tile per wavefront), and of 20,000 / 9,000 / 300 / 17 (past 1,024 blocks of 64 columns:
    each wavefront loops over several tiles) on randomly permuted slots of one pool, ring of 1,024 rows with owners
    from the dual write (the ring has wrapped: most positions are INT4 rows, the newest are ring rows), G64 ring
    scales, smoothing factors, against the oracle's gathered rows and fp32 attention."""
    from kvtier import sparse_attn as sa
    from kvtier.kvt import decode_attn_slots
    gen = torch.Generator().manual_seed(61)
    R = 1024
    slots = 8192 if sum(lens) <= 8192 else 32768
    och = ref.outlier_channels(H, D, 8, gen)
    perm = torch.randperm(slots, generator=gen).to(torch.int32)
    r2t = torch.full((len(lens) + 1, max(lens) + 100), -7, dtype=torch.int32)
    req_idx = torch.tensor([2, 0, 3, 1][:len(lens)], dtype=torch.int64)
    a = 0
    for b, L in enumerate(lens):
        r2t[int(req_idx[b]), :L] = perm[a:a + L]
        a += L
    k4 = torch.zeros(slots, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
    ks4 = torch.zeros(slots, H, 8, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
    rk = torch.zeros(R, H, D, dtype=torch.int8, device=dev); rv = torch.zeros_like(rk)
    rks = torch.zeros(R, H, 4, dtype=torch.float16, device=dev); rvs = torch.zeros_like(rks)
    owner = torch.full((R,), -1, dtype=torch.int32, device=dev)
    sm = (0.5 + torch.rand(H, D, generator=gen)).half()
    smi = (1.0 / sm.float()).half()
    xs = []
    for b, L in enumerate(lens):   # the dual write in position order, request by request
        xk, xv = ref.make_kv(L, H, D, gen, och)
        locs = r2t[int(req_idx[b]), :L].long()
        for c0 in range(0, L, 512):
            c1 = min(L, c0 + 512)
            sa.quant_store_kv_tiered(xk[c0:c1].to(dev), xv[c0:c1].to(dev), locs[c0:c1].to(dev), k4, v4, ks4, vs4, rk,
                                     rv, rks, rvs, owner, smi.to(dev), smi.to(dev), R - 1)
    torch.cuda.synchronize()
    q = ref.make_q(hq, D, gen, n=len(lens))
    seq = torch.tensor(lens, dtype=torch.int32)
    out = decode_attn_slots(q.to(dev), seq.to(dev), r2t.to(dev), req_idx.to(dev), k4, v4, ks4, vs4, rk, rv, rks, rvs,
                            owner, R - 1, sm_k=sm.to(dev), sm_v=sm.to(dev)).cpu()
    pools = [t.cpu() for t in (k4, v4, ks4, vs4, rk, rv, rks, rvs, owner)]
    for b, L in enumerate(lens):
        kk, vv = ref.dequant_slots_tiered(r2t[int(req_idx[b]), :L].long(), *pools, R - 1, group8=64, sm_k=sm,
                                          sm_v=sm)
        exp = ref.attention_rows(q[b], kk, vv, SCALE)
        err = (out[b] - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (hq, b, float(err.max()), float(err.mean()))


@pytest.mark.parametrize("deterministic", [True, False])
def test_decode_graph_replay(kvt_pkg, deterministic):
    """The decode step (split-K + combine) captured in a HIP graph: every replay, with eager work and
    synchronizations in between, equals the eager result -- bit for bit with the fixed tile order; with tiles taken
    first come only the fp32 summation order differs (partial sums carry the 1032 x excess of the raw codes until it
    is removed per tile, so reordering moves the result by about 1e-4 of its scale: bound 2e-4 absolute, a tenth of
    the oracle tolerance), and every replay stays within the oracle tolerance."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([2500, 900], [1024, 512], seed=7)
    qd = q.to(dev)
    ws = {}
    eager = kvt_decode_attn(dc, 0, qd, impl="mfma", workspace=ws, deterministic=deterministic).clone()
    out = torch.empty_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        kvt_decode_attn(dc, 0, qd, out=out, impl="mfma", workspace=ws, deterministic=deterministic)
    exp = _oracle_out(oc, q)
    for i in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        if deterministic:
            assert torch.equal(out, eager), f"replay {i}"
        else:
            assert float((out - eager).abs().max()) <= 2e-4, f"replay {i}"
        err = (out.cpu() - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (i, float(err.max()))
        _ = (qd.float() * 2).sum()          # unrelated eager work between replays
        torch.cuda.synchronize()


def test_decode_steps_with_append(kvt_pkg):
    """Decode with append (the 1,000-step configuration at a reduced size): 500 positions, ring 128, then 40 steps of
    append-one-token (each evicting the oldest ring row into INT4 pages) + MFMA decode; every step's output against the
    oracle, codes and page table bit-exact at the end."""
    from kvtier.kvt import kvt_decode_attn
    dc, oc, q = _build([500], [128], seed=21)
    gen = torch.Generator().manual_seed(22)
    och = ref.outlier_channels(H, D, 8, gen)
    alloc = oc.alloc
    ws = {}
    for step in range(40):
        xk, xv = ref.make_kv(1, H, D, gen, och)
        plan = dc.plan_append([0], [1])
        dc.append(0, plan, xk.to(dev), xv.to(dev))
        dc.commit(plan)
        oc.plan_pages(0, 1, alloc)
        oc.append(0, xk, xv)
        qs = ref.make_q(HQ, D, gen)
        out = kvt_decode_attn(dc, 0, qs.to(dev), impl="mfma", workspace=ws).cpu()
        err = (out - _oracle_out(oc, qs)).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (step, float(err.max()))
    for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
        assert torch.equal(getattr(dc, name)[0].cpu(), getattr(oc, name)), name
    assert torch.equal(dc.page_table.cpu()[0, :len(oc.seqs[0].pages)], torch.tensor(oc.seqs[0].pages, dtype=torch.int32))


def test_decode_ragged_shared_prefix(kvt_pkg):
    """Ragged batch (the 8-sequence configuration at a reduced size): 4 sequences of different lengths and rings;
    sequences 0 and 1 share a 128-position prefix held in two common INT4 pages (paged-prefix reuse); 6 iterations of
    one append + one batched MFMA decode step per sequence, each against the oracle."""
    from kvtier import sparse_attn as sa
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    gen = torch.Generator().manual_seed(23)
    och = ref.outlier_channels(H, D, 8, gen)
    lens, rings = [700, 420, 90, 1500], [256, 128, 128, 512]
    n_pages = 64
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=sum(rings), max_seqs=4, max_pages=40, device=dev,
                        page_seed=6)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=sum(rings))
    alloc = ref.PageAllocator(n_pages, seed=6)
    shared = [dc.alloc.pop(), dc.alloc.pop()]
    assert shared == [alloc.pop(), alloc.pop()]
    pk, pv = ref.make_kv(128, H, D, gen, och)
    rows = torch.tensor([p * 64 + i for p in shared for i in range(64)])
    ones = torch.ones(H, D, dtype=torch.float16)
    sa.quant_store_kv_int4(pk.to(dev), pv.to(dev), rows.to(dev), dc.k4[0], dc.v4[0], dc.ks4[0], dc.vs4[0],
                           ones.to(dev), ones.to(dev))
    ref.quant_store_int4(pk, pv, rows, oc.k4, oc.v4, oc.ks4, oc.vs4, ones, ones)
    base = 0
    for s, r in enumerate(rings):
        start, pages = (128, shared) if s < 2 else (0, ())
        dc.add_seq(r, ring_start=start, shared_pages=pages)
        oc.add_seq(base, r, ring_start=start, shared_pages=pages)
        base += r
    done = [128, 128, 0, 0]
    while any(d < l for d, l in zip(done, lens)):
        seqs = [s for s in range(4) if done[s] < lens[s]]
        cnt = [min(rings[s], lens[s] - done[s]) for s in seqs]
        plan = dc.plan_append(seqs, cnt)
        ks, vs = [], []
        for s, m in zip(seqs, cnt):
            xk, xv = ref.make_kv(m, H, D, gen, och)
            oc.plan_pages(s, m, alloc)
            oc.append(s, xk, xv)
            ks.append(xk)
            vs.append(xv)
        dc.append(0, plan, torch.cat(ks).to(dev), torch.cat(vs).to(dev))
        dc.commit(plan)
        for s, m in zip(seqs, cnt):
            done[s] += m
    for it in range(6):
        xk, xv = ref.make_kv(4, H, D, gen, och)
        plan = dc.plan_append([0, 1, 2, 3], [1, 1, 1, 1])
        dc.append(0, plan, xk.to(dev), xv.to(dev))
        dc.commit(plan)
        for s in range(4):
            oc.plan_pages(s, 1, alloc)
            oc.append(s, xk[s:s + 1], xv[s:s + 1])
        qs = ref.make_q(HQ, D, gen, n=4)
        out = kvt_decode_attn(dc, 0, qs.to(dev), impl="mfma").cpu()
        err = (out - _oracle_out(oc, qs)).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (it, float(err.max()), float(err.mean()))
