"""GPU parity of the causal prefill kernel (kvt_prefill_attn) against the oracle.

Chunked prefill as the reference serves it (patches/kv_paged_prefix.py:200, docs/KV_PAGED_PREFIX_PLAN.md:21-23): the
first chunk attends to its own fresh bf16 K/V; every later chunk is first appended to the cache (the ring's oldest
rows requantized into INT4 pages) and then attends to all positions up to its own, read back from the tiers.  The
oracle is fp32 softmax attention over the oracle cache's bf16-dequantized rows (gemv/test_kv_paged_prefix.py:506-531).
Tolerance: 2e-3 max-abs / 1e-3 mean-abs on fp32 outputs (bf16 K/Q equal to the oracle's, V the oracle's bf16 rows
/ 128 in fp16, P rounded to fp16 with the row sum over the rounded values, fp32 accumulation); the bf16 output is the
fp32 output rounded to nearest even, bit for bit.  The clamp regime (groups saturating the fp16 scale at 65504,
gemv/test_kv_tiers.py:412-456) adds 2^-10 * sum_i p_i |v_i|: P's 11 significant bits (relative rounding <= 2^-11 of
each weight, so at most 2^-11 sum_i p_i |v_i - o| <= 2^-10 sum_i p_i |v_i|) against V rows of up to 127 * 65504.  The
reference's kernel rounds P to bf16 (8 bits) before its P.V product (patches/kv_paged_prefix.py:251-252).
"""
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ = 2, 256, 16
SCALE = D ** -0.5


def _chunked(lens_chunks, ring, seed, group8=64, n_pages=64, edit=None):
    """Append chunks to a device and an oracle cache (one sequence); yield (start, n, xk, xv, dc, oc) after each
    chunk's append.  `edit(start, xk, xv)` may change a chunk's rows before they are appended."""
    from kvtier.kvt import PosTieredCache
    gen = torch.Generator().manual_seed(seed)
    och = ref.outlier_channels(H, D, 8, gen)
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=ring, max_seqs=1, max_pages=n_pages, device=dev,
                        page_seed=seed, group8=group8)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=ring, group8=group8)
    alloc = ref.PageAllocator(n_pages, seed=seed)
    dc.add_seq(ring)
    oc.add_seq(0, ring)
    a = 0
    for n in lens_chunks:
        xk, xv = ref.make_kv(n, H, D, gen, och)
        if edit is not None:
            edit(a, xk, xv)
        done = 0
        while done < n:   # one append never exceeds the ring
            m = min(ring, n - done)
            plan = dc.plan_append([0], [m])
            dc.append(0, plan, xk[done:done + m].to(dev), xv[done:done + m].to(dev))
            dc.commit(plan)
            oc.plan_pages(0, m, alloc)
            oc.append(0, xk[done:done + m], xv[done:done + m])
            done += m
        yield a, n, xk, xv, dc, oc, gen
        a += n


def _oracle_chunk(q, a, kk, vv):
    """Causal attention of queries at positions a .. a + n - 1 over rows kk / vv [>= a + n, H, D]."""
    return torch.stack([ref.attention_rows(q[j], kk[:a + j + 1], vv[:a + j + 1], SCALE) for j in range(q.shape[0])])


@pytest.mark.parametrize("group8", [64, 256])
def test_prefill_chunks_vs_oracle(kvt_pkg, group8):
    """4 chunks of 96 queries, ring 128: chunk 0 from bf16, chunks 1-3 from the tiers (positions below hot_start in
    INT4 pages after evict-requant); ragged last query tile (96 = 6 x 16)."""
    from kvtier.kvt import kvt_prefill_attn
    for a, n, xk, xv, dc, oc, gen in _chunked([96, 96, 96, 80], 128, seed=11, group8=group8):
        q = ref.make_q(HQ, D, gen, n=n)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        if a == 0:
            k_src, v_src = xk.to(dev), xv.to(dev)
            out = kvt_prefill_attn(dc, 0, q.to(dev), cu, k_src=k_src, v_src=v_src, out_dtype=torch.float32)
            outb = kvt_prefill_attn(dc, 0, q.to(dev), cu, k_src=k_src, v_src=v_src)
            exp = _oracle_chunk(q, 0, xk, xv)
        else:
            out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32)
            outb = kvt_prefill_attn(dc, 0, q.to(dev), cu)
            kk, vv = oc.rows(0)
            exp = _oracle_chunk(q, a, kk, vv)
        out = out.cpu()
        err = (out - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (a, float(err.max()), float(err.mean()))
        assert torch.equal(outb.cpu(), out.to(torch.bfloat16)), ("bf16 output != rounded fp32 output", a)


@pytest.mark.parametrize("ring", [16, 32])
def test_prefill_short_ring(kvt_pkg, ring):
    """Rings of 16 and 32 rows: a 32-key tile can hold more keys than the ring (every tile fetched per key) or exactly
    the ring; chunks of 70 / 45 / 61 queries, so most positions sit in INT4 pages and hot_start falls inside a tile."""
    from kvtier.kvt import kvt_prefill_attn
    for a, n, xk, xv, dc, oc, gen in _chunked([70, 45, 61], ring, seed=17):
        q = ref.make_q(HQ, D, gen, n=n)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        src = dict(k_src=xk.to(dev), v_src=xv.to(dev)) if a == 0 else {}
        out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32, **src).cpu()
        kk, vv = (xk, xv) if a == 0 else oc.rows(0)
        exp = _oracle_chunk(q, a, kk, vv)
        err = (out - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (ring, a, float(err.max()), float(err.mean()))


@pytest.mark.parametrize("hq", [20, 24, 32])
def test_prefill_wide_groups(kvt_pkg, hq):
    """Groups of more than 8 q heads per KV head (10, 12 -- the served model's 24 / 2 -- and 16): 16 / gs queries per
    wavefront; chunk 0 from bf16, chunks 1-2 from the tiers (ragged last query tiles), fp32 and bf16 outputs."""
    from kvtier.kvt import kvt_prefill_attn
    for a, n, xk, xv, dc, oc, gen in _chunked([96, 90, 37], 128, seed=14):
        q = ref.make_q(hq, D, gen, n=n)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        src = dict(k_src=xk.to(dev), v_src=xv.to(dev)) if a == 0 else {}
        out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32, **src).cpu()
        outb = kvt_prefill_attn(dc, 0, q.to(dev), cu, **src).cpu()
        kk, vv = (xk, xv) if a == 0 else oc.rows(0)
        exp = _oracle_chunk(q, a, kk, vv)
        err = (out - exp).abs()
        assert out.shape == (n, hq, D)
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (hq, a, float(err.max()), float(err.mean()))
        assert torch.equal(outb, out.to(torch.bfloat16)), (hq, a)


def test_prefill_first_query_closed_form(kvt_pkg):
    """Query 0 of a chunk without a prefix sees only key 0: the output is that V row (P = 1), for every q head of
    each KV head: exactly where |v| >= 2^-10 (v / 128 keeps its 8 significant bits in fp16), to 2^-18 below (fp16
    subnormals, spacing 2^-24 before the factor 128)."""
    from kvtier.kvt import kvt_prefill_attn
    for a, n, xk, xv, dc, oc, gen in _chunked([40], 64, seed=12):
        q = ref.make_q(HQ, D, gen, n=n)
        cu = torch.tensor([0, n], dtype=torch.int64, device=dev)
        out = kvt_prefill_attn(dc, 0, q.to(dev), cu, k_src=xk.to(dev), v_src=xv.to(dev),
                               out_dtype=torch.float32).cpu()
        for hq in range(HQ):
            v = xv[0, hq // 8].float()
            big = v.abs() >= 2.0 ** -10
            assert torch.equal(out[0, hq][big], v[big]), hq
            assert float((out[0, hq] - v).abs().max()) <= 2.0 ** -18, hq


def test_prefill_tail_of_small_weights(kvt_pkg):
    """One key outweighs 2,047 others by e^11.75 (their P = 2^-16.95, below fp16's normal range): the tail still
    counts.  Q = e_0, key 0 has channel 0 = 188, the others 0; V row 0 = 0, the others 1, so query j's output is
    j w / (1 + j w), w = exp(-188 / 16), in every channel (about 0.016 at the last query, which flushing the
    subnormal weights would lose)."""
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    n = 2048
    dc = PosTieredCache(1, H, D, n_pages=64, ring_total=n, max_seqs=1, max_pages=64, device=dev)
    dc.add_seq(n)
    plan = dc.plan_append([0], [n])
    q = torch.zeros(n, HQ, D)
    q[:, :, 0] = 1.0
    xk = torch.zeros(n, H, D)
    xk[0, :, 0] = 188.0
    xv = torch.ones(n, H, D)
    xv[0] = 0.0
    q, xk, xv = q.to(torch.bfloat16), xk.to(torch.bfloat16), xv.to(torch.bfloat16)
    dc.append(0, plan, xk.to(dev), xv.to(dev))
    dc.commit(plan)
    oc = ref.PosTieredCache(H, D, n_pages=64, ring_total=n)
    oc.add_seq(0, n)
    oc.plan_pages(0, n, ref.PageAllocator(64, seed=0))
    oc.append(0, xk, xv)
    cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
    w = torch.exp(torch.tensor(-188.0 / 16, dtype=torch.float64))
    j = torch.arange(n, dtype=torch.float64)
    closed = (j * w / (1 + j * w)).float()
    sample = list(range(0, n, 97)) + [n - 1]
    for src in (True, False):
        kw = dict(k_src=xk.to(dev), v_src=xv.to(dev)) if src else {}
        out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32, **kw).cpu()
        kk, vv = (xk, xv) if src else oc.rows(0)   # the tiers' rows: bf16(code * scale) of the INT8 ring
        err = (out - closed[:, None, None]).abs()
        assert float(closed[-1]) > 0.015
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (src, float(err.max()))
        exp = torch.stack([ref.attention_rows(q[i], kk[:i + 1], vv[:i + 1], SCALE) for i in sample])
        e2 = (out[sample] - exp).abs()
        assert float(e2.max()) < 2e-3 and float(e2.mean()) < 1e-3, (src, float(e2.max()))


@pytest.mark.parametrize("spread", [None, 0, 5])
def test_prefill_two_sequences_cache(kvt_pkg, spread):
    """Two sequences with their own rings and interleaved pages, chunks of 50 and 33 queries (int64 cu_q); spread
    launches by the default rule (one block per CU), none, and 5 blocks (shares that cross from one sequence to the
    other; the shorter sequence's last query tile has no queries and no key tiles)."""
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    gen = torch.Generator().manual_seed(13)
    och = ref.outlier_channels(H, D, 8, gen)
    rings = [64, 128]
    dc = PosTieredCache(1, H, D, n_pages=32, ring_total=sum(rings), max_seqs=2, max_pages=16, device=dev,
                        page_seed=3)
    oc = ref.PosTieredCache(H, D, n_pages=32, ring_total=sum(rings))
    alloc = ref.PageAllocator(32, seed=3)
    base = 0
    for r in rings:
        dc.add_seq(r)
        oc.add_seq(base, r)
        base += r
    # history: 300 and 190 positions, then the chunk (50, 33) appended
    for total in ([60, 60], [60, 60], [60, 60], [60, 10], [60, 0], [50, 33]):
        seqs = [s for s in range(2) if total[s] > 0]
        cnt = [total[s] for s in seqs]
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
    nq = [50, 33]
    q = ref.make_q(HQ, D, gen, n=sum(nq))
    cu = torch.tensor([0, 50, 83], dtype=torch.int64, device=dev)
    out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32, spread=spread).cpu()
    for s, (q0, q1) in enumerate(((0, 50), (50, 83))):
        kk, vv = oc.rows(s)
        L = kk.shape[0]
        exp = _oracle_chunk(q[q0:q1], L - (q1 - q0), kk, vv)
        err = (out[q0:q1] - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (s, float(err.max()), float(err.mean()))


@pytest.mark.parametrize("spread", [0, 7, 256, 1000])
def test_prefill_spread(kvt_pkg, spread):
    """Spread launches (blocks sharing the key tiles equally, query tiles split where a share ends and merged in the
    kernel by the block that finishes last): chunks of 400 and 600 queries over ring 256, so the second chunk's
    query tiles read up to 32 key tiles across INT4 pages and the ring (hot_start 744, inside a tile), and the
    first chunk's come from the bf16 source.  7 blocks: every block walks many query tiles; 1,000: fewer blocks are
    used (shares of at least 16 units: key tiles plus 8 per query tile), query tiles split into several pieces.  Every case matches the oracle; a
    repeated call and a call with a fresh workspace give the same bits (the merge is a fixed sum over the pieces,
    whichever block merges); the counters are back at zero after each call."""
    from kvtier.kvt import kvt_prefill_attn
    import ctypes
    from kvtier import _lib
    for a, n, xk, xv, dc, oc, gen in _chunked([400, 600], 256, seed=31):
        q = ref.make_q(HQ, D, gen, n=n).to(dev)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        src = dict(k_src=xk.to(dev), v_src=xv.to(dev)) if a == 0 else {}
        kk, vv = (xk, xv) if a == 0 else oc.rows(0)
        exp = _oracle_chunk(q.cpu(), a, kk, vv)
        need = ctypes.c_int64(0)
        _lib.call("kvt_prefill_work_bytes", 1, H, HQ, n, spread, ctypes.byref(need))
        work = torch.zeros(max(need.value, 1), dtype=torch.uint8, device=dev)
        out = kvt_prefill_attn(dc, 0, q, cu, out_dtype=torch.float32, spread=spread, work=work, **src)
        err = (out.cpu() - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (a, spread, float(err.max()), float(err.mean()))
        n_ctr = H * -(-n // 16)
        for _ in range(2):
            again = kvt_prefill_attn(dc, 0, q, cu, out_dtype=torch.float32, spread=spread, work=work, **src)
            assert torch.equal(again, out), (a, spread)
            assert int(work[:4 * n_ctr].count_nonzero()) == 0, (a, spread)
        fresh = torch.zeros(max(need.value, 1), dtype=torch.uint8, device=dev)
        assert torch.equal(kvt_prefill_attn(dc, 0, q, cu, out_dtype=torch.float32, spread=spread, work=fresh, **src),
                           out), (a, spread)
        outb = kvt_prefill_attn(dc, 0, q, cu, spread=spread, work=work, **src)
        assert torch.equal(outb, out.to(torch.bfloat16)), (a, spread)


@pytest.mark.parametrize("spread", [None, 3, 64])
def test_prefill_spread_three_sequences(kvt_pkg, spread):
    """Three sequences (rings 64 / 128 / 256, histories of 700 / 1,500 / 300 positions, mostly in INT4 pages) with
    chunks of 300 / 40 / 520 queries in one launch: spread shares cross from one sequence (and KV head) to the next,
    the short chunk's later query tiles are empty, and 3 blocks each walk many query tiles; every query against the
    oracle."""
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    gen = torch.Generator().manual_seed(41)
    och = ref.outlier_channels(H, D, 8, gen)
    rings, hist, nq = [64, 128, 256], [700, 1500, 300], [300, 40, 520]
    n_pages = 64
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=sum(rings), max_seqs=3, max_pages=48, device=dev,
                        page_seed=5)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=sum(rings))
    alloc = ref.PageAllocator(n_pages, seed=5)
    base = 0
    for r in rings:
        dc.add_seq(r)
        oc.add_seq(base, r)
        base += r
    left = [h + n for h, n in zip(hist, nq)]
    while any(left):   # appends of at most 64 positions per sequence and step (never more than a ring)
        seqs = [s for s in range(3) if left[s] > 0]
        cnt = [min(64, left[s]) for s in seqs]
        plan = dc.plan_append(seqs, cnt)
        ks, vs = [], []
        for s_, m in zip(seqs, cnt):
            xk, xv = ref.make_kv(m, H, D, gen, och)
            oc.plan_pages(s_, m, alloc)
            oc.append(s_, xk, xv)
            ks.append(xk)
            vs.append(xv)
            left[s_] -= m
        dc.append(0, plan, torch.cat(ks).to(dev), torch.cat(vs).to(dev))
        dc.commit(plan)
    q = ref.make_q(HQ, D, gen, n=sum(nq))
    cu = torch.tensor([0, nq[0], nq[0] + nq[1], sum(nq)], dtype=torch.int32, device=dev)
    out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32, spread=spread).cpu()
    q0 = 0
    for s_ in range(3):
        kk, vv = oc.rows(s_)
        L = kk.shape[0]
        assert L == hist[s_] + nq[s_]
        exp = _oracle_chunk(q[q0:q0 + nq[s_]], L - nq[s_], kk, vv)
        err = (out[q0:q0 + nq[s_]] - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3, (s_, spread, float(err.max()), float(err.mean()))
        q0 += nq[s_]


BIG_POS = (5, 40, 150, 250, 300)


def _big_row(bf16_max):
    """The reference's clamp-regime row (gemv/test_kv_tiers.py:412-415): KV head 0 channels 0-31 = +-1e6 / 5e5 / 4.6e5
    / 1e5, KV head 1 channels 64-95 = bf16 max (1e6 where the row is attended from the bf16 source chunk: there the
    V rows are the raw bf16 values, not dequantized ones bounded by 127 * 65504)."""
    big = torch.zeros(H, D)
    big[0, :32] = torch.tensor([1e6, -1e6, 5e5, -5e5, 4.6e5, -4.6e5, 1e5, -1e5] * 4)
    big[1, 64:96] = torch.finfo(torch.bfloat16).max if bf16_max else 1e6
    return big.to(torch.bfloat16)


def _place_big(a, xk, xv):
    for p in BIG_POS:
        if a <= p < a + xk.shape[0]:
            big = _big_row(bf16_max=a > 0)
            xk[p - a] = big
            xv[p - a] = -big


def _clamp_case(zero_big_channels):
    """Chunks 96 / 96 / 96 / 80 over ring 128 with the clamp rows at BIG_POS: positions 5 / 40 / 150 end in INT4 pages
    (INT8 scale 65504, requantized to INT4 scale 65504), 250 / 300 stay INT8 ring rows; chunk 0 attends them from
    the bf16 source.  Yields (out fp32, expected, bound) per chunk, bound = 2^-10 sum_i p_i |v_i| per output."""
    from kvtier.kvt import kvt_prefill_attn
    for a, n, xk, xv, dc, oc, gen in _chunked([96, 96, 96, 80], 128, seed=21, edit=_place_big):
        q = ref.make_q(HQ, D, gen, n=n)
        if zero_big_channels:
            q[:, :8, :32] = 0
            q[:, 8:, 64:96] = 0
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        if a == 0:
            out = kvt_prefill_attn(dc, 0, q.to(dev), cu, k_src=xk.to(dev), v_src=xv.to(dev), out_dtype=torch.float32)
            kk, vv = xk, xv
        else:
            out = kvt_prefill_attn(dc, 0, q.to(dev), cu, out_dtype=torch.float32)
            kk, vv = oc.rows(0)
        yield a, q, out.cpu(), _oracle_chunk(q, a, kk, vv), 2.0 ** -10 * _oracle_chunk(q, a, kk, vv.abs()), kk


def test_prefill_clamp_regime_tiers(kvt_pkg):
    """Clamp rows in every tier, queries zero on the saturated channels: the scores stay ordinary while K rows reach
    127 * 65504 (beyond fp16) and V rows carry the saturated values into every output; all outputs finite and within
    2e-3 + 2^-10 sum p|v| of the oracle."""
    for a, q, out, exp, bound, kk in _clamp_case(zero_big_channels=True):
        assert torch.isfinite(out).all(), a
        assert float(exp.abs().max()) > 1e4, a                   # the saturated V rows reach the outputs
        assert bool(((out - exp).abs() <= 2e-3 + bound).all()), (a, float(((out - exp).abs() - bound).max()))


def test_prefill_clamp_regime_scores(kvt_pkg):
    """Clamp rows with random queries: scores of order 1e4 on the saturated keys.  Every output is finite; rows whose
    softmax is one-hot (max weight > 1 - 1e-6) or ignores the clamp keys (their weight < 1e-12) match the oracle to
    2e-3 + 2^-10 sum p|v| (elsewhere the outputs are ill-conditioned: fp32 rounding of 1e4-sized scores moves the
    weights)."""
    checked = 0
    for a, q, out, exp, bound, kk in _clamp_case(zero_big_channels=False):
        assert torch.isfinite(out).all(), a
        n = q.shape[0]
        for h in range(H):
            s = torch.einsum("jgd,kd->jgk", q[:, 8 * h:8 * h + 8].float(), kk[:, h].float()) * SCALE
            keys = torch.arange(kk.shape[0])
            s = s.masked_fill(keys[None, None, :] > (a + torch.arange(n))[:, None, None], float("-inf"))
            w = torch.softmax(s, dim=-1)
            big = torch.tensor([p for p in BIG_POS if p < kk.shape[0]])
            ok = (w.max(-1).values > 1 - 1e-6) | (w[..., big].sum(-1) < 1e-12)
            err = (out[:, 8 * h:8 * h + 8] - exp[:, 8 * h:8 * h + 8]).abs() - bound[:, 8 * h:8 * h + 8]
            assert bool((err[ok] <= 2e-3).all()), (a, h, float(err[ok].max()))
            checked += int(ok.sum())
    assert checked > 2000


def test_prefill_paged_range_beyond_staged_pages(kvt_pkg):
    """A sequence whose paged key range needs more than the 8,192 page ids a block stages in LDS (524,288 paged
    positions): the wrapper refuses it from its host lengths (ValueError), and the kernel, called through the C ABI
    without that check, returns NaN for every query of the chunk instead of reading keys from clamped pages."""
    import math
    from kvtier import _lib
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    ring, n_pages = 8192, 8200
    L = 8192 * 64 + ring + 128                          # hot_start = 524,416: 8,194 pages below the ring
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=ring, max_seqs=1, max_pages=n_pages, device=dev,
                        page_seed=3)
    dc.add_seq(ring)
    g = torch.Generator(device=dev).manual_seed(3)
    k = torch.randn(ring, H, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(ring, H, D, device=dev, generator=g).to(torch.bfloat16)
    done = 0
    while done < L:
        n = min(ring, L - done)
        plan = dc.plan_append([0], [n])
        dc.append(0, plan, k[:n], v[:n])
        dc.commit(plan)
        done += n
    assert dc.hot_start(0) > 8192 * 64
    nq = 16
    q = (torch.randn(nq, HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    cu = torch.tensor([0, nq], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        kvt_prefill_attn(dc, 0, q, cu, max_q=nq)
    out = torch.zeros(nq, HQ, D, dtype=torch.float32, device=dev)
    _lib.call("kvt_prefill_attn", q.data_ptr(), q.stride(0), q.stride(1), cu.data_ptr(), 0, dc.seq_lens.data_ptr(),
              1, nq, H, HQ, D, dc.group8, dc.k4[0].data_ptr(), dc.v4[0].data_ptr(), dc.ks4[0].data_ptr(),
              dc.vs4[0].data_ptr(), dc.rk[0].data_ptr(), dc.rv[0].data_ptr(), dc.rks[0].data_ptr(),
              dc.rvs[0].data_ptr(), dc.ring_base.data_ptr(), dc.ring_len.data_ptr(), dc.ring_start.data_ptr(),
              dc.page_table.data_ptr(), dc.page_table.stride(0), dc.k4[0].shape[0], None, None, 0, 0, 0, 0, 0,
              1.0 / math.sqrt(D), out.data_ptr(), 1, out.stride(0), out.stride(1), 0, None, 0, _lib.stream())
    torch.cuda.synchronize()
    assert torch.isnan(out).all()


def test_prefill_spread_workspace_reuse(kvt_pkg):
    """One spread workspace used by a launch of few query tiles, then by one of many: the second result equals the
    same launch on a fresh zeroed workspace, bit for bit, and the oracle.  (With a counter area sized per call, the
    first launch's slot data sat where the second launch's counters are, and the second merged pieces early.)"""
    import ctypes
    from kvtier import _lib
    from kvtier.kvt import kvt_prefill_attn

    def work_bytes(max_q):
        b = ctypes.c_int64(0)
        _lib.call("kvt_prefill_work_bytes", 1, H, HQ, max_q, 256, ctypes.byref(b))
        return b.value

    for a, n, xk, xv, dc, oc, gen in _chunked([1024, 1024], 512, seed=61):
        if a == 0:
            continue
        q = ref.make_q(HQ, D, gen, n=n)
        kk, vv = oc.rows(0)
        L = kk.shape[0]
        small = torch.tensor([0, 96], dtype=torch.int32, device=dev)
        full = torch.tensor([0, n], dtype=torch.int32, device=dev)
        kv_small = torch.tensor([L - n + 96], dtype=torch.int32, device=dev)   # the chunk's first 96 queries
        need = max(work_bytes(n), work_bytes(96))
        shared = torch.zeros(need, dtype=torch.uint8, device=dev)
        q_dev = q.to(dev)
        kvt_prefill_attn(dc, 0, q_dev[:96], small, kv_lens=kv_small, max_q=96, out_dtype=torch.float32, spread=256,
                         work=shared)
        got = kvt_prefill_attn(dc, 0, q_dev, full, max_q=n, out_dtype=torch.float32, spread=256, work=shared)
        fresh = kvt_prefill_attn(dc, 0, q_dev, full, max_q=n, out_dtype=torch.float32, spread=256,
                                 work=torch.zeros(need, dtype=torch.uint8, device=dev))
        torch.cuda.synchronize()
        assert torch.equal(got, fresh)
        exp = _oracle_chunk(q[-64:], L - 64, kk, vv)
        err = (got[-64:].cpu() - exp).abs()
        assert float(err.max()) < 2e-3 and float(err.mean()) < 1e-3
