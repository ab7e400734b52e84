"""GPU parity of the write path (bit-exact codes, scales, owner table, page tables) against the CPU oracle.

Scenarios follow the reference's unit tests: gemv/test_kv_tiers.py sections 1, 2, 2b, 5 and 6;
gemv/test_kv_int4.py sections 1-2; gemv/test_kv_int8.py quant + scatter.  Inputs come from seeded CPU generators
and are copied to the device, so the oracle and the kernels see identical bits.
"""
import numpy as np
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D = 2, 256


def _bufs(slots, R, g8=64):
    return [t.to(dev) for t in (
        torch.full((slots, H, D // 2), 0x77, dtype=torch.uint8), torch.full((slots, H, D // 2), 0x99, dtype=torch.uint8),
        torch.full((slots, H, D // 32), 3.0, dtype=torch.float16), torch.full((slots, H, D // 32), 5.0, dtype=torch.float16),
        torch.full((R, H, D), 0x33, dtype=torch.int8), torch.full((R, H, D), 0x44, dtype=torch.int8),
        torch.full((R, H, D // g8), 7.0, dtype=torch.float16), torch.full((R, H, D // g8), 9.0, dtype=torch.float16),
        torch.full((R,), -1, dtype=torch.int32))]


def _cpu(bufs):
    return [t.cpu() for t in bufs]


def test_quant_store_int4_int8_golden(kvt_pkg):
    """The golden vectors (scalar model) through the INT4 and INT8 writers, every input dtype path."""
    from kvtier import sparse_attn as sa
    g = np.load("tests/golden/quant_vectors.npz")
    x = torch.from_numpy(g["x_bf16_bits"].astype(np.int16)).view(torch.bfloat16)
    n = x.shape[0] // 2
    k = x[:n].reshape(n, 1, D).expand(n, H, D).contiguous()
    v = x[n:2 * n].reshape(n, 1, D).expand(n, H, D).contiguous()
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    loc = torch.arange(n, dtype=torch.int32, device=dev) * 3 + 1
    for dt in (torch.bfloat16, torch.float32):
        k4 = torch.zeros(3 * n + 2, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
        ks = torch.zeros(3 * n + 2, H, 8, dtype=torch.float16, device=dev); vs = torch.zeros_like(ks)
        sa.quant_store_kv_int4(k.to(dev, dt), v.to(dev, dt), loc, k4, v4, ks, vs, ones, ones)
        k8 = torch.zeros(3 * n + 2, H, D, dtype=torch.int8, device=dev); v8 = torch.zeros_like(k8)
        ks8 = torch.zeros(3 * n + 2, H, 4, dtype=torch.float16, device=dev); vs8 = torch.zeros_like(ks8)
        sa.quant_store_kv_int8(k.to(dev, dt), v.to(dev, dt), loc, k8, v8, ks8, vs8, ones, ones)
        torch.cuda.synchronize()
        ll = loc.long().cpu()
        for h in range(H):
            assert np.array_equal(k4.cpu()[ll, h].numpy(), g["p4"][:n]) and np.array_equal(ks.cpu()[ll, h].numpy(), g["s4"][:n])
            assert np.array_equal(v4.cpu()[ll, h].numpy(), g["p4"][n:2 * n])
            assert np.array_equal(k8.cpu()[ll, h].numpy(), g["q8_g64"][:n]) and np.array_equal(ks8.cpu()[ll, h].numpy(), g["s8_g64"][:n])
            assert np.array_equal(vs8.cpu()[ll, h].numpy(), g["s8_g64"][n:2 * n])


def test_quant_store_int4_random_slots(kvt_pkg):
    """int32 and int64 loc, zero row / zero group / -7..7 row, other slots untouched (gemv/test_kv_int4.py:83-115),
    random smoothing factors, strided (non-contiguous) input rows."""
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(0)
    N, slots = 1000, 4096
    xk = (torch.randn(N, H, D, generator=gen) * 3).to(torch.bfloat16)
    xv = (torch.randn(N, H, D, generator=gen) * 3).to(torch.bfloat16)
    xk[5] = 0
    xv[7, 1, 64:96] = 0
    full = torch.tensor([-7, 7, -6, 6, -5, 5, -4, 4, -3, 3, -2, 2, -1, 1, 0, 7] * 16, dtype=torch.bfloat16)
    xk[3, 0] = full
    smi = (0.5 + 1.5 * torch.rand(H, D, generator=gen)).half()
    wide = torch.zeros(N, H * D + 64, dtype=torch.bfloat16)
    wide[:, :H * D] = xk.reshape(N, H * D)
    xk_strided = wide[:, :H * D].view(N, H, D)                  # row stride H * D + 64
    for loc_dtype in (torch.int32, torch.int64):
        loc = torch.randperm(slots, generator=gen)[:N].to(loc_dtype)
        b = _bufs(slots, 64)
        sa.quant_store_kv_int4(xk_strided.to(dev), xv.to(dev), loc.to(dev), b[0], b[1], b[2], b[3], smi.to(dev), smi.to(dev))
        torch.cuda.synchronize()
        c = _cpu(b)
        e = _cpu(_bufs(slots, 64))
        ref.quant_store_int4(xk, xv, loc, e[0], e[1], e[2], e[3], smi, smi)
        for i in range(4):
            assert torch.equal(c[i], e[i]), (loc_dtype, i)


@pytest.mark.parametrize("g8", [64, 256])
def test_tiered_dual_write_ring_wrap(kvt_pkg, g8):
    """N = 1000 tokens into ascending slots in alias-free chunks, R = 64 over 4096 slots: every INT4 row, the owner
    table and every hot ring row bit-exact; cold slots' ring rows hold their owner's data (gemv/test_kv_tiers.py:117-164)."""
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(1)
    N, slots, R = 1000, 4096, 64
    xk = (torch.randn(N, H, D, generator=gen) * 3).to(torch.bfloat16)
    xv = (torch.randn(N, H, D, generator=gen) * 3).to(torch.bfloat16)
    xk[5] = 0
    sl = torch.randperm(slots, generator=gen)[:N].sort().values
    sl[0] = 0
    ones = torch.ones(H, D, dtype=torch.float16)
    chunks, a = [], 0
    while a < N:
        e = a + 1
        while e < N and int(sl[e]) - int(sl[a]) < R:
            e += 1
        chunks.append((a, e))
        a = e
    for loc_dtype in (torch.int32, torch.int64):
        b = _bufs(slots, R, g8)
        e = _cpu(_bufs(slots, R, g8))
        for a, z in chunks:
            sa.quant_store_kv_tiered(xk[a:z].to(dev), xv[a:z].to(dev), sl[a:z].to(loc_dtype).to(dev), *b, ones.to(dev),
                                     ones.to(dev), R - 1)
            ref.quant_store_tiered(xk[a:z], xv[a:z], sl[a:z], *e, ones, ones, R - 1, group8=g8)
        torch.cuda.synchronize()
        c = _cpu(b)
        for i in range(9):
            assert torch.equal(c[i], e[i]), (loc_dtype, i)
        assert int(c[8][0]) >= 0


def test_tiered_boundary_and_collisions(kvt_pkg):
    """s then s + R flips the owner; s + R then s keeps s; same-launch collisions: one winner per contested ring
    row among its writers, its ring row bit-exact, losers cold, every INT4 row exact (gemv/test_kv_tiers.py:166-235)."""
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(2)
    R, slots = 64, 4096
    x = (torch.randn(R, H, D, generator=gen) * 3).to(torch.bfloat16)
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    one = lambda i: torch.tensor([i], dtype=torch.int32, device=dev)
    b = _bufs(slots, R)
    sa.quant_store_kv_tiered(x[:1].to(dev), x[:1].to(dev), one(100), *b, ones, ones, R - 1)
    sa.quant_store_kv_tiered(x[1:2].to(dev), x[1:2].to(dev), one(100 + R), *b, ones, ones, R - 1)
    torch.cuda.synchronize()
    q8, s8 = ref.quant8(x)
    p4, s4 = ref.quant4(x)
    assert int(b[8][100 & (R - 1)]) == 100 + R
    assert torch.equal(b[4][100 & (R - 1)].cpu(), q8[1]) and torch.equal(b[0][100].cpu(), p4[0])
    assert int((b[8] == -1).sum()) == R - 1
    b = _bufs(slots, R)
    sa.quant_store_kv_tiered(x[1:2].to(dev), x[1:2].to(dev), one(100 + R), *b, ones, ones, R - 1)
    sa.quant_store_kv_tiered(x[:1].to(dev), x[:1].to(dev), one(100), *b, ones, ones, R - 1)
    torch.cuda.synchronize()
    assert int(b[8][100 & (R - 1)]) == 100 and torch.equal(b[4][100 & (R - 1)].cpu(), q8[0])
    contested = 0
    for trial in range(20):
        b = _bufs(slots, R)
        classes = torch.randint(0, 8, (R,), generator=gen)
        members = torch.randperm(slots // R, generator=gen)[:R]
        loc = (members * R + classes).to(torch.int32)
        perm = torch.randperm(R, generator=gen)
        sa.quant_store_kv_tiered(x[perm].to(dev), x[perm].to(dev), loc.to(dev), *b, ones, ones, R - 1)
        torch.cuda.synchronize()
        c = _cpu(b)
        ll = loc.long()
        assert torch.equal(c[0][ll], p4[perm]) and torch.equal(c[2][ll], s4[perm])
        for r_ in range(R):
            cand = ll[(ll & (R - 1)) == r_]
            if cand.numel() == 0:
                assert int(c[8][r_]) == -1 and (c[4][r_] == 0x33).all() and (c[6][r_] == 7.0).all()
                continue
            w = int(c[8][r_])
            assert w in set(cand.tolist())
            i_w = int(perm[int(torch.nonzero(loc == w).item())])
            assert torch.equal(c[4][r_], q8[i_w]) and torch.equal(c[6][r_], s8[i_w])
            assert torch.equal(c[5][r_], q8[i_w])
            contested += int(cand.numel() > 1)
    assert contested > 100


def test_fp16_max_clamp_writers(kvt_pkg):
    """1e6 / bf16-max groups: ring and INT4 scales 65504, codes bit-exact vs the clamped references
    (gemv/test_kv_tiers.py:412-436)."""
    from kvtier import sparse_attn as sa
    big = torch.zeros(1, H, D, dtype=torch.bfloat16)
    big[0, 0, :32] = torch.tensor([1e6, -1e6, 5e5, -5e5, 4.6e5, -4.6e5, 1e5, -1e5] * 4).to(torch.bfloat16)
    big[0, 1, 64:96] = torch.finfo(torch.bfloat16).max
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    b = _bufs(256, 64)
    sa.quant_store_kv_tiered(big.to(dev), (-big).to(dev), torch.tensor([17], device=dev), *b, ones, ones, 63)
    torch.cuda.synchronize()
    q8, s8 = ref.quant8(big)
    p4, s4 = ref.quant4(big)
    assert torch.equal(b[4][17].cpu(), q8[0]) and torch.equal(b[6][17].cpu(), s8[0]) and float(b[6][17, 1, 1]) == 65504.0
    assert torch.equal(b[0][17].cpu(), p4[0]) and torch.equal(b[2][17].cpu(), s4[0])
    q8v, s8v = ref.quant8(-big)
    assert torch.equal(b[5][17].cpu(), q8v[0]) and torch.isfinite(b[7]).all()


def test_pool_set_kv_buffer(kvt_pkg, monkeypatch):
    """MHATokenToKVPoolTiered.set_kv_buffer: [N, H, D] and [N, H * D] forms, both tiers + owner bit-exact
    (gemv/test_kv_tiers.py:458-559)."""
    from kvtier.tiered_kv_pool import MHATokenToKVPoolTiered
    monkeypatch.setenv("SGLANG_KV_TIERS_W", "64")
    R = 64
    pool = MHATokenToKVPoolTiered(size=1024, page_size=64, dtype=torch.uint8, head_num=H, head_dim=D, layer_num=2,
                                  device=dev)
    gen = torch.Generator().manual_seed(3)
    loc = (torch.randperm(400, generator=gen)[:50] + 64).sort().values
    seen, keep = set(), []
    for s in loc.tolist():
        if (s & (R - 1)) not in seen:
            seen.add(s & (R - 1)); keep.append(s)
    loc = torch.tensor(keep, dtype=torch.int64)
    n = loc.numel()
    xk = (torch.randn(n, H, D, generator=gen) * 3).to(torch.bfloat16)
    xv = (torch.randn(n, H, D, generator=gen) * 3).to(torch.bfloat16)
    pool.set_kv_buffer(None, loc.to(dev), xk.to(dev), xv.to(dev), 1.0, 1.0, layer_id_override=1)
    pool.set_kv_buffer(None, loc.to(dev), xk.reshape(n, -1).to(dev), xv.reshape(n, -1).to(dev), layer_id_override=0)
    torch.cuda.synchronize()
    pk, sk = ref.quant4(xk)
    q8, s8 = ref.quant8(xk)
    for l in (0, 1):
        assert torch.equal(pool.k_buffer[l][loc].cpu(), pk) and torch.equal(pool.get_kv_scale_buffer(l)[0][loc].cpu(), sk)
        rk, rv, rks, rvs = pool.get_kv_ring_buffer(l)
        assert torch.equal(rk[loc & (R - 1)].cpu(), q8) and torch.equal(rks[loc & (R - 1)].cpu(), s8)
    assert torch.equal(pool.ring_owner.long()[loc.to(dev) & (R - 1)].cpu(), loc)
    assert int((pool.ring_owner == -1).sum()) == R - n


def test_append_evict_matches_oracle(kvt_pkg):
    """Evict mode, two sequences with rings of 128 and 64 rows, 900 / 500 tokens appended in mixed chunk sizes
    (single tokens and chunks up to the ring size): INT4 pool, ring rows and page tables bit-exact vs the oracle;
    pages come from the seeded allocator."""
    from kvtier.kvt import PosTieredCache
    gen = torch.Generator().manual_seed(4)
    n_pages = 40
    dc = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=192, max_seqs=2, max_pages=32, device=dev, page_seed=11)
    oc = ref.PosTieredCache(H, D, n_pages=n_pages, ring_total=192)
    alloc = ref.PageAllocator(n_pages, seed=11)
    s0 = dc.add_seq(128)
    s1 = dc.add_seq(64)
    oc.add_seq(0, 128)
    oc.add_seq(128, 64)
    lens = [900, 500]
    done = [0, 0]
    sched = [(1, 1), (37, 5), (128, 64), (1, 1), (100, 64), (128, 0), (1, 1)]
    while done[0] < lens[0] or done[1] < lens[1]:
        for c0, c1 in sched:
            cnt = [min(c0, lens[0] - done[0]), min(c1, lens[1] - done[1])]
            seqs = [s for s in (0, 1) if cnt[s] > 0]
            if not seqs:
                continue
            plan = dc.plan_append(seqs, [cnt[s] for s in seqs])
            ks, vs = [], []
            for s in seqs:
                xk = (torch.randn(cnt[s], H, D, generator=gen) * 2).to(torch.bfloat16)
                xv = torch.randn(cnt[s], H, D, generator=gen).to(torch.bfloat16)
                oc.plan_pages(s, cnt[s], alloc)
                oc.append(s, xk, xv)
                ks.append(xk); vs.append(xv)
            dc.append(0, plan, torch.cat(ks).to(dev), torch.cat(vs).to(dev))
            dc.commit(plan)
            for s in seqs:
                done[s] += cnt[s]
    torch.cuda.synchronize()
    assert torch.equal(dc.page_table.cpu(), oc.page_table(32))
    for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
        assert torch.equal(getattr(dc, name)[0].cpu(), getattr(oc, name)), name
    assert dc.seq_lens[:2].tolist() == lens


def _boundary_rows(n, group, qmax, seed):
    """fp32 rows [n, H, D] whose quotients x / s sit on, or one ulp either side of, half-integers: element 0 of each
    group is +-qmax * s0 (so the stored scale is exactly the fp16 value s0) and the others are +-(k + 0.5) * s0,
    k in [0, qmax), nudged by -1, 0 or +1 ulp.  All products are exact in fp32."""
    rng = np.random.default_rng(seed)
    g = n * H * D // group
    s0 = rng.uniform(2.0 ** -8, 8.0, g).astype(np.float16).astype(np.float32)
    s0[::7] = 2.0 ** rng.integers(-6, 4, s0[::7].size)                       # exact reciprocals too
    k = rng.integers(0, int(qmax), (g, group)).astype(np.float32) + np.float32(0.5)
    base = k * s0[:, None]
    nudge = rng.integers(-1, 2, (g, group))
    vals = np.where(nudge < 0, np.nextafter(base, np.float32(-np.inf)),
                    np.where(nudge > 0, np.nextafter(base, np.float32(np.inf)), base)).astype(np.float32)
    vals[:, 0] = np.float32(qmax) * s0
    vals *= rng.choice(np.array([-1.0, 1.0], np.float32), (g, group))
    return torch.from_numpy(vals.reshape(n, H, D))


@pytest.mark.parametrize("aligned", [True, False])
def test_quant_rounding_boundaries(kvt_pkg, aligned):
    """Quotients on and one ulp around x.5 (ties to even, and the cases where a reciprocal multiply would round the
    other way): INT8-G64 and INT4-G32 writers bit-exact vs the oracle's IEEE division, through the vector-load path
    (aligned rows) and the element path (row stride H * D + 1)."""
    from kvtier import sparse_attn as sa
    n = 512
    ones = torch.ones(H, D, dtype=torch.float16)
    for group, qmax in ((64, 127.0), (32, 7.0)):
        x = _boundary_rows(n, group, qmax, seed=int(qmax))
        if aligned:
            xd = x.to(dev)
        else:
            wide = torch.zeros(n, H * D + 1, dtype=torch.float32)
            wide[:, :H * D] = x.reshape(n, H * D)
            xd = wide.to(dev)[:, :H * D].view(n, H, D)
        loc = torch.arange(n, dtype=torch.int64)
        if group == 64:
            k8 = torch.zeros(n, H, D, dtype=torch.int8, device=dev); v8 = torch.zeros_like(k8)
            ks = torch.zeros(n, H, 4, dtype=torch.float16, device=dev); vs = torch.zeros_like(ks)
            sa.quant_store_kv_int8(xd, xd, loc.to(dev), k8, v8, ks, vs, ones.to(dev), ones.to(dev))
            q, s = ref.quant8(x)
            got = (k8, ks)
        else:
            k4 = torch.zeros(n, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
            ks = torch.zeros(n, H, 8, dtype=torch.float16, device=dev); vs = torch.zeros_like(ks)
            sa.quant_store_kv_int4(xd, xd, loc.to(dev), k4, v4, ks, vs, ones.to(dev), ones.to(dev))
            q, s = ref.quant4(x)
            got = (k4, ks)
        torch.cuda.synchronize()
        assert torch.equal(got[1].cpu(), s), group
        assert torch.equal(got[0].cpu(), q), group


@pytest.mark.parametrize("g8", [64, 256])
def test_append_evict_fp32_boundaries(kvt_pkg, g8):
    """The ring append with fp32 boundary rows (quotients at x.5 +- 1 ulp for the G64 ring scale): 200 tokens in
    chunks through a 64-row ring, so the requantized evictions are exercised too; every buffer bit-exact."""
    from kvtier.kvt import PosTieredCache
    dc = PosTieredCache(1, H, D, n_pages=8, ring_total=64, max_seqs=1, max_pages=8, device=dev, group8=g8,
                        page_seed=5)
    oc = ref.PosTieredCache(H, D, n_pages=8, ring_total=64, group8=g8)
    alloc = ref.PageAllocator(8, seed=5)
    dc.add_seq(64)
    oc.add_seq(0, 64)
    x = _boundary_rows(200, 64, 127.0, seed=9)
    done = 0
    for cnt in (1, 63, 64, 7, 64, 1):
        plan = dc.plan_append([0], [cnt])
        oc.plan_pages(0, cnt, alloc)
        xk, xv = x[done:done + cnt], -x[done:done + cnt]
        oc.append(0, xk, xv)
        dc.append(0, plan, xk.to(dev), xv.to(dev))
        dc.commit(plan)
        done += cnt
    torch.cuda.synchronize()
    assert torch.equal(dc.page_table.cpu(), oc.page_table(8))
    for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
        assert torch.equal(getattr(dc, name)[0].cpu(), getattr(oc, name)), name


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_unaligned_rows_all_writers(kvt_pkg, dt):
    """Rows whose stride (H * D + 1 elements) breaks the 8-byte chunk alignment take the element-load path: every
    token of the INT8, INT4 and ring-append writers bit-exact vs the oracle (600 tokens, more than one launch wave)."""
    from kvtier import sparse_attn as sa
    from kvtier.kvt import PosTieredCache
    gen = torch.Generator().manual_seed(12)
    n = 600
    x = (torch.randn(n, H, D, generator=gen) * 3).to(dt)
    wide = torch.zeros(n, H * D + 1, dtype=dt)
    wide[:, :H * D] = x.reshape(n, H * D)
    xd = wide.to(dev)[:, :H * D].view(n, H, D)
    smi = (0.5 + 1.5 * torch.rand(H, D, generator=gen)).half()
    loc = torch.arange(n, dtype=torch.int32)
    k8 = torch.zeros(n, H, D, dtype=torch.int8, device=dev); v8 = torch.zeros_like(k8)
    ks8 = torch.zeros(n, H, 4, dtype=torch.float16, device=dev); vs8 = torch.zeros_like(ks8)
    sa.quant_store_kv_int8(xd, xd, loc.to(dev), k8, v8, ks8, vs8, smi.to(dev), smi.to(dev))
    k4 = torch.zeros(n, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
    ks4 = torch.zeros(n, H, 8, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
    sa.quant_store_kv_int4(xd, xd, loc.to(dev), k4, v4, ks4, vs4, smi.to(dev), smi.to(dev))
    dc = PosTieredCache(1, H, D, n_pages=16, ring_total=512, max_seqs=1, max_pages=16, device=dev, page_seed=2)
    oc = ref.PosTieredCache(H, D, n_pages=16, ring_total=512)
    alloc = ref.PageAllocator(16, seed=2)
    dc.add_seq(512)
    oc.add_seq(0, 512)
    for a, cnt in ((0, 512), (512, 88)):
        plan = dc.plan_append([0], [cnt])
        oc.plan_pages(0, cnt, alloc)
        oc.append(0, x[a:a + cnt], x[a:a + cnt])
        dc.append(0, plan, xd[a:a + cnt], xd[a:a + cnt])
        dc.commit(plan)
    torch.cuda.synchronize()
    q8, s8 = ref.quant8(x, sm_inv=smi)
    p4, s4 = ref.quant4(x, sm_inv=smi)
    assert torch.equal(k8.cpu(), q8) and torch.equal(ks8.cpu(), s8) and torch.equal(v8.cpu(), q8)
    assert torch.equal(k4.cpu(), p4) and torch.equal(ks4.cpu(), s4) and torch.equal(vs4.cpu(), s4)
    assert torch.equal(dc.page_table.cpu(), oc.page_table(16))
    for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
        assert torch.equal(getattr(dc, name)[0].cpu(), getattr(oc, name)), name


@pytest.mark.parametrize("d", [64, 128])
def test_writers_other_head_dims(kvt_pkg, d):
    """head_dim 64 and 128 (a row uses D / 4 lanes; INT8 groups of 64 or the whole row): INT4, INT8 and tiered
    writers bit-exact vs the oracle, aligned rows and rows of stride H * d + 1 (element loads)."""
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(40 + d)
    n, slots, R = 300, 1024, 64
    x = (torch.randn(n, H, d, generator=gen) * 3).to(torch.bfloat16)
    smi = (0.5 + 1.5 * torch.rand(H, d, generator=gen)).half()
    loc = torch.randperm(slots, generator=gen)[:n]
    wide = torch.zeros(n, H * d + 1, dtype=torch.bfloat16)
    wide[:, :H * d] = x.reshape(n, H * d)
    for xd in (x.to(dev), wide.to(dev)[:, :H * d].view(n, H, d)):
        k4 = torch.zeros(slots, H, d // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
        ks4 = torch.zeros(slots, H, d // 32, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
        sa.quant_store_kv_int4(xd, xd, loc.to(dev), k4, v4, ks4, vs4, smi.to(dev), smi.to(dev))
        p4, s4 = ref.quant4(x, sm_inv=smi)
        assert torch.equal(k4.cpu()[loc], p4) and torch.equal(ks4.cpu()[loc], s4)
        for g8 in sorted({64, d}):
            k8 = torch.zeros(slots, H, d, dtype=torch.int8, device=dev); v8 = torch.zeros_like(k8)
            ks8 = torch.zeros(slots, H, d // g8, dtype=torch.float16, device=dev); vs8 = torch.zeros_like(ks8)
            sa.quant_store_kv_int8(xd, xd, loc.to(dev), k8, v8, ks8, vs8, smi.to(dev), smi.to(dev))
            q8, s8 = ref.quant8(x, group=g8, sm_inv=smi)
            assert torch.equal(k8.cpu()[loc], q8) and torch.equal(ks8.cpu()[loc], s8), g8
        # tiered: alias-free slots (distinct ring rows), so every row is hot
        tl = (torch.randperm(slots // R, generator=gen)[:1] * R + torch.randperm(R, generator=gen)[:48])
        b = [t.to(dev) for t in (
            torch.zeros(slots, H, d // 2, dtype=torch.uint8), torch.zeros(slots, H, d // 2, dtype=torch.uint8),
            torch.zeros(slots, H, d // 32, dtype=torch.float16), torch.zeros(slots, H, d // 32, dtype=torch.float16),
            torch.zeros(R, H, d, dtype=torch.int8), torch.zeros(R, H, d, dtype=torch.int8),
            torch.zeros(R, H, d // 64, dtype=torch.float16), torch.zeros(R, H, d // 64, dtype=torch.float16),
            torch.full((R,), -1, dtype=torch.int32))]
        sa.quant_store_kv_tiered(xd[:48], xd[:48], tl.to(dev), *b, smi.to(dev), smi.to(dev), R - 1)
        q8, s8 = ref.quant8(x[:48], sm_inv=smi)
        p4, s4 = ref.quant4(x[:48], sm_inv=smi)
        r = tl & (R - 1)
        assert torch.equal(b[4].cpu()[r], q8) and torch.equal(b[6].cpu()[r], s8)
        assert torch.equal(b[0].cpu()[tl], p4) and torch.equal(b[2].cpu()[tl], s4)
        assert torch.equal(b[8].cpu()[r].long(), tl)
