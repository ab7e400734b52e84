"""GPU parity of the gather-dequant kernels (bit-exact bf16 rows, store-mask rules) against the CPU oracle.

Follows gemv/test_kv_tiers.py sections 3-5 and gemv/test_kv_int4.py / test_kv_int8.py sections 3-4: random owner
pattern with poisoned unowned ring rows, invalid positions, the trtllm strided scratch, a stale owner, 32-row gaps
in the prefix gather, and the all-cold / all-hot equivalences with the single-tier gathers.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D = 2, 256
SLOTS, R, BATCH, TOPK = 4096, 64, 3, 64


@pytest.fixture(scope="module")
def tiered_state():
    """Full pool written by the GPU writer, then a random owner pattern with re-quantized hot rows and poisoned
    unowned rows (gemv/test_kv_tiers.py:237-274).  Returns device tensors and the per-slot references."""
    import kvtier  # noqa: F401
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(10)
    k16 = (torch.randn(SLOTS, H, D, generator=gen) * 3).to(torch.bfloat16)
    v16 = (torch.randn(SLOTS, H, D, generator=gen) * 3).to(torch.bfloat16)
    sm_k = (0.5 + 1.5 * torch.rand(H, D, generator=gen)).half()
    sm_v = (0.5 + 1.5 * torch.rand(H, D, generator=gen)).half()
    smi_k, smi_v = (1.0 / sm_k.float()).half(), (1.0 / sm_v.float()).half()
    k4 = torch.zeros(SLOTS, H, D // 2, dtype=torch.uint8, device=dev); v4 = torch.zeros_like(k4)
    ks4 = torch.zeros(SLOTS, H, 8, dtype=torch.float16, device=dev); vs4 = torch.zeros_like(ks4)
    rk = torch.zeros(R, H, D, dtype=torch.int8, device=dev); rv = torch.zeros_like(rk)
    rks = torch.zeros(R, H, 4, dtype=torch.float16, device=dev); rvs = torch.zeros_like(rks)
    owner = torch.full((R,), -1, dtype=torch.int32, device=dev)
    for a in range(0, SLOTS, R):
        sa.quant_store_kv_tiered(k16[a:a + R].to(dev), v16[a:a + R].to(dev), torch.arange(a, a + R, device=dev,
                                 dtype=torch.int32), k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, smi_k.to(dev),
                                 smi_v.to(dev), R - 1)
    torch.cuda.synchronize()
    pk, sk = ref.quant4(k16, smi_k)
    pv, sv = ref.quant4(v16, smi_v)
    assert torch.equal(k4.cpu(), pk) and torch.equal(ks4.cpu(), sk) and torch.equal(v4.cpu(), pv)
    assert torch.equal(owner.cpu().long(), torch.arange(SLOTS - R, SLOTS))
    n_cls = SLOTS // R
    pick = torch.randint(0, n_cls, (R,), generator=gen)
    pick = torch.where(torch.rand(R, generator=gen) < 0.35, torch.full_like(pick, -1), pick)
    own = torch.where(pick < 0, torch.full_like(pick, -1), pick * R + torch.arange(R))
    own[0], own[1], own[2] = 0, -1, 2 + R * (n_cls - 1)
    owner.copy_(own.to(torch.int32))
    hot_rows = torch.nonzero(own >= 0).flatten()
    sa.quant_store_kv_int8(k16[own[hot_rows]].to(dev), v16[own[hot_rows]].to(dev), hot_rows.to(torch.int32).to(dev),
                           rk, rv, rks, rvs, smi_k.to(dev), smi_v.to(dev))
    dead = torch.nonzero(own < 0).flatten().to(dev)
    rk[dead] = -128; rv[dead] = 127; rks[dead] = float("nan"); rvs[dead] = float("inf")
    torch.cuda.synchronize()
    kc = [t.cpu() for t in (k4, v4, ks4, vs4, rk, rv, rks, rvs, owner)]
    all_slots = torch.arange(SLOTS)
    dk_all, dv_all = ref.dequant_slots_tiered(all_slots, *kc, R - 1, sm_k, sm_v)
    is_hot = ref.is_hot(all_slots, kc[8], R - 1)
    assert 10 < int(is_hot.sum()) < R
    d4k = ref.dequant4(pk, sk, sm_k)
    return dict(k4=k4, v4=v4, ks4=ks4, vs4=vs4, rk=rk, rv=rv, rks=rks, rvs=rvs, owner=owner, sm_k=sm_k.to(dev),
                sm_v=sm_v.to(dev), dk_all=dk_all, dv_all=dv_all, is_hot=is_hot, d4k=d4k, gen=gen, k16=k16, v16=v16,
                smi_k=smi_k, smi_v=smi_v)


def _tier_kwargs(st):
    return dict(k_scale=st["ks4"], v_scale=st["vs4"], sm_k=st["sm_k"], sm_v=st["sm_v"], kv_bits=4, ring_k=st["rk"],
                ring_v=st["rv"], ring_ks=st["rks"], ring_vs=st["rvs"], owner=st["owner"], ring_mask=R - 1)


def _run_compact(st, req_to_token, req_indices, idx, seq_lens, kw):
    from kvtier import sparse_attn as sa
    cu_k = torch.empty(BATCH + 1, dtype=torch.int32, device=dev)
    counts = torch.empty(BATCH, dtype=torch.int32, device=dev)
    sa.qwen_sparse_fa2_cu_seqlens_triton(seq_lens, idx, counts, cu_k, BATCH, idx.shape[1])
    n = int(cu_k[-1])
    out_k = torch.full((BATCH * idx.shape[1] + 16, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    out_v = torch.full_like(out_k, float("nan"))
    sa.qwen_sparse_kv_extraction_compact_triton(st["k4"], st["v4"], req_to_token, req_indices, idx, seq_lens, cu_k,
                                                out_k, out_v, BATCH, idx.shape[1], **kw)
    torch.cuda.synchronize()
    return cu_k.cpu(), n, out_k.cpu(), out_v.cpu()


def test_compact_gather_tiered(tiered_state):
    st = tiered_state
    gen = st["gen"]
    seq_lens = torch.tensor([300, 1200, 4000], dtype=torch.int32)
    rtt = torch.stack([torch.randperm(SLOTS, generator=gen) for _ in range(BATCH)]).to(torch.int32)
    idx = torch.stack([torch.randperm(int(l), generator=gen)[:TOPK].sort().values for l in seq_lens]).to(torch.int32)
    for b in range(BATCH):                       # make every request select hot slots too
        hot_pos = torch.nonzero(st["is_hot"][rtt[b, :int(seq_lens[b])].long()]).flatten()
        if hot_pos.numel():
            take = hot_pos[torch.randperm(hot_pos.numel(), generator=gen)[:8]]
            rest = torch.tensor([p for p in idx[b].tolist() if p not in set(take.tolist())], dtype=torch.int64)
            idx[b] = torch.cat([rest[:TOPK - take.numel()], take]).sort().values.to(torch.int32)
    rq = torch.arange(BATCH, dtype=torch.int32)
    cu_k, n, ok, ov = _run_compact(st, rtt.to(dev), rq.to(dev), idx.to(dev), seq_lens.to(dev), _tier_kwargs(st))
    assert n == BATCH * TOPK
    n_hot = 0
    for b in range(BATCH):
        rows = rtt[b, idx[b].long()].long()
        a, e = int(cu_k[b]), int(cu_k[b + 1])
        assert torch.equal(ok[a:e], st["dk_all"][rows]) and torch.equal(ov[a:e], st["dv_all"][rows])
        n_hot += int(st["is_hot"][rows].sum())
    assert 10 < n_hot < n
    assert torch.isnan(ok[n:]).all() and torch.isfinite(ok[:n]).all()
    # int4-only call on the same buffers: plain int4 rows
    kw4 = dict(k_scale=st["ks4"], v_scale=st["vs4"], sm_k=st["sm_k"], sm_v=st["sm_v"], kv_bits=4)
    _, _, ok4, _ = _run_compact(st, rtt.to(dev), rq.to(dev), idx.to(dev), seq_lens.to(dev), kw4)
    for b in range(BATCH):
        rows = rtt[b, idx[b].long()].long()
        assert torch.equal(ok4[int(cu_k[b]):int(cu_k[b + 1])], st["d4k"][rows])
    # invalid position inside the packed region: row untouched
    bad = idx.clone(); bad[1, 0] = int(seq_lens[1]) + 5
    cu_b, n_b, ok_b, _ = _run_compact(st, rtt.to(dev), rq.to(dev), bad.to(dev), seq_lens.to(dev), _tier_kwargs(st))
    assert n_b == n - 1 and torch.isnan(ok_b[int(cu_b[1])]).all()
    # stale owner -> int4 path
    sel_slot = int(rtt[0, idx[0, 3].long()])
    saved = int(st["owner"][sel_slot & (R - 1)])
    st["owner"][sel_slot & (R - 1)] = sel_slot + R if sel_slot + R < SLOTS else sel_slot - R
    cu_t, _, ok_t, _ = _run_compact(st, rtt.to(dev), rq.to(dev), idx.to(dev), seq_lens.to(dev), _tier_kwargs(st))
    assert torch.equal(ok_t[int(cu_t[0]) + 3], st["d4k"][sel_slot])
    st["owner"][sel_slot & (R - 1)] = saved


def test_compact_gather_strided_layout(tiered_state):
    """cu_k = arange * 64 > topk 40, -1 padding, a position >= seq_len: only valid rows written
    (gemv/test_kv_tiers.py:342-368)."""
    from kvtier import sparse_attn as sa
    st = tiered_state
    gen = torch.Generator().manual_seed(12)
    seq_lens = torch.tensor([300, 1200, 4000], dtype=torch.int32)
    rtt = torch.stack([torch.randperm(SLOTS, generator=gen) for _ in range(BATCH)]).to(torch.int32)
    topk_s, stride_s = 40, 64
    cu_s = torch.arange(BATCH + 1, dtype=torch.int32) * stride_s
    nsel = [topk_s, 25, 33]
    idx_s = torch.full((BATCH, topk_s), -1, dtype=torch.int32)
    for b in range(BATCH):
        idx_s[b, :nsel[b]] = torch.randperm(int(seq_lens[b]), generator=gen)[:nsel[b]].sort().values.to(torch.int32)
    idx_s[2, 5] = int(seq_lens[2]) + 3
    ok = torch.full((BATCH * stride_s, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    ov = torch.full_like(ok, float("nan"))
    sa.qwen_sparse_kv_extraction_compact_triton(st["k4"], st["v4"], rtt.to(dev), torch.arange(BATCH, device=dev,
                                                dtype=torch.int32), idx_s.to(dev), seq_lens.to(dev), cu_s.to(dev), ok,
                                                ov, BATCH, topk_s, **_tier_kwargs(st))
    torch.cuda.synchronize()
    ok, ov = ok.cpu(), ov.cpu()
    written = torch.zeros(BATCH * stride_s, dtype=torch.bool)
    for b in range(BATCH):
        for c in range(topk_s):
            pos = int(idx_s[b, c])
            if 0 <= pos < int(seq_lens[b]):
                r_ = b * stride_s + c
                slot = int(rtt[b, pos])
                assert torch.equal(ok[r_], st["dk_all"][slot]) and torch.equal(ov[r_], st["dv_all"][slot])
                written[r_] = True
    assert int(written.sum()) == sum(nsel) - 1
    assert torch.isnan(ok[~written]).all() and torch.isnan(ov[~written]).all()


def test_prefix_gather_tiered_gaps(tiered_state):
    """3 lengths (partial last block, non-identity req_indices int64), 32-row gaps: rows bit-exact, gaps and tail
    untouched (gemv/test_kv_tiers.py:380-410)."""
    from kvtier import sparse_attn as sa
    st = tiered_state
    gen = torch.Generator().manual_seed(13)
    rtt = torch.stack([torch.randperm(SLOTS, generator=gen) for _ in range(BATCH)]).to(torch.int32)
    lens = torch.tensor([300, 1203, 4001], dtype=torch.int32)
    lens[2] = min(int(lens[2]), SLOTS)
    req_idx = torch.tensor([2, 0, 1], dtype=torch.int64)
    GAP = 32
    cu = F.pad((lens + GAP).cumsum(0), (1, 0)).to(torch.int32).contiguous()
    total = int(cu[-1])
    pk = torch.full((total + 100, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    pv = torch.full_like(pk, float("nan"))
    sa.qwen_sparse_prefix_gather_dequant_tiered(st["k4"], st["v4"], st["ks4"], st["vs4"], st["sm_k"], st["sm_v"],
                                                rtt.to(dev), req_idx.to(dev), lens.to(dev), cu.to(dev), pk, pv, BATCH,
                                                int(lens.max()), ring_k=st["rk"], ring_v=st["rv"], ring_ks=st["rks"],
                                                ring_vs=st["rvs"], owner=st["owner"], ring_mask=R - 1)
    torch.cuda.synchronize()
    pk, pv = pk.cpu(), pv.cpu()
    written = torch.zeros(pk.shape[0], dtype=torch.bool)
    for b in range(BATCH):
        rows = rtt[int(req_idx[b]), :int(lens[b])].long()
        a, e = int(cu[b]), int(cu[b]) + int(lens[b])
        assert torch.equal(pk[a:e], st["dk_all"][rows]) and torch.equal(pv[a:e], st["dv_all"][rows])
        written[a:e] = True
    assert torch.isnan(pk[~written]).all() and torch.isnan(pv[~written]).all()


def test_single_tier_gathers(tiered_state):
    """int4 and int8 pool gathers (compact + prefix) bit-exact vs the oracle's dequant (gemv/test_kv_int4.py:140-247,
    gemv/test_kv_int8.py:101-163)."""
    from kvtier import sparse_attn as sa
    st = tiered_state
    k16, v16 = st["k16"], st["v16"]
    k8 = torch.zeros(SLOTS, H, D, dtype=torch.int8, device=dev); v8 = torch.zeros_like(k8)
    ks8 = torch.zeros(SLOTS, H, 4, dtype=torch.float16, device=dev); vs8 = torch.zeros_like(ks8)
    sa.quant_store_kv_int8(k16.to(dev), v16.to(dev), torch.arange(SLOTS, device=dev), k8, v8, ks8, vs8,
                           st["smi_k"].to(dev), st["smi_v"].to(dev))
    torch.cuda.synchronize()
    q8, s8 = ref.quant8(k16, 64, st["smi_k"])
    assert torch.equal(k8.cpu(), q8) and torch.equal(ks8.cpu(), s8)
    d8 = ref.dequant8(q8, s8, st["sm_k"].cpu())
    gen = torch.Generator().manual_seed(14)
    rtt = torch.stack([torch.randperm(SLOTS, generator=gen) for _ in range(BATCH)]).to(torch.int32)
    lens = torch.tensor([77, 1000, 2049], dtype=torch.int32)
    cu = F.pad(lens.cumsum(0), (1, 0)).to(torch.int32).contiguous()
    pk = torch.full((int(cu[-1]), H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    pv = torch.full_like(pk, float("nan"))
    sa.qwen_sparse_prefix_gather_dequant_int8(k8, v8, ks8, vs8, st["sm_k"], st["sm_v"], rtt.to(dev),
                                              torch.arange(BATCH, device=dev), lens.to(dev), cu.to(dev), pk, pv, BATCH,
                                              int(lens.max()))
    torch.cuda.synchronize()
    for b in range(BATCH):
        rows = rtt[b, :int(lens[b])].long()
        assert torch.equal(pk.cpu()[int(cu[b]):int(cu[b + 1])], d8[rows])
    pk.fill_(float("nan"))
    sa.qwen_sparse_prefix_gather_dequant_int4(st["k4"], st["v4"], st["ks4"], st["vs4"], st["sm_k"], st["sm_v"],
                                              rtt.to(dev), torch.arange(BATCH, device=dev), lens.to(dev), cu.to(dev),
                                              pk, pv, BATCH, int(lens.max()))
    torch.cuda.synchronize()
    for b in range(BATCH):
        rows = rtt[b, :int(lens[b])].long()
        assert torch.equal(pk.cpu()[int(cu[b]):int(cu[b + 1])], st["d4k"][rows])
    # compact int8
    seq_lens = lens
    idx = torch.stack([torch.randperm(int(l), generator=gen)[:TOPK].sort().values for l in seq_lens]).to(torch.int32)
    kw8 = dict(k_scale=ks8, v_scale=vs8, sm_k=st["sm_k"], sm_v=st["sm_v"])
    cu_k = torch.empty(BATCH + 1, dtype=torch.int32, device=dev)
    sa.qwen_sparse_fa2_cu_seqlens_triton(seq_lens.to(dev), idx.to(dev), torch.empty(BATCH, dtype=torch.int32, device=dev),
                                         cu_k, BATCH, TOPK)
    ok = torch.full((BATCH * TOPK, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    sa.qwen_sparse_kv_extraction_compact_triton(k8, v8, rtt.to(dev), torch.arange(BATCH, device=dev, dtype=torch.int32),
                                                idx.to(dev), seq_lens.to(dev), cu_k, ok, torch.empty_like(ok), BATCH,
                                                TOPK, **kw8)
    torch.cuda.synchronize()
    cu_k = cu_k.cpu()
    for b in range(BATCH):
        rows = rtt[b, idx[b].long()].long()
        assert torch.equal(ok.cpu()[int(cu_k[b]):int(cu_k[b + 1])], d8[rows])


def test_gathers_reject_misaligned_scratch(tiered_state):
    """The gathers store 16 bytes per lane: a scratch whose base is not 16-byte aligned is refused before any launch
    (ValueError, nothing written); a row slice of an aligned allocation (offset 8 rows) is served and matches."""
    from kvtier import sparse_attn as sa
    st = tiered_state
    gen = torch.Generator().manual_seed(14)
    rtt = torch.stack([torch.randperm(SLOTS, generator=gen) for _ in range(BATCH)]).to(torch.int32).to(dev)
    lens = torch.tensor([40, 7, 100], dtype=torch.int32, device=dev)
    cu = F.pad(lens.cumsum(0), (1, 0)).to(torch.int32)
    req_idx = torch.arange(BATCH, dtype=torch.int64, device=dev)
    n = int(cu[-1])
    flat = torch.full(((n + 8) * H * D + 8,), float("nan"), device=dev, dtype=torch.bfloat16)
    bad_k = flat[1:1 + n * H * D].view(n, H, D)                 # base 2 bytes past an aligned allocation
    good = torch.full((n + 8, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    kw = dict(ring_k=st["rk"], ring_v=st["rv"], ring_ks=st["rks"], ring_vs=st["rvs"], owner=st["owner"],
              ring_mask=R - 1)
    args = (st["k4"], st["v4"], st["ks4"], st["vs4"], st["sm_k"], st["sm_v"], rtt, req_idx, lens, cu)
    with pytest.raises(ValueError):
        sa.qwen_sparse_prefix_gather_dequant_tiered(*args, bad_k, good[8:], BATCH, int(lens.max()), **kw)
    torch.cuda.synchronize()
    assert torch.isnan(flat).all() and torch.isnan(good).all()
    other = torch.full((n, H, D), float("nan"), device=dev, dtype=torch.bfloat16)
    sa.qwen_sparse_prefix_gather_dequant_tiered(*args, good[8:], other, BATCH, int(lens.max()), **kw)
    torch.cuda.synchronize()
    gk, gv = good[8:].cpu(), other.cpu()
    for b in range(BATCH):
        rows = rtt[b, :int(lens[b])].long().cpu()
        a, e = int(cu[b]), int(cu[b + 1])
        assert torch.equal(gk[a:e], st["dk_all"][rows]) and torch.equal(gv[a:e], st["dv_all"][rows])


@pytest.mark.parametrize("batch,topk,cu64,shared", [(0, 64, False, False), (1, 1, False, False), (3, 63, True, False),
                                                     (7, 2051, False, False), (1500, 65, True, False),
                                                     (2100, 130, False, False), (5, 200, False, True)])
def test_cu_seqlens_kernel(kvt_pkg, batch, topk, cu64, shared):
    """kvt_sparse_cu_seqlens against the oracle's count and prefix sum (pinned by brute force on the CPU): columns
    below 0 (the -1 padding of a top-k), at or past seq_len, ragged lengths including 0, more rows than the block's
    1024 threads (two scan chunks with a carry), a row stride of 0 (one index row shared by every request) and the
    int64 offsets; counts and cu_k bit-exact, nothing written past cu_k[batch]."""
    from kvtier import sparse_attn as sa
    g = torch.Generator().manual_seed(batch * 7 + topk)
    seq = torch.randint(0, 3000, (max(batch, 1),), generator=g, dtype=torch.int32)
    if batch:
        seq[0] = 0
    width = topk + 5
    rows = 1 if shared else max(batch, 1)
    idx = torch.randint(-3, 3200, (rows, width), generator=g, dtype=torch.int32)
    idx[:, ::7] = -1
    idx_dev = idx.to(dev)
    if shared:
        idx_dev = idx_dev[:1].expand(batch, width)
        idx_full = idx.expand(batch, width)
    else:
        idx_full = idx[:batch]
    counts = torch.full((batch + 2,), -7, dtype=torch.int32, device=dev)
    cu = torch.full((batch + 3,), -7, dtype=torch.int64 if cu64 else torch.int32, device=dev)
    sa.qwen_sparse_fa2_cu_seqlens_triton(seq.to(dev), idx_dev, counts, cu, batch, topk)
    torch.cuda.synchronize()
    want = ref.cu_seqlens_valid(seq[:batch], idx_full, topk)
    assert torch.equal(cu.cpu()[:batch + 1].to(torch.int32), want)
    assert torch.equal(counts.cpu()[:batch], (want[1:] - want[:-1]))
    assert bool((cu.cpu()[batch + 1:] == -7).all()) and bool((counts.cpu()[batch:] == -7).all())
