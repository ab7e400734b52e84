"""The no-allocation decode entry point (kvt_decode_mfma_noalloc: partials in the library's per-GPU scratch array)
against the entry points it combines (kvt_decode_mfma with caller-allocated partials + kvt_decode_combine), through
the C ABI: two calls in a row, the second on a smaller context, with tiles in the fixed order on both sides, so the
outputs must be identical bit for bit; a ragged batch through a split map; an oversized request refused before any
launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ = 2, 256, 16


def _cache(lens, ring, seed):
    from kvtier.kvt import PosTieredCache
    n_pages = sum(max(0, L - ring) // 64 + 2 for L in lens)
    c = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=ring * len(lens), max_seqs=len(lens),
                       max_pages=max(lens) // 64 + 2, device=dev, page_seed=seed)
    for _ in lens:
        c.add_seq(ring)
    g = torch.Generator(device=dev).manual_seed(seed)
    done = [0] * len(lens)
    while any(d < L for d, L in zip(done, lens)):
        act = [s for s in range(len(lens)) if done[s] < lens[s]]
        cnt = [min(ring, lens[s] - done[s]) for s in act]
        plan = c.plan_append(act, cnt)
        n = sum(cnt)
        k = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        c.append(0, plan, k, v)
        c.commit(plan)
        for s, m in zip(act, cnt):
            done[s] += m
    q = (torch.randn(len(lens), HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    return c, q


def test_noalloc_matches_allocating_entry_points(kvt_pkg):
    from kvtier.kvt import kvt_decode_attn, kvt_decode_attn_noalloc
    for lens, ring, splits, dt in (([40_000], 2048, 64, torch.float32), ([3_000], 512, 7, torch.bfloat16)):
        cache, q = _cache(lens, ring, seed=len(lens) + ring)
        want = kvt_decode_attn(cache, 0, q, impl="mfma", splits=splits, deterministic=True, out_dtype=dt)
        got = torch.full_like(want, float("nan"))
        kvt_decode_attn_noalloc(cache, 0, q, got, splits=splits, deterministic=True)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16) if dt == torch.bfloat16 else got.view(torch.int32),
                           want.view(torch.int16) if dt == torch.bfloat16 else want.view(torch.int32)), (lens, splits)


def test_noalloc_ragged_split_map(kvt_pkg):
    from kvtier.kvt import _split_map, decode_split_counts, kvt_decode_attn, kvt_decode_attn_noalloc
    cache, q = _cache([9_000, 1_500, 20_000], 1024, seed=9)
    ws = {}
    want = kvt_decode_attn(cache, 0, q, impl="mfma", deterministic=True, workspace=ws)
    counts = decode_split_counts(cache, HQ)
    smap, scounts, _ = _split_map(counts, {}, q.device)
    got = torch.empty_like(want)
    kvt_decode_attn_noalloc(cache, 0, q, got, splits=max(counts), split_map=smap, split_counts=scounts,
                            deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_noalloc_refuses_oversized_partials(kvt_pkg):
    """A request whose partials exceed the 8 MiB scratch raises ValueError and writes nothing."""
    from kvtier.kvt import kvt_decode_attn_noalloc
    cache, q = _cache([4_000], 1024, seed=3)
    out = torch.full((1, HQ, D), 7.0, device=dev)
    with pytest.raises(ValueError):
        kvt_decode_attn_noalloc(cache, 0, q, out, splits=600)    # 1 x 2 x 600 x 8 x 258 x 4 B > 8 MiB
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
