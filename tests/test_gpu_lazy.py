"""GPU tests of the lazy KV backing on HIP virtual memory (kvt_vmm_* + lazy_kv + the pools' lazy mode).

Every access stays inside the backed prefix: the arena test touches only bytes below `backed`, and the pool test
reads and writes only slots that the allocator handed out (each hand-out backs its slots first) or rows below
lazy_backed_tokens.  Parity: a lazily backed pool and an eagerly allocated one fed the same writes hold the same
bytes (bit-exact) and give the same decode output (the same kernel over the same bytes).
"""
import time

import pytest
import torch

pytestmark = pytest.mark.gpu
dev = "cuda"


def _pattern(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g).to(dev)


def test_vmm_arena_commit_release(kvt_pkg):
    from kvtier.lazy_kv import VmmArena
    a = VmmArena(40 << 20)
    g = a.granularity
    print(f"granularity {g} B, reserved {a.reserved} B", flush=True)
    assert g > 0 and a.reserved >= 40 << 20 and a.reserved % g == 0 and a.backed == 0 and a.n_mappings == 0
    t = a.tensor((a.reserved,), torch.uint8)
    assert t.data_ptr() == a.base
    a.commit(g + g // 2)                       # rounded up to 2 granules, one mapping each
    assert a.backed == 2 * g and a.n_mappings == 2
    p0 = _pattern(2 * g, 1)
    t[:2 * g].copy_(p0)
    a.commit(5 * g)                            # 3 more granules; the first two keep their contents
    assert a.backed == 5 * g and a.n_mappings == 5
    t[2 * g:5 * g].fill_(9)
    torch.cuda.synchronize()
    assert torch.equal(t[:2 * g], p0) and bool((t[2 * g:5 * g] == 9).all())
    a.commit(3 * g)                            # commits only grow
    assert a.backed == 5 * g and a.n_mappings == 5
    assert a.release_beyond(3 * g - 1) == 2 * g   # cut rounded up to 3g: granules 3 and 4 go
    assert a.backed == 3 * g and bool((t[2 * g:3 * g] == 9).all())
    assert a.release_beyond(2 * g) == g
    assert a.backed == 2 * g and a.n_mappings == 2
    assert torch.equal(t[:2 * g], p0)
    a.commit(4 * g)                            # backed again, fresh memory
    p1 = _pattern(2 * g, 2)
    t[2 * g:4 * g].copy_(p1)
    torch.cuda.synchronize()
    assert torch.equal(t[:2 * g], p0) and torch.equal(t[2 * g:4 * g], p1)
    with pytest.raises(ValueError):
        a.commit(a.reserved + g)               # beyond the reservation: KVT_ERANGE, nothing changes
    assert a.backed == 4 * g
    torch.cuda.synchronize()
    del t                                      # the arena goes with its last tensor
    a.close()


def _pool(lazy, size, layers):
    from kvtier.tiered_kv_pool import MHATokenToKVPoolTiered
    return MHATokenToKVPoolTiered(size, 64, torch.uint8, 2, 256, layers, dev, lazy=lazy)


def _write(pool, loc, k, v, layer):
    for i in range(0, loc.numel(), pool.ring_slots):   # one write holds at most a ring of tokens
        pool.set_kv_buffer(None, loc[i:i + pool.ring_slots], k[i:i + pool.ring_slots], v[i:i + pool.ring_slots],
                           layer_id_override=layer)


def _same_rows(a, b, rows):
    for lid in range(a.layer_num):
        for x, y in [(a.k_buffer, b.k_buffer), (a.v_buffer, b.v_buffer), (a.k_scale_buffer, b.k_scale_buffer),
                     (a.v_scale_buffer, b.v_scale_buffer)]:
            assert torch.equal(x[lid][rows], y[lid][rows]), lid
        for x, y in zip(a.get_kv_ring_buffer(lid), b.get_kv_ring_buffer(lid)):
            assert torch.equal(x, y), lid
    assert torch.equal(a.ring_owner, b.ring_owner)


def _decode(pool, layer, slots, q):
    """Fused top-k decode of one request whose positions 0 .. n-1 live at `slots`, every position selected."""
    from kvtier import sparse_attn as sa
    n = slots.numel()
    r2t = slots.to(dev, torch.int32).view(1, n).contiguous()
    idx = torch.arange(n, dtype=torch.int32, device=dev).view(1, n)
    seq = torch.tensor([n], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
    req = torch.zeros(1, dtype=torch.int64, device=dev)
    k, v = pool.get_kv_buffer(layer)
    ks, vs = pool.get_kv_scale_buffer(layer)
    smk, smv = pool.get_kv_smooth_buffer(layer)
    rk, rv, rks, rvs = pool.get_kv_ring_buffer(layer)
    return sa.qwen_sparse_decode_attn(q, k, v, r2t, req, idx, seq, cu, 1, n, ks, vs, smk, smv, 4, rk, rv, rks, rvs,
                                      pool.ring_owner, pool.ring_mask, scale=256 ** -0.5)


def test_lazy_tiered_pool_matches_eager(kvt_pkg, monkeypatch):
    from kvtier.tiered_kv_pool import PagedTokenAllocator
    monkeypatch.setenv("SGLANG_KV_TIERS_W", "1024")
    size, layers = 32768, 2
    lazy, eager = _pool(True, size, layers), _pool(False, size, layers)
    assert lazy.lazy_backed_tokens == 4096 and eager.lazy_backed_tokens == size + 64
    al = PagedTokenAllocator(size, 64, lazy)
    ae = PagedTokenAllocator(size, 64, eager)
    gen = torch.Generator().manual_seed(5)
    q = (torch.randn(1, 16, 256, generator=gen) / 4).to(torch.bfloat16).to(dev)
    live = []
    # rounds of hand-outs: pages 1..80 (slots < 5184 -> 8192 backed), pages 81..180 (-> 14336), then 181..200
    for rnd, n in enumerate([5120, 6400, 1280]):
        t0 = time.perf_counter()
        loc = al.alloc(n)
        dt = time.perf_counter() - t0
        loc_e = ae.alloc(n)
        assert torch.equal(loc.cpu(), loc_e.cpu())
        live.append(loc)
        want = -(-(int(loc.max()) + 1 + 2048) // 2048) * 2048
        print(f"round {rnd}: {n} slots, max slot {int(loc.max())}, backed {lazy.lazy_backed_tokens} "
              f"(alloc + commit {dt * 1e3:.2f} ms)", flush=True)
        assert lazy.lazy_backed_tokens == max(4096, want)
        for lid in range(layers):
            k = torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
            v = torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
            _write(lazy, loc.to(dev), k, v, lid)
            _write(eager, loc.to(dev), k, v, lid)
        torch.cuda.synchronize()
        _same_rows(lazy, eager, slice(0, lazy.lazy_backed_tokens))
    slots = torch.cat(live)
    for lid in range(layers):
        o_l = _decode(lazy, lid, slots, q)
        o_e = _decode(eager, lid, slots, q)
        torch.cuda.synchronize()
        assert torch.isfinite(o_e).all() and torch.equal(o_l, o_e), lid
    # every slot back: the lazy pool drops to the floor; the arenas keep only their first mappings
    for loc in live:
        al.free(loc)
        ae.free(loc)
    assert lazy.lazy_backed_tokens == 4096
    assert bool((lazy.ring_owner == -1).all())
    rows_ok = slice(0, 4096)
    _same_rows(lazy, eager, rows_ok)
    # a new hand-out past the floor backs fresh (zeroed) memory again; write and read it as before
    loc = al.alloc(64 * 90)
    assert torch.equal(loc.cpu(), ae.alloc(64 * 90).cpu()) and lazy.lazy_backed_tokens == 8192
    for lid in range(layers):
        k = torch.randn(loc.numel(), 2, 256, generator=gen).to(torch.bfloat16).to(dev)
        v = torch.randn(loc.numel(), 2, 256, generator=gen).to(torch.bfloat16).to(dev)
        _write(lazy, loc.to(dev), k, v, lid)
        _write(eager, loc.to(dev), k, v, lid)
        assert torch.equal(_decode(lazy, lid, loc, q), _decode(eager, lid, loc, q))
    torch.cuda.synchronize()
    written = loc.to(dev)
    for lid in range(layers):
        assert torch.equal(lazy.k_buffer[lid][written], eager.k_buffer[lid][written])
        assert torch.equal(lazy.v_scale_buffer[lid][written], eager.v_scale_buffer[lid][written])


def test_lazy_int8_pool_matches_eager(kvt_pkg):
    """The single-tier INT8-G64 pool in lazy mode: same bytes as the eager pool for the same hand-outs and writes;
    a hand-out that would cross the reservation is refused by the allocator, not by a fault."""
    from kvtier.tiered_kv_pool import MHATokenToKVPoolInt8, PagedTokenAllocator
    size = 16384
    lazy = MHATokenToKVPoolInt8(size, 64, torch.int8, 2, 256, 1, dev, lazy=True)
    eager = MHATokenToKVPoolInt8(size, 64, torch.int8, 2, 256, 1, dev, lazy=False)
    al, ae = PagedTokenAllocator(size, 64, lazy), PagedTokenAllocator(size, 64, eager)
    gen = torch.Generator().manual_seed(6)
    for n in (4096, 6144, 6144):
        loc = al.alloc(n)
        assert loc is not None and torch.equal(loc, ae.alloc(n))
        k = torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
        v = torch.randn(n, 2, 256, generator=gen).to(torch.bfloat16).to(dev)
        lazy.set_kv_buffer(None, loc.to(dev), k, v, layer_id_override=0)
        eager.set_kv_buffer(None, loc.to(dev), k, v, layer_id_override=0)
        torch.cuda.synchronize()
        rows = slice(0, lazy.lazy_backed_tokens)
        assert torch.equal(lazy.k_buffer[0][rows], eager.k_buffer[0][rows])
        assert torch.equal(lazy.v_scale_buffer[0][rows], eager.v_scale_buffer[0][rows])
    assert lazy.lazy_backed_tokens == size + 64          # 16,384 slots handed out: the whole pool backed
    assert al.alloc(64) is None                          # nothing left
