"""Host logic of the lazy KV backing (CPU): the commit / release policy of lazy_kv.LazyKVBacking and the allocator
hooks of tiered_kv_pool.PagedTokenAllocator, driven with stand-in arenas and pools.  The expected numbers are the
reference's rule worked by hand (patches/kv_lazy.py:119-121: want = min(size + page_size, ceil((n + margin) /
margin) * margin); :207-226: the paged hook asks for (max page + 1) * page_size slots and refuses the allocation on
failure; an idle pool returns to slot order and releases).  The arena itself (HIP VMM) is tested on the GPU."""
import pytest
import torch


class FakeArena:
    """Stand-in for VmmArena: mappings from offset 0, one per growing commit, granularity `g` bytes; memory is a CPU
    tensor poisoned with 7 so that the policy's zeroing of fresh rows shows."""

    def __init__(self, nbytes, g=4096, fail_first_commit=False):
        self.g = g
        self.reserved = -(-nbytes // g) * g
        self.maps = []
        self.mem = None
        self.fail = fail_first_commit
        self.commits = 0

    @property
    def backed(self):
        return self.maps[-1][0] + self.maps[-1][1] if self.maps else 0

    def commit(self, nbytes):
        self.commits += 1
        if self.fail:
            self.fail = False
            raise RuntimeError("kvt_vmm_commit: out of device address space or physical memory (status -5)")
        want = -(-nbytes // self.g) * self.g
        if want > self.reserved:
            raise ValueError("beyond the reservation")
        if want > self.backed:
            self.maps.append((self.backed, want - self.backed))

    def release_beyond(self, keep):
        cut = -(-keep // self.g) * self.g
        freed = 0
        while self.maps and self.maps[-1][0] >= cut:
            freed += self.maps.pop()[1]
        return freed

    def tensor(self, shape, dtype):
        self.mem = torch.full(shape, 7, dtype=dtype)
        return self.mem


def _backing(kvt_pkg, free=1 << 40, **kw):
    from kvtier.lazy_kv import LazyKVBacking
    arenas = []

    def factory(nbytes):
        arenas.append(FakeArena(nbytes, **kw))
        return arenas[-1]

    lz = LazyKVBacking(65600, 65536, 64, device="cpu", floor=4096, margin=2048, headroom_mb=1024,
                       arena_factory=factory, free_memory=lambda: free)
    return lz, arenas


def test_want_tokens_rule(kvt_pkg):
    lz, _ = _backing(kvt_pkg)
    # ceil((n + 2048) / 2048) * 2048, capped at 65536 + 64
    for n, want in [(0, 2048), (1, 4096), (2047, 4096), (2048, 4096), (2049, 6144), (5184, 8192), (11584, 14336),
                    (63487, 65536), (63489, 65600), (65600, 65600)]:
        assert lz.want_tokens(n) == want, n


def test_ensure_release_and_zeroing(kvt_pkg):
    lz, arenas = _backing(kvt_pkg)
    k = lz.add((65600, 2, 128), torch.uint8)
    s = lz.add((65600, 2, 8), torch.float16)
    assert lz.bytes_per_token() == 256 + 32 and lz.backed_tokens == 0
    lz.ensure_prefix(lz.floor)
    assert lz.backed_tokens == 4096
    assert [a.backed for a in arenas] == [4096 * 256, 4096 * 32]
    assert (k[:4096] == 0).all() and (k[4096:] == 7).all() and (s[:4096] == 0).all() and (s[4096:] == 7).all()
    k[:4096] = 3
    lz.ensure(5000)                           # slots up to 5000 -> 8192 backed, rows 4096.. zeroed, old rows kept
    assert lz.backed_tokens == 8192 and [a.backed for a in arenas] == [8192 * 256, 8192 * 32]
    assert (k[:4096] == 3).all() and (k[4096:8192] == 0).all() and (k[8192:] == 7).all()
    lz.ensure(100)                            # below the backed prefix: nothing
    assert [a.commits for a in arenas] == [2, 2]
    lz.ensure(11584)
    assert lz.backed_tokens == 14336 and [len(a.maps) for a in arenas] == [3, 3]
    freed = lz.release()                      # back to the floor: the two later mappings go
    assert lz.backed_tokens == 4096
    assert freed == (14336 - 4096) * (256 + 32)
    assert [len(a.maps) for a in arenas] == [1, 1] and [a.backed for a in arenas] == [4096 * 256, 4096 * 32]
    lz.ensure(5000)                           # recommitted rows read as zeros again
    assert (k[4096:8192] == 0).all() and (k[:4096] == 3).all()


def test_release_keeps_straddling_mapping(kvt_pkg):
    lz, arenas = _backing(kvt_pkg, g=1 << 20)   # 1 MiB granules: 4096 x 256 B = one granule, 4096 x 32 B = 1/8
    lz.add((65600, 2, 128), torch.uint8)
    lz.add((65600, 2, 8), torch.float16)
    lz.ensure_prefix(4096)
    assert arenas[1].backed == 1 << 20       # the scale buffer's first granule already holds 32,768 rows
    lz.ensure(20000)                          # want 22528: 5.5 MiB of codes, 704 KiB of scales (no new mapping)
    assert [len(a.maps) for a in arenas] == [2, 1]
    assert lz.release() == 5 << 20
    # codes: cut = align(4096 x 256 B) = 1 MiB, the second mapping starts there and goes; scales: the one mapping
    # straddles the cut (0 .. 1 MiB > 128 KiB) and stays
    assert [len(a.maps) for a in arenas] == [1, 1]
    assert arenas[1].backed == 1 << 20 and lz.backed_tokens == 4096
    lz.ensure(5000)                           # rows 4096 .. 8192 of the scales are backed already: zeroed, no commit
    assert [len(a.maps) for a in arenas] == [2, 1]


def test_headroom_refusal_and_commit_retry(kvt_pkg):
    # 1024 MB headroom: delta of ensure(5000) from the floor = 4096 x 288 B ~ 1.1 MB
    lz, arenas = _backing(kvt_pkg, free=(1024 << 20) // 2)   # below half the headroom after the commit: refused
    lz.add((65600, 2, 128), torch.uint8)
    lz.ensure_prefix(4096)
    with pytest.raises(RuntimeError, match="no headroom"):
        lz.ensure(5000)
    assert lz.backed_tokens == 4096 and arenas[0].commits == 1
    lz2, arenas2 = _backing(kvt_pkg, free=(1024 << 20) - 1)   # inside the headroom but above half: proceeds
    lz2.add((65600, 2, 128), torch.uint8)
    lz2.ensure(10)
    assert lz2.backed_tokens == 4096
    lz3, arenas3 = _backing(kvt_pkg, fail_first_commit=True)  # a failed commit is retried once
    lz3.add((65600, 2, 128), torch.uint8)
    lz3.ensure(10)
    assert lz3.backed_tokens == 4096 and arenas3[0].commits == 2


class FakePool:
    def __init__(self, fail_above=None):
        self.ensured = []
        self.released = 0
        self.fail_above = fail_above

    def lazy_ensure(self, n):
        if self.fail_above is not None and n > self.fail_above:
            raise RuntimeError("KV lazy backing: no headroom")
        self.ensured.append(n)

    def lazy_release(self):
        self.released += 1


def test_paged_allocator_hooks(kvt_pkg):
    from kvtier.tiered_kv_pool import PagedTokenAllocator
    pool = FakePool(fail_above=64 * 11)
    a = PagedTokenAllocator(64 * 16, 64, pool)
    idx = a.alloc(128)
    assert idx.tolist() == list(range(64, 192)) and pool.ensured == [192]
    idx2 = a.alloc(64 * 8)                    # pages 3..10: (10 + 1) x 64 slots, allowed
    assert pool.ensured[-1] == 704 and int(idx2.max()) == 703
    n_free = a.available_size()
    assert a.alloc(64) is None                # page 11 needs 768 slots backed: refused, the page stays free
    assert a.available_size() == n_free and pool.released == 0
    with pytest.raises(ValueError):
        a.alloc(100)
    a.free(idx)                               # not idle yet
    assert pool.released == 0 and a.available_size() == n_free + 128
    a.free(idx2)                              # every page free: slot order again, backing released
    assert pool.released == 1 and a.free_pages.tolist() == list(range(1, 17))
    assert a.alloc(64 * 16) is None           # 16 pages: (16 + 1) x 64 > 704, refused
    pool.fail_above = None
    assert a.alloc(64 * 16).numel() == 1024 and a.available_size() == 0
    assert a.alloc(64) is None                # full


def test_eager_pool_lazy_methods_are_noops(kvt_pkg):
    from kvtier.tiered_kv_pool import MHATokenToKVPoolInt4
    p = MHATokenToKVPoolInt4(1024, 64, torch.uint8, 2, 256, 1, "cpu", lazy=False)
    assert p.lazy_backed_tokens == 1024 + 64
    p.lazy_ensure(10 ** 6)
    p.lazy_release()
