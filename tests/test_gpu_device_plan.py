"""Device-side append plans (kvt_append_plan through PosTieredCache.plan_device / launch_plan): the same cache state as
the host planner (plan_append / commit) for the same inputs -- codes, scales, page tables and lengths bit for bit,
pages in the seeded allocator's order (the oracle's PageAllocator) -- eagerly and replayed in a HIP graph together
with the decode, and the refusal paths (pool exhausted)."""
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ = 2, 256, 16
NAMES = ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs")


def _pair(rings, n_pages, seed, shared=0):
    """Two identical caches (one per planner); sequence 0 starts after a shared prefix of `shared` positions whose
    pages both caches pop first (sequence 1 references them too when there are at least two sequences)."""
    from kvtier.kvt import PosTieredCache
    cs = []
    for _ in range(2):
        c = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=sum(rings), max_seqs=len(rings), max_pages=64,
                           device=dev, page_seed=seed)
        pages = [c.alloc.pop() for _ in range(shared // 64)]
        for i, r in enumerate(rings):
            if shared and i < 2:
                c.add_seq(r, ring_start=shared, shared_pages=pages)
            else:
                c.add_seq(r)
        cs.append(c)
    return cs


def _same(a, b):
    for name in NAMES:
        assert torch.equal(getattr(a, name)[0], getattr(b, name)[0]), name
    assert torch.equal(a.page_table, b.page_table) and torch.equal(a.seq_lens, b.seq_lens)
    assert a.h_len == b.h_len and a.h_pages == b.h_pages and a.alloc.next == b.alloc.next


def test_device_plan_matches_host_plan(kvt_pkg):
    """Three sequences (rings 256 / 128 / 512; the first two share a 128-position prefix): chunked appends of
    several layouts, then 200 single-token steps; after each call both caches agree bit for bit, and the final
    page lists are the allocator's pages in request order."""
    host, devc = _pair([256, 128, 512], n_pages=64, seed=3, shared=128)
    g = torch.Generator(device=dev).manual_seed(7)
    layouts = [([0, 1, 2], [100, 50, 300]), ([2, 0], [200, 256]), ([1], [128]), ([0, 1, 2], [1, 1, 1])]
    plans = {}
    for step in range(203):
        seqs, counts = layouts[min(step, 3)]
        n = sum(counts)
        k = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        hp = host.plan_append(seqs, counts)
        host.append(0, hp, k, v)
        host.commit(hp)
        key = (tuple(seqs), tuple(counts))
        if key not in plans:
            plans[key] = devc.plan_device(seqs, counts)
        dp = plans[key]
        devc.launch_plan(dp)
        devc.append(0, dp, k, v)
        devc.commit(dp)
        if step < 4 or step % 50 == 0:
            torch.cuda.synchronize()
            _same(host, devc)
    torch.cuda.synchronize()
    _same(host, devc)
    assert int(devc.plan_status.item()) == 0
    assert devc.alloc.next == int(devc.free_head.item())
    order = ref.PageAllocator(64, seed=3).free
    used = sorted(p for s in range(3) for p in devc.h_pages[s][(2 if s < 2 else 0):]) + sorted(devc.h_pages[0][:2])
    assert sorted(used) == sorted(order[:devc.alloc.next])


def test_device_plan_many_sequences(kvt_pkg):
    """80 sequences in one call (the plan kernel's scan over more than one wavefront) and 3 in another: chunked
    appends, then single-token steps of all 80; both caches agree bit for bit after every call."""
    rings = [64 << (i % 2) for i in range(80)]
    host, devc = _pair(rings, n_pages=512, seed=5)
    g = torch.Generator(device=dev).manual_seed(11)
    chunk = [20 + (i * 7) % 44 for i in range(80)]   # at most one ring (64 rows) per append
    layouts = [(list(range(80)), chunk), (list(range(80)), chunk), ([5, 79, 40], [64, 64, 1]),
               (list(range(80)), [1] * 80)]
    for step in range(14):
        seqs, counts = layouts[min(step, 3)]
        n = sum(counts)
        k = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
        hp = host.plan_append(seqs, counts)
        host.append(0, hp, k, v)
        host.commit(hp)
        dp = devc.plan_device(seqs, counts)
        devc.launch_plan(dp)
        devc.append(0, dp, k, v)
        devc.commit(dp)
        torch.cuda.synchronize()
        _same(host, devc)
    assert int(devc.plan_status.item()) == 0


def test_device_plan_graph_replay(kvt_pkg):
    """One decode step -- device plan (one token per sequence), append, decode -- captured once and replayed 300
    times with fresh inputs copied in between: the cache then equals the host planner's after the same 300 appends,
    the last replay's output equals an eager decode of the final state bit for bit (fixed tile order), and
    sync_host() restores the host mirror."""
    from kvtier.kvt import kvt_decode_attn
    host, devc = _pair([512, 256], n_pages=64, seed=4)
    g = torch.Generator(device=dev).manual_seed(8)
    pre = [700, 300]
    k = torch.randn(sum(pre), H, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(sum(pre), H, D, device=dev, generator=g).to(torch.bfloat16)
    for c in (host, devc):   # the same prefill through the host planner
        for a in range(0, 700, 256):
            n0 = min(256, 700 - a)
            n1 = min(256, max(0, 300 - a))
            seqs = [0] + ([1] if n1 else [])
            cnts = [n0] + ([n1] if n1 else [])
            p = c.plan_append(seqs, cnts)
            kk = torch.cat([k[a:a + n0]] + ([k[700 + a:700 + a + n1]] if n1 else []))
            vv = torch.cat([v[a:a + n0]] + ([v[700 + a:700 + a + n1]] if n1 else []))
            c.append(0, p, kk, vv)
            c.commit(p)
    steps = 300
    knew = torch.randn(steps, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    vnew = torch.randn(steps, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    q = (torch.randn(2, HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    kin, vin = knew[0].clone(), vnew[0].clone()
    dp = devc.plan_device([0, 1], [1, 1])
    ws = {}
    out = torch.empty(2, HQ, D, device=dev)
    # warm-up: fill the workspace (decode of the current state), then capture one step
    kvt_decode_attn(devc, 0, q, out=out, impl="mfma", workspace=ws, splits=8, deterministic=True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        devc.launch_plan(dp)
        devc.append(0, dp, kin, vin)
        kvt_decode_attn(devc, 0, q, out=out, impl="mfma", workspace=ws, splits=8, deterministic=True)
    for i in range(steps):
        kin.copy_(knew[i])
        vin.copy_(vnew[i])
        graph.replay()
        hp = host.plan_append([0, 1], [1, 1])
        host.append(0, hp, knew[i], vnew[i])
        host.commit(hp)
    torch.cuda.synchronize()
    devc.sync_host()
    _same(host, devc)
    want = kvt_decode_attn(host, 0, q, impl="mfma", splits=8, deterministic=True)
    assert torch.equal(out, want)


def _prefilled_pair(seed):
    """Two caches (rings 512 / 256) holding the same 700 / 300-position prefill through the host planner."""
    host, devc = _pair([512, 256], n_pages=64, seed=seed)
    g = torch.Generator(device=dev).manual_seed(seed + 100)
    k = torch.randn(1000, H, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1000, H, D, device=dev, generator=g).to(torch.bfloat16)
    for c in (host, devc):
        for a in range(0, 700, 256):
            n0, n1 = min(256, 700 - a), min(256, max(0, 300 - a))
            seqs, cnts = [0] + ([1] if n1 else []), [n0] + ([n1] if n1 else [])
            p = c.plan_append(seqs, cnts)
            c.append(0, p, torch.cat([k[a:a + n0]] + ([k[700 + a:700 + a + n1]] if n1 else [])),
                     torch.cat([v[a:a + n0]] + ([v[700 + a:700 + a + n1]] if n1 else [])))
            c.commit(p)
    return host, devc, g


def test_decode_plan_in_graph(kvt_pkg):
    """A decode step with the step's decode plan -- device append plan, append, kvt_decode_plan, decode with the
    plan -- captured once and replayed 120 times: the plan is rebuilt from the device state at every replay, so the
    last output equals an eager decode without plan of the host planner's cache after the same appends (8 splits per
    sequence on both sides, fixed tile order: bit for bit)."""
    from kvtier.kvt import kvt_decode_attn, kvt_decode_plan
    host, devc, g = _prefilled_pair(5)
    steps = 120
    knew = torch.randn(steps, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    vnew = torch.randn(steps, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    q = (torch.randn(2, HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    kin, vin = knew[0].clone(), vnew[0].clone()
    dp = devc.plan_device([0, 1], [1, 1])
    ws = {}
    out = torch.empty(2, HQ, D, device=dev)
    kvt_decode_attn(devc, 0, q, out=out, impl="mfma", workspace=ws,
                    plan=kvt_decode_plan(devc, HQ, splits=8, workspace=ws), deterministic=True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        devc.launch_plan(dp)
        devc.append(0, dp, kin, vin)
        plan = kvt_decode_plan(devc, HQ, splits=8, workspace=ws)
        kvt_decode_attn(devc, 0, q, out=out, impl="mfma", workspace=ws, plan=plan, deterministic=True)
    for i in range(steps):
        kin.copy_(knew[i])
        vin.copy_(vnew[i])
        graph.replay()
        hp = host.plan_append([0, 1], [1, 1])
        host.append(0, hp, knew[i], vnew[i])
        host.commit(hp)
    torch.cuda.synchronize()
    devc.sync_host()
    _same(host, devc)
    want = kvt_decode_attn(host, 0, q, impl="mfma", splits=8, deterministic=True)
    assert torch.equal(out, want)


def test_host_plan_after_replays(kvt_pkg):
    """Host planning after graph replays of a captured device plan, without an explicit sync_host(): the cache reads
    the advanced device state back first, so the pages it hands out are the ones the device has not, and the cache
    equals the host planner's after the same appends (the device free list is never rewound)."""
    host, devc, g = _prefilled_pair(6)
    steps = 40
    knew = torch.randn(steps + 1, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    vnew = torch.randn(steps + 1, 2, H, D, device=dev, generator=g).to(torch.bfloat16)
    kin, vin = knew[0].clone(), vnew[0].clone()
    dp = devc.plan_device([0, 1], [1, 1])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        devc.launch_plan(dp)
        devc.append(0, dp, kin, vin)
    for i in range(steps):
        kin.copy_(knew[i])
        vin.copy_(vnew[i])
        graph.replay()
        hp = host.plan_append([0, 1], [1, 1])
        host.append(0, hp, knew[i], vnew[i])
        host.commit(hp)
    for c in (host, devc):            # then a host-planned chunk on both (devc without sync_host)
        p = c.plan_append([0, 1], [200, 100])
        c.append(0, p, torch.cat([knew[steps]] * 150)[:300], torch.cat([vnew[steps]] * 150)[:300])
        c.commit(p)
    torch.cuda.synchronize()
    _same(host, devc)


def test_device_plan_refusals(kvt_pkg):
    """Eagerly, a plan needing more pages than the pool holds raises before any launch; a launch through the C ABI
    with an empty free list raises the status flag, assigns no page, writes no page-table entry, and sync_host()
    reports it; a plan listing a sequence twice is refused."""
    from kvtier import _lib
    from kvtier.kvt import PosTieredCache
    c = PosTieredCache(1, H, D, n_pages=2, ring_total=64, max_seqs=1, max_pages=8, device=dev, page_seed=1)
    c.add_seq(64)
    with pytest.raises(ValueError):
        c.plan_device([0, 0], [1, 1])
    p = c.plan_device([0], [64])
    g = torch.Generator(device=dev).manual_seed(9)
    for _ in range(3):   # 192 positions: pages for positions 0 .. 127
        c.launch_plan(p)
        c.append(0, p, torch.randn(64, H, D, device=dev, generator=g).to(torch.bfloat16),
                 torch.randn(64, H, D, device=dev, generator=g).to(torch.bfloat16))
    with pytest.raises(RuntimeError):
        c.launch_plan(p)                 # positions 128 .. 191 need a third page
    torch.cuda.synchronize()
    pt0 = c.page_table.clone()
    empty = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("kvt_append_plan", 1, p.seqs_dev.data_ptr(), p.cu_dev.data_ptr(), c.seq_lens.data_ptr(),
              c.ring_len.data_ptr(), c.ring_start.data_ptr(), c.page_table.data_ptr(), c.page_table.stride(0),
              c.max_pages, empty.data_ptr(), 0, c.free_head.data_ptr(), p.seq_ids.data_ptr(), p.positions.data_ptr(),
              c.plan_status.data_ptr(), _lib.stream())
    torch.cuda.synchronize()
    assert int(c.plan_status.item()) == 1 and torch.equal(c.page_table, pt0) and int(c.seq_lens[0]) == 256
    with pytest.raises(RuntimeError):
        c.sync_host()


def test_capture_requires_host_ints(kvt_pkg):
    """Wrappers whose defaults would read a device value (a host synchronization, which breaks a graph capture) raise
    ValueError under capture before any launch: kvt_prefill_attn without max_q, decode_attn_slots without max_len.
    With the host ints passed the same calls capture and replay."""
    from kvtier.kvt import decode_attn_slots, kvt_prefill_attn
    host, devc, g = _prefilled_pair(8)
    q = (torch.randn(300, HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    cu_q = torch.tensor([0, 200, 300], dtype=torch.int32, device=dev)
    kvt_prefill_attn(devc, 0, q, cu_q, max_q=200)   # the workspace exists before the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        gr = torch.cuda.CUDAGraph()
        with pytest.raises(ValueError, match="max_q"):
            with torch.cuda.graph(gr, stream=side):
                kvt_prefill_attn(devc, 0, q, cu_q)
    torch.cuda.synchronize()
    out = torch.empty_like(q)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        kvt_prefill_attn(devc, 0, q, cu_q, max_q=200, out=out)
    gr.replay()
    torch.cuda.synchronize()
    want = kvt_prefill_attn(devc, 0, q, cu_q, max_q=200)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    # the slot-indexed decode: max_len under capture
    slots, R = 1024, 64
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, device=dev)
    ks4 = torch.full((slots, H, D // 32), 0.01, dtype=torch.float16, device=dev)
    rk = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, device=dev)
    rks = torch.full((R, H, D // 64), 0.01, dtype=torch.float16, device=dev)
    owner = torch.full((R,), -1, dtype=torch.int32, device=dev)
    r2t = torch.arange(slots, dtype=torch.int32, device=dev).reshape(2, 512)
    qd = (torch.randn(2, HQ, D, device=dev, generator=g) / 16).to(torch.bfloat16)
    sl = torch.tensor([500, 77], dtype=torch.int32, device=dev)
    ridx = torch.arange(2, dtype=torch.int64, device=dev)
    args = (qd, sl, r2t, ridx, k4, k4, ks4, ks4, rk, rk, rks, rks, owner, R - 1)
    ws = {}
    eager = decode_attn_slots(*args, max_len=512, workspace=ws)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        gr = torch.cuda.CUDAGraph()
        with pytest.raises(ValueError, match="max_len"):
            with torch.cuda.graph(gr, stream=side):
                decode_attn_slots(*args, workspace=ws)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        cap = decode_attn_slots(*args, max_len=512, workspace=ws)
    gr.replay()
    torch.cuda.synchronize()
    assert torch.equal(cap, eager)
