"""GPU parity at the configurations' own shapes (the headline and configs 1, 3 and 4), against the oracle.

Inputs are seeded and generated on the device, then copied to the host, so the HIP path and the oracle see the same
bits.  Codes, scales and page tables are compared bit for bit with the oracle's closed forms: a position p older than
the ring holds requant8to4(quant8(x[p])) in the page the seeded allocator gave its logical page, a newer one
quant8(x[p]) in ring row p & (R - 1) (oracle/ref.py evict_closed_form, pinned against the token-by-token model).
Attention outputs (fp32) are held to 2e-3 max-abs / 1e-3 mean-abs of the oracle's fp32 softmax over its own bf16 rows
(ref.attention_rows, the form of gemv/test_kv_paged_prefix.py:506-531).
"""
import math

import pytest
import torch

from kvt_testutil import close
from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D, HQ, RING, PAGE = 2, 256, 16, 8192, 64
SCALE = D ** -0.5


def _dev_kv(n, seed, outlier=True):
    """n seeded tokens (K with 8 outlier channels per head x8, V ~ N(0, 1)), bf16, generated on the device; returns
    the device tensors and their host copies."""
    gc = torch.Generator().manual_seed(seed)
    mul = torch.ones(H, D)
    if outlier:
        for h in range(H):
            mul[h, torch.randperm(D, generator=gc)[:8]] = 8.0
    g = torch.Generator(device=dev).manual_seed(seed)
    k = (torch.randn(n, H, D, device=dev, generator=g) * mul.to(dev)).to(torch.bfloat16)
    v = torch.randn(n, H, D, device=dev, generator=g).to(torch.bfloat16)
    return k, v, k.cpu(), v.cpu()


class Forms:
    """Both tier forms of every appended token of one sequence: quant8 (ring) and requant8to4 of it (pages)."""

    def __init__(self, xk, xv, group8=64):
        self.g8 = group8
        self.q8k, self.s8k = ref.quant8(xk, group8)
        self.q8v, self.s8v = ref.quant8(xv, group8)
        self.p4k, self.s4k = ref.requant8to4(self.q8k, self.s8k, group8)
        self.p4v, self.s4v = ref.requant8to4(self.q8v, self.s8v, group8)

    def rows(self, hs, L):
        """Oracle bf16 K, V rows of positions 0 .. L-1 (rows of this object) with positions < hs in INT4."""
        kk = torch.cat([ref.dequant4(self.p4k[:hs], self.s4k[:hs]), ref.dequant8(self.q8k[hs:L], self.s8k[hs:L], None, self.g8)])
        vv = torch.cat([ref.dequant4(self.p4v[:hs], self.s4v[:hs]), ref.dequant8(self.q8v[hs:L], self.s8v[hs:L], None, self.g8)])
        return kk, vv


def _check_seq_codes(cache, layer, s, forms, lo, hs, L, pages, base=0):
    """Bit-exact device state of sequence s in `layer`: positions lo .. hs-1 (forms rows 0 ..) in their pages,
    positions hs .. L-1 in the ring rows of the sequence (ring base `base`, ring length from the cache)."""
    R = cache.h_ring[s][1]
    pos = torch.arange(lo, hs)
    if pos.numel():
        rows = (torch.tensor(pages, dtype=torch.long)[pos // PAGE] * PAGE + pos % PAGE).to(dev)
        f = slice(0, hs - lo)
        for name, want in (("k4", forms.p4k[f]), ("ks4", forms.s4k[f]), ("v4", forms.p4v[f]), ("vs4", forms.s4v[f])):
            assert torch.equal(getattr(cache, name)[layer][rows].cpu(), want), (name, layer, s)
    pos = torch.arange(hs, L)
    rr = (base + (pos & (R - 1))).to(dev)
    f = slice(hs - lo, L - lo)
    for name, want in (("rk", forms.q8k[f]), ("rks", forms.s8k[f]), ("rv", forms.q8v[f]), ("rvs", forms.s8v[f])):
        assert torch.equal(getattr(cache, name)[layer][rr].cpu(), want), (name, layer, s)


# ----------------------------------------------------------------------------------------------- headline (config 2)
@pytest.fixture(scope="module")
def headline():
    """bench.py's headline cache: 262,144 positions x 12 layers (ring 8,192 + 3,968 permuted INT4 pages)."""
    import bench
    cache, q = bench.build_cache()
    torch.cuda.synchronize()
    return bench, cache, q


def test_headline_page_table(kvt_pkg, headline):
    """3,968 logical pages -> the first 3,968 pages of the seeded permutation, in order (shared by all layers)."""
    bench, cache, _ = headline
    n_pages = (bench.CTX - bench.RING) // PAGE
    want = ref.PageAllocator(n_pages, seed=0).free[:n_pages]
    assert cache.page_table[0, :n_pages].cpu().tolist() == want and cache.h_pages[0] == want
    assert int(cache.seq_lens[0]) == bench.CTX and cache.hot_start(0) == bench.CTX - bench.RING


@pytest.mark.parametrize("layer", range(12))
def test_headline_layer(kvt_pkg, headline, layer):
    """One layer of the headline: every code and scale of both tiers bit-exact, and the benchmarked decode (MFMA
    split-K, 128 splits per KV head, + combine) within 2e-3 / 1e-3 of the oracle over all 262,144 positions."""
    from kvtier.kvt import kvt_decode_attn
    bench, cache, q = headline
    k, v = bench.headline_inputs(layer)
    xk, xv = k.cpu(), v.cpu()
    del k, v
    f = ref.evict_closed_form(xk, xv, RING, 0, 64)
    hs = f["hot_start"]
    assert hs == bench.CTX - RING
    pages = cache.h_pages[0]
    rows = (torch.tensor(pages, dtype=torch.long)[torch.arange(hs) // PAGE] * PAGE + torch.arange(hs) % PAGE).to(dev)
    for name in ("k4", "ks4", "v4", "vs4"):
        assert torch.equal(getattr(cache, name)[layer][rows].cpu(), f[name]), name
    rr = f["ring_rows"].to(dev)
    for name in ("rk", "rks", "rv", "rvs"):
        assert torch.equal(getattr(cache, name)[layer][rr].cpu(), f[name]), name
    out = kvt_decode_attn(cache, layer, q[layer], impl="mfma").cpu()
    kk = torch.cat([ref.dequant4(f["k4"], f["ks4"]), ref.dequant8(f["rk"], f["rks"])])
    vv = torch.cat([ref.dequant4(f["v4"], f["vs4"]), ref.dequant8(f["rv"], f["rvs"])])
    close(out[0], ref.attention_rows(q[layer, 0].cpu(), kk, vv, SCALE))


# ----------------------------------------------------------------------------------------------- config 1
def test_config1_decode_with_append(kvt_pkg):
    """10,001-token context (ring 8,192 + 1,809 paged positions), then 1,000 steps of append-one-token + decode
    (1 layer, pages permuted from seed 5): the output of every 50th step (and the first) against the oracle over
    that step's state, and the final state (11,001 positions: codes, scales, page table) bit-exact."""
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    N0, STEPS = 10_001, 1000
    n_pages = (N0 + STEPS - RING) // PAGE + 2
    cache = PosTieredCache(1, H, D, n_pages=n_pages, ring_total=RING, max_seqs=1, max_pages=n_pages + 1,
                           device=dev, page_seed=5)
    cache.add_seq(RING)
    k, v, xk, xv = _dev_kv(N0 + STEPS, seed=101)
    gq = torch.Generator(device=dev).manual_seed(102)
    qs = (torch.randn(STEPS, 1, HQ, D, device=dev, generator=gq) / 16).to(torch.bfloat16)
    for a in range(0, N0, RING):
        n = min(RING, N0 - a)
        plan = cache.plan_append([0], [n])
        cache.append(0, plan, k[a:a + n], v[a:a + n])
        cache.commit(plan)
    outs = {}
    ws = {}
    for i in range(STEPS):
        p = N0 + i
        plan = cache.plan_append([0], [1])
        cache.append(0, plan, k[p:p + 1], v[p:p + 1])
        cache.commit(plan)
        o = kvt_decode_attn(cache, 0, qs[i], impl="mfma", workspace=ws)
        if i == 0 or i % 50 == 49:
            outs[i] = o.cpu()
    forms = Forms(xk, xv)
    for i, o in outs.items():
        L = N0 + i + 1
        kk, vv = forms.rows(L - RING, L)
        close(o[0], ref.attention_rows(qs[i, 0].cpu(), kk, vv, SCALE))
    L = N0 + STEPS
    want_pages = ref.PageAllocator(n_pages, seed=5).free[:math.ceil((L - RING) / PAGE)]
    assert cache.h_pages[0] == want_pages
    assert cache.page_table[0, :len(want_pages)].cpu().tolist() == want_pages
    assert int(cache.seq_lens[0]) == L
    _check_seq_codes(cache, 0, 0, forms, 0, L - RING, L, want_pages)


# ----------------------------------------------------------------------------------------------- config 3
def test_config3_chunked_prefill(kvt_pkg):
    """10,001-token prompt in chunks of 2,048 over 12 layers (ring 8,192; the last chunk evicts 1,809 positions
    into INT4 pages): per chunk the quantize-append of every layer, then causal prefill attention of every layer,
    the first chunk over its fresh bf16 K/V (the reference attends to those there), later chunks over the tiers
    holding the chunk itself.  Checked per layer and chunk: the first and last query and 64 seeded random ones
    against the oracle over the state after that chunk's append; after the prompt every code bit-exact."""
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    N, CH, L_ = 10_001, 2048, 12
    n_pages = (N - RING) // PAGE + 2
    cache = PosTieredCache(L_, H, D, n_pages=n_pages, ring_total=RING, max_seqs=1, max_pages=n_pages + 1,
                           device=dev, page_seed=7)
    cache.add_seq(RING)
    kv = [_dev_kv(N, seed=300 + layer) for layer in range(L_)]
    gq = torch.Generator(device=dev).manual_seed(399)
    qs = [(torch.randn(N, HQ, D, device=dev, generator=gq) / 16).to(torch.bfloat16) for _ in range(L_)]
    gpick = torch.Generator().manual_seed(398)
    picks, outs = {}, {}
    for a in range(0, N, CH):
        n = min(CH, N - a)
        plan = cache.plan_append([0], [n])
        for layer in range(L_):
            cache.append(layer, plan, kv[layer][0][a:a + n], kv[layer][1][a:a + n])
        cache.commit(plan)
        cu = torch.tensor([0, n], dtype=torch.int32, device=dev)
        sel = torch.cat([torch.tensor([0, n - 1]), torch.randperm(n, generator=gpick)[:64]])
        picks[a] = sel
        for layer in range(L_):
            src = dict(k_src=kv[layer][0][:n], v_src=kv[layer][1][:n]) if a == 0 else {}
            o = kvt_prefill_attn(cache, layer, qs[layer][a:a + n], cu, max_q=n, out_dtype=torch.float32, **src)
            outs[(a, layer)] = o[sel.to(dev)].cpu()
    for layer in range(L_):
        xk, xv = kv[layer][2], kv[layer][3]
        forms = Forms(xk, xv)
        qh = qs[layer].cpu()
        for a in range(0, N, CH):
            n = min(CH, N - a)
            L = a + n
            if a == 0:
                kk, vv = xk[:n], xv[:n]                       # fresh bf16 K/V of the first chunk
            else:
                kk, vv = forms.rows(max(0, L - RING), L)
            got = outs[(a, layer)]
            for i, j in enumerate(picks[a].tolist()):
                p = a + j
                close(got[i], ref.attention_rows(qh[p], kk[:p + 1], vv[:p + 1], SCALE))
        _check_seq_codes(cache, layer, 0, forms, 0, N - RING, N, cache.h_pages[0])
    assert cache.h_pages[0] == ref.PageAllocator(n_pages, seed=7).free[:math.ceil((N - RING) / PAGE)]


# ----------------------------------------------------------------------------------------------- config 4
def test_config4_ragged_shared_prefix(kvt_pkg):
    """8 sequences with seeded log-uniform lengths in [1,024, 65,536], 12 layers, rings of min(8,192, next power of two
    of the length); sequences 0 and 1 share a 4,096-position prefix through 64 common physical pages (paged-prefix
    reuse: written once by the INT4 writer, referenced by both page tables); 256 iterations of append-one-token +
    decode per sequence and layer.  The first and the last iteration's outputs of every layer against the oracle,
    then every code of every layer and sequence (and the shared pages) bit-exact."""
    from kvtier import sparse_attn
    from kvtier.kvt import PosTieredCache, kvt_decode_attn
    ITERS, SHARED, L_ = 256, 4096, 12
    gl = torch.Generator().manual_seed(4)
    lens = [int(math.exp(math.log(1024) + (math.log(65536) - math.log(1024)) * float(u)))
            for u in torch.rand(8, generator=gl)]
    lens[0], lens[1] = max(lens[0], SHARED + 1024), max(lens[1], SHARED + 1024)
    S = len(lens)
    total = [L + ITERS for L in lens]
    rings = [min(RING, 1 << (L - 1).bit_length()) for L in lens]
    n_pages = sum(max(0, T - r) // PAGE + 2 for T, r in zip(total, rings)) + SHARED // PAGE
    cache = PosTieredCache(L_, H, D, n_pages=n_pages, ring_total=sum(rings), max_seqs=S,
                           max_pages=max(total) // PAGE + 4, device=dev, page_seed=8)
    shared_pages = [cache.alloc.pop() for _ in range(SHARED // PAGE)]
    prow = (torch.tensor(shared_pages, device=dev)[:, None] * PAGE + torch.arange(PAGE, device=dev)).reshape(-1)
    ones = torch.ones(H, D, dtype=torch.float16, device=dev)
    pre = [_dev_kv(SHARED, seed=400 + layer) for layer in range(L_)]
    for layer in range(L_):
        sparse_attn.quant_store_kv_int4(pre[layer][0], pre[layer][1], prow, cache.k4[layer], cache.v4[layer],
                                        cache.ks4[layer], cache.vs4[layer], ones, ones)
    starts = [SHARED if s < 2 else 0 for s in range(S)]
    for s in range(S):
        cache.add_seq(rings[s], ring_start=starts[s], shared_pages=shared_pages if s < 2 else ())
    # per (sequence, layer) token streams: the positions each sequence appends (from its start), host copies kept
    seqkv = [[_dev_kv(total[s] - starts[s], seed=1000 * (s + 1) + layer) for layer in range(L_)] for s in range(S)]
    done = list(starts)
    while any(d < L for d, L in zip(done, lens)):
        act = [s for s in range(S) if done[s] < lens[s]]
        cnt = [min(rings[s], lens[s] - done[s]) for s in act]
        plan = cache.plan_append(act, cnt)
        for layer in range(L_):
            kk = torch.cat([seqkv[s][layer][0][done[s] - starts[s]:done[s] - starts[s] + c] for s, c in zip(act, cnt)])
            vv = torch.cat([seqkv[s][layer][1][done[s] - starts[s]:done[s] - starts[s] + c] for s, c in zip(act, cnt)])
            cache.append(layer, plan, kk, vv)
        cache.commit(plan)
        for s, c in zip(act, cnt):
            done[s] += c
    gq = torch.Generator(device=dev).manual_seed(499)
    qs = (torch.randn(ITERS, L_, S, HQ, D, device=dev, generator=gq) / 16).to(torch.bfloat16)
    ws = {}
    got = {}
    for it in range(ITERS):
        plan = cache.plan_append(list(range(S)), [1] * S)
        for layer in range(L_):
            idx = [lens[s] + it - starts[s] for s in range(S)]
            kk = torch.cat([seqkv[s][layer][0][idx[s]:idx[s] + 1] for s in range(S)])
            vv = torch.cat([seqkv[s][layer][1][idx[s]:idx[s] + 1] for s in range(S)])
            cache.append(layer, plan, kk, vv)
        cache.commit(plan)
        for layer in range(L_):
            o = kvt_decode_attn(cache, layer, qs[it, layer], impl="mfma", workspace=ws)
            if it in (0, ITERS - 1):
                got[(it, layer)] = o.cpu()
    for layer in range(L_):
        pre_forms = ref.quant4(pre[layer][2]), ref.quant4(pre[layer][3])
        pre_k = ref.dequant4(*pre_forms[0])
        pre_v = ref.dequant4(*pre_forms[1])
        for s in range(S):
            forms = Forms(seqkv[s][layer][2], seqkv[s][layer][3])
            for it in (0, ITERS - 1):
                L = lens[s] + it + 1
                hs = max(starts[s], L - rings[s])
                kk, vv = forms.rows(hs - starts[s], L - starts[s])
                if starts[s]:
                    kk, vv = torch.cat([pre_k, kk]), torch.cat([pre_v, vv])
                q = qs[it, layer, s].cpu()
                close(got[(it, layer)][s], ref.attention_rows(q, kk, vv, SCALE))
            L = total[s]
            hs = max(starts[s], L - rings[s])
            base = sum(rings[:s])
            _check_seq_codes(cache, layer, s, forms, starts[s], hs, L, cache.h_pages[s], base)
        srows = prow
        for name, want in (("k4", pre_forms[0][0]), ("ks4", pre_forms[0][1]), ("v4", pre_forms[1][0]),
                           ("vs4", pre_forms[1][1])):
            assert torch.equal(getattr(cache, name)[layer][srows].cpu(), want), name
    # page tables: the shared pages first for sequences 0 and 1, then pages in the allocator's order of requests
    assert cache.h_pages[0][:SHARED // PAGE] == shared_pages == cache.h_pages[1][:SHARED // PAGE]
    used = [p for s in range(S) for p in cache.h_pages[s][(SHARED // PAGE if s < 2 else 0):]]
    assert sorted(used + shared_pages) == sorted(ref.PageAllocator(n_pages, seed=8).free[:len(used) + len(shared_pages)])
    for s in range(S):
        n = len(cache.h_pages[s])
        assert cache.page_table[s, :n].cpu().tolist() == cache.h_pages[s]
