"""GPU parity of sparse_gqa_fwd_interface_paged (the reference's prefix-chunk attention read straight from a
quantized pool, patches/kv_paged_prefix.py:267-365) against the oracle: each query's selection by
ref.prefill_selected_positions (the first min(topk, j + kv_len - q_len + 1) index entries in [0, kv_len),
patches/kv_paged_prefix.py:199-229), its rows dequantized as the gathers write them, fp32 softmax attention
(ref.attention_rows, gemv/test_kv_paged_prefix.py:506-531), held to 2e-3 max-abs / 1e-3 mean-abs on the fp32
output; the bf16 output the reference returns is checked to be that fp32 output rounded to nearest even (its own
rounding, up to 2^-9 relative, exceeds 2e-3 at the |values| of about 2 these pools produce).  The cases follow the reference test's (gemv/test_kv_paged_prefix.py
make_case, :275-335): three requests with prefixes of 0 / 3,000 / 1,500 positions and chunks of 256 / 300 / 128, index
rows like the indexer's (sorted positions below the visible bound, valid first, -1 padding) with empty, chunk-only,
single-position and short rows; cu_q int64 as the backend builds it; req_to_token rows with junk beyond the length.
"""
import pytest
import torch

from kvt_testutil import close, pool_args, slot_pools, slot_rows
from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, D = 2, 256
TOPK = 2051


def _case(gen, prefix_lens, chunk_lens, slots, hq, per_head=False, topk=TOPK):
    batch = len(prefix_lens)
    seq_lens = [p + c for p, c in zip(prefix_lens, chunk_lens)]
    perm = torch.randperm(slots, generator=gen)
    r2t = torch.randint(0, slots, (batch + 2, max(seq_lens) + 64), dtype=torch.int32, generator=gen)
    req_idx = torch.randperm(batch + 2, generator=gen)[:batch].to(torch.int64)
    a = 0
    for b, L in enumerate(seq_lens):
        r2t[int(req_idx[b]), :L] = perm[a:a + L].sort().values.to(torch.int32)
        a += L
    total_q = sum(chunk_lens)
    shape = (total_q, H, topk) if per_head else (total_q, topk)
    idx = torch.full(shape, -1, dtype=torch.int32)
    singles = []
    row = 0
    for b in range(batch):
        for j in range(chunk_lens[b]):
            visible = prefix_lens[b] + j + 1
            for g in (range(H) if per_head else [None]):
                n = min(topk, visible)
                u = float(torch.rand(1, generator=gen))
                if u < 0.03:
                    continue                                             # empty: all -1
                if u < 0.06 and prefix_lens[b] > 0:
                    pos = torch.arange(prefix_lens[b], visible)[:n]      # current-chunk positions only
                elif u < 0.10:
                    pos = torch.randint(0, visible, (1,), generator=gen)
                    singles.append((row, b, g, int(pos)))
                else:
                    if u < 0.25:
                        n = int(torch.randint(0, n + 1, (1,), generator=gen))
                    pos = torch.randperm(visible, generator=gen)[:n].sort().values
                if g is None:
                    idx[row, :pos.numel()] = pos.to(torch.int32)
                else:
                    idx[row, g, :pos.numel()] = pos.to(torch.int32)
            row += 1
    q = (torch.randn(total_q, hq, D, generator=gen) / 4).to(torch.bfloat16)
    cu_q = torch.nn.functional.pad(torch.tensor(chunk_lens, dtype=torch.int32).cumsum(0), (1, 0))
    assert cu_q.dtype == torch.int64
    return dict(prefix_lens=prefix_lens, chunk_lens=chunk_lens, seq_lens=seq_lens, r2t=r2t, req_idx=req_idx, idx=idx,
                q=q, cu_q=cu_q, kv_lens=torch.tensor(seq_lens, dtype=torch.int32), singles=singles, topk=topk)


def _run(c, kind, p, R, idx=None, kv_lens=None, f32=False):
    """The operator's bf16 result (as the reference returns it), or with f32 the fp32 result through `out`."""
    from kvtier import sparse_attn as sa
    idx = c["idx"] if idx is None else idx
    kv_lens = c["kv_lens"] if kv_lens is None else kv_lens
    out = torch.empty(c["q"].shape, dtype=torch.float32, device=dev) if f32 else None
    return sa.sparse_gqa_fwd_interface_paged(
        c["q"].to(dev), idx.to(dev), c["cu_q"].to(dev), kv_lens.to(dev), c["r2t"].to(dev), c["req_idx"].to(dev),
        scale=D ** -0.5, max_q=max(c["chunk_lens"]), out=out, **pool_args(kind, p, R, dev)).cpu()


def _bf16_of(got32, got16):
    """The bf16 result is the fp32 result rounded to nearest even, bit for bit (NaN rows stay NaN)."""
    nan = torch.isnan(got32)
    assert torch.equal(nan, torch.isnan(got16.float()))
    assert torch.equal(got32[~nan].to(torch.bfloat16).view(torch.int16), got16[~nan].view(torch.int16))


def _oracle(c, kind, p, R, g8, idx=None, kv_lens=None):
    """Whole pool dequantized once by the oracle, then per query: its selection and fp32 attention per KV head."""
    idx = c["idx"] if idx is None else idx
    kv_lens = c["kv_lens"] if kv_lens is None else kv_lens
    n_slots = p["k4"].shape[0]
    kk_all, vv_all = slot_rows(kind, p, torch.arange(n_slots), R, g8)
    hq = c["q"].shape[1]
    gs = hq // H
    out = torch.empty(c["q"].shape, dtype=torch.float32)
    row = 0
    for b, ql in enumerate(c["chunk_lens"]):
        L = int(kv_lens[b])
        slot_row = c["r2t"][int(c["req_idx"][b])]
        for j in range(ql):
            visible = j + L - ql + 1
            for h in range(H):
                irow = idx[row, h] if idx.dim() == 3 else idx[row]
                pos = ref.prefill_selected_positions(irow, visible, L, c["topk"])
                sl = slot_row[pos].long()
                o = ref.attention_rows(c["q"][row, h * gs:(h + 1) * gs], kk_all[sl][:, h:h + 1], vv_all[sl][:, h:h + 1],
                                       D ** -0.5)
                out[row, h * gs:(h + 1) * gs] = o
            row += 1
    return out


@pytest.mark.parametrize("kind,g8,hq", [("tiered", 64, 16), ("tiered", 256, 16), ("int4", 64, 16), ("int8", 64, 16),
                                        ("int8", 256, 16), ("tiered", 64, 24)])
def test_paged_prefill_matches_oracle(kvt_pkg, kind, g8, hq):
    gen = torch.Generator().manual_seed(41)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, g8, gen)
    c = _case(gen, [0, 3000, 1500], [256, 300, 128], slots, hq)
    got = _run(c, kind, p, R, f32=True)
    exp = _oracle(c, kind, p, R, g8)
    assert torch.isnan(exp).any()                      # empty rows are part of the case
    close(got, exp)
    got16 = _run(c, kind, p, R)
    assert got16.dtype == torch.bfloat16 and got16.shape == c["q"].shape
    _bf16_of(got, got16)


def test_paged_prefill_single_position_rows_exact(kvt_pkg):
    """A row with exactly one attended position returns that position's gathered bf16 V row, bit for bit
    (gemv/test_kv_paged_prefix.py:436-457)."""
    gen = torch.Generator().manual_seed(42)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, 64, gen)
    c = _case(gen, [0, 3000, 1500], [256, 300, 128], slots, 16)
    assert len(c["singles"]) >= 8
    got = _run(c, "tiered", p, R)
    for row, b, _, pos in c["singles"]:
        slot = c["r2t"][int(c["req_idx"][b]), pos].reshape(1)
        _, vv = slot_rows("tiered", p, slot, R, 64)
        for h in range(H):
            assert torch.equal(got[row, 8 * h:8 * h + 8], vv[0, h].expand(8, D)), (row, h)


def test_paged_prefill_dirty_indices_ignored(kvt_pkg):
    """Entries >= kv_len inside the read range are ignored: the output equals that of the same rows with -1 there,
    bit for bit (gemv/test_kv_paged_prefix.py:477-503); a context shorter than its chunk (no visible position)
    gives NaN rows."""
    gen = torch.Generator().manual_seed(43)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, 64, gen)
    c = _case(gen, [0, 3000, 1500], [256, 300, 128], slots, 16)
    dirty, clean = c["idx"].clone(), c["idx"].clone()
    rows = torch.randperm(dirty.shape[0], generator=gen)[:64]
    for r in rows.tolist():
        b = int((c["cu_q"] <= r).sum()) - 1
        j = r - int(c["cu_q"][b])
        n = min(TOPK, c["prefix_lens"][b] + j + 1)
        cols = torch.randperm(n, generator=gen)[:max(1, n // 50)]
        dirty[r, cols] = (c["seq_lens"][b] + torch.randint(0, 100, (cols.numel(),), generator=gen)).to(torch.int32)
        clean[r, cols] = -1
    for kind in ("tiered", "int4", "int8"):
        assert torch.equal(_run(c, kind, p, R, idx=dirty).view(torch.int16), _run(c, kind, p, R, idx=clean).view(torch.int16))
    close(_run(c, "tiered", p, R, idx=dirty, f32=True), _oracle(c, "tiered", p, R, 64, idx=clean))
    short = c["kv_lens"].clone()
    short[2] = 100                                       # 128-query chunk over a 100-position context
    got = _run(c, "tiered", p, R, kv_lens=short, f32=True)
    exp = _oracle(c, "tiered", p, R, 64, kv_lens=short)
    a = int(c["cu_q"][2])
    assert torch.isnan(got[a:a + 28]).all() and torch.isnan(exp[a:a + 28]).all()
    close(got, exp)


def test_paged_prefill_row_limit_is_visible(kvt_pkg):
    """A query reads exactly the first min(topk, visible) entries of its index row (the reference test's oracle,
    gemv/test_kv_paged_prefix.py:515-517).  The reference kernel reads on to the next multiple of its 16-column tile
    (row_limit = min(topk, roundup16(row_topk)), patches/kv_paged_prefix.py:201-202) and would attend valid positions
    placed there; an indexer row holds -1 at those columns, so the two agree on the reference's inputs.  Pinned here:
    valid positions (< kv_len, beyond the query's own) planted at columns visible .. roundup16(visible) - 1 change
    nothing, bit for bit.  Parity with the reference kernel on such rows stays unpinned (its rows never have them)."""
    gen = torch.Generator().manual_seed(45)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, 64, gen)
    c = _case(gen, [0, 3000, 1500], [256, 300, 128], slots, 16)
    planted, clean = c["idx"].clone(), c["idx"].clone()
    n_planted = 0
    for r in range(planted.shape[0]):
        b = int((c["cu_q"] <= r).sum()) - 1
        j = r - int(c["cu_q"][b])
        vis = c["prefix_lens"][b] + j + 1
        n = min(TOPK, vis)
        lim = min(TOPK, -(-n // 16) * 16)
        if lim > n:
            planted[r, n:lim] = torch.randint(0, c["seq_lens"][b], (lim - n,), generator=gen).to(torch.int32)
            clean[r, n:lim] = -1
            n_planted += lim - n
    assert n_planted > 1000
    for kind in ("tiered", "int4", "int8"):
        assert torch.equal(_run(c, kind, p, R, idx=planted).view(torch.int16),
                           _run(c, kind, p, R, idx=clean).view(torch.int16)), kind


@pytest.mark.parametrize("kind", ["tiered", "int8"])
def test_paged_prefill_long_selection(kvt_pkg, kind):
    """Index rows of up to 5,000 entries over a 6,000-position prefix: a query's selection takes two passes of the
    block's 4,096-entry column table (each pass runs the ring tiles, then the INT4 tiles); empty, single-position and
    short rows among them."""
    gen = torch.Generator().manual_seed(47)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, 64, gen)
    c = _case(gen, [6000], [40], slots, 16, topk=5000)
    assert max(int((c["idx"][j] >= 0).sum()) for j in range(40)) > 4096
    close(_run(c, kind, p, R, f32=True), _oracle(c, kind, p, R, 64))


def test_paged_prefill_per_head_indices(kvt_pkg):
    """3-d indices [total_q, H, topk]: each KV head attends its own selection; topk 700 (< the prefix)."""
    gen = torch.Generator().manual_seed(44)
    slots, R = 8192, 1024
    p = slot_pools(slots, R, 64, gen)
    c = _case(gen, [0, 3000, 1500], [96, 120, 64], slots, 16, per_head=True, topk=700)
    close(_run(c, "tiered", p, R, f32=True), _oracle(c, "tiered", p, R, 64))


def test_paged_prefill_reference_timing_shape(kvt_pkg):
    """The shape of the reference's published timing case (gemv/test_kv_paged_prefix.py:539-546): one request with a
    60,000-position prefix and a 1,024-query chunk, 1 KV head x 12 q heads, tiered pool whose ring of 8,192 rows is
    owned by the newest 8,192 slots (position p in slot p), topk 2,051 with indexer-like rows.  Sampled queries (the
    first, the last, spread between, single-position and empty rows) against the oracle."""
    gen = torch.Generator().manual_seed(61)
    prefix, chunk, R, hq = 60_000, 1024, 8192, 12
    ctx = prefix + chunk
    p = slot_pools(ctx, R, 64, gen, H=1)
    rows = torch.arange(R)
    p["owner"] = torch.where(rows < ctx % R, rows + (ctx // R) * R, rows + (ctx // R - 1) * R).to(torch.int32)
    c = _case(gen, [prefix], [chunk], ctx, hq)
    got = _run(c, "tiered", p, R, f32=True)
    empty = [j for j in range(chunk) if int(c["idx"][j, 0]) < 0][:2]
    singles = [r for r, _, _, _ in c["singles"]][:2]
    sample = sorted(set([0, 1, 2, chunk - 2, chunk - 1] + list(range(97, chunk, 101)) + empty + singles))
    slot_row = c["r2t"][int(c["req_idx"][0])]
    exp = torch.empty(len(sample), hq, D)
    for i, j in enumerate(sample):
        pos = ref.prefill_selected_positions(c["idx"][j], prefix + j + 1, ctx, TOPK)
        kk, vv = slot_rows("tiered", p, slot_row[pos].long(), R, 64)
        exp[i] = ref.attention_rows(c["q"][j], kk, vv, D ** -0.5)
    assert empty and singles
    close(got[sample], exp)
