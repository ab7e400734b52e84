"""GPU parity of the fused top-k sparse decode (qwen_sparse_decode_attn) against the oracle: the selected positions
dequantized exactly as the compact gather writes them (oracle/ref.py dequant4 / dequant8 / dequant_slots_tiered),
then fp32 softmax attention (ref.attention_rows, the form of gemv/test_kv_paged_prefix.py:520-528), within
2e-3 max-abs / 1e-3 mean-abs.  Pools hold seeded random codes and scales; about half of the tiered slots own their
ring row.  The reference path this replaces (compact gather + FlashAttention-2) attends the rows
[cu_k[b], cu_k[b+1]) of its scratch: with the valid positions first, those are the columns this kernel attends.
"""
import math

import numpy as np
import pytest
import torch

from oracle import ref

pytestmark = pytest.mark.gpu
dev = "cuda"
H, HQ, D = 2, 16, 256


def _pools(slots, R, g8, gen):
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    v4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=gen)
    ks4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=gen)).half()
    vs4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=gen)).half()
    rk = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, generator=gen)
    rv = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, generator=gen)
    rks = (0.002 + 0.02 * torch.rand(R, H, D // g8, generator=gen)).half()
    rvs = (0.002 + 0.02 * torch.rand(R, H, D // g8, generator=gen)).half()
    k8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=gen)
    v8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=gen)
    ks8 = (0.002 + 0.02 * torch.rand(slots, H, D // g8, generator=gen)).half()
    vs8 = (0.002 + 0.02 * torch.rand(slots, H, D // g8, generator=gen)).half()
    # owner: ring row r belongs to one slot of its class r mod R (or to none)
    owner = torch.full((R,), -1, dtype=torch.int32)
    for r in range(R):
        if torch.rand(1, generator=gen).item() < 0.8:
            owner[r] = r + R * int(torch.randint(0, slots // R, (1,), generator=gen))
    sm_k = (0.5 + torch.rand(H, D, generator=gen)).half()
    sm_v = (0.5 + torch.rand(H, D, generator=gen)).half()
    return dict(k4=k4, v4=v4, ks4=ks4, vs4=vs4, rk=rk, rv=rv, rks=rks, rvs=rvs, k8=k8, v8=v8, ks8=ks8, vs8=vs8,
                owner=owner, sm_k=sm_k, sm_v=sm_v)


def _rows(kind, p, slots, R, g8):
    if kind == "tiered":
        return ref.dequant_slots_tiered(slots, p["k4"], p["v4"], p["ks4"], p["vs4"], p["rk"], p["rv"], p["rks"],
                                        p["rvs"], p["owner"], R - 1, p["sm_k"], p["sm_v"], group8=g8)
    sl = slots.long()
    if kind == "int4":
        return ref.dequant4(p["k4"][sl], p["ks4"][sl], p["sm_k"]), ref.dequant4(p["v4"][sl], p["vs4"][sl], p["sm_v"])
    return (ref.dequant8(p["k8"][sl], p["ks8"][sl], p["sm_k"], g8),
            ref.dequant8(p["v8"][sl], p["vs8"][sl], p["sm_v"], g8))


def _call(kind, p, q, r2t, req_idx, idx, seq_lens, cu_k, batch, topk, R, out=None, splits=None):
    from kvtier import sparse_attn as sa
    d = {k: v.to(dev) for k, v in p.items()}
    common = dict(scale=D ** -0.5, out=out, splits=splits)
    if kind == "tiered":
        return sa.qwen_sparse_decode_attn(q.to(dev), d["k4"], d["v4"], r2t.to(dev), req_idx.to(dev), idx.to(dev),
                                          seq_lens.to(dev), cu_k.to(dev), batch, topk, d["ks4"], d["vs4"],
                                          d["sm_k"], d["sm_v"], 4, d["rk"], d["rv"], d["rks"], d["rvs"],
                                          d["owner"], R - 1, **common)
    if kind == "int4":
        return sa.qwen_sparse_decode_attn(q.to(dev), d["k4"], d["v4"], r2t.to(dev), req_idx.to(dev), idx.to(dev),
                                          seq_lens.to(dev), cu_k.to(dev), batch, topk, d["ks4"], d["vs4"],
                                          d["sm_k"], d["sm_v"], 4, **common)
    return sa.qwen_sparse_decode_attn(q.to(dev), d["k8"], d["v8"], r2t.to(dev), req_idx.to(dev), idx.to(dev),
                                      seq_lens.to(dev), cu_k.to(dev), batch, topk, d["ks8"], d["vs8"], d["sm_k"],
                                      d["sm_v"], 8, **common)


def _case(gen, seq_lens, topk, slots, n_reqs=6):
    """req_to_token rows (random slots), requests on shuffled rows, indices: distinct valid positions first,
    then -1 padding (and a few positions >= seq_len past the valid count, which nothing reads)."""
    batch = len(seq_lens)
    max_ctx = max(seq_lens) + 8
    r2t = torch.randint(0, slots, (n_reqs, max_ctx), dtype=torch.int32, generator=gen)
    req_idx = torch.randperm(n_reqs, generator=gen)[:batch].to(torch.int64)
    idx = torch.full((batch, topk + 5), -1, dtype=torch.int32)
    for b, L in enumerate(seq_lens):
        n = min(L, topk)
        idx[b, :n] = torch.randperm(L, generator=gen)[:n].to(torch.int32)
        if n + 2 < topk:
            idx[b, n + 1] = L + 3
    sl = torch.tensor(seq_lens, dtype=torch.int32)
    cu_k = ref.cu_seqlens_valid(sl, idx, topk)
    return r2t, req_idx, idx, sl, cu_k


def _oracle(kind, p, q, r2t, req_idx, idx, seq_lens, cu_k, topk, R, g8, skip_invalid=False):
    outs = []
    for b in range(q.shape[0]):
        L = int(seq_lens[b])
        vcount = int(cu_k[b + 1]) - int(cu_k[b])
        cols = [c for c in range(min(vcount, topk)) if 0 <= int(idx[b, c]) < L]
        if not skip_invalid:
            assert len(cols) == vcount      # valid positions first: the scratch rows the reference attends
        pos = torch.tensor([int(idx[b, c]) for c in cols], dtype=torch.long)
        slots = r2t[int(req_idx[b]), pos] if len(cols) else torch.zeros(0, dtype=torch.int32)
        kk, vv = _rows(kind, p, slots, R, g8)
        outs.append(ref.attention_rows(q[b], kk, vv, D ** -0.5))
    return torch.stack(outs)


def _close(got, exp):
    fin = torch.isfinite(exp)
    assert torch.equal(fin, torch.isfinite(got))
    err = (got[fin] - exp[fin]).abs()
    assert float(err.max()) <= 2e-3 and float(err.mean()) <= 1e-3, (float(err.max()), float(err.mean()))


@pytest.mark.parametrize("kind,g8", [("tiered", 64), ("tiered", 256), ("int4", 64), ("int8", 64), ("int8", 256)])
def test_sparse_decode_matches_oracle(kvt_pkg, kind, g8):
    """3 requests (seq_len 3000 / 700 / 9), topk 2051 (not a multiple of 16): every kind of pool."""
    gen = torch.Generator().manual_seed(31)
    slots, R = 4096, 64
    p = _pools(slots, R, g8, gen)
    r2t, req_idx, idx, sl, cu_k = _case(gen, [3000, 700, 9], 2051, slots)
    q = (torch.randn(3, HQ, D, generator=gen) / 4).to(torch.bfloat16)
    got = _call(kind, p, q, r2t, req_idx, idx, sl, cu_k, 3, 2051, R).cpu()
    _close(got, _oracle(kind, p, q, r2t, req_idx, idx, sl, cu_k, 2051, R, g8))


@pytest.mark.parametrize("kind,g8,splits", [("tiered", 64, 1), ("tiered", 256, 3), ("int4", 64, 11),
                                            ("int8", 64, 3)])
def test_sparse_decode_tiles_per_wavefront(kvt_pkg, kind, g8, splits):
    """The 2,051 selected columns of the previous case in 1 / 3 / 11 splits: each wavefront loops over 33 / 11 / 3
    tiles, resolving the next tile's positions, slots and owners beside the current one (the launch-size rule takes
    this path for long selections)."""
    gen = torch.Generator().manual_seed(31)
    slots, R = 4096, 64
    p = _pools(slots, R, g8, gen)
    r2t, req_idx, idx, sl, cu_k = _case(gen, [3000, 700, 9], 2051, slots)
    q = (torch.randn(3, HQ, D, generator=gen) / 4).to(torch.bfloat16)
    got = _call(kind, p, q, r2t, req_idx, idx, sl, cu_k, 3, 2051, R, splits=splits).cpu()
    _close(got, _oracle(kind, p, q, r2t, req_idx, idx, sl, cu_k, 2051, R, g8))


def test_sparse_decode_empty_request_and_bf16_out(kvt_pkg):
    """A request with no valid column comes out NaN (0/0, gemv/test_kv_paged_prefix.py:524-526); bf16 output is the
    rounded fp32 result; a strided q (batch stride 2 Hq D) is read in place."""
    gen = torch.Generator().manual_seed(32)
    slots, R = 2048, 64
    p = _pools(slots, R, 64, gen)
    r2t, req_idx, idx, sl, cu_k = _case(gen, [500, 1, 300], 160, slots)
    idx[1, :] = -1
    cu_k = ref.cu_seqlens_valid(sl, idx, 160)
    qw = (torch.randn(3, 2 * HQ, D, generator=gen) / 4).to(torch.bfloat16)
    q = qw[:, :HQ]
    exp = _oracle("tiered", p, q, r2t, req_idx, idx, sl, cu_k, 160, R, 64)
    assert torch.isnan(exp[1]).all()
    got = _call("tiered", p, qw.to(dev)[:, :HQ], r2t, req_idx, idx, sl, cu_k, 3, 160, R).cpu()
    _close(got, exp)
    out = torch.empty(3, HQ, D, dtype=torch.bfloat16, device=dev)
    got16 = _call("tiered", p, q, r2t, req_idx, idx, sl, cu_k, 3, 160, R, out=out).cpu()
    assert torch.isnan(got16[1].float()).all()
    assert torch.equal(got16[[0, 2]], got[[0, 2]].to(torch.bfloat16))


def test_sparse_decode_invalid_columns_inside_the_count(kvt_pkg):
    """Out-of-range and negative positions among the first cu_k columns are skipped (the reference's scratch holds
    stale rows there); columns past the count are not attended even when valid."""
    gen = torch.Generator().manual_seed(33)
    slots, R = 2048, 64
    p = _pools(slots, R, 64, gen)
    r2t, req_idx, idx, sl, _ = _case(gen, [800, 400], 96, slots)
    idx[0, 5] = -1
    idx[0, 40] = 900
    idx[1, 17] = 400
    cu_k = ref.cu_seqlens_valid(sl, idx, 96)
    q = (torch.randn(2, HQ, D, generator=gen) / 4).to(torch.bfloat16)
    got = _call("tiered", p, q, r2t, req_idx, idx, sl, cu_k, 2, 96, R).cpu()
    _close(got, _oracle("tiered", p, q, r2t, req_idx, idx, sl, cu_k, 96, R, 64, skip_invalid=True))


def test_sparse_decode_gqa12(kvt_pkg):
    """24 q heads over 2 KV heads (GQA 12, the served model's shape, tools/probe_trtllm_sm120.py:4): the 16-row
    accumulator tile holds 12 heads and the block merges them in two passes of 8."""
    gen = torch.Generator().manual_seed(34)
    slots, R = 4096, 64
    p = _pools(slots, R, 64, gen)
    r2t, req_idx, idx, sl, cu_k = _case(gen, [3000, 700, 9], 2051, slots)
    q = (torch.randn(3, 24, D, generator=gen) / 4).to(torch.bfloat16)
    for kind in ("tiered", "int8"):
        got = _call(kind, p, q, r2t, req_idx, idx, sl, cu_k, 3, 2051, R).cpu()
        _close(got, _oracle(kind, p, q, r2t, req_idx, idx, sl, cu_k, 2051, R, 64))


def test_sparse_decode_merge_in_launch_against_combine(kvt_pkg):
    """The split merge inside the launch (the last block of each (request, KV head) merges, counters left at zero)
    against the separate combine launch, on one shared workspace: 3 requests, then 2 other requests with another
    split count, then the first case again, fp32 and bf16 outputs; both within the oracle bound, and within 1e-5 of
    each other (the same partials, merged in the same split order).  The default (merge="auto") takes the in-launch
    merge for at most 8 splits: bit-identical to merge="launch" there."""
    from kvtier import sparse_attn as sa
    gen = torch.Generator().manual_seed(35)
    slots, R = 4096, 64
    p = _pools(slots, R, 64, gen)
    d = {k: v.to(dev) for k, v in p.items()}
    cases = []
    for lens, topk in (([3000, 700, 9], 2051), ([1500, 2600], 1200)):
        r2t, req_idx, idx, sl, cu_k = _case(gen, lens, topk, slots)
        q = (torch.randn(len(lens), 24, D, generator=gen) / 4).to(torch.bfloat16)
        cases.append((r2t, req_idx, idx, sl, cu_k, q, topk))
    ws = {}
    for ci, splits in ((0, None), (1, 5), (0, 7), (1, 1)):
        r2t, req_idx, idx, sl, cu_k, q, topk = cases[ci]
        batch = q.shape[0]
        args = (q.to(dev), d["k4"], d["v4"], r2t.to(dev), req_idx.to(dev), idx.to(dev), sl.to(dev), cu_k.to(dev),
                batch, topk, d["ks4"], d["vs4"], d["sm_k"], d["sm_v"], 4, d["rk"], d["rv"], d["rks"], d["rvs"],
                d["owner"], R - 1)
        fused = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=splits, merge="launch").cpu()
        assert int(ws["sparse_ctr"].abs().sum()) == 0
        sep = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=splits, merge="combine").cpu()
        _close(fused, _oracle("tiered", p, q, r2t, req_idx, idx, sl, cu_k, topk, R, 64))
        assert float((fused - sep).abs().max()) <= 1e-5
        o16 = torch.empty(batch, 24, D, dtype=torch.bfloat16, device=dev)
        f16 = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=splits, out=o16,
                                         merge="launch").cpu()
        assert float((f16.float() - fused).abs().max()) <= 2 ** -8 * float(fused.abs().max())
        auto = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=splits).cpu()
        assert torch.equal(auto, fused if (splits or 33) <= 8 else sep)
    with pytest.raises(ValueError):
        sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, merge="fold")
    # output rows the in-launch merge cannot write (batch stride not a multiple of 8): the default takes the combine
    # launch, an explicit merge="launch" is refused
    batch = args[8]
    wide = torch.full((batch, 24 * D + 4), float("nan"), dtype=torch.float32, device=dev)
    odd = wide[:, :24 * D].view(batch, 24, D)
    got = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=1, out=odd).cpu()
    ref_ = sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=1, merge="combine").cpu()
    assert torch.equal(got, ref_)
    with pytest.raises(AssertionError):
        sa.qwen_sparse_decode_attn(*args, scale=D ** -0.5, workspace=ws, splits=1, out=odd, merge="launch")
