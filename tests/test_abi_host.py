"""CPU-side checks: the C-ABI library loads and exports every entry point declared in include/kvtier.h, the ctypes
signatures cover exactly those, and the host logic (guards, env parsing, page allocator) behaves like the
reference's (patches/kv_tiers.py:91-100, :176-220; gemv/test_kv_tiers.py:463-473, :539-551).  No kernel runs."""
import ctypes
import os

import pytest
import torch


def test_library_exports_header_symbols(kvt_pkg):
    lib = kvt_pkg._lib
    declared = lib.header_symbols()
    assert declared, "no entry points parsed from include/kvtier.h"
    handle = ctypes.CDLL(lib.LIB_PATH)
    for name in declared:
        assert hasattr(handle, name), f"libkvtier.so lacks {name}"
    assert sorted(lib.SIGNATURES) == declared, "ctypes signatures out of sync with include/kvtier.h"
    lib.lib()   # binding with argtypes succeeds


def test_prefill_work_bytes(kvt_pkg):
    """Workspace of a spread prefill launch: a counter area of 16 KB (one 4-byte counter for each of the at most
    4,096 (sequence, KV head, query tile of 128 rows) items, the same for every call, so one call's slots never
    overlap another call's counters), then one 132,096-byte slot (O of 128 rows x 256 dims, m and l of 128 rows,
    fp32) per query tile and per block beyond the first."""
    lib = kvt_pkg._lib
    need = ctypes.c_int64(-1)

    def work(*args):
        lib.call("kvt_prefill_work_bytes", *args, ctypes.byref(need))
        return need.value

    slot = (128 * 256 + 128 * 2) * 4
    assert slot == 132_096
    assert work(1, 2, 16, 2048, 0) == 0                        # one block per query tile: no workspace
    assert work(1, 2, 16, 2048, 256) == 16384 + (256 + 255) * slot
    # 24 / 2 heads: a wavefront's 16 rows hold one query (12 rows), so a tile is 8 queries: 13 tiles of 100
    assert work(3, 2, 24, 100, 7) == 16384 + (6 * 13 + 6) * slot
    assert work(2, 2, 16, 0, 3) == 0
    for bad in ((1, 2, 16, 64, -1), (1, 2, 15, 64, 2), (1, 1, 32, 64, 2)):
        with pytest.raises(ValueError):
            work(*bad)
    with pytest.raises(ValueError):   # more than 4,096 query tiles
        work(17, 2, 16, 2048, 256)


def test_ring_slots_from_env(kvt_pkg, monkeypatch):
    from kvtier.tiered_kv_pool import ring_slots_from_env
    for bad in ("0", "-8", "100", "abc"):
        monkeypatch.setenv("SGLANG_KV_TIERS_W", bad)
        with pytest.raises(ValueError):
            ring_slots_from_env()
    monkeypatch.delenv("SGLANG_KV_TIERS_W", raising=False)
    assert ring_slots_from_env() == 8192
    monkeypatch.setenv("SGLANG_KV_TIERS_W", "64")
    assert ring_slots_from_env() == 64


def test_pool_layout_and_guards_cpu(kvt_pkg, monkeypatch):
    """Shapes, dtypes, byte accounting and the write guards of the tiered pool (allocated on the CPU here: the
    guards raise before any kernel would be called)."""
    from kvtier.tiered_kv_pool import MHATokenToKVPoolInt4, MHATokenToKVPoolTiered
    monkeypatch.setenv("SGLANG_KV_TIERS_W", "64")
    size, page, H, D, R = 1024, 64, 2, 256, 64
    mk = dict(size=size, page_size=page, dtype=torch.uint8, head_num=H, head_dim=D, layer_num=2, device="cpu")
    ref_pool = MHATokenToKVPoolInt4(**mk)
    ref_kb, ref_vb = ref_pool.get_kv_size_bytes()
    rows = size + page
    assert ref_kb == ref_vb == 2 * rows * (H * D // 2 + H * 8 * 2)
    pool = MHATokenToKVPoolTiered(**mk)
    assert pool.kv_tiered and pool.kv_bits == 4 and pool.ring_slots == R and pool.ring_mask == R - 1
    assert pool.ring_k[0].shape == (R, H, D) and pool.ring_k[0].dtype == torch.int8
    assert pool.ring_ks[1].shape == (R, H, 4) and pool.ring_ks[1].dtype == torch.float16
    assert pool.ring_owner.shape == (R,) and (pool.ring_owner == -1).all()
    assert pool.k_buffer[0].shape == (rows, H, D // 2) and pool.k_scale_buffer[0].shape == (rows, H, 8)
    kb, vb = pool.get_kv_size_bytes()
    ring_k_bytes = 2 * R * H * (D + 4 * 2)
    assert kb == ref_kb + ring_k_bytes + R * 4 and vb == ref_vb + ring_k_bytes
    x = torch.zeros(R + 1, H, D, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pool.set_kv_buffer(None, torch.arange(R + 1), x, x, layer_id_override=0)
    loc = torch.arange(4)
    for bad in (dict(k_scale=0.5), dict(v_scale=torch.ones(1)), dict(dcp_kv_mask=torch.ones(4))):
        with pytest.raises((ValueError, NotImplementedError)):
            pool.set_kv_buffer(None, loc, x[:4], x[:4], layer_id_override=0, **bad)
    with pytest.raises(AssertionError):           # no CPU fallback: host tensors are refused
        pool.set_kv_buffer(None, loc, x[:4], x[:4], layer_id_override=0)
    pool.ring_owner.fill_(3)
    pool.lazy_release()
    assert (pool.ring_owner == -1).all()
    for fn in (lambda: pool.get_cpu_copy(loc), lambda: pool.load_cpu_copy(None, loc),
               lambda: pool.set_kv_buffer_prefix_valid()):
        with pytest.raises(NotImplementedError):
            fn()
    pool._clear_buffers()
    assert pool.ring_k is None and pool.ring_owner is None


def test_wrapper_contracts_cpu(kvt_pkg):
    """Shape contracts raise AssertionError before any launch (patches/kv_tiers.py:396-413, :622-636)."""
    from kvtier import sparse_attn as sa
    H, D, R = 2, 256, 64
    k = torch.zeros(R + 1, H, D, dtype=torch.bfloat16)
    k4 = torch.zeros(4096, H, D // 2, dtype=torch.uint8)
    ks = torch.zeros(4096, H, 8, dtype=torch.float16)
    rk = torch.zeros(R, H, D, dtype=torch.int8)
    rks = torch.zeros(R, H, 4, dtype=torch.float16)
    owner = torch.full((R,), -1, dtype=torch.int32)
    ones = torch.ones(H, D, dtype=torch.float16)
    with pytest.raises(AssertionError):           # N > R
        sa.quant_store_kv_tiered(k, k, torch.arange(R + 1), k4, k4, ks, ks, rk, rk, rks, rks, owner, ones, ones, R - 1)
    with pytest.raises(AssertionError):           # ring_mask + 1 not a power of two
        sa.quant_store_kv_tiered(k[:4], k[:4], torch.arange(4), k4, k4, ks, ks, rk, rk, rks, rks, owner, ones, ones, 62)
    with pytest.raises(AssertionError):           # missing ring args on the tiered prefix gather
        sa.qwen_sparse_prefix_gather_dequant_tiered(k4, k4, ks, ks, ones, ones, torch.zeros(1, 8, dtype=torch.int32),
                                                    torch.zeros(1, dtype=torch.int64), torch.ones(1, dtype=torch.int32),
                                                    torch.tensor([0, 1], dtype=torch.int32),
                                                    torch.zeros(2, H, D, dtype=torch.bfloat16),
                                                    torch.zeros(2, H, D, dtype=torch.bfloat16), 1, 1)
    with pytest.raises(AssertionError):           # packed-width scratch rejected (gemv/test_kv_int4.py:216-224)
        sa.qwen_sparse_kv_extraction_compact_triton(
            k4, k4, torch.zeros(1, 8, dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
            torch.zeros(1, 4, dtype=torch.int32), torch.ones(1, dtype=torch.int32), torch.tensor([0, 1], dtype=torch.int32),
            torch.zeros(4, H, D // 2, dtype=torch.bfloat16), torch.zeros(4, H, D // 2, dtype=torch.bfloat16), 1, 4,
            k_scale=ks, v_scale=ks, sm_k=ones, sm_v=ones, kv_bits=4)


def test_page_allocator_order(kvt_pkg):
    """The page allocator hands out every page exactly once, in the order of torch.randperm under the seed (the
    permutation the configurations ask for), and refuses a pop from an empty pool."""
    from kvtier.kvt import PageAllocator
    a = PageAllocator(100, seed=3)
    got = [a.pop() for _ in range(100)]
    assert sorted(got) == list(range(100)) and got != list(range(100))
    assert got == torch.randperm(100, generator=torch.Generator().manual_seed(3)).tolist()
    with pytest.raises(RuntimeError):
        a.pop()


def test_ragged_split_counts(kvt_pkg):
    """Split counts of a ragged decode batch: never more blocks than the budget (a block past one per CU runs as a
    second wave), at least one per sequence, at most one per min_pos positions, and in proportion to each sequence's
    cost (a ring position weighs 7 / 4 of a paged one), so the per-block cost spread stays small."""
    from kvtier.kvt import HOT_COST4, _split_counts_mfma
    lens = [10498, 10474, 1497, 2452, 1055, 1204, 63627, 45661]           # the ragged 8-sequence workload
    rings = [min(8192, 1 << (L - 1).bit_length()) for L in lens]
    hot = [min(L, r) for L, r in zip(lens, rings)]
    for items, blocks, min_pos in ((1, 256, 64), (2, 256, 256), (1, 100, 64)):
        c = _split_counts_mfma(lens, items, blocks=blocks, min_pos=min_pos, hot=hot)
        assert sum(c) <= blocks // items and all(x >= 1 for x in c)
        assert all(x <= -(-L // min_pos) for x, L in zip(c, lens))
        cost = [(4 * (L - h) + HOT_COST4 * h) / x for L, h, x in zip(lens, hot, c)]
        big = [y for y, x in zip(cost, c) if x >= 8]                         # rounding dominates below that
        assert max(big) / min(big) < 1.3, (c, cost)
    # length-proportional rounding once gave 257 blocks here; the budget holds for any mix
    assert sum(_split_counts_mfma(lens, 1, min_pos=64)) <= 256
    assert _split_counts_mfma([5] * 300, 1, min_pos=64) == [1] * 300       # more sequences than blocks: one each
    assert _split_counts_mfma([100, 100_000], 1, min_pos=64) == [1, 255]
    assert _split_counts_mfma([0, 0], 1) == [1, 1]


def test_kv_buffer_descs(kvt_pkg):
    """Descriptor names and row sizes of the per-slot buffers (gemv/test_kv_int4.py:311-313): k0.., v0.., ks0..,
    vs0..; payload rows heads * D / 2 bytes (INT4) or heads * D (INT8); scale rows heads * groups * 2 bytes viewed as
    (rows, row_bytes); the tiered pool's descriptors equal the INT4 pool's (the ring is not a per-slot buffer)."""
    from kvtier.tiered_kv_pool import MHATokenToKVPoolInt4, MHATokenToKVPoolInt8, MHATokenToKVPoolTiered
    size, page, H, D = 1024, 64, 2, 256
    rows = size + page
    mk = dict(size=size, page_size=page, head_num=H, head_dim=D, layer_num=2, device="cpu")
    p4 = MHATokenToKVPoolInt4(dtype=torch.uint8, **mk)
    d4 = p4._kv_buffer_descs
    assert [d.name for d in d4] == ["k0", "k1", "v0", "v1", "ks0", "ks1", "vs0", "vs1"]
    assert all(d.row_bytes == H * D // 2 and d.shape == (rows, H, D // 2) and d.tokens_per_row == 1 for d in d4[:4])
    assert all(d.row_bytes == 32 and d.shape == (rows, 32) for d in d4[4:])
    p8 = MHATokenToKVPoolInt8(dtype=torch.int8, **mk)
    d8 = p8._kv_buffer_descs
    assert [d.name for d in d8] == [d.name for d in d4]
    assert all(d.row_bytes == H * D and d.shape == (rows, H, D) for d in d8[:4])
    assert all(d.row_bytes == H * (D // 64) * 2 and d.shape == (rows, H * (D // 64) * 2) for d in d8[4:])
    # the descriptor sizes account for every byte of the per-slot buffers
    kb, vb = p8.get_kv_size_bytes()
    assert kb + vb == sum(rows * d.row_bytes for d in d8)
    import os
    os.environ["SGLANG_KV_TIERS_W"] = "64"
    try:
        pt = MHATokenToKVPoolTiered(dtype=torch.uint8, **mk)
    finally:
        del os.environ["SGLANG_KV_TIERS_W"]
    assert pt._kv_buffer_descs == d4
    with pytest.raises(ValueError):
        MHATokenToKVPoolInt4(dtype=torch.int8, **mk)
    with pytest.raises(ValueError):
        MHATokenToKVPoolInt8(dtype=torch.uint8, **mk)


def test_hybrid_forwarders_and_backend_kwargs(kvt_pkg, monkeypatch):
    """HybridLinearKVPool translates global layer ids of the full-attention layers to the pool's local ids and
    forwards the quantized pools' accessors (patches/kv_tiers.py:787-808); the backend's dispatch helpers
    (flat patch 1789-1827) return exactly the keyword arguments the gathers and the paged prefill accept."""
    import inspect
    from types import SimpleNamespace
    from kvtier import sparse_attn as sa
    from kvtier.backend_glue import KVDispatch
    from kvtier.tiered_kv_pool import (HybridLinearKVPool, MHATokenToKVPoolInt4, MHATokenToKVPoolInt8,
                                       MHATokenToKVPoolTiered)
    monkeypatch.setenv("SGLANG_KV_TIERS_W", "64")
    mk = dict(size=1024, page_size=64, head_num=2, head_dim=256, layer_num=3, device="cpu")
    tiered = MHATokenToKVPoolTiered(dtype=torch.uint8, **mk)
    hyb = HybridLinearKVPool(tiered, full_attention_layer_ids=[3, 7, 11])
    lay = SimpleNamespace(layer_id=7)
    assert hyb.get_key_buffer(7) is tiered.k_buffer[1] and hyb.get_value_buffer(11) is tiered.v_buffer[2]
    assert [t.data_ptr() for t in hyb.get_kv_ring_buffer(7)] == [t.data_ptr() for t in tiered.get_kv_ring_buffer(1)]
    assert hyb.get_kv_ring_owner() is tiered.ring_owner
    assert hyb.get_kv_scale_buffer(3)[0] is tiered.k_scale_buffer[0]
    assert hyb.get_kv_smooth_buffer(11)[1].data_ptr() == tiered.sm_v[2].data_ptr()
    with pytest.raises(ValueError):
        hyb.get_key_buffer(5)                     # a linear-attention layer has no KV here
    glue = KVDispatch(hyb)
    kb = hyb.get_key_buffer(7)
    assert glue._kv_bits() == 4 and glue._kv_head_dim(kb) == 256 and glue._kv_scratch_dtype(kb) == torch.bfloat16
    kw = glue._int8_gather_kwargs(kb, lay)
    assert set(kw) == {"k_scale", "v_scale", "sm_k", "sm_v", "kv_bits", "ring_k", "ring_v", "ring_ks", "ring_vs",
                       "owner", "ring_mask"}
    assert kw["ring_mask"] == 63 and kw["owner"] is tiered.ring_owner and kw["k_scale"] is tiered.k_scale_buffer[1]
    assert kw["ring_ks"] is tiered.ring_ks[1]
    for fn in (sa.qwen_sparse_kv_extraction_compact_triton, sa.sparse_gqa_fwd_interface_paged):
        params = inspect.signature(fn).parameters
        assert set(kw) <= set(params), (fn.__name__, set(kw) - set(params))
    tier_only = glue._kv_tier_kwargs(lay)
    assert set(tier_only) <= set(inspect.signature(sa.qwen_sparse_prefix_gather_dequant_tiered).parameters)
    # single-tier pools: no ring arguments; an unquantized stand-in gets none at all
    p4 = MHATokenToKVPoolInt4(dtype=torch.uint8, **mk)
    g4 = KVDispatch(p4)
    assert g4._kv_tier_kwargs(SimpleNamespace(layer_id=0)) == {}
    assert set(g4._int8_gather_kwargs(p4.k_buffer[0], SimpleNamespace(layer_id=0))) == {
        "k_scale", "v_scale", "sm_k", "sm_v", "kv_bits"}
    p8 = MHATokenToKVPoolInt8(dtype=torch.int8, **mk)
    g8 = KVDispatch(p8)
    assert g8._kv_bits() == 8 and g8._kv_head_dim(p8.k_buffer[0]) == 256
    kw8 = g8._int8_gather_kwargs(p8.k_buffer[0], SimpleNamespace(layer_id=2))
    assert kw8["kv_bits"] == 8 and kw8["sm_k"].data_ptr() == p8.sm_k[2].data_ptr()
    plain = SimpleNamespace(kv_bits=None)
    gp = KVDispatch(plain)
    bf = torch.zeros(4, 2, 256, dtype=torch.bfloat16)
    assert gp._int8_gather_kwargs(bf, lay) == {} and gp._kv_scratch_dtype(bf) == torch.bfloat16
    assert gp._kv_scratch_dtype(torch.zeros(4, 2, 256, dtype=torch.float16)) == torch.float16


def test_sparse_decode_merge_arguments_refused(kvt_pkg):
    """kvt_sparse_decode with merge counters refuses, before any launch, an output it cannot write: both or neither
    output pointer, a batch stride below Hq x D or not a multiple of 8, an output not 16-byte aligned, and partials of
    one (request, KV head) that 32-bit offsets cannot address.  No kernel runs (the pointers are never touched)."""
    lib = kvt_pkg._lib
    P = 0x10000   # a 16-byte aligned stand-in; every case returns before it would be used
    H, Hq, D = 2, 16, 256

    def call(out_f32=P, out_bf16=None, stride=Hq * D, n_splits=4, counters=P):
        lib.call("kvt_sparse_decode", 2, P, Hq * D, P, P, P, P, 4096, P, P, P, P, P, 1023, None, None, P, 8192, P, 1,
                 P, 2051, P, P, 0, 1, 2051, H, Hq, D, 64, 0.0625, n_splits, P, P, counters, out_f32, out_bf16, stride,
                 None)

    for kw in (dict(out_bf16=P), dict(out_f32=None), dict(stride=Hq * D - 8), dict(stride=Hq * D + 4),
               dict(out_f32=P + 4), dict(n_splits=(1 << 31) // ((Hq // H) * D * 4))):
        with pytest.raises(ValueError):
            call(**kw)
