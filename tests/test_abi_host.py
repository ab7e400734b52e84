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
    """The device page allocator hands out pages in the same seeded order as the oracle's."""
    from kvtier.kvt import PageAllocator
    from oracle.ref import PageAllocator as RefAlloc
    a, b = PageAllocator(100, seed=3), RefAlloc(100, seed=3)
    assert [a.pop() for _ in range(100)] == [b.pop() for _ in range(100)]
    with pytest.raises(RuntimeError):
        a.pop()
