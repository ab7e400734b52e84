"""Drop-in operator surface of the tiered KV path: the write / gather / attend calls SGLang's Qwen sparse-attention
backend makes (reference ``python/sglang/srt/layers/attention/qsa/sparse_attn.py`` as patched by
``patches/kv_int8.py``, ``patches/kv_int4.py``, ``patches/kv_tiers.py``, ``patches/kv_paged_prefix.py``).

Same names, argument order, defaults, in-place semantics and host-side contract checks (AssertionError) as the
reference wrappers; the work is done by the HIP kernels of libkvtier.so through its C ABI.  There is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib

KV_INT8_GROUP = 64   # channels per fp16 scale of the INT8 tier (patches/kv_int8.py:278)
KV_INT4_GROUP = 32   # channels per fp16 scale of the INT4 tier (patches/kv_int4.py:286)

_KIND_INT8, _KIND_INT4, _KIND_TIERED = 0, 1, 2


def _pow2(n: int) -> bool:
    return n > 0 and n & (n - 1) == 0


def _group8(D: int, scale: torch.Tensor) -> int:
    """INT8 group width from a scale tensor [*, H, D // G]: 64 (the shipped format) or D (per token and head,
    patches/kv_fakeq.py:9 / docs/KV_INT8_PLAN.md:24)."""
    g = D // scale.shape[-1]
    assert g * scale.shape[-1] == D and g in (KV_INT8_GROUP, D), f"INT8 scale group {g} not in (64, {D})"
    return g


def _loc_args(loc: torch.Tensor):
    assert loc.dtype in (torch.int32, torch.int64), loc.dtype
    assert loc.is_contiguous()
    return loc.data_ptr(), int(loc.dtype == torch.int64)


# ----------------------------------------------------------------------------------------------- write path
def quant_store_kv_tiered(k, v, loc, k_buf, v_buf, k_scale, v_scale, rk, rv, rks, rvs, owner, sm_k_inv, sm_v_inv,
                          ring_mask):
    """Dual write of N tokens into the tiered pool (patches/kv_tiers.py:390-443).

    k, v: [N, H, D] (bf16 / fp16 / fp32, unit last stride); loc: [N] int32/int64 slots (N <= R); k_buf/v_buf: uint8
    [rows, H, D // 2]; k_scale/v_scale: fp16 [rows, H, D // 32]; rk/rv: int8 [R, H, D]; rks/rvs: fp16 [R, H, D // 64];
    owner: int32 [R]; sm_*_inv: fp16 [H, D]; ring_mask = R - 1.  Slots of one write that share a ring row are safe:
    the owner stamp picks one winner per row, only the winner writes the ring row, the others are cold."""
    N, H, D = k.shape
    R = int(ring_mask) + 1
    assert R > 0 and R & (R - 1) == 0, f"ring_mask + 1 = {R} is not a power of two"
    assert v.shape == (N, H, D) and k.stride(2) == 1 and v.stride(2) == 1
    assert D % KV_INT4_GROUP == 0 and D % KV_INT8_GROUP == 0 and _pow2(D)
    assert k_buf.dtype == torch.uint8 and v_buf.dtype == torch.uint8
    assert k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16
    assert k_buf.is_contiguous() and v_buf.is_contiguous() and k_scale.is_contiguous() and v_scale.is_contiguous()
    assert k_buf.shape[1:] == (H, D // 2) and v_buf.shape[1:] == (H, D // 2)
    assert k_scale.shape[1:] == (H, D // KV_INT4_GROUP) and v_scale.shape[1:] == (H, D // KV_INT4_GROUP)
    assert rk.dtype == torch.int8 and rv.dtype == torch.int8 and rk.shape == (R, H, D) and rv.shape == (R, H, D)
    assert rks.dtype == torch.float16 and rvs.dtype == torch.float16
    g8 = _group8(D, rks)
    assert rks.shape == (R, H, D // g8) and rvs.shape == (R, H, D // g8)
    assert rk.is_contiguous() and rv.is_contiguous() and rks.is_contiguous() and rvs.is_contiguous()
    assert owner.dtype == torch.int32 and owner.shape == (R,) and owner.is_contiguous()
    assert sm_k_inv.shape == (H, D) and sm_v_inv.shape == (H, D)
    assert sm_k_inv.dtype == torch.float16 and sm_v_inv.dtype == torch.float16
    assert loc.numel() == N
    assert N <= R, f"{N} tokens in one tiered write exceed the ring of {R} slots"
    assert k.dtype == v.dtype and k.dtype in _lib.DTYPE_CODE, k.dtype
    if N == 0:
        return
    _lib.require_device(k, v, loc, k_buf, rk, owner, sm_k_inv)
    lp, l64 = _loc_args(loc)
    _lib.call("kvt_quant_store_tiered", k.data_ptr(), v.data_ptr(), _lib.DTYPE_CODE[k.dtype], k.stride(0),
              k.stride(1), v.stride(0), v.stride(1), lp, l64, N, H, D, k_buf.data_ptr(), v_buf.data_ptr(),
              k_scale.data_ptr(), v_scale.data_ptr(), rk.data_ptr(), rv.data_ptr(), rks.data_ptr(), rvs.data_ptr(),
              owner.data_ptr(), sm_k_inv.contiguous().data_ptr(), sm_v_inv.contiguous().data_ptr(), R - 1, g8,
              _lib.stream())


def quant_store_kv_int8(k, v, loc, k_buf, v_buf, k_scale, v_scale, sm_k_inv, sm_v_inv):
    """INT8-G quant + scatter (patches/kv_int8.py:331-362).  k, v: [N, H, D]; loc: [N] int32/int64; k_buf/v_buf:
    int8 [rows, H, D]; k_scale/v_scale: fp16 [rows, H, D // 64]; sm_*_inv: fp16 [H, D]."""
    N, H, D = k.shape
    assert v.shape == (N, H, D) and k.stride(2) == 1 and v.stride(2) == 1
    assert k_buf.dtype == torch.int8 and v_buf.dtype == torch.int8
    assert k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16
    assert k_buf.is_contiguous() and v_buf.is_contiguous() and k_scale.is_contiguous() and v_scale.is_contiguous()
    g8 = _group8(D, k_scale)
    assert k_buf.shape[1:] == (H, D) and k_scale.shape[1:] == (H, D // g8) and v_scale.shape[1:] == (H, D // g8)
    assert sm_k_inv.shape == (H, D) and sm_v_inv.shape == (H, D)
    assert loc.numel() == N
    assert k.dtype == v.dtype and k.dtype in _lib.DTYPE_CODE, k.dtype
    if N == 0:
        return
    _lib.require_device(k, v, loc, k_buf)
    lp, l64 = _loc_args(loc)
    _lib.call("kvt_quant_store_int8", k.data_ptr(), v.data_ptr(), _lib.DTYPE_CODE[k.dtype], k.stride(0), k.stride(1),
              v.stride(0), v.stride(1), lp, l64, N, H, D, k_buf.data_ptr(), v_buf.data_ptr(), k_scale.data_ptr(),
              v_scale.data_ptr(), sm_k_inv.contiguous().data_ptr(), sm_v_inv.contiguous().data_ptr(), g8,
              _lib.stream())


def quant_store_kv_int4(k, v, loc, k_buf, v_buf, k_scale, v_scale, sm_k_inv, sm_v_inv):
    """INT4-G32 quant + nibble pack + scatter (patches/kv_int4.py:360-393).  k, v: [N, H, D]; loc: [N] int32/int64;
    k_buf/v_buf: uint8 [rows, H, D // 2]; k_scale/v_scale: fp16 [rows, H, D // 32]; sm_*_inv: fp16 [H, D]."""
    N, H, D = k.shape
    assert v.shape == (N, H, D) and k.stride(2) == 1 and v.stride(2) == 1
    assert D % KV_INT4_GROUP == 0 and _pow2(D)
    assert k_buf.dtype == torch.uint8 and v_buf.dtype == torch.uint8
    assert k_scale.dtype == torch.float16 and v_scale.dtype == torch.float16
    assert k_buf.is_contiguous() and v_buf.is_contiguous() and k_scale.is_contiguous() and v_scale.is_contiguous()
    assert k_buf.shape[1:] == (H, D // 2) and v_buf.shape[1:] == (H, D // 2)
    assert k_scale.shape[1:] == (H, D // KV_INT4_GROUP) and v_scale.shape[1:] == (H, D // KV_INT4_GROUP)
    assert sm_k_inv.shape == (H, D) and sm_v_inv.shape == (H, D)
    assert loc.numel() == N
    assert k.dtype == v.dtype and k.dtype in _lib.DTYPE_CODE, k.dtype
    if N == 0:
        return
    _lib.require_device(k, v, loc, k_buf)
    lp, l64 = _loc_args(loc)
    _lib.call("kvt_quant_store_int4", k.data_ptr(), v.data_ptr(), _lib.DTYPE_CODE[k.dtype], k.stride(0), k.stride(1),
              v.stride(0), v.stride(1), lp, l64, N, H, D, k_buf.data_ptr(), v_buf.data_ptr(), k_scale.data_ptr(),
              v_scale.data_ptr(), sm_k_inv.contiguous().data_ptr(), sm_v_inv.contiguous().data_ptr(), _lib.stream())


# ----------------------------------------------------------------------------------------------- gathers
def _check_tier_args(heads, dim, k_scale, v_scale, ring_k, ring_v, ring_ks, ring_vs, owner, ring_mask):
    """Ring / owner shape and dtype contract of the tiered readers (patches/kv_tiers.py:622-636).  Returns R."""
    assert ring_k is not None and ring_v is not None and ring_ks is not None and ring_vs is not None
    assert owner is not None and ring_mask is not None, "tiered gather needs the owner table and ring_mask"
    R = int(ring_mask) + 1
    assert R > 0 and R & (R - 1) == 0, f"ring_mask + 1 = {R} is not a power of two"
    assert dim % KV_INT4_GROUP == 0 and dim % KV_INT8_GROUP == 0 and _pow2(dim)
    assert k_scale.shape[1:] == (heads, dim // KV_INT4_GROUP) and k_scale.is_contiguous()
    assert v_scale.shape[1:] == (heads, dim // KV_INT4_GROUP) and v_scale.is_contiguous()
    assert ring_k.dtype == torch.int8 and ring_v.dtype == torch.int8
    assert ring_k.shape == (R, heads, dim) and ring_v.shape == (R, heads, dim)
    assert ring_ks.dtype == torch.float16 and ring_vs.dtype == torch.float16
    g8 = _group8(dim, ring_ks)
    assert ring_ks.shape == (R, heads, dim // g8) and ring_vs.shape == (R, heads, dim // g8)
    assert ring_k.is_contiguous() and ring_v.is_contiguous() and ring_ks.is_contiguous() and ring_vs.is_contiguous()
    assert owner.dtype == torch.int32 and owner.shape == (R,) and owner.is_contiguous()
    return R


def _idx_args(t: torch.Tensor):
    assert t.dtype in (torch.int32, torch.int64) and t.is_contiguous(), t.dtype
    return t.data_ptr(), int(t.dtype == torch.int64)


def qwen_sparse_fa2_cu_seqlens_triton(seq_lens, indices, counts, cu_k, batch, topk):
    """Valid counts (0 <= pos < seq_len among the first topk columns) and their exclusive prefix sum cu_k
    [batch + 1], in place (the upstream helper the reference's tests call before a compact gather,
    gemv/test_kv_tiers.py:297-301): one HIP launch (kvt_sparse_cu_seqlens), no host sync.  seq_lens, indices and
    counts int32; cu_k int32 or int64."""
    assert seq_lens.dtype == torch.int32 and indices.dtype == torch.int32 and counts.dtype == torch.int32
    assert cu_k.dtype in (torch.int32, torch.int64) and cu_k.is_contiguous() and counts.is_contiguous()
    assert seq_lens.is_contiguous() and indices.dim() == 2 and indices.stride(1) == 1
    assert seq_lens.numel() >= batch and counts.numel() >= batch and cu_k.numel() >= batch + 1
    assert batch == 0 or indices.shape[0] >= batch or indices.stride(0) == 0
    assert topk <= indices.shape[1]
    _lib.require_device(seq_lens, indices, counts, cu_k)
    _lib.call("kvt_sparse_cu_seqlens", seq_lens.data_ptr(), indices.data_ptr(), indices.stride(0), counts.data_ptr(),
              cu_k.data_ptr(), int(cu_k.dtype == torch.int64), int(batch), int(topk), _lib.stream())


def qwen_sparse_kv_extraction_compact_triton(
    k, v, req_to_token, req_indices, indices, seq_lens, cu_k, out_k, out_v, batch, topk,
    k_scale=None, v_scale=None, sm_k=None, sm_v=None, kv_bits=None,
    ring_k=None, ring_v=None, ring_ks=None, ring_vs=None, owner=None, ring_mask=None,
):
    """Top-k gather-dequant of the selected positions into the bf16 scratch (final signature: flat patch
    sglang/qwen4exp-serving-73a255206f.patch:1545-1550; branches patches/kv_tiers.py:688-737,
    patches/kv_int4.py:569-605, patches/kv_int8.py:509-545).  Only valid columns are written."""
    _, heads, dim = k.shape
    if k.dtype == torch.uint8 and kv_bits == 4 and owner is not None:      # tiered: int8 ring over int4 rows
        dim = 2 * dim
        assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "tiered KV gather needs a bf16 scratch"
        assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
        assert k_scale is not None and v_scale is not None and sm_k is not None and sm_v is not None
        R = _check_tier_args(heads, dim, k_scale, v_scale, ring_k, ring_v, ring_ks, ring_vs, owner, ring_mask)
        kind, g8, rks_ = _KIND_TIERED, _group8(dim, ring_ks), ring_ks
    elif k.dtype == torch.uint8 and kv_bits == 4:                          # int4_g32 pool
        dim = 2 * dim
        assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "int4 KV gather needs a bf16 scratch"
        assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
        assert k_scale is not None and v_scale is not None and sm_k is not None and sm_v is not None
        assert dim % KV_INT4_GROUP == 0 and _pow2(dim)
        assert k_scale.is_contiguous() and v_scale.is_contiguous()
        R, kind, g8 = 1, _KIND_INT4, KV_INT8_GROUP
    elif k.dtype == torch.int8:                                            # int8_g64 pool
        assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "int8 KV gather needs a bf16 scratch"
        assert k_scale is not None and v_scale is not None and sm_k is not None and sm_v is not None
        assert dim % KV_INT8_GROUP == 0 and k_scale.is_contiguous() and v_scale.is_contiguous()
        assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
        R, kind, g8 = 1, _KIND_INT8, _group8(dim, k_scale)
    else:
        raise NotImplementedError(f"pool dtype {k.dtype} / kv_bits {kv_bits}: only the int8_g64, int4_g32 and "
                                  "int8ring_int4 pools are served by this library")
    assert out_k.is_contiguous() and out_v.is_contiguous()
    assert sm_k.shape == (heads, dim) and sm_v.shape == (heads, dim)
    assert req_to_token.dtype == torch.int32 and req_to_token.stride(1) == 1
    assert indices.dtype == torch.int32 and indices.stride(-1) == 1
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
    if batch == 0 or topk == 0:
        return
    _lib.require_device(k, v, req_to_token, indices, out_k)
    rq, rq64 = _idx_args(req_indices)
    cu, cu64 = _idx_args(cu_k)
    tier = kind == _KIND_TIERED
    _lib.call("kvt_compact_gather", kind, k.data_ptr(), v.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
              _lib.ptr(ring_k) if tier else None, _lib.ptr(ring_v) if tier else None,
              _lib.ptr(ring_ks) if tier else None, _lib.ptr(ring_vs) if tier else None,
              _lib.ptr(owner) if tier else None, R - 1, sm_k.contiguous().data_ptr(), sm_v.contiguous().data_ptr(),
              req_to_token.data_ptr(), req_to_token.stride(0), rq, rq64, indices.data_ptr(), indices.stride(0),
              seq_lens.data_ptr(), cu, cu64, int(batch), int(topk), heads, dim, g8, out_k.data_ptr(),
              out_v.data_ptr(), _lib.stream())


_MULTI_BLOCKS = 768   # blocks of a long-selection launch: one per resident slot, 3 per CU (50 KB of LDS, <= 168 VGPRs)


def qwen_sparse_decode_attn(
    q, k, v, req_to_token, req_indices, indices, seq_lens, cu_k, batch, topk,
    k_scale=None, v_scale=None, sm_k=None, sm_v=None, kv_bits=None,
    ring_k=None, ring_v=None, ring_ks=None, ring_vs=None, owner=None, ring_mask=None,
    scale=None, out=None, workspace=None, splits=None, merge="auto",
):
    """Top-k sparse decode attention fused over the quantized pool: what qwen_sparse_kv_extraction_compact_triton
    followed by FlashAttention-2 over its bf16 scratch computes for one query row per request (flat patch
    sglang/qwen4exp-serving-73a255206f.patch:1832-1882), in one split-K launch, with no scratch.  merge="launch": the
    block of a (request, KV head) that finishes last merges the column splits inside the launch (counters in the
    workspace: calls sharing a workspace must not overlap); merge="combine": the splits go through
    kvt_decode_combine, a second launch; merge="auto" (default): in the launch for at most 8 splits per (request, KV
    head), where it is the faster of the two (one block then reads at most 8 partials of up to 16 x 1 KB), else the
    combine launch, whose blocks (one per request, q head and slice of dims) read the partials side by side.

    q: bf16 [batch, Hq, D]; the pool/ring/owner/scale arguments as the compact gather; cu_k: the valid counts'
    prefix sum (qwen_sparse_fa2_cu_seqlens_triton).  Column c of request b is attended when c < cu_k[b+1] - cu_k[b]
    and 0 <= indices[b, c] < seq_lens[b].  Returns out (fp32 [batch, Hq, D] unless a bf16/fp32 `out` is given);
    a request with no attended column gives NaN.  `workspace` (a dict) keeps the partial buffers across calls;
    `splits` sets the number of column splits per (request, KV head) instead of the launch-size rule below."""
    _, heads, dim = k.shape
    if k.dtype == torch.uint8 and kv_bits == 4 and owner is not None:
        dim = 2 * dim
        R = _check_tier_args(heads, dim, k_scale, v_scale, ring_k, ring_v, ring_ks, ring_vs, owner, ring_mask)
        kind, g8 = _KIND_TIERED, _group8(dim, ring_ks)
    elif k.dtype == torch.uint8 and kv_bits == 4:
        dim = 2 * dim
        assert k_scale.shape[1:] == (heads, dim // KV_INT4_GROUP) and k_scale.is_contiguous() and v_scale.is_contiguous()
        R, kind, g8 = 1, _KIND_INT4, KV_INT8_GROUP
    elif k.dtype == torch.int8:
        assert k_scale.is_contiguous() and v_scale.is_contiguous()
        R, kind, g8 = 1, _KIND_INT8, _group8(dim, k_scale)
    else:
        raise NotImplementedError(f"pool dtype {k.dtype} / kv_bits {kv_bits}: only the int8_g64, int4_g32 and "
                                  "int8ring_int4 pools are served by this library")
    assert k.is_contiguous() and v.is_contiguous() and dim == 256, "the kernel is built for head_dim 256"
    assert q.dim() == 3 and q.shape[0] >= batch and q.shape[2] == dim and q.dtype == torch.bfloat16
    assert q.stride(2) == 1 and q.stride(1) == dim and q.stride(0) % 8 == 0
    Hq = q.shape[1]
    assert Hq % heads == 0 and Hq // heads <= 16, "at most 16 q heads per KV head"
    assert sm_k is None or sm_k.shape == (heads, dim)
    assert sm_v is None or sm_v.shape == (heads, dim)
    assert req_to_token.dtype == torch.int32 and req_to_token.stride(1) == 1
    assert indices.dtype == torch.int32 and indices.stride(-1) == 1
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
    if out is None:
        out = torch.empty(batch, Hq, dim, dtype=torch.float32, device=q.device)
    assert out.shape[0] >= batch and out.shape[1:] == (Hq, dim) and out.stride(2) == 1 and out.stride(1) == dim
    assert out.dtype in (torch.float32, torch.bfloat16)
    if batch == 0:
        return out
    if topk == 0:
        out[:batch] = float("nan")
        return out
    _lib.require_device(q, k, v, req_to_token, indices, out)
    scale = float(dim ** -0.5) if scale is None else float(scale)
    # blocks of 64 selected columns (a 16-column tile per wavefront) while the launch holds at most 1,024 of them;
    # longer selections take `tiles` tiles per wavefront in about one block per resident slot (3 per CU), each
    # partial then covering 64 x tiles columns
    tiles64 = (int(topk) + 63) // 64
    blocks = batch * heads * tiles64
    tiles = 1 if blocks <= 1024 else -(-blocks // _MULTI_BLOCKS)
    n_splits = -(-tiles64 // tiles) if splits is None else int(splits)
    assert n_splits >= 1
    ws = workspace if workspace is not None else {}
    need = batch * heads * n_splits * (Hq // heads)
    if ws.get("sparse_o") is None or ws["sparse_o"].numel() < need * dim:
        ws["sparse_o"] = torch.empty(need * dim, dtype=torch.float32, device=q.device)
        ws["sparse_ml"] = torch.empty(need * 2, dtype=torch.float32, device=q.device)
    if merge not in ("auto", "launch", "combine"):
        raise ValueError(f"merge must be 'auto', 'launch' or 'combine', not {merge!r}")
    rows_ok = out.stride(0) % 8 == 0 and out.data_ptr() % 16 == 0   # the in-launch merge writes 16-byte pieces
    fused = merge == "launch" or (merge == "auto" and n_splits <= 8 and rows_ok)
    if fused:
        assert rows_ok, "merge='launch' needs out rows 16-byte aligned with a batch stride that is a multiple of 8"
        if ws.get("sparse_ctr") is None or ws["sparse_ctr"].numel() < batch * heads:
            ws["sparse_ctr"] = torch.zeros(batch * heads, dtype=torch.int32, device=q.device)   # each call leaves 0
    rq, rq64 = _idx_args(req_indices)
    cu, cu64 = _idx_args(cu_k)
    tier = kind == _KIND_TIERED
    smk = None if sm_k is None else sm_k.contiguous()
    smv = None if sm_v is None else sm_v.contiguous()
    st = _lib.stream()
    _lib.call("kvt_sparse_decode", kind, q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k_scale.data_ptr(),
              v_scale.data_ptr(), k.shape[0], _lib.ptr(ring_k) if tier else None, _lib.ptr(ring_v) if tier else None,
              _lib.ptr(ring_ks) if tier else None, _lib.ptr(ring_vs) if tier else None,
              _lib.ptr(owner) if tier else None, R - 1, _lib.ptr(smk), _lib.ptr(smv), req_to_token.data_ptr(),
              req_to_token.stride(0), rq, rq64, indices.data_ptr(), indices.stride(0), seq_lens.data_ptr(), cu, cu64,
              int(batch), int(topk), heads, Hq, dim, g8, scale, n_splits, ws["sparse_o"].data_ptr(),
              ws["sparse_ml"].data_ptr(), ws["sparse_ctr"].data_ptr() if fused else None,
              out.data_ptr() if fused and out.dtype == torch.float32 else None,
              out.data_ptr() if fused and out.dtype == torch.bfloat16 else None, out.stride(0), st)
    if fused:
        return out
    o32 = out.data_ptr() if out.dtype == torch.float32 else None
    o16 = out.data_ptr() if out.dtype == torch.bfloat16 else None
    _lib.call("kvt_decode_combine", ws["sparse_o"].data_ptr(), ws["sparse_ml"].data_ptr(), int(batch), heads, Hq, dim,
              n_splits, 0, seq_lens.data_ptr(), None, o32, o16, out.stride(0), st)
    return out


def sparse_gqa_fwd_interface_paged(
    q, indices, cu_q, kv_lens, req_to_token, req_indices, k_buf, v_buf, k_scale, v_scale, sm_k, sm_v, scale,
    max_q, kv_bits, ring_k=None, ring_v=None, ring_ks=None, ring_vs=None, owner=None, ring_mask=None, config=None,
    out=None,
):
    """Prefix-chunk sparse attention read straight from a quantized pool (patches/kv_paged_prefix.py:267-365).

    q: bf16 [total_q, Hq, D]; indices: int32 [total_q, topk] or [total_q, H, topk] (selected positions per query,
    per KV head in the 3-d form); cu_q: int32 / int64 [batch + 1] (chunk b owns rows cu_q[b] .. cu_q[b + 1]);
    kv_lens: int32 [batch], the full context lengths (prefix + chunk); req_to_token int32 [reqs, ctx] and
    req_indices [batch] map positions to slots; k_buf / v_buf + k_scale / v_scale: the pool (int8 [rows, H, D] +
    fp16 [rows, H, D / 64] for kv_bits 8, uint8 [rows, H, D / 2] + fp16 [rows, H, D / 32] for kv_bits 4); sm_k / sm_v
    [H, D]; the ring arguments select the tiered pool.  Query j of chunk b attends the entries of its index row
    among the first min(topk, j + kv_len - q_len + 1) that lie in [0, kv_len); an entry outside is ignored, and a row
    with none comes out NaN (0/0), as the reference.  (The reference kernel reads on to the next multiple of its
    16-column tile, patches/kv_paged_prefix.py:201-202; the columns between hold -1 in an indexer row, and entries
    planted there are ignored here, as the reference test's oracle does.)  K/V rows are dequantized exactly as the gathers write them,
    QK^T and P.V on bf16 matrix cores with fp32 accumulation.  max_q = the longest chunk (host int).  `config` is the
    reference's Triton tile configuration and has no meaning here (accepted and ignored).  Returns a new bf16 tensor
    shaped like q, as the reference; `out` (an addition: bf16 or fp32, shaped like q, unit last stride) receives the
    result instead, the bf16 form being the fp32 one rounded to nearest even.
    """
    total_q, num_q_heads, head_dim = q.shape
    _, heads, last = k_buf.shape
    assert q.dtype == torch.bfloat16 and q.stride(2) == 1, "paged prefix attention needs bf16 queries"
    assert k_buf.is_contiguous() and v_buf.is_contiguous() and v_buf.shape == k_buf.shape
    assert indices.dtype == torch.int32 and kv_lens.dtype == torch.int32 and kv_lens.is_contiguous()
    assert indices.dim() in (2, 3) and indices.shape[0] >= total_q
    assert cu_q.dtype in (torch.int32, torch.int64) and cu_q.is_contiguous(), cu_q.dtype
    assert req_to_token.dtype == torch.int32 and req_to_token.dim() == 2 and req_to_token.stride(1) == 1
    if owner is not None:                                   # tiered: INT8 ring over INT4 rows
        dim = 2 * last
        assert kv_bits == 4 and k_buf.dtype == torch.uint8 and v_buf.dtype == torch.uint8
        R = _check_tier_args(heads, dim, k_scale, v_scale, ring_k, ring_v, ring_ks, ring_vs, owner, ring_mask)
        kind, g8 = _KIND_TIERED, _group8(dim, ring_ks)
    elif kv_bits == 4:                                      # int4_g32 pool
        dim = 2 * last
        assert k_buf.dtype == torch.uint8 and v_buf.dtype == torch.uint8
        assert dim % KV_INT4_GROUP == 0 and _pow2(dim)
        for t in (k_scale, v_scale):
            assert t.dtype == torch.float16 and t.shape[1:] == (heads, dim // KV_INT4_GROUP) and t.is_contiguous()
        R, kind, g8 = 1, _KIND_INT4, KV_INT8_GROUP
    else:                                                   # int8_g64 pool
        dim = last
        assert k_buf.dtype == torch.int8 and v_buf.dtype == torch.int8
        assert dim % KV_INT8_GROUP == 0 and _pow2(dim)
        g8 = _group8(dim, k_scale)
        for t in (k_scale, v_scale):
            assert t.dtype == torch.float16 and t.shape[1:] == (heads, dim // g8) and t.is_contiguous()
        R, kind = 1, _KIND_INT8
    assert dim == head_dim, f"pool head_dim {dim} != query head_dim {head_dim}"
    assert dim == 256, "the kernel is built for head_dim 256"
    assert sm_k.shape == (heads, dim) and sm_v.shape == (heads, dim)
    assert num_q_heads % heads == 0 and num_q_heads // heads <= 16, "at most 16 q heads per KV head"
    if indices.dim() == 3:
        assert indices.shape[1] == heads
    assert config is None or len(config) == 3
    batch = cu_q.shape[0] - 1
    if out is None:
        out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    assert out.shape == q.shape and out.dtype in (torch.bfloat16, torch.float32) and out.stride(2) == 1
    if batch == 0 or int(max_q) == 0:
        return out
    _lib.require_device(q, indices, cu_q, kv_lens, req_to_token, k_buf, v_buf, out)
    if q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    topk = indices.shape[-1]
    si_g = indices.stride(1) if indices.dim() == 3 else 0
    rq, rq64 = _idx_args(req_indices)
    tier = kind == _KIND_TIERED
    smk, smv = sm_k.contiguous(), sm_v.contiguous()
    _lib.call("kvt_sparse_prefill", kind, q.data_ptr(), q.stride(0), q.stride(1), cu_q.data_ptr(),
              int(cu_q.dtype == torch.int64), kv_lens.data_ptr(), batch, int(max_q), indices.data_ptr(),
              indices.stride(0), si_g, indices.stride(-1), int(topk), k_buf.data_ptr(), v_buf.data_ptr(),
              k_scale.data_ptr(), v_scale.data_ptr(), k_buf.shape[0], _lib.ptr(ring_k) if tier else None,
              _lib.ptr(ring_v) if tier else None, _lib.ptr(ring_ks) if tier else None,
              _lib.ptr(ring_vs) if tier else None, _lib.ptr(owner) if tier else None, R - 1, smk.data_ptr(),
              smv.data_ptr(), req_to_token.data_ptr(), req_to_token.stride(0), rq, rq64, heads, num_q_heads, dim,
              g8, float(scale), out.data_ptr(), int(out.dtype == torch.float32), out.stride(0), out.stride(1),
              _lib.stream())
    return out


def _prefix_gather(kind, k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k, out_v,
                   batch, max_len, dim, g8, tier=None):
    assert out_k.is_contiguous() and out_v.is_contiguous()
    assert req_to_token.dtype == torch.int32 and req_to_token.stride(1) == 1
    assert seq_lens.dtype == torch.int32 and seq_lens.is_contiguous()
    if batch == 0 or max_len == 0:
        return
    heads = k.shape[1]
    _lib.require_device(k, v, req_to_token, out_k)
    rq, rq64 = _idx_args(req_indices)
    cu, cu64 = _idx_args(cu_k)
    t = tier or {}
    R = int(t.get("ring_mask", 0)) + 1
    _lib.call("kvt_prefix_gather", kind, k.data_ptr(), v.data_ptr(), k_scale.data_ptr(), v_scale.data_ptr(),
              _lib.ptr(t.get("ring_k")), _lib.ptr(t.get("ring_v")), _lib.ptr(t.get("ring_ks")),
              _lib.ptr(t.get("ring_vs")), _lib.ptr(t.get("owner")), R - 1, sm_k.contiguous().data_ptr(),
              sm_v.contiguous().data_ptr(), req_to_token.data_ptr(), req_to_token.stride(0), rq, rq64,
              seq_lens.data_ptr(), cu, cu64, int(batch), int(max_len), heads, dim, g8, out_k.data_ptr(),
              out_v.data_ptr(), _lib.stream())


def qwen_sparse_prefix_gather_dequant_tiered(
    k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k, out_v, batch, max_len,
    ring_k=None, ring_v=None, ring_ks=None, ring_vs=None, owner=None, ring_mask=None,
):
    """Whole-prefix gather-dequant of the tiered pool: rows [0, seq_lens[b]) packed at cu_k[b], each from its tier;
    rows at or beyond seq_lens[b] are not written (patches/kv_tiers.py:639-683)."""
    _, heads, dh = k.shape
    dim = 2 * dh
    assert k.dtype == torch.uint8 and v.dtype == torch.uint8
    assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "tiered KV gather needs a bf16 scratch"
    assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
    assert sm_k.shape == (heads, dim) and sm_v.shape == (heads, dim)
    _check_tier_args(heads, dim, k_scale, v_scale, ring_k, ring_v, ring_ks, ring_vs, owner, ring_mask)
    _prefix_gather(_KIND_TIERED, k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k,
                   out_v, batch, max_len, dim, _group8(dim, ring_ks),
                   dict(ring_k=ring_k, ring_v=ring_v, ring_ks=ring_ks, ring_vs=ring_vs, owner=owner,
                        ring_mask=ring_mask))


def qwen_sparse_prefix_gather_dequant_int4(
    k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k, out_v, batch, max_len
):
    """Whole-prefix gather-dequant of the int4 pool (patches/kv_int4.py:519-557)."""
    _, heads, dh = k.shape
    dim = 2 * dh
    assert k.dtype == torch.uint8 and v.dtype == torch.uint8
    assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "int4 KV gather needs a bf16 scratch"
    assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
    assert dim % KV_INT4_GROUP == 0 and _pow2(dim)
    assert k_scale.shape[1:] == (heads, dim // KV_INT4_GROUP) and k_scale.is_contiguous()
    assert v_scale.shape[1:] == (heads, dim // KV_INT4_GROUP) and v_scale.is_contiguous()
    assert sm_k.shape == (heads, dim) and sm_v.shape == (heads, dim)
    _prefix_gather(_KIND_INT4, k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k,
                   out_v, batch, max_len, dim, KV_INT8_GROUP)


def qwen_sparse_prefix_gather_dequant_int8(
    k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k, out_v, batch, max_len
):
    """Whole-prefix gather-dequant of an int8 pool (patches/kv_int8.py:469-504)."""
    _, heads, dim = k.shape
    assert k.dtype == torch.int8 and v.dtype == torch.int8
    assert out_k.dtype == torch.bfloat16 and out_v.dtype == torch.bfloat16, "int8 KV gather needs a bf16 scratch"
    assert dim % KV_INT8_GROUP == 0 and _pow2(dim)
    g8 = _group8(dim, k_scale)
    assert k_scale.shape[1:] == (heads, dim // g8) and k_scale.is_contiguous()
    assert v_scale.shape[1:] == (heads, dim // g8) and v_scale.is_contiguous()
    assert sm_k.shape == (heads, dim) and sm_v.shape == (heads, dim)
    assert out_k.shape[1:] == (heads, dim) and out_v.shape[1:] == (heads, dim)
    _prefix_gather(_KIND_INT8, k, v, k_scale, v_scale, sm_k, sm_v, req_to_token, req_indices, seq_lens, cu_k, out_k,
                   out_v, batch, max_len, dim, g8)
