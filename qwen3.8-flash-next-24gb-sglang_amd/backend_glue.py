"""How SGLang's Qwen sparse-attention backend picks the kernels and their keyword arguments for a quantized pool.

The reference adds five helper methods to ``QwenSparseAttnBackend`` (flat patch
sglang/qwen4exp-serving-73a255206f.patch:1789-1827, the tiered one also at patches/kv_tiers.py:745-761).  Every
decision is keyed on attributes of the pool (``kv_bits``, ``kv_tiered``, reached through a ``HybridLinearKVPool``'s
``full_kv_pool`` when there is one), never on the buffer dtype alone.  ``KVDispatch`` restates them as a small
object over the backend's ``token_to_kv_pool``, so that a backend can mix it in or hold one:

    glue = KVDispatch(pool)
    out_k = torch.empty(rows, H, glue._kv_head_dim(k_buf), dtype=glue._kv_scratch_dtype(k_buf), device=...)
    qwen_sparse_kv_extraction_compact_triton(k_buf, v_buf, ..., **glue._int8_gather_kwargs(k_buf, layer))

The kwargs it returns are exactly the keyword parameters of ``sparse_attn.qwen_sparse_kv_extraction_compact_triton``
and of the ``qwen_sparse_prefix_gather_dequant_*`` / ``sparse_gqa_fwd_interface_paged`` entry points.
"""
from __future__ import annotations

from typing import Optional

import torch


class KVDispatch:
    """Pool-keyed dispatch helpers of the QSA backend; ``token_to_kv_pool`` is the backend's pool (a quantized pool
    or a ``HybridLinearKVPool`` around one)."""

    def __init__(self, token_to_kv_pool):
        self.token_to_kv_pool = token_to_kv_pool

    def _full_pool(self):
        pool = self.token_to_kv_pool
        return getattr(pool, "full_kv_pool", pool)

    def _kv_bits(self) -> Optional[int]:
        """8 for ``int8_g64``, 4 for ``int4_g32`` and ``int8ring_int4``, None for an unquantized pool.  An fp8 pool
        also stores bytes, hence the pool attribute rather than the dtype."""
        return getattr(self._full_pool(), "kv_bits", None)

    def _kv_head_dim(self, k_buffer: torch.Tensor) -> int:
        """Channels per head of the rows a buffer holds (an INT4 row packs two per byte)."""
        per_byte = 2 if self._kv_bits() == 4 else 1
        return int(k_buffer.shape[2]) * per_byte

    def _kv_scratch_dtype(self, k_buffer: torch.Tensor) -> torch.dtype:
        """Dtype of the dequantized scratch the gathers write: bf16 for any quantized pool (fp8, INT8, INT4), the
        buffer's own dtype otherwise."""
        quantized = self._kv_bits() in (4, 8) or k_buffer.dtype in (torch.int8, torch.float8_e4m3fn)
        return torch.bfloat16 if quantized else k_buffer.dtype

    def _int8_gather_kwargs(self, k_buffer: torch.Tensor, layer) -> dict:
        """Keyword arguments of the gather-dequant kernels for this layer: scales, smoothing constants, kv_bits,
        and for the tiered pool the ring and owner table; {} for a pool the quantized gathers do not read."""
        bits = self._kv_bits()
        if bits != 4 and k_buffer.dtype != torch.int8:
            return {}
        pool = self.token_to_kv_pool
        k_scale, v_scale = pool.get_kv_scale_buffer(layer.layer_id)
        sm_k, sm_v = pool.get_kv_smooth_buffer(layer.layer_id)
        kwargs = {"k_scale": k_scale, "v_scale": v_scale, "sm_k": sm_k, "sm_v": sm_v, "kv_bits": bits}
        kwargs.update(self._kv_tier_kwargs(layer))
        return kwargs

    def _kv_tier_kwargs(self, layer) -> dict:
        """ring_k / ring_v / ring_ks / ring_vs of the layer, the owner table and ring_mask for a tiered pool; {} for
        any other.  The tensors live as long as the pool, so a captured graph may hold them."""
        full = self._full_pool()
        if not getattr(full, "kv_tiered", False):
            return {}
        pool = self.token_to_kv_pool
        names = ("ring_k", "ring_v", "ring_ks", "ring_vs")
        kwargs = dict(zip(names, pool.get_kv_ring_buffer(layer.layer_id)))
        kwargs["owner"] = pool.get_kv_ring_owner()
        kwargs["ring_mask"] = full.ring_mask
        return kwargs
