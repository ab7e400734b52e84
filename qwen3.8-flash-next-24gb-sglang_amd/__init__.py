"""MI355X-native tiered quantized KV cache (SGLang ``int8ring_int4`` mode): INT8 ring of the newest tokens over a
paged INT4-G32 pool, HIP kernels for gfx950 behind the C ABI in include/kvtier.h.

Modules:
  sparse_attn     the reference's operator surface (quant_store_kv_*, compact / prefix gathers, paged prefill)
  tiered_kv_pool  MHATokenToKVPoolTiered / Int4 / Int8 pool classes
  kvt             position-indexed (evict) cache, page allocator, split-K decode attention
  build           compiles libkvtier.so
"""
__version__ = "0.1.0"

from . import _lib  # noqa: F401
