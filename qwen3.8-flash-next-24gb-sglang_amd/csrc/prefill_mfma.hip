// Causal prefill attention over the position-indexed tiered cache on gfx950 matrix cores.
//
// The queries of a chunk (positions q0 .. q0 + n - 1 of a sequence whose cache already holds the chunk) attend to
// every key position <= their own (patches/kv_paged_prefix.py:200: visible = j + kv_len - q_len + 1).  Keys and
// values come from the cache tiers (INT4 pages below hot_start, INT8 ring above) or, for a chunk without a prefix,
// from the chunk's own bf16 K/V (the reference attends to fresh bf16 K/V there).
//
// Work item = (sequence, KV head, tile of queries), 8 wavefronts (2 per SIMD), heaviest (latest) query tiles
// first.  A wavefront owns 16 query rows = 16 / gs queries x the gs q heads of the KV head (gs <= 16; rows beyond
// 16 / gs * gs idle).  The block walks the keys in tiles of 32 positions.  All 512 threads dequantize a tile ONCE
// into LDS (each thread 16 channels of a K row and 8 channels of two V rows), with the next tile's codes already
// loaded into registers during the matrix work on the current one; the eight wavefronts then reuse it for their
// 16 rows each (dequantizing per query row is what made the reference's fused kernel slow,
// docs/KV_PAGED_PREFIX_PLAN.md:188-191).
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16: A = 16 K rows x 32 channels from LDS (bf16), B = Q (the wavefront's 16
//   rows) held in registers as the input bf16 values; the fp32 scores are scaled by scale * log2(e).  The D layout
//   puts 4 keys of one query row in each lane: row max / sum need two cross-lane steps, and the lane's P values are
//   directly the A operand of P.V (k = keys {4 kb .. +3, 16 + 4 kb .. +3}).
//   O += P V / 128 on v_mfma_f32_16x16x32_f16: A = P rounded to fp16, B = V rows from LDS in fp16, each value the
//   bf16 row value / 128 (two transposing 8-byte reads per 16-dim column block).  The reference's kernel rounds P to
//   bf16 for its P.V product (patches/kv_paged_prefix.py:251-252); fp16 keeps 11 significant bits, and the row sum
//   adds the rounded P, so the output is a weighted mean with exactly the weights of the products.
// Numerics: K operands are exactly the oracle's rows, bf16(code * scale) rounded to nearest even from the exact fp32
// product (or the chunk's own bf16 K/V); V operands the same values / 128 in fp16, exact for |v| >= 2^-10 up to
// 65504 * 128 (every clamp-regime value, |code * scale| <= 127 * 65504) and to 2^-18 below; Q exact; fp32
// accumulation and softmax; bf16 (as the reference) or fp32 output.  The bf16 source must keep |V| <= 65504 * 128.

#include "kvt_common.h"

using namespace kvt;

namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
typedef float f2v __attribute__((ext_vector_type(2)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef short s4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4v lds_s4;

constexpr int kD = 256;
constexpr int kT = 32;                  // key positions per tile
// LDS tiles, laid out so that the matrix operand reads are free of bank conflicts (64 banks of 4 bytes):
//   K: bf16 row per key (512 B); its 16-byte chunk c lives at chunk c ^ (key & 15).  An A-operand read takes chunk
//      4 st + kb of 16 consecutive keys: 16 distinct chunks mod 16, i.e. all 64 banks.
//   V: bf16 row per key (256 dims) at a pitch of 544 B (136 dwords, 8 banks past a multiple of 64).  The P.V B
//      operand (dims 16 c .. 16 c + 15 of keys 4 kb .. 4 kb + 3, then 16 + 4 kb .. 16 + 4 kb + 3: the k order of the
//      P operand) is two ds_read_b64_tr_b16: in each 16-lane group lane m addresses 8 bytes of row 4 kb + (m >> 2)
//      at dim 16 c + 4 (m & 3), and lane L receives element L & 3 of the 8 bytes of lanes 4 k + (L >> 2), i.e. the
//      dim 16 c + L of keys 4 kb + k; the four rows of a group sit 8 banks apart.  A converting thread stores 8
//      channels of keys tp and tp + 16 (16 bytes each) with no transposition.
constexpr int kKPitch = kD * 2;         // bytes per bf16 K row
constexpr int kVRow = kD * 2 + 32;      // bytes per bf16 V row
KVT_DEV uint32_t k_chunk(int key, int c) { return 16u * (uint32_t)(c ^ (key & 15)); }
constexpr float kLog2e = 1.4426950408889634f;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOOB = 0x80000000u;     // byte offset beyond every buffer: the load returns zeros
constexpr int kMaxLdsPages = 8192;         // page ids staged in LDS: paged key ranges up to 524,288 positions

struct KVSrc {
  const uint8_t* k4;
  const uint8_t* v4;
  const uint16_t* ks4;
  const uint16_t* vs4;
  const int8_t* rk;
  const int8_t* rv;
  const uint16_t* rks;
  const uint16_t* rvs;
  const int64_t* ring_base;
  const int32_t* ring_len;
  const int64_t* ring_start;
  const int32_t* page_table;
  int64_t pt_stride;
  uint32_t pool_rows;
  const uint16_t* kb;   // bf16 source [positions, H, D] (the BF16 kernel variant reads keys from here)
  const uint16_t* vb;
  int64_t kb_n, kb_h, vb_n, vb_h, kb_rows;
};

struct __align__(16) Lds {
  uint8_t k[2][kT * kKPitch];    // double-buffered: tile i + 1 is dequantized while tile i is in use
  uint8_t v[2][kT * kVRow];
  int32_t pages[kMaxLdsPages];
  int flag;                      // segments: "this block merges"
};

KVT_DEV f4 mfma(bf8 a, bf8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0); }
KVT_DEV f4 mfma(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// max of two scores in one v_max_f32: written as asm, the compiler adds no canonicalizing v_max_f32 x, x, x for
// values out of a lane permute (the scores are finite or -inf, never NaN)
KVT_DEV float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
KVT_DEV float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// the max over the 4 lanes l, l ^ 16, l ^ 32, l ^ 48 (v_permlane16_swap / v_permlane32_swap; all lanes active)
KVT_DEV float vmax_xor16_32(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// bf16 pair (round to nearest even, one v_cvt_pk_bf16_f32): lo in bits 0-15.
KVT_DEV uint32_t bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){lo, hi}, bf2v));
}

KVT_DEV Rsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
KVT_DEV uint4 ld128(Rsrc r, uint32_t off) {
  const v4i x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4((uint32_t)x.x, (uint32_t)x.y, (uint32_t)x.z, (uint32_t)x.w);
}
KVT_DEV uint2 ld64(Rsrc r, uint32_t off) {
  const v2i x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2((uint32_t)x.x, (uint32_t)x.y);
}
KVT_DEV uint32_t ld16(Rsrc r, uint32_t off) { return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0); }

// Segments.  A spread launch splits the key tiles of a query tile into segments held by different blocks, so that
// every block gets the same number of key tiles (the latest query tiles of a causal chunk see up to a chunk length
// more keys than the earliest).  A block writes a segment's (m, l, O) -- the online softmax state of its 128 rows
// over the segment -- into the segment's slot and counts itself on the query tile's counter; the block that counts
// last merges the nseg states in segment order, writes the output, and resets the counter to zero for the next
// call.  Slots and counters cross XCDs (each has its own L2): they are
// written and read with device-scope accesses (through to the coherence point past the L2), and a block waits for
// its slot stores to complete before it counts itself.  The merge is a fixed sum over the segments, so the output
// does not depend on which block merges; no block ever waits for another.
// Slot layout (floats): O at ((wave * 16 + c) * 64 + lane) * 4 + i (accumulator acc[c][i]: one 16-byte store per
// column block, 1 KB per wavefront store), then (m, l) of row r of wavefront w at kSlotO + 2 (16 w + r).
constexpr int kSc1 = 16;   // cache-policy operand of the raw buffer builtins: sc1 (device scope, past the L2)
constexpr int kSlotO = 8 * 64 * 64;
constexpr int kSlotFloats = kSlotO + 8 * 16 * 2;
KVT_DEV void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
KVT_DEV float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KVT_DEV void st_dev_i32(int32_t* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
KVT_DEV int ld_dev_i32(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
KVT_DEV int add_dev_i32(int32_t* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This block's view of the key source: buffer resources over the INT4 pool, the sequence's ring rows and the bf16
// source, the tier boundary and the key range.  Every key fetch issues the loads of both tiers unconditionally
// (the other tier's at an offset beyond its buffer, which returns zeros): no branch, so the loads of the next tile
// stay in flight across the matrix work of the current one.
struct Tier {
  Rsrc k4, v4, ks4, vs4, rk, rv, rks, rvs, kb, vb;
  int hs, rmask, key_end;   // positions (< 2^31: the entry point bounds the context)
  int kb_n, kb_h, vb_n, vb_h;
  int H, h;
};

// Raw K of one key row, channels 16 dc .. 16 dc + 15: INT4 (a4, s4) or INT8 (b, s8); bf16 source: a, b.
struct RawK {
  uint4 a, b;
  uint2 a4;
  uint32_t s4, s8;
  int hot;
};
// Raw V of two key rows (keys k and k + 16 of a tile), channels 8 db .. 8 db + 7 each: INT4 (c4, s4) or INT8 (a8,
// s8); bf16 source: a.
struct RawV {
  uint4 a[2];
  uint2 a8[2];
  uint32_t c4[2];
  uint32_t s4[2], s8[2];
  int hot[2];
};

KVT_DEV uint32_t ld32(Rsrc r, uint32_t off) { return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0); }

template <int G8, bool BF16>
KVT_DEV RawK fetch_k(const Tier& T, const int32_t* lpages, int p, int dc) {
  RawK x;
  p = min(p, T.key_end - 1);   // keys past the end: valid rows, masked in the scores
  if constexpr (BF16) {
    const uint32_t off = (uint32_t)(p * T.kb_n + T.h * T.kb_h + 16 * dc) * 2u;
    x.a = ld128(T.kb, off);
    x.b = ld128(T.kb, off + 16);
    x.hot = 2;
  } else {
    constexpr int NG8 = kD / G8;
    const bool hot = p >= T.hs;
    const int pg = hot ? 0 : min(p >> 6, kMaxLdsPages - 1);
    const uint32_t rh4 = ((uint32_t)lpages[pg] * kPage + (uint32_t)(p & (kPage - 1))) * T.H + T.h;
    const uint32_t rh8 = (uint32_t)(p & T.rmask) * T.H + T.h;
    x.a4 = ld64(T.k4, hot ? kOOB : rh4 * 128u + 8u * dc);
    x.s4 = ld16(T.ks4, hot ? kOOB : (rh4 * 8u + dc / 2) * 2u);
    x.b = ld128(T.rk, hot ? rh8 * 256u + 16u * dc : kOOB);
    x.s8 = ld16(T.rks, hot ? (rh8 * NG8 + (16u * dc) / G8) * 2u : kOOB);
    x.hot = hot ? 1 : 0;
  }
  return x;
}

// V of keys p0 and p0 + 16, channels 8 db .. 8 db + 7
template <int G8, bool BF16>
KVT_DEV RawV fetch_v(const Tier& T, const int32_t* lpages, int p0, int db) {
  RawV x;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int p = min(p0 + 16 * t, T.key_end - 1);
    if constexpr (BF16) {
      const uint32_t off = (uint32_t)(p * T.vb_n + T.h * T.vb_h + 8 * db) * 2u;
      x.a[t] = ld128(T.vb, off);
      x.hot[t] = 2;
    } else {
      constexpr int NG8 = kD / G8;
      const bool hot = p >= T.hs;
      const int pg = hot ? 0 : min(p >> 6, kMaxLdsPages - 1);
      const uint32_t rh4 = ((uint32_t)lpages[pg] * kPage + (uint32_t)(p & (kPage - 1))) * T.H + T.h;
      const uint32_t rh8 = (uint32_t)(p & T.rmask) * T.H + T.h;
      x.c4[t] = ld32(T.v4, hot ? kOOB : rh4 * 128u + 4u * db);
      x.s4[t] = ld16(T.vs4, hot ? kOOB : (rh4 * 8u + db / 4) * 2u);
      x.a8[t] = ld64(T.rv, hot ? rh8 * 256u + 8u * db : kOOB);
      x.s8[t] = ld16(T.rvs, hot ? (rh8 * NG8 + (8u * db) / G8) * 2u : kOOB);
      x.hot[t] = hot ? 1 : 0;
    }
  }
  return x;
}

// Fetches of a whole tile t2 .. t2 + 31 whose keys all sit in one tier and before the key end: the row base of the
// tile is uniform (a scalar offset of the buffer load) and the rest a per-lane constant (FetchLane), so the fetch
// costs no vector address arithmetic.  Ring rows: R is a power of two >= 32, so (t2 + k) & (R - 1) =
// (t2 & (R - 1)) + k; pages: the 32 keys of a tile lie on one 64-position page.  A whole-tile fetch fills only its
// tier's fields (the tile is converted by that tier's loop body); other tiles take the per-key fetch above.  The
// kind of fetch is a template parameter of the loop body, never a branch inside it: loads issued on different
// paths that join inside the loop would leave the wait counters unknown, and the body would wait for every load.
KVT_DEV uint4 ld128s(Rsrc r, uint32_t v, uint32_t s) {
  const v4i x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)v, (int)s, 0);
  return make_uint4((uint32_t)x.x, (uint32_t)x.y, (uint32_t)x.z, (uint32_t)x.w);
}
KVT_DEV uint2 ld64s(Rsrc r, uint32_t v, uint32_t s) {
  const v2i x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)v, (int)s, 0);
  return make_uint2((uint32_t)x.x, (uint32_t)x.y);
}
KVT_DEV uint32_t ld32s(Rsrc r, uint32_t v, uint32_t s) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)v, (int)s, 0);
}
KVT_DEV uint32_t ld16s(Rsrc r, uint32_t v, uint32_t s) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)v, (int)s, 0);
}

// Per-lane byte offsets within a tile: K row tk, channels 16 dc; V rows tp and tp + 16 (the second adds 16 rows'
// stride to the scalar part), channels 8 db.  INT8 codes / scales, INT4 codes / scales; the bf16 source uses k8 and v8.
struct FetchLane {
  uint32_t k8, k8s, k4, k4s, v8, v8s, v4, v4s;
};

template <int G8, bool BF16>
KVT_DEV FetchLane fetch_lane(const Tier& T, int tk, int dc, int tp, int db) {
  constexpr uint32_t NG8 = kD / G8;
  FetchLane F;
  const uint32_t H = (uint32_t)T.H;
  if constexpr (BF16) {
    F.k8 = (uint32_t)(tk * T.kb_n + 16 * dc) * 2u;
    F.v8 = (uint32_t)(tp * T.vb_n + 8 * db) * 2u;
    F.k8s = F.k4 = F.k4s = F.v8s = F.v4 = F.v4s = 0;
  } else {
    F.k8 = (uint32_t)tk * H * 256u + 16u * dc;
    F.k8s = ((uint32_t)tk * H * NG8 + (16u * dc) / G8) * 2u;
    F.k4 = (uint32_t)tk * H * 128u + 8u * dc;
    F.k4s = ((uint32_t)tk * H * 8u + dc / 2) * 2u;
    F.v8 = (uint32_t)tp * H * 256u + 8u * db;
    F.v8s = ((uint32_t)tp * H * NG8 + (8u * db) / G8) * 2u;
    F.v4 = (uint32_t)tp * H * 128u + 4u * db;
    F.v4s = ((uint32_t)tp * H * 8u + db / 4) * 2u;
  }
  return F;
}

// How tile it + 2 is fetched: per key (kFetchKeys: a tile that straddles hot_start or the key end, or a ring
// shorter than a tile), as a whole INT4 / INT8 / bf16 tile, or not at all (past the last tile).
enum { kFetchKeys = 0, kFetchInt4 = 1, kFetchInt8 = 2, kFetchBf16 = 3, kFetchNone = 4 };

template <int FETCH, int G8, bool BF16>
KVT_DEV void fetch_k_tile(const Tier& T, const int32_t* lpages, int t2, const FetchLane& F, int tk, int dc, RawK& x) {
  constexpr uint32_t NG8 = kD / G8;
  if constexpr (FETCH == kFetchKeys) {
    x = fetch_k<G8, BF16>(T, lpages, t2 + tk, dc);
  } else if constexpr (FETCH == kFetchBf16) {
    const uint32_t so = (uint32_t)(t2 * T.kb_n + T.h * T.kb_h) * 2u;
    x.a = ld128s(T.kb, F.k8, so);
    x.b = ld128s(T.kb, F.k8 + 16u, so);
  } else if constexpr (FETCH == kFetchInt8) {
    const uint32_t r8 = (uint32_t)((t2 & T.rmask) * T.H + T.h);
    x.b = ld128s(T.rk, F.k8, r8 * 256u);
    x.s8 = ld16s(T.rks, F.k8s, r8 * NG8 * 2u);
  } else if constexpr (FETCH == kFetchInt4) {
    const uint32_t pg = (uint32_t)__builtin_amdgcn_readfirstlane(lpages[min(t2 >> 6, kMaxLdsPages - 1)]);
    const uint32_t r4 = (pg * kPage + (uint32_t)(t2 & (kPage - 1))) * (uint32_t)T.H + (uint32_t)T.h;
    x.a4 = ld64s(T.k4, F.k4, r4 * 128u);
    x.s4 = ld16s(T.ks4, F.k4s, r4 * 16u);
  }
}

template <int FETCH, int G8, bool BF16>
KVT_DEV void fetch_v_tile(const Tier& T, const int32_t* lpages, int t2, const FetchLane& F, int tp, int db, RawV& x) {
  constexpr uint32_t NG8 = kD / G8;
  const uint32_t H = (uint32_t)T.H;
  if constexpr (FETCH == kFetchKeys) {
    x = fetch_v<G8, BF16>(T, lpages, t2 + tp, db);
  } else if constexpr (FETCH == kFetchBf16) {
    const uint32_t so = (uint32_t)(t2 * T.vb_n + T.h * T.vb_h) * 2u;
    x.a[0] = ld128s(T.vb, F.v8, so);
    x.a[1] = ld128s(T.vb, F.v8, so + 16u * (uint32_t)T.vb_n * 2u);
  } else if constexpr (FETCH == kFetchInt8) {
    const uint32_t r8 = (uint32_t)((t2 & T.rmask) * T.H + T.h);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      x.a8[t] = ld64s(T.rv, F.v8, (r8 + 16u * t * H) * 256u);
      x.s8[t] = ld16s(T.rvs, F.v8s, (r8 + 16u * t * H) * NG8 * 2u);
    }
  } else if constexpr (FETCH == kFetchInt4) {
    const uint32_t pg = (uint32_t)__builtin_amdgcn_readfirstlane(lpages[min(t2 >> 6, kMaxLdsPages - 1)]);
    const uint32_t r4 = (pg * kPage + (uint32_t)(t2 & (kPage - 1))) * H + (uint32_t)T.h;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      x.c4[t] = ld32s(T.v4, F.v4, (r4 + 16u * t * H) * 128u);
      x.s4[t] = ld16s(T.vs4, F.v4s, (r4 + 16u * t * H) * 16u);
    }
  }
}

// Codes -> exact bf16 rows.  A code c with offset o (c + o >= 0) is placed in the mantissa of an fp16 "magic" value
// h = 1024 + (c + o) (bits 0x6400 | (c + o)); v_fma_mix_f32 converts h and the fp16 scale s to fp32 and computes
// h * s - (1024 + o) * s in one rounding, whose exact value c * s is representable (4 or 8 bits times the scale's
// 11), so the result is the oracle's fp32 product; v_cvt_pk_bf16_f32 then rounds it to nearest even.
// V operands (VH) are fp16 for the P.V products: the magic value 0x4800 | (c + o) = 8 + (c + o) / 128 gives the
// exact product c * s / 128, v_cvt_pk_bf16_f32 rounds it (rounding commutes with the power-of-two scale) and
// v_cvt_pk_f16_f32 carries the 8-bit significand over unchanged: fp16 holds bf16(c * s) / 128 exactly for
// |bf16(c * s)| in [2^-10, 65504 * 128] (every clamp-regime value, up to bf16(127 * 65504) / 128 = 65024, included;
// below 2^-7 as subnormals of spacing 2^-24), and to within 2^-18 (in units of the row) below 2^-10.
KVT_DEV float mix(uint32_t w, int half, _Float16 s, float c) {
  return fmaf((float)__builtin_bit_cast(h2v, w)[half], (float)s, c);
}
// (x & m) | o in one VALU instruction (VOP3 takes no literal and at most one scalar operand: m from a scalar
// register, o from a vector register)
KVT_DEV uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(o));
  return r;
}
KVT_DEV _Float16 half_of(uint32_t bits) { return __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu)); }

// fp16 pair, round to nearest even (one v_cvt_pk_f16_f32): lo in bits 0-15.
KVT_DEV uint32_t h2(float lo, float hi) { return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){lo, hi}, h2v)); }
// fp16 pair of bf16(lo), bf16(hi).
KVT_DEV uint32_t bf_h2(float lo, float hi) {
  const uint32_t b = bf2(lo, hi);
  return h2(__uint_as_float(b << 16), __uint_as_float(b & 0xffff0000u));
}
template <bool VH>
KVT_DEV uint32_t pair_out(float lo, float hi) { return VH ? bf_h2(lo, hi) : bf2(lo, hi); }
// -(magic base + o) * s: INT4 o = 8, INT8 o = 128
template <bool VH>
KVT_DEV float bias4(_Float16 s) { return (VH ? -8.0625f : -1032.0f) * (float)s; }
template <bool VH>
KVT_DEV float bias8(_Float16 s) { return (VH ? -9.0f : -1152.0f) * (float)s; }

// 8 INT4 codes (one dword; byte j = channel 2 j in the low nibble, 2 j + 1 in the high one, stored as code + 8) ->
// 4 pairs in channel order; c = bias4(s).  Word A holds channels 0 / 4, B 1 / 5, C 2 / 6, D 3 / 7.
template <bool VH>
KVT_DEV void int4_pairs(uint32_t w, _Float16 s, float c, uint32_t out[4]) {
  constexpr uint32_t m = VH ? 0x48004800u : 0x64006400u;
  const uint32_t A = and_or(w, 0x000F000Fu, m), B = and_or(w >> 4, 0x000F000Fu, m);
  const uint32_t C = and_or(w >> 8, 0x000F000Fu, m), D = and_or(w >> 12, 0x000F000Fu, m);
  out[0] = pair_out<VH>(mix(A, 0, s, c), mix(B, 0, s, c));
  out[1] = pair_out<VH>(mix(C, 0, s, c), mix(D, 0, s, c));
  out[2] = pair_out<VH>(mix(A, 1, s, c), mix(B, 1, s, c));
  out[3] = pair_out<VH>(mix(C, 1, s, c), mix(D, 1, s, c));
}

// 4 INT8 codes (one dword) -> 2 pairs; c = bias8(s).  u = code + 128 per byte; e holds channels 0 / 2, o 1 / 3.
template <bool VH>
KVT_DEV void int8_pairs(uint32_t w, _Float16 s, float c, uint32_t out[2]) {
  constexpr uint32_t m = VH ? 0x48484848u : 0x64646464u;
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t e = __builtin_amdgcn_perm(m, u, 0x04020400u);
  const uint32_t o = __builtin_amdgcn_perm(m, u, 0x04030401u);
  out[0] = pair_out<VH>(mix(e, 0, s, c), mix(o, 0, s, c));
  out[1] = pair_out<VH>(mix(e, 1, s, c), mix(o, 1, s, c));
}

// bf16 source pair -> fp16 pair of the values / 128 (exact as above)
KVT_DEV uint32_t bf_src_h2(uint32_t w) {
  return h2(__uint_as_float(w << 16) * 0.0078125f, __uint_as_float(w & 0xffff0000u) * 0.0078125f);
}

// Tier of a tile's dequantization: every key INT4, every key INT8, per key (the tile straddles hot_start), the bf16
// source, or no tile (kTierNone).
enum { kTierInt4 = 0, kTierInt8 = 1, kTierMixed = 2, kTierBf16 = 3, kTierNone = 4 };
template <int N>
struct TierTag {
  static constexpr int value = N;
};

KVT_DEV void k_int8(const RawK& x, uint32_t o[8]) {
  const uint32_t w[4] = {x.b.x, x.b.y, x.b.z, x.b.w};
  const _Float16 s = half_of(x.s8);
  const float c = bias8<false>(s);
#pragma unroll
  for (int i = 0; i < 4; ++i) int8_pairs<false>(w[i], s, c, o + 2 * i);
}
KVT_DEV void k_int4(const RawK& x, uint32_t o[8]) {
  const _Float16 s = half_of(x.s4);
  const float c = bias4<false>(s);
  int4_pairs<false>(x.a4.x, s, c, o);
  int4_pairs<false>(x.a4.y, s, c, o + 4);
}

// K row fragment -> LDS (bf16, natural order): channels 16 dc .. 16 dc + 15 of key row `key` (2 chunks).
template <int TIER>
KVT_DEV void store_k(const RawK& x, uint8_t* row, int key, int dc) {
  uint32_t o[8];
  if constexpr (TIER == kTierBf16) {
    const uint32_t w[8] = {x.a.x, x.a.y, x.a.z, x.a.w, x.b.x, x.b.y, x.b.z, x.b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = w[i];
  } else if constexpr (TIER == kTierInt8) {
    k_int8(x, o);
  } else if constexpr (TIER == kTierInt4) {
    k_int4(x, o);
  } else {
    if (x.hot)
      k_int8(x, o);
    else
      k_int4(x, o);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
    *reinterpret_cast<uint4*>(row + k_chunk(key, 2 * dc + i)) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2],
                                                                          o[4 * i + 3]);
}

KVT_DEV void v_int8(const RawV& x, int t, uint32_t o[4]) {
  const _Float16 s = half_of(x.s8[t]);
  const float cc = bias8<true>(s);
  int8_pairs<true>(x.a8[t].x, s, cc, o);
  int8_pairs<true>(x.a8[t].y, s, cc, o + 2);
}
KVT_DEV void v_int4(const RawV& x, int t, uint32_t o[4]) {
  const _Float16 s = half_of(x.s4[t]);
  const float cc = bias4<true>(s);
  int4_pairs<true>(x.c4[t], s, cc, o);
}

// 8 channels of one V row -> 4 fp16 pairs of the values / 128 (natural order).
template <int TIER>
KVT_DEV void v_row8(const RawV& x, int t, uint32_t o[4]) {
  if constexpr (TIER == kTierBf16) {
    o[0] = bf_src_h2(x.a[t].x), o[1] = bf_src_h2(x.a[t].y), o[2] = bf_src_h2(x.a[t].z), o[3] = bf_src_h2(x.a[t].w);
  } else if constexpr (TIER == kTierInt8) {
    v_int8(x, t, o);
  } else if constexpr (TIER == kTierInt4) {
    v_int4(x, t, o);
  } else {
    if (x.hot[t])
      v_int8(x, t, o);
    else
      v_int4(x, t, o);
  }
}

// 8 channels of keys tp and tp + 16 -> their V rows (16 bytes each).
template <int TIER>
KVT_DEV void store_v(const RawV& x, uint8_t* vrows, int db, int tp) {
  uint32_t a[4], b[4];
  v_row8<TIER>(x, 0, a);
  v_row8<TIER>(x, 1, b);
  *reinterpret_cast<uint4*>(vrows + tp * kVRow + 16 * db) = make_uint4(a[0], a[1], a[2], a[3]);
  *reinterpret_cast<uint4*>(vrows + (tp + 16) * kVRow + 16 * db) = make_uint4(b[0], b[1], b[2], b[3]);
}

// Tile it + 1's rows are converted in pieces, one per matrix step of tile it (the loops below fence every step with
// sched_barrier, so each piece issues between two groups of products instead of in one run of vector instructions).
// K: 8 steps beside the score products; the rows go to LDS in the two steps after the conversion, and the codes of
// tile it + 2 are fetched at step kFetchK.  V: 16 steps beside P.V, likewise with kFetchV; each thread converts
// 8 channels of two keys and stores them as two 16-byte pieces of the row-major V tile.
template <int TIER>
constexpr int kConvK = TIER == kTierInt8 ? 4 : TIER == kTierInt4 ? 2 : 1;   // conversion steps of a K fragment
template <int TIER>
constexpr int kFetchK = kConvK<TIER> + 2;
template <int TIER>
constexpr int kConvV = TIER == kTierInt8 ? 4 : TIER == kTierInt4 ? 2 : 1;
template <int TIER>
constexpr int kFetchV = kConvV<TIER> + 2;

KVT_DEV uint32_t word_of(const uint4& w, int j) { return j == 0 ? w.x : j == 1 ? w.y : j == 2 ? w.z : w.w; }

template <int TIER>
KVT_DEV void k_step(int j, const RawK& x, uint32_t o[8], uint8_t* row, int key, int dc) {
  if constexpr (TIER == kTierInt8) {
    if (j < 4) {
      const _Float16 s = half_of(x.s8);
      int8_pairs<false>(word_of(x.b, j), s, bias8<false>(s), o + 2 * j);
    }
  } else if constexpr (TIER == kTierInt4) {
    if (j < 2) {
      const _Float16 s = half_of(x.s4);
      int4_pairs<false>(j == 0 ? x.a4.x : x.a4.y, s, bias4<false>(s), o + 4 * j);
    }
  } else if constexpr (TIER == kTierBf16) {
    if (j == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = word_of(x.a, i), o[4 + i] = word_of(x.b, i);
    }
  } else {
    if (j == 0) {
      if (x.hot)
        k_int8(x, o);
      else
        k_int4(x, o);
    }
  }
  constexpr int w0 = kConvK<TIER>;
  if (j == w0 || j == w0 + 1) {
    const int i = j - w0;
    *reinterpret_cast<uint4*>(row + k_chunk(key, 2 * dc + i)) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2],
                                                                          o[4 * i + 3]);
  }
}

template <int TIER>
KVT_DEV void v_step(int j, const RawV& x, uint32_t a[4], uint32_t b[4], uint8_t* vrows, int db, int tp) {
  if constexpr (TIER == kTierInt8) {
    if (j < 4) {
      const int t = j >> 1, hw = j & 1;
      const _Float16 s = half_of(x.s8[t]);
      int8_pairs<true>(hw ? x.a8[t].y : x.a8[t].x, s, bias8<true>(s), (t ? b : a) + 2 * hw);
    }
  } else if constexpr (TIER == kTierInt4) {
    if (j < 2) v_int4(x, j, j ? b : a);
  } else {
    if (j == 0) {
      v_row8<TIER>(x, 0, a);
      v_row8<TIER>(x, 1, b);
    }
  }
  constexpr int w0 = kConvV<TIER>;
  if (j == w0) *reinterpret_cast<uint4*>(vrows + tp * kVRow + 16 * db) = make_uint4(a[0], a[1], a[2], a[3]);
  if (j == w0 + 1) *reinterpret_cast<uint4*>(vrows + (tp + 16) * kVRow + 16 * db) = make_uint4(b[0], b[1], b[2], b[3]);
}

constexpr int kAheadK = 2, kAheadV = 4;   // LDS operand reads issued this many matrix steps ahead
constexpr int kWaves = 8;               // 2 per SIMD: each wavefront 16 rows (16 / gs queries x gs heads)

// The queries of one query tile (qb queries of sequence b) and the keys they see.
struct QTile {
  int64_t qs, q_len, L, q_pos0, qt0, key_end;
  int ntiles;   // key tiles of 32 positions (0: no query of the sequence falls in this tile)
};
KVT_DEV QTile qtile_of(const void* cu_q, int cu_q_is_int64, const int32_t* kv_lens, int b, int qt, int qb) {
  QTile Q;
  Q.qs = cu_q_is_int64 ? reinterpret_cast<const int64_t*>(cu_q)[b] : (int64_t)reinterpret_cast<const int32_t*>(cu_q)[b];
  const int64_t qe = cu_q_is_int64 ? reinterpret_cast<const int64_t*>(cu_q)[b + 1]
                                   : (int64_t)reinterpret_cast<const int32_t*>(cu_q)[b + 1];
  Q.q_len = qe - Q.qs;
  Q.L = kv_lens[b];
  Q.q_pos0 = Q.L - Q.q_len;   // position of the chunk's first query
  Q.qt0 = (int64_t)qt * qb;
  Q.key_end = min(Q.L, Q.q_pos0 + min(Q.q_len, Q.qt0 + qb));   // keys visible to the tile's last query
  Q.ntiles = Q.qt0 < Q.q_len && Q.key_end > 0 ? (int)((Q.key_end + kT - 1) / kT) : 0;
  return Q;
}

// One segment: key tiles [i0, i1) of query tile Q of (sequence b, KV head h).  nseg segments make up the tile, this
// is number `ord`; with nseg > 1 their states go through slots[0 .. nseg) and *count (see kSlotO), and the
// segment that finishes last writes the output.
template <int G8, bool BF16>
KVT_DEV void attend_segment(const KVSrc& S, const uint16_t* q, int64_t sq_n, int64_t sq_h, const QTile& Q, int b,
                            int h, int H, int gs, int i0, int i1, int nseg, int ord, float* slots, int32_t* count,
                            float scale, void* out, int out_f32, int64_t so_n, int64_t so_h) {
  __shared__ Lds lds;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, kb = lane >> 4;
  const int qpw = 16 / gs;   // queries per wavefront
  const int64_t qs = Q.qs, q_len = Q.q_len, L = Q.L, q_pos0 = Q.q_pos0, qt0 = Q.qt0, key_end = Q.key_end;
  constexpr uint32_t NG8 = kD / G8;
  bool pages_fit = true;   // the paged key range fits the kMaxLdsPages page ids staged in LDS
  Tier T;
  T.H = H;
  T.h = h;
  T.key_end = (int)key_end;
  T.kb_n = (int)S.kb_n;
  T.kb_h = (int)S.kb_h;
  T.vb_n = (int)S.vb_n;
  T.vb_h = (int)S.vb_h;
  if constexpr (BF16) {
    const uint32_t kbytes = (uint32_t)(((S.kb_rows - 1) * S.kb_n + (int64_t)(H - 1) * S.kb_h + kD) * 2);
    const uint32_t vbytes = (uint32_t)(((S.kb_rows - 1) * S.vb_n + (int64_t)(H - 1) * S.vb_h + kD) * 2);
    T.kb = make_rsrc(S.kb, kbytes);
    T.vb = make_rsrc(S.vb, vbytes);
    T.hs = 0;
    T.rmask = 0;
  } else {
    const int64_t R = S.ring_len[b];
    const int64_t rbase = S.ring_base[b];
    T.hs = (int)min(max(max(S.ring_start[b], L - R), (int64_t)0), L);
    T.rmask = (int)(R - 1);
    T.k4 = make_rsrc(S.k4, S.pool_rows * (uint32_t)H * 128u);
    T.v4 = make_rsrc(S.v4, S.pool_rows * (uint32_t)H * 128u);
    T.ks4 = make_rsrc(S.ks4, S.pool_rows * (uint32_t)H * 16u);
    T.vs4 = make_rsrc(S.vs4, S.pool_rows * (uint32_t)H * 16u);
    T.rk = make_rsrc(S.rk + rbase * H * kD, (uint32_t)R * (uint32_t)H * kD);
    T.rv = make_rsrc(S.rv + rbase * H * kD, (uint32_t)R * (uint32_t)H * kD);
    T.rks = make_rsrc(S.rks + rbase * H * NG8, (uint32_t)R * (uint32_t)H * NG8 * 2u);
    T.rvs = make_rsrc(S.rvs + rbase * H * NG8, (uint32_t)R * (uint32_t)H * NG8 * 2u);
    // page ids of the paged key range, once per block
    const int64_t need = (min((int64_t)T.hs, key_end) + kPage - 1) / kPage;
    pages_fit = need <= kMaxLdsPages;
    const int64_t npg = min(need, (int64_t)kMaxLdsPages);
    // (through a buffer resource over the sequence's row: 32-bit lane offsets, no per-lane 64-bit address kept live)
    const Rsrc pt = make_rsrc(S.page_table + b * S.pt_stride, (uint32_t)npg * 4u);
    for (int i = tid; i < (int)npg; i += 64 * kWaves) lds.pages[i] = (int32_t)ld32(pt, 4u * (uint32_t)i);
    if (tid == 0 && npg == 0) lds.pages[0] = 0;
  }
  __syncthreads();

  // dequantization, the same for every thread t: 16 channels (16 (t & 15) ..) of K row t >> 4, and 8 channels
  // (8 (t >> 4) ..) of V rows 2 (t & 15), 2 (t & 15) + 1
  const int tk = tid >> 4, dc = tid & 15;
  const int tp = tid & 15, db = tid >> 4;
  constexpr int kFirst = BF16 ? kTierBf16 : kTierMixed;
  // the first tile's codes go out before the Q rows, so that storing the tile waits for its own loads only
  RawK rk_next = fetch_k<G8, BF16>(T, lds.pages, i0 * kT + tk, dc);
  RawV rv_next = fetch_v<G8, BF16>(T, lds.pages, i0 * kT + tp, db);

  // ---- Q operands: row j of the wavefront's 16 = query qt0 + qpw wave + j / gs, head j % gs; channels
  // 32 st + 8 kb .. + 7 of the row in one 16-byte load per st (the host checks the 16-byte alignment)
  bf8 qop[8];
  int64_t qpos;   // position of this lane's query row (as the S^T column)
  // a paged range beyond the staged page ids would read clamped pages: the tile's outputs become NaN instead (NaN
  // scores give NaN weights, sums and outputs), never silently wrong keys
  const float qmul = pages_fit ? scale * kLog2e : __builtin_nanf("");
  {
    int gs_q = gs;                      // (computed per segment, not hoisted to the kernel start: see the output)
    asm volatile("" : "+s"(gs_q));
    const int rq = n16 / gs_q, hq = n16 - rq * gs_q;
    const int64_t qi = qt0 + (int64_t)qpw * wave + rq;
    const bool ok = rq < qpw && qi < q_len;
    qpos = q_pos0 + qi;
    const uint16_t* qr = q + (qs + (ok ? qi : 0)) * sq_n + (int64_t)(h * gs + (ok ? hq : 0)) * sq_h + 8 * kb;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const u4v w = ok ? *reinterpret_cast<const u4v*>(qr + 32 * st) : u4v{0u, 0u, 0u, 0u};
      qop[st] = __builtin_bit_cast(bf8, w);
    }
  }

  f4 acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  store_k<kFirst>(rk_next, lds.k[i0 & 1] + tk * kKPitch, tk, dc);
  store_v<kFirst>(rv_next, lds.v[i0 & 1], db, tp);
  rk_next = fetch_k<G8, BF16>(T, lds.pages, (i0 + 1) * kT + tk, dc);   // (past the end it rereads the last key)
  rv_next = fetch_v<G8, BF16>(T, lds.pages, (i0 + 1) * kT + tp, db);
  __syncthreads();
  const int qmin = (int)(q_pos0 + qt0);   // the block's first query position: tiles below it need no causal mask
  const int qp = (int)qpos, kend = (int)key_end;
  // One iteration per key tile it.  Tile it + 1's rows (codes loaded during tile it - 1) go into the other buffer
  // beside this tile's products, a piece per matrix step: its K rows beside the score products, its V rows beside
  // P.V; tile it + 2's codes go out during the same steps.  The body is specialized on the tier of tile it + 1;
  // tiers change monotonically along the keys (INT4 tiles, at most one tile that straddles hot_start, INT8 tiles),
  // so the iterations run as consecutive loops with one code path each.
  // LDS read offsets of this lane's MFMA operands, split into a per-lane part (computed once) and a constant:
  // K chunk 4 st + kb of key row n16 sits at 256 (st >> 2) + koff[st & 3] (the swizzle n16 only touches the low
  // four chunk bits); the V reads of dims 16 c .. at vlane + 32 c (keys 4 kb + (n16 >> 2)) and + 16 rows
  uint32_t koff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) koff[j] = k_chunk(n16, 4 * j + kb);
  const uint32_t vlane = (uint32_t)(4 * kb + (n16 >> 2)) * kVRow + 8u * (uint32_t)(n16 & 3);
  const FetchLane FL = fetch_lane<G8, BF16>(T, tk, dc, tp, db);
  int it = i0;
  auto body = [&](auto tag, auto ftag) {
    constexpr int TIER = decltype(tag)::value;
    constexpr int FETCH = decltype(ftag)::value;
    const int t0 = it * kT;
    const int cb = it & 1;
    const int t2 = t0 + 2 * kT;
    // ---- S^T = K Q^T: lane holds keys t0 + 16 nt + 4 kb + r of query row n16 (unscaled).  Step st: the two
    // products of k-slice st, the K operands of step st + kAheadK read from LDS, one piece of tile it + 1's K rows.
    float s[2][4];
    {
      constexpr bool kDq = TIER != kTierNone;
      const uint8_t* kbuf = lds.k[cb];
      uint8_t* krow_next = lds.k[cb ^ 1] + tk * kKPitch;
      uint32_t ko[8];
      bf8 kf[8][2];
      f4 d[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      auto kread = [&](int st) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          kf[st][nt] = __builtin_bit_cast(
              bf8, *reinterpret_cast<const u4v*>(kbuf + (16 * nt + n16) * kKPitch + koff[st & 3] + 256 * (st >> 2)));
      };
#pragma unroll
      for (int st = 0; st < kAheadK; ++st) kread(st);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st + kAheadK < 8) kread(st + kAheadK);
        d[0] = mfma(kf[st][0], qop[st], d[0]);
        d[1] = mfma(kf[st][1], qop[st], d[1]);
        if constexpr (kDq) {
          k_step<TIER>(st, rk_next, ko, krow_next, tk, dc);
          if (st == kFetchK<TIER>) fetch_k_tile<FETCH, G8, BF16>(T, lds.pages, t2, FL, tk, dc, rk_next);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[nt][r] = d[nt][r];
    }
    // the softmax (scores -> row max -> exponentials -> P) is the chain every P.V product waits for: at a higher
    // wave priority its instructions issue ahead of the other wavefront's conversion and products on the SIMD
    // (3 % less time per prompt than without)
    __builtin_amdgcn_s_setprio(1);
    // causal / end mask, only on the tiles that reach the block's first query or the key end
    if (t0 + kT > qmin || t0 + kT > kend) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int kp = t0 + 16 * nt + 4 * kb + r;
          s[nt][r] = (kp <= qp && kp < kend) ? s[nt][r] : -INFINITY;
        }
    }
    // ---- online softmax; P as the A operand of P.V (fp16, rounded to nearest even; the row sum l adds the rounded
    // values, so the weights of the output are exactly the weights of the products)
    h8 pa;
    {
      float mloc = vmax3(vmax3(s[0][0], s[0][1], s[0][2]), s[0][3], s[1][0]);
      mloc = vmax(vmax3(mloc, s[1][1], s[1][2]), s[1][3]) * qmul;   // this lane's 8 keys, log2 units
      // lazy rescale: the reference max moves (and the accumulators are rescaled) only when a row's max exceeds it
      // by more than 8 (log2 units), so P = 2^(s qmul - m) <= 256.  A row's max exceeds it iff one of the row's four
      // lanes (n16 + 16 kb) does, so the cross-lane max is taken only then, for every row (m stays uniform per row).
      if (__any(mloc > m_run + 8.0f)) {
        const float m_new = vmax(m_run, vmax_xor16_32(mloc));
        const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        float arow[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
        for (int c = 0; c < 16; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][i] *= arow[i];
        m_run = m_new;
      }
      // rows with no visible key yet keep m = -inf and contribute nothing
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[nt][r] = __builtin_amdgcn_exp2f(fmaf(s[nt][r], qmul, -m_use));
      uint32_t hw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hw[i] = h2(s[i >> 1][2 * (i & 1)], s[i >> 1][2 * (i & 1) + 1]);
        l_run = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2v, hw[i]), h2v{1.0f16, 1.0f16}, l_run, false);
      }
      pa = __builtin_bit_cast(h8, u4v{hw[0], hw[1], hw[2], hw[3]});
    }
    __builtin_amdgcn_s_setprio(0);
    // ---- O += P V / 128: B = dim 16 c + n16 of keys {4 kb .. +3, 16 + 4 kb .. +3}: two transposing 8-byte reads.
    // Step c: the product of dims 16 c .., the V operand of step c + kAheadV read from LDS, one piece of tile
    // it + 1's V rows.
    {
      constexpr bool kDq = TIER != kTierNone;
      const uint8_t* vbuf = lds.v[cb];
      uint8_t* v_next = lds.v[cb ^ 1];
      uint32_t va[4], vb[4];
      h8 vf[16];
      auto vread = [&](int c) {
        const uint32_t a0 = (uint32_t)(uintptr_t)(vbuf + vlane + 32 * c);
        const auto lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(uintptr_t)a0);
        const auto hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(uintptr_t)(a0 + 16u * kVRow));
        const uint2 lw = __builtin_bit_cast(uint2, lo), hw = __builtin_bit_cast(uint2, hi);
        vf[c] = __builtin_bit_cast(h8, u4v{lw.x, lw.y, hw.x, hw.y});
      };
#pragma unroll
      for (int c = 0; c < kAheadV; ++c) vread(c);
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        if (c + kAheadV < 16) vread(c + kAheadV);
        acc[c] = mfma(pa, vf[c], acc[c]);
        if constexpr (kDq) {
          v_step<TIER>(c, rv_next, va, vb, v_next, db, tp);
          if (c == kFetchV<TIER>) fetch_v_tile<FETCH, G8, BF16>(T, lds.pages, t2, FL, tp, db, rv_next);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();   // tile it + 1 is in LDS for everyone; nobody reads this tile's buffer any more
    ++it;
  };
  // Iteration it converts tile it + 1 and fetches tile it + 2; a whole-tile fetch needs tile it + 2 to end at or
  // before the key end (it + 3 <= kend / kT) and, for INT4, at or before hot_start.
  const int nd = i1 - 1;               // iterations that convert a tile (tile it + 1)
  const int me = kend / kT - 2;        // iterations whose tile it + 2 ends at or before the key end
  using KeysF = TierTag<kFetchKeys>;
  // s_waitcnt vmcnt(0) before a loop: loads of an earlier loop still in flight into registers this loop reuses would
  // otherwise make the loop header's wait state force vmcnt(0) inside the body, on every iteration
  auto drain = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };
  if constexpr (BF16) {
    while (it < min(nd, me)) body(TierTag<kTierBf16>{}, TierTag<kFetchBf16>{});
    drain();
    while (it < nd) body(TierTag<kTierBf16>{}, KeysF{});
  } else {
    const int n4 = T.hs / kT;          // tiles entirely below hot_start
    while (it < min(min(n4 - 1, nd), min(me, n4 - 2))) body(TierTag<kTierInt4>{}, TierTag<kFetchInt4>{});
    drain();
    while (it < min(n4 - 1, nd)) body(TierTag<kTierInt4>{}, KeysF{});
    if ((T.hs & (kT - 1)) != 0 && it == n4 - 1 && it < nd) body(TierTag<kTierMixed>{}, KeysF{});
    drain();
    if (T.rmask >= kT - 1)
      while (it < min(nd, me)) body(TierTag<kTierInt8>{}, TierTag<kFetchInt8>{});
    drain();
    while (it < nd) body(TierTag<kTierInt8>{}, KeysF{});
  }
  drain();
  while (it < i1) body(TierTag<kTierNone>{}, TierTag<kFetchNone>{});

  // ---- the row sums of accumulator rows 4 kb + i (m_run and l are uniform over the four lanes of a row)
  const float l = sum_xor16_32(l_run);
  float lrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lrow[i] = __shfl(l, 4 * kb + i, 64);
  if (nseg > 1) {   // ---- publish this segment's state, or merge every segment's if it is the last
    // (lane-derived slot offsets computed here, not hoisted to the kernel start and kept live across the loops)
    int wave_t = wave, n16_t = n16;
    asm volatile("" : "+s"(wave_t), "+v"(n16_t));
    const Rsrc rs = make_rsrc(slots, (uint32_t)nseg * kSlotFloats * 4u);
    const uint32_t olane = (uint32_t)(wave_t * 16 * 64 + lane) * 16u;   // + 1024 c: this lane's O of column block c
    if (tid == 0) lds.flag = ld_dev_i32(count) == nseg - 1;   // every other segment is in: merge at once
    __syncthreads();
    if (lds.flag == 0) {
      const uint32_t mine = (uint32_t)ord * kSlotFloats * 4u;
#pragma unroll
      for (int c = 0; c < 16; ++c)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, acc[c]), rs, (int)(mine + olane + 1024u * c),
                                               0, kSc1);
      if (kb == 0) {
        st_dev(&slots[ord * kSlotFloats + kSlotO + 2 * (16 * wave_t + n16_t)], m_run);
        st_dev(&slots[ord * kSlotFloats + kSlotO + 2 * (16 * wave_t + n16_t) + 1], l);
      }
      drain();          // the stores have reached the coherence point
      __syncthreads();  // (and every thread has read lds.flag)
      if (tid == 0) lds.flag = add_dev_i32(count, 1) == nseg - 1;
      __syncthreads();
      if (lds.flag == 0) return;   // a later segment merges
    }
    if (tid == 0) st_dev_i32(count, 0);   // every segment has counted: ready for the next call
    // merge: weight of segment o in row r 2^(m_o - M), M the max over the segments (log2 units; -inf: no visible
    // key); sums over o = 0 .. nseg - 1 in order (this segment's state from registers, the others' from their
    // slots), so the result does not depend on which segment merges
    float mo[4], M[4], Ls[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mo[i] = __shfl(m_run, 4 * kb + i, 64);
      M[i] = -INFINITY;
      Ls[i] = 0.f;
    }
    const int mlrow = kSlotO + 2 * (16 * wave_t + 4 * kb);
    if (nseg == 2) {   // (the common case) every load of the other segment at once
      const int oth = 1 - ord;
      float mx[4], lx[4];
      f4 x[16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        mx[i] = ld_dev(&slots[oth * kSlotFloats + mlrow + 2 * i]);
        lx[i] = ld_dev(&slots[oth * kSlotFloats + mlrow + 2 * i + 1]);
      }
#pragma unroll
      for (int c = 0; c < 16; ++c)
        x[c] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                          rs, (int)((uint32_t)oth * kSlotFloats * 4u + olane + 1024u * c), 0, kSc1));
      float w0[4], w1[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float m0 = ord == 0 ? mo[i] : mx[i], m1 = ord == 0 ? mx[i] : mo[i];
        const float mm = fmaxf(m0, m1);
        w0[i] = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - mm);
        w1[i] = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
        const float l0 = ord == 0 ? lrow[i] : lx[i], l1 = ord == 0 ? lx[i] : lrow[i];
        lrow[i] = fmaf(w1[i], l1, w0[i] * l0);
      }
      if (ord == 0) {
#pragma unroll
        for (int c = 0; c < 16; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][i] = fmaf(w1[i], x[c][i], w0[i] * acc[c][i]);
      } else {
#pragma unroll
        for (int c = 0; c < 16; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[c][i] = fmaf(w1[i], acc[c][i], w0[i] * x[c][i]);
      }
    } else {
      for (int o = 0; o < nseg; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          M[i] = fmaxf(M[i], o == ord ? mo[i] : ld_dev(&slots[o * kSlotFloats + mlrow + 2 * i]));
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {   // column blocks in two halves of 8
        f4 O[8];
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) O[cc] = f4{0.f, 0.f, 0.f, 0.f};
        for (int o = 0; o < nseg; ++o) {
          const bool me = o == ord;
          float wg[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float m = me ? mo[i] : ld_dev(&slots[o * kSlotFloats + mlrow + 2 * i]);
            wg[i] = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M[i]);
            if (hf == 0) Ls[i] += wg[i] * (me ? lrow[i] : ld_dev(&slots[o * kSlotFloats + mlrow + 2 * i + 1]));
          }
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {
            const int c = 8 * hf + cc;
            const f4 xo = me ? acc[c]
                             : __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          rs, (int)((uint32_t)o * kSlotFloats * 4u + olane + 1024u * c),
                                                          0, kSc1));
#pragma unroll
            for (int i = 0; i < 4; ++i) O[cc][i] += wg[i] * xo[i];
          }
        }
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) acc[8 * hf + cc] = O[cc];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) lrow[i] = Ls[i];
    }
  }
  // ---- normalize and store: accumulator row r = 4 kb + i = query qt0 + qpw wave + r / gs, head r % gs;
  // column n16 of block c = dim 16 c + n16
  // (one correctly rounded division per row: 128 / l, exact for a single visible key, where l = 1)
  // The rows' (query, head) split is computed here, after the key tiles: gs passes through an empty asm statement,
  // so the compiler cannot hoist these divisions to the kernel start, where their results stayed live across every
  // loop and spilled.
  int gs_t = gs;
  void* out_t = out;
  asm volatile("" : "+s"(gs_t), "+s"(out_t));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * kb + i, rq = r / gs_t, hq = r - rq * gs_t;
    const int64_t qi = qt0 + (int64_t)qpw * wave + rq;
    if (rq < qpw && qi < q_len) {
      const int64_t o0 = (qs + qi) * so_n + (int64_t)(h * gs_t + hq) * so_h;
      const float rl = 128.0f / lrow[i];
      if (out_f32) {
        float* orow = reinterpret_cast<float*>(out_t) + o0;
#pragma unroll
        for (int c = 0; c < 16; ++c) orow[16 * c + n16] = acc[c][i] * rl;
      } else {
        uint16_t* orow = reinterpret_cast<uint16_t*>(out_t) + o0;
#pragma unroll
        for (int c = 0; c < 16; ++c) orow[16 * c + n16] = bf16_rne(acc[c][i] * rl);
      }
    }
  }
}

// Spread launches: the work of all query tiles, laid end to end (items j = (sequence, KV head) j / n_qtiles, query
// tile j % n_qtiles, in that order) in units of one key tile, is cut into equal shares, one per block; a block
// walks the segments of its share (the end of one query tile, whole tiles, the start of another).  An item costs
// kItemCost units (a segment's Q load, first tile and output: about what 8 key tiles take) followed by one unit per
// key tile, so a share of many short query tiles holds fewer key tiles.  Every block computes the same prefix sums
// of the item costs.  Block w takes units [T w / G, T (w + 1) / G); the block holding unit t is ((t + 1) G - 1) / T;
// a segment is a share's part of an item's key tile units.  Segment (item j, block w) uses slot j + w: that sum
// grows along the segments, so slots are distinct, at most n_items + G - 1 of them.
constexpr int kMaxItems = 4096;   // items of a spread launch (the prefix sums live in LDS)
constexpr int kItemCost = 8;      // units of an item before its key tiles
constexpr int kMinShare = 16;     // units per block at least: shorter launches use fewer blocks

template <int G8, bool BF16>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
prefill_mfma_kernel(KVSrc S, const uint16_t* q, int64_t sq_n, int64_t sq_h, const void* cu_q, int cu_q_is_int64,
                    const int32_t* kv_lens, int H, int gs, int n_qtiles, int bh_n, int spread, float* part,
                    int32_t* ctr, float scale, void* out, int out_f32, int64_t so_n, int64_t so_h) {
  static_assert(kWaves == 8, "slot layout");
  __shared__ int pfx[kMaxItems + 1];
  __shared__ int wsum[kWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qb = kWaves * (16 / gs);
  const int n_items = bh_n * n_qtiles;
  int w = (int)blockIdx.x, G = 0, j;
  int64_t pos = 0, e = 0, T = 0;
  if (spread) {
    // prefix sums of the item costs (units): thread t counts items per t .. per t + per - 1
    const int per = (n_items + 64 * kWaves - 1) / (64 * kWaves);   // <= 8
    int cnt[8], sum = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int jj = tid * per + k;
      cnt[k] = 0;
      if (k < per && jj < n_items) {
        const int bh = jj / n_qtiles, b = bh / H;
        const int nt = qtile_of(cu_q, cu_q_is_int64, kv_lens, b, jj - bh * n_qtiles, qb).ntiles;
        cnt[k] = nt > 0 ? kItemCost + nt : 0;
      }
      sum += cnt[k];
    }
    int x = sum;   // inclusive scan over the wavefront
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int base = 0;
    for (int v = 0; v < wave; ++v) base += wsum[v];
    int excl = base + x - sum;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int jj = tid * per + k;
      if (k < per && jj < n_items) pfx[jj] = excl;
      excl += cnt[k];
    }
    if (tid == 64 * kWaves - 1) pfx[n_items] = base + x;
    __syncthreads();
    T = pfx[n_items];
    if (T == 0) return;
    G = (int)min((int64_t)gridDim.x, max((int64_t)1, T / kMinShare));
    if (w >= G) return;
    pos = T * w / G;
    e = T * (w + 1) / G;
    int lo = 0, hi = n_items;   // the item holding unit pos: pfx[lo] <= pos < pfx[lo + 1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pfx[mid] <= pos) lo = mid; else hi = mid;
    }
    j = lo;
  } else {   // one block per item, the latest (heaviest) query tiles first
    j = (w % bh_n) * n_qtiles + n_qtiles - 1 - w / bh_n;
  }
  for (;;) {
    const int bh = j / n_qtiles, qt = j - bh * n_qtiles, b = bh / H, h = bh - b * H;
    const QTile Q = qtile_of(cu_q, cu_q_is_int64, kv_lens, b, qt, qb);
    int64_t p1 = Q.ntiles;
    int i0 = 0, nseg = 1, ord = 0;
    float* slots = nullptr;
    if (spread) {
      const int64_t t0 = pfx[j] + kItemCost;   // units of the item's key tiles: [t0, p1)
      p1 = pfx[j + 1];
      if (max(pos, t0) >= min(e, p1)) return;   // the share ends before the item's first key tile
      const int wf = (int)(((t0 + 1) * G - 1) / T);   // the blocks holding the item's first and last key tile
      const int wl = (int)((p1 * G - 1) / T);
      i0 = (int)(max(pos, t0) - t0);
      nseg = wl - wf + 1;
      ord = w - wf;
      slots = part + (int64_t)(j + wf) * kSlotFloats;
      p1 = min(e, p1) - t0;
    } else if (Q.ntiles == 0) {
      return;
    }
    attend_segment<G8, BF16>(S, q, sq_n, sq_h, Q, b, h, H, gs, i0, (int)p1, nseg, ord, slots,
                             ctr + (spread ? j : 0), scale, out, out_f32, so_n, so_h);
    if (!spread) return;
    p1 = pfx[j + 1];
    pos = min(e, p1);
    if (pos >= e) return;
    do ++j; while (pfx[j + 1] == pfx[j]);   // the next item with tiles (pos < e <= T: one exists)
    __syncthreads();                        // the segment's LDS is free again
  }
}

// query tiles of a launch, and the counter area at the start of the spread workspace: one int32 per possible item
// (kMaxItems), the same for every call, so the slots of one call never overlap the counters of another (a call with
// more items than the previous one would otherwise find that call's slot data in its counters and merge early)
int prefill_qtiles(int max_q, int H, int Hq) {
  const int qb = kWaves * (16 / (Hq / H));   // queries per block
  return (max_q + qb - 1) / qb;
}
constexpr int64_t kCounterBytes = (int64_t)kMaxItems * 4;   // 16 KB, a multiple of 256

}  // namespace

extern "C" {

int kvt_prefill_work_bytes(int batch, int H, int Hq, int max_q, int spread_blocks, int64_t* bytes) {
  if (bytes == nullptr || batch < 0 || H <= 0 || Hq % H != 0 || Hq / H > 16 || max_q < 0 || spread_blocks < 0)
    return KVT_EINVAL;
  if (spread_blocks == 0 || batch == 0 || max_q == 0) {
    *bytes = 0;
    return KVT_OK;
  }
  const int64_t n_items = (int64_t)batch * H * prefill_qtiles(max_q, H, Hq);
  if (n_items > kMaxItems || spread_blocks > (1 << 20)) return KVT_ERANGE;
  *bytes = kCounterBytes + (n_items + spread_blocks - 1) * kSlotFloats * 4;
  return KVT_OK;
}

int kvt_prefill_attn(const void* q, int64_t sq_n, int64_t sq_h, const void* cu_q, int cu_q_is_int64,
                     const void* kv_lens, int batch, int max_q, int H, int Hq, int D, int group8, const void* k4,
                     const void* v4, const void* ks4, const void* vs4, const void* rk, const void* rv,
                     const void* rks, const void* rvs, const void* ring_base, const void* ring_len,
                     const void* ring_start, const void* page_table, int64_t pt_stride, int64_t pool_rows,
                     const void* k_bf16, const void* v_bf16, int64_t kb_rows, int64_t kb_n, int64_t kb_h,
                     int64_t vb_n, int64_t vb_h, float scale, void* out, int out_f32, int64_t so_n, int64_t so_h,
                     int spread_blocks, void* work, int64_t work_bytes, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || D != kD || Hq / H > 16 || max_q < 0) return KVT_EINVAL;
  if (spread_blocks < 0) return KVT_EINVAL;
  // Q rows are read 8 channels (16 bytes) at a time
  if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || sq_n % 8 != 0 || sq_h % 8 != 0) return KVT_EINVAL;
  if ((k_bf16 == nullptr) != (v_bf16 == nullptr)) return KVT_EINVAL;
  const bool bf16 = k_bf16 != nullptr;
  // 32-bit byte offsets inside each buffer
  if (!bf16 && (pool_rows <= 0 || pool_rows * H * (kD / 2) > 0x7fffffffLL)) return KVT_ERANGE;
  if (bf16 && (kb_rows <= 0 || (kb_rows * kb_n + H * kb_h) * 2 > 0x7fffffffLL ||
               (kb_rows * vb_n + H * vb_h) * 2 > 0x7fffffffLL))
    return KVT_ERANGE;
  if (max_q == 0) return KVT_OK;
  KVSrc S{(const uint8_t*)k4,        (const uint8_t*)v4,       (const uint16_t*)ks4,    (const uint16_t*)vs4,
          (const int8_t*)rk,         (const int8_t*)rv,        (const uint16_t*)rks,    (const uint16_t*)rvs,
          (const int64_t*)ring_base, (const int32_t*)ring_len, (const int64_t*)ring_start,
          (const int32_t*)page_table, pt_stride,               (uint32_t)pool_rows,      (const uint16_t*)k_bf16,
          (const uint16_t*)v_bf16,   kb_n, kb_h, vb_n, vb_h, kb_rows};
  const int n_qtiles = prefill_qtiles(max_q, H, Hq);
  const int bh_n = batch * H;
  float* part = nullptr;
  int32_t* ctr = nullptr;
  if (spread_blocks > 0) {
    int64_t need = 0;
    const int rc = kvt_prefill_work_bytes(batch, H, Hq, max_q, spread_blocks, &need);
    if (rc != KVT_OK) return rc;
    if (work == nullptr || work_bytes < need) return KVT_EINVAL;
    ctr = static_cast<int32_t*>(work);
    part = reinterpret_cast<float*>(static_cast<char*>(work) + kCounterBytes);
  } else if ((int64_t)n_qtiles * bh_n > 0x7fffffffLL) {
    return KVT_ERANGE;
  }
  const dim3 grid((unsigned)(spread_blocks > 0 ? spread_blocks : n_qtiles * bh_n));
  hipStream_t st = (hipStream_t)stream;
#define KVT_PF(G, B)                                                                                              \
  hipLaunchKernelGGL((prefill_mfma_kernel<G, B>), grid, dim3(64 * kWaves), 0, st, S, (const uint16_t*)q, sq_n, sq_h, cu_q,  \
                     cu_q_is_int64, (const int32_t*)kv_lens, H, Hq / H, n_qtiles, bh_n, spread_blocks > 0, part, ctr,  \
                     scale, out, out_f32, so_n, so_h)
  if (bf16) {
    KVT_PF(64, true);
  } else if (group8 == 64) {
    KVT_PF(64, false);
  } else if (group8 == 256) {
    KVT_PF(256, false);
  } else {
    return KVT_EINVAL;
  }
#undef KVT_PF
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
