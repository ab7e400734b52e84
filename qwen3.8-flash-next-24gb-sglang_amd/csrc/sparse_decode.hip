// Sparse attention over selected positions of the quantized pools, fused: the selected positions of each query row
// are resolved (position -> slot through req_to_token -> tier through the owner table), dequantized exactly as the
// reference's compact gather does (bf16(q * s * sm), patches/kv_tiers.py:446-538) and attended in one pass, with no
// bf16 scratch.  Two entry points share the kernel:
//   * kvt_sparse_decode (one query row per request): the reference's decode gathers the top-k positions into that
//     scratch and runs FlashAttention-2 over it (sglang/qwen4exp-serving-73a255206f.patch:1832-1882).  A block takes
//     64 selected columns of one (request, KV head) and writes an unnormalized partial; kvt_decode_combine merges
//     the column splits as it merges the dense decode's.
//   * kvt_sparse_prefill (one query row per chunk query): the reference's paged prefix-chunk attention
//     sparse_gqa_fwd_interface_paged (patches/kv_paged_prefix.py:141-365).  A block takes every selected column of
//     one (query, KV head): query j of a chunk of q_len queries over a context of kv_len attends the valid entries
//     (0 <= idx < kv_len) among the first min(topk, j + kv_len - q_len + 1) of its index row
//     (patches/kv_paged_prefix.py:199-229) and writes its normalized output (0/0 = NaN when nothing is attended).
//
// Inside a block, 4 wavefronts take 16-column tiles in turn.  Blocks with many columns (prefill rows, decode blocks
// of several tiles per wavefront) first resolve all of them into an LDS column table partitioned by tier, so every
// tile holds rows of one tier and padding columns cost nothing; a block of one tile per wavefront resolves its own
// tile.  A tile's K and V rows are dequantized into the wavefront's LDS rows as bf16, then QK^T and P.V run as bf16
// 16x16x16 matrix-core steps with fp32 accumulation:
//   S^T[row][head] = K[row][:] . Q[head][:]   (A = K tile, B = Q^T; 16 steps over the 256 channels)
//   O[head][ch]   += P[head][row] V[row][ch]  (A = P straight from S^T's accumulator layout as bf16 high part
//                                               + bf16 remainder, B = V tile by the transposing LDS read)
// with an online softmax across a wavefront's tiles.  The 16 accumulator rows hold up to 16 q heads per KV head
// (GQA 8 of the configurations, 12 of the served model).  The 4 wavefronts merge through LDS, 8 heads per pass.
// In decode, columns c of request b attend when c < the request's valid count (cu_k[b + 1] - cu_k[b]) and
// 0 <= indices[b][c] < seq_lens[b] - the columns the reference's gather writes and its attention reads when the
// valid positions come first (the indexer pads with -1 at the end).
//
// Kinds (the compact gather's codes): 0 INT8-G pool, 1 INT4-G32 pool, 2 tiered (INT8-G ring over INT4-G32 rows,
// owner test).

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kD = 256;
constexpr int kRows = 16;          // rows per MFMA tile
constexpr int kWaves = 4;          // wavefronts per block, one tile each
constexpr int kCols = kWaves * kRows;  // selected columns per block (one partial)
constexpr int kHeads = 16;         // q heads per KV head the tile holds (rows beyond the group are zero)
constexpr int kKPitch = kD + 8;    // bf16 per K row in LDS (the pad spreads a column of rows over the banks)

typedef short bf4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf4 lds_v4s;
typedef float f4 __attribute__((ext_vector_type(4)));

struct SparseArgs {
  const void* k;           // tiered / INT4: uint8 [rows, H, D/2]; INT8: int8 [rows, H, D]
  const void* v;
  const uint16_t* ks;      // scales of k / v: fp16 [rows, H, D/32] (INT4) or [rows, H, D/G8] (INT8)
  const uint16_t* vs;
  const int8_t* rk;        // tiered: INT8 ring [R, H, D], scales [R, H, D/G8], owner [R]
  const int8_t* rv;
  const uint16_t* rks;
  const uint16_t* rvs;
  const int32_t* owner;
  int64_t ring_mask;
  const uint16_t* sm_k;    // smoothing factors [H, D] fp16 (may be null: identity)
  const uint16_t* sm_v;
  const int32_t* req_to_token;
  int64_t req_stride;
  const void* req_indices;
  int req64;
  const int32_t* indices;  // [batch, idx_stride], the first topk columns used
  int64_t idx_stride;
  const int32_t* seq_lens;
  const void* cu_k;
  int cu64;
  int topk;
  int H;
  int gs;
  int n_splits;
  int tiles;             // decode: 16-column tiles per wavefront (a block takes kCols x tiles columns)
  uint32_t rows8;        // rows of the INT8 tensors (ring R when tiered, the pool otherwise)
  uint32_t rows4;        // rows of the INT4 pool
  float scale;
  const uint16_t* q;       // bf16 query rows: row r, q head j at q + r sq_n + j sq_h
  int64_t sq_n, sq_h;
  int64_t si_m, si_g, si_n;  // indices of row r, KV head h, column c at indices + r si_m + h si_g + c si_n
  float* part_o;           // decode: [(b H + h) n_splits + split][gs][D]
  float* part_ml;          // decode: [(b H + h) n_splits + split][gs][2]
  int32_t* counters;       // decode, merged in the launch: [b H + h] arrivals (zero between calls); null: partials only
  float* mout_f32;         // decode, merged in the launch: out[b][h gs + j][D] fp32 or bf16, batch stride mout_b
  uint16_t* mout_bf16;
  int64_t mout_b;
  // prefill rows: chunk b holds rows cu_q[b] .. cu_q[b + 1] over a context of kv_lens[b] positions
  const void* cu_q;
  int cuq64;
  const int32_t* kv_lens;
  void* out;               // bf16 or fp32 (out_f32) rows: row r, q head j at out + r so_n + j so_h
  int out_f32;
  int64_t so_n, so_h;
};

// Entry i of an int32 or int64 index array (is64: exactly 0 or 1, as the launchers store it) without a branch on the
// width: both words are loaded unconditionally (an int32 entry reads its own word twice) and combined with integer
// arithmetic only.  Split in two (the loads, then the value) so that a caller can issue several entries' loads
// before it waits for any of them.
struct IdxWords {
  uint32_t lo, hi, wide;
};
KVT_DEV IdxWords idx_words(const void* p, int is64, int64_t i) {
  const uint32_t wide = (uint32_t)is64;
  const int32_t* w = reinterpret_cast<const int32_t*>(p) + (i << wide);
  return IdxWords{(uint32_t)w[0], (uint32_t)w[wide], wide};
}
KVT_DEV int64_t idx_value(const IdxWords& x) {
  const uint32_t mask = 0u - x.wide;   // all ones for int64 entries
  const uint32_t top = (x.hi & mask) | ((uint32_t)((int32_t)x.lo >> 31) & ~mask);
  return (int64_t)(((uint64_t)top << 32) | x.lo);
}

KVT_DEV f4 mfma_bf16(bf4 a, bf4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0); }

// bf16 pair (round to nearest even, one v_cvt_pk_bf16_f32): lo in bits 0-15.
KVT_DEV uint32_t bf16x2(float lo, float hi) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){lo, hi}, bf2v));
}

KVT_DEV __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Channels 4 lane .. 4 lane + 3 of one row, dequantized: bf16((c * s) * sm) for code c, the row's fp16 scale s
// (bits sbits) and the channel's smoothing factor sm, as the gathers write them.  INT8 rows give 4 codes in the
// loaded word; INT4 rows the 16-bit half (lane & 1) of the word holding channel pairs 4 (lane >> 1) .. + 3 (low
// nibble = even channel), stored as c + 8.  A code with offset o (c + o >= 0) goes into the mantissa of an fp16 magic
// value h = 1024 + (c + o) (v_perm_b32 for bytes, v_and_or_b32 for nibble pairs); v_fma_mix_f32 converts h and s and
// computes h * s - (1024 + o) * s in one rounding, whose exact value c * s is representable (4 or 8 bits times the
// scale's 11), so the fp32 product equals the plain c * s; the smoothing factor then multiplies in fp32 and
// v_cvt_pk_bf16_f32 rounds each pair to nearest even.
KVT_DEV uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(o));
  return r;
}
KVT_DEV float mix(uint32_t w, int half, _Float16 s, float c) {
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  return fmaf((float)__builtin_bit_cast(h2v, w)[half], (float)s, c);
}
KVT_DEV uint2 dequant4(bool hot, uint32_t w, uint32_t sbits, int lane, const float sm[4]) {
  const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(sbits & 0xffffu));
  uint32_t a, b;   // fp16 magic pairs: hot a = channels (0, 2), b = (1, 3); INT4 a = (0, 1), b = (2, 3)
  float c;
  if (hot) {
    const uint32_t u = w ^ 0x80808080u;
    a = __builtin_amdgcn_perm(0x64646464u, u, 0x04020400u);
    b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030401u);
    c = -1152.0f * (float)s;
  } else {
    const uint32_t h = (w >> (16 * (lane & 1))) & 0xffffu;
    const uint32_t x = h | (h << 12);   // nibble 1 at bits 16-19, nibble 3 at bits 24-27
    a = and_or(x, 0x000F000Fu, 0x64006400u);
    b = and_or(x >> 8, 0x000F000Fu, 0x64006400u);
    c = -1032.0f * (float)s;
  }
  float v[4];
  if (hot) {
    v[0] = mix(a, 0, s, c), v[1] = mix(b, 0, s, c), v[2] = mix(a, 1, s, c), v[3] = mix(b, 1, s, c);
  } else {
    v[0] = mix(a, 0, s, c), v[1] = mix(a, 1, s, c), v[2] = mix(b, 0, s, c), v[3] = mix(b, 1, s, c);
  }
  return uint2{bf16x2(v[0] * sm[0], v[1] * sm[1]), bf16x2(v[2] * sm[2], v[3] * sm[3])};
}

// One tile's raw row data for this lane (channels 4 lane .. + 3 of K and V, and their scales).
struct TileLoads {
  uint32_t kw[kRows], vw[kRows], ks[kRows], vs[kRows];
  int fl[kRows];
};

constexpr uint32_t kNoRow = 0x80000000u;   // a row offset past every buffer: its loads return zero

// Buffer resources over whole tensors (byte offsets are 32-bit: the launcher checks the sizes).
struct PoolRsrc {
  __amdgpu_buffer_rsrc_t k8, v8, ks8, vs8, k4, v4, ks4, vs4;
};

// Issue the loads of the wavefront's tile: row r's byte offsets (codes and scales, in the row's tier) come from
// lane r by readlane and go in the scalar offset of the loads, so every row costs a few scalar instructions and no
// vector address math; the lane offsets are fixed per tier.
// TIERS: the tile's rows are all INT8 (kRowsInt8), all INT4 (kRowsInt4) or each in its own tier (kRowsMixed: a
// wavefront-uniform branch per row).
enum { kRowsInt8 = 0, kRowsInt4 = 1, kRowsMixed = 2 };

template <int G8, int TIERS>
KVT_DEV void issue_tile(const PoolRsrc& P, int flags, uint32_t coff, uint32_t soff, int lane, TileLoads& L) {
  const uint32_t off8 = 4u * lane, off4 = 4u * (lane >> 1);
  const uint32_t soff8 = 2u * ((4u * lane) / G8), soff4 = 2u * (lane >> 3);
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int f = TIERS == kRowsMixed ? __builtin_amdgcn_readlane(flags, r) : (TIERS == kRowsInt8 ? 2 : 0);
    L.fl[r] = f;
    const uint32_t co = (uint32_t)__builtin_amdgcn_readlane((int)coff, r);
    const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)soff, r);
    if ((f & 2) != 0) {
      L.kw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.k8, off8, co, 0);
      L.vw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.v8, off8, co, 0);
      L.ks[r] = __builtin_amdgcn_raw_buffer_load_b16(P.ks8, soff8, so, 0);
      L.vs[r] = __builtin_amdgcn_raw_buffer_load_b16(P.vs8, soff8, so, 0);
    } else {
      L.kw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.k4, off4, co, 0);
      L.vw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.v4, off4, co, 0);
      L.ks[r] = __builtin_amdgcn_raw_buffer_load_b16(P.ks4, soff4, so, 0);
      L.vs[r] = __builtin_amdgcn_raw_buffer_load_b16(P.vs4, soff4, so, 0);
    }
  }
}

// A tile's 16 columns resolved by lanes 0-15 (lane r: column c0 + r): attended or not, tier, and the row's byte
// offsets in its tier (codes: INT8 rows D bytes, INT4 rows D / 2; scales).
struct TileCols {
  int flags;   // bit 0 attended, bit 1 ring (INT8) row
  uint32_t coff, soff;
};

// Resolve a tile's columns: position from the index row, slot from req_to_token, tier from the owner table (three
// dependent loads, independent of Q).
template <int KIND, int G8>
KVT_DEV TileCols resolve_tile(const SparseArgs& A, int64_t c0, int64_t c_end, const int32_t* idx_row, int64_t L,
                              int64_t req, int h, int lane) {
  const int64_t col = c0 + (lane & 15);
  bool valid = false, hot = KIND == 0;
  int64_t row = 0;
  if (lane < kRows && col < c_end) {
    const int64_t pos = idx_row[col * A.si_n];
    if (pos >= 0 && pos < L) {
      valid = true;
      const int64_t slot = A.req_to_token[req * A.req_stride + pos];
      row = slot;
      if constexpr (KIND == 2) {
        const int64_t r = slot & A.ring_mask;
        if ((int64_t)A.owner[r] == slot) {
          hot = true;
          row = r;
        }
      }
    }
  }
  const int64_t rh = row * A.H + h;
  TileCols tc;
  tc.flags = (valid ? 1 : 0) | (hot ? 2 : 0);
  tc.coff = !valid ? kNoRow : (uint32_t)(hot ? rh * kD : rh * (kD / 2));
  tc.soff = !valid ? kNoRow : (uint32_t)(hot ? rh * (kD / G8) * 2 : rh * (kD / kG4) * 2);
  return tc;
}

// One resolved 16-column tile of a wavefront, folded into its running softmax state (m, l per q head n16 of this
// lane, o): load and dequantize K into the wavefront's LDS rows, S^T = K Q^T, dequantize V into the same rows,
// online softmax, O += P V.
// hook(k) runs other work at three points: k = 0 before the tile's loads, 1 after its K rows are in LDS, 2 after
// S^T.
template <int KIND, int G8, int TIERS, typename Hook>
KVT_DEV void attend_tile(const SparseArgs& A, const PoolRsrc& P, const uint16_t* qs, uint16_t* kt, const TileCols& tc,
                         int lane, const float smk[4], const float smv[4], float& m_run, float& l_run, f4 o[16],
                         Hook&& hook) {
  const int n16 = lane & 15, kq = lane >> 4;
  const int flags = tc.flags;
  TileLoads T;
  hook(0);
  issue_tile<G8, TIERS>(P, flags, tc.coff, tc.soff, lane, T);

  // K rows into this wavefront's LDS rows (row-major); a wavefront's LDS accesses complete in order, so these
  // stores land after the previous tile's V reads
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    *reinterpret_cast<uint2*>(&kt[r * kKPitch + 4 * lane]) = dequant4((T.fl[r] & 2) != 0, T.kw[r], T.ks[r], lane, smk);
  hook(1);
  // S^T = K Q^T: lane l holds rows 4 (l >> 4) + i of q head l & 15
  f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint2 ka = *reinterpret_cast<const uint2*>(&kt[n16 * kKPitch + 16 * k + 4 * kq]);
    const uint2 qb = *reinterpret_cast<const uint2*>(&qs[n16 * kKPitch + 16 * k + 4 * kq]);
    s = mfma_bf16(__builtin_bit_cast(bf4, ka), __builtin_bit_cast(bf4, qb), s);
  }
  hook(2);
  // from here to P the tile's chain runs at a raised wave priority: the V rows and the softmax issue ahead of the
  // other wavefronts' work on the SIMD, which keeps the products that wait for them fed (slot-pool decode and the
  // paged prefix-chunk attention ~6 % faster than without)
  __builtin_amdgcn_s_setprio(1);
  // V rows into the same LDS rows (the stores stay behind the K reads above, which may alias them)
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    *reinterpret_cast<uint2*>(&kt[r * kKPitch + 4 * lane]) = dequant4((T.fl[r] & 2) != 0, T.vw[r], T.vs[r], lane, smv);
  // online softmax (log2 units): rows 4 kq + i of this lane's head, the other 12 rows in lanes n16 + 16 j
  constexpr float kLog2e = 1.4426950408889634f;
  const float cs = A.scale * kLog2e;
  float tv[4], mloc = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = __shfl(flags, 4 * kq + i, 64);   // the row's resolve lane
    tv[i] = (f & 1) ? s[i] * cs : -INFINITY;
    mloc = fmaxf(mloc, tv[i]);
  }
  const float m_new = fmaxf(m_run, max_xor16_32(mloc));
  const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
  float p[4], lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = m_new == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(tv[i] - m_new);
    lsum += p[i];
  }
  l_run = l_run * alpha + sum_xor16_32(lsum);
  m_run = m_new;
  // o[n][i] is head 4 kq + i: its rescale factor lives in lane 4 kq + i; only when some head's max has grown
  if (__any(alpha != 1.0f)) {
    float ai[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ai[i] = __shfl(alpha, 4 * kq + i, 64);
#pragma unroll
    for (int n = 0; n < 16; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[n][i] *= ai[i];
  }
  // P as bf16 high part + bf16 remainder (two products per step): P keeps ~16 significant bits, against 8 for a
  // plain bf16 cast, so a peaked softmax stays within the fp32 reference's tolerance
  const uint32_t h01 = bf16x2(p[0], p[1]), h23 = bf16x2(p[2], p[3]);
  const uint32_t l01 = bf16x2(p[0] - __uint_as_float(h01 << 16), p[1] - __uint_as_float(h01 & 0xffff0000u));
  const uint32_t l23 = bf16x2(p[2] - __uint_as_float(h23 << 16), p[3] - __uint_as_float(h23 & 0xffff0000u));
  const bf4 pa = __builtin_bit_cast(bf4, uint2{h01, h23});
  const bf4 pb = __builtin_bit_cast(bf4, uint2{l01, l23});
  __builtin_amdgcn_s_setprio(0);
  // O = P V.  B = V[rows 4 kq + k][channel 16 n + n16] by the transposing read: in each 16-lane group, lane L's
  // element k comes from element L & 3 of the 8 bytes lane 4 k + (L >> 2) addresses, so lane m addresses
  // V[4 kq + (m >> 2)][16 n + 4 (m & 3)]
  const uint32_t vbase = (uint32_t)(uintptr_t)&kt[(4 * kq + (n16 >> 2)) * kKPitch + 4 * (n16 & 3)];
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    const bf4 vop = __builtin_bit_cast(
        bf4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vbase + 32u * (uint32_t)n)));
    o[n] = mfma_bf16(pb, vop, mfma_bf16(pa, vop, o[n]));
  }
}

// A tile through the body for its rows' tiers: single-tier pools know them; in the tiered pool a tile whose 16 rows
// all sit in one tier (most of them: the ring holds a small share of the slots) takes a body without a branch per row.
template <int KIND, int G8, typename Hook>
KVT_DEV void attend_tile_any(const SparseArgs& A, const PoolRsrc& P, const uint16_t* qs, uint16_t* kt,
                             const TileCols& tc, int lane, const float smk[4], const float smv[4], float& m_run,
                             float& l_run, f4 o[16], Hook&& hook) {
  if constexpr (KIND != 2) {
    attend_tile<KIND, G8, KIND == 0 ? kRowsInt8 : kRowsInt4>(A, P, qs, kt, tc, lane, smk, smv, m_run, l_run, o, hook);
  } else {
    const uint64_t hot = __builtin_amdgcn_ballot_w64((tc.flags & 2) != 0) & 0xffffu;
    if (hot == 0)
      attend_tile<KIND, G8, kRowsInt4>(A, P, qs, kt, tc, lane, smk, smv, m_run, l_run, o, hook);
    else if (hot == 0xffffu)
      attend_tile<KIND, G8, kRowsInt8>(A, P, qs, kt, tc, lane, smk, smv, m_run, l_run, o, hook);
    else
      attend_tile<KIND, G8, kRowsMixed>(A, P, qs, kt, tc, lane, smk, smv, m_run, l_run, o, hook);
  }
}

// LDS of a block: one tile buffer per wavefront (K rows until S is formed, then V rows; 42 KB per block), after the
// tiles the same space holds the merge of the 4 wavefronts; and the group's q heads, bf16 (zero beyond gs)
template <int CAP>
struct BlockLds {
  uint16_t kv[kWaves][kRows * kKPitch];
  uint16_t qs[kHeads * kKPitch];
  uint2 cols[CAP];             // prefill rows: the query's resolved columns, ring rows first and INT4 rows last
  int counts[2 * kWaves];
  int last;                    // decode merged in the launch: this block counted last for its (request, KV head)
};
constexpr int kRowCols = 4096;   // prefill rows: selected columns resolved per pass (74 KB of LDS per block)
constexpr int kMultiCols = 1024; // decode blocks of several tiles per wavefront (50 KB of LDS per block)

// The selected columns [k0, k1) (at most kRowCols) of a prefill block's query row, resolved by all its threads
// together into the column table and partitioned by tier: ring (INT8) rows to cols[0 .. nh), INT4 rows to
// cols[CAP - nc .. CAP) (from the end), unattended columns dropped (patches/kv_paged_prefix.py:199-229: position in
// [0, L)).  J columns per thread, so the position, slot and owner loads of many columns are in flight at once; a
// block scan of the per-thread counts places them, in an order fixed by the columns (thread, then j), so the result
// does not depend on timing.  Every tile of 16 table entries then sits in one tier.
template <int KIND, int G8, int CAP, int J>
KVT_DEV void resolve_rows(const SparseArgs& A, int64_t k0, int64_t k1, const int32_t* idx_row, int64_t L,
                          int64_t req, int h, BlockLds<CAP>& S, int& nh, int& nc) {
  constexpr int kThreads = 64 * kWaves;
  static_assert(J * kThreads >= CAP, "a pass covers the table");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* r2t = A.req_to_token + req * A.req_stride;
  int pos[J], slot[J], own[J];
  bool live[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t c = k0 + tid + (int64_t)j * kThreads;
    pos[j] = c < k1 ? idx_row[c * A.si_n] : -1;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    live[j] = pos[j] >= 0 && (int64_t)pos[j] < L;
    slot[j] = live[j] ? r2t[pos[j]] : 0;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) own[j] = (KIND == 2 && live[j]) ? A.owner[(int64_t)slot[j] & A.ring_mask] : -1;
  bool hot[J];
  int mh = 0, mc = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    hot[j] = KIND == 0 || (KIND == 2 && live[j] && own[j] == slot[j]);
    mh += (live[j] && hot[j]) ? 1 : 0;
    mc += (live[j] && !hot[j]) ? 1 : 0;
  }
  // inclusive scan over the wavefront, then the wavefronts' totals through LDS
  int sh = mh, sc = mc;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int th = __shfl_up(sh, d, 64), tc = __shfl_up(sc, d, 64);
    if (lane >= d) sh += th, sc += tc;
  }
  if (lane == 63) S.counts[wave] = sh, S.counts[kWaves + wave] = sc;
  __syncthreads();
  int oh = sh - mh, oc = sc - mc;
  nh = 0, nc = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int a = S.counts[w], c = S.counts[kWaves + w];
    if (w < wave) oh += a, oc += c;
    nh += a, nc += c;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (!live[j]) continue;
    const int64_t row = hot[j] && KIND == 2 ? ((int64_t)slot[j] & A.ring_mask) : (int64_t)slot[j];
    const int64_t rh = row * A.H + h;
    const uint2 e = hot[j] ? uint2{(uint32_t)(rh * kD), (uint32_t)(rh * (kD / G8) * 2)}
                           : uint2{(uint32_t)(rh * (kD / 2)), (uint32_t)(rh * (kD / kG4) * 2)};
    if (hot[j])
      S.cols[oh++] = e;
    else
      S.cols[CAP - 1 - oc++] = e;
  }
}

// Tile t of a partitioned table: hot tiles 0 .. ceil(nh / 16) - 1 read entries 16 t .. from the front, the INT4
// tiles after them entries from the end; lane r < 16 takes one entry (past the part's count: not attended).
template <int CAP>
KVT_DEV TileCols table_tile(const BlockLds<CAP>& S, int t, int th, int nh, int nc, int lane) {
  const int r = lane & 15;
  const bool hot = t < th;
  const int i = hot ? 16 * t + r : 16 * (t - th) + r;
  const bool ok = lane < kRows && i < (hot ? nh : nc);
  TileCols x;
  x.flags = ok ? (hot ? 3 : 1) : 0;
  x.coff = kNoRow, x.soff = kNoRow;
  if (ok) {
    const uint2 e = S.cols[hot ? i : CAP - 1 - i];
    x.coff = e.x, x.soff = e.y;
  }
  return x;
}

// Device-scope stores and loads of the split partials: the partials cross XCDs (each has its own L2), so they are
// written through to the coherence point (read by the combine kernel, or by the block of this launch that merges
// them, which reads past its own L2: cache policy sc1 on the raw buffer accesses).
typedef unsigned int u4v __attribute__((vector_size(16)));   // the raw buffer builtins' 16- and 8-byte operands
typedef unsigned int u2v __attribute__((vector_size(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
constexpr int kSc1 = 16;
KVT_DEV void wait_vm0() {   // s_waitcnt vmcnt(0), the other counters untouched
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}
// The partials of (request b, KV head h): n_splits x gs rows of D floats, then n_splits x gs (m, l) pairs.
KVT_DEV __amdgpu_buffer_rsrc_t part_o_rsrc(const SparseArgs& A, int64_t bh) {
  const int64_t rows = (int64_t)A.n_splits * A.gs;
  return rsrc(A.part_o + bh * rows * kD, (uint32_t)(rows * kD * 4));
}
KVT_DEV __amdgpu_buffer_rsrc_t part_ml_rsrc(const SparseArgs& A, int64_t bh) {
  const int64_t rows = (int64_t)A.n_splits * A.gs;
  return rsrc(A.part_ml + bh * rows * 2, (uint32_t)(rows * 8));
}

// The split merge inside the decode launch: after its partial's device-scope stores have completed, a block counts
// itself on its (request, KV head) counter; the block that counts last resets the counter for the next call and
// merges the n_splits partials in split order (so the result does not depend on which block is last), as
// kvt_decode_combine does for a separate launch: (m, num, den) <- (max(m, m_s), num e^(m - m') + o_s e^(m_s - m'),
// den e^(m - m') + l_s e^(m_s - m')), out = num / den (0 / 0 = NaN when no column was attended).  No block waits for
// another.  Thread t merges q head t / 16, dims 16 (t % 16) .. + 15, with the loads of 4 splits in flight at once.
template <int CAP>
KVT_DEV void merge_last(const SparseArgs& A, BlockLds<CAP>& S, int b, int h) {
  wait_vm0();
  __syncthreads();   // every thread's partial stores have completed
  const int64_t bh = (int64_t)b * A.H + h;
  if (threadIdx.x == 0)
    S.last = __hip_atomic_fetch_add(&A.counters[bh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == A.n_splits - 1;
  __syncthreads();
  if (!S.last) return;
  if (threadIdx.x == 0) __hip_atomic_store(&A.counters[bh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  constexpr float kL2e = 1.4426950408889634f;
  constexpr int kB = 4;
  const int gs = A.gs, ns = A.n_splits;
  const int hq = (int)(threadIdx.x >> 4), c0 = 16 * (int)(threadIdx.x & 15);
  if (hq >= gs) return;
  const auto ro = part_o_rsrc(A, bh), rml = part_ml_rsrc(A, bh);
  float m = -INFINITY, den = 0.f, num[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) num[i] = 0.f;
  for (int s0 = 0; s0 < ns; s0 += kB) {
    f4 o[kB][4];
    f2 ml[kB];
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      const int s = s0 + k < ns ? s0 + k : s0;
      const int row = s * gs + hq;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[k][j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(ro, (row * kD + c0 + 4 * j) * 4, 0,
                                                                                kSc1));
      ml[k] = __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(rml, row * 8, 0, kSc1));
    }
#pragma unroll
    for (int k = 0; k < kB; ++k) {
      if (s0 + k >= ns) break;
      const float ms = ml[k][0], ls = ml[k][1];
      const float mn = fmaxf(m, ms);
      if (mn == -INFINITY) continue;   // both empty
      const float a = __builtin_amdgcn_exp2f((m - mn) * kL2e), c = __builtin_amdgcn_exp2f((ms - mn) * kL2e);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) num[4 * j + i] = num[4 * j + i] * a + o[k][j][i] * c;
      den = den * a + ls * c;
      m = mn;
    }
  }
  const int64_t off = (int64_t)b * A.mout_b + (int64_t)(h * gs + hq) * kD + c0;
  if (A.mout_f32 != nullptr) {
    float* dst = A.mout_f32 + off;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<float4*>(dst + 4 * j) =
          float4{num[4 * j] / den, num[4 * j + 1] / den, num[4 * j + 2] / den, num[4 * j + 3] / den};
  } else {
    uint16_t* dst = A.mout_bf16 + off;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<uint4*>(dst + 8 * j) =
          uint4{bf16x2(num[8 * j] / den, num[8 * j + 1] / den), bf16x2(num[8 * j + 2] / den, num[8 * j + 3] / den),
                bf16x2(num[8 * j + 4] / den, num[8 * j + 5] / den), bf16x2(num[8 * j + 6] / den, num[8 * j + 7] / den)};
  }
}

// XCD-aware work mapping.  The workgroups of a launch go to the 8 XCDs round robin by linear id, and each XCD has
// its own L2, so the block with linear id L takes the work item that shares lines with the items of ids L +- 8:
// * decode (grid n_splits x batch H): item i = b n_splits + split, in groups of 8 items whose H KV heads take ids
//   8 H g + 8 h + (i % 8) -- the blocks of one (request, split) run on one XCD side by side and share the lines of
//   the index, req_to_token and owner reads and of the rows' scales (both heads' scales sit in one 32-byte run);
// * prefill rows (grid max_q x batch H): XCD x takes the x-th eighth of the (query, KV head) items, consecutive
//   queries of one chunk, whose selections overlap.
// A tail of fewer than 8 items (decode) or ids (rows) keeps a plain order.
constexpr int kXcds = 8;
template <bool ROWS>
KVT_DEV void work_of_block(int H, int& wx, int& wy) {
  const uint32_t nx = gridDim.x, n = nx * gridDim.y, L = blockIdx.x + blockIdx.y * nx;
  if constexpr (ROWS) {
    const uint32_t m = n / kXcds * kXcds;
    const uint32_t w = L < m ? (L % kXcds) * (m / kXcds) + L / kXcds : L;
    wx = (int)(w % nx), wy = (int)(w / nx);
  } else {
    const uint32_t T = n / (uint32_t)H, full = T / kXcds * kXcds, gh = kXcds * (uint32_t)H;
    uint32_t i, hh;
    if (L < full * (uint32_t)H) {
      hh = (L % gh) / kXcds;
      i = L / gh * kXcds + L % kXcds;
    } else {
      const uint32_t t = T - full, r = L - full * (uint32_t)H;
      hh = r / t;
      i = full + r % t;
    }
    const uint32_t b = i / nx;
    wx = (int)(i - b * nx), wy = (int)(b * (uint32_t)H + hh);
  }
}

// The buffer resources of one tier (HOT: the INT8 tensors -- the ring when tiered --, else the INT4 pool), the
// other tier's left empty.  A block with a column table builds them just before that tier's tiles: the pointers
// pass through empty asm statements, so the compiler cannot hoist them to the kernel start and keep both tiers'
// 8 descriptors (32 scalar registers) live through the tile loops.
template <int KIND, int G8, bool HOT>
KVT_DEV PoolRsrc tier_rsrc(const SparseArgs& A, int H) {
  const void* pk = HOT && KIND == 2 ? (const void*)A.rk : A.k;
  const void* pv = HOT && KIND == 2 ? (const void*)A.rv : A.v;
  const void* pks = HOT && KIND == 2 ? (const void*)A.rks : (const void*)A.ks;
  const void* pvs = HOT && KIND == 2 ? (const void*)A.rvs : (const void*)A.vs;
  asm volatile("" : "+s"(pk), "+s"(pv), "+s"(pks), "+s"(pvs));
  PoolRsrc P{};
  if constexpr (HOT) {
    const uint32_t n8 = A.rows8 * (uint32_t)H * kD, s8 = A.rows8 * (uint32_t)H * (kD / G8) * 2;
    P.k8 = rsrc(pk, n8), P.v8 = rsrc(pv, n8), P.ks8 = rsrc(pks, s8), P.vs8 = rsrc(pvs, s8);
    P.k4 = P.v4 = P.ks4 = P.vs4 = rsrc(nullptr, 0u);
  } else {
    const uint32_t n4 = A.rows4 * (uint32_t)H * (kD / 2), s4 = A.rows4 * (uint32_t)H * (kD / kG4) * 2;
    P.k4 = rsrc(pk, n4), P.v4 = rsrc(pv, n4), P.ks4 = rsrc(pks, s4), P.vs4 = rsrc(pvs, s4);
    P.k8 = P.v8 = P.ks8 = P.vs8 = rsrc(nullptr, 0u);
  }
  return P;
}

// ROWS: prefill rows (one query row per block) instead of decode splits; MULTI: a decode block of several tiles per
// wavefront; CAP > 1: the block resolves its columns into a column table of CAP entries partitioned by tier first.
template <int KIND, int G8, bool ROWS, bool MULTI, int CAP>
KVT_DEV void sparse_attn_block(const SparseArgs& A, BlockLds<CAP>& S) {
  auto& kv = S.kv;
  uint16_t* qs = S.qs;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = A.H, gs = A.gs;
  int wx, wy;   // the work item: split (decode) or query (rows), and request / chunk x H + KV head
  work_of_block<ROWS>(H, wx, wy);
  const int b = wy / H;
  const int h = wy - b * H;
  // The start-up loads go out in as few dependent rounds as the data allows: the request's index-array entries and
  // length together (no wait between them), with the decode's q rows and the smoothing factors into registers; then
  // the first tile's resolve chain (position, slot, owner).  The q rows reach LDS after the chain.
  const IdxWords wreq = idx_words(A.req_indices, A.req64, b);
  const IdxWords w0 = ROWS ? idx_words(A.cu_q, A.cuq64, b) : idx_words(A.cu_k, A.cu64, b);
  const IdxWords w1 = ROWS ? idx_words(A.cu_q, A.cuq64, b + 1) : idx_words(A.cu_k, A.cu64, b + 1);
  const int32_t len = ROWS ? A.kv_lens[b] : A.seq_lens[b];   // widened after the barrier (no wait before it)
  // the group's q heads (512 16-byte chunks, 2 per thread; heads beyond the group read head 0 and are zeroed)
  constexpr int kQChunks = kHeads * kD / 8 / (64 * kWaves);
  uint4 qv[kQChunks];
  auto load_q = [&](int64_t row) {
#pragma unroll
    for (int k = 0; k < kQChunks; ++k) {
      const int i = (int)threadIdx.x + 64 * kWaves * k;
      const int hq = i / (kD / 8), ch = i - hq * (kD / 8);
      const int hr = hq < gs ? hq : 0;
      const uint4 w = *reinterpret_cast<const uint4*>(A.q + row * A.sq_n + (int64_t)(h * gs + hr) * A.sq_h + 8 * ch);
      qv[k] = hq < gs ? w : uint4{0u, 0u, 0u, 0u};
    }
  };
  if constexpr (!ROWS) load_q(b);
  // smoothing factors of this lane's channels 4 lane .. 4 lane + 3 (an absent factor: an empty buffer, read as 0)
  const uint32_t smb = (uint32_t)H * kD * 2;
  const uint2 wsk = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                  rsrc(A.sm_k, A.sm_k != nullptr ? smb : 0u), (h * kD + 4 * lane) * 2, 0, 0));
  const uint2 wsv = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                  rsrc(A.sm_v, A.sm_v != nullptr ? smb : 0u), (h * kD + 4 * lane) * 2, 0, 0));
  __builtin_amdgcn_sched_barrier(0);
  const int64_t req = idx_value(wreq), x0 = idx_value(w0), x1 = idx_value(w1), L = len;
  // the block's query row and column range
  int64_t qrow, c_begin, c_end;
  if constexpr (ROWS) {
    const int64_t j = wx;
    if (x0 + j >= x1) return;   // block-uniform: the chunk is shorter than the grid
    qrow = x0 + j;
    load_q(qrow);
    const int64_t visible = j + L - (x1 - x0) + 1;
    c_begin = 0;
    c_end = visible < (int64_t)A.topk ? (visible > 0 ? visible : 0) : (int64_t)A.topk;
  } else {
    qrow = b;
    const int64_t vcount = x1 - x0;
    const int64_t span = (int64_t)kCols * (MULTI ? A.tiles : 1);
    c_begin = (int64_t)wx * span;
    const int64_t lim = vcount < (int64_t)A.topk ? vcount : (int64_t)A.topk;
    c_end = c_begin + span < lim ? c_begin + span : lim;
  }

  const int32_t* idx_row = A.indices + qrow * A.si_m + (int64_t)h * A.si_g;
  // every scalar the resolve chain needs, in registers here: the compiler would otherwise sink these loads (and the
  // kernel-argument reads) into the chain's branch, one wait each, behind the index load
  asm volatile("" ::"s"(idx_row), "s"(L), "s"(req), "s"(c_end), "s"(A.req_to_token), "s"(A.req_stride),
               "s"(A.owner), "s"(A.ring_mask), "s"(A.si_n));
  // the wavefront's first tile (prefill rows: the first pass of the column table)
  TileCols tc0{};
  const bool has_tile = c_begin + kRows * wave < c_end;
  int nh = 0, nc = 0;
  if constexpr (CAP > 1)
    resolve_rows<KIND, G8, CAP, CAP / (64 * kWaves)>(A, c_begin, c_begin + CAP < c_end ? c_begin + CAP : c_end, idx_row,
                                                     L, req, h, S, nh, nc);
  else if (has_tile)
    tc0 = resolve_tile<KIND, G8>(A, c_begin + kRows * wave, c_end, idx_row, L, req, h, lane);
#pragma unroll
  for (int k = 0; k < kQChunks; ++k) {
    const int i = (int)threadIdx.x + 64 * kWaves * k;
    const int hq = i / (kD / 8), ch = i - hq * (kD / 8);
    *reinterpret_cast<uint4*>(&qs[hq * kKPitch + 8 * ch]) = qv[k];
  }
  PoolRsrc P;
  {
    const uint32_t n8 = A.rows8 * (uint32_t)H * kD, n4 = A.rows4 * (uint32_t)H * (kD / 2);
    const uint32_t s8 = A.rows8 * (uint32_t)H * (kD / G8) * 2, s4 = A.rows4 * (uint32_t)H * (kD / kG4) * 2;
    P.k8 = rsrc(KIND == 2 ? (const void*)A.rk : A.k, KIND == 1 ? 0u : n8);
    P.v8 = rsrc(KIND == 2 ? (const void*)A.rv : A.v, KIND == 1 ? 0u : n8);
    P.ks8 = rsrc(KIND == 2 ? A.rks : A.ks, KIND == 1 ? 0u : s8);
    P.vs8 = rsrc(KIND == 2 ? A.rvs : A.vs, KIND == 1 ? 0u : s8);
    P.k4 = rsrc(A.k, KIND == 0 ? 0u : n4);
    P.v4 = rsrc(A.v, KIND == 0 ? 0u : n4);
    P.ks4 = rsrc(A.ks, KIND == 0 ? 0u : s4);
    P.vs4 = rsrc(A.vs, KIND == 0 ? 0u : s4);
  }
  float smk[4], smv[4];
  const uint32_t swk[4] = {wsk.x, wsk.x >> 16, wsk.y, wsk.y >> 16}, swv[4] = {wsv.x, wsv.x >> 16, wsv.y, wsv.y >> 16};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    smk[i] = A.sm_k != nullptr ? f16_bits_to_f32((uint16_t)swk[i]) : 1.f;
    smv[i] = A.sm_v != nullptr ? f16_bits_to_f32((uint16_t)swv[i]) : 1.f;
  }
  __syncthreads();   // q staged

  float m_run = -INFINITY, l_run = 0.f;   // of q head lane & 15
  f4 o[16];                               // O[head 4 (lane >> 4) + i][channel 16 n + (lane & 15)]
#pragma unroll
  for (int n = 0; n < 16; ++n) o[n] = f4{0.f, 0.f, 0.f, 0.f};
  if constexpr (CAP > 1) {
    // passes of the column table (the first resolved above): wavefront w takes tiles w, w + 4, ..., ring tiles first
    for (int64_t k0 = c_begin; k0 < c_end; k0 += CAP) {
      const int64_t k1 = k0 + CAP < c_end ? k0 + CAP : c_end;
      if (k0 > c_begin) {
        __syncthreads();   // the previous pass's entries are read
        resolve_rows<KIND, G8, CAP, CAP / (64 * kWaves)>(A, k0, k1, idx_row, L, req, h, S, nh, nc);
        __syncthreads();
      }
      const int th = (nh + kRows - 1) / kRows, nt = th + (nc + kRows - 1) / kRows;
      int t = wave;
      if constexpr (KIND != 1) {   // the ring (INT8) tiles, then the INT4 ones, each tier's descriptors in turn
        const PoolRsrc P8 = tier_rsrc<KIND, G8, true>(A, H);
        for (; t < th; t += kWaves)
          attend_tile<KIND, G8, kRowsInt8>(A, P8, qs, kv[wave], table_tile(S, t, th, nh, nc, lane), lane, smk, smv,
                                           m_run, l_run, o, [](int) {});
      }
      if constexpr (KIND != 0) {
        const PoolRsrc P4 = tier_rsrc<KIND, G8, false>(A, H);
        for (; t < nt; t += kWaves)
          attend_tile<KIND, G8, kRowsInt4>(A, P4, qs, kv[wave], table_tile(S, t, th, nh, nc, lane), lane, smk, smv,
                                           m_run, l_run, o, [](int) {});
      }
    }
  } else {   // at most one tile per wavefront (64 columns per block): no state is live across its loads
    if (has_tile) attend_tile_any<KIND, G8>(A, P, qs, kv[wave], tc0, lane, smk, smv, m_run, l_run, o, [](int) {});
  }

  // merge the 4 wavefronts through LDS, 8 q heads per pass: wavefront w stores the O rows of the pass's heads and
  // (m, l) of every head; thread t then merges head t / 32 of the pass, channels 8 (t % 32) .. + 7, over the 4
  __syncthreads();   // every wavefront is done with its tile rows
  float* mo = reinterpret_cast<float*>(&kv[0][0]);   // [wave][8 heads][256]
  float* mml = mo + kWaves * 8 * kD;                  // [wave][16 heads][2]
  const int kq = lane >> 4, n16 = lane & 15;
  if (lane < gs) {
    mml[(wave * kHeads + lane) * 2] = m_run;
    mml[(wave * kHeads + lane) * 2 + 1] = l_run;
  }
  for (int hh = 0; hh < gs; hh += 8) {
    if (hh > 0) __syncthreads();   // the previous pass's reads are done
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hq = 4 * kq + i - hh;
      if (hq >= 0 && hq < 8 && hq + hh < gs) {
#pragma unroll
        for (int n = 0; n < 16; ++n) mo[(wave * 8 + hq) * kD + 16 * n + n16] = o[n][i];
      }
    }
    __syncthreads();
    const int hq = hh + (threadIdx.x >> 5), c0 = 8 * (threadIdx.x & 31);
    if (hq < gs) {
      float mw[kWaves], M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        mw[w] = mml[(w * kHeads + hq) * 2];
        M = fmaxf(M, mw[w]);
      }
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, lt = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float a = mw[w] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
        lt += a * mml[(w * kHeads + hq) * 2 + 1];
        const float* src = &mo[(w * 8 + (hq - hh)) * kD + c0];
        const float4 o0 = *reinterpret_cast<const float4*>(src);
        const float4 o1 = *reinterpret_cast<const float4*>(src + 4);
        acc[0] += a * o0.x;
        acc[1] += a * o0.y;
        acc[2] += a * o0.z;
        acc[3] += a * o0.w;
        acc[4] += a * o1.x;
        acc[5] += a * o1.y;
        acc[6] += a * o1.z;
        acc[7] += a * o1.w;
      }
      if constexpr (ROWS) {
        // normalized output; nothing attended gives 0 / 0 = NaN (patches/kv_paged_prefix.py:259)
        const int64_t off = qrow * A.so_n + (int64_t)(h * gs + hq) * A.so_h + c0;
        if (A.out_f32) {
          float* dst = reinterpret_cast<float*>(A.out) + off;
          *reinterpret_cast<float4*>(dst) = float4{acc[0] / lt, acc[1] / lt, acc[2] / lt, acc[3] / lt};
          *reinterpret_cast<float4*>(dst + 4) = float4{acc[4] / lt, acc[5] / lt, acc[6] / lt, acc[7] / lt};
        } else {
          uint16_t* dst = reinterpret_cast<uint16_t*>(A.out) + off;
          *reinterpret_cast<uint4*>(dst) = uint4{bf16x2(acc[0] / lt, acc[1] / lt), bf16x2(acc[2] / lt, acc[3] / lt),
                                                 bf16x2(acc[4] / lt, acc[5] / lt), bf16x2(acc[6] / lt, acc[7] / lt)};
        }
      } else {
        // The partial, read after this launch by the combine kernel or inside it by the block that counts last, on
        // any XCD: device-scope stores (sc1), written through past this XCD's L2, so that no write-back of them is
        // left for the kernel's end (top-k decode 182.8 -> 180.4 us per step against plain stores)
        constexpr float kLn2 = 0.6931471805599453f;
        const float mnat = M == -INFINITY ? -INFINITY : M * kLn2;   // m of the block's partial in natural-log units
        const int row = wx * gs + hq;
        const auto ro = part_o_rsrc(A, (int64_t)b * H + h);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, f4{acc[0], acc[1], acc[2], acc[3]}), ro,
                                               (row * kD + c0) * 4, 0, kSc1);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, f4{acc[4], acc[5], acc[6], acc[7]}), ro,
                                               (row * kD + c0 + 4) * 4, 0, kSc1);
        if (c0 == 0)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, f2{mnat, lt}),
                                                part_ml_rsrc(A, (int64_t)b * H + h), row * 8, 0, kSc1);
      }
    }
  }
  if constexpr (!ROWS) {
    if (A.counters != nullptr) merge_last(A, S, b, h);
  }
}

// decode: one tile per wavefront, 3 blocks per CU
template <int KIND, int G8>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3))) sparse_decode_kernel(SparseArgs A) {
  __shared__ __align__(16) BlockLds<1> S;
  sparse_attn_block<KIND, G8, false, false, 1>(A, S);
}

// decode of long selections: the block's 64 A.tiles columns resolved into its column table, a wavefront looping over
// its tiles with the accumulators live; 2 blocks per CU
template <int KIND, int G8>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2)))
sparse_decode_multi_kernel(SparseArgs A) {
  __shared__ __align__(16) BlockLds<kMultiCols> S;
  sparse_attn_block<KIND, G8, false, true, kMultiCols>(A, S);
}

// prefill rows: the query's selection resolved into the column table, a wavefront looping over its tiles with the
// accumulators live; 2 blocks per CU
template <int KIND, int G8>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) sparse_prefill_kernel(SparseArgs A) {
  __shared__ __align__(16) BlockLds<kRowCols> S;
  sparse_attn_block<KIND, G8, true, false, kRowCols>(A, S);
}

// Shared argument checks and pool resources of both entry points; returns KVT_OK or a status.
int pool_args(int kind, int64_t pool_rows, const void* ring_k, const void* owner, int64_t ring_mask, int H, int Hq,
              int D, int group8, int64_t* rows8, int64_t* rows4) {
  if (H <= 0 || Hq % H != 0 || Hq / H > kHeads || D != kD || kind < 0 || kind > 2) return KVT_EINVAL;
  if (kind == 2 && (owner == nullptr || ring_k == nullptr || ((ring_mask + 1) & ring_mask) != 0)) return KVT_EINVAL;
  if (pool_rows <= 0 || (kind != 1 && group8 != 64 && group8 != 256)) return KVT_EINVAL;
  // byte offsets are 32-bit and must stay below kNoRow (rows * H * D bytes of INT8 codes, / 2 for INT4)
  *rows8 = kind == 2 ? ring_mask + 1 : (kind == 0 ? pool_rows : 0);
  *rows4 = kind == 0 ? 0 : pool_rows;
  if (*rows8 * H * kD >= (int64_t)kNoRow || *rows4 * H * (kD / 2) >= (int64_t)kNoRow) return KVT_ERANGE;
  return KVT_OK;
}

template <bool ROWS>
int launch(int kind, int group8, dim3 grid, hipStream_t st, const SparseArgs& A) {
#define KVT_SD(KIND_, G_)                                                                                  \
  do {                                                                                                     \
    if constexpr (ROWS)                                                                                    \
      hipLaunchKernelGGL((sparse_prefill_kernel<KIND_, G_>), grid, dim3(64 * kWaves), 0, st, A);           \
    else if (A.tiles > 1)                                                                                  \
      hipLaunchKernelGGL((sparse_decode_multi_kernel<KIND_, G_>), grid, dim3(64 * kWaves), 0, st, A);      \
    else                                                                                                   \
      hipLaunchKernelGGL((sparse_decode_kernel<KIND_, G_>), grid, dim3(64 * kWaves), 0, st, A);            \
  } while (0)
  if (kind == 1) {
    KVT_SD(1, 64);
  } else if (group8 == 64) {
    if (kind == 2) {
      KVT_SD(2, 64);
    } else {
      KVT_SD(0, 64);
    }
  } else {
    if (kind == 2) {
      KVT_SD(2, 256);
    } else {
      KVT_SD(0, 256);
    }
  }
#undef KVT_SD
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // namespace

extern "C" {

int kvt_sparse_decode(int kind, const void* q, int64_t q_stride_b, const void* k, const void* v, const void* k_scale,
                      const void* v_scale, int64_t pool_rows, const void* ring_k, const void* ring_v, const void* ring_ks,
                      const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                      int cu_is_int64, int batch, int topk, int H, int Hq, int D, int group8, float scale,
                      int n_splits, void* part_o, void* part_ml, void* counters, void* out_f32, void* out_bf16,
                      int64_t out_stride_b, void* stream) {
  if (batch <= 0 || topk <= 0 || n_splits <= 0) return KVT_EINVAL;
  // one (request, KV head)'s partials are addressed with 32-bit offsets
  if ((int64_t)n_splits * (Hq / (H > 0 ? H : 1)) * D * 4 >= (1ll << 31)) return KVT_EINVAL;
  if (counters != nullptr && ((out_f32 == nullptr) == (out_bf16 == nullptr) || out_stride_b < (int64_t)Hq * D ||
                              ((uintptr_t)(out_f32 != nullptr ? out_f32 : out_bf16) & 15) != 0 ||
                              (out_stride_b & 7) != 0))
    return KVT_EINVAL;   // merged in the launch: 16-byte output pieces
  // n_splits blocks per (request, KV head) cover the topk columns with `tiles` 16-column tiles per wavefront
  const int tiles64 = (topk + kCols - 1) / kCols;
  const int tiles = (tiles64 + n_splits - 1) / n_splits;
  if ((q_stride_b & 7) != 0 || ((uintptr_t)q & 15) != 0) return KVT_EINVAL;
  int64_t rows8 = 0, rows4 = 0;
  const int st_ = pool_args(kind, pool_rows, ring_k, owner, ring_mask, H, Hq, D, group8, &rows8, &rows4);
  if (st_ != KVT_OK) return st_;
  SparseArgs A{};
  A.k = k, A.v = v, A.ks = (const uint16_t*)k_scale, A.vs = (const uint16_t*)v_scale;
  A.rk = (const int8_t*)ring_k, A.rv = (const int8_t*)ring_v, A.rks = (const uint16_t*)ring_ks;
  A.rvs = (const uint16_t*)ring_vs, A.owner = (const int32_t*)owner, A.ring_mask = ring_mask;
  A.sm_k = (const uint16_t*)sm_k, A.sm_v = (const uint16_t*)sm_v;
  A.req_to_token = (const int32_t*)req_to_token, A.req_stride = req_stride, A.req_indices = req_indices;
  A.req64 = req_is_int64 != 0, A.indices = (const int32_t*)indices, A.idx_stride = idx_stride;
  A.seq_lens = (const int32_t*)seq_lens, A.cu_k = cu_k, A.cu64 = cu_is_int64 != 0, A.topk = topk;
  A.H = H, A.gs = Hq / H, A.n_splits = n_splits, A.tiles = tiles, A.rows8 = (uint32_t)rows8;
  A.rows4 = (uint32_t)rows4, A.scale = scale, A.q = (const uint16_t*)q, A.sq_n = q_stride_b, A.sq_h = kD;
  A.si_m = idx_stride, A.si_g = 0, A.si_n = 1, A.part_o = (float*)part_o, A.part_ml = (float*)part_ml;
  A.counters = (int32_t*)counters, A.mout_f32 = (float*)out_f32, A.mout_bf16 = (uint16_t*)out_bf16;
  A.mout_b = out_stride_b;
  return launch<false>(kind, group8, dim3((unsigned)n_splits, (unsigned)(batch * H)), (hipStream_t)stream, A);
}

int kvt_sparse_prefill(int kind, const void* q, int64_t sq_n, int64_t sq_h, const void* cu_q, int cu_q_is_int64,
                       const void* kv_lens, int batch, int max_q, const void* indices, int64_t si_m, int64_t si_g,
                       int64_t si_n, int topk, const void* k, const void* v, const void* k_scale, const void* v_scale,
                       int64_t pool_rows, const void* ring_k, const void* ring_v, const void* ring_ks,
                       const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                       const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64, int H,
                       int Hq, int D, int group8, float scale, void* out, int out_f32, int64_t so_n, int64_t so_h,
                       void* stream) {
  if (batch < 0 || max_q < 0 || topk < 0) return KVT_EINVAL;
  // 16-byte q loads and output stores: row and head strides multiples of 8 elements (4 for fp32 output)
  if ((sq_n & 7) != 0 || (sq_h & 7) != 0 || ((uintptr_t)q & 15) != 0) return KVT_EINVAL;
  if (((uintptr_t)out & 15) != 0 || (so_n & (out_f32 ? 3 : 7)) != 0 || (so_h & (out_f32 ? 3 : 7)) != 0) return KVT_EINVAL;
  int64_t rows8 = 0, rows4 = 0;
  const int st_ = pool_args(kind, pool_rows, ring_k, owner, ring_mask, H, Hq, D, group8, &rows8, &rows4);
  if (st_ != KVT_OK) return st_;
  if (batch == 0 || max_q == 0) return KVT_OK;
  SparseArgs A{};
  A.k = k, A.v = v, A.ks = (const uint16_t*)k_scale, A.vs = (const uint16_t*)v_scale;
  A.rk = (const int8_t*)ring_k, A.rv = (const int8_t*)ring_v, A.rks = (const uint16_t*)ring_ks;
  A.rvs = (const uint16_t*)ring_vs, A.owner = (const int32_t*)owner, A.ring_mask = ring_mask;
  A.sm_k = (const uint16_t*)sm_k, A.sm_v = (const uint16_t*)sm_v;
  A.req_to_token = (const int32_t*)req_to_token, A.req_stride = req_stride, A.req_indices = req_indices;
  A.req64 = req_is_int64 != 0, A.indices = (const int32_t*)indices, A.topk = topk;
  A.H = H, A.gs = Hq / H, A.n_splits = 1, A.tiles = 1, A.rows8 = (uint32_t)rows8, A.rows4 = (uint32_t)rows4;
  A.scale = scale, A.q = (const uint16_t*)q, A.sq_n = sq_n, A.sq_h = sq_h;
  A.si_m = si_m, A.si_g = si_g, A.si_n = si_n;
  A.cu_q = cu_q, A.cuq64 = cu_q_is_int64 != 0, A.kv_lens = (const int32_t*)kv_lens;
  A.out = out, A.out_f32 = out_f32, A.so_n = so_n, A.so_h = so_h;
  return launch<true>(kind, group8, dim3((unsigned)max_q, (unsigned)(batch * H)), (hipStream_t)stream, A);
}

}  // extern "C"
