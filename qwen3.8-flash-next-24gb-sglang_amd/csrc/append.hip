// Write path of the tiered KV cache: quantize-append kernels for gfx950.
//
// One wavefront (64 lanes) owns one (token, KV head) row; lane l holds channels 4l..4l+3, so a 32-channel INT4
// group is 8 lanes and a 64-channel INT8 group is 16 lanes: the group absmax is a lane butterfly inside the wave
// and every load/store is a contiguous per-lane chunk (row-coalesced).  Four rows per 256-thread block.
// The arithmetic is the reference's bit for bit (IEEE quotients, round-half-even, fp16 scales) but avoids the
// division on the common path: scales from a * fl(1/qmax) and codes from x * rcp(s), each checked against the
// rounding ties it could get wrong, with the IEEE division for the lanes that are close to one.
//
//   kvt_quant_store_tiered  dual write (patches/kv_tiers.py:272-443): owner stamp launch, then the INT8 ring row
//                           (owner only) + INT4 pool row (always) launch.
//   kvt_quant_store_int8    INT8-G quant + scatter (patches/kv_int8.py:281-362, with the fp16-max clamp).
//   kvt_quant_store_int4    INT4-G32 quant + nibble pack + scatter (patches/kv_int4.py:289-393).
//   kvt_page_table_update   writes (seq, logical page) -> physical page entries before an evicting append.
//   kvt_append_plan         the same plan on the device: positions, page pops from a free list, seq_lens advance.
//   kvt_append_evict        position-indexed ring append: requantizes the ring row being overwritten into the
//                           INT4 page of its position (docs/KV_TIERS_PLAN.md:53, :63-67), then stores the new
//                           token's INT8 row.

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kWavesPerBlock = 4;  // one (token, KV head) row per wavefront, four per block
struct RowIn {
  const void* base;
  int64_t stride_n;  // elements
  int64_t stride_h;  // elements
};

// Raw buffer over [p, p + bytes): a load outside it returns zero without a memory access, so a row that is not
// needed costs no traffic and no branch.
KVT_DEV __amdgpu_buffer_rsrc_t row_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// How a kernel reads its 4 input channels per lane (chosen by the launcher):
//   kLoadElem   element loads, smoothing inverse optional at run time (any strides);
//   kLoadVec    one 8-byte (16-bit types) or 16-byte (fp32) load, no smoothing inverse;
//   kLoadVecSm  the same plus one 8-byte load of the 4 smoothing values.
// The vector forms need the base and both strides to keep every 4-channel chunk aligned.
enum LoadMode : int { kLoadElem = 0, kLoadVec = 1, kLoadVecSm = 2 };

// The 4 input channels c0..c0+3 of row (t, h), loaded (load4_raw) and later converted to fp32 times the smoothing
// inverse when one is given: x = f32(k) * f32(sm_inv) (patches/kv_tiers.py:332-333).  Splitting the two lets the
// kernels put the input loads first and the metadata chain behind them without waiting for the inputs.
struct In4 {
  uint32_t w[4];  // 16-bit types: w[0..1] hold the 4 values; fp32: w[0..3]; kLoadElem: the converted fp32 bits
  uint2 m;        // kLoadVecSm: the 4 smoothing values (fp16)
};

template <int DT, int LM>
KVT_DEV In4 load4_raw(const RowIn& in, int64_t t, int h, int c0, const uint16_t* sm_inv, int D) {
  const int64_t off = t * in.stride_n + (int64_t)h * in.stride_h + c0;
  In4 r{};
  if constexpr (LM == kLoadElem) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = load_in<DT>(in.base, off + i);
      r.w[i] = __float_as_uint(sm_inv ? v * f16_bits_to_f32(sm_inv[h * D + c0 + i]) : v);
    }
  } else {
    if constexpr (DT == kF32) {
      const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(in.base) + off);
      r.w[0] = v.x;
      r.w[1] = v.y;
      r.w[2] = v.z;
      r.w[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(in.base) + off);
      r.w[0] = v.x;
      r.w[1] = v.y;
    }
    if constexpr (LM == kLoadVecSm) r.m = *reinterpret_cast<const uint2*>(sm_inv + h * D + c0);
  }
  return r;
}

template <int DT, int LM>
KVT_DEV void to_f32(const In4& r, float x[4]) {
  if constexpr (LM == kLoadElem || DT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(r.w[i]);
  } else {
    const uint16_t e[4] = {(uint16_t)r.w[0], (uint16_t)(r.w[0] >> 16), (uint16_t)r.w[1], (uint16_t)(r.w[1] >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = DT == kBF16 ? bf16_to_f32(e[i]) : f16_bits_to_f32(e[i]);
  }
  if constexpr (LM == kLoadVecSm) {
    x[0] *= f16_bits_to_f32((uint16_t)r.m.x);
    x[1] *= f16_bits_to_f32((uint16_t)(r.m.x >> 16));
    x[2] *= f16_bits_to_f32((uint16_t)r.m.y);
    x[3] *= f16_bits_to_f32((uint16_t)(r.m.y >> 16));
  }
}

// ------------------------------------------------------------------------------------------- lane quantizers
// The group absmax works on |x| bit patterns: for non-negative floats the unsigned order of the patterns is the
// float order, and a NaN sorts above +inf, so a NaN in a group reaches its absmax (as with torch's amax) and the
// scale falls back to 1 (a > 0 is false for NaN).
KVT_DEV uint32_t absmax4_bits(const float x[4]) {
  const uint32_t m = 0x7fffffffu;
  return max(max(__float_as_uint(x[0]) & m, __float_as_uint(x[1]) & m),
             max(__float_as_uint(x[2]) & m, __float_as_uint(x[3]) & m));
}

template <int CTRL>
KVT_DEV uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}

// Max over aligned groups of `width` lanes.  Inside a 16-lane row DPP does it: quad_perm [1,0,3,2] and [2,3,0,1]
// reduce each quad, row_half_mirror (lane i <- 7 - i) joins the two quads of a half-row and row_mirror
// (i <- 15 - i) the two half-rows; wider groups finish with LDS permutes.  Every lane of a group must be active.
template <int width>
KVT_DEV uint32_t group_max_bits(uint32_t v) {
  static_assert(width >= 8 && width <= 64 && (width & (width - 1)) == 0, "group width");
  v = max(v, dpp_u32<0xb1>(v));
  v = max(v, dpp_u32<0x4e>(v));
  v = max(v, dpp_u32<0x141>(v));
  if constexpr (width >= 16) v = max(v, dpp_u32<0x140>(v));
#pragma unroll
  for (int o = 16; o < width; o <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

// group_scale(a, QMAX) (fp16 bits) from a * fl(1 / QMAX) where that is safe: the product carries at most ~1.5 ulp
// of relative error against a / QMAX, so it lies within 2.5 fp32 ulps of fl(a / QMAX), and both round to the same
// fp16 value when the product is in the normal fp16 range below 32768 (the min with 65504 then does nothing) and
// its 13 discarded mantissa bits are more than 4 away from the rounding tie 0x1000.  Anything else (zero, tiny,
// huge, NaN, near a tie) takes the IEEE division.
template <int QMAX>
KVT_DEV uint16_t scale_bits(float a) {
  constexpr float kInv = 1.0f / QMAX;
  const float z = a * kInv;
  const uint32_t b = __float_as_uint(z);
  const bool fast = b - 0x38800000u < 0x47000000u - 0x38800000u && (b & 0x1fffu) - 0x0ffcu > 8u;
  uint16_t h = f32_to_f16_bits(z);
  if (!fast) h = group_scale(a, (float)QMAX);
  return h;
}

// Codes q_i = clamp(rne(fl(x_i / s)), -QMAX, QMAX) of one lane, returned as floats.  The common path uses
// y = x * k with k ~ 1 / s (k = rcp(s), or a product of exact factors with it; relative error within a few ulps):
// after the clamp, |y| <= QMAX < 128 where a few ulps are below 2^-15, so rne(y) equals rne(fl(x / s)) unless y is
// within 2^-12 of a half-integer; lanes holding such a value redo their four quotients with the IEEE division.
// Clamping first is exact (the bounds are integers) and leaves clamped values far from any tie.
template <int QMAX, typename ExactX>
KVT_DEV void round_codes(const float y_in[4], float s, ExactX exact_x, float q[4]) {
  float dmax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float y = __builtin_amdgcn_fmed3f(y_in[i], -(float)QMAX, (float)QMAX);
    q[i] = rintf(y);
    dmax = fmaxf(dmax, fabsf(y - q[i]));
  }
  if (dmax > 0.5f - 0x1p-12f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = quant_code(exact_x(i), s, (float)QMAX);
  }
}

// 4 INT8 codes, little-endian bytes of one dword.
KVT_DEV uint32_t pack8(const float q[4]) {
  const uint32_t c0 = (uint32_t)(int)q[0], c1 = (uint32_t)(int)q[1], c2 = (uint32_t)(int)q[2], c3 = (uint32_t)(int)q[3];
  return __builtin_amdgcn_perm(c1, c0, 0x0c0c0400u) | __builtin_amdgcn_perm(c3, c2, 0x04000c0cu);
}

// 4 INT4 codes as offset-binary nibbles (low nibble = even channel, patches/kv_int4.py:337-339):
// sum_i (q_i + 8) 16^i, every partial sum an integer below 2^16 and so exact in fp32.
KVT_DEV uint32_t pack4(const float q[4]) {
  const float p = fmaf(q[3], 4096.0f, fmaf(q[2], 256.0f, fmaf(q[1], 16.0f, q[0] + 34952.0f)));
  return (uint32_t)p;
}

// INT8-G row part held by this lane: 4 codes packed little-endian, plus the group scale (fp16 bits).
template <int LANES_PER_GROUP>
KVT_DEV uint32_t quant8_lane(const float x[4], uint16_t* scale_bits_out) {
  const float a = __uint_as_float(group_max_bits<LANES_PER_GROUP>(absmax4_bits(x)));
  const uint16_t sb = scale_bits<127>(a);
  const float s = f16_bits_to_f32(sb);
  const float r = __builtin_amdgcn_rcpf(s);
  const float y[4] = {x[0] * r, x[1] * r, x[2] * r, x[3] * r};
  float q[4];
  round_codes<127>(y, s, [&](int i) { return x[i]; }, q);
  *scale_bits_out = sb;
  return pack8(q);
}

// INT4-G32 row part held by this lane: 2 bytes (4 nibbles), plus the group scale (fp16 bits).
KVT_DEV uint32_t quant4_lane(const float x[4], uint16_t* scale_bits_out) {
  const float a = __uint_as_float(group_max_bits<8>(absmax4_bits(x)));
  const uint16_t sb = scale_bits<7>(a);
  const float s = f16_bits_to_f32(sb);
  const float r = __builtin_amdgcn_rcpf(s);
  const float y[4] = {x[0] * r, x[1] * r, x[2] * r, x[3] * r};
  float q[4];
  round_codes<7>(y, s, [&](int i) { return x[i]; }, q);
  *scale_bits_out = sb;
  return pack4(q);
}

// INT4-G32 requantization of 4 INT8 ring codes with scale s8: x_i = c_i * s8 is exact, so the group absmax is
// s8 * max|c_i| and y_i = c_i * (s8 * rcp(s4)) stays within a few ulps of x_i / s4.
KVT_DEV uint32_t requant4_lane(uint32_t codes, uint16_t s8bits, uint16_t* scale_bits_out) {
  const float s8 = f16_bits_to_f32(s8bits);
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = (float)(int8_t)(codes >> (8 * i));
  const float a = __uint_as_float(group_max_bits<8>(absmax4_bits(c))) * s8;
  const uint16_t sb = scale_bits<7>(a);
  const float s = f16_bits_to_f32(sb);
  const float k = s8 * __builtin_amdgcn_rcpf(s);
  const float y[4] = {c[0] * k, c[1] * k, c[2] * k, c[3] * k};
  float q[4];
  round_codes<7>(y, s, [&](int i) { return c[i] * s8; }, q);
  *scale_bits_out = sb;
  return pack4(q);
}

// Stores of the quantized ring and pool rows: non-temporal (streaming).  The rows are read by later launches, not by
// this one; plain stores measured 12.16 against 11.74 us per 8,192-token evicting launch, device-scope (write-through)
// stores 14.6 us.
template <typename T>
KVT_DEV void st_row(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

template <int D, int G8>
KVT_DEV void store_ring_row(int8_t* rbuf, uint16_t* rscale, int64_t r, int H, int h, int lane, const float x[4]) {
  constexpr int NG8 = D / G8;
  uint16_t sb;
  const uint32_t packed = quant8_lane<G8 / 4>(x, &sb);
  st_row(&reinterpret_cast<uint32_t*>(rbuf + (r * H + h) * D)[lane], packed);
  if ((lane & (G8 / 4 - 1)) == 0) st_row(&rscale[(r * H + h) * NG8 + lane / (G8 / 4)], sb);
}

template <int D>
KVT_DEV void store_pool_row(uint8_t* pbuf, uint16_t* pscale, int64_t row, int H, int h, int lane, const float x[4]) {
  constexpr int NG4 = D / kG4;
  uint16_t sb;
  const uint32_t b = quant4_lane(x, &sb);
  reinterpret_cast<uint16_t*>(pbuf + (row * H + h) * (D / 2))[lane] = (uint16_t)b;
  if ((lane & 7) == 0) pscale[(row * H + h) * NG4 + lane / 8] = sb;
}

KVT_DEV int64_t load_loc(const void* loc, int loc64, int64_t t) {
  return loc64 ? reinterpret_cast<const int64_t*>(loc)[t] : (int64_t) reinterpret_cast<const int32_t*>(loc)[t];
}

// Blocks are dealt to the 8 XCDs round-robin (block b runs on XCD b % 8), each XCD with its own L2.  Renumbered
// this way, every XCD takes one contiguous range of blocks, so rows that share cache lines (scale rows, per-token
// indices) are fetched into one L2 rather than several.
KVT_DEV uint32_t xcd_block() {
  const uint32_t b = blockIdx.x, n = gridDim.x;
  const uint32_t q = n / 8, r = n % 8, x = b % 8;
  return x * q + min(x, r) + b / 8;
}

// This wavefront's (token, head) row, or false past the last one.
KVT_DEV bool wave_row(uint32_t NH, int H, uint32_t* t, int* h) {
  const uint32_t item = xcd_block() * kWavesPerBlock + (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  *t = item / (uint32_t)H;
  *h = (int)(item - *t * (uint32_t)H);
  return item < NH;
}

__global__ void __launch_bounds__(256) stamp_owner_kernel(const void* loc, int loc64, int64_t N, int32_t* owner,
                                                          int64_t ring_mask) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int64_t slot = load_loc(loc, loc64, t);
  owner[slot & ring_mask] = (int32_t)slot;  // one winner per contested ring row (patches/kv_tiers.py:272-280)
}

// MODE 0: tiered dual write; 1: INT8 only (ring buffers are the pool); 2: INT4 only.  The row's slot index (and
// in MODE 0 the owner word of its ring row) are wave-uniform scalar loads, issued behind the input loads; the
// scheduling barriers keep the compiler from interleaving input-dependent arithmetic into that chain.
template <int DT, int D, int G8, int MODE, int LM>
__global__ void __launch_bounds__(256) quant_store_kernel(
    RowIn kin, RowIn vin, const void* loc, int loc64, uint32_t NH, int H, uint8_t* k4, uint8_t* v4, uint16_t* ks4,
    uint16_t* vs4, int8_t* rk, int8_t* rv, uint16_t* rks, uint16_t* rvs, const int32_t* owner,
    const uint16_t* sm_k_inv, const uint16_t* sm_v_inv, int64_t ring_mask) {
  const int lane = threadIdx.x & 63;
  uint32_t t;
  int h;
  if (!wave_row(NH, H, &t, &h) || lane >= D / 4) return;
  const int c0 = 4 * lane;
  const In4 rk_in = load4_raw<DT, LM>(kin, t, h, c0, sm_k_inv, D);
  const In4 rv_in = load4_raw<DT, LM>(vin, t, h, c0, sm_v_inv, D);
  __builtin_amdgcn_sched_barrier(0);
  const int64_t slot = load_loc(loc, loc64, t);
  bool hot = false;
  if constexpr (MODE == 0) {
    __builtin_amdgcn_sched_barrier(0);
    hot = (int64_t)owner[slot & ring_mask] == slot;  // stamped by the preceding launch
  }
  __builtin_amdgcn_sched_barrier(0);
  float xk[4], xv[4];
  to_f32<DT, LM>(rk_in, xk);
  to_f32<DT, LM>(rv_in, xv);
  if constexpr (MODE == 0) {
    if (hot) {  // wave-uniform: the whole row belongs to one token
      store_ring_row<D, G8>(rk, rks, slot & ring_mask, H, h, lane, xk);
      store_ring_row<D, G8>(rv, rvs, slot & ring_mask, H, h, lane, xv);
    }
    store_pool_row<D>(k4, ks4, slot, H, h, lane, xk);
    store_pool_row<D>(v4, vs4, slot, H, h, lane, xv);
  } else if constexpr (MODE == 1) {
    store_ring_row<D, G8>(rk, rks, slot, H, h, lane, xk);
    store_ring_row<D, G8>(rv, rvs, slot, H, h, lane, xv);
  } else {
    store_pool_row<D>(k4, ks4, slot, H, h, lane, xk);
    store_pool_row<D>(v4, vs4, slot, H, h, lane, xv);
  }
}

// The ring row about to be overwritten, as loaded ahead of its requantization: this lane's 4 INT8 codes of K and
// of V and the scales of their groups.
struct RingRow {
  uint32_t ck, cv;
  uint16_t sk, sv;
};

template <int D, int G8>
KVT_DEV RingRow load_ring_row(const int8_t* rk, const int8_t* rv, const uint16_t* rks, const uint16_t* rvs,
                              int64_t r, int H, int h, int lane, bool live) {
  constexpr int NG8 = D / G8;
  const int64_t row = r * H + h;
  const uint32_t nc = live ? D : 0, ns = live ? NG8 * 2 : 0;
  const int soff = (4 * lane) / G8 * 2;
  RingRow o;
  o.ck = __builtin_amdgcn_raw_buffer_load_b32(row_rsrc(rk + row * D, nc), 4 * lane, 0, 0);
  o.cv = __builtin_amdgcn_raw_buffer_load_b32(row_rsrc(rv + row * D, nc), 4 * lane, 0, 0);
  o.sk = __builtin_amdgcn_raw_buffer_load_b16(row_rsrc(rks + row * NG8, ns), soff, 0, 0);
  o.sv = __builtin_amdgcn_raw_buffer_load_b16(row_rsrc(rvs + row * NG8, ns), soff, 0, 0);
  return o;
}

// The INT8 ring row part of this lane (codes + group scale) requantized into INT4 pool row `row`.
template <int D>
KVT_DEV void store_pool_requant(uint8_t* pbuf, uint16_t* pscale, int64_t row, int H, int h, int lane, uint32_t codes,
                                uint16_t s8bits) {
  constexpr int NG4 = D / kG4;
  uint16_t sb;
  const uint32_t b = requant4_lane(codes, s8bits, &sb);
  st_row(&reinterpret_cast<uint16_t*>(pbuf + (row * H + h) * (D / 2))[lane], (uint16_t)b);
  if ((lane & 7) == 0) st_row(&pscale[(row * H + h) * NG4 + lane / 8], sb);
}

// Position-indexed ring append with eviction, one (token, head) row per wavefront.  The new K/V inputs are
// loaded first; the row's metadata is wave-uniform and read with scalar loads (their counter is separate from the
// vector loads', so the chain does not wait for the inputs), in dependency levels held apart by scheduling
// barriers: sequence id and position; the sequence's ring placement; then the ring row being overwritten (vector
// loads, none when nothing is evicted) and its page-table entry.  The new token's INT8 row then takes the ring
// row's place and the evicted row, held in registers, is requantized into its INT4 page.
template <int DT, int G8, int LM>
__global__ void __launch_bounds__(256) append_evict_kernel(
    RowIn kin, RowIn vin, const int32_t* seq_ids, const int64_t* positions, uint32_t NH, int H, uint8_t* k4,
    uint8_t* v4, uint16_t* ks4, uint16_t* vs4, int8_t* rk, int8_t* rv, uint16_t* rks, uint16_t* rvs,
    const int64_t* ring_base, const int32_t* ring_len, const int64_t* ring_start, const int32_t* page_table,
    int64_t pt_stride, const uint16_t* sm_k_inv, const uint16_t* sm_v_inv) {
  constexpr int D = 256;
  const int lane = threadIdx.x & 63;
  uint32_t t;
  int h;
  if (!wave_row(NH, H, &t, &h)) return;
  const int c0 = 4 * lane;
  const In4 rk_in = load4_raw<DT, LM>(kin, t, h, c0, sm_k_inv, D);
  const In4 rv_in = load4_raw<DT, LM>(vin, t, h, c0, sm_v_inv, D);
  __builtin_amdgcn_sched_barrier(0);
  const int sq = seq_ids[t];
  const int64_t p = positions[t];
  __builtin_amdgcn_sched_barrier(0);
  const int64_t len = ring_len[sq];
  const int64_t base = ring_base[sq];
  const int64_t start = ring_start[sq];
  __builtin_amdgcn_sched_barrier(0);
  const int64_t r = base + (p & (len - 1));
  const int64_t e = p - len;  // the position whose ring row this token overwrites
  const bool ev = e >= start;
  const RingRow old = load_ring_row<D, G8>(rk, rv, rks, rvs, r, H, h, lane, ev);
  const int pg = page_table[sq * pt_stride + (ev ? e >> 6 : 0)];  // entry 0 of the row when unused
  __builtin_amdgcn_sched_barrier(0);
  const int64_t row = ev && pg >= 0 ? (int64_t)pg * kPage + (e & (kPage - 1)) : -1;  // INT4 row of the evictee
  float xk[4], xv[4];
  to_f32<DT, LM>(rk_in, xk);
  to_f32<DT, LM>(rv_in, xv);
  // The new row goes in first: its stores alias the old row's loads, which keeps those loads up front.
  store_ring_row<D, G8>(rk, rks, r, H, h, lane, xk);
  store_ring_row<D, G8>(rv, rvs, r, H, h, lane, xv);
  if (row >= 0) {
    store_pool_requant<D>(k4, ks4, row, H, h, lane, old.ck, old.sk);
    store_pool_requant<D>(v4, vs4, row, H, h, lane, old.cv, old.sv);
  }
}

// Device-side plan of an evicting append (one block; see kvt_append_plan).  Sequence j of the call appends
// cu[j + 1] - cu[j] tokens at positions L0 .. L0 + n - 1 (L0 = seq_lens[s] before the call).  Positions e that leave
// the ring (e = p - R >= ring_start) and start a page (e % 64 == 0) take the next pages of the free list, in call
// order (sequence j before j + 1, positions ascending): the order in which a host allocator walking the same plan
// pops them.  Then seq_lens[s] = L0 + n.
constexpr int kPlanThreads = 1024;

__global__ void __launch_bounds__(kPlanThreads) append_plan_kernel(
    int n, const int32_t* seqs, const int32_t* cu, int32_t* seq_lens, const int32_t* ring_len,
    const int64_t* ring_start, int32_t* page_table, int64_t pt_stride, int max_pages, const int32_t* free_list,
    int n_pages, int32_t* free_head, int32_t* seq_ids, int64_t* positions, int32_t* status) {
  __shared__ int64_t s_l0[kPlanThreads];
  __shared__ int32_t s_off[kPlanThreads + 1];
  __shared__ int32_t s_cu[kPlanThreads + 1];
  const int j = threadIdx.x;
  int s = 0, np = 0;
  int64_t L0 = 0, lp0 = 0;
  if (j < n) {
    s = seqs[j];
    const int cnt = cu[j + 1] - cu[j];
    L0 = seq_lens[s];
    const int64_t R = ring_len[s], st = ring_start[s];
    const int64_t e0 = max(st, L0 - R), e1 = L0 + cnt - R;
    lp0 = (e0 + kPage - 1) >> 6;
    if (e1 > e0) np = (int)(((e1 + kPage - 1) >> 6) - lp0);
    s_l0[j] = L0;
  }
  if (j < n) s_cu[j] = cu[j];
  if (j == 0) s_cu[n] = cu[n];
  // exclusive scan of the new-page counts over the call's sequences (Hillis-Steele in LDS)
  s_off[j] = np;
  __syncthreads();
  for (int d = 1; d < kPlanThreads; d <<= 1) {
    const int v = j >= d ? s_off[j - d] : 0;
    __syncthreads();
    s_off[j] += v;
    __syncthreads();
  }
  const int incl = s_off[j];
  const int total = s_off[kPlanThreads - 1];
  const int head0 = *free_head;
  if (j < n) {
    const int off = incl - np;
    for (int k = 0; k < np; ++k) {
      const int64_t lp = lp0 + k;
      const int idx = head0 + off + k;
      if (idx >= n_pages) {
        atomicOr(status, 1);        // free list exhausted: the page stays unassigned (the requant is skipped)
      } else if (lp >= max_pages) {
        atomicOr(status, 2);        // page-table row full
      } else {
        page_table[(int64_t)s * pt_stride + lp] = free_list[idx];
      }
    }
  }
  // the tokens' sequence ids and positions (binary search of the token's sequence over cu)
  const int N = s_cu[n];
  for (int i = j; i < N; i += kPlanThreads) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_cu[mid] <= i) lo = mid; else hi = mid - 1;
    }
    seq_ids[i] = seqs[lo];
    positions[i] = s_l0[lo] + (i - s_cu[lo]);
  }
  __syncthreads();   // every thread has read seq_lens (L0) and the head
  if (j < n) seq_lens[s] = (int32_t)(L0 + (s_cu[j + 1] - s_cu[j]));
  if (j == 0) *free_head = min(head0 + total, n_pages);
}

__global__ void page_table_update_kernel(int32_t* pt, int64_t pt_stride, int64_t n, const int32_t* seq,
                                         const int32_t* lpage, const int32_t* ppage) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) pt[(int64_t)seq[i] * pt_stride + lpage[i]] = ppage[i];
}

// ---------------------------------------------------------------------------------------------- dispatch helpers
// The load mode of a launch: vector loads when every 4-channel chunk of k, v (and of the smoothing inverses) is
// aligned to its size and the smoothing inverses are both given or both absent; element loads otherwise.
int load_mode(const RowIn& kin, const RowIn& vin, int dtype, const void* smk, const void* smv) {
  const uintptr_t chunk = dtype == kF32 ? 16 : 8;
  auto ok = [&](const RowIn& in) {
    return (uintptr_t)in.base % chunk == 0 && in.stride_n % 4 == 0 && in.stride_h % 4 == 0;
  };
  if (!ok(kin) || !ok(vin) || (uintptr_t)smk % 8 != 0 || (uintptr_t)smv % 8 != 0) return kLoadElem;
  if (smk == nullptr && smv == nullptr) return kLoadVec;
  return smk != nullptr && smv != nullptr ? kLoadVecSm : kLoadElem;
}

template <int MODE>
int launch_quant_store(const RowIn& kin, const RowIn& vin, int dtype, const void* loc, int loc64, int64_t N, int H,
                       int D, int group8, uint8_t* k4, uint8_t* v4, uint16_t* ks4, uint16_t* vs4, int8_t* rk,
                       int8_t* rv, uint16_t* rks, uint16_t* rvs, const int32_t* owner, const uint16_t* smk,
                       const uint16_t* smv, int64_t ring_mask, hipStream_t stream) {
  const dim3 grid((unsigned)((N * H + kWavesPerBlock - 1) / kWavesPerBlock));
  const int lm = load_mode(kin, vin, dtype, smk, smv);
  const uint32_t NH = (uint32_t)(N * H);
#define KVT_QS1(DT_, D_, G_, LM_)                                                                                  \
  hipLaunchKernelGGL((quant_store_kernel<DT_, D_, G_, MODE, LM_>), grid, dim3(256), 0, stream, kin, vin, loc,      \
                     loc64, NH, H, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, smk, smv, ring_mask)
#define KVT_QS(DT_, D_, G_)              \
  if (lm == kLoadVec) {                  \
    KVT_QS1(DT_, D_, G_, kLoadVec);      \
  } else if (lm == kLoadVecSm) {         \
    KVT_QS1(DT_, D_, G_, kLoadVecSm);    \
  } else {                               \
    KVT_QS1(DT_, D_, G_, kLoadElem);     \
  }
#define KVT_QS_G(DT_, D_)                     \
  if (group8 == 64) {                         \
    KVT_QS(DT_, D_, 64)                       \
  } else if (group8 == D_ && D_ != 64) {      \
    KVT_QS(DT_, D_, D_)                       \
  } else {                                    \
    return KVT_EINVAL;                        \
  }
#define KVT_QS_D(DT_)          \
  if (D == 256) {              \
    KVT_QS_G(DT_, 256)         \
  } else if (D == 128) {       \
    KVT_QS_G(DT_, 128)         \
  } else if (D == 64) {        \
    KVT_QS(DT_, 64, 64)        \
  } else {                     \
    return KVT_EINVAL;         \
  }
  if (dtype == kBF16) {
    KVT_QS_D(kBF16)
  } else if (dtype == kF16) {
    KVT_QS_D(kF16)
  } else if (dtype == kF32) {
    KVT_QS_D(kF32)
  } else {
    return KVT_EINVAL;
  }
#undef KVT_QS_D
#undef KVT_QS_G
#undef KVT_QS
#undef KVT_QS1
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // namespace

extern "C" {

int kvt_quant_store_tiered(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                           int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                           void* v_buf, void* k_scale, void* v_scale, void* ring_k, void* ring_v, void* ring_ks,
                           void* ring_vs, void* owner, const void* sm_k_inv, const void* sm_v_inv, int64_t ring_mask,
                           int group8, void* stream) {
  if (N < 0 || H <= 0 || N > INT32_MAX / H || ring_mask < 0 || ((ring_mask + 1) & ring_mask) != 0) return KVT_EINVAL;
  if (N == 0) return KVT_OK;
  hipStream_t st = (hipStream_t)stream;
  const unsigned sblocks = (unsigned)((N + 255) / 256);
  hipLaunchKernelGGL(stamp_owner_kernel, dim3(sblocks), dim3(256), 0, st, loc, loc_is_int64, N, (int32_t*)owner,
                     ring_mask);
  KVT_CHECK_LAUNCH();
  return launch_quant_store<0>(RowIn{k, sk_n, sk_h}, RowIn{v, sv_n, sv_h}, dtype, loc, loc_is_int64, N, H, D, group8,
                               (uint8_t*)k_buf, (uint8_t*)v_buf, (uint16_t*)k_scale, (uint16_t*)v_scale,
                               (int8_t*)ring_k, (int8_t*)ring_v, (uint16_t*)ring_ks, (uint16_t*)ring_vs,
                               (const int32_t*)owner, (const uint16_t*)sm_k_inv, (const uint16_t*)sm_v_inv,
                               ring_mask, st);
}

int kvt_quant_store_int8(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                         int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                         void* v_buf, void* k_scale, void* v_scale, const void* sm_k_inv, const void* sm_v_inv,
                         int group8, void* stream) {
  if (N < 0 || H <= 0 || N > INT32_MAX / H) return KVT_EINVAL;
  if (N == 0) return KVT_OK;
  return launch_quant_store<1>(RowIn{k, sk_n, sk_h}, RowIn{v, sv_n, sv_h}, dtype, loc, loc_is_int64, N, H, D, group8,
                               nullptr, nullptr, nullptr, nullptr, (int8_t*)k_buf, (int8_t*)v_buf,
                               (uint16_t*)k_scale, (uint16_t*)v_scale, nullptr, (const uint16_t*)sm_k_inv,
                               (const uint16_t*)sm_v_inv, 0, (hipStream_t)stream);
}

int kvt_quant_store_int4(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n,
                         int64_t sv_h, const void* loc, int loc_is_int64, int64_t N, int H, int D, void* k_buf,
                         void* v_buf, void* k_scale, void* v_scale, const void* sm_k_inv, const void* sm_v_inv,
                         void* stream) {
  if (N < 0 || H <= 0 || N > INT32_MAX / H) return KVT_EINVAL;
  if (N == 0) return KVT_OK;
  return launch_quant_store<2>(RowIn{k, sk_n, sk_h}, RowIn{v, sv_n, sv_h}, dtype, loc, loc_is_int64, N, H, D, 64,
                               (uint8_t*)k_buf, (uint8_t*)v_buf, (uint16_t*)k_scale, (uint16_t*)v_scale, nullptr,
                               nullptr, nullptr, nullptr, nullptr, (const uint16_t*)sm_k_inv,
                               (const uint16_t*)sm_v_inv, 0, (hipStream_t)stream);
}

int kvt_page_table_update(void* page_table, int64_t pt_stride, int64_t n, const void* seq, const void* lpage,
                          const void* ppage, void* stream) {
  if (n < 0 || pt_stride <= 0) return KVT_EINVAL;
  if (n == 0) return KVT_OK;
  hipLaunchKernelGGL(page_table_update_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (int32_t*)page_table, pt_stride, n, (const int32_t*)seq, (const int32_t*)lpage,
                     (const int32_t*)ppage);
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

int kvt_append_plan(int n, const void* seqs, const void* cu, void* seq_lens, const void* ring_len,
                    const void* ring_start, void* page_table, int64_t pt_stride, int max_pages, const void* free_list,
                    int n_pages, void* free_head, void* seq_ids, void* positions, void* status, void* stream) {
  if (n < 0 || n > kPlanThreads || pt_stride <= 0 || max_pages <= 0 || max_pages > pt_stride || n_pages < 0)
    return n > kPlanThreads ? KVT_ERANGE : KVT_EINVAL;
  if (n == 0) return KVT_OK;
  hipLaunchKernelGGL(append_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, n, (const int32_t*)seqs,
                     (const int32_t*)cu, (int32_t*)seq_lens, (const int32_t*)ring_len, (const int64_t*)ring_start,
                     (int32_t*)page_table, pt_stride, max_pages, (const int32_t*)free_list, n_pages,
                     (int32_t*)free_head, (int32_t*)seq_ids, (int64_t*)positions, (int32_t*)status);
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

int kvt_append_evict(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n, int64_t sv_h,
                     const void* seq_ids, const void* positions, int64_t N, int H, int D, void* k_buf, void* v_buf,
                     void* k_scale, void* v_scale, void* ring_k, void* ring_v, void* ring_ks, void* ring_vs,
                     const void* ring_base, const void* ring_len, const void* ring_start, const void* page_table,
                     int64_t pt_stride, const void* sm_k_inv, const void* sm_v_inv, int group8, void* stream) {
  if (N < 0 || H <= 0 || N > INT32_MAX / H) return KVT_EINVAL;
  if (N == 0) return KVT_OK;
  const dim3 grid((unsigned)((N * H + kWavesPerBlock - 1) / kWavesPerBlock));
  hipStream_t st = (hipStream_t)stream;
  const RowIn kin{k, sk_n, sk_h}, vin{v, sv_n, sv_h};
  const int lm = load_mode(kin, vin, dtype, sm_k_inv, sm_v_inv);
  const uint32_t NH = (uint32_t)(N * H);
#define KVT_AE1(DT_, G_, LM_)                                                                                      \
  hipLaunchKernelGGL((append_evict_kernel<DT_, G_, LM_>), grid, dim3(256), 0, st, kin, vin,                        \
                     (const int32_t*)seq_ids, (const int64_t*)positions, NH, H, (uint8_t*)k_buf, (uint8_t*)v_buf,  \
                     (uint16_t*)k_scale, (uint16_t*)v_scale, (int8_t*)ring_k, (int8_t*)ring_v, (uint16_t*)ring_ks, \
                     (uint16_t*)ring_vs, (const int64_t*)ring_base, (const int32_t*)ring_len,                      \
                     (const int64_t*)ring_start, (const int32_t*)page_table, pt_stride, (const uint16_t*)sm_k_inv, \
                     (const uint16_t*)sm_v_inv)
#define KVT_AE(DT_, G_)                \
  if (lm == kLoadVec) {                \
    KVT_AE1(DT_, G_, kLoadVec);        \
  } else if (lm == kLoadVecSm) {       \
    KVT_AE1(DT_, G_, kLoadVecSm);      \
  } else {                             \
    KVT_AE1(DT_, G_, kLoadElem);       \
  }
#define KVT_AE_G(DT_)              \
  if (group8 == 64) {              \
    KVT_AE(DT_, 64)                \
  } else if (group8 == 256) {      \
    KVT_AE(DT_, 256)               \
  } else {                         \
    return KVT_EINVAL;             \
  }
  if (D != 256) return KVT_EINVAL;
  if (dtype == kBF16) {
    KVT_AE_G(kBF16)
  } else if (dtype == kF16) {
    KVT_AE_G(kF16)
  } else if (dtype == kF32) {
    KVT_AE_G(kF32)
  } else {
    return KVT_EINVAL;
  }
#undef KVT_AE_G
#undef KVT_AE
#undef KVT_AE1
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
