// Split-K GQA decode attention over the position-indexed tiered cache, full pool rows per wavefront (gfx950 matrix
// cores).  For two KV heads with up to 8 q heads each (the configurations' 16 / 2): a wavefront reads and computes
// BOTH KV heads of every position it takes, so each copy instruction covers whole pool rows (2 heads x 128 B of INT4
// codes, 2 x 256 B of INT8 ring codes) and the 16 accumulator rows are 16 distinct q heads.
//
// Work split: a sequence's positions are cut into n_b block ranges of equal cost (a ring position costs kHotCost4 / 4
// of a paged one; paged boundaries are multiples of 16), one block of 8 wavefronts per range and CU.  Inside a block,
// 16-position paged tiles (one quarter page: 2 x 2 KB of K codes, 2 x 2 KB of V codes, 1 KB of scales) and
// 8-position ring tiles go to the wavefronts one at a time from counters in LDS (first come) or in a fixed order
// (bit-reproducible), double-buffered per wavefront with direct-to-LDS copies.
//
// Start-up: a decode plan (kvt_decode_plan, one small launch per decode step shared by every layer) holds each
// block's ranges and the pool rows of its first tiles, so a block's first copies go out after one load.  A block
// checks the plan against the sequence's current length and ring placement (loaded at the same time) and computes
// its ranges itself when they differ or when no plan is given.
//
// Paged tile math (one 16 x 16 x 32 f16 MFMA shape throughout):
//   QK^T: the contraction index k = 8 kb + e of lane (n16, kb) covers head kb >> 1 and 8 channels of one half of a
//     32-channel scale group, so one MFMA takes 16 channels of both heads and its B operand (Q) is zero wherever the
//     q head of the column belongs to the other KV head: D[token, q head] = K_head(q) . Q over those channels.  Two
//     MFMAs per scale group; the A operand is the raw magic-number values of the codes (0x6400 | nibble = 1024 + n,
//     0x6400 | nibble << 4 = 1024 + 16 n for odd channels, whose Q entries are divided by 16).  The constant excess
//     (1032 q, resp. 1152 q / 16) is removed by one bias MFMA per tile whose A operand is the token's 8 group scales
//     of each head and whose B operand is -bias as two fp16 parts, zero for the other head; group scales fold into
//     the fp32 group results.  Lane (q head n16, kb) ends with the scores of tokens 4 kb .. 4 kb + 3 of its own head.
//   P.V: k = 8 kb + e <-> (head e >= 4, token 4 kb + (e & 3)): the A operand is P * s_v of the lane's 4 tokens in the
//     positions of its head and zero in the other head's, B the raw magic V codes of the 8 (head, token) rows from
//     one ds_read_b64_tr_b4 (a 16 x 16 nibble transpose per 16 lanes), C = -(1032 | 1152): one pass over 2 x 16
//     positions per scale group and 16-channel half, no V code ever multiplied on the VALU.
// Ring tiles (INT8 codes, exact fp16): QK^T rows are (head, token) pairs (8 tokens x 2 heads), the scores of a row
//   whose head is not the column's are dropped (-inf); P.V on 16 x 16 x 16 f16 with k = the same (head, token)
//   pairs, B from ds_read_b64_tr_b8.
// The block's wavefronts merge (max, sum, o) of the 16 q heads in LDS; one fp32 partial per (split, q head) goes to
// kvt_decode_combine, in the slot layout of the head-wise kernel (decode_mfma.hip).
//
// Numerics versus the oracle (bf16(code * scale) rows, fp32 softmax) as in the head-wise kernel: codes enter exactly,
// K scales in fp32, V scales through fp16 P * s (P <= 1), fp32 accumulation.

#include "decode_common.h"
#include "kvtier.h"

using namespace kvt;
using namespace kvt::dec;

namespace {

constexpr int kWaves = 8;
constexpr int kD = 256;
constexpr int kH = 2;
constexpr int kTile = 16;          // positions per paged tile
constexpr int kRingTile = 8;       // positions per ring tile
constexpr int kHotCost4 = 7;       // cost of a ring position in the split (a paged position costs 4)
constexpr int kBlockPages = 1024;  // page ids of a block's paged range staged in LDS per round
constexpr int kPlanWords = 64;     // int32 words of one block's plan entry
constexpr int kPlanRows = 32;      // plan word of the first tile row
constexpr int kPlanTiles = 16;     // tile rows in a plan entry (tiles w and w + kWaves of every wavefront)
constexpr uint32_t kNoRow = 0xffffffffu;

// One 16-position paged tile of both KV heads in LDS.
struct RowStage {
  uint8_t k[kTile * 256];   // K codes [token][head][128 B]; 16-B chunk c = 8 head + group of token t in slot
                            // slot_of(t, c)
  uint8_t v[kTile * 256];   // V codes, same layout
  uint16_t ks[kTile][16];   // K scales [token][8 head + group], as copied
  union {
    uint16_t vsn[kTile][16];  // V scales as copied ...
    uint16_t sv[8][32];       // ... then in place [group][k], k = 8 kb + e <-> (head e >= 4, token 4 kb + (e & 3))
  };
};

// One 8-position ring tile of both KV heads in LDS.
struct RingStage {
  uint8_t k[kRingTile * 512];   // K codes [token][head][256 B]; 16-B chunk c = 16 head + j in slot ring_slot(t, c)
  uint8_t v[kRingTile * 512];   // V codes, same layout
  uint16_t ks[kRingTile][8];    // 16 B copied from the dword holding the token's first scale (both heads)
  uint16_t vs[kRingTile][8];
};

// A wavefront's result at the end, in its own staging area (no other wavefront touches it, so it is written as soon
// as the wavefront's last tile is done): o[dim][16 q head columns] unscaled, the float4 of columns 4 j .. 4 j + 3 in
// slot j ^ ((dim >> 2) & 3) (16 lanes of a write or a read then cover all 64 banks), and the column's (max, sum).
struct WaveResult {
  float o[kD * 16];
  float m[16];
  float l[16];
};

union WaveArea {
  RowStage row[2];
  RingStage ring[2];
  WaveResult res;
};

struct BlockQueue {
  int32_t cold_next;
  int32_t hot_next;
  int32_t pages[kBlockPages];   // physical page of the round's page pg0 + i
};

// The B operands of the paged QK^T, built once per block: column n16, half hf of group g, channel octet dsel at byte
// n16 * kQPitch + 64 g + 32 hf + 16 dsel (the pitch of 512 + 16 bytes spreads 8 consecutive columns over the bank
// groups); lanes whose column belongs to the other KV head read the zero rows instead.
constexpr int kQPitch = 528;
struct alignas(16) QArea {
  uint8_t op[16 * kQPitch];
  uint8_t zero[512];
  float bias[16][8];   // bias_g of each column (the constant excess of its magic-number products)
};

struct Lds {
  WaveArea w[kWaves];
  BlockQueue q;
  union {
    QArea qa;
    float wgt[kWaves][16];   // merge weights e^(m_w - M) per wavefront and column (after the tiles)
  };
};

// Slot of 16-byte chunk c (head c >> 3, group c & 7) in token row t: head-0 chunks stay in slots 0-7, head-1 chunks
// in 8-15, and the group is XORed with (t & 7) ^ 4 head.  The QK^T reads then hit each 16-byte bank group twice per
// 32 lanes (the minimum for one dword per lane) and the transposed P.V reads (4 tokens x 2 heads x 2 halves per 16
// lanes) hit 8 distinct bank groups (conflict-free).  An involution: slot_of(t, slot_of(t, c)) = c.
KVT_DEV uint32_t slot_of(int t, int c) { return (uint32_t)(c ^ ((t & 7) ^ (4 * (c >> 3)))); }

// Slot of 16-byte chunk c (head c >> 4, 16 channels c & 15) in ring token row t (32 chunks of 16 B): the 16 channels
// are XORed with (t & 7) ^ 4 head, so the transposed P.V reads (4 tokens x 2 channel blocks x 2 halves per 16 lanes)
// are conflict-free.
KVT_DEV uint32_t ring_slot(int t, int c) { return (uint32_t)(c ^ ((t & 7) ^ (4 * (c >> 4)))); }

struct RowCtx {
  i32x4 rk4, rv4, rks4, rvs4;   // buffer resources of this layer's INT4 pool (codes K/V, scales K/V)
  uint32_t coff[4];             // this lane's code byte offset in copy j of a tile, relative to row0 * 256
};

KVT_DEV void row_lane_offsets(RowCtx& C) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 4 * j + (lane >> 4);
    C.coff[j] = (uint32_t)t * 256u + 16u * slot_of(t, lane & 15);
  }
}

// Direct-to-LDS copies of one 16-position paged tile (pool rows row0 .. row0 + 15, n valid) into `st`:
// row_issue_k copies the K codes and K scales, row_issue_v the V codes and V scales, exactly 5 vector-memory
// instructions each; the tile loop's vmcnt accounting relies on these counts.  Copy j of the codes moves 4 whole rows
// (1 KB); rows beyond n are copied as they are (they lie in the same page: finite codes, masked scores), the scale
// rows of tokens beyond n repeat row n - 1, so every scale that meets a zero probability is finite.  row0 = kNoRow:
// the copies fall outside the buffer (zeros, no memory traffic), so the instruction count stays fixed.  The V scales
// travel with the V codes because the P.V operand's transposed scales take their place in LDS (row_scatter_vs): a
// stage's V half is rewritten only after its P.V has read it.
KVT_DEV uint32_t row_scale_off(uint32_t row0, int n) {
  const int lane = threadIdx.x & 63;
  const uint32_t tl = (uint32_t)min((lane & 31) >> 1, n - 1);
  return row0 == kNoRow ? 0x80000000u : (row0 + tl) * 32u + 16u * (uint32_t)(lane & 1);
}

KVT_DEV void row_issue_k(const RowCtx& C, RowStage& st, uint32_t row0, int n) {
  const int lane = threadIdx.x & 63;
  const uint32_t cb = row0 == kNoRow ? 0x80000000u : row0 * 256u;
#pragma unroll
  for (int j = 0; j < 4; ++j) copy16_to_lds(C.rk4, st.k + 1024 * j, cb + C.coff[j]);
  const uint32_t soff = row_scale_off(row0, n);
  if (lane < 32) copy16_to_lds(C.rks4, &st.ks[0][0], soff);
}

KVT_DEV void row_issue_v(const RowCtx& C, RowStage& st, uint32_t row0, int n) {
  const int lane = threadIdx.x & 63;
  const uint32_t cb = row0 == kNoRow ? 0x80000000u : row0 * 256u;
#pragma unroll
  for (int j = 0; j < 4; ++j) copy16_to_lds(C.rv4, st.v + 1024 * j, cb + C.coff[j]);
  const uint32_t soff = row_scale_off(row0, n);
  if (lane < 32) copy16_to_lds(C.rvs4, &st.vsn[0][0], soff);
}

// V scales of the tile into the [group][k] layout of the P.V operand, in place (lanes 0-31: one (token, head) each;
// every lane's read returns before any lane writes: one wavefront, reads then writes).
KVT_DEV void row_scatter_vs(RowStage& st) {
  const int lane = threadIdx.x & 63;
  uint4 vs = {0u, 0u, 0u, 0u};
  const int t = (lane & 31) >> 1, h = lane & 1;
  if (lane < 32) vs = *reinterpret_cast<const uint4*>(&st.vsn[t][8 * h]);
  wait_lgkm0();
  if (lane < 32) {
    const uint32_t v[4] = {vs.x, vs.y, vs.z, vs.w};
    const int k = 8 * (t >> 2) + 4 * h + (t & 3);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      st.sv[2 * g][k] = (uint16_t)(v[g] & 0xffffu);
      st.sv[2 * g + 1][k] = (uint16_t)(v[g] >> 16);
    }
  }
}

// Constants of the paged tile math for lane (n16, kb): qb = LDS address of the lane's QK^T B operands (column n16,
// octet kb & 1, or the zero rows when the column's KV head is not kb >> 1); kbias the B operand of the bias MFMA (kb
// even / odd: leading / remainder fp16 part of -bias_g * 2^-bexp, zero for the other head); bexp the column's power of
// two, the same in all 4 lanes of a column.
struct RowMath {
  uint32_t qb;
  h8 kbias;
  int bexp;
  float cscale;
  NibbleMasks nm;
};

// Wavefront w builds the QK^T B operands of scale group g = w for every column: channels 32 g + 16 hf + 8 (kb & 1) +
// [0, 4, 1, 5, 2, 6, 3, 7] of the column's q head (odd channels / 16) in fp16, written by the lanes whose column belongs
// to KV head kb >> 1, and bias_g = sum (1032 | 1152) * operand over the group's 32 channels (lanes kb and kb ^ 1 hold
// 16 each).  Wavefront 0 also clears the zero rows.  Published by the caller's next barrier.
KVT_DEV void q_build(QArea& qa, const uint16_t* qrow, bool valid, int wave) {
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4, dsel = kb & 1;
  const bool own = (kb >> 1) == (n16 >> 3);
  const int g = wave;
  uint4 raw[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) raw[hf] = *reinterpret_cast<const uint4*>(qrow + 32 * g + 16 * hf + 8 * dsel);
  float part = 0.0f;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const uint32_t w[4] = {raw[hf].x, raw[hf].y, raw[hf].z, raw[hf].w};
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = __uint_as_float(w[j] << 16);
      x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
    h8 op;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool odd = (e & 2) != 0;   // positions 2, 3, 6, 7 hold channels 1, 5, 3, 7 of the octet
      const float xv = valid ? x[perm[e]] : 0.0f;
      const _Float16 hq = (_Float16)(odd ? xv * 0.0625f : xv);
      op[e] = hq;
      part = fmaf(odd ? 1152.0f : 1032.0f, (float)hq, part);
    }
    if (own) *reinterpret_cast<u4v*>(&qa.op[n16 * kQPitch + 64 * g + 32 * hf + 16 * dsel]) = as_u4(op);
  }
  // the other 16 channels of the group sit in lane kb ^ 1 (lane ^ 16)
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(part), __float_as_uint(part), false, false);
  const float bias = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  if (own && dsel == 0) qa.bias[n16][g] = bias;
  if (wave == 0) *reinterpret_cast<uint2*>(&qa.zero[8 * lane]) = make_uint2(0u, 0u);
}

// After q_build's barrier: the lane's operand address, bexp and bias operand.
KVT_DEV void q_finish(const QArea& qa, RowMath& M) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4, dsel = kb & 1;
  const bool own = (kb >> 1) == (n16 >> 3);
  M.qb = own ? lds_off(&qa.op[n16 * kQPitch + 16 * dsel]) : lds_off(&qa.zero[16 * dsel]);
  const f4 b0 = *reinterpret_cast<const f4*>(&qa.bias[n16][0]);
  const f4 b1 = *reinterpret_cast<const f4*>(&qa.bias[n16][4]);
  const float bias[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
  float amax = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) amax = fmaxf(amax, fabsf(bias[g]));
  M.bexp = amax > 0.0f ? ilogbf(amax) - 14 : 0;   // |bias| * 2^-bexp < 2^15
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const float sb = -ldexpf(bias[g], -M.bexp);
    const _Float16 hi = (_Float16)sb;
    const _Float16 lo = (_Float16)(sb - (float)hi);
    M.kbias[g] = own ? (dsel ? lo : hi) : (_Float16)0.0f;
  }
}

// QK^T of one staged tile: lane (n16, kb) gets the scores (log2 units) of its column's q head for tokens 4 kb + r.
KVT_DEV void row_qk(const RowStage& st, const RowMath& M, float s[4]) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  const int ha = kb >> 1, hc = n16 >> 3;
  const uint32_t mlo = M.nm.lo, mhi = M.nm.hi, magic = M.nm.magic;
  // A operand: dword 2 hf + (kb & 1) of chunk 8 ha + g of token n16 (slot 8 ha + (g ^ key))
  const uint32_t key = (uint32_t)((n16 & 7) ^ (4 * ha));
  const uint32_t base = lds_off(st.k) + (uint32_t)(n16 * 256 + 128 * ha + 4 * (kb & 1));
  uint32_t w[8][2];
#pragma unroll
  for (int g = 0; g < 8; ++g)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) w[g][hf] = *(const lds_u32*)(uintptr_t)(base + 16u * ((uint32_t)g ^ key) + 8u * hf);
  uint4 ksr[4];   // the group scales of the lane's 4 tokens, head hc
#pragma unroll
  for (int r = 0; r < 4; ++r) ksr[r] = *reinterpret_cast<const uint4*>(&st.ks[4 * kb + r][8 * hc]);
  // bias term -sum_g s_g(t) bias_g: A = the 8 group scales of token n16, head ha (scaled by 2^-bexp in the MFMA)
  const h8 srow = as_h8(*reinterpret_cast<const u4v*>(&st.ks[n16][8 * ha]));
  const f4 bsum = mfma(srow, M.kbias, f4{0.f, 0.f, 0.f, 0.f});
  auto qop = [&](int g, int hf) -> h8 { return as_h8(*(const lds_u4v*)(uintptr_t)(M.qb + 64u * g + 32u * hf)); };
  f4 dp = mfma(int4_codes_raw(w[0][0], mlo, mhi, magic), qop(0, 0), f4{0.f, 0.f, 0.f, 0.f});
  dp = mfma(int4_codes_raw(w[0][1], mlo, mhi, magic), qop(0, 1), dp);
  f4 sc;
#pragma unroll
  for (int r = 0; r < 4; ++r) sc[r] = ldexpf(bsum[r], M.bexp);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    f4 dn = dp;
    if (g + 1 < 8) {
      dn = mfma(int4_codes_raw(w[g + 1][0], mlo, mhi, magic), qop(g + 1, 0), f4{0.f, 0.f, 0.f, 0.f});
      dn = mfma(int4_codes_raw(w[g + 1][1], mlo, mhi, magic), qop(g + 1, 1), dn);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t pairw = g < 2 ? ksr[r].x : g < 4 ? ksr[r].y : g < 6 ? ksr[r].z : ksr[r].w;
      const float sg = f16_bits_to_f32((uint16_t)((g & 1) ? (pairw >> 16) : (pairw & 0xffffu)));
      sc[r] = fmaf(sg, dp[r], sc[r]);
    }
    dp = dn;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) s[r] = sc[r] * M.cscale;
}

// Scores of tokens >= n (a partial last tile) to -inf.
KVT_DEV void row_mask(float s[4], int n) {
  const int kb = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) s[r] = (4 * kb + r) < n ? s[r] : -INFINITY;
}

// Online softmax over a lane's 4 scores (the 16 tokens of a column across its 4 lanes).  Rescales acc and l_run when
// the running max grows; returns P in the A operand layout of P.V: the lane's 4 weights (tokens 2, 3 divided by 16) in
// positions 4 hc .. 4 hc + 3, zero in the other head's.
KVT_DEV u4v row_softmax(const float s[4], f4 acc[16], float& m_run, float& l_run) {
  const int lane = threadIdx.x & 63;
  const int kb = lane >> 4, hc = (lane & 15) >> 3;
  float mloc = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mloc = max_xor16_32(mloc);
  const float m_new = fmaxf(m_run, mloc);
  if (__any(m_new > m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * kb + i, 64);   // lane 4 kb + i: the head of row 4 kb + i
#pragma unroll
    for (int a = 0; a < 16; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[a][i] *= arow[i];
  }
  m_run = m_new;
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
  l_run += (p[0] + p[1]) + (p[2] + p[3]);
  const h2 sc16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t p01 = as_u32(h2{(_Float16)p[0], (_Float16)p[1]});
  const uint32_t p23 = as_u32(h2{(_Float16)p[2], (_Float16)p[3]} * sc16);
  return hc == 0 ? u4v{p01, p23, 0u, 0u} : u4v{0u, 0u, p01, p23};
}

// P.V of one staged tile: acc[2 g + hf] += A_g * B_{g,hf} + A_g * C, A_g = P16 * s_v (k = (head, token) pairs),
// B_{g,hf} = raw magic V codes of channels 32 g + 16 hf + j, C = -(1032 | 1152).  Source lane s (< 8) of a 16-lane
// group supplies 8 bytes of (head (s >> 1) & 1, token 4 kb + 2 (s & 1) + (s >> 2)), lanes 8-15 the same rows' next 8
// bytes: after the transpose the nibbles n0..n7 of a lane hold operand positions [0, 2, 4, 6, 1, 3, 5, 7], which
// int4_codes_raw puts back in order.
KVT_DEV void row_pv(const RowStage& st, u4v p16, NibbleMasks nm, f4 acc[16]) {
  const int lane = threadIdx.x & 63;
  const int k = lane & 15, kb = lane >> 4;
  const int s = k & 7;
  const int h = (s >> 1) & 1;
  const int t = 4 * kb + 2 * (s & 1) + (s >> 2);
  const uint32_t key = (uint32_t)((t & 7) ^ (4 * h));
  const uint32_t vbase = lds_off(st.v) + (uint32_t)(t * 256 + 128 * h + 8 * (k >> 3));
  const h8 bc = {(_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1152.0f, (_Float16)-1152.0f,
                 (_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1152.0f, (_Float16)-1152.0f};
  const h8 pa = as_h8(p16);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const v2i raw = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i*)(uintptr_t)(vbase + 16u * ((uint32_t)g ^ key)));
    const h8 sg = as_h8(*reinterpret_cast<const u4v*>(&st.sv[g][8 * kb]));
    const h8 a = pa * sg;
    acc[2 * g] = mfma(a, int4_codes_raw((uint32_t)raw.x, nm.lo, nm.hi, nm.magic), acc[2 * g]);
    acc[2 * g + 1] = mfma(a, int4_codes_raw((uint32_t)raw.y, nm.lo, nm.hi, nm.magic), acc[2 * g + 1]);
    acc[2 * g] = mfma(a, bc, acc[2 * g]);
    acc[2 * g + 1] = mfma(a, bc, acc[2 * g + 1]);
  }
}

// One round of a block's paged range: positions [c0, c1) (c0 16-aligned) in 16-position tiles; the round's page ids
// sit in LDS.
struct RowRound {
  int64_t c0, c1, pg0;
  int ntiles;
  int32_t* next;
  const int32_t* pages;
  bool dyn;
  mutable int taken;
  KVT_DEV int grab() const { return take_tile<kWaves>(next, dyn, taken); }
  KVT_DEV uint32_t row0(int t) const {
    const int64_t p = c0 + kTile * (int64_t)t;
    const uint32_t page = (uint32_t)__builtin_amdgcn_readfirstlane(pages[(p >> 6) - pg0]);
    return page * (uint32_t)kPage + (uint32_t)(p & (kPage - 1));
  }
  KVT_DEV int n(int t) const { return (int)min((int64_t)kTile, c1 - (c0 + kTile * (int64_t)t)); }
};

// The tiles a wavefront has in hand: ta (P in p16, V in stage S), tb (stage S ^ 1), tc (next to issue), td (taken
// during the step).
struct Hand {
  int ta, tb, tc, td;
};

// One step of the software pipeline: P.V of tile ta (stage S), then QK^T + softmax of tile tb (stage S ^ 1).  In
// flight on entry, oldest first: V half of ta (5 copies), K half of tb (5), V half of tb (5).  The step issues tc's K
// half into stage S (whose K codes and scales ta no longer needs) before the math and tc's V half right after P.V
// (the bytes in flight per CU set the streaming rate).
template <int S>
KVT_DEV void row_step(const RowCtx& C, WaveArea& W, const RowRound& Q, Hand& hd, const RowMath& M, f4 acc[16],
                      float& m_run, float& l_run, u4v& p16) {
  const bool more = hd.tc < Q.ntiles;
  const uint32_t rowc = more ? Q.row0(hd.tc) : kNoRow;
  const int nc = more ? Q.n(hd.tc) : kTile;
  row_issue_k(C, W.row[S], rowc, nc);     // (dummies past the end: fixed counts)
  wait_vmcnt<10>();                       // K half of tb has landed (and V half of ta before it)
  hd.td = more ? Q.grab() : Q.ntiles;
  row_scatter_vs(W.row[S]);               // ta's V scales, in place
  wave_sync();
  float s[4];
  row_pv(W.row[S], p16, M.nm, acc);
  wait_lgkm0();                           // ta's V reads are done before its stage takes new V copies
  row_issue_v(C, W.row[S], rowc, nc);     // (as early as possible: the copies in flight bound the stream)
  row_qk(W.row[S ^ 1], M, s);
  __builtin_amdgcn_s_setprio(1);          // the softmax chain ahead of the other wavefront's work on the SIMD
  row_mask(s, Q.n(hd.tb));
  p16 = row_softmax(s, acc, m_run, l_run);
  __builtin_amdgcn_s_setprio(0);
  hd.ta = hd.tb;
  hd.tb = hd.tc;
  hd.tc = hd.td;
}

// The rest of a round once tiles ta (stage 0) and tb (stage 1, if any) are in flight: the pipeline until the block's
// tiles run out.
KVT_DEV void row_round_run(const RowCtx& C, WaveArea& W, const RowRound& Q, Hand& hd, const RowMath& M, f4 acc[16],
                           float& m_run, float& l_run) {
  if (hd.tb < Q.ntiles) wait_vmcnt<15>(); else wait_vmcnt<5>();   // K half of ta
  wave_sync();
  u4v p16;
  {
    float s[4];
    row_qk(W.row[0], M, s);
    const int n0 = Q.n(hd.ta);
    if (n0 < kTile) row_mask(s, n0);
    p16 = row_softmax(s, acc, m_run, l_run);
  }
  int sa = 0;   // stage of ta
  while (hd.tb < Q.ntiles) {
    row_step<0>(C, W, Q, hd, M, acc, m_run, l_run, p16);
    sa = 1;
    if (hd.tb >= Q.ntiles) break;
    row_step<1>(C, W, Q, hd, M, acc, m_run, l_run, p16);
    sa = 0;
  }
  wait_vmcnt<0>();
  wave_sync();
  row_scatter_vs(W.row[sa]);
  wave_sync();
  row_pv(W.row[sa], p16, M.nm, acc);
  wait_lgkm0();
  wave_sync();
}

// A later round of a block's paged range: tiles from the block counter until none is left.
KVT_DEV void row_round(const RowCtx& C, WaveArea& W, const RowRound& Q, const RowMath& M, f4 acc[16], float& m_run,
                       float& l_run) {
  Hand hd;
  hd.ta = Q.grab();
  if (hd.ta >= Q.ntiles) return;
  hd.tb = Q.grab();
  hd.tc = hd.tb < Q.ntiles ? Q.grab() : Q.ntiles;
  hd.td = Q.ntiles;
  wave_sync();
  const uint32_t r0 = Q.row0(hd.ta);
  row_issue_k(C, W.row[0], r0, Q.n(hd.ta));
  row_issue_v(C, W.row[0], r0, Q.n(hd.ta));
  if (hd.tb < Q.ntiles) {
    const uint32_t r1 = Q.row0(hd.tb);
    row_issue_k(C, W.row[1], r1, Q.n(hd.tb));
    row_issue_v(C, W.row[1], r1, Q.n(hd.tb));
  }
  row_round_run(C, W, Q, hd, M, acc, m_run, l_run);
}

// ---- ring tiles: 8 positions x 2 heads, INT8 codes, scale groups of G8 channels

struct RingCtx {
  i32x4 rk, rv, rks, rvs;   // buffer resources over this sequence's ring rows (codes K/V, scales K/V)
  uint32_t srowbytes;       // H * (256 / G8) * 2: scale bytes per ring row (both heads)
  int64_t rmask;            // ring length - 1
};

KVT_DEV uint32_t ring_row(const RingCtx& C, int64_t p) { return (uint32_t)(p & C.rmask); }

// Direct-to-LDS copies of the ring tile of positions p0 .. p0 + n - 1: exactly 10 vector-memory instructions, like
// the paged tiles.  Copy j of the codes moves 2 whole rows (2 x 512 B; a row of a token beyond n repeats row n - 1);
// scales: each token copies the 16 bytes from the dword that holds its first scale.
KVT_DEV void ring_issue(const RingCtx& C, RingStage& st, int64_t p0, int n) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 2 * j + (lane >> 5);
    const int tt = t < n ? t : n - 1;
    const uint32_t off = ring_row(C, p0 + tt) * 512u + 16u * ring_slot(t, lane & 31);
    copy16_to_lds(C.rk, st.k + 1024 * j, off);
    copy16_to_lds(C.rv, st.v + 1024 * j, off);
  }
  const int tl = (lane & 7) < n ? (lane & 7) : n - 1;
  const uint32_t soff = (ring_row(C, p0 + tl) * C.srowbytes) & ~3u;
  if (lane < 8) {
    copy16_to_lds(C.rks, &st.ks[0][0], soff);
    copy16_to_lds(C.rvs, &st.vs[0][0], soff);
  }
}

// Scale of group g of head h of token t (the token's row of scales starts at half-word sh of its LDS row).
template <int NG8>
KVT_DEV uint32_t ring_scale(const uint16_t (*sc)[8], int t, int h, int g, int sh) {
  return sc[t][sh + NG8 * h + g];
}

template <int G8>
KVT_DEV void ring_compute(const RingCtx& C, const RingStage& st, int64_t p0, int n, const h8 qop[8], float cscale,
                          f4 acc[16], float& m_run, float& l_run) {
  constexpr int NG8 = kD / G8;
  constexpr int STEPS = G8 / 32;
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  const int hr = kb >> 1;                 // head of the lane's D rows (4 kb .. 4 kb + 3)
  const int tr0 = 4 * (kb & 1);           // their first token
  // half-word offset of a token's first scale in its LDS row (odd only for per-token scales at an odd row)
  auto sh_of = [&](int t) -> int { return (int)(((ring_row(C, p0 + t) * C.srowbytes) & 3u) >> 1); };
  // ---- QK^T: A row n16 = (head n16 >> 3, token n16 & 7); lane (col n16, kb) holds rows 4 kb + r
  f4 sc = {0.f, 0.f, 0.f, 0.f};
  {
    const int ta = n16 & 7, ha = n16 >> 3;
    uint2 w[8];
#pragma unroll
    for (int stp = 0; stp < 8; ++stp) {
      const int c = 16 * ha + 2 * stp + (kb >> 1);
      w[stp] = *reinterpret_cast<const uint2*>(st.k + ta * 512 + 16 * ring_slot(ta, c) + 8 * (kb & 1));
    }
    int shr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) shr[r] = NG8 == 1 ? sh_of(tr0 + r) : 0;
#pragma unroll
    for (int g = 0; g < NG8; ++g) {
      f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < STEPS; ++u) {
        const int stp = g * STEPS + u;
        d = mfma(int8_codes_to_h8(w[stp].x, w[stp].y), qop[stp], d);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sg = f16_bits_to_f32((uint16_t)ring_scale<NG8>(st.ks, tr0 + r, hr, g, shr[r]));
        sc[r] = fmaf(sg, d[r], sc[r]);
      }
    }
  }
  const bool own = hr == (n16 >> 3);
  float s[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) s[r] = (own && tr0 + r < n) ? sc[r] * cscale : -INFINITY;
  __builtin_amdgcn_s_setprio(1);
  float mloc = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mloc = max_xor16_32(mloc);
  const float m_new = fmaxf(m_run, mloc);
  if (__any(m_new > m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
    for (int a = 0; a < 16; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[a][i] *= arow[i];
  }
  m_run = m_new;
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
    psum += s[r];
  }
  l_run += psum;
  __builtin_amdgcn_s_setprio(0);
  // ---- P.V on 16x16x16: k = 4 kb + r <-> (head hr, token tr0 + r), the rows of the QK^T output above.  B from
  // ds_read_b64_tr_b8: source lane 2 k8 + p supplies 8 bytes (channels 16 a + 8 p ..) of token tr0 + (k8 & 3) of head
  // hr, block a = a0 (k8 < 4) or a0 + 4; lane j then holds channel 16 a0 + j of the 4 rows in its low dword and channel
  // 16 (a0 + 4) + j in its high dword.
  const h4 pown = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
  h4 pa[NG8];
#pragma unroll
  for (int g = 0; g < NG8; ++g) {
    h4 sg;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      sg[e] = __builtin_bit_cast(_Float16, (uint16_t)ring_scale<NG8>(st.vs, tr0 + e, hr, g,
                                                                     NG8 == 1 ? sh_of(tr0 + e) : 0));
    pa[g] = pown * sg;
  }
  const int k8 = n16 >> 1, pb = n16 & 1;
  const int tv = tr0 + (k8 & 3);
  const uint32_t vrow = lds_off(st.v) + (uint32_t)(tv * 512 + 8 * pb);
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int a0 = (r & 3) + 8 * (r >> 2);
    const int a = k8 < 4 ? a0 : a0 + 4;
    const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (lds_v2i*)(uintptr_t)(vrow + 16u * ring_slot(tv, 16 * hr + a)));
    const uint32_t u0 = (uint32_t)raw.x ^ 0x80808080u, u1 = (uint32_t)raw.y ^ 0x80808080u;
    const h2 l0 = int8_pair_lo(u0), h0 = int8_pair_hi(u0), l1 = int8_pair_lo(u1), h1 = int8_pair_hi(u1);
    acc[a0] = mfma16(pa[(16 * a0) / G8], h4{l0.x, l0.y, h0.x, h0.y}, acc[a0]);
    acc[a0 + 4] = mfma16(pa[(16 * (a0 + 4)) / G8], h4{l1.x, l1.y, h1.x, h1.y}, acc[a0 + 4]);
  }
}

// Q of the ring tiles for lane (n16, kb): channels 32 s + 8 kb .. + 7 of the column's q head, natural order (zero
// for columns beyond the group).
KVT_DEV void load_q_ring(const uint16_t* qrow, bool valid, int kb, h8 qop[8]) {
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * s + 8 * kb);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qop[s][2 * j] = (_Float16)(valid ? __uint_as_float(w[j] << 16) : 0.0f);
      qop[s][2 * j + 1] = (_Float16)(valid ? __uint_as_float(w[j] & 0xffff0000u) : 0.0f);
    }
  }
}

// The block's ring positions [p0, p1) in 8-position tiles handed out from the block counter, double-buffered.
template <int G8>
KVT_DEV void ring_block(const RingCtx& C, WaveArea& W, int32_t* next, bool dyn, int64_t p0, int64_t p1,
                        const uint16_t* qrow, bool qvalid, float cscale, f4 acc[16], float& m_run, float& l_run) {
  const int ntiles = (int)((p1 - p0 + kRingTile - 1) / kRingTile);
  int taken = 0;
  auto grab = [&]() -> int { return take_tile<kWaves>(next, dyn, taken); };
  auto tile_n = [&](int t) -> int { return (int)min((int64_t)kRingTile, p1 - p0 - kRingTile * (int64_t)t); };
  int ta = grab();
  if (ta >= ntiles) return;
  int tb = grab();
  wave_sync();
  ring_issue(C, W.ring[0], p0 + kRingTile * (int64_t)ta, tile_n(ta));
  h8 qop[8];   // while the first tile is in flight
  load_q_ring(qrow, qvalid, (threadIdx.x & 63) >> 4, qop);
  int sa = 0;
  for (;;) {
    const bool more = tb < ntiles;
    int tc = ntiles;
    if (more) {
      ring_issue(C, W.ring[sa ^ 1], p0 + kRingTile * (int64_t)tb, tile_n(tb));
      wait_vmcnt<10>();
      tc = grab();
    } else {
      wait_vmcnt<0>();
    }
    wave_sync();
    ring_compute<G8>(C, W.ring[sa], p0 + kRingTile * (int64_t)ta, tile_n(ta), qop, cscale, acc, m_run, l_run);
    wave_sync();
    if (!more) break;
    ta = tb;
    tb = tc;
    sa ^= 1;
  }
}

// Partials cross XCDs (each has its own L2): written with device-coherent stores (sc1: through to the coherence
// point past the L2), which the combine kernel reads after the kernel boundary.
KVT_DEV void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// A block's ranges: paged positions [w0, ce), ring positions [max(w0, hs), w1).
struct Ranges {
  int64_t hs, w0, w1;
};

KVT_DEV Ranges block_ranges(int64_t L, int64_t R, int64_t rs, int c, int n_b) {
  Ranges g;
  g.hs = hot_start(L, R, rs);
  g.w0 = split_bound<kHotCost4, kTile>(L, g.hs, c, n_b);
  g.w1 = split_bound<kHotCost4, kTile>(L, g.hs, c + 1, n_b);
  return g;
}

KVT_DEV int64_t lane_i64(int v, int i) {
  return (int64_t)(uint32_t)__builtin_amdgcn_readlane(v, i) | ((int64_t)__builtin_amdgcn_readlane(v, i + 1) << 32);
}

template <int G8>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
decode_rows_kernel(const int32_t* plan, const int32_t* seq_lens, const int32_t* ring_len, const int64_t* ring_start,
                   const int64_t* ring_base, const int32_t* page_table, int64_t pt_stride, int n_splits, int flags,
                   const uint16_t* q, int64_t q_stride_b, const int32_t* split_map, int gs, const uint8_t* k4,
                   const uint8_t* v4, const uint16_t* ks4, const uint16_t* vs4, const int8_t* rk, const int8_t* rv,
                   const uint16_t* rks, const uint16_t* rvs, float scale, float* part_o, float* part_ml,
                   uint32_t pool_rows) {
  // (the arguments the start-up chain needs come first: the first 16 dwords are preloaded into SGPRs)
  __shared__ __align__(128) Lds lds;
  const bool dyn = (flags & KVT_DECODE_DYNAMIC) != 0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, kb = lane >> 4;
  const int bid = (int)blockIdx.x;
  // the block's plan entry (one word per lane) and the sequence's placement, loaded at once
  int pv = 0;
  if (plan != nullptr) pv = plan[(int64_t)kPlanWords * bid + lane];
  int b, c, n_b;
  if (split_map != nullptr) {
    b = split_map[3 * bid];
    c = split_map[3 * bid + 1];
    n_b = split_map[3 * bid + 2];
  } else {
    b = bid / n_splits;
    c = bid - b * n_splits;
    n_b = n_splits;
  }
  const int32_t len32 = seq_lens[b], ring32 = ring_len[b];
  const int64_t rs = ring_start[b];
  const int64_t rbase = ring_base[b];
  // the four placement loads in flight together: the compiler would widen each int32 right after its load, one wait
  // before the next load's issue
  asm volatile("" ::"s"(len32), "s"(ring32), "s"(rs), "s"(rbase));
  const int64_t L = len32, R = ring32;
  // the plan holds this block's ranges and first tile rows when it was made for the current placement
  const bool planned = plan != nullptr && __builtin_amdgcn_readlane(pv, 0) == b &&
                       __builtin_amdgcn_readlane(pv, 1) == c && __builtin_amdgcn_readlane(pv, 2) == n_b &&
                       (int64_t)__builtin_amdgcn_readlane(pv, 3) == R && lane_i64(pv, 4) == L &&
                       lane_i64(pv, 6) == rs && lane_i64(pv, 8) == rbase;
  Ranges rg;
  if (planned) {
    rg.hs = lane_i64(pv, 10);
    rg.w0 = lane_i64(pv, 12);
    rg.w1 = lane_i64(pv, 14);
  } else {
    rg = block_ranges(L, R, rs, c, n_b);
  }
  const int64_t w0 = rg.w0, w1 = rg.w1, hs = rg.hs;
  const float cscale = scale * kLog2e;
  const int hc = n16 >> 3, j = n16 & 7;
  const bool qvalid = j < gs;
  const uint16_t* qrow = q + b * q_stride_b + (int64_t)(hc * gs + (qvalid ? j : 0)) * kD;
  if (threadIdx.x == 0) {
    lds.q.cold_next = 2 * kWaves;   // the first round starts with tiles w and w + kWaves of each wavefront
    lds.q.hot_next = 0;
  }

  f4 acc[16];   // acc[a]: channels 16 a + n16 (lane n16 + 16 kb), q head column 4 kb + i in row i
#pragma unroll
  for (int a = 0; a < 16; ++a) acc[a] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // ---- paged positions [w0, min(w1, hs)) from INT4 pages
  const int64_t ce = min(w1, hs);
  const bool has_cold = w0 < ce;
  if (has_cold) {
    RowCtx C{buffer_rsrc(k4, pool_rows * 256u), buffer_rsrc(v4, pool_rows * 256u), buffer_rsrc(ks4, pool_rows * 32u),
             buffer_rsrc(vs4, pool_rows * 32u), {0u, 0u, 0u, 0u}};
    row_lane_offsets(C);
    RowMath M;
    M.cscale = cscale;
    M.nm = nibble_masks();
    const int32_t* pt = page_table + b * pt_stride;
    // First round: the round's page ids (2 direct-to-LDS copies of 64 ids per wavefront; copies past the round read
    // nothing and land in this wavefront's stage 1, which tile wave + kWaves overwrites afterwards), tile wave and the
    // Q loads go out at once; tile wave + kWaves only once they have landed (a first burst of one tile per wavefront
    // lands sooner than one of two).  One barrier publishes the page ids.
    int64_t s0 = w0;
    {
      const int64_t s1 = min(ce, ((s0 >> 6) + kBlockPages) << 6);
      const int64_t pg0 = s0 >> 6;
      const int npg = (int)(((s1 - 1) >> 6) - pg0 + 1);
      const i32x4 rp = buffer_rsrc(pt + pg0, (uint32_t)npg * 4u);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int chunk = wave + kWaves * jj;
        void* dst = chunk * 64 < kBlockPages ? (void*)&lds.q.pages[64 * chunk] : (void*)lds.w[wave].row[1].k;
        copy4_to_lds(rp, dst, (uint32_t)(256 * chunk + 4 * lane));
      }
      RowRound Q{s0, s1, pg0, (int)((s1 - s0 + kTile - 1) / kTile), &lds.q.cold_next, lds.q.pages, dyn, 2};
      Hand hd;
      hd.ta = wave;
      hd.tb = wave + kWaves;
      auto first_row = [&](int t) -> uint32_t {
        if (planned) return (uint32_t)__builtin_amdgcn_readlane(pv, kPlanRows + t);
        const int64_t p = s0 + kTile * (int64_t)t;
        return (uint32_t)pt[p >> 6] * (uint32_t)kPage + (uint32_t)(p & (kPage - 1));
      };
      uint32_t r1 = 0;
      if (hd.ta < Q.ntiles) {
        const uint32_t r0 = first_row(hd.ta);
        row_issue_k(C, lds.w[wave].row[0], r0, Q.n(hd.ta));
        row_issue_v(C, lds.w[wave].row[0], r0, Q.n(hd.ta));
      }
      if (hd.tb < Q.ntiles) r1 = first_row(hd.tb);
      q_build(lds.qa, qrow, qvalid, wave);
      wait_vmcnt<0>();   // the first tile and the page ids have landed
      __syncthreads();
      if (hd.tb < Q.ntiles) {
        row_issue_k(C, lds.w[wave].row[1], r1, Q.n(hd.tb));
        row_issue_v(C, lds.w[wave].row[1], r1, Q.n(hd.tb));
      }
      q_finish(lds.qa, M);
      if (hd.ta < Q.ntiles) {
        hd.tc = hd.tb < Q.ntiles ? Q.grab() : Q.ntiles;
        hd.td = Q.ntiles;
        row_round_run(C, lds.w[wave], Q, hd, M, acc, m_run, l_run);
      }
      s0 = s1;
    }
    while (s0 < ce) {
      const int64_t s1 = min(ce, ((s0 >> 6) + kBlockPages) << 6);
      const int64_t pg0 = s0 >> 6;
      const int npg = (int)(((s1 - 1) >> 6) - pg0 + 1);
      wait_vmcnt<0>();
      __syncthreads();                      // the previous round's tiles and page ids are done with
      if (threadIdx.x == 0) lds.q.cold_next = 0;
      for (int i = threadIdx.x; i < npg; i += 64 * kWaves) lds.q.pages[i] = pt[pg0 + i];
      __syncthreads();
      RowRound Q{s0, s1, pg0, (int)((s1 - s0 + kTile - 1) / kTile), &lds.q.cold_next, lds.q.pages, dyn, 0};
      row_round(C, lds.w[wave], Q, M, acc, m_run, l_run);
      s0 = s1;
    }
  }
  // ---- ring positions [max(w0, hs), w1) from the INT8 ring
  const int64_t hp = max(w0, hs);
  if (hp < w1) {
    if (!has_cold) {   // counters set
      wait_vmcnt<0>();
      __syncthreads();
    }
    constexpr uint32_t NG8 = kD / G8;
    const uint32_t ring_rows = (uint32_t)R;
    RingCtx C{buffer_rsrc(rk + rbase * kH * kD, ring_rows * (uint32_t)(kH * kD)),
              buffer_rsrc(rv + rbase * kH * kD, ring_rows * (uint32_t)(kH * kD)),
              buffer_rsrc(rks + rbase * kH * NG8, ring_rows * kH * NG8 * 2u),
              buffer_rsrc(rvs + rbase * kH * NG8, ring_rows * kH * NG8 * 2u), kH * NG8 * 2u, R - 1};
    ring_block<G8>(C, lds.w[wave], &lds.q.hot_next, dyn, hp, w1, qrow, qvalid, cscale, acc, m_run, l_run);
  }

  // ---- merge the wavefronts.  Each wavefront first leaves its unscaled result in its own area (acc row i of lane
  // (n16, kb) is column 4 kb + i); after one barrier 128 threads compute the weights e^(m_w - M) of every wavefront and
  // column, after a second every thread sums the wavefronts' o of one dim and 8 columns with them.
  l_run = sum_xor16_32(l_run);
  wait_vmcnt<0>();                        // no copy of this wavefront is in flight into its area
  wait_lgkm0();
  wave_sync();
  WaveResult& res = lds.w[wave].res;
#pragma unroll
  for (int a = 0; a < 16; ++a) {
    const int dim = 16 * a + n16;
    *reinterpret_cast<f4*>(&res.o[dim * 16 + 4 * (kb ^ ((dim >> 2) & 3))]) = acc[a];
  }
  if (kb == 0) {
    res.m[n16] = m_run;
    res.l[n16] = l_run;
  }
  __syncthreads();
  const int tid = threadIdx.x;
  float mb = -INFINITY, lb = 0.f;   // natural-log units; thread tid < 16: column tid
  if (tid < kWaves * 16) {
    const int w = tid >> 4, col = tid & 15;
    float M = lds.w[0].res.m[col];
#pragma unroll
    for (int v = 1; v < kWaves; ++v) M = fmaxf(M, lds.w[v].res.m[col]);
    const float mw = lds.w[w].res.m[col];
    lds.wgt[w][col] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
    if (tid < 16) {
#pragma unroll
      for (int v = 0; v < kWaves; ++v) {
        const float mv = lds.w[v].res.m[col];
        lb += mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - M) * lds.w[v].res.l[col];
      }
      mb = M == -INFINITY ? -INFINITY : M / kLog2e;
    }
  }
  __syncthreads();
  // thread (d, half): dim d of columns 8 half .. 8 half + 7 (float4 j = 2 half + jj)
  const int d = tid & (kD - 1), half = tid / kD;
  f4 ob[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    ob[jj] = f4{0.f, 0.f, 0.f, 0.f};
    const int j4 = 2 * half + jj;
    const int off = d * 16 + 4 * (j4 ^ ((d >> 2) & 3));
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const f4 wv = *reinterpret_cast<const f4*>(&lds.wgt[w][4 * j4]);
      ob[jj] += wv * *reinterpret_cast<const f4*>(&lds.w[w].res.o[off]);
    }
  }
  // partial slots: n_splits per (sequence, KV head), gs q heads each (the head-wise kernel's layout)
#pragma unroll
  for (int jj = 0; jj < 2; ++jj)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 8 * half + 4 * jj + i;
      const int ch = col >> 3, cj = col & 7;
      if (cj < gs) {
        const int64_t item = ((int64_t)b * kH + ch) * n_splits + c;
        st_dev(&part_o[(item * gs + cj) * kD + d], ob[jj][i]);
      }
    }
  if (tid < 16 && (tid & 7) < gs) {
    const int64_t item = ((int64_t)b * kH + (tid >> 3)) * n_splits + c;
    st_dev(&part_ml[(item * gs + (tid & 7)) * 2 + 0], mb);
    st_dev(&part_ml[(item * gs + (tid & 7)) * 2 + 1], lb);
  }
}

// One thread per word of the plan: entry i (the block i of the decode grid) holds the block's sequence, split, split
// count, ring length, length, ring start, ring base, first ring position, range [w0, w1) and the pool rows of its first
// kPlanTiles paged tiles (see decode_rows_kernel).  Every thread of an entry computes the entry's ranges (the loads of
// the sequence's placement are shared through the cache); the stores of a wavefront cover one entry, coalesced.
__global__ void __launch_bounds__(256) decode_plan_kernel(int32_t* plan, const int32_t* seq_lens,
                                                          const int32_t* ring_len, const int64_t* ring_start,
                                                          const int64_t* ring_base, const int32_t* page_table,
                                                          int64_t pt_stride, int n_splits, const int32_t* split_map,
                                                          int n_blocks) {
  const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int i = (int)(gi / kPlanWords), k = (int)(gi - (int64_t)i * kPlanWords);
  if (i >= n_blocks) return;
  int b, c, n_b;
  if (split_map != nullptr) {
    b = split_map[3 * i];
    c = split_map[3 * i + 1];
    n_b = split_map[3 * i + 2];
  } else {
    b = i / n_splits;
    c = i - b * n_splits;
    n_b = n_splits;
  }
  const int64_t L = seq_lens[b], R = ring_len[b], rs = ring_start[b], rbase = ring_base[b];
  const Ranges g = block_ranges(L, R, rs, c, n_b);
  int64_t v = 0;
  switch (k >> 1) {   // 64-bit fields: words 4-15
    case 2: v = L; break;
    case 3: v = rs; break;
    case 4: v = rbase; break;
    case 5: v = g.hs; break;
    case 6: v = g.w0; break;
    case 7: v = g.w1; break;
    default: break;
  }
  int32_t word = (k & 1) ? (int32_t)(v >> 32) : (int32_t)(uint32_t)v;
  if (k == 0) word = b;
  if (k == 1) word = c;
  if (k == 2) word = n_b;
  if (k == 3) word = (int32_t)R;
  if (k >= 16) word = 0;
  if (k >= kPlanRows && k < kPlanRows + kPlanTiles) {
    const int64_t p = g.w0 + kTile * (int64_t)(k - kPlanRows);
    const int64_t ce = min(g.w1, g.hs);
    word = p < ce ? (int32_t)((uint32_t)page_table[b * pt_stride + (p >> 6)] * (uint32_t)kPage +
                              (uint32_t)(p & (kPage - 1)))
                  : (int32_t)kNoRow;
  }
  plan[gi] = word;
}

}  // namespace

namespace kvt {
namespace dec {

int rows_launch(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int gs, int group8, const void* k4,
                const void* v4, const void* ks4, const void* vs4, const void* rk, const void* rv, const void* rks,
                const void* rvs, const void* ring_base, const void* ring_len, const void* ring_start,
                const void* page_table, int64_t pt_stride, int64_t pool_rows, float scale, int n_splits,
                const void* split_map, int n_map, void* part_o, void* part_ml, int flags, const void* plan,
                hipStream_t stream) {
  if (pool_rows * kH * (kD / 2) > 0x7fffffffLL) return KVT_ERANGE;
  const int64_t n_blocks = split_map != nullptr ? (int64_t)n_map : (int64_t)batch * n_splits;
  if (n_blocks <= 0 || n_blocks > 0x7fffffff) return KVT_ERANGE;
#define KVT_ROWS_ARGS                                                                                               \
  (const int32_t*)plan, (const int32_t*)seq_lens, (const int32_t*)ring_len, (const int64_t*)ring_start,            \
      (const int64_t*)ring_base, (const int32_t*)page_table, pt_stride, n_splits, flags, (const uint16_t*)q,        \
      q_stride_b, (const int32_t*)split_map, gs, (const uint8_t*)k4, (const uint8_t*)v4, (const uint16_t*)ks4,     \
      (const uint16_t*)vs4, (const int8_t*)rk, (const int8_t*)rv, (const uint16_t*)rks, (const uint16_t*)rvs, scale, \
      (float*)part_o, (float*)part_ml, (uint32_t)pool_rows
  if (group8 == 64) {
    hipLaunchKernelGGL((decode_rows_kernel<64>), dim3((unsigned)n_blocks), dim3(64 * kWaves), 0, stream,
                       KVT_ROWS_ARGS);
  } else {
    hipLaunchKernelGGL((decode_rows_kernel<256>), dim3((unsigned)n_blocks), dim3(64 * kWaves), 0, stream,
                       KVT_ROWS_ARGS);
  }
#undef KVT_ROWS_ARGS
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // namespace dec
}  // namespace kvt

extern "C" {

int kvt_decode_plan(const void* seq_lens, const void* ring_len, const void* ring_start, const void* ring_base,
                    const void* page_table, int64_t pt_stride, int batch, int n_splits, const void* split_map,
                    int n_map, void* plan, void* stream) {
  if (plan == nullptr || batch <= 0 || n_splits <= 0 || (split_map != nullptr && n_map <= 0)) return KVT_EINVAL;
  const int64_t n_blocks = split_map != nullptr ? (int64_t)n_map : (int64_t)batch * n_splits;
  if (n_blocks > 0x7fffffff / kPlanWords) return KVT_ERANGE;
  hipLaunchKernelGGL(decode_plan_kernel, dim3((unsigned)((n_blocks * kPlanWords + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (int32_t*)plan, (const int32_t*)seq_lens, (const int32_t*)ring_len,
                     (const int64_t*)ring_start, (const int64_t*)ring_base, (const int32_t*)page_table, pt_stride,
                     n_splits, (const int32_t*)split_map, (int)n_blocks);
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
