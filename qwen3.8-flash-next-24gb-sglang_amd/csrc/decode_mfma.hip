// Split-K GQA decode attention over the position-indexed tiered cache on gfx950 matrix cores.
//
// Work split: every (sequence, KV head) has n_splits blocks of 8 wavefronts, one block per CU (the block takes all
// of the CU's LDS).  The position range [0, L) is cut into n_splits block ranges of equal cost (a ring position costs
// kHotCost4 / 4 of a paged one; boundaries in the paged part are multiples of 32).  Inside a block, 32-position paged
// tiles and 16-position ring tiles go to the wavefronts one at a time, from a counter in LDS (first come: the
// wavefronts finish together although the oldest get more issue slots) or in a fixed order (bit-reproducible).
// GQA groups of up to 16 q heads per KV head, one per column of the MFMA B operand: groups of up to 8 fill columns
// 0-7 and repeat them in 8-15, and the block copies the group's Q rows to LDS once; wider groups (up to 16) take a
// column each and every wavefront reads its Q rows from memory (the LDS holds no 16 rows beside the tile stages).
//   Paged positions (< hot_start, INT4-G32 pages through the page table): a 32-aligned tile lies in one 64-position
//   page, i.e. 32 consecutive pool rows.  Each wavefront double-buffers its tiles in LDS with direct-to-LDS copies
//   (buffer_load_dwordx4 ... lds, 16 B per lane): the next-but-one tile's K codes and scale rows are issued before a
//   step's math, its V codes after the step's P.V reads.  16-byte chunks are XOR-swizzled at the source address
//   (slot = chunk ^ ckey(token)), so the LDS reads below spread over the banks.
//   Software pipeline: one step is P.V of tile i and QK^T of tile i + 1 in one basic block, so the matrix and VALU
//   work of the two tiles interleave; then the online softmax of tile i + 1.
//   Ring positions (the INT8 ring row, position mod R) take 16-position tiles (K 4 KB + V 4 KB), double-buffered.
//
// QK^T (paged) on v_mfma_f32_16x16x32_f16, one instruction per 16 tokens x 32 channels (= one INT4 scale group):
//   A = raw magic-number values of the codes (0x6400 | nibble = 1024 + n for even channels, 0x6400 | nibble << 4 =
//   1024 + 16 n for odd channels: one v_and_or_b32 per two values), channel order [0,4,1,5,2,6,3,7] of each 8; B = Q
//   in the same order with odd channels divided by 16, one q head per column (narrow groups: 0-7, again in 8-15).  Each
//   product carries a constant excess: (1024 + n) q = (n - 8) q + 1032 q and (1024 + 16 n) q / 16 = (n - 8) q +
//   1152 (q / 16); the per-(group, head) excess bias_g is token independent, so the score of token t is
//   sum_g s_g(t) D_g(t) - sum_g s_g(t) bias_g.  The first sum folds the fp32 group results with the fp16 scales
//   (v_fma_mix); the second is one more MFMA per 16 tokens (A = the token's 8 scales, B = -bias as two fp16 parts
//   scaled by a per-head power of two; the products are exact in fp32).  A rows are ordered so that the D layout
//   leaves each lane the scores of 8 consecutive tokens: the A operand of P.V, no transpose.
// P.V (paged) per scale group g and half: acc[2 g + hf] += A_g * B + A_g * C, A_g = P * s_v(t, g) (fp16; tokens
//   whose codes arrive as 16 n carry P / 16), B = the raw magic values of the V codes, C = -(1032 | 1152) per k.
//   The V scale never multiplies a code and the constant excess is removed per tile (exact fp32 products).  B comes
//   from ds_read_b64_tr_b4, a 16 x 16 nibble transpose per 16 lanes, which turns token-major code rows into the
//   channel-major operand layout in one LDS instruction.
// Ring P.V: v_mfma_f32_16x16x16_f16 with B from ds_read_b64_tr_b8 (exact fp16 codes) and the ring scale folded
//   into P the same way.  Accumulators: acc[a] = 16 channels x 16 head rows (narrow groups: rows 8-15 repeat 0-7).
// The block's wavefronts merge (max, sum, o) in LDS; one fp32 partial per (split, q head) goes to kvt_decode_combine.
//
// Numerics versus the oracle (bf16(code * scale) rows, fp32 softmax): codes enter exactly, K scales in fp32, V scales
// through fp16 P * s (P <= 1, so P * s stays in the fp16 range of the scale itself); fp32 accumulation.  A single
// position returns exactly code * scale.

#include "decode_common.h"
#include "kvtier.h"

#include <mutex>

using namespace kvt;
using namespace kvt::dec;

// Split partials of kvt_decode_mfma_noalloc: a file-scope device array (each GPU the library runs on holds its own
// copy until the process ends).  Host code never uses this name as an address: scratch_base() resolves the device
// address per GPU with hipGetSymbolAddress.
constexpr size_t kScratchBytes = size_t(8) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kWaves = 8;          // wavefronts per block (one block per CU: all of the CU's LDS)
constexpr int kD = 256;
constexpr int kHotCost4 = 7;       // cost of a ring position when blocks split a sequence; a paged position costs 4
                                   // (measured: with 5 the blocks that hold ring positions finish last)
constexpr int kBlockPages = 896;   // page ids of a block's paged range staged in LDS per round (14 x 64)

struct PosArgs {
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
};

// One 32-token tile of one KV head in LDS (cold path).
struct ColdStage {
  uint8_t k[32 * 128];    // K codes, token-major rows; 16-B slot s of token t holds chunk s ^ ckey(t)
  uint8_t v[32 * 128];    // V codes, same layout
  uint16_t ks[32][8];     // K scales [token][group]
  uint16_t vsn[32][8];    // V scales [token][group], as copied
  uint16_t sv[8][32];     // V scales [group][token]
};

// One 16-token tile of ring rows of one KV head in LDS (hot path).
struct HotStage {
  uint8_t k[16 * 256];    // K codes [token][256 channels]; 16-B slot s of token t holds chunk s ^ t
  uint8_t v[16 * 256];    // V codes, same layout
  uint16_t ks[16][8];     // 16 B copied from the dword holding the token's first K scale (see hot_issue)
  uint16_t vs[16][8];     // same for the V scales
};

union WaveArea {
  ColdStage cold[2];
  HotStage hot[2];
};

// floats per wavefront of the merge: [dim][8 or 16 heads], 4 floats of padding per 8 dims
template <bool WIDE>
constexpr int merge_pitch() { return kD * (WIDE ? 16 : 8) + (kD / 8) * 4; }

struct MergeArea {
  float m[kWaves][16];
  float l[kWaves][16];
  float o[kWaves * merge_pitch<true>()];
};

// Block-wide data: the group's q heads (copied once; rows beyond the group read as zero) and the work handed out
// inside the block (the next paged tile of the current round, the next ring tile, the round's page ids).
struct BlockQueue {
  uint16_t q[8][kD];
  int32_t cold_next;
  int32_t hot_next;
  int32_t pages[kBlockPages];   // physical page of the round's page pg0 + i
};

struct Lds {
  union {
    WaveArea w[kWaves];
    MergeArea merge;
  };
  BlockQueue q;
};

// Channels 32 g + 8 kb .. + 7 (g = 0..7) of one q head row as fp32, natural order.  Every load is unconditional (a
// lane whose head is beyond the group reads head 0 of the group and zeroes the values afterwards), so the loads go out
// back to back; 16-byte loads when the rows are 16-byte aligned.
KVT_DEV void load_q_rows(const uint16_t* qrow, bool vec16, int kb, float x[8][8]) {
  if (vec16) {
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * g + 8 * kb);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[g][2 * j] = __uint_as_float(w[j] << 16);
        x[g][2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < 8; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[g][e] = bf16_to_f32(qrow[32 * g + 8 * kb + e]);
  }
}

// Q of the INT8 ring path (q head n % 8 of the group, channel block kb) as 8 MFMA B operands in natural channel
// order; zero for heads beyond the group.
KVT_DEV void load_q_ring(const uint16_t* qrow, bool vec16, bool valid, int kb, h8 qop[8]) {
  float x[8][8];
  load_q_rows(qrow, vec16, kb, x);
#pragma unroll
  for (int g = 0; g < 8; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) qop[g][e] = (_Float16)(valid ? x[g][e] : 0.0f);
}

// Q of the INT4 path in the order [0,4,1,5,2,6,3,7] with odd channels divided by 16, and the B operand of the bias
// MFMA: lanes kb = 0 / 1 hold the leading / remainder fp16 parts of -bias_g * 2^-bexp for g = 0..7, kb >= 2 zero.
KVT_DEV void load_q_int4(const uint16_t* qrow, bool vec16, bool valid, int kb, h8 qop[8], h8& kbias, int& bexp) {
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
  float x[8][8];
  load_q_rows(qrow, vec16, kb, x);
  float bias[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool odd = (e & 2) != 0;   // e = 2, 3, 6, 7 hold channels 1, 5, 3, 7 of the block
      const float xv = valid ? x[g][perm[e]] : 0.0f;
      const _Float16 hq = (_Float16)(odd ? xv * 0.0625f : xv);
      qop[g][e] = hq;
      part = fmaf(odd ? 1152.0f : 1032.0f, (float)hq, part);
    }
    part = sum_xor16_32(part);
    bias[g] = part;
  }
  float amax = 0.0f;
#pragma unroll
  for (int g = 0; g < 8; ++g) amax = fmaxf(amax, fabsf(bias[g]));
  bexp = amax > 0.0f ? ilogbf(amax) - 14 : 0;   // |bias| * 2^-bexp < 2^15
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const float sb = -ldexpf(bias[g], -bexp);
    const _Float16 hi = (_Float16)sb;
    const _Float16 lo = (_Float16)(sb - (float)hi);
    kbias[g] = kb == 0 ? hi : kb == 1 ? lo : (_Float16)0.0f;
  }
}

struct ColdCtx {
  i32x4 rk4, rv4, rks4, rvs4;   // buffer resources of this layer's INT4 pool (codes K/V, scales K/V)
  uint32_t rowbytes;            // H * 128
  uint32_t hoff;                // h * 128
  int H, h;
  uint32_t coff[4];             // this lane's code byte offset in copy j of a full tile, relative to row0 * rowbytes
  uint32_t soff;                // this lane's scale byte offset (lanes < 32), relative to row0 * H * 16
};

// Swizzle of a paged tile in LDS: the 16-byte chunk c (one INT4 scale group) of token t (0..31) sits in slot
// c ^ ckey(t) of the token's 128-byte row.  The QK^T reads (16 tokens 8 a + b, b < 4, one dword of one chunk) then
// hit 8 slots twice each (2-way, the minimum for 128-byte rows), the transposed P.V reads (8 consecutive tokens of
// one chunk, 8 bytes per lane) hit 8 distinct slots (conflict-free).
KVT_DEV int ckey(int t) { return (t ^ ((t >> 3) << 1)) & 7; }

// Per-lane parts of the copy offsets of a full 32-token tile (computed once per wavefront).
KVT_DEV void cold_lane_offsets(ColdCtx& C) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 8 * j + (lane >> 3);
    C.coff[j] = (uint32_t)t * C.rowbytes + C.hoff + 16u * (uint32_t)((lane & 7) ^ ckey(t));
  }
  C.soff = ((uint32_t)(lane & 31) * (uint32_t)C.H + (uint32_t)C.h) * 16u;
}

// row0 = kNoRow: the copies fall outside the buffer (zeros, no memory traffic), so the instruction count stays fixed.
constexpr uint32_t kNoRow = 0xffffffffu;

// Direct-to-LDS copies of one 32-token cold tile (pool rows row0 .. row0 + 31, n valid) into `st`, in two parts:
// cold_issue_k copies the K codes and both scale rows (exactly 6 vector-memory instructions), cold_issue_v the V codes
// (exactly 4).  The vmcnt accounting of the tile loop relies on these counts.  Rows beyond n are copied as they are
// (they lie in the same page: finite codes, masked scores); the scale rows of tokens beyond n repeat row n - 1, so
// every scale that meets a zero probability is finite.
KVT_DEV void cold_issue_k(const ColdCtx& C, ColdStage& st, uint32_t row0, int n) {
  const int lane = threadIdx.x & 63;
  const bool none = row0 == kNoRow;
  const uint32_t cb = none ? 0x80000000u : row0 * C.rowbytes;
#pragma unroll
  for (int j = 0; j < 4; ++j) copy16_to_lds(C.rk4, st.k + 1024 * j, cb + C.coff[j]);
  const uint32_t tl = (uint32_t)min(lane & 31, n - 1);
  const uint32_t soff = none ? 0x80000000u : ((row0 + tl) * (uint32_t)C.H + (uint32_t)C.h) * 16u;
  if (lane < 32) {
    copy16_to_lds(C.rks4, &st.ks[0][0], soff);
    copy16_to_lds(C.rvs4, &st.vsn[0][0], soff);
  }
}

KVT_DEV void cold_issue_v(const ColdCtx& C, ColdStage& st, uint32_t row0) {
  const uint32_t cb = row0 == kNoRow ? 0x80000000u : row0 * C.rowbytes;
#pragma unroll
  for (int j = 0; j < 4; ++j) copy16_to_lds(C.rv4, st.v + 1024 * j, cb + C.coff[j]);
}

// V scales of the tile into the transposed [group][token] layout (lanes 0-31 move one token each).
KVT_DEV void cold_scatter_vs(ColdStage& st) {
  const int lane = threadIdx.x & 63;
  if (lane < 32) {
    const uint4 vs = *reinterpret_cast<const uint4*>(&st.vsn[lane][0]);
    const uint32_t v[4] = {vs.x, vs.y, vs.z, vs.w};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      st.sv[2 * g][lane] = (uint16_t)(v[g] & 0xffffu);
      st.sv[2 * g + 1][lane] = (uint16_t)(v[g] >> 16);
    }
  }
}

// QK^T of one staged tile.  Block nt (0, 1) of 16 A rows: row i is token 8 (i >> 2) + 4 nt + (i & 3), so that the
// D layout leaves lane (n16, kb) with the scores of q head n16 % 8 for tokens 8 kb + 4 nt + r in s[4 nt + r]: the
// lane's 8 scores are tokens 8 kb .. 8 kb + 7 in natural order, the A operand of P.V.  Scores in log2 units.
KVT_DEV void cold_qk(const ColdStage& st, const h8 qop[8], h8 kbias, int bexp, float cscale, NibbleMasks nm,
                     float s[8]) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  const uint32_t mlo = nm.lo, mhi = nm.hi, magic = nm.magic;
  const int t0 = 8 * (n16 >> 2) + (n16 & 3);   // A row n16 of block 0; block 1 reads token t0 + 4 (key ^ 4)
  // chunk g of token t0 at byte t0 * 128 + 16 (g ^ ckey(t0)); dword kb of the chunk
  const uint32_t base = lds_off(st.k) + (uint32_t)(t0 * 128 + 16 * ckey(t0) + 4 * kb);
  uint32_t addr[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) addr[g] = base ^ (16u * (uint32_t)g);
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    uint32_t w[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) w[g] = *(const lds_u32*)(uintptr_t)(addr[g ^ (4 * nt)] + 512u * nt);
    uint4 ksr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ksr[r] = *reinterpret_cast<const uint4*>(&st.ks[8 * kb + 4 * nt + r][0]);
    // bias term -sum_g s_g(t) bias_g (scaled by 2^-bexp in the MFMA, restored here)
    const h8 srow = as_h8(*reinterpret_cast<const u4v*>(&st.ks[t0 + 4 * nt][0]));
    const f4 bsum = mfma(srow, kbias, f4{0.f, 0.f, 0.f, 0.f});
    f4 dp = mfma(int4_codes_raw(w[0], mlo, mhi, magic), qop[0], f4{0.f, 0.f, 0.f, 0.f});
    f4 sc;
#pragma unroll
    for (int r = 0; r < 4; ++r) sc[r] = ldexpf(bsum[r], bexp);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      f4 dn = dp;
      if (g + 1 < 8) dn = mfma(int4_codes_raw(w[g + 1], mlo, mhi, magic), qop[g + 1], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t pairw = g < 2 ? ksr[r].x : g < 4 ? ksr[r].y : g < 6 ? ksr[r].z : ksr[r].w;
        const float sg = f16_bits_to_f32((uint16_t)((g & 1) ? (pairw >> 16) : (pairw & 0xffffu)));
        sc[r] = fmaf(sg, dp[r], sc[r]);
      }
      dp = dn;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) s[4 * nt + r] = sc[r] * cscale;
  }
}

// Scores of tokens >= n (a partial last tile) to -inf.
KVT_DEV void cold_mask(float s[8], int n) {
  const int kb = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = (8 * kb + e) < n ? s[e] : -INFINITY;
}

// Online softmax over a tile's scores.  Rescales acc and l_run when the running max grows; returns P of the lane's 8
// tokens as fp16 with tokens 2, 3, 6, 7 divided by 16 (the A operand layout of cold_pv).
KVT_DEV u4v cold_softmax(const float s[8], f4 acc[16], float& m_run, float& l_run) {
  const int kb = (threadIdx.x & 63) >> 4;
  float mloc = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
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
  float p[8], psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = __builtin_amdgcn_exp2f(s[e] - m_new);
    psum += p[e];
  }
  l_run += psum;
  const h2 sc16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 p01 = {(_Float16)p[0], (_Float16)p[1]}, p23 = h2{(_Float16)p[2], (_Float16)p[3]} * sc16;
  const h2 p45 = {(_Float16)p[4], (_Float16)p[5]}, p67 = h2{(_Float16)p[6], (_Float16)p[7]} * sc16;
  return u4v{as_u32(p01), as_u32(p23), as_u32(p45), as_u32(p67)};
}

// P.V of one staged tile.  Per scale group g (32 channels) and half hf (16 channels 32 g + 16 hf + j):
//   acc[2 g + hf] += A_g * B_{g,hf} + A_g * C,  A_g = P16 * s_v(t, g)  (one head per row),
// where B_{g,hf} holds the raw magic values of the codes (1024 + n for tokens 0, 1, 4, 5 of the k block, 1024 + 16 n
// for tokens 2, 3, 6, 7, whose P16 entries carry the 1/16) and C = -(1032 | 1152) removes the constant excess: the
// products are exact in fp32 and the V scale never multiplies a code.  B comes from ds_read_b64_tr_b4, a 16 x 16
// nibble transpose per 16 lanes: source lane k supplies 8 bytes (16 channels) of token 8 kb + pi(k & 7), half k >> 3,
// and receives channel 32 g + 16 (word) + (k) of the 8 tokens, in the nibble order that int4_codes_raw turns into
// natural token order (pi = 0, 2, 4, 6, 1, 3, 5, 7).
KVT_DEV void cold_pv(const ColdStage& st, u4v p16, NibbleMasks nm, f4 acc[16]) {
  const int lane = threadIdx.x & 63;
  const int k = lane & 15, kb = lane >> 4;
  const uint32_t mlo = nm.lo, mhi = nm.hi, magic = nm.magic;
  const int tv = 8 * kb + 2 * (k & 3) + ((k >> 2) & 1);
  const uint32_t vbase = lds_off(st.v) + (uint32_t)(tv * 128 + 16 * ckey(tv) + 8 * (k >> 3));
  const h8 bc = {(_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1152.0f, (_Float16)-1152.0f,
                 (_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1152.0f, (_Float16)-1152.0f};
  const h8 pa = as_h8(p16);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const v2i raw = __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i*)(uintptr_t)(vbase ^ (16u * (uint32_t)g)));
    const h8 sg = as_h8(*reinterpret_cast<const u4v*>(&st.sv[g][8 * kb]));
    const h8 a = pa * sg;
    acc[2 * g] = mfma(a, int4_codes_raw((uint32_t)raw.x, mlo, mhi, magic), acc[2 * g]);
    acc[2 * g + 1] = mfma(a, int4_codes_raw((uint32_t)raw.y, mlo, mhi, magic), acc[2 * g + 1]);
    acc[2 * g] = mfma(a, bc, acc[2 * g]);
    acc[2 * g + 1] = mfma(a, bc, acc[2 * g + 1]);
  }
}

// One round of a block's paged range: positions [c0, c1) (c0 32-aligned) in 32-position tiles, handed out one at
// a time from the block's counter; the round's page ids sit in LDS.
struct ColdRound {
  int64_t c0, c1, pg0;
  int ntiles;
  int32_t* next;
  const int32_t* pages;
  bool dyn;           // tiles from the shared counter (first come), else wavefront w takes w, w + kWaves, ...
  mutable int taken;  // tiles this wavefront has taken (static order)
  KVT_DEV int grab() const { return take_tile<kWaves>(next, dyn, taken); }
  KVT_DEV uint32_t row0(int t) const {
    const int64_t p = c0 + 32 * (int64_t)t;
    const uint32_t page = (uint32_t)__builtin_amdgcn_readfirstlane(pages[(p >> 6) - pg0]);
    return page * (uint32_t)kPage + (uint32_t)(p & (kPage - 1));
  }
  KVT_DEV int n(int t) const { return (int)min((int64_t)32, c1 - (c0 + 32 * (int64_t)t)); }
};

// Q operands of the paged tiles (filled by the first round, from the block's copy of Q in LDS, while the first
// tiles' copies are in flight) and the constants of the tile math.
struct ColdMath {
  h8 qop[8];
  h8 kbias;
  int bexp;
  float cscale;
  NibbleMasks nm;
  const uint16_t* qrow;   // this lane's q head in LDS
  bool qvalid;
  bool ready;
};

// The tiles a wavefront has in hand: ta (P in p16, V in stage S), tb (stage S ^ 1, copies in flight or landed),
// tc (next to issue), td (taken during the step).
struct ColdHand {
  int ta, tb, tc, td;
};

// One step of the software pipeline: P.V of tile ta (stage S) and QK^T + softmax of tile tb (stage S ^ 1).
// In flight on entry, oldest first: K/scales of tb (6 copies), V of tb (4).  The step issues tc's K/scales into
// stage S (whose K and scale rows ta no longer needs) before the math and tc's V after P.V.
template <int S>
KVT_DEV void cold_step(const ColdCtx& C, WaveArea& W, const ColdRound& Q, ColdHand& hd, const ColdMath& M,
                       f4 acc[16], float& m_run, float& l_run, u4v& p16) {
  const bool more = hd.tc < Q.ntiles;
  const uint32_t rowc = more ? Q.row0(hd.tc) : kNoRow;
  cold_issue_k(C, W.cold[S], rowc, more ? Q.n(hd.tc) : 32);   // (dummies past the end: fixed counts)
  wait_vmcnt<10>();                       // K/scales of tb have landed (and V of ta before them)
  hd.td = more ? Q.grab() : Q.ntiles;
  cold_scatter_vs(W.cold[S ^ 1]);
  wave_sync();
  float s[8];
  cold_pv(W.cold[S], p16, M.nm, acc);     // one basic block: the two tiles' matrix and VALU work interleave
  cold_qk(W.cold[S ^ 1], M.qop, M.kbias, M.bexp, M.cscale, M.nm, s);
  wait_lgkm0();                           // ta's V reads are done before its stage takes new V copies
  cold_issue_v(C, W.cold[S], rowc);       // unconditional: no branch splits the math above
  __builtin_amdgcn_s_setprio(1);   // the softmax chain ahead of the other wavefront's work on the SIMD
  cold_mask(s, Q.n(hd.tb));
  p16 = cold_softmax(s, acc, m_run, l_run);
  __builtin_amdgcn_s_setprio(0);
  hd.ta = hd.tb;
  hd.tb = hd.tc;
  hd.tc = hd.td;
}

// A wavefront's share of one round: tiles taken from the block counter until none is left, through the two-stage
// pipeline.
// The rest of a round once tiles ta (stage 0) and tb (stage 1, if any) are in flight: the pipeline until the block's
// tiles run out.
KVT_DEV void cold_round_run(const ColdCtx& C, WaveArea& W, const ColdRound& Q, ColdHand& hd, ColdMath& M,
                            f4 acc[16], float& m_run, float& l_run) {
  if (!M.ready) {   // Q operands while the first tiles are in flight
    load_q_int4(M.qrow, true, M.qvalid, (threadIdx.x & 63) >> 4, M.qop, M.kbias, M.bexp);
    M.ready = true;
  }
  if (hd.tb < Q.ntiles) wait_vmcnt<14>(); else wait_vmcnt<4>();
  cold_scatter_vs(W.cold[0]);
  wave_sync();
  u4v p16;
  {
    float s[8];
    cold_qk(W.cold[0], M.qop, M.kbias, M.bexp, M.cscale, M.nm, s);
    const int n0 = Q.n(hd.ta);
    if (n0 < 32) cold_mask(s, n0);
    p16 = cold_softmax(s, acc, m_run, l_run);
  }
  int sa = 0;   // stage of ta
  while (hd.tb < Q.ntiles) {
    cold_step<0>(C, W, Q, hd, M, acc, m_run, l_run, p16);
    sa = 1;
    if (hd.tb >= Q.ntiles) break;
    cold_step<1>(C, W, Q, hd, M, acc, m_run, l_run, p16);
    sa = 0;
  }
  // epilogue: P.V of the last tile
  wait_vmcnt<0>();
  wave_sync();
  cold_pv(W.cold[sa], p16, M.nm, acc);
  wait_lgkm0();
  wave_sync();
}

// A wavefront's share of one round: tiles taken from the block counter until none is left.
KVT_DEV void cold_round(const ColdCtx& C, WaveArea& W, const ColdRound& Q, ColdMath& M, f4 acc[16],
                        float& m_run, float& l_run) {
  ColdHand hd;
  hd.ta = Q.grab();
  if (hd.ta >= Q.ntiles) return;
  hd.tb = Q.grab();
  hd.tc = hd.tb < Q.ntiles ? Q.grab() : Q.ntiles;
  hd.td = Q.ntiles;
  wave_sync();
  const uint32_t r0 = Q.row0(hd.ta);
  cold_issue_k(C, W.cold[0], r0, Q.n(hd.ta));
  cold_issue_v(C, W.cold[0], r0);
  if (hd.tb < Q.ntiles) {
    const uint32_t r1 = Q.row0(hd.tb);
    cold_issue_k(C, W.cold[1], r1, Q.n(hd.tb));
    cold_issue_v(C, W.cold[1], r1);
  }
  cold_round_run(C, W, Q, hd, M, acc, m_run, l_run);
}

// The block's paged range [c0, c1) (c0 32-aligned), in rounds of at most kBlockPages pages.  Every wavefront of the
// block calls this (the rounds synchronize the block).
KVT_DEV void cold_block(const PosArgs& A, const ColdCtx& C, Lds& L, int wave, int b, int64_t c0, int64_t c1,
                        bool dyn, ColdMath& M, f4 acc[16], float& m_run, float& l_run) {
  // First round: the round's page ids (2 direct-to-LDS copies of 64 ids per wavefront; copies past the round read
  // nothing and land in this wavefront's stage 1, which tile wave + kWaves overwrites afterwards) and tile wave (page
  // id by a scalar load) go out at once.  Tile wave + kWaves goes out only once they have landed: at start-up every
  // CU asks at once, and a first burst of one tile per wavefront lands sooner than one of two (the second lands
  // while the first is computed).  One barrier publishes the page ids and the block's Q.  The shared counter starts
  // at 2 kWaves.
  {
    const int64_t s1 = min(c1, ((c0 >> 6) + kBlockPages) << 6);
    const int64_t pg0 = c0 >> 6;
    const int npg = (int)(((s1 - 1) >> 6) - pg0 + 1);
    const int lane = threadIdx.x & 63;
    const i32x4 rp = buffer_rsrc(A.page_table + b * A.pt_stride + pg0, (uint32_t)npg * 4u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int chunk = wave + kWaves * j;
      void* dst = chunk * 64 < kBlockPages ? (void*)&L.q.pages[64 * chunk] : (void*)L.w[wave].cold[1].k;
      copy4_to_lds(rp, dst, (uint32_t)(256 * chunk + 4 * lane));
    }
    ColdRound Q{c0, s1, pg0, (int)((s1 - c0 + 31) >> 5), &L.q.cold_next, L.q.pages, dyn, 2};
    ColdHand hd;
    hd.ta = wave;
    hd.tb = wave + kWaves;
    auto page_row = [&](int t) -> uint32_t {
      const int64_t p = c0 + 32 * (int64_t)t;
      return (uint32_t)A.page_table[b * A.pt_stride + (p >> 6)] * (uint32_t)kPage + (uint32_t)(p & (kPage - 1));
    };
    uint32_t r0 = 0, r1 = 0;
    if (hd.ta < Q.ntiles) {
      r0 = page_row(hd.ta);
      cold_issue_k(C, L.w[wave].cold[0], r0, Q.n(hd.ta));
      cold_issue_v(C, L.w[wave].cold[0], r0);
    }
    if (hd.tb < Q.ntiles) r1 = page_row(hd.tb);
    wait_vmcnt<0>();   // the first tile, the Q copy and the page ids have landed
    __syncthreads();
    if (hd.tb < Q.ntiles) {
      cold_issue_k(C, L.w[wave].cold[1], r1, Q.n(hd.tb));
      cold_issue_v(C, L.w[wave].cold[1], r1);
    }
    if (hd.ta < Q.ntiles) {
      hd.tc = hd.tb < Q.ntiles ? Q.grab() : Q.ntiles;
      hd.td = Q.ntiles;
      cold_round_run(C, L.w[wave], Q, hd, M, acc, m_run, l_run);
    }
    c0 = s1;
  }
  for (int64_t s0 = c0; s0 < c1;) {
    const int64_t s1 = min(c1, ((s0 >> 6) + kBlockPages) << 6);
    const int64_t pg0 = s0 >> 6;
    const int npg = (int)(((s1 - 1) >> 6) - pg0 + 1);
    wait_vmcnt<0>();                      // (the first round: this wavefront's part of the Q copy has landed)
    __syncthreads();                      // the previous round's tiles and page ids are done with
    if (threadIdx.x == 0) L.q.cold_next = 0;
    for (int i = threadIdx.x; i < npg; i += 64 * kWaves) L.q.pages[i] = A.page_table[b * A.pt_stride + pg0 + i];
    __syncthreads();
    ColdRound Q{s0, s1, pg0, (int)((s1 - s0 + 31) >> 5), &L.q.cold_next, L.q.pages, dyn, 0};
    cold_round(C, L.w[wave], Q, M, acc, m_run, l_run);
    s0 = s1;
  }
}

// ---- ring (hot) tiles: 16 positions, INT8 codes, scale groups of G8 channels

struct HotCtx {
  i32x4 rk, rv, rks, rvs;   // buffer resources over this sequence's ring rows (codes K/V, scales K/V)
  uint32_t rowbytes;        // H * 256
  uint32_t hoff;            // h * 256
  uint32_t srowbytes;       // H * (256 / G8) * 2
  uint32_t shoff;           // h * (256 / G8) * 2
  int64_t rmask;            // ring length - 1
};

KVT_DEV uint32_t hot_row(const HotCtx& C, int64_t p) { return (uint32_t)(p & C.rmask); }

// Issue the direct-to-LDS copies of the ring tile of positions p0 .. p0 + n - 1 into `st`: exactly 10 vector-memory
// instructions per wavefront, like cold_issue.  Scales: each token copies the 16 bytes from the dword that holds its
// first scale (byte offset srow & ~3); the scale of group g then sits at byte (srow & 3) + 2 g of its LDS row.
KVT_DEV void hot_issue(const HotCtx& C, HotStage& st, int64_t p0, int n) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 4 * j + (lane >> 4);
    const int tt = t < n ? t : n - 1;
    const uint32_t chunk = (uint32_t)((lane & 15) ^ t);
    const uint32_t off = hot_row(C, p0 + tt) * C.rowbytes + C.hoff + 16u * chunk;
    copy16_to_lds(C.rk, st.k + 1024 * j, off);
    copy16_to_lds(C.rv, st.v + 1024 * j, off);
  }
  const int tl = (lane & 15) < n ? (lane & 15) : n - 1;
  const uint32_t soff = (hot_row(C, p0 + tl) * C.srowbytes + C.shoff) & ~3u;
  if (lane < 16) {
    copy16_to_lds(C.rks, &st.ks[0][0], soff);
    copy16_to_lds(C.rvs, &st.vs[0][0], soff);
  }
}

// fp16 bits of the scale of group g of token t (sh = half-word offset of the token's first scale, 0 or 1).
KVT_DEV uint32_t hot_scale(const uint16_t (*sc)[8], int t, int g, int sh) { return sc[t][sh + g]; }

template <int G8>
KVT_DEV void hot_compute(const HotCtx& C, const HotStage& st, int64_t p0, int n, const h8 qop[8], float cscale,
                         f4 acc[16], float& m_run, float& l_run) {
  constexpr int NG8 = kD / G8;
  constexpr int STEPS = G8 / 32;
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  // half-word offset of a token's first scale in its LDS row (only odd for one scale per row and odd row * H + h)
  auto sh_of = [&](int t) -> int {
    return (int)(((hot_row(C, p0 + t) * C.srowbytes + C.shoff) & 3u) >> 1);
  };
  // ---- QK^T: lane holds scores of q head n16 % 8 for tokens 4 kb + r
  f4 sc = {0.f, 0.f, 0.f, 0.f};
  {
    const int t = n16;
    uint2 w[8];
#pragma unroll
    for (int stp = 0; stp < 8; ++stp) {
      const int chunk = 2 * stp + (kb >> 1);
      w[stp] = *reinterpret_cast<const uint2*>(st.k + t * 256 + 16 * (chunk ^ t) + 8 * (kb & 1));
    }
    int shr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) shr[r] = NG8 == 1 ? sh_of(4 * kb + r) : 0;
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
        const float sg = f16_bits_to_f32((uint16_t)hot_scale(st.ks, 4 * kb + r, g, shr[r]));
        sc[r] = fmaf(sg, d[r], sc[r]);
      }
    }
  }
  float s[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) s[r] = (4 * kb + r) < n ? sc[r] * cscale : -INFINITY;
  __builtin_amdgcn_s_setprio(1);   // (as on the paged tiles)
  // ---- online softmax over the tile
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
  float psum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    s[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
    psum += s[r];
  }
  l_run += psum;
  __builtin_amdgcn_s_setprio(0);
  // ---- P.V on 16x16x16 (k = tokens 4 kb .. + 3 of the lane's block), same accumulator layout as the paged tiles:
  // acc[a] += (P * s_v(t, g(a))) * V(t, 16 a + j).  B from ds_read_b64_tr_b8: source lane 2 k8 + p supplies 8 bytes
  // (channels 16 a + 8 p ..) of token 4 kb + (k8 & 3), block a = a0 (k8 < 4) or a0 + 4; lane j then holds channel
  // 16 a0 + j of the 4 tokens in its low dword and channel 16 (a0 + 4) + j in its high dword (8 distinct slots per
  // 16 lanes: conflict-free).  Codes convert exactly (b + 128 as the low byte of 1024 + u, minus 1152).
  const h4 pown = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
  h4 pa[NG8];
#pragma unroll
  for (int g = 0; g < NG8; ++g) {
    h4 sg;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 4 * kb + e;
      sg[e] = __builtin_bit_cast(_Float16, (uint16_t)hot_scale(st.vs, t, g, NG8 == 1 ? sh_of(t) : 0));
    }
    pa[g] = pown * sg;
  }
  const int k8 = n16 >> 1, pb = n16 & 1;
  const int tv = 4 * kb + (k8 & 3);
  const uint32_t vrow = lds_off(st.v) + (uint32_t)(tv * 256 + 8 * pb);
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int a0 = (r & 3) + 8 * (r >> 2);
    const int a = k8 < 4 ? a0 : a0 + 4;
    const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(uintptr_t)(vrow + 16u * (uint32_t)(a ^ tv)));
    const uint32_t u0 = (uint32_t)raw.x ^ 0x80808080u, u1 = (uint32_t)raw.y ^ 0x80808080u;
    const h2 l0 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) + off;
    const h2 h0 = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) + off;
    const h2 l1 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) + off;
    const h2 h1 = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) + off;
    acc[a0] = mfma16(pa[(16 * a0) / G8], h4{l0.x, l0.y, h0.x, h0.y}, acc[a0]);
    acc[a0 + 4] = mfma16(pa[(16 * (a0 + 4)) / G8], h4{l1.x, l1.y, h1.x, h1.y}, acc[a0 + 4]);
  }
}

// The block's ring positions [p0, p1) in 16-position tiles handed out from the block counter, double-buffered: the
// next tile's copies are issued before the current tile's math.
template <int G8>
KVT_DEV void hot_block(const HotCtx& C, WaveArea& W, int32_t* next, bool dyn, int64_t p0, int64_t p1,
                       const uint16_t* qrow, bool qvalid, float cscale, f4 acc[16], float& m_run, float& l_run) {
  const int ntiles = (int)((p1 - p0 + 15) >> 4);
  int taken = 0;
  auto grab = [&]() -> int { return take_tile<kWaves>(next, dyn, taken); };
  auto tile_n = [&](int t) -> int { return (int)min((int64_t)16, p1 - p0 - 16 * (int64_t)t); };
  int ta = grab();
  if (ta >= ntiles) return;
  int tb = grab();
  wave_sync();
  hot_issue(C, W.hot[0], p0 + 16 * (int64_t)ta, tile_n(ta));
  h8 qop[8];   // while the first tile is in flight
  load_q_ring(qrow, true, qvalid, (threadIdx.x & 63) >> 4, qop);
  int sa = 0;
  for (;;) {
    const bool more = tb < ntiles;
    int tc = ntiles;
    if (more) {
      hot_issue(C, W.hot[sa ^ 1], p0 + 16 * (int64_t)tb, tile_n(tb));
      wait_vmcnt<10>();
      tc = grab();
    } else {
      wait_vmcnt<0>();
    }
    wave_sync();
    hot_compute<G8>(C, W.hot[sa], p0 + 16 * (int64_t)ta, tile_n(ta), qop, cscale, acc, m_run, l_run);
    wave_sync();
    if (!more) break;
    ta = tb;
    tb = tc;
    sa ^= 1;
  }
}

// Partials cross XCDs (each has its own L2): they are written with device-coherent stores (sc1: written through to
// the coherence point past the L2), which the combine kernel reads after the kernel boundary.
KVT_DEV void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

template <int G8, bool WIDE>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
decode_mfma_kernel(const int32_t* seq_lens, const int32_t* ring_len, const int64_t* ring_start,
                   const int32_t* page_table, int64_t pt_stride, const int32_t* split_map, int H, int n_splits,
                   int gs, int flags, const uint16_t* q, int64_t q_stride_b, const int64_t* ring_base,
                   const uint8_t* k4, const uint8_t* v4, const uint16_t* ks4, const uint16_t* vs4, const int8_t* rk,
                   const int8_t* rv, const uint16_t* rks, const uint16_t* rvs, float scale, float* part_o,
                   float* part_ml, uint32_t pool_rows, int n_map) {
  // (the arguments the start-up chain needs come first: the first 16 dwords are preloaded into SGPRs)
  const PosArgs A{k4, v4, ks4, vs4, rk, rv, rks, rvs, ring_base, ring_len, ring_start, page_table, pt_stride};
  __shared__ __align__(128) Lds lds;
  // 1-D grid: block i = (row i / gx, split i % gx)
  const int gx = split_map != nullptr ? n_map : n_splits;
  const int bid = (int)blockIdx.x;
  const bool dyn = (flags & KVT_DECODE_DYNAMIC) != 0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n16 = lane & 15, kb = lane >> 4;
  // split c of n_b for sequence b: uniform (grid.x = n_splits, grid.y = batch x H) or from the split map
  // (grid.x = total splits, grid.y = H; entry = {b, c, n_b})
  int b, c, h, n_b;
  const int bx = bid % gx, by = bid / gx;
  if (split_map != nullptr) {
    b = split_map[3 * bx];
    c = split_map[3 * bx + 1];
    n_b = split_map[3 * bx + 2];
    h = by;
  } else {
    c = bx;
    b = by / H;
    h = by - b * H;
    n_b = n_splits;
  }
  const int64_t item = ((int64_t)b * H + h) * n_splits + c;   // partial slots: n_splits per (sequence, head)
  const int64_t L = seq_lens[b];
  const int64_t R = A.ring_len[b];
  const int64_t rbase = A.ring_base[b];
  const int64_t hs = min(max(max(A.ring_start[b], L - R), (int64_t)0), L);   // first ring position
  // this block's positions [w0, w1): equal shares of the cost 4 hs + kHotCost4 (L - hs) (paged boundaries 32-aligned)
  const int64_t cost = 4 * hs + kHotCost4 * (L - hs);
  auto bound = [&](int64_t w) -> int64_t {
    if (w >= n_b) return L;
    const int64_t x = cost * w / n_b;
    if (x <= 4 * hs) return (x >> 2) & ~(int64_t)31;
    return hs + (x - 4 * hs + kHotCost4 - 1) / kHotCost4;
  };
  const int64_t w0 = bound(c);
  const int64_t w1 = bound(c + 1);
  const float cscale = scale * kLog2e;
  const int hq = WIDE ? n16 : n16 & 7;   // the lane's q head (column n16 of the B operand)
  const bool qvalid = hq < gs;
  const uint16_t* qrow;                   // its Q row (a valid row of the group when the head is beyond it)
  if constexpr (WIDE) {
    qrow = q + b * q_stride_b + (int64_t)(h * gs + (qvalid ? hq : 0)) * kD;
  } else {
    // the group's q heads into LDS (waves 0-3, 1 KB each; heads beyond the group read as zero)
    if (wave < 4) {
      const i32x4 rq = buffer_rsrc(q + b * q_stride_b + (int64_t)h * gs * kD, (uint32_t)gs * kD * 2u);
      copy16_to_lds(rq, &lds.q.q[2 * wave][0], (uint32_t)(1024 * wave + 16 * lane));
    }
    qrow = &lds.q.q[hq][0];
  }
  if (threadIdx.x == 0) {
    lds.q.cold_next = 2 * kWaves;   // the first round starts with tiles w and w + kWaves of each wavefront
    lds.q.hot_next = 0;
  }

  f4 acc[16];   // acc[a]: channels 16 a + j (lane j + 16 kb), q head 4 kb + i in row 4 kb + i (narrow groups:
                // head (4 kb + i) % 8, rows of kb 2, 3 repeat kb 0, 1)
#pragma unroll
  for (int a = 0; a < 16; ++a) acc[a] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  // paged positions [w0, min(w1, hs)) from INT4 pages
  const int64_t ce = min(w1, hs);
  const bool has_cold = w0 < ce;
  if (has_cold) {   // (cold_block's first barrier publishes the counters and Q)
    ColdCtx C{buffer_rsrc(A.k4, pool_rows * (uint32_t)H * 128u), buffer_rsrc(A.v4, pool_rows * (uint32_t)H * 128u),
              buffer_rsrc(A.ks4, pool_rows * (uint32_t)H * 16u), buffer_rsrc(A.vs4, pool_rows * (uint32_t)H * 16u),
              (uint32_t)H * 128u, (uint32_t)h * 128u, H, h, {0u, 0u, 0u, 0u}, 0u};
    cold_lane_offsets(C);
    ColdMath M;
    M.cscale = cscale;
    M.nm = nibble_masks();
    M.qrow = qrow;
    M.qvalid = qvalid;
    M.ready = false;
    cold_block(A, C, lds, wave, b, w0, ce, dyn, M, acc, m_run, l_run);
  }
  // ring positions [max(w0, hs), w1) from the INT8 ring
  const int64_t hp = max(w0, hs);
  if (hp < w1) {
    if (!has_cold) {   // Q copied and counters set
      wait_vmcnt<0>();
      __syncthreads();
    }
    constexpr uint32_t NG8 = kD / G8;
    const uint32_t ring_rows = (uint32_t)R;
    HotCtx C{buffer_rsrc(A.rk + rbase * H * kD, ring_rows * (uint32_t)H * kD),
             buffer_rsrc(A.rv + rbase * H * kD, ring_rows * (uint32_t)H * kD),
             buffer_rsrc(A.rks + rbase * H * NG8, ring_rows * (uint32_t)H * NG8 * 2u),
             buffer_rsrc(A.rvs + rbase * H * NG8, ring_rows * (uint32_t)H * NG8 * 2u),
             (uint32_t)H * kD, (uint32_t)h * kD, (uint32_t)H * NG8 * 2u, (uint32_t)h * NG8 * 2u, R - 1};
    hot_block<G8>(C, lds.w[wave], &lds.q.hot_next, dyn, hp, w1, qrow, qvalid, cscale, acc, m_run, l_run);
  }

  // ---- merge the wavefronts (narrow groups: heads 0-7, lanes n16 >= 8 duplicate n16 - 8)
  constexpr int kPitch = merge_pitch<WIDE>();
  constexpr int kRows = WIDE ? 16 : 8;    // distinct accumulator rows
  l_run = sum_xor16_32(l_run);
  wait_vmcnt<0>();                        // (a block without positions still has its Q copy in flight)
  __syncthreads();                        // every wavefront is done with its staging area
  const int tid = threadIdx.x;
  if (kb == 0 && n16 < kRows) {
    lds.merge.m[wave][n16] = m_run;
    lds.merge.l[wave][n16] = l_run;
  }
  __syncthreads();
  // accumulator row 4 kb + i holds q head 4 kb + i (narrow: (4 kb + i) % 8, lanes kb < 2 write heads 0-7)
  const bool writer = WIDE || kb < 2;
  const int hrow = WIDE ? 4 * kb : 4 * (kb & 1);
  f4 wrow;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hr = hrow + i;
    float M = lds.merge.m[0][hr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.merge.m[w][hr]);
    const float mw = lds.merge.m[wave][hr];
    wrow[i] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
  }
  float* ow = lds.merge.o + wave * kPitch;
  if (writer) {
#pragma unroll
    for (int a = 0; a < 16; ++a) {
      const int dim = 16 * a + n16;
      *reinterpret_cast<f4*>(&ow[dim * kRows + (dim >> 3) * 4 + hrow]) = acc[a] * wrow;
    }
  }
  __syncthreads();
  // the block's partial: thread (d, half) holds o of dim d for q heads kRows / 2 * half + 4 j + i; threads < gs
  // (m, l) of a head
  constexpr int kF4 = kRows / 8;          // float4s per thread
  const int d = tid & (kD - 1), half = tid / kD;
  f4 ob[kF4];
#pragma unroll
  for (int j = 0; j < kF4; ++j) {
    ob[j] = f4{0.f, 0.f, 0.f, 0.f};
    const int base = d * kRows + (d >> 3) * 4 + (kRows / 2) * half + 4 * j;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) ob[j] += *reinterpret_cast<const f4*>(&lds.merge.o[w * kPitch + base]);
  }
  float mb = -INFINITY, lb = 0.f;   // natural-log units
  if (tid < gs) {
    float M = lds.merge.m[0][tid];
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.merge.m[w][tid]);
    for (int w = 0; w < kWaves; ++w) {
      const float mw = lds.merge.m[w][tid];
      lb += mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M) * lds.merge.l[w][tid];
    }
    mb = M == -INFINITY ? -INFINITY : M / kLog2e;
  }
  // the partial, in the slot of this split (read by the combine kernel or by the mergers below)
#pragma unroll
  for (int j = 0; j < kF4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hd = (kRows / 2) * half + 4 * j + i;
      if (hd < gs) st_dev(&part_o[(item * gs + hd) * kD + d], ob[j][i]);
    }
  if (tid < gs) {
    st_dev(&part_ml[(item * gs + tid) * 2 + 0], mb);
    st_dev(&part_ml[(item * gs + tid) * 2 + 1], lb);
  }
}

}  // namespace

extern "C" {

int kvt_decode_mfma(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                    int group8, const void* k4, const void* v4, const void* ks4, const void* vs4, const void* rk,
                    const void* rv, const void* rks, const void* rvs, const void* ring_base, const void* ring_len,
                    const void* ring_start, const void* page_table, int64_t pt_stride, int64_t pool_rows,
                    float scale, int n_splits, const void* split_map, int n_map, void* part_o, void* part_ml,
                    int flags, const void* plan, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || D != kD) return KVT_EINVAL;
  if ((((uintptr_t)q) | (uintptr_t)(q_stride_b * 2)) & 15) return KVT_EINVAL;   // Q rows are copied in 16-byte pieces
  if (pool_rows <= 0 || pool_rows * H * (kD / 2) > 0x7fffffffLL) return KVT_ERANGE;   // 32-bit byte offsets
  const int gs = Hq / H;
  if (gs > 16 || n_splits <= 0 || (split_map != nullptr && n_map <= 0)) return KVT_EINVAL;
  if (group8 != 64 && group8 != 256) return KVT_EINVAL;
  hipStream_t st = (hipStream_t)stream;
  // both KV heads per wavefront (full pool rows) where the shape allows it
  if (H == 2 && gs <= 8 && (flags & KVT_DECODE_HEADWISE) == 0)
    return rows_launch(q, q_stride_b, seq_lens, batch, gs, group8, k4, v4, ks4, vs4, rk, rv, rks, rvs, ring_base,
                       ring_len, ring_start, page_table, pt_stride, pool_rows, scale, n_splits, split_map, n_map,
                       part_o, part_ml, flags, plan, st);
  // grid: one block per (split, sequence x KV head) or per (split map entry, KV head)
  const unsigned gx = split_map != nullptr ? (unsigned)n_map : (unsigned)n_splits;
  const int work_rows = split_map != nullptr ? H : batch * H;
  const int64_t n_blocks = (int64_t)work_rows * gx;
  if (n_blocks > 0x7fffffff) return KVT_ERANGE;
#define KVT_DECODE_ARGS                                                                                          \
  (const int32_t*)seq_lens, (const int32_t*)ring_len, (const int64_t*)ring_start, (const int32_t*)page_table,       \
      pt_stride, (const int32_t*)split_map, H, n_splits, gs, flags, (const uint16_t*)q, q_stride_b,                \
      (const int64_t*)ring_base, (const uint8_t*)k4, (const uint8_t*)v4, (const uint16_t*)ks4, (const uint16_t*)vs4, \
      (const int8_t*)rk, (const int8_t*)rv, (const uint16_t*)rks, (const uint16_t*)rvs, scale, (float*)part_o,     \
      (float*)part_ml, (uint32_t)pool_rows, n_map
  const dim3 grid((unsigned)n_blocks);
  const bool wide = gs > 8;
  if (group8 == 64 && !wide) {
    hipLaunchKernelGGL((decode_mfma_kernel<64, false>), grid, dim3(64 * kWaves), 0, st, KVT_DECODE_ARGS);
  } else if (group8 == 64) {
    hipLaunchKernelGGL((decode_mfma_kernel<64, true>), grid, dim3(64 * kWaves), 0, st, KVT_DECODE_ARGS);
  } else if (!wide) {
    hipLaunchKernelGGL((decode_mfma_kernel<256, false>), grid, dim3(64 * kWaves), 0, st, KVT_DECODE_ARGS);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<256, true>), grid, dim3(64 * kWaves), 0, st, KVT_DECODE_ARGS);
  }
#undef KVT_DECODE_ARGS
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

// Device address of `scratch` on the current device: resolved once per device (hipGetSymbolAddress with that device
// current), then kept.  Returns KVT_OK or KVT_EHIP.
static int scratch_base(float** base) {
  static std::mutex mu;
  static float* addr[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return KVT_EHIP;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return KVT_EHIP;
    addr[dev] = static_cast<float*>(p);
  }
  *base = addr[dev];
  return KVT_OK;
}

int kvt_decode_mfma_noalloc(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                            int group8, const void* k4, const void* v4, const void* ks4, const void* vs4,
                            const void* rk, const void* rv, const void* rks, const void* rvs, const void* ring_base,
                            const void* ring_len, const void* ring_start, const void* page_table, int64_t pt_stride,
                            int64_t pool_rows, float scale, int n_splits, const void* split_map, int n_map,
                            const void* split_counts, int flags, void* out_f32, void* out_bf16, int64_t out_stride_b,
                            void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || D != kD || n_splits <= 0) return KVT_EINVAL;
  if (out_f32 == nullptr && out_bf16 == nullptr) return KVT_EINVAL;
  if ((split_map == nullptr) != (split_counts == nullptr)) return KVT_EINVAL;
  // partials: o fp32 [batch H n_splits][Hq / H][D], then (m, l) [..][Hq / H][2] at a 256-byte boundary
  const int64_t rows = (int64_t)batch * H * n_splits * (Hq / H);
  const int64_t o_floats = (rows * kD + 63) & ~(int64_t)63;
  if ((o_floats + rows * 2) * (int64_t)sizeof(float) > (int64_t)kScratchBytes) return KVT_ERANGE;
  float* base = nullptr;
  const int st = scratch_base(&base);
  if (st != KVT_OK) return st;
  const int s1 = kvt_decode_mfma(q, q_stride_b, seq_lens, batch, H, Hq, D, group8, k4, v4, ks4, vs4, rk, rv, rks, rvs,
                                 ring_base, ring_len, ring_start, page_table, pt_stride, pool_rows, scale, n_splits,
                                 split_map, n_map, base, base + o_floats, flags, nullptr, stream);
  if (s1 != KVT_OK) return s1;
  return kvt_decode_combine(base, base + o_floats, batch, H, Hq, D, n_splits, 0, seq_lens, split_counts, out_f32,
                            out_bf16, out_stride_b, stream);
}

}  // extern "C"
