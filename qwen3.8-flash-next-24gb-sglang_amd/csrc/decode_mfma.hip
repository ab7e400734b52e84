// Split-K GQA decode attention over the position-indexed tiered cache on gfx950 matrix cores.
//
// Work item = (sequence, KV head, split of `chunk` positions); 4 wavefronts per block, each owning a quarter of the
// split.  GQA groups of up to 8 q heads per KV head.
//   Cold positions (< hot_start, INT4-G32 pages through the page table) stream in 32-token tiles: a 32-aligned tile
//   lies in one 64-token page, i.e. 32 consecutive pool rows.  Each wavefront double-buffers its tiles in LDS with
//   direct-to-LDS copies (buffer_load_dwordx4 ... lds, 16 B per lane) issued one tile ahead, so HBM traffic of tile
//   i+1 overlaps the matrix work of tile i.  16-byte chunks are XOR-swizzled with the token index at the source
//   address, which keeps the per-lane LDS reads bank-conflict free.
//   Hot positions (the INT8 ring row, position mod R) are walked in sub-chunks of 128 with direct global loads.
//
// QK^T on v_mfma_f32_16x16x32_f16, one instruction per 16 tokens x 32 channels (= one INT4 scale group):
//   A = K codes as exact fp16 integers (row = token), B = Q (32 channels x 16 columns: the group's q heads in
//   columns 0-7 and again in 8-15).  Codes come from the magic-number conversion (0x6400 | nibble) = 1024 + nibble,
//   minus 1032 (high nibble: (1024 + 16 n) / 16 - 72), channels in the order [0,4,1,5,2,6,3,7] of each 8 with Q
//   loaded in the same order.  The per-(token, group) fp16 scale is folded into the fp32 group result:
//   score += s_g(t) * D_g.
// Softmax: scores stay in the D layout (lane = q head, 4 tokens of each 16-token tile), which is the A operand
//   layout of P.V, so P needs no transpose.  exp2 with log2(e) folded into the score scale; the running max is
//   rescaled only when it grows (wave-uniform test).
// P.V, block-diagonal: a 16 x 16 accumulator tile holds 8 heads x 16 dims in rows 0-7 and the same 8 heads x 16
//   other dims in rows 8-15.  Because columns 8-15 of Q duplicate 0-7, lane (row m >= 8) holds P of head m - 8;
//   A_X = (m < 8 ? own P : 0) with B = V(own tokens, dims A) and A_Y = (m >= 8 ? P of lane ^ 32 : 0) with
//   B = V(tokens of lane ^ 32, dims B) accumulate into the same tile: 32 accumulator registers for 256 dims.
//   V is dequantized to fp16 (exact code conversion, then one packed multiply by the per-(token, group) scale pair).
// The four wavefronts merge (max, sum, o) in LDS; one fp32 partial per work item goes to kvt_decode_combine.
//
// Numerics versus the oracle (bf16(code * scale) rows, fp32 softmax): K enters exactly (integer codes, fp32 scale
// fold); V as fp16(code * scale) (finer than the oracle's bf16 rounding); P as fp16; fp32 accumulation.  V entries
// beyond the fp16 range (|v| > 65504) are not representable on this path (the reference-precision kernel handles
// them).

#include "kvt_common.h"

using namespace kvt;

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kSub = 128;      // positions per wave sub-chunk (8 QK tiles of 16, 4 PV tiles of 32)
constexpr int kD = 256;
constexpr float kLog2e = 1.4426950408889634f;

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

KVT_DEV f4 mfma(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

KVT_DEV h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
KVT_DEV uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }
KVT_DEV h8 as_h8(u4v u) { return __builtin_bit_cast(h8, u); }
KVT_DEV u4v as_u4(h8 h) { return __builtin_bit_cast(u4v, h); }

// (a & m) | o in one VOP3 instruction (the compiler otherwise splits it in two around the literal constants).
KVT_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
  return r;
}

// 8 INT4 codes (one dword, channels c0..c7 = nibbles 0..7) -> fp16 (c - 8) in the order [c0,c4,c1,c5,c2,c6,c3,c7].
KVT_DEV h8 int4_codes_to_h8(uint32_t w, uint32_t mlo, uint32_t mhi, uint32_t magic) {
  const uint32_t w8 = w >> 8;
  const h2 lo0 = as_h2(and_or(w, mlo, magic));    // 1024 + (c0, c4)
  const h2 hi0 = as_h2(and_or(w, mhi, magic));    // 1024 + 16 (c1, c5)
  const h2 lo1 = as_h2(and_or(w8, mlo, magic));   // 1024 + (c2, c6)
  const h2 hi1 = as_h2(and_or(w8, mhi, magic));   // 1024 + 16 (c3, c7)
  const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 sc = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 off2 = {(_Float16)-72.0f, (_Float16)-72.0f};
  const h2 a = lo0 + off, b = hi0 * sc + off2, c = lo1 + off, d = hi1 * sc + off2;
  return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// 8 INT8 codes (two dwords, natural channel order) -> fp16 exact.
KVT_DEV h8 int8_codes_to_h8(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;   // b + 128 as unsigned bytes
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const h2 a = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) + off;
  const h2 b = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) + off;
  const h2 c = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) + off;
  const h2 d = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) + off;
  return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

struct WaveLds {
  int32_t rows[kSub];
  uint16_t sk[kSub][8];   // K scales, [token][group]
  uint16_t sv[8][kSub];   // V scales, [group][token]
};

// One 32-token tile of one KV head in LDS (cold path).
struct ColdStage {
  uint8_t k[32 * 128];    // K codes, token-major rows; 16-B slot s of token t holds chunk s ^ (t & 7)
  uint8_t v[32 * 128];    // V codes, same layout
  uint16_t ks[32][8];     // K scales [token][group]
  uint16_t vsn[32][8];    // V scales [token][group], as copied
  uint16_t sv[8][32];     // V scales [group][token]
};

union WaveArea {
  WaveLds hot;
  ColdStage cold[2];
};

struct MergeArea {
  float m[kWaves][8];
  float l[kWaves][8];
  float o[8][kD];
};

union Lds {
  WaveArea w[kWaves];
  MergeArea merge;
};

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [p, p + bytes): loads beyond the range return zero instead of faulting.
KVT_DEV i32x4 buffer_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = (uint64_t)p;
  i32x4 r;
  r.x = (int)(uint32_t)a;
  r.y = (int)(uint32_t)(a >> 32);
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}

// 16 bytes per lane from rsrc + voffset into lds + 16 * lane (M0 = LDS base).  Written as inline assembly so that
// the compiler does not treat every later LDS read as dependent on it: completion is tracked explicitly with
// wait_vmcnt by the caller.
KVT_DEV void copy16_to_lds(i32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(base), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// s_waitcnt vmcnt(<= n) leaving the other counters alone (gfx9 encoding).
template <int N>
KVT_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// Q (q head n % 8 of the group, channel block kb) as 8 MFMA B operands, one per 32-channel step: INT4 order
// [0,4,1,5,2,6,3,7] (PERM) or natural (INT8).  Zero for heads beyond the group.
template <bool PERM>
KVT_DEV void load_q(const uint16_t* qrow, bool valid, int kb, h8 qop[8]) {
  constexpr int perm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
#pragma unroll
  for (int g = 0; g < 8; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = 32 * g + 8 * kb + (PERM ? perm[e] : e);
      qop[g][e] = valid ? (_Float16)bf16_to_f32(qrow[c]) : (_Float16)0.0f;
    }
  }
}

// Compiler-level ordering point for LDS traffic inside one wavefront (the hardware executes a wavefront's LDS
// instructions in order, so no memory fence is needed).
KVT_DEV void wave_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// One sub-chunk (up to kSub positions starting at p0, n valid) of one segment type.
template <bool HOT, int G8>
KVT_DEV void sub_chunk(const PosArgs& A, WaveLds& L, int b, int H, int h, int64_t p0, int n, int64_t rbase,
                       int64_t rmask, const h8 qop[8], float cscale, f4 acc[8], float& m_run, float& l_run) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  constexpr int NG8 = kD / G8;
  constexpr uint32_t kRowStride4 = kD / 2;   // INT4 bytes per (row, head)
  const uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, magic = 0x64006400u;
  wave_sync();
  // ---- stage rows and scales of the sub-chunk (2 positions per lane)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = lane + 64 * i;
    const bool ok = t < n;
    const int64_t p = p0 + (ok ? t : 0);
    int32_t row;
    if constexpr (HOT) {
      row = (int32_t)(rbase + (p & rmask));
    } else {
      row = A.page_table[b * A.pt_stride + (p >> 6)] * kPage + (int32_t)(p & (kPage - 1));
    }
    L.rows[t] = row;
    const uint32_t srow = (uint32_t)row * (uint32_t)H + (uint32_t)h;
    if constexpr (!HOT) {
      const uint4 ks = *reinterpret_cast<const uint4*>(A.ks4 + srow * 8u);
      uint4 vs = *reinterpret_cast<const uint4*>(A.vs4 + srow * 8u);
      if (!ok) vs = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(&L.sk[t][0]) = ks;
      const uint32_t v[4] = {vs.x, vs.y, vs.z, vs.w};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        L.sv[2 * g][t] = (uint16_t)(v[g] & 0xffffu);
        L.sv[2 * g + 1][t] = (uint16_t)(v[g] >> 16);
      }
    } else {
#pragma unroll
      for (int g = 0; g < NG8; ++g) {
        L.sk[t][g] = A.rks[srow * NG8 + g];
        L.sv[g][t] = ok ? A.rvs[srow * NG8 + g] : (uint16_t)0;
      }
    }
  }
  wave_sync();

  // ---- QK^T: 8 tiles of 16 tokens; lane holds scores of q head n16 % 8 for tokens 16 nt + 4 kb + r
  float s[8][4];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const uint32_t row = (uint32_t)L.rows[16 * nt + n16];   // token of this lane's A-operand row
    f4 sc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!HOT) {
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(A.k4 + (row * (uint32_t)H + h) * kRowStride4) + kb;
      uint32_t w[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) w[g] = kp[4 * g];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const f4 d = mfma(int4_codes_to_h8(w[g], mlo, mhi, magic), qop[g], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sg = f16_bits_to_f32(L.sk[16 * nt + 4 * kb + r][g]);
          sc[r] = fmaf(sg, d[r], sc[r]);
        }
      }
    } else {
      const uint2* kp = reinterpret_cast<const uint2*>(A.rk + (row * (uint32_t)H + h) * (uint32_t)kD) + kb;
      uint2 w[8];
#pragma unroll
      for (int st = 0; st < 8; ++st) w[st] = kp[4 * st];
      constexpr int STEPS_PER_GROUP = G8 / 32;
#pragma unroll
      for (int g = 0; g < NG8; ++g) {
        f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < STEPS_PER_GROUP; ++st) {
          const int stp = g * STEPS_PER_GROUP + st;
          d = mfma(int8_codes_to_h8(w[stp].x, w[stp].y), qop[stp], d);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sg = f16_bits_to_f32(L.sk[16 * nt + 4 * kb + r][g]);
          sc[r] = fmaf(sg, d[r], sc[r]);
        }
      }
    }
    if (n == kSub) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[nt][r] = sc[r] * cscale;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[nt][r] = (16 * nt + 4 * kb + r) < n ? sc[r] * cscale : -INFINITY;
    }
  }

  // ---- online softmax over the sub-chunk
  float mloc = -INFINITY;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) mloc = fmaxf(mloc, s[nt][r]);
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
  const float m_new = fmaxf(m_run, mloc);
  if (__any(m_new > m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // 0 on the first sub-chunk (m_run = -inf)
    l_run *= alpha;
    // accumulator rows are q heads (4 kb + i) % 8: fetch each row's alpha from a lane of that head
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, (4 * kb + i) & 7, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] *= arow[i];
  }
  m_run = m_new;
  float psum = 0.f;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[nt][r] = __builtin_amdgcn_exp2f(s[nt][r] - m_new);
      psum += s[nt][r];
    }
  l_run += psum;

  // ---- P.V: 4 tiles of 32 tokens; k slot e of lane block kb = token 32 pt + (e < 4 ? 4 kb + e : 16 + 4 kb + e - 4)
  const int kbp = kb ^ 2;                 // block of the partner lane (lane ^ 32)
  const bool lowrow = n16 < 8;
  const int cblk_a = n16, cblk_b = n16 + 16;   // 8-dim blocks: dims A = 8 n16 + e, dims B = 8 (n16 + 16) + e
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    const h8 pown = {(_Float16)s[2 * pt][0],     (_Float16)s[2 * pt][1],     (_Float16)s[2 * pt][2],
                     (_Float16)s[2 * pt][3],     (_Float16)s[2 * pt + 1][0], (_Float16)s[2 * pt + 1][1],
                     (_Float16)s[2 * pt + 1][2], (_Float16)s[2 * pt + 1][3]};
    const u4v po = as_u4(pown);
    u4v pp;
#pragma unroll
    for (int i = 0; i < 4; ++i) pp[i] = (uint32_t)__shfl_xor((int)po[i], 32, 64);
    const u4v zero = {0u, 0u, 0u, 0u};
    const h8 ax = as_h8(lowrow ? po : zero);
    const h8 ay = as_h8(lowrow ? zero : pp);
    int tok_o[8], tok_p[8];
    uint32_t row_o[8], row_p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int te = e < 4 ? e : 12 + e;    // 0..3, 16..19
      tok_o[e] = 32 * pt + 4 * kb + te;
      tok_p[e] = 32 * pt + 4 * kbp + te;
      row_o[e] = (uint32_t)L.rows[tok_o[e]];
      row_p[e] = (uint32_t)L.rows[tok_p[e]];
    }
    if constexpr (!HOT) {
      const int ga = cblk_a >> 2, gb = cblk_b >> 2;   // INT4 scale group of each dim block
      uint32_t wo[8], wp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        wo[e] = reinterpret_cast<const uint32_t*>(A.v4 + (row_o[e] * (uint32_t)H + h) * kRowStride4)[cblk_a];
        wp[e] = reinterpret_cast<const uint32_t*>(A.v4 + (row_p[e] * (uint32_t)H + h) * kRowStride4)[cblk_b];
      }
      h2 so[4], sp[4];
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        so[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[ga][tok_o[2 * pr]]));
        sp[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[gb][tok_p[2 * pr]]));
      }
      const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
      const h2 sc16 = {(_Float16)0.0625f, (_Float16)0.0625f};
      const h2 off2 = {(_Float16)-72.0f, (_Float16)-72.0f};
#pragma unroll
      for (int byte = 0; byte < 4; ++byte) {
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
        h8 olo, ohi, plo, phi;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t xo = __builtin_amdgcn_perm(wo[2 * pr + 1], wo[2 * pr], sel);  // [b(t0), 0, b(t1), 0]
          const uint32_t xp = __builtin_amdgcn_perm(wp[2 * pr + 1], wp[2 * pr], sel);
          const h2 lo_o = (as_h2(and_or(xo, mlo, magic)) + off) * so[pr];
          const h2 hi_o = (as_h2(and_or(xo, mhi, magic)) * sc16 + off2) * so[pr];
          const h2 lo_p = (as_h2(and_or(xp, mlo, magic)) + off) * sp[pr];
          const h2 hi_p = (as_h2(and_or(xp, mhi, magic)) * sc16 + off2) * sp[pr];
          olo[2 * pr] = lo_o.x; olo[2 * pr + 1] = lo_o.y;
          ohi[2 * pr] = hi_o.x; ohi[2 * pr + 1] = hi_o.y;
          plo[2 * pr] = lo_p.x; plo[2 * pr + 1] = lo_p.y;
          phi[2 * pr] = hi_p.x; phi[2 * pr + 1] = hi_p.y;
        }
        acc[2 * byte] = mfma(ax, olo, acc[2 * byte]);
        acc[2 * byte] = mfma(ay, plo, acc[2 * byte]);
        acc[2 * byte + 1] = mfma(ax, ohi, acc[2 * byte + 1]);
        acc[2 * byte + 1] = mfma(ay, phi, acc[2 * byte + 1]);
      }
    } else {
      const int ga = (8 * cblk_a) / G8, gb = (8 * cblk_b) / G8;   // INT8 scale groups of the dim blocks
      uint2 wo[8], wp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        wo[e] = reinterpret_cast<const uint2*>(A.rv + (row_o[e] * (uint32_t)H + h) * (uint32_t)kD)[cblk_a];
        wp[e] = reinterpret_cast<const uint2*>(A.rv + (row_p[e] * (uint32_t)H + h) * (uint32_t)kD)[cblk_b];
        wo[e].x ^= 0x80808080u; wo[e].y ^= 0x80808080u;
        wp[e].x ^= 0x80808080u; wp[e].y ^= 0x80808080u;
      }
      h2 so[4], sp[4];
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        so[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[ga][tok_o[2 * pr]]));
        sp[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[gb][tok_p[2 * pr]]));
      }
      const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t bsel = (uint32_t)(q & 3);
        const uint32_t sel = 0x0C000C00u | ((4 + bsel) << 16) | bsel;
        h8 bo, bp;
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
          const uint32_t xo = __builtin_amdgcn_perm(q < 4 ? wo[2 * pr + 1].x : wo[2 * pr + 1].y,
                                                    q < 4 ? wo[2 * pr].x : wo[2 * pr].y, sel);
          const uint32_t xp = __builtin_amdgcn_perm(q < 4 ? wp[2 * pr + 1].x : wp[2 * pr + 1].y,
                                                    q < 4 ? wp[2 * pr].x : wp[2 * pr].y, sel);
          const h2 vo = (as_h2(xo | magic) + off) * so[pr];
          const h2 vp = (as_h2(xp | magic) + off) * sp[pr];
          bo[2 * pr] = vo.x; bo[2 * pr + 1] = vo.y;
          bp[2 * pr] = vp.x; bp[2 * pr + 1] = vp.y;
        }
        acc[q] = mfma(ax, bo, acc[q]);
        acc[q] = mfma(ay, bp, acc[q]);
      }
    }
  }
}


struct ColdCtx {
  i32x4 rk4, rv4, rks4, rvs4;   // buffer resources of this layer's INT4 pool (codes K/V, scales K/V)
  uint32_t rowbytes;            // H * 128
  uint32_t hoff;                // h * 128
  int H, h;
};

// Issue the direct-to-LDS copies of one 32-token cold tile (pool rows row0 .. row0 + 31, n valid) into `st`:
// exactly 10 vector-memory instructions per wavefront (the vmcnt accounting of cold_segment relies on it).
KVT_DEV void cold_issue(const ColdCtx& C, ColdStage& st, uint32_t row0, int n) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 8 * j + (lane >> 3);
    const int tt = t < n ? t : n - 1;
    const uint32_t chunk = (uint32_t)((lane & 7) ^ (t & 7));
    const uint32_t off = (row0 + tt) * C.rowbytes + C.hoff + 16u * chunk;
    copy16_to_lds(C.rk4, st.k + 1024 * j, off);
    copy16_to_lds(C.rv4, st.v + 1024 * j, off);
  }
  const int tl = (lane & 31) < n ? (lane & 31) : n - 1;
  const uint32_t srow = (row0 + tl) * (uint32_t)C.H + (uint32_t)C.h;
  if (lane < 32) {
    copy16_to_lds(C.rks4, &st.ks[0][0], srow * 16u);
    copy16_to_lds(C.rvs4, &st.vsn[0][0], srow * 16u);
  }
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

KVT_DEV uint32_t lds_code_dword(const uint8_t* base, int t, int chunk, int dw) {
  return *reinterpret_cast<const uint32_t*>(base + t * 128 + 16 * (chunk ^ (t & 7)) + 4 * dw);
}

// Attention over one staged cold tile (n valid tokens).
KVT_DEV void cold_compute(const ColdStage& st, int n, const h8 qop[8], float cscale, f4 acc[8], float& m_run,
                          float& l_run) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  const uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, magic = 0x64006400u;
  float s[2][4];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int t = 16 * nt + n16;
    uint32_t w[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) w[g] = lds_code_dword(st.k, t, g, kb);
    f4 sc = {0.f, 0.f, 0.f, 0.f};
    uint4 ksr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ksr[r] = *reinterpret_cast<const uint4*>(&st.ks[16 * nt + 4 * kb + r][0]);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const f4 d = mfma(int4_codes_to_h8(w[g], mlo, mhi, magic), qop[g], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t pairw = g < 2 ? ksr[r].x : g < 4 ? ksr[r].y : g < 6 ? ksr[r].z : ksr[r].w;
        const float sg = f16_bits_to_f32((uint16_t)((g & 1) ? (pairw >> 16) : (pairw & 0xffffu)));
        sc[r] = fmaf(sg, d[r], sc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) s[nt][r] = (16 * nt + 4 * kb + r) < n ? sc[r] * cscale : -INFINITY;
  }
  // online softmax over the tile
  float mloc = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
  const float m_new = fmaxf(m_run, mloc);
  if (__any(m_new > m_run)) {
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, (4 * kb + i) & 7, 64);
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] *= arow[i];
  }
  m_run = m_new;
  float psum = 0.f;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[nt][r] = __builtin_amdgcn_exp2f(s[nt][r] - m_new);
      psum += s[nt][r];
    }
  l_run += psum;
  // P.V (block-diagonal, see the file header)
  const int kbp = kb ^ 2;
  const bool lowrow = n16 < 8;
  const h8 pown = {(_Float16)s[0][0], (_Float16)s[0][1], (_Float16)s[0][2], (_Float16)s[0][3],
                   (_Float16)s[1][0], (_Float16)s[1][1], (_Float16)s[1][2], (_Float16)s[1][3]};
  const u4v po = as_u4(pown);
  u4v pp;
#pragma unroll
  for (int i = 0; i < 4; ++i) pp[i] = (uint32_t)__shfl_xor((int)po[i], 32, 64);
  const u4v zero = {0u, 0u, 0u, 0u};
  const h8 ax = as_h8(lowrow ? po : zero);
  const h8 ay = as_h8(lowrow ? zero : pp);
  const int ga = n16 >> 2, gb = 4 + (n16 >> 2);      // INT4 scale groups of dims A (8 n16 ..) and B (8 (n16+16) ..)
  uint32_t wo[8], wp[8];
  int tok_o[8], tok_p[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int te = e < 4 ? e : 12 + e;
    tok_o[e] = 4 * kb + te;
    tok_p[e] = 4 * kbp + te;
    wo[e] = lds_code_dword(st.v, tok_o[e], n16 >> 2, n16 & 3);
    wp[e] = lds_code_dword(st.v, tok_p[e], 4 + (n16 >> 2), n16 & 3);
  }
  h2 so[4], sp[4];
#pragma unroll
  for (int pr = 0; pr < 4; ++pr) {
    so[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&st.sv[ga][tok_o[2 * pr]]));
    sp[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&st.sv[gb][tok_p[2 * pr]]));
  }
  const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
  const h2 sc16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 off2 = {(_Float16)-72.0f, (_Float16)-72.0f};
#pragma unroll
  for (int byte = 0; byte < 4; ++byte) {
    const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
    h8 olo, ohi, plo, phi;
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
      const uint32_t xo = __builtin_amdgcn_perm(wo[2 * pr + 1], wo[2 * pr], sel);
      const uint32_t xp = __builtin_amdgcn_perm(wp[2 * pr + 1], wp[2 * pr], sel);
      const h2 lo_o = (as_h2(and_or(xo, mlo, magic)) + off) * so[pr];
      const h2 hi_o = (as_h2(and_or(xo, mhi, magic)) * sc16 + off2) * so[pr];
      const h2 lo_p = (as_h2(and_or(xp, mlo, magic)) + off) * sp[pr];
      const h2 hi_p = (as_h2(and_or(xp, mhi, magic)) * sc16 + off2) * sp[pr];
      olo[2 * pr] = lo_o.x; olo[2 * pr + 1] = lo_o.y;
      ohi[2 * pr] = hi_o.x; ohi[2 * pr + 1] = hi_o.y;
      plo[2 * pr] = lo_p.x; plo[2 * pr + 1] = lo_p.y;
      phi[2 * pr] = hi_p.x; phi[2 * pr + 1] = hi_p.y;
    }
    acc[2 * byte] = mfma(ax, olo, acc[2 * byte]);
    acc[2 * byte] = mfma(ay, plo, acc[2 * byte]);
    acc[2 * byte + 1] = mfma(ax, ohi, acc[2 * byte + 1]);
    acc[2 * byte + 1] = mfma(ay, phi, acc[2 * byte + 1]);
  }
}

// The cold range [c0, c1) of one wavefront: c0 is 32-aligned, every tile lies in one page.
KVT_DEV void cold_segment(const PosArgs& A, const ColdCtx& C, WaveArea& W, int b, int64_t c0, int64_t c1,
                          const h8 qop[8], float cscale, f4 acc[8], float& m_run, float& l_run) {
  const int ntiles = (int)((c1 - c0 + 31) >> 5);
  // physical pages of the range, one per lane (a range is at most 64 pages), read back per tile with readlane
  const int lane = threadIdx.x & 63;
  const int64_t pg0 = c0 >> 6;
  const int npg = (int)(((c1 - 1) >> 6) - pg0 + 1);
  const int32_t pages = lane < npg ? A.page_table[b * A.pt_stride + pg0 + lane] : 0;
  auto tile_row0 = [&](int i) -> uint32_t {
    const int64_t p = c0 + 32 * (int64_t)i;
    const uint32_t page = (uint32_t)__builtin_amdgcn_readlane(pages, (int)((p >> 6) - pg0));
    return page * (uint32_t)kPage + (uint32_t)(p & (kPage - 1));
  };
  auto tile_n = [&](int i) -> int { return (int)min((int64_t)32, c1 - (c0 + 32 * (int64_t)i)); };
  wave_sync();
  cold_issue(C, W.cold[0], tile_row0(0), tile_n(0));
  for (int i = 0; i < ntiles; ++i) {
    // (the loop issues no vector-memory instruction besides the tile copies: the vmcnt counts below are exact)
    ColdStage& cur = W.cold[i & 1];
    if (i + 1 < ntiles) {
      cold_issue(C, W.cold[(i + 1) & 1], tile_row0(i + 1), tile_n(i + 1));
      wait_vmcnt<10>();                   // tile i's copies have landed
    } else {
      wait_vmcnt<0>();
    }
    cold_scatter_vs(cur);
    wave_sync();
    wave_sync();
    cold_compute(cur, tile_n(i), qop, cscale, acc, m_run, l_run);
    wave_sync();
  }
}

template <int G8>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) decode_mfma_kernel(PosArgs A, const uint16_t* q, int64_t q_stride_b,
                                                          const int32_t* seq_lens, int H, int gs, int chunk,
                                                          int n_chunks, float scale, float* part_o, float* part_ml,
                                                          uint32_t pool_rows_arg) {
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar addressing of the page table
  const int n16 = lane & 15, kb = lane >> 4;
  const int c = blockIdx.x;
  const int b = blockIdx.y / H;
  const int h = blockIdx.y - b * H;
  const int64_t item = ((int64_t)b * H + h) * n_chunks + c;
  const int64_t L = seq_lens[b];
  const int64_t R = A.ring_len[b];
  const int64_t rbase = A.ring_base[b];
  const int64_t hot_start = max(A.ring_start[b], L - R);
  const int cw = chunk / kWaves;
  const int64_t w0 = (int64_t)c * chunk + (int64_t)wave * cw;
  const int64_t w1 = min(w0 + cw, L);
  const float cscale = scale * kLog2e;
  const int hq = n16 & 7;
  const bool qvalid = hq < gs;
  const uint16_t* qrow = q + b * q_stride_b + (int64_t)(h * gs + (qvalid ? hq : 0)) * kD;

  f4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  h8 qop[8];

  // cold segment [w0, min(w1, hot_start)) from INT4 pages
  const int64_t ce = min(w1, hot_start);
  if (w0 < ce) {
    load_q<true>(qrow, qvalid, kb, qop);
    const uint32_t pool_rows = pool_rows_arg;
    ColdCtx C{buffer_rsrc(A.k4, pool_rows * (uint32_t)H * 128u), buffer_rsrc(A.v4, pool_rows * (uint32_t)H * 128u),
              buffer_rsrc(A.ks4, pool_rows * (uint32_t)H * 16u), buffer_rsrc(A.vs4, pool_rows * (uint32_t)H * 16u),
              (uint32_t)H * 128u, (uint32_t)h * 128u, H, h};
    cold_segment(A, C, lds.w[wave], b, w0, ce, qop, cscale, acc, m_run, l_run);
  }
  // hot segment [max(w0, hot_start), w1) from the INT8 ring
  const int64_t hs = max(w0, hot_start);
  if (hs < w1) {
    load_q<false>(qrow, qvalid, kb, qop);
    for (int64_t p = hs; p < w1; p += kSub)
      sub_chunk<true, G8>(A, lds.w[wave].hot, b, H, h, p, (int)min((int64_t)kSub, w1 - p), rbase, R - 1, qop, cscale,
                          acc, m_run, l_run);
  }

  // ---- merge the four wavefronts (heads 0-7 of the group; lanes n16 >= 8 duplicate n16 - 8)
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  __syncthreads();                        // every wavefront is done with its staging area
  if (kb == 0 && n16 < 8) {
    lds.merge.m[wave][n16] = m_run;
    lds.merge.l[wave][n16] = l_run;
  }
  __syncthreads();
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hr = (4 * kb + i) & 7;
    float M = lds.merge.m[0][hr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.merge.m[w][hr]);
    const float mw = lds.merge.m[wave][hr];
    wrow[i] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
  }
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * kb + i;
          const int dim = 8 * (n16 + (r >= 8 ? 16 : 0)) + j;
          const float v = acc[j][i] * wrow[i];
          if (w == 0) lds.merge.o[r & 7][dim] = v;
          else lds.merge.o[r & 7][dim] += v;
        }
      }
    }
    __syncthreads();
  }
  const int tid = threadIdx.x;
  for (int idx = tid; idx < gs * kD; idx += 256) {
    const int hh = idx / kD, d = idx - hh * kD;
    part_o[(item * gs + hh) * kD + d] = lds.merge.o[hh][d];
  }
  if (tid < gs) {
    float M = lds.merge.m[0][tid];
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.merge.m[w][tid]);
    float l = 0.f;
    for (int w = 0; w < kWaves; ++w) {
      const float mw = lds.merge.m[w][tid];
      l += mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M) * lds.merge.l[w][tid];
    }
    part_ml[(item * gs + tid) * 2 + 0] = M == -INFINITY ? -INFINITY : M / kLog2e;   // natural-log units
    part_ml[(item * gs + tid) * 2 + 1] = l;
  }
}

}  // namespace

extern "C" {

int kvt_decode_mfma(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                    int group8, const void* k4, const void* v4, const void* ks4, const void* vs4, const void* rk,
                    const void* rv, const void* rks, const void* rvs, const void* ring_base, const void* ring_len,
                    const void* ring_start, const void* page_table, int64_t pt_stride, int64_t pool_rows,
                    float scale, int chunk, int n_chunks, void* part_o, void* part_ml, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || D != kD) return KVT_EINVAL;
  if (pool_rows <= 0 || pool_rows * H * (kD / 2) > 0x7fffffffLL) return KVT_ERANGE;   // 32-bit byte offsets
  const int gs = Hq / H;
  if (gs > 8 || chunk <= 0 || chunk % (kWaves * 32) != 0 || chunk > 64 * 64 * kWaves || n_chunks <= 0)
    return KVT_EINVAL;   // a wavefront's range spans at most 64 pages
  PosArgs A{(const uint8_t*)k4,         (const uint8_t*)v4,        (const uint16_t*)ks4,     (const uint16_t*)vs4,
            (const int8_t*)rk,          (const int8_t*)rv,         (const uint16_t*)rks,     (const uint16_t*)rvs,
            (const int64_t*)ring_base,  (const int32_t*)ring_len,  (const int64_t*)ring_start,
            (const int32_t*)page_table, pt_stride};
  const dim3 grid((unsigned)n_chunks, (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
  if (group8 == 64) {
    hipLaunchKernelGGL(decode_mfma_kernel<64>, grid, dim3(256), 0, st, A, (const uint16_t*)q, q_stride_b,
                       (const int32_t*)seq_lens, H, gs, chunk, n_chunks, scale, (float*)part_o, (float*)part_ml,
                       (uint32_t)pool_rows);
  } else if (group8 == 256) {
    hipLaunchKernelGGL(decode_mfma_kernel<256>, grid, dim3(256), 0, st, A, (const uint16_t*)q, q_stride_b,
                       (const int32_t*)seq_lens, H, gs, chunk, n_chunks, scale, (float*)part_o, (float*)part_ml,
                       (uint32_t)pool_rows);
  } else {
    return KVT_EINVAL;
  }
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
