// Split-K GQA decode attention over the position-indexed tiered cache on gfx950 matrix cores.
//
// Work item = (sequence, KV head, split of `chunk` positions); 4 wavefronts per block, each owning a quarter of the
// split, which it walks in sub-chunks of 128 positions: cold positions (< hot_start) read INT4-G32 pages through the
// page table, hot positions the INT8 ring row (position mod R).  GQA groups of up to 8 q heads per KV head.
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

struct Lds {
  WaveLds w[kWaves];
  float m[kWaves][8];
  float l[kWaves][8];
  float o[8][kD];
};

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

KVT_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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

template <int G8>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) decode_mfma_kernel(PosArgs A, const uint16_t* q, int64_t q_stride_b,
                                                          const int32_t* seq_lens, int H, int gs, int chunk,
                                                          int n_chunks, float scale, float* part_o, float* part_ml) {
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
    for (int64_t p = w0; p < ce; p += kSub)
      sub_chunk<false, G8>(A, lds.w[wave], b, H, h, p, (int)min((int64_t)kSub, ce - p), rbase, R - 1, qop, cscale,
                           acc, m_run, l_run);
  }
  // hot segment [max(w0, hot_start), w1) from the INT8 ring
  const int64_t hs = max(w0, hot_start);
  if (hs < w1) {
    load_q<false>(qrow, qvalid, kb, qop);
    for (int64_t p = hs; p < w1; p += kSub)
      sub_chunk<true, G8>(A, lds.w[wave], b, H, h, p, (int)min((int64_t)kSub, w1 - p), rbase, R - 1, qop, cscale,
                          acc, m_run, l_run);
  }

  // ---- merge the four wavefronts (heads 0-7 of the group; lanes n16 >= 8 duplicate n16 - 8)
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (kb == 0 && n16 < 8) {
    lds.m[wave][n16] = m_run;
    lds.l[wave][n16] = l_run;
  }
  __syncthreads();
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hr = (4 * kb + i) & 7;
    float M = lds.m[0][hr];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.m[w][hr]);
    const float mw = lds.m[wave][hr];
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
          if (w == 0) lds.o[r & 7][dim] = v;
          else lds.o[r & 7][dim] += v;
        }
      }
    }
    __syncthreads();
  }
  const int tid = threadIdx.x;
  for (int idx = tid; idx < gs * kD; idx += 256) {
    const int hh = idx / kD, d = idx - hh * kD;
    part_o[(item * gs + hh) * kD + d] = lds.o[hh][d];
  }
  if (tid < gs) {
    float M = lds.m[0][tid];
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.m[w][tid]);
    float l = 0.f;
    for (int w = 0; w < kWaves; ++w) {
      const float mw = lds.m[w][tid];
      l += mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M) * lds.l[w][tid];
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
                    const void* ring_start, const void* page_table, int64_t pt_stride, float scale, int chunk,
                    int n_chunks, void* part_o, void* part_ml, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || D != kD) return KVT_EINVAL;
  const int gs = Hq / H;
  if (gs > 8 || chunk <= 0 || chunk % (kWaves * 32) != 0 || n_chunks <= 0) return KVT_EINVAL;
  PosArgs A{(const uint8_t*)k4,         (const uint8_t*)v4,        (const uint16_t*)ks4,     (const uint16_t*)vs4,
            (const int8_t*)rk,          (const int8_t*)rv,         (const uint16_t*)rks,     (const uint16_t*)rvs,
            (const int64_t*)ring_base,  (const int32_t*)ring_len,  (const int64_t*)ring_start,
            (const int32_t*)page_table, pt_stride};
  const dim3 grid((unsigned)n_chunks, (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
  if (group8 == 64) {
    hipLaunchKernelGGL(decode_mfma_kernel<64>, grid, dim3(256), 0, st, A, (const uint16_t*)q, q_stride_b,
                       (const int32_t*)seq_lens, H, gs, chunk, n_chunks, scale, (float*)part_o, (float*)part_ml);
  } else if (group8 == 256) {
    hipLaunchKernelGGL(decode_mfma_kernel<256>, grid, dim3(256), 0, st, A, (const uint16_t*)q, q_stride_b,
                       (const int32_t*)seq_lens, H, gs, chunk, n_chunks, scale, (float*)part_o, (float*)part_ml);
  } else {
    return KVT_EINVAL;
  }
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
