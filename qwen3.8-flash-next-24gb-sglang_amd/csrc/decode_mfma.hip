// Split-K GQA decode attention over the position-indexed tiered cache on gfx950 matrix cores.
//
// Work item = (sequence, KV head, split of `chunk` positions); 4 wavefronts per block, each owning a quarter of
// the split, which it walks in sub-chunks of 128 positions: cold positions (< hot_start) read INT4-G32 pages through
// the page table, hot positions the INT8 ring row (position mod R).
//
// QK^T on v_mfma_f32_16x16x32_f16, one instruction per 16 tokens x 32 channels (= one INT4 scale group):
//   A = K codes as exact fp16 integers (16 tokens x 32 channels); B = Q (32 channels x 16 columns, the GQA group's
//   q heads, zero beyond the group).  The fp16 codes come from the magic-number conversion
//   (0x6400 | nibble) = 1024 + nibble, minus 1032 (for the high nibble: (1024 + 16 n) / 16 - 72); channels appear in
//   the order [0,4,1,5,2,6,3,7] of each 8, and Q is loaded in the same order (a contraction is order-free).
//   The per-(token, group) fp16 scale is folded into the fp32 group result: score += s_g(t) * D_g.
// Softmax: scores sit in the MFMA D layout (lane = q head, 4 tokens of each 16-token tile); that layout is exactly
//   the A operand of P.V (lane = q head, 8 tokens), so P needs no transpose.  exp2 with the log2(e) factor folded
//   into the score scale; the running max is rescaled only when it grows (wave-uniform test).
// P.V on the same instruction: A = P (fp16), B = V dequantized to fp16 (code * scale, exact code conversion then one
//   packed multiply by the per-(token, group) scale pair), 16 instructions per 32 tokens, fp32 accumulators.
// The four wavefronts merge their (max, sum, o) in LDS; one fp32 partial per work item goes to kvt_decode_combine.
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

// 8 INT4 codes (one dword, channels c0..c7 = nibbles 0..7) -> fp16 (c - 8) in the order [c0,c4,c1,c5,c2,c6,c3,c7].
KVT_DEV h8 int4_codes_to_h8(uint32_t w) {
  const uint32_t w8 = w >> 8;
  const h2 lo0 = as_h2((w & 0x000F000Fu) | 0x64006400u);   // 1024 + (c0, c4)
  const h2 hi0 = as_h2((w & 0x00F000F0u) | 0x64006400u);   // 1024 + 16 (c1, c5)
  const h2 lo1 = as_h2((w8 & 0x000F000Fu) | 0x64006400u);  // 1024 + (c2, c6)
  const h2 hi1 = as_h2((w8 & 0x00F000F0u) | 0x64006400u);  // 1024 + 16 (c3, c7)
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

// Row of position p of sequence b (cold: INT4 pool row through the page table; hot: ring row).
template <bool HOT>
KVT_DEV int64_t pos_row(const PosArgs& A, int b, int64_t p, int64_t rbase, int64_t rmask) {
  if constexpr (HOT) {
    return rbase + (p & rmask);
  } else {
    return (int64_t)A.page_table[b * A.pt_stride + (p >> 6)] * kPage + (p & (kPage - 1));
  }
}

struct WaveLds {
  int32_t rows[kSub];
  uint16_t sk[kSub][8];   // K scales, [token][group]
  uint16_t sv[8][kSub];   // V scales, [group][token]
};

struct Lds {
  WaveLds w[kWaves];
  float m[kWaves][16];
  float l[kWaves][16];
  float o[16][kD];
};

// Q of this lane (q head n = lane % 16, channel block kb = lane / 16) as 8 MFMA B operands, one per 32-channel
// step: INT4 order [0,4,1,5,2,6,3,7] (PERM) or natural (INT8).  Zero beyond the GQA group.
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

// One sub-chunk (up to kSub positions starting at p0, n valid) of one segment type.
template <bool HOT, int G8>
KVT_DEV void sub_chunk(const PosArgs& A, WaveLds& L, int b, int H, int h, int64_t p0, int n, int64_t rbase,
                       int64_t rmask, const h8 qop[8], float cscale, f4 acc[16], float& m_run, float& l_run) {
  const int lane = threadIdx.x & 63;
  const int n16 = lane & 15, kb = lane >> 4;
  constexpr int NG8 = kD / G8;
  // ---- stage rows and scales of the sub-chunk (2 positions per lane)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int t = lane + 64 * i;
    const bool ok = t < n;
    const int64_t row = pos_row<HOT>(A, b, p0 + (ok ? t : 0), rbase, rmask);
    L.rows[t] = (int32_t)row;
    if constexpr (!HOT) {
      const uint4 ks = *reinterpret_cast<const uint4*>(A.ks4 + (row * H + h) * 8);
      uint4 vs = *reinterpret_cast<const uint4*>(A.vs4 + (row * H + h) * 8);
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
        L.sk[t][g] = A.rks[(row * H + h) * NG8 + g];
        L.sv[g][t] = ok ? A.rvs[(row * H + h) * NG8 + g] : (uint16_t)0;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- QK^T: 8 tiles of 16 tokens; lane holds scores of q head n16 for tokens 16 nt + 4 kb + r
  float s[8][4];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) {
    const int trow = 16 * nt + n16;  // token of this lane's A-operand row
    const int64_t row = L.rows[trow];
    f4 sc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!HOT) {
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(A.k4 + (row * H + h) * (kD / 2)) + kb;
      uint32_t w[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) w[g] = kp[4 * g];
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const f4 d = mfma(int4_codes_to_h8(w[g]), qop[g], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sg = f16_bits_to_f32(L.sk[16 * nt + 4 * kb + r][g]);
          sc[r] = fmaf(sg, d[r], sc[r]);
        }
      }
    } else {
      const uint2* kp = reinterpret_cast<const uint2*>(A.rk + (row * H + h) * kD) + kb;
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
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * nt + 4 * kb + r;
      s[nt][r] = t < n ? sc[r] * cscale : -INFINITY;
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
    const float alpha = exp2f(m_run - m_new);   // 0 on the first sub-chunk (m_run = -inf)
    l_run *= alpha;
    // acc rows are q heads 4 kb + i: fetch each head's alpha from its owner lane (head column)
    float arow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) arow[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
    for (int j = 0; j < 16; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[j][i] *= arow[i];
  }
  m_run = m_new;
  float psum = 0.f;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[nt][r] = exp2f(s[nt][r] - m_new);
      psum += s[nt][r];
    }
  l_run += psum;

  // ---- P.V: 4 tiles of 32 tokens; k slot e of lane (kb) = token 32 pt + (e < 4 ? 4 kb + e : 16 + 4 kb + e - 4)
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) {
    const h8 pa = {(_Float16)s[2 * pt][0],     (_Float16)s[2 * pt][1],     (_Float16)s[2 * pt][2],
                   (_Float16)s[2 * pt][3],     (_Float16)s[2 * pt + 1][0], (_Float16)s[2 * pt + 1][1],
                   (_Float16)s[2 * pt + 1][2], (_Float16)s[2 * pt + 1][3]};
    int tok[8];
    int64_t rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      tok[e] = 32 * pt + (e < 4 ? 4 * kb + e : 16 + 4 * kb + e - 4);
      rows[e] = L.rows[tok[e]];
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int cblk = n16 + 16 * half;     // this lane's 8-dim block: dims 8 cblk .. 8 cblk + 7
      if constexpr (!HOT) {
        const int g = cblk >> 2;            // INT4 scale group of those dims
        uint32_t w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          w[e] = reinterpret_cast<const uint32_t*>(A.v4 + (rows[e] * H + h) * (kD / 2))[cblk];
        h2 spair[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr)
          spair[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[g][tok[2 * pr]]));
        const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
        const h2 sc16 = {(_Float16)0.0625f, (_Float16)0.0625f};
        const h2 off2 = {(_Float16)-72.0f, (_Float16)-72.0f};
#pragma unroll
        for (int byte = 0; byte < 4; ++byte) {
          h8 blo, bhi;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
            const uint32_t x = __builtin_amdgcn_perm(w[2 * pr + 1], w[2 * pr], sel);  // [b(t0), 0, b(t1), 0]
            const h2 lo = (as_h2((x & 0x000F000Fu) | 0x64006400u) + off) * spair[pr];
            const h2 hi = (as_h2((x & 0x00F000F0u) | 0x64006400u) * sc16 + off2) * spair[pr];
            blo[2 * pr] = lo.x;
            blo[2 * pr + 1] = lo.y;
            bhi[2 * pr] = hi.x;
            bhi[2 * pr + 1] = hi.y;
          }
          acc[8 * half + 2 * byte] = mfma(pa, blo, acc[8 * half + 2 * byte]);
          acc[8 * half + 2 * byte + 1] = mfma(pa, bhi, acc[8 * half + 2 * byte + 1]);
        }
      } else {
        const int g = (8 * cblk) / G8;      // INT8 scale group of those dims
        uint2 w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          w[e] = reinterpret_cast<const uint2*>(A.rv + (rows[e] * H + h) * kD)[cblk];
          w[e].x ^= 0x80808080u;
          w[e].y ^= 0x80808080u;
        }
        h2 spair[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr)
          spair[pr] = as_h2(*reinterpret_cast<const uint32_t*>(&L.sv[g][tok[2 * pr]]));
        const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          h8 bv;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            const uint32_t a0 = q < 4 ? w[2 * pr].x : w[2 * pr].y;
            const uint32_t a1 = q < 4 ? w[2 * pr + 1].x : w[2 * pr + 1].y;
            const uint32_t bsel = (uint32_t)(q & 3);
            const uint32_t x = __builtin_amdgcn_perm(a1, a0, 0x0C000C00u | ((4 + bsel) << 16) | bsel);
            const h2 v = (as_h2(x | 0x64006400u) + off) * spair[pr];
            bv[2 * pr] = v.x;
            bv[2 * pr + 1] = v.y;
          }
          acc[8 * half + q] = mfma(pa, bv, acc[8 * half + q]);
        }
      }
    }
  }
}

template <int G8>
__global__ void __launch_bounds__(256) decode_mfma_kernel(PosArgs A, const uint16_t* q, int64_t q_stride_b,
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
  const uint16_t* qrow = q + b * q_stride_b + (int64_t)(h * gs + min(n16, gs - 1)) * kD;
  const bool qvalid = n16 < gs;

  f4 acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
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

  // ---- merge the four wavefronts
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  if (kb == 0) {
    lds.m[wave][n16] = m_run;
    lds.l[wave][n16] = l_run;
  }
  __syncthreads();
  // per acc row (q head 4 kb + i) the wave's weight exp2(m_wave - M)
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hq = 4 * kb + i;
    float M = lds.m[0][hq];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.m[w][hq]);
    const float mw = lds.m[wave][hq];
    wrow[i] = mw == -INFINITY ? 0.f : exp2f(mw - M);
  }
  for (int w = 0; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int dim = 8 * (n16 + 16 * (j >> 3)) + (j & 7);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int hq = 4 * kb + i;
          const float v = acc[j][i] * wrow[i];
          if (w == 0) lds.o[hq][dim] = v;
          else lds.o[hq][dim] += v;
        }
      }
    }
    __syncthreads();
  }
  const int tid = threadIdx.x;
  for (int idx = tid; idx < gs * kD; idx += 256) {
    const int hq = idx / kD, d = idx - hq * kD;
    part_o[(item * gs + hq) * kD + d] = lds.o[hq][d];
  }
  if (tid < gs) {
    float M = lds.m[0][tid];
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, lds.m[w][tid]);
    float l = 0.f;
    for (int w = 0; w < kWaves; ++w) {
      const float mw = lds.m[w][tid];
      l += mw == -INFINITY ? 0.f : exp2f(mw - M) * lds.l[w][tid];
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
  if (gs > 16 || chunk <= 0 || chunk % (kWaves * 32) != 0 || n_chunks <= 0) return KVT_EINVAL;
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
