// Top-k sparse decode attention over the quantized pools, fused: the selected positions of each request are
// resolved (position -> slot through req_to_token -> tier through the owner table), dequantized exactly as the
// reference's compact gather does (bf16(q * s * sm), patches/kv_tiers.py:446-538) and attended in one pass, with no
// bf16 scratch.  The reference's decode gathers into that scratch and runs FlashAttention-2 over it
// (sglang/qwen4exp-serving-73a255206f.patch:1832-1882); this kernel replaces both launches' work, and its partials
// go through the same combine as the dense decode.
//
// One wavefront per (request, KV head, 16 selected columns): the 16 rows' K (row-major) and V (transposed) are
// dequantized into LDS as bf16, then QK^T and P.V run as bf16 16x16x16 matrix-core steps with fp32 accumulation:
//   S^T[row][head] = K[row][:] . Q[head][:]   (A = K tile, B = Q^T; 16 steps over the 256 channels)
//   O[head][ch]   += P[head][row] V[row][ch]  (A = P straight from S^T's accumulator layout as bf16 high part
//                                               + bf16 remainder, B = V^T tile)
// The wavefront writes an unnormalized partial (m, l, o) per q head (m in natural-log units, as the dense
// decode's); kvt_decode_combine merges the column splits.  Columns c of request b attend when c < the request's
// valid count (cu_k[b + 1] - cu_k[b]) and 0 <= indices[b][c] < seq_lens[b] - the columns the reference's gather
// writes and its attention reads when the valid positions come first (the indexer pads with -1 at the end).
//
// Kinds (the compact gather's codes): 0 INT8-G pool, 1 INT4-G32 pool, 2 tiered (INT8-G ring over INT4-G32 rows,
// owner test).

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kD = 256;
constexpr int kRows = 16;          // selected columns per wavefront (one MFMA tile)
constexpr int kHeads = 16;         // q heads per KV head the tile holds (rows beyond the group are zero)
constexpr int kKPitch = kD + 8;    // bf16 per K row in LDS (the pad spreads a column of rows over the banks)
constexpr int kVPitch = kRows + 4;  // bf16 per channel of the transposed V tile

typedef short bf4 __attribute__((ext_vector_type(4)));
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
  float scale;
  const uint16_t* q;       // bf16 [batch, Hq, D] with batch stride q_stride_b
  int64_t q_stride_b;
  float* part_o;           // [(b H + h) n_splits + split][gs][D]
  float* part_ml;          // [(b H + h) n_splits + split][gs][2]
};

KVT_DEV int64_t load_idx(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

// bf16 of code * scale * sm (the gather's rounding, patches/kv_tiers.py:516-526).
KVT_DEV uint32_t deq_bits(float code, float s, float sm) { return bf16_rne(code * s * sm); }

KVT_DEV float sm_at(const uint16_t* sm_s, int c) { return f16_bits_to_f32(sm_s[c]); }

// The 4 fp32 values of a bf16x4 operand.
KVT_DEV bf4 pack_bf4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return bf4{(short)a, (short)b, (short)c, (short)d};
}

KVT_DEV f4 mfma_bf16(bf4 a, bf4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0); }

template <int KIND, int G8>
__global__ void __launch_bounds__(64) sparse_decode_kernel(SparseArgs A) {
  constexpr int NG8 = kD / G8;
  __shared__ __align__(16) uint16_t kt[kRows * kKPitch];   // K rows, bf16
  __shared__ __align__(16) uint16_t vt[kD * kVPitch];      // V transposed: vt[ch][row], bf16
  __shared__ __align__(16) uint16_t qs[kHeads * kD];       // the group's q heads, bf16 (zero beyond gs)
  __shared__ __align__(16) uint16_t sms[2][kD];            // sm_k, sm_v of this KV head (fp16)
  const int lane = threadIdx.x;
  const int split = blockIdx.x;
  const int b = blockIdx.y / A.H;
  const int h = blockIdx.y - b * A.H;
  const int H = A.H, gs = A.gs;
  const int64_t item = ((int64_t)b * H + h) * A.n_splits + split;

  // 1. this tile's columns: lane r < 16 resolves column split * 16 + r to (valid, hot, row)
  const int64_t vcount = load_idx(A.cu_k, A.cu64, b + 1) - load_idx(A.cu_k, A.cu64, b);
  const int64_t L = A.seq_lens[b];
  const int64_t req = load_idx(A.req_indices, A.req64, b);
  const int col = split * kRows + (lane & (kRows - 1));
  bool valid = false, hot = KIND == 0;
  int64_t row = 0;
  if (lane < kRows && col < vcount && col < A.topk) {
    const int64_t pos = A.indices[(int64_t)b * A.idx_stride + col];
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
  // q heads and smoothing factors into LDS meanwhile (16-byte chunks: 512 of q, 64 of sm)
  for (int i = lane; i < kHeads * kD / 8; i += 64) {
    const int hq = i / (kD / 8), ch = i - hq * (kD / 8);
    uint4 w = {0u, 0u, 0u, 0u};
    if (hq < gs) w = *reinterpret_cast<const uint4*>(A.q + b * A.q_stride_b + (int64_t)(h * gs + hq) * kD + 8 * ch);
    *reinterpret_cast<uint4*>(&qs[hq * kD + 8 * ch]) = w;
  }
  {
    const int which = lane >> 5, ch = lane & 31;
    const uint16_t* sm = which ? A.sm_v : A.sm_k;
    uint4 w = {0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};   // fp16 1.0: no smoothing
    if (sm != nullptr) w = *reinterpret_cast<const uint4*>(sm + (int64_t)h * kD + 8 * ch);
    *reinterpret_cast<uint4*>(&sms[which][8 * ch]) = w;
  }
  const uint32_t rlo = (uint32_t)row, rhi = (uint32_t)((uint64_t)row >> 32);
  const int flags = (valid ? 1 : 0) | (hot ? 2 : 0);
  __syncthreads();   // q and sm staged

  // 2. K rows: lane = (row r = lane >> 2, channels 64 cq .. 64 cq + 63 with cq = lane & 3)
  {
    const int r = lane >> 2, cq = lane & 3;
    const int f = __shfl(flags, r, 64);
    const int64_t rr = (int64_t)(((uint64_t)(uint32_t)__shfl((int)rhi, r, 64) << 32) | (uint32_t)__shfl((int)rlo, r, 64));
    uint32_t outw[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) outw[j] = 0u;
    if (f & 1) {
      if (f & 2) {   // INT8 row (the ring when tiered, the pool when KIND 0)
        const int8_t* src = KIND == 2 ? A.rk : reinterpret_cast<const int8_t*>(A.k);
        const uint16_t* ssrc = KIND == 2 ? A.rks : A.ks;
        const int64_t base = (rr * H + h) * kD + 64 * cq;
        uint4 w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = *reinterpret_cast<const uint4*>(src + base + 16 * j);
        const float s = f16_bits_to_f32(ssrc[(rr * H + h) * NG8 + (64 * cq) / G8]);
        const uint32_t words[16] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w,
                                    w[2].x, w[2].y, w[2].z, w[2].w, w[3].x, w[3].y, w[3].z, w[3].w};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t word = words[j];
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            const int c = 64 * cq + 4 * j + e;
            const uint32_t lo = deq_bits((float)(int8_t)(word >> (8 * e)), s, sm_at(sms[0], c));
            const uint32_t hi = deq_bits((float)(int8_t)(word >> (8 * e + 8)), s, sm_at(sms[0], c + 1));
            outw[2 * j + e / 2] = lo | (hi << 16);
          }
        }
      } else {       // INT4-G32 row
        const uint8_t* src = reinterpret_cast<const uint8_t*>(A.k);
        const int64_t base = (rr * H + h) * (kD / 2) + 32 * cq;
        const uint4 w0 = *reinterpret_cast<const uint4*>(src + base);
        const uint4 w1 = *reinterpret_cast<const uint4*>(src + base + 16);
        const uint32_t sc = *reinterpret_cast<const uint32_t*>(A.ks + (rr * H + h) * (kD / kG4) + 2 * cq);
        const float s0 = f16_bits_to_f32((uint16_t)sc), s1 = f16_bits_to_f32((uint16_t)(sc >> 16));
        const uint32_t words[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float s = j < 4 ? s0 : s1;
#pragma unroll
          for (int e = 0; e < 4; ++e) {   // byte e: channel pair 2 (4 j + e), + 1
            const int c = 64 * cq + 8 * j + 2 * e;
            const uint32_t byte = (words[j] >> (8 * e)) & 0xffu;
            const uint32_t lo = deq_bits((float)((int)(byte & 15u) - 8), s, sm_at(sms[0], c));
            const uint32_t hi = deq_bits((float)((int)(byte >> 4) - 8), s, sm_at(sms[0], c + 1));
            outw[4 * j + e] = lo | (hi << 16);
          }
        }
      }
    }
    uint4* dst = reinterpret_cast<uint4*>(&kt[r * kKPitch + 64 * cq]);
#pragma unroll
    for (int j = 0; j < 8; ++j) dst[j] = uint4{outw[4 * j], outw[4 * j + 1], outw[4 * j + 2], outw[4 * j + 3]};
  }

  // 3. V rows, transposed: lane = (channels 16 g .. 16 g + 15 with g = lane & 15, rows 4 rq .. 4 rq + 3)
  {
    const int g = lane & 15, rq = lane >> 4;
    uint32_t vals[4][8];   // [row][channel pair]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * rq + i;
      const int f = __shfl(flags, r, 64);
      const int64_t rr = (int64_t)(((uint64_t)(uint32_t)__shfl((int)rhi, r, 64) << 32) | (uint32_t)__shfl((int)rlo, r, 64));
#pragma unroll
      for (int j = 0; j < 8; ++j) vals[i][j] = 0u;
      if (f & 1) {
        if (f & 2) {
          const int8_t* src = KIND == 2 ? A.rv : reinterpret_cast<const int8_t*>(A.v);
          const uint16_t* ssrc = KIND == 2 ? A.rvs : A.vs;
          const uint4 w = *reinterpret_cast<const uint4*>(src + (rr * H + h) * kD + 16 * g);
          const float s = f16_bits_to_f32(ssrc[(rr * H + h) * NG8 + (16 * g) / G8]);
          const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int c = 16 * g + 2 * j;
            const uint32_t word = words[j >> 1];
            const int sh = 16 * (j & 1);
            const uint32_t lo = deq_bits((float)(int8_t)(word >> sh), s, sm_at(sms[1], c));
            const uint32_t hi = deq_bits((float)(int8_t)(word >> (sh + 8)), s, sm_at(sms[1], c + 1));
            vals[i][j] = lo | (hi << 16);
          }
        } else {
          const uint8_t* src = reinterpret_cast<const uint8_t*>(A.v);
          const uint2 w = *reinterpret_cast<const uint2*>(src + (rr * H + h) * (kD / 2) + 8 * g);
          const float s = f16_bits_to_f32(A.vs[(rr * H + h) * (kD / kG4) + (g >> 1)]);
          const uint32_t words[2] = {w.x, w.y};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int c = 16 * g + 2 * j;
            const uint32_t byte = (words[j >> 2] >> (8 * (j & 3))) & 0xffu;
            const uint32_t lo = deq_bits((float)((int)(byte & 15u) - 8), s, sm_at(sms[1], c));
            const uint32_t hi = deq_bits((float)((int)(byte >> 4) - 8), s, sm_at(sms[1], c + 1));
            vals[i][j] = lo | (hi << 16);
          }
        }
      }
    }
    // vt[ch][4 rq .. 4 rq + 3]: 8 bytes per channel
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int ch = 16 * g + 2 * j + e;
        const uint32_t r01 = e ? ((vals[0][j] >> 16) | (vals[1][j] & 0xffff0000u)) : ((vals[0][j] & 0xffffu) | (vals[1][j] << 16));
        const uint32_t r23 = e ? ((vals[2][j] >> 16) | (vals[3][j] & 0xffff0000u)) : ((vals[2][j] & 0xffffu) | (vals[3][j] << 16));
        *reinterpret_cast<uint2*>(&vt[ch * kVPitch + 4 * rq]) = uint2{r01, r23};
      }
    }
  }
  __syncthreads();

  // 4. S^T = K Q^T: lane l holds rows 4 (l >> 4) + i of q head l & 15
  const int n16 = lane & 15, kq = lane >> 4;
  f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k0 = 0; k0 < kD; k0 += 16) {
    const uint2 ka = *reinterpret_cast<const uint2*>(&kt[n16 * kKPitch + k0 + 4 * kq]);
    const uint2 qb = *reinterpret_cast<const uint2*>(&qs[n16 * kD + k0 + 4 * kq]);
    s = mfma_bf16(pack_bf4(ka.x & 0xffffu, ka.x >> 16, ka.y & 0xffffu, ka.y >> 16),
                  pack_bf4(qb.x & 0xffffu, qb.x >> 16, qb.y & 0xffffu, qb.y >> 16), s);
  }
  // softmax over the tile's rows (log2 units): rows 4 kq + i of this lane, the other 12 in lanes n16 + 16 j
  constexpr float kLog2e = 1.4426950408889634f;
  const float cs = A.scale * kLog2e;
  float t[4];
  float mloc = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = (__shfl(flags, 4 * kq + i, 64) & 1) != 0;
    t[i] = ok ? s[i] * cs : -INFINITY;
    mloc = fmaxf(mloc, t[i]);
  }
  const float m = max_xor16_32(mloc);
  float p[4], lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(t[i] - m);
    lsum += p[i];
  }
  const float l = sum_xor16_32(lsum);
  // P as bf16 high part + bf16 remainder (two products per step): P keeps ~16 significant bits, against 8 for a
  // plain bf16 cast, so a peaked softmax (few columns) stays within the fp32 reference's tolerance
  uint32_t ph[4], pl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ph[i] = bf16_rne(p[i]);
    pl[i] = bf16_rne(p[i] - bf16_to_f32((uint16_t)ph[i]));
  }
  const bf4 pa = pack_bf4(ph[0], ph[1], ph[2], ph[3]);
  const bf4 pb = pack_bf4(pl[0], pl[1], pl[2], pl[3]);

  // 5. O = P V: lane l holds q heads 4 (l >> 4) + i, channel n0 + (l & 15)
  const int64_t obase = item * gs;
#pragma unroll
  for (int n0 = 0; n0 < kD; n0 += 16) {
    const uint2 vb = *reinterpret_cast<const uint2*>(&vt[(n0 + n16) * kVPitch + 4 * kq]);
    const bf4 vop = pack_bf4(vb.x & 0xffffu, vb.x >> 16, vb.y & 0xffffu, vb.y >> 16);
    const f4 o = mfma_bf16(pb, vop, mfma_bf16(pa, vop, f4{0.f, 0.f, 0.f, 0.f}));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hq = 4 * kq + i;
      if (hq < gs) A.part_o[(obase + hq) * kD + n0 + n16] = o[i];
    }
  }
  if (lane < gs) {   // lanes 0 .. gs - 1 hold q heads 0 .. gs - 1 in the softmax layout
    constexpr float kLn2 = 0.6931471805599453f;
    A.part_ml[(obase + lane) * 2 + 0] = m == -INFINITY ? -INFINITY : m * kLn2;
    A.part_ml[(obase + lane) * 2 + 1] = l;
  }
}

}  // namespace

extern "C" {

int kvt_sparse_decode(int kind, const void* q, int64_t q_stride_b, const void* k, const void* v, const void* k_scale,
                      const void* v_scale, const void* ring_k, const void* ring_v, const void* ring_ks,
                      const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                      int cu_is_int64, int batch, int topk, int H, int Hq, int D, int group8, float scale,
                      int n_splits, void* part_o, void* part_ml, void* stream) {
  if (batch <= 0 || topk <= 0 || H <= 0 || Hq % H != 0 || Hq / H > kHeads || D != kD) return KVT_EINVAL;
  if (n_splits < (topk + kRows - 1) / kRows || kind < 0 || kind > 2) return KVT_EINVAL;
  if (kind == 2 && (owner == nullptr || ring_k == nullptr || ((ring_mask + 1) & ring_mask) != 0)) return KVT_EINVAL;
  SparseArgs A{k, v, (const uint16_t*)k_scale, (const uint16_t*)v_scale, (const int8_t*)ring_k, (const int8_t*)ring_v,
               (const uint16_t*)ring_ks, (const uint16_t*)ring_vs, (const int32_t*)owner, ring_mask,
               (const uint16_t*)sm_k, (const uint16_t*)sm_v, (const int32_t*)req_to_token, req_stride, req_indices,
               req_is_int64, (const int32_t*)indices, idx_stride, (const int32_t*)seq_lens, cu_k, cu_is_int64, topk,
               H, Hq / H, n_splits, scale, (const uint16_t*)q, q_stride_b, (float*)part_o, (float*)part_ml};
  const dim3 grid((unsigned)n_splits, (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
#define KVT_SD(KIND_, G_) hipLaunchKernelGGL((sparse_decode_kernel<KIND_, G_>), grid, dim3(64), 0, st, A)
  if (kind == 1) {
    KVT_SD(1, 64);
  } else if (group8 == 64) {
    if (kind == 2) {
      KVT_SD(2, 64);
    } else {
      KVT_SD(0, 64);
    }
  } else if (group8 == 256) {
    if (kind == 2) {
      KVT_SD(2, 256);
    } else {
      KVT_SD(0, 256);
    }
  } else {
    return KVT_EINVAL;
  }
#undef KVT_SD
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
