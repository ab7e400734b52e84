// Split-K GQA decode attention over the tiered cache, reference-precision variant, and the split combine.
//
// Every K/V element is dequantized exactly as the reference's gathers do (bf16(q * s * sm),
// patches/kv_tiers.py:516-526) and the softmax attention runs in fp32 (the oracle form,
// gemv/test_kv_paged_prefix.py:520-528).  It serves the slot-indexed (dual-write) layout, where the tier of a
// token is only known from the owner table, and is the on-device cross-check of the MFMA kernel.
//
// Work item = (sequence, KV head, chunk of `chunk` positions); 256 threads:
//   phase 1  thread-per-token scores for the GQA group's q heads (q * scale in LDS, fp32)
//   phase 2  per-head max / exp / sum over the chunk in LDS
//   phase 3  thread-per-channel P.V accumulation
// and writes an unnormalized partial (m, l, o) per q head.  kvt_decode_combine merges the chunks.

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunk = 512;
constexpr int kMaxGroup = 16;  // q heads per KV head

struct TierArgs {
  // pools (INT4 codes [rows, H, D/2], scales [rows, H, D/32]; INT8 ring [R, H, D], scales [R, H, D/G8])
  const uint8_t* k4;
  const uint8_t* v4;
  const uint16_t* ks4;
  const uint16_t* vs4;
  const int8_t* rk;
  const int8_t* rv;
  const uint16_t* rks;
  const uint16_t* rvs;
  const uint16_t* sm_k;  // may be null (identity)
  const uint16_t* sm_v;
  // mode 0 (position rings): per sequence
  const int64_t* ring_base;
  const int32_t* ring_len;
  const int64_t* ring_start;
  const int32_t* page_table;
  int64_t pt_stride;
  // mode 1 (slot rings): req_to_token[req_indices[b]][p] -> slot, owner table
  const int32_t* req_to_token;
  int64_t req_stride;
  const int64_t* req_indices;
  const int32_t* owner;
  int64_t ring_mask;
};

// Resolve position p of sequence b to (hot, row): row is the ring row when hot, the INT4 pool row otherwise.
template <int MODE>
KVT_DEV bool resolve(const TierArgs& A, int b, int64_t p, int64_t hot_start, int64_t* row) {
  if constexpr (MODE == 0) {
    if (p >= hot_start) {
      *row = A.ring_base[b] + (p & ((int64_t)A.ring_len[b] - 1));
      return true;
    }
    *row = (int64_t)A.page_table[b * A.pt_stride + (p >> 6)] * kPage + (p & (kPage - 1));
    return false;
  } else {
    const int64_t slot = A.req_to_token[A.req_indices[b] * A.req_stride + p];
    const int64_t r = slot & A.ring_mask;
    if ((int64_t)A.owner[r] == slot) {
      *row = r;
      return true;
    }
    *row = slot;
    return false;
  }
}

template <int D, int G8>
KVT_DEV float dequant_elem(bool hot, const int8_t* r8, const uint16_t* rs8, const uint8_t* p4, const uint16_t* ps4,
                           int64_t row, int H, int h, int c, const uint16_t* sm) {
  float x;
  if (hot) {
    x = (float)r8[(row * H + h) * D + c] * f16_bits_to_f32(rs8[(row * H + h) * (D / G8) + c / G8]);
  } else {
    const uint32_t b = p4[(row * H + h) * (D / 2) + (c >> 1)];
    const int n = (int)((c & 1) ? (b >> 4) : (b & 15u)) - 8;
    x = (float)n * f16_bits_to_f32(ps4[(row * H + h) * (D / kG4) + c / kG4]);
  }
  if (sm) x *= f16_bits_to_f32(sm[h * D + c]);
  return bf16_to_f32(bf16_rne(x));
}

template <int MODE, int D, int G8>
__global__ void __launch_bounds__(kThreads) decode_ref_kernel(TierArgs A, const uint16_t* q, int64_t q_stride_b,
                                                              const int32_t* seq_lens, int H, int gs, int chunk,
                                                              int n_chunks, float scale, float* part_o,
                                                              float* part_ml) {
  __shared__ float q_s[kMaxGroup * D];
  __shared__ float p_s[kMaxGroup * kMaxChunk];
  __shared__ float red[kThreads / 64][kMaxGroup];
  const int c = blockIdx.x;
  const int b = blockIdx.y / H;
  const int h = blockIdx.y - b * H;
  const int tid = threadIdx.x;
  const int64_t L = seq_lens[b];
  const int64_t p0 = (int64_t)c * chunk;
  const int64_t item = ((int64_t)b * H + h) * n_chunks + c;
  const int n = (int)max((int64_t)0, min((int64_t)chunk, L - p0));
  int64_t hot_start = 0;
  if constexpr (MODE == 0) hot_start = max(A.ring_start[b], L - (int64_t)A.ring_len[b]);

  for (int i = tid; i < gs * D; i += kThreads) {
    const int hq = i / D, d = i - hq * D;
    q_s[i] = bf16_to_f32(q[b * q_stride_b + (int64_t)(h * gs + hq) * D + d]) * scale;
  }
  __syncthreads();

  // phase 1: scores
  for (int t = tid; t < n; t += kThreads) {
    int64_t row;
    const bool hot = resolve<MODE>(A, b, p0 + t, hot_start, &row);
    float acc[kMaxGroup];
    for (int j = 0; j < gs; ++j) acc[j] = 0.0f;
    for (int d = 0; d < D; ++d) {
      const float kv = dequant_elem<D, G8>(hot, A.rk, A.rks, A.k4, A.ks4, row, H, h, d, A.sm_k);
      for (int j = 0; j < gs; ++j) acc[j] = fmaf(q_s[j * D + d], kv, acc[j]);
    }
    for (int j = 0; j < gs; ++j) p_s[j * kMaxChunk + t] = acc[j];
  }
  __syncthreads();

  // phase 2: per-head max and sum of exp (each wave reduces all heads over its slice, then across waves)
  const int wave = tid >> 6, lane = tid & 63;
  for (int j = 0; j < gs; ++j) {
    float m = -INFINITY;
    for (int t = tid; t < n; t += kThreads) m = fmaxf(m, p_s[j * kMaxChunk + t]);
    m = group_max<64>(m);
    if (lane == 0) red[wave][j] = m;
  }
  __syncthreads();
  float mrow[kMaxGroup];
  for (int j = 0; j < gs; ++j) {
    float m = red[0][j];
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w][j]);
    mrow[j] = m;
  }
  __syncthreads();
  for (int j = 0; j < gs; ++j) {
    float s = 0.0f;
    for (int t = tid; t < n; t += kThreads) {
      const float e = expf(p_s[j * kMaxChunk + t] - mrow[j]);
      p_s[j * kMaxChunk + t] = e;
      s += e;
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wave][j] = s;
  }
  __syncthreads();
  if (tid < gs) {
    float s = 0.0f;
    for (int w = 0; w < kThreads / 64; ++w) s += red[w][tid];
    part_ml[(item * gs + tid) * 2 + 0] = n > 0 ? mrow[tid] : -INFINITY;
    part_ml[(item * gs + tid) * 2 + 1] = s;
  }

  // phase 3: o[j][d] = sum_t p[j][t] * v[t][d]
  for (int d = tid; d < D; d += kThreads) {
    float acc[kMaxGroup];
    for (int j = 0; j < gs; ++j) acc[j] = 0.0f;
    for (int t = 0; t < n; ++t) {
      int64_t row;
      const bool hot = resolve<MODE>(A, b, p0 + t, hot_start, &row);
      const float vv = dequant_elem<D, G8>(hot, A.rv, A.rvs, A.v4, A.vs4, row, H, h, d, A.sm_v);
      for (int j = 0; j < gs; ++j) acc[j] = fmaf(p_s[j * kMaxChunk + t], vv, acc[j]);
    }
    for (int j = 0; j < gs; ++j) part_o[(item * gs + j) * D + d] = acc[j];
  }
}

// out[b, hq, d] = sum_c exp(m_c - M) o_c / sum_c exp(m_c - M) l_c over the splits of (b, hq / gs).
// grid (D / 32, Hq, batch), WAVES = min(4, ceil(n_chunks / 64)) wavefronts per block: lane l of wavefront w holds
// dims 4 (l & 7) .. + 3 of the block's 32 and takes splits c = 8 WAVES k + WAVES (l >> 3) + w, k < KL, of each round
// of 8 WAVES KL (KL 16-byte loads of o and KL 8-byte loads of (m, l) per lane, all in flight at once: one round for
// up to 256 splits; KL = 8, or ceil(n_chunks / 8) in a one-wavefront block, so that few lanes repeat slot 0).  A round's maximum over the wavefront's splits comes first (the partials' m
// is per split and q head, the same for every dim), then every split's weight e^(m_c - M_w) independently of the
// others; a later round rescales the running sums once.  The sums of the 32 lanes of a dim quad reduce without LDS
// traffic (a DPP row rotation by 8 lanes, then the permlane16 / permlane32 swaps), and the wavefronts merge with
// e^(M_w - M) in LDS.  Slots beyond the splits in use may hold anything, NaN included: they are selected out, never
// scaled by zero.  An empty context gives 0/0 = NaN (gemv/test_kv_paged_prefix.py:524-526).
constexpr int kCombDims = 32;     // dims per block

typedef float f4c __attribute__((ext_vector_type(4)));

// The value of lane l ^ 8 (DPP rotation by 8 within each row of 16 lanes) and the sum / max with the lane 16 and 32
// apart (gfx950 permlane swaps: with both operands the same register, the two results are the value of the lane
// itself and of its partner).  All 64 lanes must be active.
KVT_DEV float lane_x8(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}
KVT_DEV float sum_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
KVT_DEV float sum_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
KVT_DEV float max_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
KVT_DEV float max_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int WAVES, int KL>
__global__ void __launch_bounds__(64 * WAVES) decode_combine_kernel(
    const float* part_o, const float* part_ml, int H, int gs, int D, int n_chunks, int64_t chunk,
    const int32_t* seq_lens, const int32_t* split_counts, float* out_f32, uint16_t* out_bf16,
    int64_t out_stride_b) {
  constexpr float kL2e = 1.4426950408889634f;   // partial maxima are in natural-log units
  constexpr int kCombRound = 8 * WAVES * KL;    // splits per round (KL loads of o and (m, l) per lane)
  __shared__ f4c nred[WAVES][8];
  __shared__ float dred[WAVES][8];
  __shared__ float mred[WAVES];
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int h = hq / gs, j = hq - h * gs;
  const int lane = threadIdx.x & 63, w = WAVES == 1 ? 0 : (int)(threadIdx.x >> 6);
  const int dq = lane & 7, sub = lane >> 3;
  const int d0 = blockIdx.x * kCombDims + 4 * dq;
  const int sl = WAVES * sub + w;   // the lane's split in each group of 8 WAVES
  const int64_t base = ((int64_t)b * H + h) * n_chunks;
  float m_run = -INFINITY, den = 0.0f;   // m_run: the wavefront's running maximum (uniform)
  f4c num = {0.f, 0.f, 0.f, 0.f};
  // the loads of a round index the n_chunks slots only: the first round's go out before the sequence length (which
  // bounds the splits in use) has arrived
  int used = 0;
  for (int r0 = 0; r0 < n_chunks; r0 += kCombRound) {
    f4c ov[KL];
    float2 ml[KL];
#pragma unroll
    for (int k = 0; k < KL; ++k) {
      const int c = r0 + 8 * WAVES * k + sl;
      const int64_t it = (base + (c < n_chunks ? c : 0)) * gs + j;
      ov[k] = *reinterpret_cast<const f4c*>(&part_o[it * D + d0]);
      ml[k] = *reinterpret_cast<const float2*>(&part_ml[it * 2]);
    }
    if (r0 == 0) {
      // chunk > 0: split c covers positions [c chunk, (c + 1) chunk); chunk 0: every split holds a partial
      // split_counts (chunk 0): sequence b uses the first split_counts[b] slots
      const int64_t L = seq_lens[b];
      used = chunk > 0 ? (int)min((int64_t)n_chunks, (L + chunk - 1) / chunk)
                       : (split_counts != nullptr ? split_counts[b] : n_chunks);
    }
    float mk[KL];
#pragma unroll
    for (int k = 0; k < KL; ++k) mk[k] = (r0 + 8 * WAVES * k + sl < used) ? ml[k].x : -INFINITY;
    float mr = mk[0];
#pragma unroll
    for (int k = 1; k < KL; ++k) mr = fmaxf(mr, mk[k]);
    mr = fmaxf(mr, lane_x8(mr));
    mr = max_x32(max_x16(mr));
    const float mn = fmaxf(m_run, mr);
    if (mn != -INFINITY) {   // (uniform)
      if (m_run != mn) {
        const float a = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_run - mn) * kL2e);
        num *= a;
        den *= a;
      }
#pragma unroll
      for (int k = 0; k < KL; ++k) {
        const bool ok = mk[k] != -INFINITY;
        const float wk = ok ? __builtin_amdgcn_exp2f((mk[k] - mn) * kL2e) : 0.f;
        num += (ok ? ov[k] : f4c{0.f, 0.f, 0.f, 0.f}) * wk;
        den += (ok ? ml[k].y : 0.f) * wk;
      }
      m_run = mn;
    }
    if (r0 + kCombRound >= used) break;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) num[i] = sum_x32(sum_x16(num[i] + lane_x8(num[i])));
  den = sum_x32(sum_x16(den + lane_x8(den)));
  if constexpr (WAVES == 1) {
    if (sub == 0) {
      const int64_t oi = b * out_stride_b + (int64_t)hq * D + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float o = num[i] / den;
        if (out_f32) out_f32[oi + i] = o;
        if (out_bf16) out_bf16[oi + i] = bf16_rne(o);
      }
    }
    return;
  }
  if (sub == 0) {
    nred[w][dq] = num;
    dred[w][dq] = den;
  }
  if (lane == 0) mred[w] = m_run;
  __syncthreads();
  if (w == 0 && sub == 0) {
    float M = mred[0];
#pragma unroll
    for (int v = 1; v < WAVES; ++v) M = fmaxf(M, mred[v]);
    f4c n4 = {0.f, 0.f, 0.f, 0.f};
    float d4 = 0.f;
#pragma unroll
    for (int v = 0; v < WAVES; ++v) {
      const float a = mred[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((mred[v] - M) * kL2e);
      n4 += nred[v][dq] * a;
      d4 += dred[v][dq] * a;
    }
    const int64_t oi = b * out_stride_b + (int64_t)hq * D + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float o = n4[i] / d4;
      if (out_f32) out_f32[oi + i] = o;
      if (out_bf16) out_bf16[oi + i] = bf16_rne(o);
    }
  }
}

}  // namespace

extern "C" {

// mode 0: position rings + page tables; mode 1: slot rings + owner table (req_to_token).
int kvt_decode_ref(int mode, const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int H, int Hq, int D,
                   int group8, const void* k4, const void* v4, const void* ks4, const void* vs4, const void* rk,
                   const void* rv, const void* rks, const void* rvs, const void* sm_k, const void* sm_v,
                   const void* ring_base, const void* ring_len, const void* ring_start, const void* page_table,
                   int64_t pt_stride, const void* req_to_token, int64_t req_stride, const void* req_indices,
                   const void* owner, int64_t ring_mask, float scale, int chunk, int n_chunks, void* part_o,
                   void* part_ml, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0) return KVT_EINVAL;
  const int gs = Hq / H;
  if (gs > kMaxGroup || chunk <= 0 || chunk > kMaxChunk || n_chunks <= 0) return KVT_EINVAL;
  TierArgs A{(const uint8_t*)k4,      (const uint8_t*)v4,         (const uint16_t*)ks4,       (const uint16_t*)vs4,
             (const int8_t*)rk,       (const int8_t*)rv,          (const uint16_t*)rks,       (const uint16_t*)rvs,
             (const uint16_t*)sm_k,   (const uint16_t*)sm_v,      (const int64_t*)ring_base,  (const int32_t*)ring_len,
             (const int64_t*)ring_start, (const int32_t*)page_table, pt_stride,               (const int32_t*)req_to_token,
             req_stride,              (const int64_t*)req_indices, (const int32_t*)owner,     ring_mask};
  const dim3 grid((unsigned)n_chunks, (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
#define KVT_DR(MODE_, D_, G_)                                                                                     \
  hipLaunchKernelGGL((decode_ref_kernel<MODE_, D_, G_>), grid, dim3(kThreads), 0, st, A, (const uint16_t*)q,      \
                     q_stride_b, (const int32_t*)seq_lens, H, gs, chunk, n_chunks, scale, (float*)part_o,        \
                     (float*)part_ml)
  if (D != 256) return KVT_EINVAL;
  if (mode == 0 && group8 == 64) {
    KVT_DR(0, 256, 64);
  } else if (mode == 0 && group8 == 256) {
    KVT_DR(0, 256, 256);
  } else if (mode == 1 && group8 == 64) {
    KVT_DR(1, 256, 64);
  } else if (mode == 1 && group8 == 256) {
    KVT_DR(1, 256, 256);
  } else {
    return KVT_EINVAL;
  }
#undef KVT_DR
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

int kvt_decode_combine(const void* part_o, const void* part_ml, int batch, int H, int Hq, int D, int n_chunks,
                       int64_t chunk, const void* seq_lens, const void* split_counts, void* out_f32, void* out_bf16,
                       int64_t out_stride_b, void* stream) {
  if (batch <= 0 || H <= 0 || Hq % H != 0 || n_chunks <= 0 || chunk < 0 || D % kCombDims != 0) return KVT_EINVAL;
  const dim3 grid((unsigned)(D / kCombDims), (unsigned)Hq, (unsigned)batch);
#define KVT_COMB(W_, KL_)                                                                                          \
  hipLaunchKernelGGL((decode_combine_kernel<W_, KL_>), grid, dim3(64 * W_), 0, (hipStream_t)stream,                \
                     (const float*)part_o, (const float*)part_ml, H, Hq / H, D, n_chunks, chunk,                   \
                     (const int32_t*)seq_lens, (const int32_t*)split_counts, (float*)out_f32, (uint16_t*)out_bf16, \
                     out_stride_b)
  // one round of ceil(n_chunks / 64) wavefronts (4 from 193 splits on, in rounds of 256): no lane issues loads
  // that only repeat slot 0, and with one wavefront there is no LDS merge; a one-wavefront block issues
  // ceil(n_chunks / 8) loads per lane (33 splits: 5)
  if (n_chunks <= 64) {
    switch ((n_chunks + 7) / 8) {
      case 1: KVT_COMB(1, 1); break;
      case 2: KVT_COMB(1, 2); break;
      case 3: KVT_COMB(1, 3); break;
      case 4: KVT_COMB(1, 4); break;
      case 5: KVT_COMB(1, 5); break;
      case 6: KVT_COMB(1, 6); break;
      case 7: KVT_COMB(1, 7); break;
      default: KVT_COMB(1, 8); break;
    }
  } else if (n_chunks <= 128) {
    KVT_COMB(2, 8);
  } else if (n_chunks <= 192) {
    KVT_COMB(3, 8);
  } else {
    KVT_COMB(4, 8);
  }
#undef KVT_COMB
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
