// Gather-dequant kernels of the tiered KV cache (drop-in for the reference's compact and prefix gathers).
//
// A wavefront writes 2 (top-k) or 4 (prefix) output rows (all KV heads, K and V).  Lane l owns unit u = l (+ 64, ... while u < H D / 8):
// KV head u / (D / 8), channels 8 (u % (D / 8)) .. + 7, whose smoothing constants it loads once.  Per row it reads
// 4 bytes of INT4 codes (or 8 bytes of INT8 codes) and one fp16 group scale for K and for V, and stores 16 bytes of
// bf16 for each: a row of one tensor is one contiguous read and one contiguous 1 KiB store across the wavefront.
// All rows' loads go out before the first conversion.  The row -> slot chain (request, req_to_token, owner) is
// wave-uniform scalar work.  The tier is decided per row on the device: hot = owner[slot & mask] == slot
// (patches/kv_tiers.py:500-504).  Only valid rows are written (store mask = valid, patches/kv_tiers.py:476-480: the
// trtllm strided scratch relies on it).  Values: bf16(code * s * sm) in fp32 (patches/kv_tiers.py:519-525), rounded
// to nearest even by v_cvt_pk_bf16_f32.
//
//   kvt_compact_gather  top-k selection -> packed rows (patches/kv_tiers.py:446-538, :688-737;
//                       patches/kv_int4.py:396-460; patches/kv_int8.py:365-420)
//   kvt_prefix_gather   rows [0, seq_len) -> packed at cu_k[b] (patches/kv_tiers.py:541-683;
//                       patches/kv_int4.py:463-557; patches/kv_int8.py:423-504)
//   kvt_sparse_cu_seqlens  valid top-k counts and their prefix sum, the offsets kvt_compact_gather packs at (the
//                       upstream qwen_sparse_fa2_cu_seqlens_triton the reference calls first, gemv/test_kv_tiers.py:297-301)

#include "kvt_common.h"

using namespace kvt;

namespace {

// pool kind: 0 = INT8 pool (codes [rows, H, D], scales [rows, H, D / G8]); 1 = INT4 pool;
// 2 = tiered (INT4 pool + INT8 ring + owner).
struct Pools {
  const uint8_t* k;   // INT4 codes, or INT8 codes for kind 0
  const uint8_t* v;
  const uint16_t* ks;
  const uint16_t* vs;
  const int8_t* rk;   // INT8 ring (kind 2)
  const int8_t* rv;
  const uint16_t* rks;
  const uint16_t* rvs;
  const int32_t* owner;
  const uint16_t* sm_k;  // [H, D] fp16, multiplied after the scale (identity in the served setup)
  const uint16_t* sm_v;
  int64_t ring_mask;
};

// rows per wavefront: 2 for the top-k gather (random rows: more wavefronts in flight), 4 for the whole-prefix
// gather (streaming) -- 174.7 against 192 us and 1.55 against 1.69 ms per 12-layer step, the better of 2, 4 and 8
constexpr int kCompactRows = 2;
constexpr int kPrefixRows = 4;
constexpr int kWaves = 4;    // wavefronts per block

// bf16 pair (round to nearest even, one v_cvt_pk_bf16_f32): lo in bits 0-15.
KVT_DEV uint32_t bf16x2(float lo, float hi) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){lo, hi}, bf2v));
}

// The raw codes and scale of one unit of one row: INT4 (w.x, 8 nibbles) or INT8 (w.x, w.y, 8 bytes).
struct Raw {
  uint2 w;
  uint16_t s;
};

template <int D, int G8>
KVT_DEV Raw load_int8(const int8_t* codes, const uint16_t* scales, int64_t row, int H, int h, int cg) {
  constexpr int NG8 = D / G8;
  Raw r;
  r.w = *reinterpret_cast<const uint2*>(codes + (row * H + h) * D + 8 * cg);
  r.s = scales[(row * H + h) * NG8 + (8 * cg) / G8];
  return r;
}

template <int D>
KVT_DEV Raw load_int4(const uint8_t* codes, const uint16_t* scales, int64_t row, int H, int h, int cg) {
  Raw r;
  r.w.x = *reinterpret_cast<const uint32_t*>(codes + (row * H + h) * (D / 2) + 4 * cg);
  r.w.y = 0;
  r.s = scales[(row * H + h) * (D / kG4) + cg / 4];
  return r;
}

KVT_DEV uint4 dequant8(const Raw& r, const float m[8]) {   // q * s * sm (patches/kv_tiers.py:525)
  const float s = f16_bits_to_f32(r.s);
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)(int8_t)((i < 4 ? r.w.x : r.w.y) >> (8 * (i & 3))) * s * m[i];
  return make_uint4(bf16x2(x[0], x[1]), bf16x2(x[2], x[3]), bf16x2(x[4], x[5]), bf16x2(x[6], x[7]));
}

KVT_DEV uint4 dequant4(const Raw& r, const float m[8]) {   // ((b & 15) - 8) * s * sm (patches/kv_tiers.py:519-523)
  const float s = f16_bits_to_f32(r.s);
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)((int)((r.w.x >> (4 * i)) & 15u) - 8) * s * m[i];
  return make_uint4(bf16x2(x[0], x[1]), bf16x2(x[2], x[3]), bf16x2(x[4], x[5]), bf16x2(x[6], x[7]));
}

// ROWS rows of one wavefront: slot[j] (wave-uniform; < 0 = row not written) -> output row dst[j].
template <int KIND, int D, int G8, int ROWS>
KVT_DEV void gather_rows(const Pools& P, const int64_t slot[ROWS], const int64_t dst[ROWS], int H, int lane,
                         uint16_t* out_k, uint16_t* out_v) {
  bool hot[ROWS];
  int64_t ring[ROWS];
#pragma unroll
  for (int j = 0; j < ROWS; ++j) {
    hot[j] = KIND == 0;
    ring[j] = 0;
    if constexpr (KIND == 2) {
      if (slot[j] >= 0) {
        ring[j] = slot[j] & P.ring_mask;
        hot[j] = (int64_t)P.owner[ring[j]] == slot[j];
      }
    }
  }
  constexpr int CG = D / 8;
  const int U = H * CG;
  for (int u = lane; u < U; u += 64) {
    const int h = u / CG, cg = u - h * CG;
    float mk[8], mv[8];   // once per unit (element loads: the constants need only 2-byte alignment)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mk[i] = f16_bits_to_f32(P.sm_k[h * D + 8 * cg + i]);
      mv[i] = f16_bits_to_f32(P.sm_v[h * D + 8 * cg + i]);
    }
    Raw rk[ROWS], rv[ROWS];
#pragma unroll
    for (int j = 0; j < ROWS; ++j) {
      if (slot[j] < 0) continue;
      if constexpr (KIND == 0) {
        rk[j] = load_int8<D, G8>(reinterpret_cast<const int8_t*>(P.k), P.ks, slot[j], H, h, cg);
        rv[j] = load_int8<D, G8>(reinterpret_cast<const int8_t*>(P.v), P.vs, slot[j], H, h, cg);
      } else {
        if (hot[j]) {
          rk[j] = load_int8<D, G8>(P.rk, P.rks, ring[j], H, h, cg);
          rv[j] = load_int8<D, G8>(P.rv, P.rvs, ring[j], H, h, cg);
        } else {
          rk[j] = load_int4<D>(P.k, P.ks, slot[j], H, h, cg);
          rv[j] = load_int4<D>(P.v, P.vs, slot[j], H, h, cg);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < ROWS; ++j) {
      if (slot[j] < 0) continue;
      const uint4 ok = hot[j] ? dequant8(rk[j], mk) : dequant4(rk[j], mk);
      const uint4 ov = hot[j] ? dequant8(rv[j], mv) : dequant4(rv[j], mv);
      *reinterpret_cast<uint4*>(out_k + (dst[j] * H + h) * D + 8 * cg) = ok;
      *reinterpret_cast<uint4*>(out_v + (dst[j] * H + h) * D + 8 * cg) = ov;
    }
  }
}

KVT_DEV int64_t ld_idx(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

KVT_DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// grid.x = column blocks of kWaves * kCompactRows, grid.y = batch
template <int KIND, int D, int G8>
__global__ void __launch_bounds__(64 * kWaves) compact_kernel(Pools P, const int32_t* req_to_token, int64_t req_stride,
                                                              const void* req_indices, int req64,
                                                              const int32_t* indices, int64_t idx_stride,
                                                              const int32_t* seq_lens, const void* cu_k, int cu64,
                                                              int topk, int H, uint16_t* out_k, uint16_t* out_v) {
  const int lane = threadIdx.x & 63;
  constexpr int kRows = kCompactRows;
  const int64_t col0 = ((int64_t)blockIdx.x * kWaves + wave_id()) * kRows;
  const int b = blockIdx.y;
  if (col0 >= topk) return;
  const int64_t length = seq_lens[b];
  const int64_t start = ld_idx(cu_k, cu64, b);
  const int64_t vcount = ld_idx(cu_k, cu64, b + 1) - start;
  const int64_t req = ld_idx(req_indices, req64, b);
  int64_t slot[kRows], dst[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int64_t col = col0 + j;
    slot[j] = -1;
    dst[j] = start + col;
    if (col < topk && col < vcount) {
      const int64_t pos = indices[(int64_t)b * idx_stride + col];
      if (pos >= 0 && pos < length) slot[j] = req_to_token[req * req_stride + pos];   // store mask = valid
    }
  }
  gather_rows<KIND, D, G8, kRows>(P, slot, dst, H, lane, out_k, out_v);
}

// grid.x = row blocks of kWaves * kPrefixRows, grid.y = batch
template <int KIND, int D, int G8>
__global__ void __launch_bounds__(64 * kWaves) prefix_kernel(Pools P, const int32_t* req_to_token, int64_t req_stride,
                                                             const void* req_indices, int req64,
                                                             const int32_t* seq_lens, const void* cu_k, int cu64,
                                                             int H, uint16_t* out_k, uint16_t* out_v) {
  const int lane = threadIdx.x & 63;
  constexpr int kRows = kPrefixRows;
  const int64_t t0 = ((int64_t)blockIdx.x * kWaves + wave_id()) * kRows;
  const int b = blockIdx.y;
  const int64_t length = seq_lens[b];
  if (t0 >= length) return;
  const int64_t req = ld_idx(req_indices, req64, b);
  const int64_t start = ld_idx(cu_k, cu64, b);
  int64_t slot[kRows], dst[kRows];
#pragma unroll
  for (int j = 0; j < kRows; ++j) {
    const int64_t t = t0 + j;
    slot[j] = t < length ? (int64_t)req_to_token[req * req_stride + t] : -1;
    dst[j] = start + t;
  }
  gather_rows<KIND, D, G8, kRows>(P, slot, dst, H, lane, out_k, out_v);
}

// Vector access widths: INT4 codes 4 bytes, INT8 codes 8 bytes, bf16 rows 16 bytes per lane.
bool aligned_args(int kind, const void* k, const void* v, const void* rk, const void* rv, const void* ok,
                  const void* ov) {
  const auto al = [](const void* p, uintptr_t a) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0; };
  const uintptr_t ca = kind == 0 ? 8 : 4;
  return al(k, ca) && al(v, ca) && al(rk, 8) && al(rv, 8) && al(ok, 16) && al(ov, 16);
}


// counts[b] = #{c < topk : 0 <= indices[b * idx_stride + c] < seq_lens[b]}; cu_k[0] = 0, cu_k[b + 1] = counts[0] + ..
// + counts[b].  One block of kCuThreads: rows go to the wavefronts in turn (64 columns per coalesced load, a wavefront
// sum per row), then the block scans a chunk of kCuThreads counts in LDS (Hillis-Steele, double-buffered) and adds
// the running total of the earlier chunks.
constexpr int kCuThreads = 1024;

__global__ void __launch_bounds__(kCuThreads) cu_seqlens_kernel(const int32_t* seq_lens, const int32_t* indices,
                                                                 int64_t idx_stride, int32_t* counts, void* cu_k,
                                                                 int cu_is_int64, int batch, int topk) {
  __shared__ int32_t buf[2][kCuThreads];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  constexpr int kW = kCuThreads / 64;
  auto put = [&](int64_t i, int64_t v) {
    if (cu_is_int64) ((int64_t*)cu_k)[i] = v;
    else ((int32_t*)cu_k)[i] = (int32_t)v;
  };
  if (t == 0) put(0, 0);
  int64_t carry = 0;
  for (int r0 = 0; r0 < batch; r0 += kCuThreads) {
    const int nrows = min(kCuThreads, batch - r0);
    for (int r = wave; r < nrows; r += kW) {
      const int b = r0 + r;
      const int64_t L = seq_lens[b];
      const int32_t* row = indices + (int64_t)b * idx_stride;
      int n = 0;
      for (int c0 = 0; c0 < topk; c0 += 64) {
        const int c = c0 + lane;
        if (c < topk) {
          const int64_t p = row[c];
          n += (p >= 0 && p < L) ? 1 : 0;
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) n += __shfl_xor(n, o, 64);
      if (lane == 0) {
        buf[0][r] = n;
        counts[b] = n;
      }
    }
    __syncthreads();
    int cur = 0;
    if (t >= nrows) buf[0][t] = 0;
    __syncthreads();
    for (int d = 1; d < kCuThreads; d <<= 1) {
      const int v = buf[cur][t] + (t >= d ? buf[cur][t - d] : 0);
      buf[cur ^ 1][t] = v;
      cur ^= 1;
      __syncthreads();
    }
    if (t < nrows) put((int64_t)r0 + t + 1, carry + buf[cur][t]);
    carry += buf[cur][kCuThreads - 1];
    __syncthreads();   // the next chunk overwrites buf
  }
}

}  // namespace

#define KVT_GATHER_DISPATCH(LAUNCH)                        \
  if (D == 256 && group8 == 64) {                          \
    LAUNCH(256, 64);                                       \
  } else if (D == 256 && group8 == 256) {                  \
    LAUNCH(256, 256);                                      \
  } else if (D == 128 && group8 == 64) {                   \
    LAUNCH(128, 64);                                       \
  } else if (D == 128 && group8 == 128) {                  \
    LAUNCH(128, 128);                                      \
  } else {                                                 \
    return KVT_EINVAL;                                     \
  }

extern "C" {

int kvt_sparse_cu_seqlens(const void* seq_lens, const void* indices, int64_t idx_stride, void* counts, void* cu_k,
                          int cu_is_int64, int batch, int topk, void* stream) {
  if (batch < 0 || topk < 0 || idx_stride < 0) return KVT_EINVAL;
  hipLaunchKernelGGL(cu_seqlens_kernel, dim3(1), dim3(kCuThreads), 0, (hipStream_t)stream, (const int32_t*)seq_lens,
                     (const int32_t*)indices, idx_stride, (int32_t*)counts, cu_k, cu_is_int64, batch, topk);
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

// kind: 0 = INT8 pool, 1 = INT4 pool, 2 = tiered.  All pointers are device pointers of torch-owned tensors.
int kvt_compact_gather(int kind, const void* k, const void* v, const void* k_scale, const void* v_scale,
                       const void* ring_k, const void* ring_v, const void* ring_ks, const void* ring_vs,
                       const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                       const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                       const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                       int cu_is_int64, int batch, int topk, int H, int D, int group8, void* out_k, void* out_v,
                       void* stream) {
  if (batch < 0 || topk < 0 || H <= 0) return KVT_EINVAL;
  if (!aligned_args(kind, k, v, ring_k, ring_v, out_k, out_v)) return KVT_EINVAL;
  if (batch == 0 || topk == 0) return KVT_OK;
  Pools P{(const uint8_t*)k,        (const uint8_t*)v,       (const uint16_t*)k_scale, (const uint16_t*)v_scale,
          (const int8_t*)ring_k,    (const int8_t*)ring_v,   (const uint16_t*)ring_ks, (const uint16_t*)ring_vs,
          (const int32_t*)owner,    (const uint16_t*)sm_k,   (const uint16_t*)sm_v,    ring_mask};
  constexpr int kPerBlock = kWaves * kCompactRows;
  const dim3 grid((unsigned)((topk + kPerBlock - 1) / kPerBlock), (unsigned)batch);
  hipStream_t st = (hipStream_t)stream;
#define KVT_CG(KIND_, D_, G_)                                                                                   \
  hipLaunchKernelGGL((compact_kernel<KIND_, D_, G_>), grid, dim3(64 * kWaves), 0, st, P, (const int32_t*)req_to_token, \
                     req_stride, req_indices, req_is_int64, (const int32_t*)indices, idx_stride,               \
                     (const int32_t*)seq_lens, cu_k, cu_is_int64, topk, H, (uint16_t*)out_k, (uint16_t*)out_v)
#define KVT_CG0(D_, G_) KVT_CG(0, D_, G_)
#define KVT_CG1(D_, G_) KVT_CG(1, D_, G_)
#define KVT_CG2(D_, G_) KVT_CG(2, D_, G_)
  if (kind == 0) {
    KVT_GATHER_DISPATCH(KVT_CG0)
  } else if (kind == 1) {
    KVT_GATHER_DISPATCH(KVT_CG1)
  } else if (kind == 2) {
    KVT_GATHER_DISPATCH(KVT_CG2)
  } else {
    return KVT_EINVAL;
  }
#undef KVT_CG0
#undef KVT_CG1
#undef KVT_CG2
#undef KVT_CG
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

int kvt_prefix_gather(int kind, const void* k, const void* v, const void* k_scale, const void* v_scale,
                      const void* ring_k, const void* ring_v, const void* ring_ks, const void* ring_vs,
                      const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* seq_lens, const void* cu_k, int cu_is_int64, int batch, int64_t max_len, int H,
                      int D, int group8, void* out_k, void* out_v, void* stream) {
  if (batch < 0 || max_len < 0 || H <= 0) return KVT_EINVAL;
  if (!aligned_args(kind, k, v, ring_k, ring_v, out_k, out_v)) return KVT_EINVAL;
  if (batch == 0 || max_len == 0) return KVT_OK;
  Pools P{(const uint8_t*)k,        (const uint8_t*)v,       (const uint16_t*)k_scale, (const uint16_t*)v_scale,
          (const int8_t*)ring_k,    (const int8_t*)ring_v,   (const uint16_t*)ring_ks, (const uint16_t*)ring_vs,
          (const int32_t*)owner,    (const uint16_t*)sm_k,   (const uint16_t*)sm_v,    ring_mask};
  constexpr int kPerBlock = kWaves * kPrefixRows;
  if ((max_len + kPerBlock - 1) / kPerBlock > 0x7fffffffLL) return KVT_ERANGE;
  const dim3 grid((unsigned)((max_len + kPerBlock - 1) / kPerBlock), (unsigned)batch);
  hipStream_t st = (hipStream_t)stream;
#define KVT_PG(KIND_, D_, G_)                                                                                  \
  hipLaunchKernelGGL((prefix_kernel<KIND_, D_, G_>), grid, dim3(64 * kWaves), 0, st, P, (const int32_t*)req_to_token, \
                     req_stride, req_indices, req_is_int64, (const int32_t*)seq_lens, cu_k, cu_is_int64, H,   \
                     (uint16_t*)out_k, (uint16_t*)out_v)
#define KVT_PG0(D_, G_) KVT_PG(0, D_, G_)
#define KVT_PG1(D_, G_) KVT_PG(1, D_, G_)
#define KVT_PG2(D_, G_) KVT_PG(2, D_, G_)
  if (kind == 0) {
    KVT_GATHER_DISPATCH(KVT_PG0)
  } else if (kind == 1) {
    KVT_GATHER_DISPATCH(KVT_PG1)
  } else if (kind == 2) {
    KVT_GATHER_DISPATCH(KVT_PG2)
  } else {
    return KVT_EINVAL;
  }
#undef KVT_PG0
#undef KVT_PG1
#undef KVT_PG2
#undef KVT_PG
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
