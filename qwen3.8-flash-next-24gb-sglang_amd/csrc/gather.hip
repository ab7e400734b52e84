// Gather-dequant kernels of the tiered KV cache (drop-in for the reference's compact and prefix gathers).
//
// One wavefront per (output row, KV head); lane l produces channels 4l..4l+3 as bf16 (one 8-byte store), reading
// 2 bytes of INT4 codes or 4 bytes of INT8 codes plus its group's fp16 scale.  The tier is decided per row on the
// device: hot = owner[slot & mask] == slot (patches/kv_tiers.py:500-504).  Only valid rows are written (store mask
// = valid, patches/kv_tiers.py:476-480: the trtllm strided scratch relies on it).
//
//   kvt_compact_gather  top-k selection -> packed rows (patches/kv_tiers.py:446-538, :688-737;
//                       patches/kv_int4.py:396-460; patches/kv_int8.py:365-420)
//   kvt_prefix_gather   rows [0, seq_len) -> packed at cu_k[b] (patches/kv_tiers.py:541-683;
//                       patches/kv_int4.py:463-557; patches/kv_int8.py:423-504)

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

template <int D, int G8>
KVT_DEV void dequant_int8_lane(const int8_t* codes, const uint16_t* scales, int64_t row, int H, int h, int lane,
                               const uint16_t* sm, uint16_t out[4]) {
  constexpr int NG8 = D / G8;
  const uint32_t c = reinterpret_cast<const uint32_t*>(codes + (row * H + h) * D)[lane];
  const float s = f16_bits_to_f32(scales[(row * H + h) * NG8 + (4 * lane) / G8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float m = f16_bits_to_f32(sm[h * D + 4 * lane + i]);
    out[i] = bf16_rne((float)(int8_t)(c >> (8 * i)) * s * m);  // q * s * sm (patches/kv_tiers.py:525)
  }
}

template <int D>
KVT_DEV void dequant_int4_lane(const uint8_t* codes, const uint16_t* scales, int64_t row, int H, int h, int lane,
                               const uint16_t* sm, uint16_t out[4]) {
  constexpr int NG4 = D / kG4;
  const uint32_t b = reinterpret_cast<const uint16_t*>(codes + (row * H + h) * (D / 2))[lane];
  const float s = f16_bits_to_f32(scales[(row * H + h) * NG4 + lane / 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float m = f16_bits_to_f32(sm[h * D + 4 * lane + i]);
    const int n = (int)((b >> (4 * i)) & 15u) - 8;
    out[i] = bf16_rne((float)n * s * m);  // ((b & 15) - 8) * s * sm (patches/kv_tiers.py:519-523)
  }
}

template <int KIND, int D, int G8>
KVT_DEV void gather_row(const Pools& P, int64_t slot, int H, int h, int lane, uint16_t* out_k, uint16_t* out_v,
                        int64_t dst) {
  uint16_t ok[4], ov[4];
  if constexpr (KIND == 0) {
    dequant_int8_lane<D, G8>(reinterpret_cast<const int8_t*>(P.k), P.ks, slot, H, h, lane, P.sm_k, ok);
    dequant_int8_lane<D, G8>(reinterpret_cast<const int8_t*>(P.v), P.vs, slot, H, h, lane, P.sm_v, ov);
  } else {
    bool hot = false;
    int64_t r = 0;
    if constexpr (KIND == 2) {
      r = slot & P.ring_mask;
      hot = (int64_t)P.owner[r] == slot;
    }
    if (hot) {
      dequant_int8_lane<D, G8>(P.rk, P.rks, r, H, h, lane, P.sm_k, ok);
      dequant_int8_lane<D, G8>(P.rv, P.rvs, r, H, h, lane, P.sm_v, ov);
    } else {
      dequant_int4_lane<D>(P.k, P.ks, slot, H, h, lane, P.sm_k, ok);
      dequant_int4_lane<D>(P.v, P.vs, slot, H, h, lane, P.sm_v, ov);
    }
  }
  const uint2 wk = make_uint2((uint32_t)ok[0] | ((uint32_t)ok[1] << 16), (uint32_t)ok[2] | ((uint32_t)ok[3] << 16));
  const uint2 wv = make_uint2((uint32_t)ov[0] | ((uint32_t)ov[1] << 16), (uint32_t)ov[2] | ((uint32_t)ov[3] << 16));
  reinterpret_cast<uint2*>(out_k + (dst * H + h) * D)[lane] = wk;
  reinterpret_cast<uint2*>(out_v + (dst * H + h) * D)[lane] = wv;
}

KVT_DEV int64_t ld_idx(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

// grid.x = column blocks of 4, grid.y = batch * H
template <int KIND, int D, int G8>
__global__ void __launch_bounds__(256) compact_kernel(Pools P, const int32_t* req_to_token, int64_t req_stride,
                                                      const void* req_indices, int req64, const int32_t* indices,
                                                      int64_t idx_stride, const int32_t* seq_lens, const void* cu_k,
                                                      int cu64, int topk, int H, uint16_t* out_k, uint16_t* out_v) {
  const int lane = threadIdx.x & 63;
  const int col = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y / H;
  const int h = blockIdx.y - b * H;
  if (col >= topk || lane >= D / 4) return;
  const int64_t length = seq_lens[b];
  const int64_t start = ld_idx(cu_k, cu64, b);
  const int64_t vcount = ld_idx(cu_k, cu64, b + 1) - start;
  const int64_t pos = indices[(int64_t)b * idx_stride + col];
  if (!(col < vcount && pos >= 0 && pos < length)) return;  // store mask = valid
  const int64_t req = ld_idx(req_indices, req64, b);
  const int64_t slot = req_to_token[req * req_stride + pos];
  gather_row<KIND, D, G8>(P, slot, H, h, lane, out_k, out_v, start + col);
}

// grid.x = row blocks of 4, grid.y = batch * H
template <int KIND, int D, int G8>
__global__ void __launch_bounds__(256) prefix_kernel(Pools P, const int32_t* req_to_token, int64_t req_stride,
                                                     const void* req_indices, int req64, const int32_t* seq_lens,
                                                     const void* cu_k, int cu64, int H, uint16_t* out_k,
                                                     uint16_t* out_v) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int b = blockIdx.y / H;
  const int h = blockIdx.y - b * H;
  if (lane >= D / 4) return;
  if (t >= (int64_t)seq_lens[b]) return;
  const int64_t req = ld_idx(req_indices, req64, b);
  const int64_t slot = req_to_token[req * req_stride + t];
  gather_row<KIND, D, G8>(P, slot, H, h, lane, out_k, out_v, ld_idx(cu_k, cu64, b) + t);
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

// kind: 0 = INT8 pool, 1 = INT4 pool, 2 = tiered.  All pointers are device pointers of torch-owned tensors.
int kvt_compact_gather(int kind, const void* k, const void* v, const void* k_scale, const void* v_scale,
                       const void* ring_k, const void* ring_v, const void* ring_ks, const void* ring_vs,
                       const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                       const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                       const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                       int cu_is_int64, int batch, int topk, int H, int D, int group8, void* out_k, void* out_v,
                       void* stream) {
  if (batch < 0 || topk < 0 || H <= 0) return KVT_EINVAL;
  if (batch == 0 || topk == 0) return KVT_OK;
  Pools P{(const uint8_t*)k,        (const uint8_t*)v,       (const uint16_t*)k_scale, (const uint16_t*)v_scale,
          (const int8_t*)ring_k,    (const int8_t*)ring_v,   (const uint16_t*)ring_ks, (const uint16_t*)ring_vs,
          (const int32_t*)owner,    (const uint16_t*)sm_k,   (const uint16_t*)sm_v,    ring_mask};
  const dim3 grid((unsigned)((topk + 3) / 4), (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
#define KVT_CG(KIND_, D_, G_)                                                                                   \
  hipLaunchKernelGGL((compact_kernel<KIND_, D_, G_>), grid, dim3(256), 0, st, P, (const int32_t*)req_to_token, \
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
  if (batch == 0 || max_len == 0) return KVT_OK;
  Pools P{(const uint8_t*)k,        (const uint8_t*)v,       (const uint16_t*)k_scale, (const uint16_t*)v_scale,
          (const int8_t*)ring_k,    (const int8_t*)ring_v,   (const uint16_t*)ring_ks, (const uint16_t*)ring_vs,
          (const int32_t*)owner,    (const uint16_t*)sm_k,   (const uint16_t*)sm_v,    ring_mask};
  const dim3 grid((unsigned)((max_len + 3) / 4), (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
#define KVT_PG(KIND_, D_, G_)                                                                                  \
  hipLaunchKernelGGL((prefix_kernel<KIND_, D_, G_>), grid, dim3(256), 0, st, P, (const int32_t*)req_to_token, \
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
