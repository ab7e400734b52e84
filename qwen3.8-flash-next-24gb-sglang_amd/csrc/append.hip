// Write path of the tiered KV cache: quantize-append kernels for gfx950.
//
// One wavefront (64 lanes) owns one (token, KV head) row; lane l holds channels 4l..4l+3, so a 32-channel INT4
// group is 8 lanes and a 64-channel INT8 group is 16 lanes: the group absmax is a lane butterfly inside the wave
// and every load/store is a contiguous per-lane chunk (row-coalesced).  Four rows per 256-thread block.
//
//   kvt_quant_store_tiered  dual write (patches/kv_tiers.py:272-443): owner stamp launch, then the INT8 ring row
//                           (owner only) + INT4 pool row (always) launch.
//   kvt_quant_store_int8    INT8-G quant + scatter (patches/kv_int8.py:281-362, with the fp16-max clamp).
//   kvt_quant_store_int4    INT4-G32 quant + nibble pack + scatter (patches/kv_int4.py:289-393).
//   kvt_page_table_update   writes (seq, logical page) -> physical page entries before an evicting append.
//   kvt_append_evict        position-indexed ring append: requantizes the ring row being overwritten into the
//                           INT4 page of its position (docs/KV_TIERS_PLAN.md:53, :63-67), then stores the new
//                           token's INT8 row.

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kRowsPerBlock = 4;

struct RowIn {
  const void* base;
  int64_t stride_n;  // elements
  int64_t stride_h;  // elements
};

template <int DT>
KVT_DEV void load4(const RowIn& in, int64_t t, int h, int c0, const uint16_t* sm_inv, int D, float x[4]) {
  const int64_t off = t * in.stride_n + (int64_t)h * in.stride_h + c0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = load_in<DT>(in.base, off + i);
    float m = sm_inv ? f16_bits_to_f32(sm_inv[h * D + c0 + i]) : 1.0f;
    x[i] = v * m;  // x = f32(k) * f32(sm_inv)  (patches/kv_tiers.py:332-333)
  }
}

// INT8-G row part held by this lane: 4 codes packed little-endian, plus the group scale (fp16 bits).
template <int LANES_PER_GROUP>
KVT_DEV uint32_t quant8_lane(const float x[4], uint16_t* scale_bits) {
  float a = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
  a = group_max<LANES_PER_GROUP>(a);
  const uint16_t sb = group_scale(a, 127.0f);
  const float s = f16_bits_to_f32(sb);
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = (int)quant_code(x[i], s, 127.0f);
    packed |= ((uint32_t)(q & 0xff)) << (8 * i);
  }
  *scale_bits = sb;
  return packed;
}

// INT4-G32 row part held by this lane: 2 bytes (4 nibbles), plus the group scale (fp16 bits).
KVT_DEV uint32_t quant4_lane(const float x[4], uint16_t* scale_bits) {
  float a = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
  a = group_max<8>(a);
  const uint16_t sb = group_scale(a, 7.0f);
  const float s = f16_bits_to_f32(sb);
  const uint32_t b0 = pack_pair(quant_code(x[0], s, 7.0f), quant_code(x[1], s, 7.0f));
  const uint32_t b1 = pack_pair(quant_code(x[2], s, 7.0f), quant_code(x[3], s, 7.0f));
  *scale_bits = sb;
  return b0 | (b1 << 8);
}

template <int D, int G8>
KVT_DEV void store_ring_row(int8_t* rbuf, uint16_t* rscale, int64_t r, int H, int h, int lane, const float x[4]) {
  constexpr int NG8 = D / G8;
  uint16_t sb;
  const uint32_t packed = quant8_lane<G8 / 4>(x, &sb);
  reinterpret_cast<uint32_t*>(rbuf + (r * H + h) * D)[lane] = packed;
  if ((lane & (G8 / 4 - 1)) == 0) rscale[(r * H + h) * NG8 + lane / (G8 / 4)] = sb;
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

__global__ void __launch_bounds__(256) stamp_owner_kernel(const void* loc, int loc64, int64_t N, int32_t* owner,
                                                          int64_t ring_mask) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N) return;
  const int64_t slot = load_loc(loc, loc64, t);
  owner[slot & ring_mask] = (int32_t)slot;  // one winner per contested ring row (patches/kv_tiers.py:272-280)
}

// MODE 0: tiered dual write; 1: INT8 only (ring buffers are the pool); 2: INT4 only.
template <int DT, int D, int G8, int MODE>
__global__ void __launch_bounds__(256) quant_store_kernel(
    RowIn kin, RowIn vin, const void* loc, int loc64, int64_t N, int H, uint8_t* k4, uint8_t* v4, uint16_t* ks4,
    uint16_t* vs4, int8_t* rk, int8_t* rv, uint16_t* rks, uint16_t* rvs, const int32_t* owner,
    const uint16_t* sm_k_inv, const uint16_t* sm_v_inv, int64_t ring_mask) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (item >= N * H) return;
  const int64_t t = item / H;
  const int h = (int)(item - t * H);
  if (lane >= D / 4) return;
  const int64_t slot = load_loc(loc, loc64, t);
  const int c0 = 4 * lane;
  float xk[4], xv[4];
  load4<DT>(kin, t, h, c0, sm_k_inv, D, xk);
  load4<DT>(vin, t, h, c0, sm_v_inv, D, xv);
  if constexpr (MODE == 0) {
    const int64_t r = slot & ring_mask;
    const bool hot = (int64_t)owner[r] == slot;  // owner stamped by the preceding launch
    if (hot) {  // wave-uniform: the whole row belongs to one token
      store_ring_row<D, G8>(rk, rks, r, H, h, lane, xk);
      store_ring_row<D, G8>(rv, rvs, r, H, h, lane, xv);
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

// Requantize the INT8 ring row r (its 4 codes held by this lane) into INT4 pool row `row`.
template <int D, int G8>
KVT_DEV void evict_row(const int8_t* rbuf, const uint16_t* rscale, int64_t r, uint8_t* pbuf, uint16_t* pscale,
                       int64_t row, int H, int h, int lane) {
  constexpr int NG8 = D / G8;
  const uint32_t codes = reinterpret_cast<const uint32_t*>(rbuf + (r * H + h) * D)[lane];
  const float s8 = f16_bits_to_f32(rscale[(r * H + h) * NG8 + (4 * lane) / G8]);
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = (float)(int8_t)(codes >> (8 * i)) * s8;  // exact in fp32
  store_pool_row<D>(pbuf, pscale, row, H, h, lane, x);
}

template <int DT, int D, int G8>
__global__ void __launch_bounds__(256) append_evict_kernel(
    RowIn kin, RowIn vin, const int32_t* seq_ids, const int64_t* positions, int64_t N, int H, uint8_t* k4,
    uint8_t* v4, uint16_t* ks4, uint16_t* vs4, int8_t* rk, int8_t* rv, uint16_t* rks, uint16_t* rvs,
    const int64_t* ring_base, const int32_t* ring_len, const int64_t* ring_start, const int32_t* page_table,
    int64_t pt_stride, const uint16_t* sm_k_inv, const uint16_t* sm_v_inv) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (item >= N * H) return;
  const int64_t t = item / H;
  const int h = (int)(item - t * H);
  if (lane >= D / 4) return;
  const int s = seq_ids[t];
  const int64_t p = positions[t];
  const int64_t R = ring_len[s];
  const int64_t r = ring_base[s] + (p & (R - 1));
  const int64_t e = p - R;  // the position whose ring row this token overwrites
  if (e >= ring_start[s]) {
    const int32_t page = page_table[s * pt_stride + (e >> 6)];
    if (page >= 0) {
      const int64_t row = (int64_t)page * kPage + (e & (kPage - 1));
      evict_row<D, G8>(rk, rks, r, k4, ks4, row, H, h, lane);
      evict_row<D, G8>(rv, rvs, r, v4, vs4, row, H, h, lane);
    }
  }
  float xk[4], xv[4];
  const int c0 = 4 * lane;
  load4<DT>(kin, t, h, c0, sm_k_inv, D, xk);
  load4<DT>(vin, t, h, c0, sm_v_inv, D, xv);
  store_ring_row<D, G8>(rk, rks, r, H, h, lane, xk);
  store_ring_row<D, G8>(rv, rvs, r, H, h, lane, xv);
}

__global__ void page_table_update_kernel(int32_t* pt, int64_t pt_stride, int64_t n, const int32_t* seq,
                                         const int32_t* lpage, const int32_t* ppage) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) pt[(int64_t)seq[i] * pt_stride + lpage[i]] = ppage[i];
}

// ---------------------------------------------------------------------------------------------- dispatch helpers
template <int MODE>
int launch_quant_store(const RowIn& kin, const RowIn& vin, int dtype, const void* loc, int loc64, int64_t N, int H,
                       int D, int group8, uint8_t* k4, uint8_t* v4, uint16_t* ks4, uint16_t* vs4, int8_t* rk,
                       int8_t* rv, uint16_t* rks, uint16_t* rvs, const int32_t* owner, const uint16_t* smk,
                       const uint16_t* smv, int64_t ring_mask, hipStream_t stream) {
  const dim3 grid((unsigned)((N * H + kRowsPerBlock - 1) / kRowsPerBlock));
#define KVT_QS(DT_, D_, G_)                                                                                    \
  hipLaunchKernelGGL((quant_store_kernel<DT_, D_, G_, MODE>), grid, dim3(256), 0, stream, kin, vin, loc, loc64, \
                     N, H, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, smk, smv, ring_mask)
#define KVT_QS_G(DT_, D_)                     \
  if (group8 == 64) {                         \
    KVT_QS(DT_, D_, 64);                      \
  } else if (group8 == D_ && D_ != 64) {      \
    KVT_QS(DT_, D_, D_);                      \
  } else {                                    \
    return KVT_EINVAL;                        \
  }
#define KVT_QS_D(DT_)          \
  if (D == 256) {              \
    KVT_QS_G(DT_, 256)         \
  } else if (D == 128) {       \
    KVT_QS_G(DT_, 128)         \
  } else if (D == 64) {        \
    KVT_QS(DT_, 64, 64);       \
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
  if (N < 0 || H <= 0 || ring_mask < 0 || ((ring_mask + 1) & ring_mask) != 0) return KVT_EINVAL;
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
  if (N < 0 || H <= 0) return KVT_EINVAL;
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
  if (N < 0 || H <= 0) return KVT_EINVAL;
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

int kvt_append_evict(const void* k, const void* v, int dtype, int64_t sk_n, int64_t sk_h, int64_t sv_n, int64_t sv_h,
                     const void* seq_ids, const void* positions, int64_t N, int H, int D, void* k_buf, void* v_buf,
                     void* k_scale, void* v_scale, void* ring_k, void* ring_v, void* ring_ks, void* ring_vs,
                     const void* ring_base, const void* ring_len, const void* ring_start, const void* page_table,
                     int64_t pt_stride, const void* sm_k_inv, const void* sm_v_inv, int group8, void* stream) {
  if (N < 0 || H <= 0) return KVT_EINVAL;
  if (N == 0) return KVT_OK;
  const dim3 grid((unsigned)((N * H + kRowsPerBlock - 1) / kRowsPerBlock));
  hipStream_t st = (hipStream_t)stream;
  const RowIn kin{k, sk_n, sk_h}, vin{v, sv_n, sv_h};
#define KVT_AE(DT_, D_, G_)                                                                                        \
  hipLaunchKernelGGL((append_evict_kernel<DT_, D_, G_>), grid, dim3(256), 0, st, kin, vin, (const int32_t*)seq_ids, \
                     (const int64_t*)positions, N, H, (uint8_t*)k_buf, (uint8_t*)v_buf, (uint16_t*)k_scale,         \
                     (uint16_t*)v_scale, (int8_t*)ring_k, (int8_t*)ring_v, (uint16_t*)ring_ks,                     \
                     (uint16_t*)ring_vs, (const int64_t*)ring_base, (const int32_t*)ring_len,                      \
                     (const int64_t*)ring_start, (const int32_t*)page_table, pt_stride, (const uint16_t*)sm_k_inv, \
                     (const uint16_t*)sm_v_inv)
#define KVT_AE_G(DT_)              \
  if (group8 == 64) {              \
    KVT_AE(DT_, 256, 64);          \
  } else if (group8 == 256) {      \
    KVT_AE(DT_, 256, 256);         \
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
  KVT_CHECK_LAUNCH();
  return KVT_OK;
}

}  // extern "C"
