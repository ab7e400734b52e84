// Top-k sparse decode attention over the quantized pools, fused: the selected positions of each request are
// resolved (position -> slot through req_to_token -> tier through the owner table), dequantized exactly as the
// reference's compact gather does (bf16(q * s * sm), patches/kv_tiers.py:446-538) and attended in one pass, with no
// bf16 scratch.  The reference's decode gathers into that scratch and runs FlashAttention-2 over it
// (sglang/qwen4exp-serving-73a255206f.patch:1832-1882); this kernel replaces both launches' work, and its partials
// go through the same combine as the dense decode.
//
// One block of 4 wavefronts per (request, KV head, 64 selected columns), a wavefront per tile of 16: the tile's
// K and V rows are dequantized into LDS as bf16, then QK^T and P.V run as bf16 16x16x16 matrix-core steps with
// fp32 accumulation:
//   S^T[row][head] = K[row][:] . Q[head][:]   (A = K tile, B = Q^T; 16 steps over the 256 channels)
//   O[head][ch]   += P[head][row] V[row][ch]  (A = P straight from S^T's accumulator layout as bf16 high part
//                                               + bf16 remainder, B = V tile by the transposing LDS read)
// The 4 wavefronts merge through LDS and the block writes an unnormalized partial (m, l, o) per q head (m in
// natural-log units, as the dense decode's); kvt_decode_combine merges the column splits.  Columns c of request b attend when c < the request's
// valid count (cu_k[b + 1] - cu_k[b]) and 0 <= indices[b][c] < seq_lens[b] - the columns the reference's gather
// writes and its attention reads when the valid positions come first (the indexer pads with -1 at the end).
//
// Kinds (the compact gather's codes): 0 INT8-G pool, 1 INT4-G32 pool, 2 tiered (INT8-G ring over INT4-G32 rows,
// owner test).

#include "kvt_common.h"

using namespace kvt;

namespace {

constexpr int kD = 256;
constexpr int kRows = 16;          // rows per MFMA tile
constexpr int kWaves = 4;          // wavefronts per block, one tile each
constexpr int kCols = kWaves * kRows;  // selected columns per block (one partial)
constexpr int kHeads = 16;         // q heads per KV head the tile holds (rows beyond the group are zero)
constexpr int kKPitch = kD + 8;    // bf16 per K row in LDS (the pad spreads a column of rows over the banks)

typedef short bf4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf4 lds_v4s;
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
  uint32_t rows8;        // rows of the INT8 tensors (ring R when tiered, the pool otherwise)
  uint32_t rows4;        // rows of the INT4 pool
  float scale;
  const uint16_t* q;       // bf16 [batch, Hq, D] with batch stride q_stride_b
  int64_t q_stride_b;
  float* part_o;           // [(b H + h) n_splits + split][gs][D]
  float* part_ml;          // [(b H + h) n_splits + split][gs][2]
};

KVT_DEV int64_t load_idx(const void* p, int is64, int64_t i) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t) reinterpret_cast<const int32_t*>(p)[i];
}

KVT_DEV f4 mfma_bf16(bf4 a, bf4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0); }

// bf16 pair (round to nearest even, v_cvt_pk_bf16_f32): lo in bits 0-15.
KVT_DEV uint32_t bf16x2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)hi) << 16);
}

KVT_DEV __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// The 4 codes of this lane's channels in a loaded word: INT8 rows give 4 bytes; INT4 rows give the 16-bit half
// (lane & 1) of the dword holding channel pairs 4 (lane >> 1) .. + 3 (low nibble = even channel).
KVT_DEV void codes4(bool hot, uint32_t w, int lane, float c[4]) {
  if (hot) {
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = (float)(int8_t)(w >> (8 * i));
  } else {
    const uint32_t h16 = w >> (16 * (lane & 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = (float)((int)((h16 >> (4 * i)) & 15u) - 8);
  }
}

// One tile's raw row data for this lane (channels 4 lane .. + 3 of K and V, and their scales).
struct TileLoads {
  uint32_t kw[kRows], vw[kRows], ks[kRows], vs[kRows];
  int fl[kRows];
};

constexpr uint32_t kNoRow = 0x80000000u;   // a row offset past every buffer: its loads return zero

// Buffer resources over whole tensors (byte offsets are 32-bit: the launcher checks the sizes).
struct PoolRsrc {
  __amdgpu_buffer_rsrc_t k8, v8, ks8, vs8, k4, v4, ks4, vs4;
};

// Issue the loads of the wavefront's tile: row r's byte offsets (codes and scales, in the row's tier) come from
// lane r by readlane and go in the scalar offset of the loads, so every row costs a few scalar instructions and no
// vector address math; the lane offsets are fixed per tier.
template <int G8>
KVT_DEV void issue_tile(const PoolRsrc& P, int flags, uint32_t coff, uint32_t soff, int lane, TileLoads& L) {
  const uint32_t off8 = 4u * lane, off4 = 4u * (lane >> 1);
  const uint32_t soff8 = 2u * ((4u * lane) / G8), soff4 = 2u * (lane >> 3);
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int f = __builtin_amdgcn_readlane(flags, r);
    L.fl[r] = f;
    const uint32_t co = (uint32_t)__builtin_amdgcn_readlane((int)coff, r);
    const uint32_t so = (uint32_t)__builtin_amdgcn_readlane((int)soff, r);
    if ((f & 2) != 0) {
      L.kw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.k8, off8, co, 0);
      L.vw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.v8, off8, co, 0);
      L.ks[r] = __builtin_amdgcn_raw_buffer_load_b16(P.ks8, soff8, so, 0);
      L.vs[r] = __builtin_amdgcn_raw_buffer_load_b16(P.vs8, soff8, so, 0);
    } else {
      L.kw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.k4, off4, co, 0);
      L.vw[r] = __builtin_amdgcn_raw_buffer_load_b32(P.v4, off4, co, 0);
      L.ks[r] = __builtin_amdgcn_raw_buffer_load_b16(P.ks4, soff4, so, 0);
      L.vs[r] = __builtin_amdgcn_raw_buffer_load_b16(P.vs4, soff4, so, 0);
    }
  }
}

template <int KIND, int G8>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(3))) sparse_decode_kernel(SparseArgs A) {
  // per wavefront: its tile's K and V rows (bf16); after the tiles, the same space holds the 4 partials' merge
  // one tile buffer per wavefront: K rows until S is formed, then V rows (LDS per block 42 KB: 3 blocks per CU)
  __shared__ __align__(16) uint16_t kv[kWaves][kRows * kKPitch];
  __shared__ __align__(16) uint16_t qs[kHeads * kKPitch];   // the group's q heads, bf16 (zero beyond gs)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = blockIdx.x;
  const int b = blockIdx.y / A.H;
  const int h = blockIdx.y - b * A.H;
  const int H = A.H, gs = A.gs;
  const int64_t item = ((int64_t)b * H + h) * A.n_splits + split;
  const int n16 = lane & 15, kq = lane >> 4;
  uint16_t* kt = kv[wave];
  uint16_t* vr = kv[wave];   // the same rows: V is dequantized once the K reads of S are issued

  // the group's q heads into LDS (512 16-byte chunks; heads beyond the group read as zero)
#pragma unroll
  for (int i = threadIdx.x; i < kHeads * kD / 8; i += 64 * kWaves) {
    const int hq = i / (kD / 8), ch = i - hq * (kD / 8);
    uint4 w = {0u, 0u, 0u, 0u};
    if (hq < gs) w = *reinterpret_cast<const uint4*>(A.q + b * A.q_stride_b + (int64_t)(h * gs + hq) * kD + 8 * ch);
    *reinterpret_cast<uint4*>(&qs[hq * kKPitch + 8 * ch]) = w;
  }

  // resolve: lane r < 16 of wavefront w resolves column split * 64 + 16 w + r to (valid, hot, row)
  const int64_t vcount = load_idx(A.cu_k, A.cu64, b + 1) - load_idx(A.cu_k, A.cu64, b);
  const int64_t L = A.seq_lens[b];
  const int64_t req = load_idx(A.req_indices, A.req64, b);
  const int64_t col = (int64_t)split * kCols + kRows * wave + n16;
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
  const int flags = (valid ? 1 : 0) | (hot ? 2 : 0);
  // the row's byte offsets in its tier: codes (INT8 rows D bytes, INT4 rows D / 2) and scales
  const int64_t rh = row * H + h;
  const uint32_t coff = !valid ? kNoRow : (uint32_t)(hot ? rh * kD : rh * (kD / 2));
  const uint32_t soff = !valid ? kNoRow : (uint32_t)(hot ? rh * (kD / G8) * 2 : rh * (kD / kG4) * 2);
  PoolRsrc P;
  {
    const uint32_t n8 = A.rows8 * (uint32_t)H * kD, n4 = A.rows4 * (uint32_t)H * (kD / 2);
    const uint32_t s8 = A.rows8 * (uint32_t)H * (kD / G8) * 2, s4 = A.rows4 * (uint32_t)H * (kD / kG4) * 2;
    P.k8 = rsrc(KIND == 2 ? (const void*)A.rk : A.k, KIND == 1 ? 0u : n8);
    P.v8 = rsrc(KIND == 2 ? (const void*)A.rv : A.v, KIND == 1 ? 0u : n8);
    P.ks8 = rsrc(KIND == 2 ? A.rks : A.ks, KIND == 1 ? 0u : s8);
    P.vs8 = rsrc(KIND == 2 ? A.rvs : A.vs, KIND == 1 ? 0u : s8);
    P.k4 = rsrc(A.k, KIND == 0 ? 0u : n4);
    P.v4 = rsrc(A.v, KIND == 0 ? 0u : n4);
    P.ks4 = rsrc(A.ks, KIND == 0 ? 0u : s4);
    P.vs4 = rsrc(A.vs, KIND == 0 ? 0u : s4);
  }
  TileLoads T;
  issue_tile<G8>(P, flags, coff, soff, lane, T);

  // smoothing factors of this lane's channels 4 lane .. 4 lane + 3
  float smk[4] = {1.f, 1.f, 1.f, 1.f}, smv[4] = {1.f, 1.f, 1.f, 1.f};
  if (A.sm_k != nullptr) {
    const uint2 w = *reinterpret_cast<const uint2*>(A.sm_k + (int64_t)h * kD + 4 * lane);
    smk[0] = f16_bits_to_f32((uint16_t)w.x);
    smk[1] = f16_bits_to_f32((uint16_t)(w.x >> 16));
    smk[2] = f16_bits_to_f32((uint16_t)w.y);
    smk[3] = f16_bits_to_f32((uint16_t)(w.y >> 16));
  }
  if (A.sm_v != nullptr) {
    const uint2 w = *reinterpret_cast<const uint2*>(A.sm_v + (int64_t)h * kD + 4 * lane);
    smv[0] = f16_bits_to_f32((uint16_t)w.x);
    smv[1] = f16_bits_to_f32((uint16_t)(w.x >> 16));
    smv[2] = f16_bits_to_f32((uint16_t)w.y);
    smv[3] = f16_bits_to_f32((uint16_t)(w.y >> 16));
  }

  // dequantize the tile's K rows into this wavefront's LDS rows (row-major)
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const bool ht = (T.fl[r] & 2) != 0;
    float c[4], x[4];
    codes4(ht, T.kw[r], lane, c);
    const float sk = f16_bits_to_f32((uint16_t)T.ks[r]);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = c[i] * sk * smk[i];
    *reinterpret_cast<uint2*>(&kt[r * kKPitch + 4 * lane]) = uint2{bf16x2(x[0], x[1]), bf16x2(x[2], x[3])};
  }
  __syncthreads();   // q staged (the tile rows are this wavefront's own: its LDS accesses are in order)

  // S^T = K Q^T: lane l holds rows 4 (l >> 4) + i of q head l & 15
  f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint2 ka = *reinterpret_cast<const uint2*>(&kt[n16 * kKPitch + 16 * k + 4 * kq]);
    const uint2 qb = *reinterpret_cast<const uint2*>(&qs[n16 * kKPitch + 16 * k + 4 * kq]);
    s = mfma_bf16(__builtin_bit_cast(bf4, ka), __builtin_bit_cast(bf4, qb), s);
  }
  // V rows into the same LDS rows: a wavefront's LDS accesses complete in order, so these stores land after the K
  // reads above (the compiler keeps stores behind loads that may alias them)
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const bool ht = (T.fl[r] & 2) != 0;
    float c[4], x[4];
    codes4(ht, T.vw[r], lane, c);
    const float sv = f16_bits_to_f32((uint16_t)T.vs[r]);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = c[i] * sv * smv[i];
    *reinterpret_cast<uint2*>(&vr[r * kKPitch + 4 * lane]) = uint2{bf16x2(x[0], x[1]), bf16x2(x[2], x[3])};
  }
  // softmax over the tile's rows (log2 units): rows 4 kq + i of this lane, the other 12 in lanes n16 + 16 j
  constexpr float kLog2e = 1.4426950408889634f;
  const float cs = A.scale * kLog2e;
  float tv[4], mloc = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = __shfl(flags, 4 * kq + i, 64);   // the row's resolve lane
    tv[i] = (f & 1) ? s[i] * cs : -INFINITY;
    mloc = fmaxf(mloc, tv[i]);
  }
  const float m = max_xor16_32(mloc);
  float p[4], lsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(tv[i] - m);
    lsum += p[i];
  }
  const float l = sum_xor16_32(lsum);
  // P as bf16 high part + bf16 remainder (two products per step): P keeps ~16 significant bits, against 8 for a
  // plain bf16 cast, so a peaked softmax stays within the fp32 reference's tolerance
  const uint32_t h01 = bf16x2(p[0], p[1]), h23 = bf16x2(p[2], p[3]);
  const uint32_t l01 = bf16x2(p[0] - __uint_as_float(h01 << 16), p[1] - __uint_as_float(h01 & 0xffff0000u));
  const uint32_t l23 = bf16x2(p[2] - __uint_as_float(h23 << 16), p[3] - __uint_as_float(h23 & 0xffff0000u));
  const bf4 pa = __builtin_bit_cast(bf4, uint2{h01, h23});
  const bf4 pb = __builtin_bit_cast(bf4, uint2{l01, l23});
  // O = P V.  B = V[rows 4 kq + k][channel 16 n + n16] by the transposing read: in each 16-lane group, lane L's
  // element k comes from element L & 3 of the 8 bytes lane 4 k + (L >> 2) addresses, so lane m addresses
  // V[4 kq + (m >> 2)][16 n + 4 (m & 3)]
  f4 o[16];   // O[head 4 kq + i][channel 16 n + n16]
  const uint32_t vbase = (uint32_t)(uintptr_t)&vr[(4 * kq + (n16 >> 2)) * kKPitch + 4 * (n16 & 3)];
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    const bf4 vop = __builtin_bit_cast(
        bf4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vbase + 32u * (uint32_t)n)));
    o[n] = mfma_bf16(pb, vop, mfma_bf16(pa, vop, f4{0.f, 0.f, 0.f, 0.f}));
  }

  // merge the 4 wavefronts' partials through LDS (the tile rows are done with): wavefront w stores O rows of heads
  // < gs and (m, l) per head; then thread t merges head t / 32, channels 8 (t % 32) .. + 7 over the 4
  __syncthreads();
  float* mo = reinterpret_cast<float*>(&kv[0][0]);                 // [wave][head < 8][256]
  float* mml = mo + kWaves * 8 * kD;                                // [wave][head][2]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int hq = 4 * kq + i;
    if (hq < gs) {
#pragma unroll
      for (int n = 0; n < 16; ++n) mo[(wave * 8 + hq) * kD + 16 * n + n16] = o[n][i];
    }
  }
  if (lane < gs) {
    mml[(wave * 8 + lane) * 2] = m;
    mml[(wave * 8 + lane) * 2 + 1] = l;
  }
  __syncthreads();
  {
    const int hq = threadIdx.x >> 5, c0 = 8 * (threadIdx.x & 31);
    if (hq < gs) {
      float mw[kWaves], M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        mw[w] = mml[(w * 8 + hq) * 2];
        M = fmaxf(M, mw[w]);
      }
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, lt = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float a = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[w] - M);
        lt += a * mml[(w * 8 + hq) * 2 + 1];
        const float4 o0 = *reinterpret_cast<const float4*>(&mo[(w * 8 + hq) * kD + c0]);
        const float4 o1 = *reinterpret_cast<const float4*>(&mo[(w * 8 + hq) * kD + c0 + 4]);
        acc[0] += a * o0.x;
        acc[1] += a * o0.y;
        acc[2] += a * o0.z;
        acc[3] += a * o0.w;
        acc[4] += a * o1.x;
        acc[5] += a * o1.y;
        acc[6] += a * o1.z;
        acc[7] += a * o1.w;
      }
      float* dst = A.part_o + (item * gs + hq) * kD + c0;
      *reinterpret_cast<float4*>(dst) = float4{acc[0], acc[1], acc[2], acc[3]};
      *reinterpret_cast<float4*>(dst + 4) = float4{acc[4], acc[5], acc[6], acc[7]};
      if (c0 == 0) {   // (m, l) of the block's partial, m in natural-log units
        constexpr float kLn2 = 0.6931471805599453f;
        A.part_ml[(item * gs + hq) * 2 + 0] = M == -INFINITY ? -INFINITY : M * kLn2;
        A.part_ml[(item * gs + hq) * 2 + 1] = lt;
      }
    }
  }
}

}  // namespace

extern "C" {

int kvt_sparse_decode(int kind, const void* q, int64_t q_stride_b, const void* k, const void* v, const void* k_scale,
                      const void* v_scale, int64_t pool_rows, const void* ring_k, const void* ring_v, const void* ring_ks,
                      const void* ring_vs, const void* owner, int64_t ring_mask, const void* sm_k, const void* sm_v,
                      const void* req_to_token, int64_t req_stride, const void* req_indices, int req_is_int64,
                      const void* indices, int64_t idx_stride, const void* seq_lens, const void* cu_k,
                      int cu_is_int64, int batch, int topk, int H, int Hq, int D, int group8, float scale,
                      int n_splits, void* part_o, void* part_ml, void* stream) {
  if (batch <= 0 || topk <= 0 || H <= 0 || Hq % H != 0 || Hq / H > 8 || D != kD) return KVT_EINVAL;
  if (n_splits < (topk + kCols - 1) / kCols || kind < 0 || kind > 2) return KVT_EINVAL;
  if (kind == 2 && (owner == nullptr || ring_k == nullptr || ((ring_mask + 1) & ring_mask) != 0)) return KVT_EINVAL;
  if (pool_rows <= 0) return KVT_EINVAL;
  // byte offsets are 32-bit and must stay below kNoRow (rows * H * D bytes of INT8 codes, / 2 for INT4)
  const int64_t rows8 = kind == 2 ? ring_mask + 1 : (kind == 0 ? pool_rows : 0);
  const int64_t rows4 = kind == 0 ? 0 : pool_rows;
  if (rows8 * H * kD >= (int64_t)kNoRow || rows4 * H * (kD / 2) >= (int64_t)kNoRow) return KVT_ERANGE;
  SparseArgs A{k, v, (const uint16_t*)k_scale, (const uint16_t*)v_scale, (const int8_t*)ring_k, (const int8_t*)ring_v,
               (const uint16_t*)ring_ks, (const uint16_t*)ring_vs, (const int32_t*)owner, ring_mask,
               (const uint16_t*)sm_k, (const uint16_t*)sm_v, (const int32_t*)req_to_token, req_stride, req_indices,
               req_is_int64, (const int32_t*)indices, idx_stride, (const int32_t*)seq_lens, cu_k, cu_is_int64, topk,
               H, Hq / H, n_splits, (uint32_t)rows8, (uint32_t)rows4, scale, (const uint16_t*)q, q_stride_b,
               (float*)part_o, (float*)part_ml};
  const dim3 grid((unsigned)n_splits, (unsigned)(batch * H));
  hipStream_t st = (hipStream_t)stream;
#define KVT_SD(KIND_, G_) hipLaunchKernelGGL((sparse_decode_kernel<KIND_, G_>), grid, dim3(64 * kWaves), 0, st, A)
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
