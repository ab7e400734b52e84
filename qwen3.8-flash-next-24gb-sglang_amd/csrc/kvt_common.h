// Shared device helpers for the tiered KV-cache kernels (gfx950).
//
// Rounding contract (the reference's torch forms, gemv/test_kv_tiers.py:65-87):
//   * fp32 scale math with IEEE-exact division (__fdiv_rn), never a reciprocal approximation;
//   * round-half-to-even quantization (rintf -> v_rndne_f32);
//   * RNE conversions to fp16 (__float2half_rn) and bf16 (bf16_rne below).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define KVT_DEV __device__ __forceinline__

namespace kvt {

constexpr int kG4 = 32;              // INT4 pool: channels per fp16 scale
constexpr int kPage = 64;            // tokens per INT4 page
constexpr float kFp16Max = 65504.0f;

// Input element types of the write path ("any float dtype", patches/kv_tiers.py:391).
enum DType : int { kBF16 = 0, kF16 = 1, kF32 = 2 };

KVT_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16 with round-to-nearest-even; NaN stays a quiet NaN (torch's conversion).
KVT_DEV uint16_t bf16_rne(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

KVT_DEV float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
KVT_DEV uint16_t f32_to_f16_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }

template <int DT>
KVT_DEV float load_in(const void* base, int64_t idx) {
  if constexpr (DT == kBF16) {
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  } else if constexpr (DT == kF16) {
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
  } else {
    return reinterpret_cast<const float*>(base)[idx];
  }
}

// Butterfly max over aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
KVT_DEV float group_max(float v) {
#pragma unroll
  for (int o = width / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Cross-lane steps on the VALU (v_permlane16_swap / v_permlane32_swap, gfx950) instead of LDS permutes.  With both
// operands equal, the two results at lane l are the values of lanes l and l ^ 16 (resp. l ^ 32), in an order that
// depends on l: a max or a sum of the two is the pairwise reduction.  All 64 lanes must be active.
KVT_DEV float max_xor16_32(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
KVT_DEV float sum_xor16_32(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// The value of lane l ^ 32.
KVT_DEV uint32_t xor32_u32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}

// Stored scale of a group with absmax a: fp16(min(a > 0 ? a / qmax : 1, 65504))
// (patches/kv_tiers.py:337, :367).  Returns the fp16 bits.
KVT_DEV uint16_t group_scale(float a, float qmax) {
  float s = a > 0.0f ? __fdiv_rn(a, qmax) : 1.0f;
  s = fminf(s, kFp16Max);
  return f32_to_f16_bits(s);
}

// q = clamp(rne(x / s), -qmax, qmax) with an IEEE division (patches/kv_int4.py:334-338).
KVT_DEV float quant_code(float x, float s, float qmax) {
  float q = rintf(__fdiv_rn(x, s));
  return fminf(fmaxf(q, -qmax), qmax);
}

// Offset-binary nibble pair: low nibble = even channel, high = odd channel (patches/kv_int4.py:337-339).
KVT_DEV uint32_t pack_pair(float qe, float qo) {
  return (uint32_t)((int)qe + 8) | ((uint32_t)((int)qo + 8) << 4);
}

}  // namespace kvt

// Status codes returned by every C-ABI entry point (mapped to Python exceptions by the wrappers).
#define KVT_OK 0
#define KVT_EINVAL -1       // a shape / size / dtype argument the kernel does not support
#define KVT_ELAUNCH -2      // hipGetLastError after the launch
#define KVT_ERANGE -3       // a size beyond a documented maximum
#define KVT_ENOTSUP -4      // the device lacks a needed capability (virtual memory management)
#define KVT_ENOMEM -5       // the HIP runtime could not provide address space or physical memory
#define KVT_EHIP -6         // another HIP runtime call failed
#define KVT_DECODE_DYNAMIC 1   // kvt_decode_mfma flag: tiles to wavefronts first come
#define KVT_DECODE_HEADWISE 2  // kvt_decode_mfma flag: one KV head per block even where both fit one wavefront

#define KVT_CHECK_LAUNCH()                                   \
  do {                                                       \
    if (hipGetLastError() != hipSuccess) return KVT_ELAUNCH; \
  } while (0)
