// Device helpers shared by the split-K decode kernels (decode_mfma.hip, decode_rows.hip): matrix-core operand
// types, the magic-number code conversions, direct-to-LDS buffer copies and their wait counts.
#pragma once

#include "kvt_common.h"

namespace kvt {
namespace dec {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) v2i lds_v2i;
typedef __attribute__((address_space(3))) u4v lds_u4v;

constexpr float kLog2e = 1.4426950408889634f;

KVT_DEV f4 mfma(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
KVT_DEV f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

KVT_DEV h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
KVT_DEV uint32_t as_u32(h2 h) { return __builtin_bit_cast(uint32_t, h); }
KVT_DEV h8 as_h8(u4v u) { return __builtin_bit_cast(h8, u); }
KVT_DEV u4v as_u4(h8 h) { return __builtin_bit_cast(u4v, h); }

// (a & m) | o: one v_and_or_b32 when m and o are VGPR values the compiler cannot fold into literals (see
// NibbleMasks).  Plain code, not inline assembly, so that the compiler's hazard checks see every write (an MFMA may
// still be reading its source registers when the next instruction overwrites them).
KVT_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) { return (a & m) | o; }

// A value in a VGPR that the compiler treats as unknown (no literal folding, no instruction emitted here).
KVT_DEV uint32_t opaque_vgpr(uint32_t x) {
  asm("" : "+v"(x));
  return x;
}

// Masks of the magic-number code conversion, held in VGPRs once per wavefront.
struct NibbleMasks {
  uint32_t lo, hi, magic;
};
KVT_DEV NibbleMasks nibble_masks() {
  return NibbleMasks{opaque_vgpr(0x000F000Fu), opaque_vgpr(0x00F000F0u), opaque_vgpr(0x64006400u)};
}

// 8 INT4 codes (one dword, nibbles n0..n7) -> raw magic-number fp16 values in the order [n0, n4, n1, n5, n2, n6, n3,
// n7]: 1024 + n for even nibbles, 1024 + 16 n for odd ones (operand positions 2, 3, 6, 7).
KVT_DEV h8 int4_codes_raw(uint32_t w, uint32_t mlo, uint32_t mhi, uint32_t magic) {
  const uint32_t w8 = w >> 8;
  const u4v r = {and_or(w, mlo, magic), and_or(w, mhi, magic), and_or(w8, mlo, magic), and_or(w8, mhi, magic)};
  return as_h8(r);
}

// Two INT8 codes per half of a dword -> fp16 exact: b + 128 as the low byte of 1024 + u, minus 1152.
KVT_DEV h2 int8_pair_lo(uint32_t u) {
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  return as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off;
}
KVT_DEV h2 int8_pair_hi(uint32_t u) {
  const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  return as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off;
}

// 8 INT8 codes (two dwords, natural channel order) -> fp16 exact.
KVT_DEV h8 int8_codes_to_h8(uint32_t w0, uint32_t w1) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;   // b + 128 as unsigned bytes
  const h2 a = int8_pair_lo(u0), b = int8_pair_hi(u0), c = int8_pair_lo(u1), d = int8_pair_hi(u1);
  return h8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

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

// 16 bytes per lane from rsrc + voffset into lds + 16 * lane.  M0 (the LDS base) is an input operand of the
// statement, so the compiler sets it.  The s_nop 4 gives the 5 wait states a vector-memory instruction needs after a
// VALU write of an SGPR it reads (v_readfirstlane of the descriptor words, below): the compiler's hazard checks do
// not look inside inline assembly, and with fewer wait states the load may use stale descriptor words (a wrong base
// or range: an access outside the buffer).  It also covers the one wait state an LDS DMA needs after an SALU write
// of M0.
// Inline assembly rather than the builtin so that the compiler does not treat every later LDS read as dependent on
// the copy: completion is tracked explicitly with wait_vmcnt by the caller.  The loads are non-temporal (nt): a
// layer streams its KV bytes through the caches once, and marked as streaming they leave the small per-step metadata
// every layer starts from (sequence lengths, ring placement, page ids, the decode plan) cached.
// The descriptor words pass through readfirstlane: they are uniform by construction, and this keeps them in SGPRs
// (the "s" operand) even where register pressure would otherwise leave a copy of them in VGPRs.
KVT_DEV i32x4 uniform_rsrc(i32x4 r) {
  return i32x4{__builtin_amdgcn_readfirstlane(r.x), __builtin_amdgcn_readfirstlane(r.y),
               __builtin_amdgcn_readfirstlane(r.z), __builtin_amdgcn_readfirstlane(r.w)};
}

KVT_DEV void copy16_to_lds(i32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds" : : "v"(voffset), "s"(uniform_rsrc(rsrc)),
               "{m0}"(base) : "memory");
}

// 4 bytes per lane from rsrc + voffset into lds + 4 * lane (same conventions).
KVT_DEV void copy4_to_lds(i32x4 rsrc, void* lds, uint32_t voffset) {
  const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds" : : "v"(voffset), "s"(uniform_rsrc(rsrc)),
               "{m0}"(base) : "memory");
}

// s_waitcnt vmcnt(<= n) leaving the other counters alone (gfx9 encoding).
template <int N>
KVT_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// s_waitcnt lgkmcnt(0): every LDS read of this wavefront has returned.
KVT_DEV void wait_lgkm0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
}

// Compiler-level ordering point for LDS traffic inside one wavefront (the hardware executes a wavefront's LDS
// instructions in order, so no memory fence is needed).
KVT_DEV void wave_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

// 32-bit LDS address of a pointer into the shared block.
KVT_DEV uint32_t lds_off(const void* p) { return (uint32_t)(uintptr_t)p; }

// The next tile of this wavefront: from the block's shared counter (dyn: the wavefronts that run ahead take more
// tiles, so the block's wavefronts finish together; the floating-point summation order then depends on timing) or in
// the fixed order w, w + waves, w + 2 waves, ... (bit-reproducible).
template <int kWaves>
KVT_DEV int take_tile(int32_t* next, bool dyn, int& taken) {
  int t = 0;
  if (dyn) {
    if ((threadIdx.x & 63) == 0) t = atomicAdd(next, 1);
  } else {
    t = (int)(threadIdx.x >> 6) + kWaves * taken;
  }
  ++taken;
  return __builtin_amdgcn_readfirstlane(t);
}

// Positions [0, L) of a sequence split into n_b blocks of equal cost: a paged position costs 4, a ring position
// kHotCost4 (its bytes are about 7 / 4 of a paged one's); paged boundaries are multiples of `align`.  hs = the first
// ring position.  Returns the start of block w (w = n_b gives L).
template <int kHotCost4, int align>
KVT_DEV int64_t split_bound(int64_t L, int64_t hs, int64_t w, int64_t n_b) {
  if (w >= n_b) return L;
  const int64_t cost = 4 * hs + kHotCost4 * (L - hs);
  const int64_t x = cost * w / n_b;
  if (x <= 4 * hs) return (x >> 2) & ~(int64_t)(align - 1);
  return hs + (x - 4 * hs + kHotCost4 - 1) / kHotCost4;
}

// First ring position of a sequence: max(ring_start, L - R) clamped to [0, L].
KVT_DEV int64_t hot_start(int64_t L, int64_t R, int64_t ring_start) {
  return min(max(max(ring_start, L - R), (int64_t)0), L);
}

// Launch of the full-row split-K decode (decode_rows.hip): H = 2 KV heads, up to 8 q heads per KV head; plan is a
// per-step decode plan (kvt_decode_plan) or nullptr.  Returns a KVT_ status.
int rows_launch(const void* q, int64_t q_stride_b, const void* seq_lens, int batch, int gs, int group8, const void* k4,
                const void* v4, const void* ks4, const void* vs4, const void* rk, const void* rv, const void* rks,
                const void* rvs, const void* ring_base, const void* ring_len, const void* ring_start,
                const void* page_table, int64_t pt_stride, int64_t pool_rows, float scale, int n_splits,
                const void* split_map, int n_map, void* part_o, void* part_ml, int flags, const void* plan,
                hipStream_t stream);

}  // namespace dec
}  // namespace kvt
