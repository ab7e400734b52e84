// Lazily backed device buffers on HIP virtual memory: an arena is one reserved range of device address space whose
// prefix is backed by physical memory on demand and handed back beyond a floor.
//
// Behaviour follows the reference's lazy KV backing (patches/kv_lazy.py:39-63 uncommit_beyond, :70-88 ensure_prefix /
// release_beyond over SGLang's VMM owner): the whole pool is reserved as address space; commits back a growing
// prefix; a release unmaps every mapping that starts at or beyond the (granularity-aligned) cut.  Every mapping is
// one physical allocation of one 2 MiB granule (a 262,144-token pool's 64 MiB code buffer backed in full is 32
// mappings), so no mapping straddles a granule-aligned cut.
//
// Host code only (no kernels).  Every entry point is synchronous with respect to the host; before unmapping, the
// device's queued work is waited for (hipDeviceSynchronize, as the reference's release_beyond does with
// torch.cuda.synchronize()).  A failed runtime call is reported on stderr.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <new>
#include <vector>

#include "kvt_common.h"

namespace {

struct Mapping {
  uint64_t offset;   // from the arena base
  uint64_t bytes;
  hipMemGenericAllocationHandle_t handle;
};

struct Arena {
  int device;
  char* base;
  uint64_t reserved;    // bytes of address space (a multiple of gran)
  uint64_t gran;        // mapping granularity
  uint64_t backed;      // bytes backed from the base: mappings are contiguous from offset 0
  std::vector<Mapping> maps;
  std::mutex mu;
};

uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// Mappings are single 2 MiB granules at 2 MiB-aligned addresses, whatever smaller granularity the runtime
// recommends (4 KiB on MI355X): on ROCm 7.2, hipMemSetAccess rejected (invalid argument) maps of 2.5 MiB at a 1 MiB
// offset and, intermittently, 6 MiB allocations at 2 MiB-aligned offsets, while one-granule maps never failed.
constexpr uint64_t kGranule = 2ull << 20;

hipMemAllocationProp device_prop(int device) {
  hipMemAllocationProp p = {};
  p.type = hipMemAllocationTypePinned;
  p.location.type = hipMemLocationTypeDevice;
  p.location.id = device;
  return p;
}

int granularity_of(int device, uint64_t* gran) {
  int vmm = 0;
  if (hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported, device) != hipSuccess)
    return KVT_EHIP;
  if (!vmm) return KVT_ENOTSUP;
  const hipMemAllocationProp p = device_prop(device);
  size_t g = 0;
  if (hipMemGetAllocationGranularity(&g, &p, hipMemAllocationGranularityRecommended) != hipSuccess || g == 0)
    return KVT_EHIP;
  *gran = align_up(kGranule, g);
  return KVT_OK;
}


// A failed runtime call is reported on stderr (which call, where, the runtime's message) and mapped to a status.
int report(const char* what, hipError_t e, uint64_t off, uint64_t len, int status) {
  std::fprintf(stderr, "kvtier vmm: %s (offset %llu, %llu bytes) failed: %s (%d)\n", what, (unsigned long long)off,
               (unsigned long long)len, hipGetErrorString(e), (int)e);
  return status;
}

// Current device <-> the arena's device for the duration of a call.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Unmap and release mappings [first, end) of the list (the tail), newest first.  The device's queued work is waited
// for first: a kernel still reading the range would otherwise fault.
int drop_tail(Arena* a, size_t first, uint64_t* freed) {
  uint64_t f = 0;
  int st = KVT_OK;
  if (a->maps.size() > first) {
    const hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return report("hipDeviceSynchronize", e, 0, 0, KVT_EHIP);
  }
  while (a->maps.size() > first) {
    const Mapping m = a->maps.back();
    const hipError_t e = hipMemUnmap(a->base + m.offset, m.bytes);
    if (e != hipSuccess) {
      st = report("hipMemUnmap", e, m.offset, m.bytes, KVT_EHIP);
      break;
    }
    (void)hipMemRelease(m.handle);
    a->maps.pop_back();
    a->backed = m.offset;
    f += m.bytes;
  }
  if (freed) *freed = f;
  return st;
}

}  // namespace

extern "C" {

int kvt_vmm_granularity(int device, uint64_t* granularity) {
  if (granularity == nullptr) return KVT_EINVAL;
  return granularity_of(device, granularity);
}

int kvt_vmm_reserve(int device, uint64_t bytes, void** arena, void** base) {
  if (arena == nullptr || base == nullptr || bytes == 0) return KVT_EINVAL;
  uint64_t gran = 0;
  const int st = granularity_of(device, &gran);
  if (st != KVT_OK) return st;
  Arena* a = new (std::nothrow) Arena();
  if (a == nullptr) return KVT_ENOMEM;
  a->device = device;
  a->gran = gran;
  a->reserved = align_up(bytes, gran);
  a->backed = 0;
  DeviceGuard g(device);
  void* p = nullptr;
  if (hipMemAddressReserve(&p, a->reserved, gran, nullptr, 0) != hipSuccess || p == nullptr) {
    delete a;
    return KVT_ENOMEM;
  }
  if (reinterpret_cast<uintptr_t>(p) % gran != 0) {   // every mapping must start on a granule
    (void)hipMemAddressFree(p, a->reserved);
    delete a;
    return report("hipMemAddressReserve (base not granule-aligned)", hipErrorInvalidValue, 0, bytes, KVT_EHIP);
  }
  a->base = static_cast<char*>(p);
  *arena = a;
  *base = p;
  return KVT_OK;
}

int kvt_vmm_commit(void* arena, uint64_t bytes) {
  if (arena == nullptr) return KVT_EINVAL;
  Arena* a = static_cast<Arena*>(arena);
  std::lock_guard<std::mutex> lk(a->mu);
  const uint64_t want = align_up(bytes, a->gran);
  if (want > a->reserved) return KVT_ERANGE;
  if (want <= a->backed) return KVT_OK;   // commits only grow
  DeviceGuard g(a->device);
  const hipMemAllocationProp p = device_prop(a->device);
  hipMemAccessDesc acc = {};
  acc.location.type = hipMemLocationTypeDevice;
  acc.location.id = a->device;
  acc.flags = hipMemAccessFlagsProtReadWrite;
  // one physical allocation per granule: on failure the granules mapped so far stay (the arena is consistent)
  for (uint64_t off = a->backed; off < want; off += a->gran) {
    hipMemGenericAllocationHandle_t h;
    hipError_t e = hipMemCreate(&h, a->gran, &p, 0);
    if (e != hipSuccess) return report("hipMemCreate", e, off, a->gran, KVT_ENOMEM);
    e = hipMemMap(a->base + off, a->gran, 0, h, 0);
    if (e != hipSuccess) {
      (void)hipMemRelease(h);
      return report("hipMemMap", e, off, a->gran, KVT_EHIP);
    }
    e = hipMemSetAccess(a->base + off, a->gran, &acc, 1);
    if (e != hipSuccess) {
      (void)hipMemUnmap(a->base + off, a->gran);
      (void)hipMemRelease(h);
      return report("hipMemSetAccess", e, off, a->gran, KVT_EHIP);
    }
    a->maps.push_back(Mapping{off, a->gran, h});
    a->backed = off + a->gran;
  }
  return KVT_OK;
}

int kvt_vmm_release_beyond(void* arena, uint64_t keep_bytes, uint64_t* freed) {
  if (arena == nullptr) return KVT_EINVAL;
  Arena* a = static_cast<Arena*>(arena);
  std::lock_guard<std::mutex> lk(a->mu);
  const uint64_t cut = align_up(keep_bytes, a->gran);
  size_t first = a->maps.size();
  while (first > 0 && a->maps[first - 1].offset >= cut) --first;   // mappings starting at or beyond the cut
  DeviceGuard g(a->device);
  return drop_tail(a, first, freed);
}

int kvt_vmm_backed(void* arena, uint64_t* bytes, uint64_t* reserved, uint64_t* n_mappings) {
  if (arena == nullptr) return KVT_EINVAL;
  Arena* a = static_cast<Arena*>(arena);
  std::lock_guard<std::mutex> lk(a->mu);
  if (bytes) *bytes = a->backed;
  if (reserved) *reserved = a->reserved;
  if (n_mappings) *n_mappings = a->maps.size();
  return KVT_OK;
}

int kvt_vmm_destroy(void* arena) {
  if (arena == nullptr) return KVT_OK;
  Arena* a = static_cast<Arena*>(arena);
  int st;
  {
    std::lock_guard<std::mutex> lk(a->mu);
    DeviceGuard g(a->device);
    st = drop_tail(a, 0, nullptr);
    if (st == KVT_OK && hipMemAddressFree(a->base, a->reserved) != hipSuccess) st = KVT_EHIP;
  }
  if (st == KVT_OK) delete a;   // on failure the arena stays valid (and leaks) rather than dangling
  return st;
}

}  // extern "C"
