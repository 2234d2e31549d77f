// Host-side caches of per-device and per-shape launch facts.
//
// Every entry point used to ask the runtime for the CU count and a kernel's
// occupancy, and to rebuild the single-pass work map (a sort of up to 1024
// entries), on every call.  These depend only on the device and the problem
// shape, so they are computed once and kept for the life of the process.
// Each cache is guarded by its own mutex; entries are never modified after
// insertion, and lookups return copies, so concurrent calls are safe.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <utility>

namespace fdp {
namespace host {

constexpr int kMaxDevices = 64;

// Number of compute units of the current device (256 on MI355X).
inline int device_cus() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < kMaxDevices) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 256, v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
    cus = v;
  if (dev < kMaxDevices) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Resident workgroups per CU of kernel `fn` with `threads` threads and
// `dyn_lds` bytes of dynamic LDS on the current device (0 on failure).
inline int occupancy(const void* fn, int threads, size_t dyn_lds) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, size_t>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  const auto key = std::make_tuple(dev, fn, threads, dyn_lds);
  {
    std::lock_guard<std::mutex> g(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, threads, dyn_lds) != hipSuccess) occ = 0;
  std::lock_guard<std::mutex> g(mu);
  cache.emplace(key, occ);
  return occ;
}

// A bounded map from a shape key to a plain-data value, computed on first use.
template <class Key, class Value, size_t kCap = 512>
class ShapeCache {
 public:
  template <class Make>
  Value get(const Key& k, Make make) {
    {
      std::lock_guard<std::mutex> g(mu_);
      const auto it = map_.find(k);
      if (it != map_.end()) return it->second;
    }
    Value v = make();
    std::lock_guard<std::mutex> g(mu_);
    if (map_.size() >= kCap) map_.clear();
    map_.emplace(k, v);
    return v;
  }

 private:
  std::mutex mu_;
  std::map<Key, Value> map_;
};

}  // namespace host
}  // namespace fdp
