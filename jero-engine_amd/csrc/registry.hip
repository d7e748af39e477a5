// registry.hip -- device copies of host (mmaped) weight tensors, uploaded once.
//
// The reference's kernels read weights straight from the mmaped GGUF bytes that
// LockedModelWeights owns (src/weights.rs:729-734), and repacked copies are cached per tensor
// by RepackedTensorStore (src/weights.rs:189-277).  Here a tensor's bytes are copied to HBM on
// its first registration and found again by host address: registering the same range again is
// free, and any sub-range (a slice_rows / slice_expert view) of a registered tensor maps to the
// matching device address, so a binding can hand the GPU the view the reference's callers pass.
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "jero_common.h"
#include "runtime.h"

namespace jero {
namespace {

struct Region {
  size_t nbytes;
  int device;
  void* dev;
  // the device allocation holding dev: one per tensor, or one per stack of tensors
  // (jero_hip_weights_register_stacked), freed with the last region that holds it
  std::shared_ptr<void> mem;
};

std::shared_ptr<void> own(void* dev) {
  return std::shared_ptr<void>(dev, [](void* q) { (void)hipFree(q); });
}


std::mutex g_mu;
// keyed by (device, host start address)
std::map<std::pair<int, uintptr_t>, Region> g_regions;

int current_device(int* dev) { return check_hip(hipGetDevice(dev), "hipGetDevice"); }

// Registered region of `device` holding [p, p + n), or nullptr.
const Region* find_region(int device, uintptr_t p, size_t n, uintptr_t* start) {
  auto it = g_regions.upper_bound({device, p});
  if (it == g_regions.begin()) return nullptr;
  --it;
  if (it->first.first != device) return nullptr;
  const uintptr_t s = it->first.second;
  if (p < s || p + n > s + it->second.nbytes) return nullptr;
  *start = s;
  return &it->second;
}

// Does [p, p + n) overlap a registered range of `device`?  (g_mu held)
bool overlaps(int device, uintptr_t p, size_t n) {
  auto it = g_regions.lower_bound({device, p});
  if (it != g_regions.end() && it->first.first == device && it->first.second < p + n) return true;
  if (it != g_regions.begin()) {
    auto pr = std::prev(it);
    if (pr->first.first == device && pr->first.second + pr->second.nbytes > p) return true;
  }
  return false;
}

}  // namespace
}  // namespace jero

using namespace jero;

extern "C" int jero_hip_weights_register(const void* host, size_t nbytes, const void** dev_out) {
  if (!host || !dev_out) return fail(JERO_ERR_INVALID_ARGUMENT, "weights_register: null pointer");
  if (nbytes == 0) return fail(JERO_ERR_TENSOR_BOUNDS, "weights_register: empty tensor");
  int device = 0;
  int rc = current_device(&device);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  const uintptr_t p = reinterpret_cast<uintptr_t>(host);
  uintptr_t start = 0;
  if (const Region* r = find_region(device, p, nbytes, &start)) {
    *dev_out = static_cast<const uint8_t*>(r->dev) + (p - start);
    return JERO_OK;
  }
  // a new range must not overlap an existing one partially
  if (overlaps(device, p, nbytes))
    return fail(JERO_ERR_TENSOR_BOUNDS, "weights_register: range overlaps a registered tensor");
  void* dev = nullptr;
  if (hipMalloc(&dev, nbytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(JERO_ERR_INSUFFICIENT_MEMORY, "weights_register: no device memory for " + std::to_string(nbytes) +
                                                  " bytes");
  }
  rc = check_hip(hipMemcpy(dev, host, nbytes, hipMemcpyHostToDevice), "weights_register upload");
  if (rc) {
    (void)hipFree(dev);
    return rc;
  }
  g_regions[{device, p}] = Region{nbytes, device, dev, own(dev)};
  *dev_out = dev;
  return JERO_OK;
}

extern "C" int jero_hip_weights_register_stacked(const void* const* hosts, size_t nbytes, int64_t n,
                                                 const void** dev_out) {
  if (!hosts || !dev_out) return fail(JERO_ERR_INVALID_ARGUMENT, "weights_register_stacked: null pointer");
  if (nbytes == 0 || n <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "weights_register_stacked: empty tensors");
  for (int64_t e = 0; e < n; e++)
    if (!hosts[e]) return fail(JERO_ERR_INVALID_ARGUMENT, "weights_register_stacked: null tensor " + std::to_string(e));
  int device = 0;
  int rc = current_device(&device);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  // registered before as this same stack: every tensor at its place in one allocation
  int64_t found = 0;
  const Region* first = nullptr;
  bool same_stack = true;
  for (int64_t e = 0; e < n; e++) {
    const uintptr_t p = reinterpret_cast<uintptr_t>(hosts[e]);
    uintptr_t start = 0;
    const Region* r = find_region(device, p, nbytes, &start);
    if (!r) {
      if (overlaps(device, p, nbytes)) same_stack = false;
      continue;
    }
    found++;
    if (e == 0) first = r;
    if (start != p || r->nbytes != nbytes || !first ||
        static_cast<const uint8_t*>(r->dev) != static_cast<const uint8_t*>(first->dev) + size_t(e) * nbytes ||
        r->mem != first->mem)
      same_stack = false;
  }
  if (found == n && same_stack) {
    *dev_out = first->dev;
    return JERO_OK;
  }
  if (found > 0 || !same_stack)
    return fail(JERO_ERR_TENSOR_BOUNDS, "weights_register_stacked: some of the tensors are registered apart");
  for (int64_t e = 0; e < n; e++)
    for (int64_t f = e + 1; f < n; f++) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(hosts[e]), b = reinterpret_cast<uintptr_t>(hosts[f]);
      if (a < b + nbytes && b < a + nbytes)
        return fail(JERO_ERR_TENSOR_BOUNDS, "weights_register_stacked: tensors " + std::to_string(e) + " and " +
                                                std::to_string(f) + " overlap");
    }
  void* dev = nullptr;
  if (hipMalloc(&dev, nbytes * size_t(n)) != hipSuccess) {
    (void)hipGetLastError();
    return fail(JERO_ERR_INSUFFICIENT_MEMORY, "weights_register_stacked: no device memory for " +
                                                  std::to_string(nbytes * size_t(n)) + " bytes");
  }
  std::shared_ptr<void> mem = own(dev);
  for (int64_t e = 0; e < n; e++) {
    rc = check_hip(hipMemcpy(static_cast<uint8_t*>(dev) + size_t(e) * nbytes, hosts[e], nbytes, hipMemcpyHostToDevice),
                   "weights_register_stacked upload");
    if (rc) return rc;  // mem frees the allocation
  }
  for (int64_t e = 0; e < n; e++)
    g_regions[{device, reinterpret_cast<uintptr_t>(hosts[e])}] =
        Region{nbytes, device, static_cast<uint8_t*>(dev) + size_t(e) * nbytes, mem};
  *dev_out = dev;
  return JERO_OK;
}

extern "C" int jero_hip_weights_lookup(const void* host, size_t nbytes, const void** dev_out) {
  if (!host || !dev_out) return fail(JERO_ERR_INVALID_ARGUMENT, "weights_lookup: null pointer");
  int device = 0;
  int rc = current_device(&device);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  const uintptr_t p = reinterpret_cast<uintptr_t>(host);
  uintptr_t start = 0;
  const Region* r = find_region(device, p, nbytes, &start);
  if (!r) return fail(JERO_ERR_TENSOR_BOUNDS, "weights_lookup: range is not inside a registered tensor");
  *dev_out = static_cast<const uint8_t*>(r->dev) + (p - start);
  return JERO_OK;
}

extern "C" int jero_hip_weights_release_all(void) {
  int device = 0;
  int rc = current_device(&device);
  if (rc) return rc;
  rc = check_hip(hipDeviceSynchronize(), "weights_release_all sync");
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  for (auto it = g_regions.begin(); it != g_regions.end();) {
    if (it->first.first == device) {
      it = g_regions.erase(it);  // the last region of an allocation frees it
    } else {
      ++it;
    }
  }
  return JERO_OK;
}

extern "C" int jero_hip_weights_release(const void* host, size_t nbytes) {
  if (!host) return fail(JERO_ERR_INVALID_ARGUMENT, "weights_release: null pointer");
  const uintptr_t lo = reinterpret_cast<uintptr_t>(host), hi = lo + nbytes;
  int cur = 0;
  int rc = current_device(&cur);
  if (rc) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  std::vector<int> synced;
  for (auto it = g_regions.begin(); it != g_regions.end();) {
    const uintptr_t s = it->first.second;
    if (s < lo || s + it->second.nbytes > hi) {
      ++it;
      continue;
    }
    const int d = it->first.first;
    // enqueued work on that device may still read the copy
    if (std::find(synced.begin(), synced.end(), d) == synced.end()) {
      if (d != cur) (void)hipSetDevice(d);
      rc = check_hip(hipDeviceSynchronize(), "weights_release sync");
      if (d != cur) (void)hipSetDevice(cur);
      if (rc) return rc;
      synced.push_back(d);
    }
    it = g_regions.erase(it);  // the last region of an allocation frees it
  }
  return JERO_OK;
}

extern "C" int jero_hip_sync(void* stream) {
  return check_hip(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "stream synchronize");
}
