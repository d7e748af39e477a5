// runtime.hip -- jero_hip_init / errors / shape helpers of the C ABI.
#include "runtime.h"

#include <mutex>
#include <vector>

#include "jero_common.h"

namespace jero {

static thread_local std::string g_last_error;

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int check_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return JERO_OK;
  return fail(JERO_ERR_DEVICE, std::string(where) + ": " + hipGetErrorString(e));
}

int check_launch(const char* where) { return check_hip(hipGetLastError(), where); }

int64_t row_bytes(int quant, int64_t n) {
  FmtInfo f = fmt_info(quant);
  if (f.block_elems <= 0 || n < 0 || n % f.block_elems) return -1;
  return (n / f.block_elems) * f.block_bytes;
}

int act_format(int weight_quant) {
  switch (weight_quant) {
    case JERO_Q8_0:
    case JERO_Q4_0: return JERO_ACT_Q8;
    case JERO_Q4_K:
    case JERO_Q4_K_R:
    case JERO_Q6_K:
    case JERO_Q6_K_R: return JERO_Q8_K;
    case JERO_F32:
    case JERO_F16:
    case JERO_BF16: return JERO_F32;  // the f32 input, unquantized
    default: return -1;
  }
}

bool is_weight_quant(int quant) { return act_format(quant) >= 0; }

static std::mutex g_mu;
static std::vector<DeviceInfo> g_info;
static std::vector<std::pair<void*, size_t>> g_ws;

const DeviceInfo& device_info() {
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_info.size() <= dev) g_info.resize(dev + 1);
  DeviceInfo& d = g_info[dev];
  if (d.device < 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
      d.cus = cus;
    d.device = dev;
  }
  return d;
}

int workspace(size_t bytes, void** ptr) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1, {nullptr, 0});
  auto& ws = g_ws[dev];
  if (ws.second < bytes) {
    if (ws.first) {
      // the old buffer may still be read by enqueued work
      rc = check_hip(hipDeviceSynchronize(), "workspace sync");
      if (rc) return rc;
      (void)hipFree(ws.first);
      ws = {nullptr, 0};
    }
    size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess)
      return fail(JERO_ERR_INSUFFICIENT_MEMORY, "workspace hipMalloc of " + std::to_string(want) + " bytes failed");
    ws = {p, want};
  }
  *ptr = ws.first;
  return JERO_OK;
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_init(int device) {
  int n = 0;
  int rc = check_hip(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (rc) return rc;
  if (device < 0 || device >= n)
    return fail(JERO_ERR_INVALID_ARGUMENT, "device " + std::to_string(device) + " out of range (" +
                                               std::to_string(n) + " devices)");
  rc = check_hip(hipSetDevice(device), "hipSetDevice");
  if (rc) return rc;
  (void)device_info();
  return JERO_OK;
}

extern "C" const char* jero_hip_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* jero_hip_status_name(int status) {
  switch (status) {
    case JERO_OK: return "Ok";
    case JERO_ERR_CAPABILITY_MISMATCH: return "CapabilityMismatch";
    case JERO_ERR_INSUFFICIENT_MEMORY: return "InsufficientLockableMemory";
    case JERO_ERR_CONTEXT_LENGTH_EXCEEDED: return "ContextLengthExceeded";
    case JERO_ERR_TENSOR_BOUNDS: return "TensorBoundsError";
    case JERO_ERR_ROUTING_UNAVAILABLE: return "RoutingUnavailable";
    case JERO_ERR_DEVICE: return "DeviceError";
    case JERO_ERR_INVALID_ARGUMENT: return "InvalidArgument";
    default: return "Unknown";
  }
}

extern "C" int64_t jero_hip_row_bytes(int quant, int64_t n) { return row_bytes(quant, n); }

extern "C" int jero_hip_act_format(int weight_quant) { return act_format(weight_quant); }
