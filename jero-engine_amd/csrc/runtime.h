// runtime.h -- host-side helpers of libjero_hip: error reporting, argument checks,
// per-device state.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "jero_hip.h"

namespace jero {

// Records `msg` as the calling thread's last error and returns `status`.
int fail(int status, const std::string& msg);
// Maps a HIP error to JERO_ERR_DEVICE (recording where it came from); JERO_OK if none.
int check_hip(hipError_t e, const char* where);
// Checks the launch that was just enqueued.
int check_launch(const char* where);

int64_t row_bytes(int quant, int64_t n);
int act_format(int weight_quant);
bool is_weight_quant(int quant);

// Device properties needed by the launch heuristics (cached per device).
struct DeviceInfo {
  int device = -1;
  int cus = 256;
};
const DeviceInfo& device_info();

// Library-owned per-device workspace (grown with hipMalloc, kept until exit).
int workspace(size_t bytes, void** ptr);

inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace jero
