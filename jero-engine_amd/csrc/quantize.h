// quantize.h -- activation quantization launchers shared by the entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jero {

// x: m rows of k f32 (16-byte aligned); q: m * row_bytes(act_quant, k) bytes.
int launch_quantize_act(int act_quant, const float* x, int64_t m, int64_t k, void* q, hipStream_t stream);

}  // namespace jero
