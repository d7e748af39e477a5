// dequant.h -- row dequantization launcher.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jero {

int launch_dequant_rows(int quant, const void* w, int64_t n_in, int64_t row0, int64_t n_rows, float* out,
                        hipStream_t s);

}  // namespace jero
