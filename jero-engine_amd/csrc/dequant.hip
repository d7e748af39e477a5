// dequant.hip -- dequantize_token_row on gfx950 (src/qwen_deepseek.rs:514,569): GGUF rows
// to f32, one thread per output element.  Used for the embedding lookup of the decode step.
#include "dequant.h"

#include "jero_common.h"
#include "runtime.h"

namespace jero {

__global__ void __launch_bounds__(256) dequant_rows_kernel(int quant, const uint8_t* __restrict__ w, int64_t rb,
                                                           int64_t n_in, int64_t row0, int64_t total,
                                                           float* __restrict__ out) {
  int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= total) return;
  int64_t r = e / n_in, col = e % n_in;
  out[e] = dequant_elem(quant, w + (row0 + r) * rb, col);
}

int launch_dequant_rows(int quant, const void* w, int64_t n_in, int64_t row0, int64_t n_rows, float* out,
                        hipStream_t s) {
  int64_t total = n_rows * n_in;
  hipLaunchKernelGGL(dequant_rows_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, quant,
                     static_cast<const uint8_t*>(w), row_bytes(quant, n_in), n_in, row0, total, out);
  return check_launch("dequantize_rows");
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_dequantize_rows(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t row0,
                                        int64_t n_rows, float* out_dev, void* stream) {
  if (!is_weight_quant(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "dequantize_rows: unsupported quantization " + std::to_string(quant));
  if (!w_dev || !out_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "dequantize_rows: null pointer");
  if (n_in <= 0 || n_rows <= 0 || row0 < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "dequantize_rows: empty range");
  int64_t rb = row_bytes(quant, n_in);
  if (rb < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "dequantize_rows: n_in is not a multiple of the block");
  if (uint64_t(rb) * uint64_t(row0 + n_rows) > w_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "dequantize_rows: rows [" + std::to_string(row0) + ", " +
                                            std::to_string(row0 + n_rows) + ") beyond the tensor");
  if (!aligned4(w_dev) || !aligned4(out_dev))
    return fail(JERO_ERR_INVALID_ARGUMENT, "dequantize_rows: pointers must be 4-byte aligned");
  return launch_dequant_rows(quant, w_dev, n_in, row0, n_rows, out_dev, static_cast<hipStream_t>(stream));
}
