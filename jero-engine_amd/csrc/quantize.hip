// quantize.hip -- Q8 activation quantization on gfx950.
//
// Replaces repack::QuantizedActQ8::quantize (src/weights.rs:1416-1417) and the activation
// quantization inside vec_dot_* (src/gemma.rs:73-86).
//   ACT_Q8 (for Q8_0 / Q4_0 weights): 32-element blocks, f32 d = amax/127 and
//     q = rint(x * (1/d)); d stays f32 (the reference's golden llama Q8_0 logits are only
//     reproduced with an f32 activation scale).
//   Q8_K (for Q4_K / Q6_K weights): ggml's format; the signed element of largest
//     magnitude (first one on ties) sets iscale = -127/max, q = min(127, rint(iscale x)),
//     d = 1/iscale, bsums = sums of 16 consecutive q.
// Both are bit-exact against the CPU oracle: the ops are one IEEE division, one multiply
// and one round-half-even conversion per element, with no contraction possible.
#include "quantize.h"
#include "runtime.h"
#include "jero_common.h"

namespace jero {

// One 32-lane half-wave per block, one element per lane.
__global__ void __launch_bounds__(256) quant_act_q8_kernel(const float* __restrict__ x, int64_t nblocks,
                                                           uint8_t* __restrict__ q) {
  int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t blk = gid >> 5;
  int l = threadIdx.x & 31;
  bool ok = blk < nblocks;
  float v = ok ? x[blk * 32 + l] : 0.0f;
  float a = fabsf(v);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, kWave));
  if (!ok) return;
  float d = a / 127.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  int qi = int(__builtin_rintf(v * id));
  uint8_t* ob = q + blk * 36;
  ob[4 + l] = uint8_t(int8_t(qi));
  if (l == 0) *reinterpret_cast<float*>(ob) = d;
}

__global__ void __launch_bounds__(256) quant_q8k_kernel(const float* __restrict__ x, int64_t nblocks,
                                                        uint8_t* __restrict__ q) {
  int64_t blk = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  int lane = threadIdx.x & 63;
  if (blk >= nblocks) return;
  const float4 v = reinterpret_cast<const float4*>(x + blk * 256)[lane];
  const float e[4] = {v.x, v.y, v.z, v.w};
  q8k_block_wave(e, lane, q + blk * 292);
}

int launch_quantize_act(int act_quant, const float* x, int64_t m, int64_t k, void* q, hipStream_t stream) {
  if (act_quant == JERO_ACT_Q8) {
    int64_t nb = m * (k / 32);
    int64_t threads = nb * 32;
    dim3 grid(unsigned((threads + 255) / 256));
    hipLaunchKernelGGL(quant_act_q8_kernel, grid, dim3(256), 0, stream, x, nb, static_cast<uint8_t*>(q));
  } else {
    int64_t nb = m * (k / 256);
    dim3 grid(unsigned((nb * 64 + 255) / 256));
    hipLaunchKernelGGL(quant_q8k_kernel, grid, dim3(256), 0, stream, x, nb, static_cast<uint8_t*>(q));
  }
  return check_launch("quantize_act");
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_quantize_act(int act_quant, const float* x_dev, int64_t m, int64_t k, void* q_dev,
                                     void* stream) {
  if (act_quant != JERO_ACT_Q8 && act_quant != JERO_Q8_K)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "quantize_act: activation format must be ACT_Q8 or Q8_K");
  if (!x_dev || !q_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "quantize_act: null pointer");
  if (m <= 0 || k <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "quantize_act: empty input");
  if (row_bytes(act_quant, k) < 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "quantize_act: k=" + std::to_string(k) + " is not a multiple of the block");
  if (!aligned4(q_dev) || (reinterpret_cast<uintptr_t>(x_dev) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "quantize_act: x must be 16-byte and q 4-byte aligned");
  return launch_quantize_act(act_quant, x_dev, m, k, q_dev, static_cast<hipStream_t>(stream));
}
