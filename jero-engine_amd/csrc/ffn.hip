// ffn.hip -- the dense SwiGLU FFNs that dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) runs
// beside or instead of the routed experts, on one token row:
//   * the shared expert (run_single_swiglu_expert, :748-771, called at :860-871), and
//   * a layer without a router (run_dense_swiglu_ffn, :696-727, called at :873-880), each of its
//     three projections project_or_deterministic_slice (src/gemma.rs:841-860).
// Both are r = down(silu(gate x) * up x); y = (accumulate ? y : 0) + r, the reference's
// `out.fill(0.0)` followed by `*dst += src` over the result.  The projections run the GEMV kernels
// of jero_hip_vec_dot (the activation quantized to the weight format's blocks first), the
// deterministic fallback and SwiGLU the decode step's kernels.
#include <string>

#include "decode.h"
#include "gemv.h"
#include "jero_common.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {
namespace {

// y[i] = (acc ? y[i] : 0) + r[i]: one f32 addition per element.
__global__ void __launch_bounds__(256) ffn_add_kernel(float* __restrict__ y, const float* __restrict__ r, int64_t n,
                                                      int acc) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float base = acc ? y[i] : 0.0f;
  y[i] = base + r[i];
}

constexpr size_t kAlign = 256;
size_t up256(size_t b) { return (b + kAlign - 1) & ~(kAlign - 1); }
// bytes of any activation-block row of n elements (Q8_K: 292 per 256, ACT_Q8: 36 per 32)
size_t act_bound(int64_t n) { return size_t(n / 32 + 1) * 36 + size_t(n / 256 + 1) * 292; }

size_t ffn_ws_bytes(int64_t H, int64_t F) {
  return up256(sizeof(float) * size_t(2 * F)) + up256(sizeof(float) * size_t(F)) + up256(sizeof(float) * size_t(H)) +
         up256(act_bound(H > F ? H : F));
}

// y[n_out] = W x[n_in] for an f32 x (jero_hip_vec_dot's path): checked, x quantized into xq first
// unless W is an f32-input format.
int gemv_f32in(const jero_hip_tensor& w, const float* x, int64_t n_in, int64_t n_out, float* y, void* xq,
               hipStream_t s, const char* what) {
  const int act = act_format(w.quant);
  int rc = check_matvec_args(w.quant, w.dev, w.bytes, n_in, n_out, x, y);
  if (rc) return fail(rc, std::string("swiglu_ffn: ") + what + ": " + jero_hip_last_error());
  if (act == JERO_F32) return launch_matvec(w.quant, w.dev, n_in, n_out, x, y, nullptr, s);
  if ((rc = launch_quantize_act(act, x, 1, n_in, xq, s))) return rc;
  return launch_matvec(w.quant, w.dev, n_in, n_out, xq, y, nullptr, s);
}

bool usable(const jero_hip_tensor* t) { return t && t->dev; }

}  // namespace
}  // namespace jero

using namespace jero;

extern "C" size_t jero_hip_swiglu_ffn_workspace_bytes(int64_t hidden, int64_t ffn) {
  if (hidden <= 0) return 0;
  return ffn_ws_bytes(hidden, ffn < 4 ? 4 : ffn);
}

extern "C" int jero_hip_swiglu_ffn(int mode, const float* x_dev, int64_t hidden, int64_t ffn,
                                   const jero_hip_tensor* gate, const jero_hip_tensor* up,
                                   const jero_hip_tensor* down, int accumulate, float* y_dev, void* workspace_dev,
                                   size_t workspace_bytes, void* stream) {
  if (!x_dev || !y_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "swiglu_ffn: null pointer");
  if (mode != JERO_FFN_SHARED_EXPERT && mode != JERO_FFN_DENSE)
    return fail(JERO_ERR_INVALID_ARGUMENT, "swiglu_ffn: mode " + std::to_string(mode));
  if (hidden <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "swiglu_ffn: empty input");
  if (reinterpret_cast<uintptr_t>(x_dev) & 15u) return fail(JERO_ERR_INVALID_ARGUMENT, "swiglu_ffn: x must be 16-byte aligned");
  const int64_t H = hidden;
  const int64_t ffn4 = ffn > 4 ? ffn : 4;
  int64_t F = ffn4;
  if (mode == JERO_FFN_SHARED_EXPERT) {
    if (!usable(gate) || !usable(up) || !usable(down))
      return fail(JERO_ERR_INVALID_ARGUMENT, "swiglu_ffn: the shared expert needs its gate, up and down tensors");
    // run_single_swiglu_expert's eff_ffn (src/qwen_deepseek.rs:757-762)
    if (gate->n_elements > 0 && gate->n_elements % H == 0) F = gate->n_elements / H;
  }
  const size_t need = ffn_ws_bytes(H, F);
  void* ws = workspace_dev;
  int rc;
  if (ws) {
    if (workspace_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "swiglu_ffn: workspace of " + std::to_string(workspace_bytes) +
                                              " bytes, need " + std::to_string(need));
    if (reinterpret_cast<uintptr_t>(ws) & (kAlign - 1))
      return fail(JERO_ERR_INVALID_ARGUMENT, "swiglu_ffn: workspace must be 256-byte aligned");
  } else if ((rc = workspace(need, &ws))) {
    return rc;
  }
  uint8_t* p = static_cast<uint8_t*>(ws);
  float* gu = reinterpret_cast<float*>(p);  // gate [F] then up [F]
  p += up256(sizeof(float) * size_t(2 * F));
  float* act = reinterpret_cast<float*>(p);
  p += up256(sizeof(float) * size_t(F));
  float* r = reinterpret_cast<float*>(p);
  p += up256(sizeof(float) * size_t(H));
  void* xq = p;
  hipStream_t s = static_cast<hipStream_t>(stream);

  // project_or_deterministic_slice uses a tensor only when it holds exactly out_len * in_len
  // elements; run_single_swiglu_expert always uses it (matvec_any checks its bytes)
  auto proj = [&](const jero_hip_tensor* w, const float* in, int64_t in_len, int64_t out_len, float scale, float* out,
                  const char* what) -> int {
    if (mode == JERO_FFN_SHARED_EXPERT || (usable(w) && w->n_elements == out_len * in_len))
      return gemv_f32in(*w, in, in_len, out_len, out, xq, s, what);
    return launch_det_proj(in, in_len, nullptr, 0.f, scale, out, out_len, false, s);
  };
  if ((rc = proj(gate, x_dev, H, F, 0.5f, gu, "gate")) || (rc = proj(up, x_dev, H, F, 0.25f, gu + F, "up")) ||
      (rc = launch_swiglu(gu, F, act, s)) || (rc = proj(down, act, F, H, 0.125f, r, "down")))
    return rc;
  hipLaunchKernelGGL(ffn_add_kernel, dim3(unsigned((H + 255) / 256)), dim3(256), 0, s, y_dev, r, H, accumulate ? 1 : 0);
  return check_launch("swiglu_ffn add");
}
