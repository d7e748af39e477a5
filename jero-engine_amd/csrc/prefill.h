// prefill.h -- row kernels of the batched prefill (jero_hip_model_prefill).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jero {

// X[t] = embed_token(tokens[t]) (device array), t < n: a row of the `rows` rows of rb bytes at w,
// or the deterministic row of a token past them.
int launch_embed_rows(int quant, const void* w, int64_t rb, int64_t rows, int H, const int32_t* tokens, int64_t n,
                      float* X, hipStream_t s);
// XN[t] = RMSNorm(X[t]) * w, rows of H floats.
int launch_rmsnorm_rows(const float* X, int64_t n, int64_t H, const float* w, float eps, float* XN, hipStream_t s);
// Per token t < n (position pos0 + t): QK-norm (when given) and RoPE of its q heads (row t at q +
// t q_stride) and k heads (k + t k_stride), in place, the k and v heads (v + t v_stride, plus v2 +
// t v_stride when v2 is given: the second K half of a split V projection) appended to ring slot
// (pos0 + t) % capacity, and the RoPE table of the token into rope_cs[t][hd].
int launch_qk_rope_rows(float* q, int64_t q_stride, float* k, int64_t k_stride, const float* v, int64_t v_stride,
                        const float* v2, int64_t n, int nq, int nkv, int hd, const float* q_norm, const float* k_norm, float eps,
                        int64_t pos0, float theta, float* rope_cs, void* k_ring, void* v_ring, bool kv_f16,
                        int64_t capacity, hipStream_t s);
// act[t][i] = silu(g[t][i]) * u[t][i], act rows of F floats.
int launch_swiglu_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* act, int64_t n,
                       int64_t F, hipStream_t s);
// x[i] += d[i], i < count.
int launch_add_rows(float* x, const float* d, int64_t count, hipStream_t s);
// Per row t < n: X[t] += D[t] (+ D2[t], summed first, when given) when D is given, then the Q8_K
// blocks of RMSNorm(X[t]) * w into Q (rows of H / 256 blocks), bit for bit what launch_add_rows,
// launch_rmsnorm_rows and launch_quantize_act make; XN[t] (when given) receives the normalised
// row.  H % 256 == 0, H <= 8192.
int launch_add_rmsnorm_q8k_rows(float* X, const float* D, const float* D2, int64_t n, int64_t H, const float* w,
                                float eps, float* XN, void* Q, hipStream_t s);
// The Q8_K blocks of act[t] = silu(g[t]) * u[t] into Q, bit for bit what launch_swiglu_rows and
// launch_quantize_act make; act (when given) receives the f32 rows.  F % 256 == 0.
int launch_swiglu_q8k_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* act, int64_t n,
                           int64_t F, void* Q, hipStream_t s);

}  // namespace jero
