// decode.h -- fused decode-step kernels and their launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jero {

constexpr int kDecodeThreads = 512;     // 8 waves per workgroup
constexpr int kDecodeBlocksPerCU = 2;   // persistent grid: workgroups per CU
constexpr int kDecodeMaxActBlocks = 8;  // activation blocks per wave in the prologue
constexpr int kDecodeMaxLongActBytes = 60 * 1024;  // LDS activation of the long-row kernel

enum { kOutStore = 0, kOutResid = 1, kOutSwiglu = 2, kOutArgmax = 3 };

struct DGemvArgs {
  const uint8_t* w;   // weight rows (GGUF layout, or Q4_K_R / Q6_K_R planes)
  int64_t rb;         // bytes per row (GGUF layouts)
  int U;              // units per row
  int64_t N;          // rows of the tensor
  int64_t n_groups;   // row groups (set by the launcher)
  const float* x;     // f32 input [K] (16-byte aligned)
  const float* norm_w;  // RMSNorm weight [K] or null
  float eps;
  int K;
  float* y;           // output (store / residual target / SwiGLU act / logits)
  int64_t half;       // SwiGLU: rows [0, half) gate, [half, 2 half) up
  float* amax_v;      // argmax partials per workgroup
  int64_t* amax_i;
  int max_blocks;     // 0: grid capped at kDecodeBlocksPerCU workgroups per CU
  // second tensor of a two-tensor launch (launch_dgemv_dual)
  const uint8_t* w2;
  int64_t rb2;
  int64_t N2;
  // debug trace (null: off), written by workgroup 0: the f32 values the prologue quantized
  // (after RMSNorm), the activation blocks it built, and the raw gate|up outputs of SwiGLU
  float* tr_xn;
  uint8_t* tr_q8;
  float* tr_gu;
};

// Enqueues the fused GEMV; *blocks (if given) receives the workgroups launched, which is the
// number of argmax partials an argmax launch leaves in amax_v / amax_i.
int launch_dgemv(int quant, int out_mode, const DGemvArgs& a, hipStream_t s, int* blocks = nullptr);
// rmsnorm(x) . [W1; W2] into y[0, N + N2) for two K-quant tensors of different formats sharing
// n_in = K <= 4096 (Q4_K_R with Q6_K_R, either order): one launch, one prologue.
int launch_dgemv_dual(int quant1, int quant2, const DGemvArgs& a, hipStream_t s);
// Longest row the register-resident fused decode GEMV takes for a weight format; rows up to
// dgemv_long_max_k run the long-row variant.
int dgemv_max_k(int quant);
int dgemv_long_max_k(int quant);
// hidden = embed_token(*token): a row of the `rows` rows of rb bytes at w (null: no token_embd), or
// the deterministic row of a token past them; also the step's RoPE table rope_cs[hd/2][cos, sin].
int launch_embed(int quant, const void* w, int64_t rb, int H, int64_t rows, const int32_t* token, float* out,
                 const int64_t* pos, float theta, int hd, float* rope_cs, hipStream_t s);
// read_f32_weight_or_default (src/qwen_deepseek.rs:491-519) of a norm weight into out[len] (raw
// null: absent; deq: dequantize the first len elements of a non-F32 tensor).
int launch_norm_weight(int quant, const void* raw, int64_t n_el, int64_t len, bool deq, float* out, hipStream_t s);
// xn[H] = RMSNorm(x) * nw for an LM head read with an f32 input.
int launch_head_norm(const float* x, const float* nw, float eps, int64_t H, float* xn, hipStream_t s);
// project_lm_head's logits [start, L) that no head row gives (src/qwen_deepseek.rs:584-632): mode 0
// rows past the head's `start` rows (xn[i % H] * 0.05), mode 1 no usable head (start 0; tanh of
// the sum of xn / 16 + xn[i % H] * 0.1 + (i % 13) * 0.01).  head_tail_blocks(start, L) workgroups,
// each writing its argmax partial at pv / pi (unless null).
constexpr int64_t kHeadTailRows = 4096;
int head_tail_blocks(int64_t start, int64_t L);
int launch_head_tail(const float* x, const float* nw, float eps, int64_t H, int mode, int64_t start, int64_t L,
                     float* logits, float* pv, int64_t* pi, float* tr_xn, hipStream_t s);
// Per-workgroup (max, first index) partials of x[n] into pv / pi; returns their count (argmax_partials(n)),
// or -1 on a launch error.
int launch_argmax_partials(const float* x, int64_t n, float* pv, int64_t* pi, hipStream_t s);
// The greedy token from the head's per-workgroup partials; all-NaN logits set the sticky *status
// (token -1, position kept) instead of producing a token.
int launch_argmax_final(const float* v, const int64_t* idx, int n, int32_t* token, int64_t* pos, int32_t* status,
                        hipStream_t s);
// Standalone argmax_f32 of n floats into *out_idx (-1: empty or all NaN); pv / pi hold
// argmax_partials(n) partial pairs.
int argmax_partials(int64_t n);
int launch_argmax(const float* x, int64_t n, int64_t* out_idx, float* pv, int64_t* pi, hipStream_t s);
int launch_set_state(int32_t* token, int64_t* pos, int32_t* status, int32_t t, int64_t p, hipStream_t s);
// A projection whose tensor the model lacks (project_or_deterministic_slice, src/gemma.rs:841-860):
// y[i] (+)= in[i % len] * scale, in = x or RMSNorm(x) * norm_w.
// rows > 1: a batch of rows x_stride / y_stride floats apart.
int launch_det_proj(const float* x, int64_t len, const float* norm_w, float eps, float scale, float* y,
                    int64_t out_len, bool resid, hipStream_t s, int64_t rows = 1, int64_t x_stride = 0,
                    int64_t y_stride = 0);
// act[i] = silu(gu[i]) * gu[F + i] for gate | up rows computed apart.
int launch_swiglu(const float* gu, int64_t F, float* act, hipStream_t s);

}  // namespace jero
