/*
 * oracle.h -- CPU restatement of jero-engine's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (libjero_hip.so) never calls it.
 *
 * The reference keeps every hot-path arithmetic routine in the un-vendored crate
 * jero-kernels-rvv @ 93a778ef690ac2171aab915f7b58daf5d8bbfe79 (Cargo.lock:456-461),
 * so this file restates:
 *   - the public GGUF/ggml block formats Q8_0, Q4_0, Q4_K, Q6_K and the Q8_K
 *     activation format (closed forms);
 *   - the reference's Q8 activation format for Q8_0/Q4_0 weights, pinned by the
 *     reference's golden fixture tests/fixtures/golden_parity/llama_authentic_q8_0.json:
 *     32-element blocks with an f32 scale d = amax/127, q = round(x/d);
 *   - the reference's call sites: matvec_any (src/gemma.rs:100-138), the per-quant
 *     dispatch (src/gemma.rs:66-95), select_top_k_experts (src/gemma.rs:362-442),
 *     dispatch_qwen3_moe_ffn / run_single_swiglu_expert (src/qwen_deepseek.rs:748-951),
 *     run_gqa_causal_with_cache_scaled (src/qwen_deepseek.rs:643-694),
 *     execute_token_standard_with_hidden (src/qwen_deepseek.rs:1239-1314),
 *     sample_greedy_argmax (src/engine.rs:1873-1895),
 *     the scalar reference model of tests/wave1_engine_regression_test.rs:680-712,945-1004.
 *
 * Parity pins (each checked by a test under tests/):
 *   formats + dequant   : reference KATs src/gemma.rs:1627-1662, byte facts
 *                         tests/wave1_engine_regression_test.rs:250-282, src/weights.rs:1208,
 *                         an independent numpy restatement (oracle/ref_numpy.py)
 *   Q8_0 vec_dot + ACT_Q8 quantizer + rmsnorm + interleaved RoPE + attention + SwiGLU:
 *                         the golden llama Q8_0 logits (16 values, |d| <= 1e-4)
 *   Q8_K quantizer      : ggml closed form, independent numpy restatement, invariants
 *   int32 partial sums  : brute force integer einsum (numpy), exact
 *   fp32 GEMV outputs   : f64 dequantize-then-dot brute force
 *   top-k routing       : reference KATs src/gemma.rs:1722-1740
 *   argmax              : reference KATs src/engine.rs:2677-2727
 *   int8 GEMM           : brute force integer matmul (numpy), exact
 *   int8 ForwardModel   : SplitMix64's published first outputs, isqrt against math.isqrt,
 *                         rmsnorm / attention closed forms, brute force numpy pieces, and the
 *                         prefill == token-by-token invariant of the whole forward
 */
#ifndef JERO_ORACLE_H
#define JERO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantization ids: GGUF/ggml type ids; JO_ACT_Q8 is the activation block format. */
enum {
  JO_F32 = 0,
  JO_F16 = 1,
  JO_BF16 = 30,
  JO_Q4_0 = 2,
  JO_Q8_0 = 8,
  JO_Q4_K = 12,
  JO_Q6_K = 14,
  JO_Q8_K = 15,
  JO_ACT_Q8 = 100
};

float jo_f16_to_f32(uint16_t h);
uint16_t jo_f32_to_f16(float f);

/* Elements per block and bytes per block of a format (0 if unknown). */
int64_t jo_block_elems(int quant);
int64_t jo_block_bytes(int quant);
/* Bytes of one row of n elements (-1 if n is not a multiple of the block). */
int64_t jo_row_bytes(int quant, int64_t n);
/* Activation format the dot product of a weight format consumes. */
int jo_act_format(int weight_quant);

/* Dequantize one row of n elements (dequantize_token_row). 0 ok, else -1. */
int jo_dequantize_row(int quant, const void *row, int64_t n, float *out);

/* Activation quantizers over m rows of k elements each. */
void jo_quantize_act_q8(const float *x, int64_t m, int64_t k, void *out);
void jo_quantize_q8_k(const float *x, int64_t m, int64_t k, void *out);
/* Dispatch on the activation format. */
void jo_quantize_act(int act_quant, const float *x, int64_t m, int64_t k, void *out);

/* Number of int32 partial sums per row of k elements for a weight format:
 * Q8_0/Q4_0: one per 32-block; Q4_K: one per 32-element sub-block; Q6_K: one per 16. */
int64_t jo_partials_per_row(int quant, int64_t k);

/* One row dot product: W-row (k elements) against the quantized activation.
 * Writes the exact int32 partial sums if partials != NULL.  Accumulates in f64. */
double jo_vec_dot_row(int quant, const void *wrow, int64_t k, const void *xq, int32_t *partials);

/* y[n] = W[n x k] . x.  Rows split in chunks of clamp(ceil(n/threads), 16, 2048) as in
 * matvec_any (src/gemma.rs:114-134); each row is reduced by one thread. */
int jo_matvec(int quant, const void *w, int64_t k, int64_t n, const void *xq, float *y, int threads);
/* Same over f32 input: quantizes x first (the reference vec_dot_* signature). */
int jo_vec_dot(int quant, const void *w, int64_t k, int64_t n, const float *x, float *y, int threads);
/* f64 brute force: dequantize weights and activations, dot in double. */
int jo_matvec_dequant_f64(int quant, const void *w, int64_t k, int64_t n, const void *xq, double *y);
/* Int32 partial sums of all rows: partials[n][jo_partials_per_row]. */
int jo_matvec_partials(int quant, const void *w, int64_t k, int64_t n, const void *xq, int32_t *partials);
/* Y[m][n] = sum over rows of X: row-by-row GEMV (the reference prefills token by token). */
int jo_gemm(int quant, const void *w, int64_t k, int64_t n, const void *xq, int64_t m, float *y, int threads);

/* Exact int8 GEMM: out[m][n] = sum_k x[m][k] * w[n][k] (ime::gemm_i8_* semantics). */
void jo_gemm_i8(const int8_t *x, int64_t m, const int8_t *w, int64_t n, int64_t k, int32_t *out);

/* gqa_causal_attention_f32: q [nq*hd], k/v [seq_len][nkv*hd]. */
int jo_gqa_attention(float *out, const float *q, const float *k, const float *v, int nq, int nkv,
                     int hd, int64_t seq_len, float scale);

void jo_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps);
/* Interleaved-pair RoPE, angle = pos / theta^(2i/hd) (tests/wave1_engine_regression_test.rs:698-712). */
void jo_rope_inplace(float *x, int64_t len, int hd, int64_t pos, float theta);
void jo_swiglu(float *out, const float *gate, const float *up, int64_t n);
/* First maximum, NaN skipped; -1 if empty or all NaN. */
int64_t jo_argmax(const float *x, int64_t n);
/* select_top_k_experts: writes k pairs; returns k (0 if empty). */
int jo_select_top_k(const float *logits, int64_t n, int top_k, int normalize, int32_t *idx, float *w);

/* One MoE expert FFN for one token: y = down(silu(gate x) * up x); weights are expert-local. */
int jo_swiglu_expert(int gate_quant, const void *gate, int up_quant, const void *up, int down_quant,
                     const void *down, int64_t hidden, int64_t ffn, const float *x, float *y);
/* dispatch_qwen3_moe_ffn for t tokens from router logits [t][E] and stacked expert
 * tensors (expert e = rows [e*ffn, (e+1)*ffn) of gate/up, rows [e*hidden, ...) of down). */
int jo_moe_ffn(const float *router_logits, int64_t t, int64_t n_experts, int top_k,
               int gate_quant, const void *gate, int up_quant, const void *up, int down_quant,
               const void *down, int64_t hidden, int64_t ffn, const float *x, float *y,
               int32_t *sel_idx, float *sel_w, int threads);

/* ---- decode step (execute_token_standard_with_hidden) ---- */
typedef struct jo_tensor {
  int quant;
  const void *data; /* GGUF bytes, row-major [rows][k] */
} jo_tensor;

typedef struct jo_layer {
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm; /* q_norm/k_norm NULL if absent */
  jo_tensor wq, wk, wv, wo, w_gate, w_up, w_down;
} jo_layer;

typedef struct jo_model {
  int64_t hidden, ffn, n_layers, vocab;
  int nq, nkv, hd;
  float eps, theta;
  int64_t kv_capacity; /* slots per layer in the K and V rings */
  jo_tensor tok_embd, output;
  const float *output_norm;
  const jo_layer *layers;
  int kv_f16; /* nonzero: the rings hold f16 values (each new K/V row rounded before it is attended) */
  /* Embedding and LM head as ModelWeights presents them (src/weights.rs:1097-1144):
   *   embd_rows   rows of `hidden` elements in tok_embd (num_elements / hidden; 0: no token_embd)
   *   out_in, out_rows   the head tensor's shape [out_in, out_rows] (`output`: output.weight, or
   *               token_embd.weight when output.weight is absent; out_rows 0: no head at all)
   *   logits_len  infer_logits_buffer_len (jo_logits_len) */
  int64_t embd_rows, out_in, out_rows, logits_len;
} jo_model;

/* read_f32_weight_or_default (src/qwen_deepseek.rs:491-519): out[len] = the weight's first len
 * values -- data NULL (absent): all `def`; F32: each of the n_elements stored values that is
 * finite, `def` for a non-finite value and past the tensor's end; another format with at least
 * len elements: row 0 (the first len elements) dequantized, all `def` if that fails (len not a
 * whole number of blocks, an unsupported format); fewer elements: all `def`. */
void jo_read_f32_weight_or_default(int quant, const void *data, int64_t n_elements, int64_t len, float def,
                                   float *out);
/* infer_logits_buffer_len (src/engine.rs:1781-1792): the head's rows when it has more than
 * vocab, a multiple of 64, at most 1024 past vocab; else vocab. */
int64_t jo_logits_len(int64_t vocab, int has_head, int64_t head_rows);
/* embed_token (src/qwen_deepseek.rs:558-582): row `token` of tok_embd dequantized when the
 * tensor has that row; else (token_embd absent or too short) the deterministic row
 * x[i] = ((token % 31) * 0.05 + 0.25) + (i % 7) * 0.01 in f32. */
int jo_embed_token(const jo_model *mdl, uint32_t token, float *x);

/* Intermediate values of one layer of the decode step (every pointer optional):
 *   xn_attn  rmsnorm(x) * attn_norm, the f32 input of the Q|K|V projections [hidden]
 *   q8_attn  its activation blocks in attn_q's activation format (Q8_K or ACT_Q8)
 *   qkv      the raw projections q | k | v [q_dim + 2 kv_dim]
 *   q_rope, k_rope   q and k after QK-norm and RoPE [q_dim], [kv_dim]
 *   attn     the attention output [q_dim];  q8_wo its activation blocks (attn_output's format)
 *   x_mid    the hidden state after the attention residual [hidden]
 *   xn_ffn, q8_ffn   the FFN input after RMSNorm and its activation blocks (ffn_gate's format)
 *   gu       the raw gate | up projections [2 ffn];  act  silu(gate) * up [ffn]
 *   q8_down  act's activation blocks (ffn_down's format) */
typedef struct jo_layer_trace {
  float *xn_attn;
  void *q8_attn;
  float *qkv, *q_rope, *k_rope, *attn;
  void *q8_wo;
  float *x_mid, *xn_ffn;
  void *q8_ffn;
  float *gu, *act;
  void *q8_down;
} jo_layer_trace;

/* The attention sublayer of layer L (src/qwen_deepseek.rs:1262-1275, run_dense_attention_sublayer_scaled
 * :984-1097): x += Wo(attention(RMSNorm(x))) in place; writes K/V of `pos` into layer L's rings;
 * fills tr's fields up to x_mid.  A Qwen3-MoE layer's FFN (dispatch_qwen3_moe_ffn) follows it in
 * pyoracle.moe_decode_step. */
int jo_decode_attn(const jo_model *mdl, float *kv, int64_t layer, float *x, int64_t pos, int threads,
                   const jo_layer_trace *tr);
/* Layer L of execute_token_standard_with_hidden (src/qwen_deepseek.rs:1262-1302, with
 * run_dense_attention_sublayer_scaled :984-1097 and run_dense_swiglu_ffn :696-727): x [hidden]
 * in, the layer's output out (in place); writes K/V of `pos` into layer L's rings of kv. */
int jo_decode_layer(const jo_model *mdl, float *kv, int64_t layer, float *x, int64_t pos, int threads,
                    const jo_layer_trace *tr);
/* Final RMSNorm and project_lm_head (:1305-1312, :584-632): logits [logits_len] from the last
 * hidden state.  A head of shape [hidden, rows]: its first min(logits_len, rows) rows, the rest
 * xn[i % hidden] * 0.05; a head of logits_len * hidden elements in another shape: its rows of
 * `hidden` elements; no usable head: tanh(sum(xn) / 16) + xn[i % hidden] * 0.1 + (i % 13) * 0.01.
 * xn_head / q8_head (optional) receive the normalised input and its activation blocks. */
int jo_decode_head(const jo_model *mdl, const float *x, float *logits, int threads, float *xn_head, void *q8_head);
/* kv: f32 [n_layers][2][kv_capacity][nkv*hd].  logits [logits_len].  token >= 0 (embed_token). */
int jo_decode_step(const jo_model *mdl, float *kv, int32_t token, int64_t pos, float *logits,
                   int threads);

/* Synthetic all-int8 transformer of src/forward.rs (ForwardModel, :834-1075): DIM 512, FFN 1024,
 * 4 layers (:124-128), one 512-wide attention head, exact integer arithmetic throughout. */
#define JO_FWD_DIM 512
#define JO_FWD_FFN 1024
#define JO_FWD_LAYERS 4
uint64_t jo_splitmix(uint64_t x);
void jo_fill_small(uint64_t seed, int64_t len, int8_t *out);
uint64_t jo_isqrt(uint64_t v);
void jo_fwd_rmsnorm(const int8_t *x, int64_t m, int8_t *out);
void jo_fwd_attention(const int8_t *q, const int8_t *k_cache, const int8_t *v_cache, int64_t m, int64_t start_pos,
                      int8_t *out);
void jo_fwd_embed(uint64_t seed, uint32_t token, int8_t *out);
typedef struct jo_fwd_model jo_fwd_model;
/* NULL on a bad argument or allocation failure; the cache holds max_positions positions. */
jo_fwd_model *jo_fwd_new(uint64_t seed, int64_t vocab, int64_t max_positions);
void jo_fwd_free(jo_fwd_model *f);
int64_t jo_fwd_head_rows(const jo_fwd_model *f);
int64_t jo_fwd_len(const jo_fwd_model *f);
void jo_fwd_reset(jo_fwd_model *f);
/* Worker threads of the forward's products and attention (1 by default). */
void jo_fwd_set_threads(jo_fwd_model *f, int threads);
/* layer 0..3 with which 0..5 = wq wk wv wo up down, or layer -1: the LM head. Row-major [n][k]. */
const int8_t *jo_fwd_weight(const jo_fwd_model *f, int layer, int which, int64_t *n, int64_t *k, int *shift);
/* 0, or -1 for m < 1, start_pos != cached positions or past the capacity. logits [head rows]. */
int jo_fwd_forward(jo_fwd_model *f, const uint32_t *tokens, int64_t m, int64_t start_pos, int32_t *logits);
uint32_t jo_fwd_sample(const int32_t *logits, int64_t vocab);
int jo_fwd_evaluate(jo_fwd_model *f, const uint32_t *prompt, int64_t n, int64_t max_tokens, uint32_t *generated);

#ifdef __cplusplus
}
#endif
#endif
