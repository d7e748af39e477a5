/*
 * jero_hip.h -- C ABI of libjero_hip.so, the MI355X (gfx950) implementation of
 * jero-engine's quantized-matmul hot path.
 *
 * The reference's hot path is the jero_kernels_rvv Rust API called by the recipes
 * (src/gemma.rs:66-138, src/qwen_deepseek.rs:643-951, src/forward.rs:763-811).  Each entry
 * point below names the reference interface it replaces.  All pointers named *_dev are
 * device pointers; `stream` is a hipStream_t (NULL = the null stream).  Work is enqueued on
 * the stream and the call returns; argument errors are reported before anything is enqueued.
 *
 * Status codes mirror the K3Error variants with the numbers the reference's CLI maps them
 * to (src/bin/jero-diag/main.rs:595-605); JERO_ERR_DEVICE and JERO_ERR_INVALID_ARGUMENT have
 * no K3Error counterpart (HIP runtime failure, null pointer).
 */
#ifndef JERO_HIP_H
#define JERO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum jero_status {
  JERO_OK = 0,
  JERO_ERR_CAPABILITY_MISMATCH = 10, /* K3Error::CapabilityMismatch: unsupported quant / shape */
  JERO_ERR_INSUFFICIENT_MEMORY = 11, /* K3Error::InsufficientLockableMemory: device allocation */
  JERO_ERR_CONTEXT_LENGTH_EXCEEDED = 12, /* K3Error::ContextLengthExceeded */
  JERO_ERR_TENSOR_BOUNDS = 14,       /* K3Error::TensorBoundsError: byte/shape mismatch, empty */
  JERO_ERR_ROUTING_UNAVAILABLE = 15, /* K3Error::RoutingUnavailable: no expert selectable */
  JERO_ERR_DEVICE = 20,              /* HIP runtime error */
  JERO_ERR_INVALID_ARGUMENT = 21     /* null pointer or nonsensical argument */
} jero_status;

/* Quantization ids: GGUF/ggml type ids, plus the activation block formats. */
typedef enum jero_quant {
  JERO_F32 = 0,
  JERO_F16 = 1,
  JERO_BF16 = 30,
  JERO_Q4_0 = 2,
  JERO_Q8_0 = 8,
  JERO_Q4_K = 12, /* the reference's QuantType::Q4_K_M */
  JERO_Q6_K = 14,
  JERO_Q8_K = 15,  /* activation blocks for Q4_K / Q6_K weights: f32 d, i8 q[256], i16 bsums[16] */
  JERO_Q4_K_R = 112, /* Q4_K bytes re-laid out by jero_hip_repack into aligned planes (same size) */
  JERO_Q4_K_T = 113, /* stacked expert Q4_K re-laid out by jero_hip_repack_experts (16-row tiles) */
  JERO_Q6_K_R = 114, /* Q6_K bytes re-laid out by jero_hip_repack into aligned planes (same size) */
  JERO_Q6_K_T = 115, /* stacked expert Q6_K re-laid out by jero_hip_repack_experts (16-row tiles) */
  JERO_Q4_K_G = 116, /* Q4_K in the GEMM's fragment order, by jero_hip_repack_gemm (GEMM only) */
  JERO_Q6_K_P = 117, /* Q6_K as exact int8 planes, by jero_hip_repack_gemm (GEMM only) */
  JERO_ACT_Q8 = 100 /* activation blocks for Q8_0 / Q4_0 weights: f32 d, i8 q[32] (36 B) */
} jero_quant;

/* Element type of the K/V rings. */
typedef enum jero_kv_dtype { JERO_KV_F32 = 0, JERO_KV_F16 = 1 } jero_kv_dtype;

/* ---- runtime ---- */

/* Selects the device for the calling thread and prepares per-device state. */
int jero_hip_init(int device);
/* Text of the last error raised on the calling thread ("" if none). */
const char *jero_hip_last_error(void);
const char *jero_hip_status_name(int status);
/* Bytes of one row of n elements in `quant` (-1 if n is not a multiple of the block). */
int64_t jero_hip_row_bytes(int quant, int64_t n);
/* Activation format consumed by the dot product of `weight_quant` (-1 if unsupported): Q8_K for
 * Q4_K / Q6_K, ACT_Q8 for Q8_0 / Q4_0, JERO_F32 (the f32 vector itself) for F32 / F16 / BF16. */
int jero_hip_act_format(int weight_quant);

/* ---- device copies of host weight tensors ----
 * The device-side RepackedTensorStore (src/weights.rs:189-277): the reference's kernels read
 * weights from mmaped host bytes (LockedModelWeights, src/weights.rs:729-734); a binding
 * registers each tensor once and then passes the device address to the entry points below.
 * Registering [host, host + nbytes) copies it to the current device on first use; registering
 * it again, or any sub-range of it, returns the matching device address without copying.
 * Partially overlapping ranges are rejected (TensorBoundsError). */
int jero_hip_weights_register(const void *host, size_t nbytes, const void **dev_out);
/* Device address of [host, host + nbytes), which must lie inside a registered tensor
 * (slice_rows / slice_expert views of it). */
int jero_hip_weights_lookup(const void *host, size_t nbytes, const void **dev_out);
/* Frees every tensor registered on the current device (after a device synchronize). */
int jero_hip_weights_release_all(void);
/* Frees, on every device, the registered tensors that lie inside [host, host + nbytes) (after a
 * synchronize of each such device), so that a new mapping at the same host addresses registers
 * its own bytes.  The owner of an mmaped weight file calls it before unmapping (munmap of
 * LockedModelWeights, src/weights.rs:729-734); jero_hip_gguf_close does so itself. */
int jero_hip_weights_release(const void *host, size_t nbytes);
/* n host tensors of nbytes each (per-expert tensors blk.L.ffn_*_exps.{e}.weight, looked up by
 * slice_or_lookup_expert, src/qwen_deepseek.rs:729-746) registered as ONE stacked device tensor,
 * expert e at *dev_out + e * nbytes, the layout of a stacked [n_in, rows, n] tensor, so the routed
 * expert kernels take them as they take a stacked tensor.  Registering the same n tensors again
 * returns the same address; each host range is then also registered on its own (lookup and
 * release find it).  Some of the ranges registered otherwise (apart, or in another stack):
 * TensorBoundsError. */
int jero_hip_weights_register_stacked(const void *const *hosts, size_t nbytes, int64_t n, const void **dev_out);
/* Waits for the work enqueued on `stream`. */
int jero_hip_sync(void *stream);

/* ---- Q8 activation quantization ----
 * Replaces repack::QuantizedActQ8::quantize(acts, m, k) (src/weights.rs:1416-1417) and the
 * quantization implied inside vec_dot_* (src/gemma.rs:73-86).  x_dev: m rows of k f32;
 * q_dev: m * jero_hip_row_bytes(act_quant, k) bytes.  act_quant is JERO_ACT_Q8 or JERO_Q8_K. */
int jero_hip_quantize_act(int act_quant, const float *x_dev, int64_t m, int64_t k, void *q_dev, void *stream);

/* ---- GEMV over GGUF weight bytes ----
 * Replaces matvec_any (src/gemma.rs:100-138) -> matvec_any_slice (src/gemma.rs:66-95) ->
 * vec_dot_q8_0 / vec_dot_q4_0 / BaselineKernel::vec_dot_q4_k_m / vec_dot_q6_k, and matvec_f32 /
 * vec_dot_f16 / vec_dot_bf16 (src/gemma.rs:72-74,140-189) for unquantized rows, whose
 * "activation" is the f32 input itself (any n_in; rows need only their element alignment).
 * w_dev: n_out rows of n_in elements in `quant` (GGUF tensor shape [n_in, n_out]);
 * xq_dev: the activation already quantized to jero_hip_act_format(quant); y_dev: n_out f32.
 * Any row length up to 2^30 elements: rows longer than 16384 (Q8_0 / Q4_0) or 32768 (K-quants)
 * elements run a K-looped kernel that stages the activation through LDS. */
int jero_hip_matvec(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                    const void *xq_dev, float *y_dev, void *stream);

/* The reference signature vec_dot_*(out, &TensorView, &[f32]): quantizes x_dev first into
 * `workspace_dev` (jero_hip_row_bytes(act, n_in) bytes).  A NULL workspace uses a
 * library-owned per-device buffer: such calls must not overlap on one device. */
int jero_hip_vec_dot(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                     const float *x_dev, float *y_dev, void *workspace_dev, size_t workspace_bytes,
                     void *stream);

/* jero_hip_vec_dot without allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  The quantized activation is staged in a static device array of 128 KiB
 * held by each device the library runs on, so the call never allocates; n_in whose activation
 * blocks exceed it (above 114688 elements for Q4_K / Q6_K, 116508 for Q8_0 / Q4_0) is
 * CapabilityMismatch.  Every call on a device shares that array: calls that overlap on one
 * device (other streams, other threads) race and must be serialized by the caller. */
int jero_hip_vec_dot_noalloc(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                             const float *x_dev, float *y_dev, void *stream);

/* The exact int32 partial sums of the same GEMV kernel: partials_dev[n_out][P] with P = n_in/32
 * (Q8_0, Q4_0: per block; Q4_K: per 32-element sub-block) or n_in/16 (Q6_K).  Debug export for
 * the bit-exact tests; y_dev receives the same outputs as jero_hip_matvec. */
int jero_hip_matvec_partials(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                             const void *xq_dev, float *y_dev, int32_t *partials_dev, void *stream);

/* ---- GEMM over GGUF weight bytes (m activation rows at once) ----
 * Row r of the result is jero_hip_matvec of activation row r: it replaces the prefill token loop
 * (src/qwen_deepseek.rs:2298-2312, one matvec_any per token) and PackedNibbleMatrix::gemm(out,
 * &QuantizedActQ8) (src/weights.rs:1416-1426).  xq_dev: m rows of jero_hip_row_bytes(act, n_in)
 * bytes (jero_hip_quantize_act with m rows); y_dev: [m][n_out] f32.  Q4_K / Q4_K_R with n_out
 * a multiple of 128 run the int8-MFMA kernel; Q6_K / Q6_K_R from 8 rows run an int8-MFMA kernel
 * over the tensor's two exact int8 planes, built for the call in the library-owned per-device
 * workspace (2 bytes per weight), so such calls must not overlap on one device; other formats and
 * shapes run one GEMV per row. */
int jero_hip_gemm(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                  const void *xq_dev, int64_t m, float *y_dev, void *stream);

/* Load-time re-layout of a Q4_K / Q6_K tensor (GGUF bytes or JERO_Q4_K_R / JERO_Q6_K_R) for
 * jero_hip_gemm, the RepackedWeight role of repack_tensor_parallel (src/weights.rs:914-955) for
 * the prefill.  Q4_K -> JERO_Q4_K_G: the quants regrouped per 32-row tile and 256-block in the
 * order of the int8-MFMA fragments, with each block's 6-bit scales and mins unpacked to bytes
 * (160 bytes per 256-block of a row against Q4_K's 144).  Q6_K -> JERO_Q6_K_P: every weight as the exact integer sc*(q6-32) under the block's d,
 * split into two int8 planes (128*hi + lo) in the fragment order, plus d as f32 (2 bytes per
 * weight and 4 per 256-block of a row: about 2.3x the Q6_K bytes).  Rows are padded to a
 * multiple of 32.  jero_hip_gemm_layout_bytes(quant, n_in, n_out) bytes (n_in a multiple of 256;
 * 0 for other formats or shapes).  dst_dev (16-byte aligned, dst_bytes bytes) is then passed to
 * jero_hip_gemm as *dst_quant with the same n_in and n_out and w_bytes = the layout's size, and
 * computes what the source tensor computes (the GEMV of each activation row); the GEMV entry
 * points reject these formats. */
size_t jero_hip_gemm_layout_bytes(int quant, int64_t n_in, int64_t n_out);
int jero_hip_repack_gemm(int quant, const void *src_dev, size_t src_bytes, int64_t n_in, int64_t n_out,
                         void *dst_dev, size_t dst_bytes, int *dst_quant, void *stream);

/* The exact integer product of ForwardExec::matmul (src/forward.rs:555-655) -> matmul_rows
 * (:763-811) -> gemm_i8_ime / gemm_i8_vector: out[m][n] = sum_k x[m][k] * w[n][k] in int32.
 * x_dev [m][k] and w_dev [n][k] int8 row-major, out_dev [m][n] int32; k <= 131071 so no sum
 * can overflow.  k a multiple of 16 (and 4-byte aligned operands) runs the MFMA kernel. */
int jero_hip_gemm_i8(const int8_t *x_dev, int64_t m, int64_t k, const int8_t *w_dev, int64_t n, int32_t *out_dev,
                     void *stream);

/* requant_all(&ForwardExec::matmul(..), shift) (src/forward.rs:813-815, called at :957-970) in one
 * launch: jero_hip_gemm_i8's int32 sums requantized as forward.rs's requant (:345-350) does,
 * out[m][n] = clamp((acc + 2^(shift-1)) >> shift, -127, 127) as int8 row-major; the add wraps as
 * two's complement (the reference's release build), the shift is arithmetic.  shift in 1..31. */
int jero_hip_gemm_i8_requant(const int8_t *x_dev, int64_t m, int64_t k, const int8_t *w_dev, int64_t n, int shift,
                             int8_t *out_dev, void *stream);
/* requant_all (src/forward.rs:813-815) alone: n int32 -> int8, as above. */
int jero_hip_requant_i8(const int32_t *raw_dev, int64_t n, int shift, int8_t *out_dev, void *stream);

/* The packed-tile form of the int8 product, the ime::{TILE_*, tile_count, pack_tiles,
 * gemm_i8_ime} names forward.rs imports (src/forward.rs:26-29, used at :365-372, :569, :779-796).
 * Tiles of JERO_TILE_N rows (weights) or JERO_TILE_M rows (activations), K in chunks of
 * JERO_TILE_K.  Packed layout: element (r, c) of a [rows][k] matrix, rows padded with zero rows
 * to jero_hip_tile_count(rows) whole tiles, sits at byte
 *   ((r / 8 * (k / 32) + c / 32) * 8 + r % 8) * 32 + c % 32. */
#define JERO_TILE_M 8
#define JERO_TILE_N 8
#define JERO_TILE_K 32
#define JERO_TILE_C 64
/* ime::tile_count: whole tiles covering `rows` rows. */
int64_t jero_hip_tile_count(int64_t rows);
/* ime::pack_tiles: src_dev [rows][k] int8 row-major -> dst_dev, jero_hip_tile_count(rows) * 8 * k
 * bytes in the packed layout; k a multiple of 32. */
int jero_hip_pack_tiles(const int8_t *src_dev, int64_t rows, int64_t k, int8_t *dst_dev, void *stream);
/* ime::gemm_i8_ime(a, m_tiles, packed_w, tile_begin..tile_end, k_chunks, |mt, nt, &[i32; TILE_C]|):
 * the C block of every activation tile mt < m_tiles and weight tile nt in [tile_begin, tile_end),
 * C[i * 8 + j] = sum_k a[8 mt + i][k] * w[8 nt + j][k] (exact int32), written to c_dev as
 * [m_tiles][tile_end - tile_begin][JERO_TILE_C]; the callback then reads block (mt, nt) at
 * (mt * (tile_end - tile_begin) + nt - tile_begin) * 64.  Both operands packed (4-byte aligned),
 * k = 32 * k_chunks <= 131071. */
int jero_hip_gemm_i8_tiles(const int8_t *a_packed_dev, int64_t m_tiles, const int8_t *w_packed_dev, int64_t tile_begin,
                           int64_t tile_end, int64_t k_chunks, int32_t *c_dev, void *stream);

/* The synthetic all-int8 transformer the reference benchmarks its int8 GEMM with: ForwardModel
 * (src/forward.rs:834-1075), 4 layers of width 512, FFN 1024, one 512-wide attention head, every
 * value an exact integer, so results are bit-identical to the reference.  The device holds the
 * weights (generated from seed, as ForwardModel::new does, src/forward.rs:879-903), a K/V cache of
 * max_positions positions per layer and the activation rows of max_positions tokens. */
typedef struct jero_forward_model jero_forward_model;
/* ForwardModel::new(seed, vocab) (src/forward.rs:879-903) on the current device; vocab in
 * 0..2^24, max_positions in 1..2^22 (TensorBounds otherwise).  Synchronous. */
int jero_hip_forward_model_create(uint64_t seed, int64_t vocab, int64_t max_positions, jero_forward_model **out);
int jero_hip_forward_model_destroy(jero_forward_model *model);
/* Logit rows of the LM head: max(vocab, 1) rounded up to whole 8-row tiles (Matrix::random,
 * src/forward.rs:364-377); -1 for a null model. */
int64_t jero_hip_forward_model_head_rows(const jero_forward_model *model);
/* Positions held in the K/V cache (the KvState's length); -1 for a null model. */
int64_t jero_hip_forward_model_positions(const jero_forward_model *model);
/* Empties the K/V cache (a fresh KvState, src/forward.rs:1010-1013). */
int jero_hip_forward_model_reset(jero_forward_model *model);
/* Device address and shape of a matrix: layer 0..3 with which 0..5 = wq wk wv wo up down, or
 * layer -1 for the LM head (which ignored); row-major int8 [n][k] and its requant shift. */
int jero_hip_forward_model_weight(const jero_forward_model *model, int layer, int which, const int8_t **w_dev,
                                  int64_t *n, int64_t *k, int *shift);
/* ForwardModel::forward (src/forward.rs:930-976): the m >= 1 host tokens at positions
 * start_pos.., which must be the cached position count (InvalidArgument otherwise), appended to
 * the cache (ContextLengthExceeded past max_positions); logits_dev (device, int32
 * [jero_hip_forward_model_head_rows]) receives the last token's logits.  Enqueued on stream. */
int jero_hip_forward_model_forward(jero_forward_model *model, const uint32_t *tokens, int64_t m, int64_t start_pos,
                                   int32_t *logits_dev, void *stream);
/* ForwardModel::evaluate's token loop (src/forward.rs:995-1043): empties the cache, runs the
 * prompt's forward, then greedy steps (ForwardModel::sample, :978-986) until max_tokens tokens;
 * each step's token stays on the device for the next step.  generated (host) receives max_tokens
 * ids; timing_ms (host, 2 floats, or NULL) the device time of the prefill (through the first
 * sample) and of the decode steps.  An empty prompt is CapabilityMismatch, as in the reference;
 * n + max_tokens - 1 positions past max_positions ContextLengthExceeded.  Synchronous. */
int jero_hip_forward_model_evaluate(jero_forward_model *model, const uint32_t *prompt, int64_t n, int64_t max_tokens,
                                    uint32_t *generated, float *timing_ms, void *stream);

/* Load-time re-layout of a weight tensor for the GEMV kernels; replaces repack_tensor_parallel
 * (src/weights.rs:914-955) -> RepackedWeight.  Q4_K -> JERO_Q4_K_R and Q6_K -> JERO_Q6_K_R:
 * the n_out x n_in tensor's bytes are regrouped into 16-byte aligned planes of the same total
 * size (src and dst may not overlap).  The result is passed to jero_hip_matvec / _partials /
 * _vec_dot as the returned quant with the same n_in and n_out and computes exactly what the
 * GGUF tensor computes; it must be used whole (its rows are not contiguous).
 * Other formats: CapabilityMismatch. */
int jero_hip_repack(int quant, const void *src_dev, size_t src_bytes, int64_t n_in, int64_t n_out,
                    void *dst_dev, int *dst_quant, void *stream);

/* Load-time re-layout of a stacked expert tensor (GGUF [n_in, rows_per_expert, n_experts], expert
 * e = rows e*rows_per_expert ..) for jero_hip_moe_ffn; the same repack_tensor_parallel
 * (src/weights.rs:914-955) step for the expert tensors.  Q4_K -> JERO_Q4_K_T, Q6_K -> JERO_Q6_K_T:
 * each block of 16 consecutive rows stores, per 256-element block column, the 16 rows' bytes as
 * one contiguous piece (same total size; src and dst may not overlap; dst 16-byte aligned), so
 * the expert kernels stream whole pieces.  rows_per_expert must be a multiple of 16; other
 * formats: CapabilityMismatch. */
int jero_hip_repack_experts(int quant, const void *src_dev, size_t src_bytes, int64_t n_in, int64_t rows_per_expert,
                            int64_t n_experts, void *dst_dev, int *dst_quant, void *stream);

/* ---- attention ----
 * gqa_causal_attention_f32(out, q, k, v, n_heads_q, n_heads_kv, head_dim, seq_len, scale)
 * (called at src/qwen_deepseek.rs:669-691): softmax(q . k_t * scale) . v over t < seq_len for
 * each q head h, kv head h / (n_heads_q / n_heads_kv).  q_dev: [n_heads_q][head_dim] f32 (8-byte
 * aligned);
 * k_dev, v_dev: [seq_len][n_heads_kv * head_dim] of kv_dtype (16-byte aligned); out_dev:
 * [n_heads_q][head_dim] f32.  head_dim: any even value up to 256 (even_head_dim,
 * src/qwen_deepseek.rs:58-65, gives the recipes only even ones; 32, 64 and 128 run the head_dim-built
 * kernels, the rest one q head per workgroup); above 256 or odd: CapabilityMismatch.  Any number of
 * q heads per kv head.
 * seq_len <= JERO_MAX_ATTENTION_POSITIONS, else ContextLengthExceeded.  Workspace: n_heads_q * ceil(seq_len/64) * (head_dim + 2) floats, 16-byte
 * aligned (NULL: library-owned, calls must not overlap on one device). */
#define JERO_MAX_ATTENTION_POSITIONS 131072
int jero_hip_gqa_attention(float *out_dev, const float *q_dev, const void *k_dev, const void *v_dev, int kv_dtype,
                           int n_heads_q, int n_heads_kv, int head_dim, int64_t seq_len, float scale,
                           void *workspace_dev, size_t workspace_bytes, void *stream);

/* ---- routed experts ----
 * dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) from router logits, with
 * select_top_k_experts(logits, top_k, normalize = true) (src/gemma.rs:362-442) and
 * run_single_swiglu_expert (:748-771) per selected expert:
 *   y[t] = sum_j w[t][j] * down_e(silu(gate_e x_t) * up_e x_t),  e = sel_idx[t][j].
 * x_dev [n_tokens][hidden] f32 (16-byte aligned); router_logits_dev [n_tokens][n_experts] f32;
 * gate/up: stacked [n_experts][ffn rows][hidden] in one format; down: [n_experts][hidden rows][ffn];
 * each Q4_K, Q6_K, Q8_0 or Q4_0 (GGUF stacked [hidden, ffn, n_experts] tensors, expert e = rows
 * e*ffn..), the K-quants also after jero_hip_repack_experts (JERO_Q4_K_T / JERO_Q6_K_T, the layouts
 * the expert GEMMs read fastest) or jero_hip_repack over all their rows (JERO_Q4_K_R /
 * JERO_Q6_K_R); repacked tensors 16-byte aligned.  Activations are quantized as matvec_any
 * quantizes them for each format (Q8_K for the K-quants, ACT_Q8 for Q8_0 / Q4_0); the expert
 * GEMMs on the matrix cores take the K-quants, the 32-element formats run the GEMV kernels at
 * any token count.
 * Outputs y_dev [n_tokens][hidden], sel_idx_dev / sel_w_dev [n_tokens][top_k].
 * Limits the reference does not have, refused with CapabilityMismatch: hidden <= 8192 (the gate/up
 * rows' lane pairing; 4096 for Q8_0 / Q4_0), ffn <= 16384 (the down rows'; 8192 for Q8_0 / Q4_0),
 * top_k <= 16 and n_experts <= 1024 (the routing kernels' per-lane columns); hidden and ffn
 * multiples of 256 whatever the format (TensorBoundsError; the activations are quantized in
 * 256-element groups); Qwen3-MoE (128 experts, top-8, hidden up to 4096, ffn 768 /
 * 1536) and DeepSeek-style routers (256 experts, top-8) sit well inside them.  Workspace:
 * jero_hip_moe_workspace_bytes(...) bytes, 256-byte aligned (NULL: library-owned). */
int jero_hip_moe_ffn(const float *x_dev, const float *router_logits_dev, int64_t n_tokens, int64_t n_experts,
                     int top_k, int gate_quant, const void *gate_dev, size_t gate_bytes, int up_quant,
                     const void *up_dev, size_t up_bytes, int down_quant, const void *down_dev, size_t down_bytes,
                     int64_t hidden, int64_t ffn, float *y_dev, int32_t *sel_idx_dev, float *sel_w_dev,
                     void *workspace_dev, size_t workspace_bytes, void *stream);
size_t jero_hip_moe_workspace_bytes(int64_t n_tokens, int64_t n_experts, int top_k, int64_t hidden, int64_t ffn);
/* jero_hip_moe_ffn with y_dev holding, on entry, values the routed sum is added onto, in the
 * reference's order: y[t][i] = ((y[t][i] + w[t][0] * e_0[i]) + w[t][1] * e_1[i]) + ...  -- the
 * shared expert's output that dispatch_qwen3_moe_ffn adds first (src/qwen_deepseek.rs:860-871,
 * 925-936).  Same arguments, limits and workspace as jero_hip_moe_ffn. */
int jero_hip_moe_ffn_acc(const float *x_dev, const float *router_logits_dev, int64_t n_tokens, int64_t n_experts,
                         int top_k, int gate_quant, const void *gate_dev, size_t gate_bytes, int up_quant,
                         const void *up_dev, size_t up_bytes, int down_quant, const void *down_dev,
                         size_t down_bytes, int64_t hidden, int64_t ffn, float *y_dev, int32_t *sel_idx_dev,
                         float *sel_w_dev, void *workspace_dev, size_t workspace_bytes, void *stream);

/* A weight tensor as the reference's ModelWeights hands it out: format, device bytes (NULL: the
 * model has no such tensor) and TensorView::num_elements. */
typedef struct jero_hip_tensor {
  int quant;
  const void *dev;
  size_t bytes;
  int64_t n_elements;
} jero_hip_tensor;

/* The dense SwiGLU FFNs of dispatch_qwen3_moe_ffn on one token row x_dev[hidden] (16-byte aligned):
 *   r = down(silu(gate x) * up x),   y_dev[hidden] = (accumulate ? y_dev : 0) + r.
 * JERO_FFN_SHARED_EXPERT -- run_single_swiglu_expert (src/qwen_deepseek.rs:748-771) of the shared
 *   expert blk.L.ffn_{gate,up,down}_shexp (:860-871): F = gate.n_elements / hidden when that
 *   divides, else max(ffn, 4); gate and up give their first F rows of hidden, down H rows of F
 *   (matvec_any); each tensor must be present and hold them (TensorBoundsError).
 * JERO_FFN_DENSE -- run_dense_swiglu_ffn (:696-727), the layer's FFN when it has no router (:873-880):
 *   F = max(ffn, 4); each of blk.L.ffn_{gate,up,down} is project_or_deterministic_slice
 *   (src/gemma.rs:841-860): its GEMV when present with exactly out_len * in_len elements, else
 *   in[i % in_len] * scale (gate 0.5, up 0.25, down 0.125).
 * Formats: those of jero_hip_vec_dot.  Workspace: jero_hip_swiglu_ffn_workspace_bytes(hidden, F)
 * bytes with F as above, 256-byte aligned (NULL: library-owned, calls must not overlap on one
 * device). */
enum { JERO_FFN_SHARED_EXPERT = 0, JERO_FFN_DENSE = 1 };
int jero_hip_swiglu_ffn(int mode, const float *x_dev, int64_t hidden, int64_t ffn, const jero_hip_tensor *gate,
                        const jero_hip_tensor *up, const jero_hip_tensor *down, int accumulate, float *y_dev,
                        void *workspace_dev, size_t workspace_bytes, void *stream);
size_t jero_hip_swiglu_ffn_workspace_bytes(int64_t hidden, int64_t ffn);
/* Debug view of a workspace after jero_hip_moe_ffn returned and its stream was synchronized, for
 * the per-expert parity tests (no counterpart in the reference, where the expert's SwiGLU
 * vector is a local of run_single_swiglu_expert, src/qwen_deepseek.rs:748-771): *act_dev holds the
 * f32 rows silu(gate_e x_t) * up_e x_t [ffn] that the down projections quantized to Q8_K, one per
 * (token t, slot j); the row of (t, j) is t * top_k + j when *identity, else the int32 at
 * (*pair_row_dev)[t * top_k + j] (device memory). */
int jero_hip_moe_trace_view(void *workspace_dev, int64_t n_tokens, int64_t n_experts, int top_k, int64_t hidden,
                            int64_t ffn, float **act_dev, int32_t **pair_row_dev, int *identity);

/* dequantize_token_row (src/qwen_deepseek.rs:514,569): rows [row0, row0+n_rows) of a tensor
 * with n_in elements per row, written as f32 to out_dev[n_rows][n_in]. */
int jero_hip_dequantize_rows(int quant, const void *w_dev, size_t w_bytes, int64_t n_in, int64_t row0,
                             int64_t n_rows, float *out_dev, void *stream);

/* ---- device-resident decoder (batch-1 decode step) ----
 * The Qwen3/Llama dense decode path: embed_token -> n_layers x [RMSNorm -> Q|K|V -> (QK-norm)
 * -> interleaved RoPE -> KV-ring append + GQA attention -> Wo + residual -> RMSNorm -> SwiGLU
 * FFN + residual] -> RMSNorm -> LM head -> greedy argmax.  Replaces
 * execute_token_standard_with_hidden (src/qwen_deepseek.rs:1239-1314) as called by
 * Qwen3Recipe::decode_step (:1441-1460) and sample_greedy_argmax (src/engine.rs:1873-1895).
 * Tensors are given by GGUF name (ModelWeights::tensor): token_embd.weight, output.weight,
 * output_norm.weight, blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output, attn_q_norm,
 * attn_k_norm, ffn_norm, ffn_gate, ffn_up, ffn_down}.weight; projections in Q8_0/Q4_0/Q4_K/Q6_K
 * with GGUF shape [n_in, n_out] (rows of up to 54592 elements for Q8_0/Q4_0, 53760 for Q4_K/Q6_K:
 * the activation of a row is held in LDS).  Norms, the embedding and the head may also be
 * F32/F16/BF16 and of any shape, and any of them may be absent; they are read as the reference
 * reads them:
 *   norms  read_f32_weight_or_default (src/qwen_deepseek.rs:491-519): absent -> all 1.0; F32 ->
 *          the stored values with 1.0 for a non-finite one or past the tensor's end; another
 *          format with at least len elements -> its first len elements dequantized (1.0 if they
 *          are not whole blocks); fewer -> all 1.0;
 *   token_embd  embed_token (:558-582): rows of `hidden` elements (num_elements / hidden of
 *          them); a token past them (or with no token_embd) embeds as the deterministic row
 *          ((token % 31) * 0.05 + 0.25) + (i % 7) * 0.01;
 *   head   project_lm_head (:584-632): output.weight, else token_embd.weight (ModelWeights' tied
 *          fallback, src/weights.rs:1110-1126); jero_hip_model_logits_len logits
 *          (infer_logits_buffer_len, src/engine.rs:1781-1792: the head's rows when they exceed
 *          vocab by at most 1024 and are a multiple of 64, else vocab); a [hidden, rows] head
 *          gives the first min(logits, rows) of them and xn[i % hidden] * 0.05 past them; a head
 *          of logits * hidden elements in another shape is read as rows of hidden; with no
 *          usable head every logit is tanh(sum(xn) / 16) + xn[i % hidden] * 0.1 + (i % 13) * 0.01
 *          (xn the final RMSNorm's output).  The greedy token is the argmax over all logits.
 * The KV arena is one device buffer of [n_layers][K ring, V ring][kv_capacity][n_heads_kv *
 * head_dim] (the recipes' flat layout). */
typedef struct jero_model_config {
  int64_t hidden, ffn, n_layers, vocab;
  int n_heads_q, n_heads_kv, head_dim;
  float rms_eps, rope_theta;
  int64_t kv_capacity; /* ring slots per layer (n_ctx) */
  int kv_dtype;        /* JERO_KV_F16 or JERO_KV_F32 */
  int qk_norm;         /* nonzero: per-head RMSNorm of q and k (Qwen3) */
} jero_model_config;
typedef struct jero_model jero_model;

int jero_hip_model_create(const jero_model_config *cfg, jero_model **model);
/* A Qwen3-MoE model (StandardExecSpec's `moe`, MoeDispatchSpec { num_experts, top_k,
 * expert_ffn_dim, use_shared }, src/qwen_deepseek.rs:81-87, 1465-1487): every layer's FFN is then
 * dispatch_qwen3_moe_ffn (:847-951, called at :1286-1300) instead of the dense SwiGLU FFN.  Call it
 * after jero_hip_model_create and before any FFN tensor.  The model then also takes, per layer,
 * blk.N.ffn_gate_inp.weight (the router, [hidden, E]), the stacked routed experts
 * blk.N.ffn_{gate,up}_exps.weight ([hidden, F, E], n_out = F * E) and blk.N.ffn_down_exps.weight
 * ([F, hidden, E]), and the shared expert blk.N.ffn_{gate,up,down}_shexp.weight; a layer's dense
 * ffn_{gate,up,down}.weight have the expert FFN dimension (the fallback of a layer without router
 * or experts, :873-880, 942-946).  The routed experts run jero_hip_moe_ffn's kernels (same formats
 * and limits; Q4_K / Q6_K experts re-laid out at finalize as jero_hip_repack_experts does) on the
 * router's eff_experts = min(its elements / hidden, num_experts) experts; the router and the shared
 * expert take jero_hip_vec_dot's formats.  blk.N.exp_probs_b.bias (a routing bias) and an
 * incomplete set of expert tensors make finalize return CapabilityMismatch.  The decode trace of
 * such a layer holds xn_ffn (the FFN's normalised input) and, in gu, the router logits (when
 * 2 * ffn >= E); its q8_ffn, act and q8_down are not written.  jero_hip_model_prefill runs the
 * prompt's rows through each layer at once when every layer is routed over an F32 router and no
 * shared expert runs (the Qwen3-MoE recipe's form): the router logits as one f32 MFMA product
 * over the rows, the experts as GEMMs over the tokens routed to each; any other MoE model's
 * prompt runs as decode steps, the reference's own token loop. */
int jero_hip_model_set_moe(jero_model *model, int64_t n_experts, int top_k, int64_t expert_ffn, int use_shared);
int jero_hip_model_destroy(jero_model *model);
/* Copies one tensor to the device (src host memory, or device memory if src_on_device).  A layer
 * projection (blk.N.attn_q/attn_k/attn_v/attn_output/ffn_gate/ffn_up/ffn_down.weight) whose
 * element count differs from its expected shape is ignored, as project_or_deterministic_slice
 * (src/gemma.rs:841-860) ignores it: the step then takes that projection's fallback. */
int jero_hip_model_set_tensor(jero_model *model, const char *name, int quant, const void *src, size_t nbytes,
                              int64_t n_in, int64_t n_out, int src_on_device);
/* Builds the device layout (norm weights as f32 vectors, fused Q|K|V and gate|up rows, Q4_K_R /
 * Q6_K_R planes, the LM head).  Required before the first decode step.  A
 * projection left out takes project_or_deterministic_slice's fallback (src/gemma.rs:841-860):
 * out[i] = in[i % in_len] * scale with the Qwen3 call sites' scales (Q 0.5, K 0.25, V 0.125 of the
 * normalised input, src/qwen_deepseek.rs:1011-1031; Wo 0.25 of the attention output, :1086-1092;
 * gate 0.5, up 0.25 of the normalised input and down 0.125 of the SwiGLU vector, :696-725); the
 * layer's present projections then run unfused. */
int jero_hip_model_finalize(jero_model *model);
/* Device addresses of layer `layer`'s K and V rings (to pre-fill or inspect the cache). */
int jero_hip_model_kv(jero_model *model, int64_t layer, void **k_ring_dev, void **v_ring_dev);
/* Device addresses of the current token, the position and the last step's logits
 * [jero_hip_model_logits_len]. */
int jero_hip_model_state(jero_model *model, int32_t **token_dev, int64_t **pos_dev, float **logits_dev);
/* Logits per step once finalized (infer_logits_buffer_len, src/engine.rs:1781-1792), vocab before;
 * -1 for a null model. */
int64_t jero_hip_model_logits_len(const jero_model *model);
/* Enqueues: token (>= 0; embed_token takes any id) and position of the next decode step. */
int jero_hip_model_set_position(jero_model *model, int32_t token, int64_t pos, void *stream);
/* Enqueues one decode step at the device position: writes logits, replaces the token with the
 * greedy next token and advances the position.  Enqueues kernels only (graph-capturable).
 * Logits with no argmax (all NaN) fail closed as the reference's engine does
 * (src/engine.rs:636-641): the step stores token -1, keeps the position and sets a sticky device
 * status; later steps then store -1 and leave the position until jero_hip_model_set_position. */
int jero_hip_decode_step(jero_model *model, void *stream);
/* Waits for `stream` and returns the model's status: JERO_OK, or CapabilityMismatch ("empty
 * logits buffer after decode step (or all-NaN)") once a step has failed closed. */
int jero_hip_model_status(jero_model *model, void *stream);
/* run_prefill_with_hidden (src/qwen_deepseek.rs:2217-2316) without its token loop: the n prompt
 * tokens (host array) at positions pos0 .. pos0 + n - 1 go through each layer at once -- every
 * projection one GEMM over the n activation rows (jero_hip_gemm's kernels), every token's
 * attention causal over the ring up to its own position -- and leave the state n decode steps
 * would leave: the n K/V rows in the ring, the last token's logits, its greedy next token and
 * position pos0 + n.  pos0 + n <= kv_capacity, else ContextLengthExceeded (as engine.rs:727
 * rejects a prompt past n_ctx).  Allocates its row buffers on first use, and from prompts of 8
 * tokens builds the GEMM layout of each Q4_K and Q6_K tensor (jero_hip_repack_gemm's: 1.11x the
 * Q4_K and 2.3x the Q6_K bytes); both are held by the model until jero_hip_model_destroy.
 * With a trace set (jero_hip_model_trace, n * jero_hip_model_trace_bytes bytes or more), token t's
 * trace in the decode step's layout lands at t * jero_hip_model_trace_bytes; the head's fields
 * only for the last token. */
int jero_hip_model_prefill(jero_model *model, const int32_t *tokens, int64_t n, int64_t pos0, void *stream);

/* Debug trace of the decode step, for the layer-by-layer parity tests (no counterpart in the
 * reference; the reference's intermediate vectors are locals of
 * execute_token_standard_with_hidden, src/qwen_deepseek.rs:1239-1314).  While a buffer is set,
 * every decode step overwrites it with its intermediate values; NULL turns tracing off.  The
 * buffer (device, 16-byte aligned, jero_hip_model_trace_bytes bytes) holds per layer, each field
 * starting on a 16-byte boundary, with A(n) = the larger of the Q8_K and ACT_Q8 block sizes of
 * n elements rounded up to 16:
 *   x_in f32[H]  xn_attn f32[H]  q8_attn u8[A(H)]  qkv f32[Q+2KV]  q_rope f32[Q]  k_rope f32[KV]
 *   attn f32[Q]  q8_wo u8[A(Q)]  x_mid f32[H]  xn_ffn f32[H]  q8_ffn u8[A(H)]  gu f32[2F]
 *   act f32[F]  q8_down u8[A(F)]
 * then x_final f32[H]  xn_head f32[H]  q8_head u8[A(H)]  rope_cs f32[hd] (the step's RoPE table,
 * (cos, sin) of pos / theta^(2i/hd) for pair i).  xn_* are the f32 values a GEMV's
 * prologue quantized (after RMSNorm), q8_* the activation blocks it built (the format of the
 * tensor it feeds: attn_q, attn_output, ffn_gate, ffn_down, output), qkv and gu the raw
 * projections, q_rope / k_rope q and the new k after QK-norm and RoPE (before the softmax
 * scale), attn the attention output, act silu(gate) * up. */
int jero_hip_model_trace(jero_model *model, void *trace_dev, size_t trace_bytes);
int64_t jero_hip_model_trace_bytes(const jero_model *model);

/* sample_greedy_argmax -> argmax_f32 (src/engine.rs:1873-1895): the first index of the largest
 * non-NaN value of x_dev[n] into *idx_dev (int64, device), -1 when n == 0 or every value is NaN
 * (Option::None).  The same (max, first index) reduction as the decode step's LM-head epilogue.
 * Workspace: 12304 bytes, 8-byte aligned (NULL: library-owned, calls must not overlap on one
 * device). */
int jero_hip_argmax(const float *x_dev, int64_t n, int64_t *idx_dev, void *workspace_dev, size_t workspace_bytes,
                    void *stream);

/* ---- GGUF v3 model files ----
 * The weight source of LockedModelWeights (src/weights.rs:338-570): the file is mapped
 * read-only and its header, metadata and tensor descriptors parsed (GGUF v2/v3, little-endian,
 * data section aligned to general.alignment, default 32).  A malformed or truncated file, a
 * misaligned tensor or one that runs past the end is TensorBoundsError.  flock/mlock residency
 * policy is the host's and is not done here. */
typedef struct jero_gguf jero_gguf;
int jero_hip_gguf_open(const char *path, jero_gguf **out);
/* Releases the device copies jero_hip_gguf_upload made of the file's tensors
 * (jero_hip_weights_release over the mapping), then unmaps the file. */
void jero_hip_gguf_close(jero_gguf *g);
/* Number of tensors and general.architecture ("" if absent); strings live until close. */
int jero_hip_gguf_info(const jero_gguf *g, int64_t *n_tensors, const char **arch);
/* Metadata by key (ModelWeights metadata accessors): integers (any integer or bool type),
 * numbers (integer or float types) and strings.  A missing key or another type is
 * JERO_ERR_INVALID_ARGUMENT. */
int jero_hip_gguf_meta_int(const jero_gguf *g, const char *key, int64_t *v);
int jero_hip_gguf_meta_float(const jero_gguf *g, const char *key, double *v);
int jero_hip_gguf_meta_str(const jero_gguf *g, const char *key, const char **v);
/* Name of the i-th tensor in file order. */
int jero_hip_gguf_tensor_name(const jero_gguf *g, int64_t i, const char **name);
/* ModelWeights::tensor (src/weights.rs:1097-1144): ggml type, dims (dims[0] = row length, unused
 * dims 1), mapped host bytes and their size.  A missing output.weight of an autoregressive
 * (architecture_requires_kv_cache, src/memory.rs:863-868), non-BitNet model is token_embd.weight
 * (tied embeddings, src/weights.rs:1110-1126); any other missing name is TensorBoundsError.
 * A ggml type with no row size here is CapabilityMismatch (descriptor outputs still filled). */
int jero_hip_gguf_tensor(const jero_gguf *g, const char *name, int *quant, int *n_dims, int64_t *dims,
                         const void **host, size_t *nbytes);
/* The tensor's bytes registered on the current device (jero_hip_weights_register): copied to HBM
 * once, the device address returned. */
int jero_hip_gguf_upload(const jero_gguf *g, const char *name, const void **dev_out);

/* Measurement probe, no counterpart in the reference: one launch that reads `bytes` (a non-zero
 * multiple of 16) at the 16-byte aligned src_dev and nothing else, two non-temporal 16-byte loads
 * per thread.
 * Timed over the same buffers as a GEMV, it is the bandwidth ceiling that launch could reach.
 * sink_dev: 1 KiB of device memory it may write. */
int jero_hip_read_probe(const void *src_dev, size_t bytes, uint32_t *sink_dev, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* JERO_HIP_H */
