// attention.h -- decode attention launchers shared by the entry points and the decode step.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jero {

struct AttnParams {
  const float* q;        // [nq][hd] f32 (fused: before QK-norm and RoPE)
  const void* k;         // K ring of the layer, [capacity][nkv*hd] of kv_dtype
  const void* v;         // V ring of the layer
  int kv_dtype;          // JERO_KV_F32 / JERO_KV_F16
  int nkv, group, hd;
  int active;            // slots attended: [0, active)
  float scale;
  float* part_o;         // workspace: [nq][S][hd] then [nq][S][2] (set by launch_attention)
  float* part_ml;
  // fused decode-step mode
  const float* k_new;    // [nkv][hd] f32 before QK-norm and RoPE
  const float* v_new;    // [nkv][hd] f32
  const float* q_norm;   // [hd] or null
  const float* k_norm;   // [hd] or null
  float eps;
  int64_t pos;
  float theta;
  int slot;              // ring slot of the new token (-1: none)
  void* k_write;         // same rings, writable
  void* v_write;
  const int64_t* pos_dev;  // if set: pos = *pos_dev, slot = pos % capacity, active = min(pos+1, capacity)
  const float* rope_cs;    // if set: [hd/2][cos, sin] of this step's RoPE angles
  int64_t capacity;        // ring slots (grid is sized for all of them when pos_dev is set)
  // fused mode debug trace (null: off): q [nq][hd] and the new k [nkv][hd] after QK-norm and
  // RoPE, before the softmax scale
  float* tr_q;
  float* tr_k;
  // a batch of queries (prefill, not fused): grid z is the token t, whose q row starts t *
  // q_stride floats on, which attends to active + t slots, and whose partials start t * part_tok
  // (part_o) and t * part_tok_ml (part_ml) floats on; all zero for one query
  int64_t q_stride, part_tok, part_tok_ml;
  int n_tok;  // queries of the batch (set by the launcher)
};

int attn_splits(int active, int hd);
size_t attn_workspace_bytes(int nq, int hd, int active);
int check_attention_shape(int nq, int nkv, int hd, int64_t seq_len);
// Enqueues the split-K kernel and the merge; out: [nq][hd] f32.
int launch_attention(const AttnParams& p, bool fused, float* out, hipStream_t s);
// Causal attention of n_tok consecutive queries (prefill): token t's q heads at p.q + t *
// q_stride, attending to the first p.active + t slots of the rings; out row t at out + t *
// out_stride.  f16 rings at head_dim 64 or 128, at most 8 q heads per kv head, with more than one
// query (attn_flash_ok) run the flash kernel, which needs no workspace; otherwise the split kernels need
// attn_workspace_bytes(nq, hd, p.active + n_tok - 1) * n_tok bytes at p.part_o.  With q8k given
// (the flash kernel only, attn_flash_q8k_ok: group * hd a multiple of 256) each row's Q8_K
// blocks are written at q8k + t * row_bytes(Q8_K, nq * hd), and the f32 rows only when out is
// given.
int launch_attention_tokens(const AttnParams& p, int n_tok, int64_t q_stride, float* out, int64_t out_stride,
                            hipStream_t s, void* q8k = nullptr);
bool attn_flash_ok(int kv_dtype, int hd, int n_tok, int group);
bool attn_templated(int hd, int group);
bool attn_flash_q8k_ok(int group, int hd);

}  // namespace jero
