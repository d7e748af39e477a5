// model.hip -- device-resident dense decoder and its decode step (host orchestration).
//
// Mirrors the Qwen/Llama decode path of the reference: ModelWeights::tensor(name) lookups of
// GGUF tensor names, the KV arena (src/kv.rs:43-122; used by the recipes as flat per-layer
// K/V rings, src/qwen_deepseek.rs:643-694) and execute_token_standard_with_hidden
// (src/qwen_deepseek.rs:1239-1314) followed by sample_greedy_argmax (src/engine.rs:1873-1895).
//
// Weights are uploaded once (set_tensor) and regrouped once (finalize): Q|K|V rows become one
// tensor when they share a format, gate and up rows one tensor (rows [0, ffn) gate, [ffn, 2ffn)
// up) so one kernel produces silu(gate) * up, and every Q4_K / Q6_K matrix is re-laid out in
// its planar device layout (Q4_K_R / Q6_K_R).
// The step itself only enqueues kernels -- no allocation, copy or memset -- so it can be captured
// in a HIP graph.  Token and position live in device memory: the step reads them, and its last
// kernel stores the greedy token and advances the position, so replaying the graph decodes
// consecutive tokens.
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "attention.h"
#include "decode.h"
#include "gemv.h"
#include "moe.h"
#include "jero_common.h"
#include "prefill.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {

struct DevTensor {
  int quant = -1;
  void* dev = nullptr;
  size_t bytes = 0;
  int64_t n_in = 0, n_out = 0;
  bool present() const { return dev != nullptr; }
};

struct LayerW {
  DevTensor attn_norm, ffn_norm, q_norm, k_norm;
  DevTensor wq, wk, wv, wo, gate, up, down;
  DevTensor qkv;      // fused Q|K|V (or Q|K when V's format differs)
  bool v_separate = false;
  DevTensor gate_up;  // fused gate|up
  // a projection tensor absent (or Q, K / gate, up in different formats): the present ones run
  // unfused, the absent ones as project_or_deterministic_slice's fallback
  bool qkv_split = false, gu_split = false;
  // a model with an MoE spec (jero_hip_model_set_moe): dispatch_qwen3_moe_ffn's tensors
  // (src/qwen_deepseek.rs:847-951) -- the router ffn_gate_inp, the stacked routed experts
  // ffn_{gate,up,down}_exps, the shared expert ffn_{gate,up,down}_shexp; exp_probs_b is refused
  DevTensor router, gate_exps, up_exps, down_exps, gate_shexp, up_shexp, down_shexp;
  bool probs_bias = false;
  bool routed = false;  // router and experts present: the routed path, else the dense fallback
  int64_t n_experts = 0, exp_ffn = 0;  // the router's experts (eff_experts, :882-888), rows per expert
};

// Row buffers of the batched prefill, grown on demand (rows tokens at a time).
struct PrefillBufs {
  int64_t rows = 0;
  size_t ws_bytes = 0;
  int32_t* tok = nullptr;
  float *X = nullptr, *XN = nullptr, *T = nullptr, *T2 = nullptr, *QKV = nullptr, *ATT = nullptr, *GU = nullptr,
        *ACT = nullptr, *RC = nullptr, *ws = nullptr;
  uint8_t* XQ = nullptr;
  // the MoE FFN over token rows: router logits and selections of one chunk, its workspace
  float *LG = nullptr, *SW = nullptr;
  int32_t* SI = nullptr;
  void* MWS = nullptr;
};

}  // namespace jero

struct jero_model {
  jero_model_config cfg{};
  jero::DevTensor tok_embd, output, output_norm;
  // The LM head as the step runs it (set by finalize; project_lm_head, src/qwen_deepseek.rs:584-632):
  // head_mode says how, `head` is the tensor read as [hidden, head_rows] rows (output.weight, or a
  // copy of token_embd.weight when output.weight is absent), logits_len = infer_logits_buffer_len.
  int head_mode = 0;
  jero::DevTensor head;
  int64_t head_rows = 0, logits_len = 0;
  int64_t embd_rows = 0;  // rows of `hidden` elements in token_embd.weight (0: absent)
  float* head_xn = nullptr;  // the normalised head input of an f32-input (F32 / F16 / BF16) head
  std::vector<jero::LayerW> layers;
  bool finalized = false;
  // device state
  float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
  float* attn_ws = nullptr;
  float* gu = nullptr;  // gate | up rows of layers that compute them apart [2 ffn]
  float* amax_v = nullptr;
  int64_t* amax_i = nullptr;
  int32_t* token = nullptr;
  int64_t* pos = nullptr;
  int32_t* status = nullptr;  // sticky: nonzero after a step whose logits held no argmax
  // the MoE spec (MoeDispatchSpec, src/qwen_deepseek.rs:81-87): set by jero_hip_model_set_moe
  // before the tensors; every layer's FFN is then dispatch_qwen3_moe_ffn (:1286-1300)
  bool moe = false, moe_shared = false;
  int64_t moe_experts = 0, moe_ffn = 0;
  int moe_top_k = 0;
  // its step buffers: RMSNorm(hidden) * ffn_norm, router logits, the shared expert's or dense
  // FFN's output, the selections, a Q8 row of the router input, the workspaces
  float *moe_xn = nullptr, *moe_logits = nullptr, *moe_y = nullptr, *moe_selw = nullptr;
  int32_t* moe_sel = nullptr;
  void *moe_xq = nullptr, *moe_ws = nullptr, *ffn_ws = nullptr;
  size_t moe_ws_bytes = 0, ffn_ws_bytes = 0;
  float* rope_cs = nullptr;
  void* kv = nullptr;
  size_t kv_bytes = 0;
  std::vector<void*> owned;
  uint8_t* trace = nullptr;  // debug trace buffer of the caller (jero_hip_model_trace), or null
  size_t trace_bytes = 0;
  jero::PrefillBufs pf;
  // GEMM layouts of the Q4_K / Q6_K tensors for the prefill (Q4_K_G, Q6_K_P), built on first use
  std::map<const void*, void*> laid;
  // the prefill's second stream (default priority) and its fork / join events, made on first use
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace jero {

static int dev_alloc(jero_model* m, size_t bytes, void** p) {
  if (hipMalloc(p, bytes < 256 ? 256 : bytes) != hipSuccess)
    return fail(JERO_ERR_INSUFFICIENT_MEMORY, "model: hipMalloc of " + std::to_string(bytes) + " bytes failed");
  m->owned.push_back(*p);
  return JERO_OK;
}

static void dev_free(jero_model* m, void* p) {
  for (auto& q : m->owned)
    if (q == p) {
      (void)hipFree(q);
      q = nullptr;
    }
}

static int64_t q_dim(const jero_model_config& c) { return int64_t(c.n_heads_q) * c.head_dim; }
static int64_t kv_dim(const jero_model_config& c) { return int64_t(c.n_heads_kv) * c.head_dim; }

// Expected (n_in, n_out) of a named tensor; returns false if the name is unknown.
// ffn: the dense FFN's rows (a model with an MoE spec runs its dense fallback with the expert
// FFN dimension, src/qwen_deepseek.rs:873-880).
static bool expected_shape(const jero_model_config& c, int64_t ffn, const std::string& base, int64_t& n_in,
                           int64_t& n_out) {
  const int64_t H = c.hidden, F = ffn, Q = q_dim(c), KV = kv_dim(c);
  static const std::map<std::string, int> kinds = {
      {"attn_norm.weight", 0}, {"ffn_norm.weight", 1}, {"attn_q_norm.weight", 2}, {"attn_k_norm.weight", 3},
      {"attn_q.weight", 4},    {"attn_k.weight", 5},   {"attn_v.weight", 6},      {"attn_output.weight", 7},
      {"ffn_gate.weight", 8},  {"ffn_up.weight", 9},   {"ffn_down.weight", 10}};
  auto it = kinds.find(base);
  if (it == kinds.end()) return false;
  switch (it->second) {
    case 0:
    case 1: n_in = H, n_out = 1; break;
    case 2:
    case 3: n_in = c.head_dim, n_out = 1; break;
    case 4: n_in = H, n_out = Q; break;
    case 5:
    case 6: n_in = H, n_out = KV; break;
    case 7: n_in = Q, n_out = H; break;
    case 8:
    case 9: n_in = H, n_out = F; break;
    case 10: n_in = F, n_out = H; break;
  }
  return true;
}

static DevTensor* find_slot(jero_model* m, const std::string& name, int64_t& n_in, int64_t& n_out) {
  const auto& c = m->cfg;
  if (name == "token_embd.weight") {
    n_in = c.hidden, n_out = c.vocab;
    return &m->tok_embd;
  }
  if (name == "output.weight") {
    n_in = c.hidden, n_out = c.vocab;
    return &m->output;
  }
  if (name == "output_norm.weight") {
    n_in = c.hidden, n_out = 1;
    return &m->output_norm;
  }
  if (name.rfind("blk.", 0) != 0) return nullptr;
  size_t dot = name.find('.', 4);
  if (dot == std::string::npos) return nullptr;
  int64_t L = -1;
  try {
    L = std::stoll(name.substr(4, dot - 4));
  } catch (...) {
    return nullptr;
  }
  if (L < 0 || L >= c.n_layers) return nullptr;
  std::string base = name.substr(dot + 1);
  LayerW& l = m->layers[size_t(L)];
  if (m->moe) {  // dispatch_qwen3_moe_ffn's tensors: shapes checked at finalize (n_in, n_out 0 here)
    static const std::map<std::string, DevTensor LayerW::*> moe_slots = {
        {"ffn_gate_inp.weight", &LayerW::router},     {"ffn_gate_exps.weight", &LayerW::gate_exps},
        {"ffn_up_exps.weight", &LayerW::up_exps},     {"ffn_down_exps.weight", &LayerW::down_exps},
        {"ffn_gate_shexp.weight", &LayerW::gate_shexp}, {"ffn_up_shexp.weight", &LayerW::up_shexp},
        {"ffn_down_shexp.weight", &LayerW::down_shexp}};
    auto it = moe_slots.find(base);
    if (it != moe_slots.end()) {
      n_in = n_out = 0;
      return &(l.*(it->second));
    }
  }
  if (!expected_shape(c, m->moe ? m->moe_ffn : c.ffn, base, n_in, n_out)) return nullptr;
  static const std::map<std::string, DevTensor LayerW::*> slots = {
      {"attn_norm.weight", &LayerW::attn_norm}, {"ffn_norm.weight", &LayerW::ffn_norm},
      {"attn_q_norm.weight", &LayerW::q_norm},  {"attn_k_norm.weight", &LayerW::k_norm},
      {"attn_q.weight", &LayerW::wq},           {"attn_k.weight", &LayerW::wk},
      {"attn_v.weight", &LayerW::wv},           {"attn_output.weight", &LayerW::wo},
      {"ffn_gate.weight", &LayerW::gate},       {"ffn_up.weight", &LayerW::up},
      {"ffn_down.weight", &LayerW::down}};
  return &(l.*(slots.at(base)));
}

static bool is_norm(const std::string& name) {
  return name.size() >= 12 && name.compare(name.size() - 12, 12, "_norm.weight") == 0;
}

// The layer projections that project_or_deterministic_slice computes (src/gemma.rs:841-860).
static bool is_projection(const std::string& name) {
  static const char* const kinds[] = {".attn_q.weight", ".attn_k.weight", ".attn_v.weight", ".attn_output.weight",
                                      ".ffn_gate.weight", ".ffn_up.weight", ".ffn_down.weight"};
  if (name.compare(0, 4, "blk.") != 0) return false;
  for (const char* k : kinds) {
    const size_t n = strlen(k);
    if (name.size() > n && name.compare(name.size() - n, n, k) == 0) return true;
  }
  return false;
}

// Rows of a and b stacked into one new tensor (same format and n_in).
static int concat_rows(jero_model* m, std::vector<DevTensor*> parts, DevTensor& out) {
  size_t total = 0;
  for (auto* t : parts) total += t->bytes;
  void* p = nullptr;
  int rc = dev_alloc(m, total, &p);
  if (rc) return rc;
  size_t off = 0;
  int64_t rows = 0;
  for (auto* t : parts) {
    rc = check_hip(hipMemcpy(static_cast<uint8_t*>(p) + off, t->dev, t->bytes, hipMemcpyDeviceToDevice), "concat");
    if (rc) return rc;
    off += t->bytes;
    rows += t->n_out;
  }
  out = {parts[0]->quant, p, total, parts[0]->n_in, rows};
  for (auto* t : parts) {
    dev_free(m, t->dev);
    t->dev = nullptr;
  }
  return JERO_OK;
}

// Q4_K / Q6_K tensors become Q4_K_R / Q6_K_R (same bytes, aligned planes).
static int repack_planar(jero_model* m, DevTensor& t) {
  if (t.quant != JERO_Q4_K && t.quant != JERO_Q6_K) return JERO_OK;
  void* p = nullptr;
  int rc = dev_alloc(m, t.bytes, &p);
  if (rc) return rc;
  int q = 0;
  rc = launch_repack(t.quant, t.dev, t.n_in, t.n_out, p, &q, nullptr);
  if (rc) return rc;
  rc = check_hip(hipDeviceSynchronize(), "repack");
  if (rc) return rc;
  dev_free(m, t.dev);
  t.dev = p;
  t.quant = q;
  return JERO_OK;
}

constexpr int kArgmaxSlots = 4096;

// How the LM head runs (chosen at finalize):
//   kHeadFused  a quantized GEMV over all logits_len rows, argmax in its epilogue;
//   kHeadTail   a quantized GEMV over head_rows < logits_len rows, then the 0.05 slice for the rest;
//   kHeadFloat  an F32 / F16 / BF16 head: RMSNorm, the float GEMV over head_rows, the slice for any
//               rest, then an argmax over all logits;
//   kHeadNone   no usable head: the tanh fallback for every logit.
enum { kHeadFused = 0, kHeadTail = 1, kHeadFloat = 2, kHeadNone = 3 };

// Byte offsets of the debug trace of one decode step (the layout include/jero_hip.h documents):
// per layer the fields below in this order, each starting on a 16-byte boundary, then the
// head's fields.  act_bytes(n) is the larger of the Q8_K and ACT_Q8 block sizes of n elements.
struct TraceLayout {
  enum { kXIn, kXnAttn, kQ8Attn, kQkv, kQRope, kKRope, kAttn, kQ8Wo, kXMid, kXnFfn, kQ8Ffn, kGu, kAct, kQ8Down, kFields };
  size_t field[kFields];
  size_t layer_bytes, x_final, xn_head, q8_head, rope_cs, total;
};

static size_t round16(size_t n) { return (n + 15) & ~size_t(15); }
static size_t trace_act_bytes(int64_t n) {
  const size_t a = size_t(n / 32) * 36, b = n % 256 == 0 ? size_t(n / 256) * 292 : 0;
  return round16(a > b ? a : b);
}

static TraceLayout trace_layout(const jero_model_config& c) {
  const int64_t H = c.hidden, F = c.ffn, Q = q_dim(c), KV = kv_dim(c);
  const size_t sizes[TraceLayout::kFields] = {
      round16(4 * size_t(H)),  round16(4 * size_t(H)), trace_act_bytes(H),     round16(4 * size_t(Q + 2 * KV)),
      round16(4 * size_t(Q)),  round16(4 * size_t(KV)), round16(4 * size_t(Q)), trace_act_bytes(Q),
      round16(4 * size_t(H)),  round16(4 * size_t(H)), trace_act_bytes(H),     round16(8 * size_t(F)),
      round16(4 * size_t(F)),  trace_act_bytes(F)};
  TraceLayout t{};
  size_t off = 0;
  for (int i = 0; i < TraceLayout::kFields; i++) {
    t.field[i] = off;
    off += sizes[i];
  }
  t.layer_bytes = off;
  const size_t tail = t.layer_bytes * size_t(c.n_layers);
  t.x_final = tail;
  t.xn_head = tail + round16(4 * size_t(H));
  t.q8_head = t.xn_head + round16(4 * size_t(H));
  t.rope_cs = t.q8_head + trace_act_bytes(H);
  t.total = t.rope_cs + round16(4 * size_t(c.head_dim));
  return t;
}

static int gemv(jero_model* m, const DevTensor& w, const float* x, const float* norm, float eps, int out_mode,
                float* y, int64_t half, hipStream_t s, int* blocks = nullptr, float* tr_xn = nullptr,
                uint8_t* tr_q8 = nullptr, float* tr_gu = nullptr, int max_blocks = kArgmaxSlots) {
  DGemvArgs a{};
  a.w = static_cast<const uint8_t*>(w.dev);
  a.rb = row_bytes(w.quant, w.n_in);
  a.U = int(w.n_in / ((w.quant == JERO_Q8_0 || w.quant == JERO_Q4_0) ? 32 : 64));
  a.N = w.n_out;
  a.x = x;
  a.norm_w = norm;
  a.eps = eps;
  a.K = int(w.n_in);
  a.y = y;
  a.half = half;
  a.amax_v = m->amax_v;
  a.amax_i = m->amax_i;
  a.max_blocks = max_blocks;  // one argmax partial slot per workgroup
  a.tr_xn = tr_xn;
  a.tr_q8 = tr_q8;
  a.tr_gu = tr_gu;
  return launch_dgemv(w.quant, out_mode, a, s, blocks);
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_model_create(const jero_model_config* cfg, jero_model** out) {
  if (!cfg || !out) return fail(JERO_ERR_INVALID_ARGUMENT, "model_create: null pointer");
  *out = nullptr;
  const auto& c = *cfg;
  if (c.hidden <= 0 || c.ffn <= 0 || c.n_layers <= 0 || c.vocab <= 0 || c.kv_capacity <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "model_create: empty dimension");
  int rc = check_attention_shape(c.n_heads_q, c.n_heads_kv, c.head_dim, c.kv_capacity);
  if (rc) return rc;
  if (c.kv_dtype != JERO_KV_F16 && c.kv_dtype != JERO_KV_F32)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "model_create: kv_dtype must be JERO_KV_F16 or JERO_KV_F32");
  if (c.hidden % 32 || c.ffn % 32 || q_dim(c) % 32)
    return fail(JERO_ERR_TENSOR_BOUNDS, "model_create: hidden, ffn and q dims must be multiples of 32");
  auto* m = new jero_model();
  m->cfg = c;
  m->layers.resize(size_t(c.n_layers));
  const int64_t Q = q_dim(c), KV = kv_dim(c);
  const size_t es = c.kv_dtype == JERO_KV_F16 ? 2 : 4;
  m->kv_bytes = size_t(c.n_layers) * 2 * size_t(c.kv_capacity) * size_t(KV) * es;
  const int max_blocks = kArgmaxSlots;
  void* p;
  if ((rc = dev_alloc(m, m->kv_bytes, &m->kv)) ||
      (rc = check_hip(hipMemset(m->kv, 0, m->kv_bytes), "kv zero")) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(c.hidden), &p)) || ((m->hidden = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(Q + 2 * KV), &p)) || ((m->qkv = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(Q), &p)) || ((m->attn = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(c.ffn), &p)) || ((m->act = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(c.vocab), &p)) || ((m->logits = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, attn_workspace_bytes(c.n_heads_q, c.head_dim, int(c.kv_capacity)), &p)) ||
      ((m->attn_ws = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * max_blocks, &p)) || ((m->amax_v = static_cast<float*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(int64_t) * max_blocks, &p)) || ((m->amax_i = static_cast<int64_t*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(int32_t), &p)) || ((m->token = static_cast<int32_t*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(int64_t), &p)) || ((m->pos = static_cast<int64_t*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(int32_t), &p)) || ((m->status = static_cast<int32_t*>(p)), false) ||
      (rc = dev_alloc(m, sizeof(float) * size_t(c.head_dim), &p)) || ((m->rope_cs = static_cast<float*>(p)), false)) {
    for (void* q : m->owned)
      if (q) (void)hipFree(q);
    delete m;
    return rc;
  }
  if ((rc = check_hip(hipMemset(m->token, 0, sizeof(int32_t)), "state")) ||
      (rc = check_hip(hipMemset(m->pos, 0, sizeof(int64_t)), "state")) ||
      (rc = check_hip(hipMemset(m->status, 0, sizeof(int32_t)), "state"))) {
    for (void* q : m->owned)
      if (q) (void)hipFree(q);
    delete m;
    return rc;
  }
  *out = m;
  return JERO_OK;
}

extern "C" int jero_hip_model_destroy(jero_model* m) {
  if (!m) return JERO_OK;
  (void)hipDeviceSynchronize();
  for (void* q : m->owned)
    if (q) (void)hipFree(q);
  if (m->ev_fork) (void)hipEventDestroy(m->ev_fork);
  if (m->ev_join) (void)hipEventDestroy(m->ev_join);
  if (m->side) (void)hipStreamDestroy(m->side);
  delete m;
  return JERO_OK;
}

extern "C" int jero_hip_model_set_tensor(jero_model* m, const char* name, int quant, const void* src, size_t nbytes,
                                         int64_t n_in, int64_t n_out, int src_on_device) {
  if (!m || !name || !src) return fail(JERO_ERR_INVALID_ARGUMENT, "set_tensor: null pointer");
  if (m->finalized) return fail(JERO_ERR_INVALID_ARGUMENT, "set_tensor: model already finalized");
  int64_t ein = 0, eout = 0;
  const std::string nm(name);
  static const std::string kProbsBias = ".exp_probs_b.bias";
  if (m->moe && nm.rfind("blk.", 0) == 0 && nm.size() > kProbsBias.size() &&
      nm.compare(nm.size() - kProbsBias.size(), kProbsBias.size(), kProbsBias) == 0) {
    // select_experts_with_optional_bias's routing bias (DeepSeek; src/qwen_deepseek.rs:773-834):
    // recorded so that finalize refuses the model
    const int64_t L = std::atoll(nm.c_str() + 4);
    if (L < 0 || L >= m->cfg.n_layers) return fail(JERO_ERR_CAPABILITY_MISMATCH, "set_tensor: unknown tensor '" + nm + "'");
    m->layers[size_t(L)].probs_bias = true;
    return JERO_OK;
  }
  DevTensor* slot = find_slot(m, name, ein, eout);
  if (!slot) return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string("set_tensor: unknown tensor '") + name + "'");
  if (ein == 0) {  // an MoE tensor: any shape here, its bytes must match it
    const int64_t rb = row_bytes(quant, n_in);
    if (n_in <= 0 || n_out <= 0 || !is_weight_quant(quant))
      return fail(JERO_ERR_TENSOR_BOUNDS, "set_tensor: '" + nm + "' is empty or of an unknown format");
    if (rb < 0 || size_t(rb) * size_t(n_out) != nbytes)
      return fail(JERO_ERR_TENSOR_BOUNDS, "set_tensor: '" + nm + "' byte size " + std::to_string(nbytes) +
                                              " does not match its shape");
    if (slot->dev) dev_free(m, slot->dev);
    void* p = nullptr;
    int rc = dev_alloc(m, nbytes, &p);
    if (rc) return rc;
    if ((rc = check_hip(hipMemcpy(p, src, nbytes, src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice),
                        "set_tensor upload")))
      return rc;
    *slot = {quant, p, nbytes, n_in, n_out};
    return JERO_OK;
  }
  if (is_projection(name) && n_in * n_out != ein * eout) {
    // project_or_deterministic_slice (src/gemma.rs:841-860) uses a tensor only when its element count
    // is out_len * in_len; any other takes the deterministic fallback, as if it were absent
    if (slot->dev) dev_free(m, slot->dev);
    *slot = DevTensor{};
    return JERO_OK;
  }
  const bool norm = is_norm(name);
  const bool embd = std::string(name) == "token_embd.weight";
  const bool head = std::string(name) == "output.weight";
  const bool float_w = quant == JERO_F32 || quant == JERO_F16 || quant == JERO_BF16;
  // Norms, the embedding and the head are read the way the reference reads them, whatever their
  // shape (read_f32_weight_or_default, embed_token, project_lm_head); the projections must have
  // their layer shape.
  if (n_in <= 0 || n_out <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, std::string("set_tensor: '") + name + "' is empty");
  if (!norm && !embd && !head && (n_in != ein || n_out != eout))
    return fail(JERO_ERR_TENSOR_BOUNDS, std::string("set_tensor: '") + name + "' has shape [" + std::to_string(n_in) +
                                            ", " + std::to_string(n_out) + "], expected [" + std::to_string(ein) +
                                            ", " + std::to_string(eout) + "]");
  if (!is_weight_quant(quant) || (float_w && !norm && !embd && !head))
    return fail(JERO_ERR_CAPABILITY_MISMATCH,
                std::string("set_tensor: '") + name + "' quantization " + std::to_string(quant) +
                    " unsupported by the decode step (projections: Q8_0, Q4_0, Q4_K, Q6_K; norms, the embedding "
                    "and the head also F32, F16, BF16)");
  const int64_t rb = row_bytes(quant, n_in);
  if (rb < 0 || size_t(rb) * size_t(n_out) != nbytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, std::string("set_tensor: '") + name + "' byte size " + std::to_string(nbytes) +
                                            " does not match its shape");
  if (embd && row_bytes(quant, m->cfg.hidden) < 0)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string("set_tensor: token_embd.weight rows of ") +
                                                  std::to_string(m->cfg.hidden) + " elements are not whole blocks");
  if (!norm && !embd && !head && n_in > dgemv_long_max_k(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string("set_tensor: '") + name + "' rows of " +
                                                  std::to_string(n_in) + " elements exceed the decode limit " +
                                                  std::to_string(dgemv_long_max_k(quant)));
  if (slot->dev) dev_free(m, slot->dev);
  void* p = nullptr;
  int rc = dev_alloc(m, nbytes, &p);
  if (rc) return rc;
  rc = check_hip(hipMemcpy(p, src, nbytes, src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice),
                 "set_tensor upload");
  if (rc) return rc;
  *slot = {quant, p, nbytes, n_in, n_out};
  return JERO_OK;
}

namespace jero {

static jero_hip_tensor view_of(const DevTensor& t) {
  return jero_hip_tensor{t.quant, t.dev, t.bytes, t.present() ? t.n_in * t.n_out : 0};
}

// One layer of a model with an MoE spec, at finalize: dispatch_qwen3_moe_ffn's choices
// (src/qwen_deepseek.rs:873-946) made once.  A router with experts takes the routed path: the
// router's experts eff_experts = its elements / hidden (at most num_experts, :882-888), the stacked
// gate / up / down tensors of that many experts re-laid out in 16-row tiles for the expert kernels.
// Without a router (or with num_experts or top_k 0, or without expert tensors: ran_any_expert false)
// the layer runs run_dense_swiglu_ffn with the expert FFN dimension (:873-880, :942-946).
// The launch arguments of layer l's routed experts (its router's E, top-k, the stacked expert
// tensors as finalize left them); the caller sets the tokens, inputs and outputs.
static MoeArgs moe_args_of(const jero_model* m, const LayerW& l) {
  MoeArgs a{};
  a.E = l.n_experts;
  a.top_k = m->moe_top_k;
  a.gate_quant = l.gate_exps.quant;
  a.up_quant = l.up_exps.quant;
  a.down_quant = l.down_exps.quant;
  a.gate = l.gate_exps.dev;
  a.up = l.up_exps.dev;
  a.down = l.down_exps.dev;
  a.hidden = m->cfg.hidden;
  a.ffn = l.exp_ffn;
  return a;
}

static int moe_layer_finalize(jero_model* m, int64_t L, LayerW& l) {
  const int64_t H = m->cfg.hidden;
  const std::string at = "finalize: layer " + std::to_string(L) + ": ";
  if (l.probs_bias)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, at + "exp_probs_b.bias (the routing bias of "
                                                   "select_experts_with_optional_bias) is not supported");
  const int n_exp = int(l.gate_exps.present()) + int(l.up_exps.present()) + int(l.down_exps.present());
  l.routed = m->moe_experts > 0 && m->moe_top_k > 0 && l.router.present() && n_exp == 3;
  if (m->moe_experts > 0 && m->moe_top_k > 0 && l.router.present() && n_exp != 0 && n_exp != 3)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, at + "an incomplete set of ffn_{gate,up,down}_exps tensors");
  if (!l.routed) return JERO_OK;
  const int64_t re = l.router.n_in * l.router.n_out;
  const int64_t E = (re > 0 && re % H == 0) ? std::min(re / H, m->moe_experts) : m->moe_experts;
  if (E * H > re || !(is_float_weight(l.router.quant) || act_format(l.router.quant) >= 0))
    return fail(JERO_ERR_TENSOR_BOUNDS, at + "the router does not hold " + std::to_string(E) + " rows of " +
                                            std::to_string(H) + " elements in a GEMV format");
  if (l.gate_exps.n_in != H || l.up_exps.n_in != H || l.gate_exps.n_out % E || l.gate_exps.n_out != l.up_exps.n_out)
    return fail(JERO_ERR_TENSOR_BOUNDS, at + "ffn_gate_exps / ffn_up_exps must be [hidden, ffn, n_experts]");
  const int64_t F = l.gate_exps.n_out / E;
  if (l.down_exps.n_in != F || l.down_exps.n_out != H * E)
    return fail(JERO_ERR_TENSOR_BOUNDS, at + "ffn_down_exps must be [ffn, hidden, n_experts]");
  if (l.gate_exps.quant != l.up_exps.quant)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, at + "ffn_gate_exps and ffn_up_exps in different formats");
  if (m->moe_top_k > E)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, at + "top_k above the router's " + std::to_string(E) + " experts");
  l.n_experts = E;
  l.exp_ffn = F;
  // the expert kernels read the 16-row tile layouts fastest (Q4_K_T / Q6_K_T, jero_hip_repack_experts)
  for (DevTensor* t : {&l.gate_exps, &l.up_exps, &l.down_exps}) {
    const int64_t rows_per = t->n_out / E;
    if ((t->quant == JERO_Q4_K || t->quant == JERO_Q6_K) && rows_per % 16 == 0) {
      void* p = nullptr;
      int dq = -1;
      int rc = dev_alloc(m, t->bytes, &p);
      if (rc || (rc = launch_repack_experts(t->quant, t->dev, t->n_in, t->n_out, p, &dq, nullptr)) ||
          (rc = check_hip(hipDeviceSynchronize(), "expert repack")))
        return rc;
      dev_free(m, t->dev);
      t->dev = p;
      t->quant = dq;
    }
  }
  MoeArgs a = moe_args_of(m, l);
  a.x = a.logits = reinterpret_cast<const float*>(l.router.dev);  // non-null stand-ins for the check
  a.T = 1;
  a.y = reinterpret_cast<float*>(l.router.dev);
  a.sel_idx = reinterpret_cast<int32_t*>(l.router.dev);
  a.sel_w = a.y;
  const int rc = check_moe_args(a, l.gate_exps.bytes, l.up_exps.bytes, l.down_exps.bytes);
  return rc ? fail(rc, at + jero_hip_last_error()) : JERO_OK;
}

// The step buffers of a model with an MoE spec (sized for its largest layer).
static int moe_buffers(jero_model* m) {
  const auto& c = m->cfg;
  const int64_t H = c.hidden;
  int64_t E = 1, F = 4;
  for (const LayerW& l : m->layers) {
    E = std::max(E, l.n_experts);
    F = std::max(F, l.exp_ffn);
  }
  const int k = std::max(1, m->moe_top_k);
  // the dense FFNs (the shared expert, the fallback): their row counts as jero_hip_swiglu_ffn takes them
  int64_t Fd = std::max<int64_t>(m->moe_ffn, 4);
  for (const LayerW& l : m->layers) {
    const int64_t ge = l.gate_shexp.present() ? l.gate_shexp.n_in * l.gate_shexp.n_out : 0;
    if (ge > 0 && ge % H == 0) Fd = std::max(Fd, ge / H);
  }
  m->moe_ws_bytes = moe_workspace_bytes(1, E, k, H, F);
  m->ffn_ws_bytes = jero_hip_swiglu_ffn_workspace_bytes(H, Fd);
  void* p = nullptr;
  int rc;
  if ((rc = dev_alloc(m, sizeof(float) * size_t(H), &p))) return rc;
  m->moe_xn = static_cast<float*>(p);
  if ((rc = dev_alloc(m, sizeof(float) * size_t(E), &p))) return rc;
  m->moe_logits = static_cast<float*>(p);
  if ((rc = dev_alloc(m, sizeof(float) * size_t(H), &p))) return rc;
  m->moe_y = static_cast<float*>(p);
  if ((rc = dev_alloc(m, sizeof(float) * size_t(k), &p))) return rc;
  m->moe_selw = static_cast<float*>(p);
  if ((rc = dev_alloc(m, sizeof(int32_t) * size_t(k), &p))) return rc;
  m->moe_sel = static_cast<int32_t*>(p);
  if ((rc = dev_alloc(m, size_t(H / 32 + 1) * 36 + size_t(H / 256 + 1) * 292, &m->moe_xq))) return rc;
  if ((rc = dev_alloc(m, m->moe_ws_bytes, &m->moe_ws))) return rc;
  return dev_alloc(m, m->ffn_ws_bytes, &m->ffn_ws);
}

// The FFN of layer L of a model with an MoE spec (src/qwen_deepseek.rs:1278-1303):
// xn = rmsnorm(hidden) * ffn_norm, out = dispatch_qwen3_moe_ffn(xn) -- the shared expert first,
// then either the routed sum added onto it in selection order or the dense fallback -- and
// hidden += out.  The routed path adds out to hidden in its last kernel; the trace (when set)
// gets xn and the router logits.
static int moe_ffn_step(jero_model* m, const LayerW& l, float eps, hipStream_t s, float* tr_xn, float* tr_logits) {
  const int64_t H = m->cfg.hidden;
  const float* nw = static_cast<const float*>(l.ffn_norm.dev);
  // an F32 router computes the norm itself (one launch for both); otherwise the norm runs alone
  const bool fused = l.routed && router_norm_fits(l.router.quant, l.router.dev, H, m->hidden, m->moe_xn);
  int rc = fused ? launch_router_norm(l.router.dev, H, l.n_experts, m->hidden, nw, eps, m->moe_xn, m->moe_logits, s)
                 : launch_head_norm(m->hidden, nw, eps, H, m->moe_xn, s);
  if (rc) return rc;
  const bool shared = m->moe_shared && l.gate_shexp.present() && l.up_shexp.present() && l.down_shexp.present();
  if (shared) {  // :860-871
    const jero_hip_tensor g = view_of(l.gate_shexp), u = view_of(l.up_shexp), d = view_of(l.down_shexp);
    if ((rc = jero_hip_swiglu_ffn(JERO_FFN_SHARED_EXPERT, m->moe_xn, H, m->moe_ffn, &g, &u, &d, 0, m->moe_y, m->ffn_ws,
                                  m->ffn_ws_bytes, s)))
      return rc;
  }
  if (!l.routed) {  // run_dense_swiglu_ffn with the expert FFN dimension (:873-880, :942-946)
    const jero_hip_tensor g = view_of(l.gate), u = view_of(l.up), d = view_of(l.down);
    if ((rc = jero_hip_swiglu_ffn(JERO_FFN_DENSE, m->moe_xn, H, m->moe_ffn, &g, &u, &d, shared ? 1 : 0, m->moe_y,
                                  m->ffn_ws, m->ffn_ws_bytes, s)))
      return rc;
    rc = launch_det_proj(m->moe_y, H, nullptr, 0.f, 1.0f, m->hidden, H, true, s);  // hidden += out (x * 1 exact)
  } else {
    // router logits (matvec_any over the router's eff_experts rows, :882-890): the fused launch
    // above wrote them; otherwise the GEMV of float rows, or of quantized rows over xn quantized
    const int E = int(l.n_experts);
    if (!fused) {
      if (is_float_weight(l.router.quant))
        rc = launch_matvec_float(l.router.quant, l.router.dev, H, E, m->moe_xn, m->moe_logits, s);
      else if (!(rc = launch_quantize_act(act_format(l.router.quant), m->moe_xn, 1, H, m->moe_xq, s)))
        rc = launch_matvec(l.router.quant, l.router.dev, H, E, m->moe_xq, m->moe_logits, nullptr, s);
      if (rc) return rc;
    }
    if (tr_logits && (rc = check_hip(hipMemcpyAsync(tr_logits, m->moe_logits, sizeof(float) * size_t(E),
                                                    hipMemcpyDeviceToDevice, s), "decode trace copy")))
      return rc;
    // select_top_k_experts and the experts' SwiGLU, summed in selection order onto the shared
    // expert's output (or zero) and that sum added to hidden (:890-938, :1301-1303)
    MoeArgs a = moe_args_of(m, l);
    a.x = m->moe_xn;
    a.logits = m->moe_logits;
    a.T = 1;
    a.y = m->moe_y;
    a.accumulate = shared;
    a.resid = m->hidden;
    a.sel_idx = m->moe_sel;
    a.sel_w = m->moe_selw;
    rc = launch_moe(a, m->moe_ws, s);
  }
  if (rc) return rc;
  if (tr_xn)
    rc = check_hip(hipMemcpyAsync(tr_xn, m->moe_xn, sizeof(float) * size_t(H), hipMemcpyDeviceToDevice, s),
                   "decode trace copy");
  return rc;
}

}  // namespace jero

extern "C" int jero_hip_model_set_moe(jero_model* m, int64_t n_experts, int top_k, int64_t expert_ffn,
                                      int use_shared) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "set_moe: null model");
  if (m->finalized) return fail(JERO_ERR_INVALID_ARGUMENT, "set_moe: model already finalized");
  if (n_experts < 0 || top_k < 0 || expert_ffn <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "set_moe: negative experts or top_k, or an empty expert FFN");
  for (const LayerW& l : m->layers)
    if (l.gate.present() || l.up.present() || l.down.present())
      return fail(JERO_ERR_INVALID_ARGUMENT, "set_moe: call it before the FFN tensors are set");
  m->moe = true;
  m->moe_experts = n_experts;
  m->moe_top_k = top_k;
  m->moe_ffn = expert_ffn;
  m->moe_shared = use_shared != 0;
  return JERO_OK;
}

extern "C" int jero_hip_model_finalize(jero_model* m) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "finalize: null model");
  if (m->finalized) return JERO_OK;
  const auto& c = m->cfg;
  const int64_t H = c.hidden;
  int rc;
  // Norm weights as read_f32_weight_or_default reads them (src/qwen_deepseek.rs:491-519): an
  // absent one is all ones, F32 values that are not finite become 1.0, other formats are
  // dequantized from their first len elements (when they hold whole blocks of them); each
  // becomes an f32 vector of len.
  auto norm_weight = [&](DevTensor& t, int64_t len) -> int {
    void* p = nullptr;
    int r = dev_alloc(m, sizeof(float) * size_t(len), &p);
    if (r) return r;
    const int64_t n_el = t.present() ? t.n_in * t.n_out : 0;
    const bool deq = t.present() && t.quant != JERO_F32 && n_el >= len && row_bytes(t.quant, len) >= 0;
    if ((r = launch_norm_weight(t.quant, t.dev, n_el, len, deq, static_cast<float*>(p), nullptr)) ||
        (r = check_hip(hipDeviceSynchronize(), "norm weight")))
      return r;
    if (t.dev) dev_free(m, t.dev);
    t = {JERO_F32, p, sizeof(float) * size_t(len), len, 1};
    return JERO_OK;
  };
  if ((rc = norm_weight(m->output_norm, H))) return rc;
  for (int64_t L = 0; L < c.n_layers; L++) {
    LayerW& l = m->layers[size_t(L)];
    if ((rc = norm_weight(l.attn_norm, H)) || (rc = norm_weight(l.ffn_norm, H))) return rc;
    if (c.qk_norm && ((rc = norm_weight(l.q_norm, c.head_dim)) || (rc = norm_weight(l.k_norm, c.head_dim)))) return rc;
    // the projections may be absent (project_or_deterministic_slice's fallback)
    l.qkv_split = !l.wq.present() || !l.wk.present() || !l.wv.present() || l.wq.quant != l.wk.quant;
    l.gu_split = !l.gate.present() || !l.up.present() || l.gate.quant != l.up.quant;
    if (l.qkv_split) {
      for (DevTensor* t : {&l.wq, &l.wk, &l.wv})
        if (t->present() && (rc = repack_planar(m, *t))) return rc;
    } else {
      l.v_separate = l.wv.quant != l.wq.quant;
      if (l.v_separate) {
        if ((rc = concat_rows(m, {&l.wq, &l.wk}, l.qkv))) return rc;
        if ((rc = repack_planar(m, l.wv))) return rc;
      } else {
        if ((rc = concat_rows(m, {&l.wq, &l.wk, &l.wv}, l.qkv))) return rc;
      }
      if ((rc = repack_planar(m, l.qkv))) return rc;
    }
    if (m->moe) {  // the dense tensors, if any, serve the MoE dispatch's fallback in their GGUF layout
      if ((rc = moe_layer_finalize(m, L, l))) return rc;
    } else if (l.gu_split) {
      for (DevTensor* t : {&l.gate, &l.up})
        if (t->present() && (rc = repack_planar(m, *t))) return rc;
      if (!m->gu) {
        void* g = nullptr;
        if ((rc = dev_alloc(m, sizeof(float) * 2 * size_t(c.ffn), &g))) return rc;
        m->gu = static_cast<float*>(g);
      }
    } else {
      if ((rc = concat_rows(m, {&l.gate, &l.up}, l.gate_up))) return rc;
      if ((rc = repack_planar(m, l.gate_up))) return rc;
    }
    if (l.wo.present() && (rc = repack_planar(m, l.wo))) return rc;
    if (!m->moe && l.down.present() && (rc = repack_planar(m, l.down))) return rc;
  }
  if (m->moe && (rc = moe_buffers(m))) return rc;
  // embed_token's rows (num_elements / hidden) and the LM head of project_lm_head
  // (src/qwen_deepseek.rs:584-632): output.weight, else token_embd.weight (ModelWeights' tied
  // fallback, src/weights.rs:1110-1126), with logits_len = infer_logits_buffer_len
  // (src/engine.rs:1781-1792): the head's rows when they exceed vocab by at most 1024 and are a
  // multiple of 64.
  m->embd_rows = m->tok_embd.present() ? m->tok_embd.n_in * m->tok_embd.n_out / H : 0;
  const bool tied = !m->output.present() && m->tok_embd.present();
  const DevTensor* src = m->output.present() ? &m->output : tied ? &m->tok_embd : nullptr;
  int64_t Ln = c.vocab;
  if (src && src->n_out > c.vocab && src->n_out % 64 == 0 && src->n_out - c.vocab <= 1024) Ln = src->n_out;
  if (Ln > int64_t(kArgmaxSlots) * kHeadTailRows)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "finalize: " + std::to_string(Ln) + " logits exceed the head's limit");
  m->logits_len = Ln;
  if (Ln > c.vocab) {
    void* p = nullptr;
    if ((rc = dev_alloc(m, sizeof(float) * size_t(Ln), &p))) return rc;
    dev_free(m, m->logits);
    m->logits = static_cast<float*>(p);
  }
  DevTensor hd{};
  int64_t rows = 0;
  if (src && src->n_in == H) {  // [hidden, rows]: its first min(logits_len, rows) rows (:607-618)
    hd = *src;
    rows = std::min(Ln, src->n_out);
  } else if (src && src->n_in * src->n_out == Ln * H && row_bytes(src->quant, H) >= 0) {
    hd = *src;  // logits_len * hidden elements in another shape: rows of hidden (:620-623)
    hd.n_in = H;
    hd.n_out = Ln;
    rows = Ln;
  }
  m->head_rows = rows;
  const bool float_head = hd.present() && (hd.quant == JERO_F32 || hd.quant == JERO_F16 || hd.quant == JERO_BF16);
  if (!hd.present()) {
    m->head_mode = kHeadNone;
  } else if (float_head) {
    m->head_mode = kHeadFloat;  // read in place (the embedding's own bytes when tied)
    m->head = hd;
    void* p = nullptr;
    if ((rc = dev_alloc(m, sizeof(float) * size_t(H), &p))) return rc;
    m->head_xn = static_cast<float*>(p);
  } else {
    if (H > dgemv_long_max_k(hd.quant))
      return fail(JERO_ERR_CAPABILITY_MISMATCH, "finalize: head rows of " + std::to_string(H) +
                                                    " elements exceed the decode limit");
    if (tied) {  // the head's own copy: the embedding keeps its GGUF layout, the head goes planar
      void* p = nullptr;
      if ((rc = dev_alloc(m, hd.bytes, &p)) ||
          (rc = check_hip(hipMemcpy(p, hd.dev, hd.bytes, hipMemcpyDeviceToDevice), "head copy")))
        return rc;
      hd.dev = p;
    } else {
      m->output = DevTensor{};  // the head owns output.weight's buffer from here on
    }
    m->head = hd;
    if ((rc = repack_planar(m, m->head))) return rc;
    m->head_mode = rows < Ln ? kHeadTail : kHeadFused;
  }
  m->finalized = true;
  return JERO_OK;
}

extern "C" int jero_hip_model_kv(jero_model* m, int64_t layer, void** k_ring, void** v_ring) {
  if (!m || !k_ring || !v_ring) return fail(JERO_ERR_INVALID_ARGUMENT, "model_kv: null pointer");
  if (layer < 0 || layer >= m->cfg.n_layers) return fail(JERO_ERR_TENSOR_BOUNDS, "model_kv: layer out of range");
  const size_t es = m->cfg.kv_dtype == JERO_KV_F16 ? 2 : 4;
  const size_t ring = size_t(m->cfg.kv_capacity) * size_t(kv_dim(m->cfg)) * es;
  uint8_t* base = static_cast<uint8_t*>(m->kv) + size_t(layer) * 2 * ring;
  *k_ring = base;
  *v_ring = base + ring;
  return JERO_OK;
}

extern "C" int jero_hip_model_state(jero_model* m, int32_t** token_dev, int64_t** pos_dev, float** logits_dev) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "model_state: null model");
  if (token_dev) *token_dev = m->token;
  if (pos_dev) *pos_dev = m->pos;
  if (logits_dev) *logits_dev = m->logits;
  return JERO_OK;
}

extern "C" int jero_hip_model_set_position(jero_model* m, int32_t token, int64_t pos, void* stream) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "set_position: null model");
  if (token < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "set_position: negative token " + std::to_string(token));
  if (pos < 0) return fail(JERO_ERR_CONTEXT_LENGTH_EXCEEDED, "set_position: negative position");
  return launch_set_state(m->token, m->pos, m->status, token, pos, static_cast<hipStream_t>(stream));
}

extern "C" int64_t jero_hip_model_logits_len(const jero_model* m) {
  if (!m) return -1;
  return m->finalized ? m->logits_len : m->cfg.vocab;
}

extern "C" int64_t jero_hip_model_trace_bytes(const jero_model* m) {
  return m ? int64_t(trace_layout(m->cfg).total) : -1;
}

extern "C" int jero_hip_model_trace(jero_model* m, void* trace_dev, size_t trace_bytes) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "model_trace: null model");
  if (!trace_dev) {
    m->trace = nullptr;
    return JERO_OK;
  }
  const size_t need = trace_layout(m->cfg).total;
  if (trace_bytes < need)
    return fail(JERO_ERR_TENSOR_BOUNDS, "model_trace: buffer of " + std::to_string(trace_bytes) + " bytes, need " +
                                            std::to_string(need));
  if (reinterpret_cast<uintptr_t>(trace_dev) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "model_trace: buffer must be 16-byte aligned");
  m->trace = static_cast<uint8_t*>(trace_dev);
  m->trace_bytes = trace_bytes;
  return JERO_OK;
}

extern "C" int jero_hip_model_status(jero_model* m, void* stream) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "model_status: null model");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t st = 0;
  int rc = check_hip(hipStreamSynchronize(s), "model_status sync");
  if (rc) return rc;
  rc = check_hip(hipMemcpy(&st, m->status, sizeof(st), hipMemcpyDeviceToHost), "model_status read");
  if (rc) return rc;
  if (st != 0)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "empty logits buffer after decode step (or all-NaN)");
  return JERO_OK;
}

namespace jero {

// Final RMSNorm, project_lm_head (src/qwen_deepseek.rs:584-632) and the greedy token
// (sample_greedy_argmax, src/engine.rs:1873-1895) from the hidden state x [hidden] on the device,
// as finalize chose to run the head; tr_xn / tr_q8: the trace's head fields (or null).
static int head_step(jero_model* m, const float* x, hipStream_t s, float* tr_xn, uint8_t* tr_q8) {
  const auto& c = m->cfg;
  const int64_t H = c.hidden, Ln = m->logits_len;
  const float eps = c.rms_eps > 1e-6f ? c.rms_eps : 1e-6f;  // rms_eps.max(1e-6), :1250
  const float* nw = static_cast<const float*>(m->output_norm.dev);
  int nb = 0, rc = JERO_OK;
  switch (m->head_mode) {
    case kHeadFused:
    case kHeadTail: {
      const int tb = m->head_mode == kHeadTail ? head_tail_blocks(m->head_rows, Ln) : 0;
      DevTensor h = m->head;
      h.n_out = m->head_rows;
      if ((rc = gemv(m, h, x, nw, eps, kOutArgmax, m->logits, 0, s, &nb, tr_xn, tr_q8, nullptr, kArgmaxSlots - tb)))
        return rc;
      if (tb > 0) {  // the rows past the head: its argmax partials follow the GEMV's
        if ((rc = launch_head_tail(x, nw, eps, H, 0, m->head_rows, Ln, m->logits, m->amax_v + nb, m->amax_i + nb,
                                   nullptr, s)))
          return rc;
        nb += tb;
      }
      break;
    }
    case kHeadFloat: {
      if ((rc = launch_head_norm(x, nw, eps, H, m->head_xn, s))) return rc;
      if (tr_xn && (rc = check_hip(hipMemcpyAsync(tr_xn, m->head_xn, sizeof(float) * size_t(H),
                                                  hipMemcpyDeviceToDevice, s),
                                   "head trace copy")))
        return rc;
      if ((rc = launch_matvec_float(m->head.quant, m->head.dev, H, m->head_rows, m->head_xn, m->logits, s)) ||
          (rc = launch_head_tail(x, nw, eps, H, 0, m->head_rows, Ln, m->logits, nullptr, nullptr, nullptr, s)))
        return rc;
      nb = launch_argmax_partials(m->logits, Ln, m->amax_v, m->amax_i, s);
      if (nb < 0) return JERO_ERR_DEVICE;
      break;
    }
    default:  // no usable head: the tanh fallback for every logit
      if ((rc = launch_head_tail(x, nw, eps, H, 1, 0, Ln, m->logits, m->amax_v, m->amax_i, tr_xn, s))) return rc;
      nb = head_tail_blocks(0, Ln);
  }
  return launch_argmax_final(m->amax_v, m->amax_i, nb, m->token, m->pos, m->status, s);
}

}  // namespace jero

extern "C" int jero_hip_decode_step(jero_model* m, void* stream) {
  if (!m) return fail(JERO_ERR_INVALID_ARGUMENT, "decode_step: null model");
  if (!m->finalized) return fail(JERO_ERR_INVALID_ARGUMENT, "decode_step: call jero_hip_model_finalize first");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto& c = m->cfg;
  const int64_t Q = q_dim(c), KV = kv_dim(c);
  const float eps_attn = c.rms_eps;
  const float eps_ffn = c.rms_eps > 1e-6f ? c.rms_eps : 1e-6f;  // rms_eps.max(1e-6), :1250
  int rc = launch_embed(m->tok_embd.quant, m->tok_embd.dev, row_bytes(m->tok_embd.quant, c.hidden), int(c.hidden),
                        m->embd_rows, m->token, m->hidden, m->pos, c.rope_theta, c.head_dim, m->rope_cs, s);
  if (rc) return rc;
  const size_t es = c.kv_dtype == JERO_KV_F16 ? 2 : 4;
  const size_t ring = size_t(c.kv_capacity) * size_t(KV) * es;
  const TraceLayout tl = trace_layout(c);
  // debug trace: field f of layer L (null when tracing is off)
  auto tr = [&](int64_t L, int f) -> uint8_t* {
    return m->trace ? m->trace + size_t(L) * tl.layer_bytes + tl.field[f] : nullptr;
  };
  auto trf = [&](int64_t L, int f) -> float* { return reinterpret_cast<float*>(tr(L, f)); };
  auto snap = [&](uint8_t* dst, const void* src, size_t bytes) -> int {
    if (!dst) return JERO_OK;
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s), "decode trace copy");
  };
  if (m->trace && (rc = snap(m->trace + tl.rope_cs, m->rope_cs, 4 * size_t(c.head_dim)))) return rc;
  for (int64_t L = 0; L < c.n_layers; L++) {
    const LayerW& l = m->layers[size_t(L)];
    if ((rc = snap(tr(L, TraceLayout::kXIn), m->hidden, 4 * size_t(c.hidden)))) return rc;
    // attention sublayer: RMSNorm -> Q|K|V
    const bool dual = !l.qkv_split && l.v_separate && l.qkv.n_in <= 4096 &&
                      ((l.qkv.quant == JERO_Q4_K_R && l.wv.quant == JERO_Q6_K_R) ||
                       (l.qkv.quant == JERO_Q6_K_R && l.wv.quant == JERO_Q4_K_R));
    if (dual) {  // Q|K and V of different formats in one launch
      DGemvArgs a{};
      a.w = static_cast<const uint8_t*>(l.qkv.dev);
      a.rb = row_bytes(l.qkv.quant, l.qkv.n_in);
      a.U = int(l.qkv.n_in / 64);
      a.N = l.qkv.n_out;
      a.w2 = static_cast<const uint8_t*>(l.wv.dev);
      a.rb2 = row_bytes(l.wv.quant, l.wv.n_in);
      a.N2 = l.wv.n_out;
      a.x = m->hidden;
      a.norm_w = static_cast<const float*>(l.attn_norm.dev);
      a.eps = eps_attn;
      a.K = int(l.qkv.n_in);
      a.y = m->qkv;
      a.tr_xn = trf(L, TraceLayout::kXnAttn);
      a.tr_q8 = tr(L, TraceLayout::kQ8Attn);
      rc = launch_dgemv_dual(l.qkv.quant, l.wv.quant, a, s);
      if (rc) return rc;
    } else if (l.qkv_split) {
      // each of Q, K, V projected on its own or, absent, the fallback slice of the normalised input
      // (scales 0.5, 0.25, 0.125: src/qwen_deepseek.rs:1011-1031)
      const float* nw = static_cast<const float*>(l.attn_norm.dev);
      const DevTensor* w3[3] = {&l.wq, &l.wk, &l.wv};
      const int64_t off[3] = {0, Q, Q + KV}, len[3] = {Q, KV, KV};
      const float sc[3] = {0.5f, 0.25f, 0.125f};
      bool traced = false;
      for (int j = 0; j < 3; j++) {
        if (w3[j]->present()) {
          rc = gemv(m, *w3[j], m->hidden, nw, eps_attn, kOutStore, m->qkv + off[j], 0, s, nullptr,
                    traced ? nullptr : trf(L, TraceLayout::kXnAttn), traced ? nullptr : tr(L, TraceLayout::kQ8Attn));
          traced = true;
        } else {
          rc = launch_det_proj(m->hidden, c.hidden, nw, eps_attn, sc[j], m->qkv + off[j], len[j], false, s);
        }
        if (rc) return rc;
      }
    } else {
      rc = gemv(m, l.qkv, m->hidden, static_cast<const float*>(l.attn_norm.dev), eps_attn, kOutStore, m->qkv, 0, s,
                nullptr, trf(L, TraceLayout::kXnAttn), tr(L, TraceLayout::kQ8Attn));
      if (rc) return rc;
      if (l.v_separate) {
        rc = gemv(m, l.wv, m->hidden, static_cast<const float*>(l.attn_norm.dev), eps_attn, kOutStore,
                  m->qkv + Q + KV, 0, s);
        if (rc) return rc;
      }
    }
    // QK-norm, RoPE, KV append, attention over the ring
    AttnParams p{};
    uint8_t* base = static_cast<uint8_t*>(m->kv) + size_t(L) * 2 * ring;
    p.q = m->qkv;
    p.k = base;
    p.v = base + ring;
    p.kv_dtype = c.kv_dtype;
    p.nkv = c.n_heads_kv;
    p.group = c.n_heads_q / c.n_heads_kv;
    p.hd = c.head_dim;
    p.active = int(c.kv_capacity);
    p.scale = 1.0f / sqrtf(float(c.head_dim));
    p.part_o = m->attn_ws;
    p.k_new = m->qkv + Q;
    p.v_new = m->qkv + Q + KV;
    p.q_norm = c.qk_norm ? static_cast<const float*>(l.q_norm.dev) : nullptr;
    p.k_norm = c.qk_norm ? static_cast<const float*>(l.k_norm.dev) : nullptr;
    p.eps = eps_attn;
    p.theta = c.rope_theta;
    p.slot = -1;
    p.k_write = base;
    p.v_write = base + ring;
    p.pos_dev = m->pos;
    p.rope_cs = m->rope_cs;
    p.capacity = c.kv_capacity;
    p.tr_q = trf(L, TraceLayout::kQRope);
    p.tr_k = trf(L, TraceLayout::kKRope);
    if ((rc = snap(tr(L, TraceLayout::kQkv), m->qkv, 4 * size_t(Q + 2 * KV)))) return rc;
    rc = launch_attention(p, true, m->attn, s);
    if (rc) return rc;
    if ((rc = snap(tr(L, TraceLayout::kAttn), m->attn, 4 * size_t(Q)))) return rc;
    // output projection + residual (absent: the fallback slice of the attention output, scale 0.25)
    if (l.wo.present())
      rc = gemv(m, l.wo, m->attn, nullptr, 0.f, kOutResid, m->hidden, 0, s, nullptr, nullptr,
                tr(L, TraceLayout::kQ8Wo));
    else
      rc = launch_det_proj(m->attn, Q, nullptr, 0.f, 0.25f, m->hidden, c.hidden, true, s);
    if (rc) return rc;
    if ((rc = snap(tr(L, TraceLayout::kXMid), m->hidden, 4 * size_t(c.hidden)))) return rc;
    // FFN: RMSNorm -> gate|up -> SwiGLU -> down + residual
    if (m->moe) {  // dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:1286-1300)
      float* tr_logits = m->trace && 2 * c.ffn >= l.n_experts ? trf(L, TraceLayout::kGu) : nullptr;
      if ((rc = moe_ffn_step(m, l, eps_ffn, s, trf(L, TraceLayout::kXnFfn), tr_logits))) return rc;
      continue;
    }
    if (l.gu_split) {
      // gate and up apart (absent: fallback slices of the normalised input, scales 0.5 and 0.25,
      // run_dense_swiglu_ffn src/qwen_deepseek.rs:696-725), then SwiGLU
      const float* nw = static_cast<const float*>(l.ffn_norm.dev);
      const DevTensor* w2[2] = {&l.gate, &l.up};
      const float sc[2] = {0.5f, 0.25f};
      bool traced = false;
      for (int j = 0; j < 2; j++) {
        if (w2[j]->present()) {
          rc = gemv(m, *w2[j], m->hidden, nw, eps_ffn, kOutStore, m->gu + j * c.ffn, 0, s, nullptr,
                    traced ? nullptr : trf(L, TraceLayout::kXnFfn), traced ? nullptr : tr(L, TraceLayout::kQ8Ffn));
          traced = true;
        } else {
          rc = launch_det_proj(m->hidden, c.hidden, nw, eps_ffn, sc[j], m->gu + j * c.ffn, c.ffn, false, s);
        }
        if (rc) return rc;
      }
      if ((rc = launch_swiglu(m->gu, c.ffn, m->act, s))) return rc;
      if ((rc = snap(tr(L, TraceLayout::kGu), m->gu, 8 * size_t(c.ffn)))) return rc;
    } else {
      rc = gemv(m, l.gate_up, m->hidden, static_cast<const float*>(l.ffn_norm.dev), eps_ffn, kOutSwiglu, m->act,
                c.ffn, s, nullptr, trf(L, TraceLayout::kXnFfn), tr(L, TraceLayout::kQ8Ffn), trf(L, TraceLayout::kGu));
      if (rc) return rc;
    }
    if ((rc = snap(tr(L, TraceLayout::kAct), m->act, 4 * size_t(c.ffn)))) return rc;
    if (l.down.present())
      rc = gemv(m, l.down, m->act, nullptr, 0.f, kOutResid, m->hidden, 0, s, nullptr, nullptr,
                tr(L, TraceLayout::kQ8Down));
    else  // the fallback slice of the SwiGLU vector, scale 0.125
      rc = launch_det_proj(m->act, c.ffn, nullptr, 0.f, 0.125f, m->hidden, c.hidden, true, s);
    if (rc) return rc;
  }
  // final norm -> LM head -> greedy token
  uint8_t* tr_tail = m->trace;
  if (tr_tail && (rc = snap(tr_tail + tl.x_final, m->hidden, 4 * size_t(c.hidden)))) return rc;
  return head_step(m, m->hidden, s, tr_tail ? reinterpret_cast<float*>(tr_tail + tl.xn_head) : nullptr,
                   tr_tail ? tr_tail + tl.q8_head : nullptr);
}

namespace jero {

// The GEMM layout of a Q4_K / Q6_K tensor for the prefill (JERO_Q4_K_G, the Q4_K bytes in the
// MFMA fragment order; JERO_Q6_K_P, the exact int8 planes), null for other formats; built on
// the stream at first use.  Weights cannot change after finalize, so it stays valid.
static int laid_of(jero_model* m, const DevTensor& w, hipStream_t s, const void** out) {
  *out = nullptr;
  if (w.quant != JERO_Q4_K && w.quant != JERO_Q4_K_R && w.quant != JERO_Q6_K && w.quant != JERO_Q6_K_R) return JERO_OK;
  auto it = m->laid.find(w.dev);
  if (it != m->laid.end()) {
    *out = it->second;
    return JERO_OK;
  }
  void* p = nullptr;
  int rc = dev_alloc(m, gemm_layout_bytes(w.quant, w.n_in, w.n_out), &p);
  if (!rc) rc = launch_gemm_layout(w.quant, w.dev, w.n_in, w.n_out, p, s);
  if (rc) return rc;
  m->laid[w.dev] = p;
  *out = p;
  return JERO_OK;
}

// Attention queries per launch of the batched prefill: bounds its split workspace.
constexpr int64_t kPrefillAttnTokens = 256;

// Work on the model's second stream after everything enqueued on s so far.
static int fork_side(jero_model* m, hipStream_t s) {
  if (!m->side &&
      (hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking) != hipSuccess ||
       hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming) != hipSuccess ||
       hipEventCreateWithFlags(&m->ev_join, hipEventDisableTiming) != hipSuccess))
    return fail(JERO_ERR_DEVICE, "prefill: cannot create the second stream");
  if (hipEventRecord(m->ev_fork, s) != hipSuccess || hipStreamWaitEvent(m->side, m->ev_fork, 0) != hipSuccess)
    return fail(JERO_ERR_DEVICE, "prefill: stream fork failed");
  return JERO_OK;
}

// s waits for what was enqueued on the second stream.
static int join_side(jero_model* m, hipStream_t s) {
  if (hipEventRecord(m->ev_join, m->side) != hipSuccess || hipStreamWaitEvent(s, m->ev_join, 0) != hipSuccess)
    return fail(JERO_ERR_DEVICE, "prefill: stream join failed");
  return JERO_OK;
}

// Token rows per MoE launch of the batched prefill: the grouping step places at most
// kRouteLdsPairs (token, slot) pairs.
static int64_t moe_prefill_chunk(const jero_model* m) { return std::max<int64_t>(1, 8192 / std::max(1, m->moe_top_k)); }

// Whether a model with an MoE spec prefills in batches of token rows: every layer routed over an
// F32 router (the Qwen3-MoE GGUF form) and no shared expert to run; otherwise the token loop.
static bool moe_prefill_batched(const jero_model* m) {
  for (const LayerW& l : m->layers) {
    if (!l.routed || l.router.quant != JERO_F32 || m->cfg.hidden % 64 != 0) return false;
    if (m->moe_shared && l.gate_shexp.present() && l.up_shexp.present() && l.down_shexp.present()) return false;
  }
  return true;
}

static int prefill_buffers(jero_model* m, int64_t n, int64_t pos0) {
  const auto& c = m->cfg;
  const int64_t H = c.hidden, F = c.ffn, Q = q_dim(c), KV = kv_dim(c);
  // the split attention path's partials (f32 ring, head_dim 32, or a batch of one query): the
  // flash kernel needs none and leaves at most a trailing one-query batch to the split path
  const bool flash = attn_flash_ok(c.kv_dtype, int(c.head_dim), 2, c.n_heads_q / c.n_heads_kv);
  const int64_t tq = flash ? 1 : std::min(n, kPrefillAttnTokens);
  const size_t ws = size_t(tq) * attn_workspace_bytes(c.n_heads_q, c.head_dim, int(pos0 + n));
  PrefillBufs& b = m->pf;
  if (n <= b.rows && ws <= b.ws_bytes) return JERO_OK;
  const int64_t rows = std::max(n, b.rows);
  for (void* p : {static_cast<void*>(b.tok), static_cast<void*>(b.X), static_cast<void*>(b.XN),
                  static_cast<void*>(b.T), static_cast<void*>(b.T2), static_cast<void*>(b.QKV), static_cast<void*>(b.ATT),
                  static_cast<void*>(b.GU), static_cast<void*>(b.ACT), static_cast<void*>(b.RC),
                  static_cast<void*>(b.ws), static_cast<void*>(b.XQ), static_cast<void*>(b.LG),
                  static_cast<void*>(b.SW), static_cast<void*>(b.SI), b.MWS})
    if (p) dev_free(m, p);
  b = PrefillBufs{};
  auto act_row = [](int64_t k) { return std::max(k / 32 * 36, k / 256 * 292); };
  const size_t xq_row = size_t(std::max({act_row(H), act_row(Q), act_row(F)}));
  void* p = nullptr;
  int rc;
  auto f32 = [&](int64_t count, float** out) -> int {
    int r = dev_alloc(m, sizeof(float) * size_t(count), &p);
    if (!r) *out = static_cast<float*>(p);
    return r;
  };
  if ((rc = dev_alloc(m, sizeof(int32_t) * size_t(rows), &p))) return rc;
  b.tok = static_cast<int32_t*>(p);
  if ((rc = f32(rows * H, &b.X)) || (rc = f32(rows * H, &b.XN)) || (rc = f32(rows * H, &b.T)) ||
      (rc = f32(rows * H, &b.T2)) ||
      (rc = f32(rows * (Q + 2 * KV), &b.QKV)) || (rc = f32(rows * Q, &b.ATT)) || (rc = f32(rows * 2 * F, &b.GU)) ||
      (rc = f32(rows * F, &b.ACT)) || (rc = f32(rows * c.head_dim, &b.RC)))
    return rc;
  if ((rc = dev_alloc(m, ws, &p))) return rc;
  b.ws = static_cast<float*>(p);
  if ((rc = dev_alloc(m, xq_row * size_t(rows), &p))) return rc;
  b.XQ = static_cast<uint8_t*>(p);
  if (m->moe) {
    const int64_t ch = std::min(rows, moe_prefill_chunk(m)), k = std::max(1, m->moe_top_k);
    int64_t E = 1, Fe = 1;
    for (const LayerW& l : m->layers) E = std::max(E, l.n_experts), Fe = std::max(Fe, l.exp_ffn);
    if ((rc = f32(ch * E, &b.LG)) || (rc = f32(ch * k, &b.SW))) return rc;
    if ((rc = dev_alloc(m, sizeof(int32_t) * size_t(ch * k), &p))) return rc;
    b.SI = static_cast<int32_t*>(p);
    if ((rc = dev_alloc(m, moe_workspace_bytes(ch, E, int(k), H, Fe), &b.MWS))) return rc;
  }
  b.rows = rows;
  b.ws_bytes = ws;
  return JERO_OK;
}

}  // namespace jero

extern "C" int jero_hip_model_prefill(jero_model* m, const int32_t* tokens, int64_t n, int64_t pos0, void* stream) {
  if (!m || !tokens) return fail(JERO_ERR_INVALID_ARGUMENT, "prefill: null pointer");
  if (!m->finalized) return fail(JERO_ERR_INVALID_ARGUMENT, "prefill: model not finalized");
  const auto& c = m->cfg;
  if (n <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "prefill: no tokens");
  if (pos0 < 0 || pos0 + n > c.kv_capacity)
    return fail(JERO_ERR_CONTEXT_LENGTH_EXCEEDED, "prefill: positions " + std::to_string(pos0) + " .. " +
                                                      std::to_string(pos0 + n - 1) + " exceed the ring of " +
                                                      std::to_string(c.kv_capacity));
  for (int64_t t = 0; t < n; t++)
    if (tokens[t] < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "prefill: negative token " + std::to_string(tokens[t]));
  const TraceLayout tl = trace_layout(c);
  if (m->trace && m->trace_bytes < size_t(n) * tl.total)
    return fail(JERO_ERR_TENSOR_BOUNDS, "prefill: the trace buffer holds fewer than " + std::to_string(n) + " steps");
  if (m->moe && !moe_prefill_batched(m)) {
    // a model with an MoE spec that the batched pass does not take (a shared expert, a layer
    // without a router or with a non-F32 one): run_prefill_with_hidden's own token loop
    // (src/qwen_deepseek.rs:2298-2312), one decode step per prompt token (its trace at
    // t * jero_hip_model_trace_bytes)
    uint8_t* const trace0 = m->trace;
    int rc = JERO_OK;
    for (int64_t t = 0; t < n && !rc; t++) {
      m->trace = trace0 ? trace0 + size_t(t) * tl.total : nullptr;
      rc = launch_set_state(m->token, m->pos, m->status, tokens[t], pos0 + t, static_cast<hipStream_t>(stream));
      if (!rc) rc = jero_hip_decode_step(m, stream);
    }
    m->trace = trace0;
    return rc;
  }
  int rc = prefill_buffers(m, n, pos0);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  PrefillBufs& b = m->pf;
  const int64_t H = c.hidden, F = c.ffn, Q = q_dim(c), KV = kv_dim(c);
  const float eps_attn = c.rms_eps;
  const float eps_ffn = c.rms_eps > 1e-6f ? c.rms_eps : 1e-6f;
  const size_t es = c.kv_dtype == JERO_KV_F16 ? 2 : 4;
  const size_t ring = size_t(c.kv_capacity) * size_t(KV) * es;
  if ((rc = check_hip(hipMemcpyAsync(b.tok, tokens, sizeof(int32_t) * size_t(n), hipMemcpyHostToDevice, s),
                      "prefill tokens")))
    return rc;
  // token t's trace (the decode step's layout) at t * tl.total: one strided copy per field
  auto snap = [&](size_t off, const void* src, size_t pitch, size_t width) -> int {
    if (!m->trace) return JERO_OK;
    return check_hip(hipMemcpy2DAsync(m->trace + off, tl.total, src, pitch, width, size_t(n), hipMemcpyDeviceToDevice, s),
                     "prefill trace copy");
  };
  auto fld = [&](int64_t L, int f) { return size_t(L) * tl.layer_bytes + tl.field[f]; };
  // quantizes n rows of k floats into b.XQ in `fmt`; returns its row bytes
  auto quant_rows = [&](int fmt, const float* x, int64_t k, int64_t* xrb) -> int {
    *xrb = row_bytes(fmt, k);
    return launch_quantize_act(fmt, x, n, k, b.XQ, s);
  };
  if ((rc = launch_embed_rows(m->tok_embd.quant, m->tok_embd.dev, row_bytes(m->tok_embd.quant, H), m->embd_rows, int(H),
                              b.tok, n, b.X, s)))
    return rc;
  // the residual of the last projection, added to X by the next row step (null: none pending);
  // pending2: the second K half of a split projection (the residual is pending + pending2)
  const float* pending = nullptr;
  const float* pending2 = nullptr;
  auto q8k_input = [](const DevTensor& w) { return !w.present() || act_format(w.quant) == JERO_Q8_K; };
  for (int64_t L = 0; L < c.n_layers; L++) {
    const LayerW& l = m->layers[size_t(L)];
    const float* anw = static_cast<const float*>(l.attn_norm.dev);
    int64_t xrb = 0;
    int have_fmt = -1;
    // X += the pending residual, then RMSNorm rows: fused with the Q8_K quantization when every
    // projection of the sublayer reads Q8_K (XN then only for the trace), else apart (the
    // projections quantize XN themselves)
    auto norm_step = [&](const float* nw, float eps, bool all_q8k, int f_xin, int f_xn, int f_q8) -> int {
      int r = JERO_OK;
      if (all_q8k && H % 256 == 0 && H <= 8192) {
        if ((r = launch_add_rmsnorm_q8k_rows(b.X, pending, pending2, n, H, nw, eps, m->trace ? b.XN : nullptr, b.XQ,
                                             s)))
          return r;
        have_fmt = JERO_Q8_K;
        xrb = row_bytes(JERO_Q8_K, H);
        pending = pending2 = nullptr;
        if ((r = snap(fld(L, f_xin), b.X, 4 * H, 4 * H)) || (r = snap(fld(L, f_xn), b.XN, 4 * H, 4 * H)))
          return r;
        return snap(fld(L, f_q8), b.XQ, size_t(xrb), size_t(xrb));
      }
      if (pending2 && (r = launch_add_rows(b.T, pending2, n * H, s))) return r;  // pending is b.T
      if (pending && (r = launch_add_rows(b.X, pending, n * H, s))) return r;
      pending = pending2 = nullptr;
      have_fmt = -1;
      if ((r = snap(fld(L, f_xin), b.X, 4 * H, 4 * H)) || (r = launch_rmsnorm_rows(b.X, n, H, nw, eps, b.XN, s)))
        return r;
      return snap(fld(L, f_xn), b.XN, 4 * H, 4 * H);
    };
    // attention sublayer: RMSNorm rows -> Q, K, V rows
    const bool attn_q8k = l.qkv_split ? q8k_input(l.wq) && q8k_input(l.wk) && q8k_input(l.wv)
                                      : q8k_input(l.qkv) && (!l.v_separate || q8k_input(l.wv));
    if ((rc = norm_step(anw, eps_attn, attn_q8k, TraceLayout::kXIn, TraceLayout::kXnAttn, TraceLayout::kQ8Attn)))
      return rc;
    float *qp, *kp, *vp;
    int64_t qs, ks, vs;
    bool vsplit = false;  // V's split-K halves in vp and b.T2 (added by the QK-norm / RoPE step)
    // split: a projection into b.T whose split-K halves may land in b.T and b.T2 (then *split)
    auto project = [&](const DevTensor& w, const float* in, int64_t k, float* out, int trace_field,
                       bool* split = nullptr) -> int {
      const int fmt = act_format(w.quant);
      int r = JERO_OK;
      if (fmt != have_fmt) {
        if ((r = quant_rows(fmt, in, k, &xrb))) return r;
        have_fmt = fmt;
        if (trace_field >= 0 && (r = snap(fld(L, trace_field), b.XQ, size_t(xrb), size_t(xrb)))) return r;
      }
      const void* laid = nullptr;
      if (n >= kLaidMinRows && (r = laid_of(m, w, s, &laid))) return r;
      return launch_gemm(w.quant, w.dev, k, w.n_out, b.XQ, n, out, s, laid, split ? b.T2 : nullptr, split);
    };
    if (!l.qkv_split) {
      const int64_t w1 = l.qkv.n_out;  // Q + 2 KV, or Q + KV with V apart
      qp = b.QKV, qs = w1, kp = b.QKV + Q, ks = w1;
      // V apart (a Q6_K attn_v) runs on the second stream beside Q|K when both read the Q8_K rows
      // already built: its few workgroups fill the CUs the Q|K GEMM leaves idle
      const bool vside = l.v_separate && attn_q8k && have_fmt == JERO_Q8_K && n >= kLaidMinRows;
      if (vside) {
        vp = b.QKV + n * w1, vs = KV;
        const void* laid_v = nullptr;
        if ((rc = laid_of(m, l.wv, s, &laid_v)) || (rc = fork_side(m, s)) ||
            (rc = launch_gemm(l.wv.quant, l.wv.dev, H, l.wv.n_out, b.XQ, n, vp, m->side, laid_v, b.T2, &vsplit)))
          return rc;
      }
      if ((rc = project(l.qkv, b.XN, H, b.QKV, TraceLayout::kQ8Attn))) return rc;
      if (vside) {
        if ((rc = join_side(m, s))) return rc;
      } else if (l.v_separate) {
        vp = b.QKV + n * w1, vs = KV;
        if ((rc = project(l.wv, b.XN, H, vp, -1, &vsplit))) return rc;
      } else {
        vp = b.QKV + Q + KV, vs = w1;
      }
    } else {
      qp = b.QKV, qs = Q, kp = b.QKV + n * Q, ks = KV, vp = b.QKV + n * (Q + KV), vs = KV;
      const DevTensor* w3[3] = {&l.wq, &l.wk, &l.wv};
      float* o3[3] = {qp, kp, vp};
      const int64_t len[3] = {Q, KV, KV};
      const float sc[3] = {0.5f, 0.25f, 0.125f};
      bool first = true;  // the trace holds the first present projection's activation rows
      for (int j = 0; j < 3; j++) {
        if (w3[j]->present()) {
          rc = project(*w3[j], b.XN, H, o3[j], first ? TraceLayout::kQ8Attn : -1);
          first = false;
        } else {  // project_or_deterministic_slice's fallback of the normalised rows
          rc = launch_det_proj(b.X, H, anw, eps_attn, sc[j], o3[j], len[j], false, s, n, H, len[j]);
        }
        if (rc) return rc;
      }
    }
    if (vsplit && m->trace && (rc = launch_add_rows(vp, b.T2, n * KV, s))) return rc;  // the trace's V rows
    const float* v2 = vsplit && !m->trace ? b.T2 : nullptr;
    const size_t fq = fld(L, TraceLayout::kQkv);
    if ((rc = snap(fq, qp, 4 * qs, 4 * Q)) || (rc = snap(fq + 4 * Q, kp, 4 * ks, 4 * KV)) ||
        (rc = snap(fq + 4 * (Q + KV), vp, 4 * vs, 4 * KV)))
      return rc;
    // QK-norm, RoPE, the K/V rows into the ring, causal attention of every token
    uint8_t* base = static_cast<uint8_t*>(m->kv) + size_t(L) * 2 * ring;
    if ((rc = launch_qk_rope_rows(qp, qs, kp, ks, vp, vs, v2, n, c.n_heads_q, c.n_heads_kv, c.head_dim,
                                  c.qk_norm ? static_cast<const float*>(l.q_norm.dev) : nullptr,
                                  c.qk_norm ? static_cast<const float*>(l.k_norm.dev) : nullptr, eps_attn, pos0,
                                  c.rope_theta, b.RC, base, base + ring, c.kv_dtype == JERO_KV_F16, c.kv_capacity, s)))
      return rc;
    if ((rc = snap(fld(L, TraceLayout::kQRope), qp, 4 * qs, 4 * Q)) ||
        (rc = snap(fld(L, TraceLayout::kKRope), kp, 4 * ks, 4 * KV)))
      return rc;
    // on an f16 ring (head_dim 64 or 128) the flash kernel takes up to 65535 queries per launch
    // and writes the Q8_K rows of Wo's input itself when Wo reads Q8_K, the group's heads fill
    // whole 256-blocks and no batch holds a single token (the f32 rows then only for the trace)
    const int64_t rbq = row_bytes(JERO_Q8_K, Q);
    const bool flash =
        attn_flash_ok(c.kv_dtype, int(c.head_dim), int(std::min<int64_t>(n, 2)), c.n_heads_q / c.n_heads_kv);
    const int64_t batch = flash ? 65535 : kPrefillAttnTokens;
    const bool att_q8k = flash && l.wo.present() && act_format(l.wo.quant) == JERO_Q8_K && n % batch != 1 &&
                         attn_flash_q8k_ok(int(c.n_heads_q / c.n_heads_kv), int(c.head_dim));
    for (int64_t t0 = 0; t0 < n; t0 += batch) {
      const int64_t nt = std::min(batch, n - t0);
      AttnParams p{};
      p.q = qp + t0 * qs;
      p.k = base;
      p.v = base + ring;
      p.kv_dtype = c.kv_dtype;
      p.nkv = c.n_heads_kv;
      p.group = c.n_heads_q / c.n_heads_kv;
      p.hd = c.head_dim;
      p.active = int(pos0 + t0 + 1);
      p.scale = 1.0f / sqrtf(float(c.head_dim));
      p.part_o = b.ws;
      p.slot = -1;
      if ((rc = launch_attention_tokens(p, int(nt), qs, !att_q8k || m->trace ? b.ATT + t0 * Q : nullptr, Q, s,
                                        att_q8k ? b.XQ + t0 * rbq : nullptr)))
        return rc;
    }
    if ((rc = snap(fld(L, TraceLayout::kAttn), b.ATT, 4 * Q, 4 * Q))) return rc;
    // output projection; its residual is added by the FFN's row step
    have_fmt = -1;
    if (att_q8k) {
      have_fmt = JERO_Q8_K;
      xrb = rbq;
      if ((rc = snap(fld(L, TraceLayout::kQ8Wo), b.XQ, size_t(rbq), size_t(rbq)))) return rc;
    }
    if (l.wo.present()) {
      bool split = false;
      if ((rc = project(l.wo, b.ATT, Q, b.T, TraceLayout::kQ8Wo, &split))) return rc;
      pending = b.T;
      pending2 = split ? b.T2 : nullptr;
    } else if ((rc = launch_det_proj(b.ATT, Q, nullptr, 0.f, 0.25f, b.X, H, true, s, n, Q, H))) {
      return rc;
    }
    const float* fnw = static_cast<const float*>(l.ffn_norm.dev);
    if (m->moe) {
      // dispatch_qwen3_moe_ffn over the token rows (src/qwen_deepseek.rs:1286-1300, 882-938):
      // RMSNorm rows, the F32 router's logits rows, then the routed experts of every token (the
      // expert GEMMs over the tokens each expert was given), each token's sum in selection order
      // added to its hidden row
      if ((rc = norm_step(fnw, eps_ffn, false, TraceLayout::kXMid, TraceLayout::kXnFfn, TraceLayout::kQ8Ffn)))
        return rc;
      const int64_t E = l.n_experts, chunk = moe_prefill_chunk(m);
      for (int64_t t0 = 0; t0 < n; t0 += chunk) {
        const int64_t nt = std::min(chunk, n - t0);
        if ((rc = launch_matmul_f32_rows(l.router.dev, H, E, b.XN + t0 * H, nt, b.LG, s))) return rc;
        if (m->trace && 2 * F >= E &&
            (rc = check_hip(hipMemcpy2DAsync(m->trace + size_t(t0) * tl.total + fld(L, TraceLayout::kGu), tl.total,
                                             b.LG, sizeof(float) * size_t(E), sizeof(float) * size_t(E), size_t(nt),
                                             hipMemcpyDeviceToDevice, s),
                            "prefill trace copy")))
          return rc;
        MoeArgs a = moe_args_of(m, l);
        a.x = b.XN + t0 * H;
        a.logits = b.LG;
        a.T = nt;
        a.y = b.T;  // not written: the sums go to the hidden rows
        a.accumulate = false;
        a.resid = b.X + t0 * H;
        a.sel_idx = b.SI;
        a.sel_w = b.SW;
        if ((rc = launch_moe(a, b.MWS, s))) return rc;
      }
      continue;
    }
    // FFN: (residual +) RMSNorm rows -> gate | up -> SwiGLU -> down + residual
    const bool ffn_q8k = l.gu_split ? q8k_input(l.gate) && q8k_input(l.up) : q8k_input(l.gate_up);
    if ((rc = norm_step(fnw, eps_ffn, ffn_q8k, TraceLayout::kXMid, TraceLayout::kXnFfn, TraceLayout::kQ8Ffn)))
      return rc;
    // SwiGLU fused with the Q8_K quantization when down reads Q8_K (act then only for the trace)
    const bool act_q8k = l.down.present() && act_format(l.down.quant) == JERO_Q8_K && F % 256 == 0;
    auto swiglu = [&](const float* g, int64_t gst, const float* u, int64_t ust) -> int {
      if (!act_q8k) return launch_swiglu_rows(g, gst, u, ust, b.ACT, n, F, s);
      return launch_swiglu_q8k_rows(g, gst, u, ust, m->trace ? b.ACT : nullptr, n, F, b.XQ, s);
    };
    const size_t fg = fld(L, TraceLayout::kGu);
    if (!l.gu_split) {
      if ((rc = project(l.gate_up, b.XN, H, b.GU, TraceLayout::kQ8Ffn)) ||
          (rc = swiglu(b.GU, 2 * F, b.GU + F, 2 * F)) || (rc = snap(fg, b.GU, 8 * F, 8 * F)))
        return rc;
    } else {
      float* g2[2] = {b.GU, b.GU + n * F};
      const DevTensor* w2[2] = {&l.gate, &l.up};
      const float sc[2] = {0.5f, 0.25f};
      bool first = true;
      for (int j = 0; j < 2; j++) {
        if (w2[j]->present()) {
          rc = project(*w2[j], b.XN, H, g2[j], first ? TraceLayout::kQ8Ffn : -1);
          first = false;
        } else {
          rc = launch_det_proj(b.X, H, fnw, eps_ffn, sc[j], g2[j], F, false, s, n, H, F);
        }
        if (rc) return rc;
      }
      if ((rc = swiglu(g2[0], F, g2[1], F)) || (rc = snap(fg, g2[0], 4 * F, 4 * F)) ||
          (rc = snap(fg + 4 * F, g2[1], 4 * F, 4 * F)))
        return rc;
    }
    if ((rc = snap(fld(L, TraceLayout::kAct), b.ACT, 4 * F, 4 * F))) return rc;
    have_fmt = -1;
    if (act_q8k) {  // the SwiGLU step left the Q8_K rows in XQ
      have_fmt = JERO_Q8_K;
      xrb = row_bytes(JERO_Q8_K, F);
      if ((rc = snap(fld(L, TraceLayout::kQ8Down), b.XQ, size_t(xrb), size_t(xrb)))) return rc;
    }
    if (l.down.present()) {
      bool split = false;
      if ((rc = project(l.down, b.ACT, F, b.T, TraceLayout::kQ8Down, &split))) return rc;
      pending = b.T;  // added by the next layer's row step
      pending2 = split ? b.T2 : nullptr;
    } else if ((rc = launch_det_proj(b.ACT, F, nullptr, 0.f, 0.125f, b.X, H, true, s, n, F, H))) {
      return rc;
    }
  }
  if (pending2 && (rc = launch_add_rows(b.T, pending2, n * H, s))) return rc;
  if (pending && (rc = launch_add_rows(b.X, pending, n * H, s))) return rc;
  // every token's final hidden state and RoPE table; the head on the last token only
  if ((rc = snap(tl.x_final, b.X, 4 * H, 4 * H)) || (rc = snap(tl.rope_cs, b.RC, 4 * size_t(c.head_dim), 4 * size_t(c.head_dim))))
    return rc;
  if ((rc = launch_set_state(m->token, m->pos, m->status, tokens[n - 1], pos0 + n - 1, s))) return rc;
  uint8_t* tr_last = m->trace ? m->trace + size_t(n - 1) * tl.total : nullptr;
  return head_step(m, b.X + (n - 1) * H, s, tr_last ? reinterpret_cast<float*>(tr_last + tl.xn_head) : nullptr,
                   tr_last ? tr_last + tl.q8_head : nullptr);
}
