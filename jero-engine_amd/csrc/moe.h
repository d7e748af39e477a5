// moe.h -- routed expert FFN launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jero {

// Expert grouping produced by the routing kernel (device arrays).
struct MoeLists {
  int32_t* offset;    // [E+1] first list position of each expert
  int32_t* active;    // [E] ascending ids of experts with at least one (token, slot)
  int32_t* n_active;  // [1]
  int32_t* entry;     // [T*k] (token*k + slot), grouped by expert, ascending within an expert
  int32_t* inv;       // [T*k] list position of (token*k + slot)
  int32_t* pass;      // [passes][4 + pass_tokens] per pass (up to pass_tokens of one expert's
                      // list entries, experts ascending): expert, first list position, count, 0,
                      // then the pass's tokens (or null: no pass descriptors)
  int pass_tokens;    // kMoePassTokens or kMoePassTokensWide
  int32_t* ctr;       // [kMoeCtrInts]: the number of passes, then the work counters of the
                      // expert GEMMs, each on its own 128-byte line (with pass)
};

constexpr int kMoePassTokens = 8;       // tokens per expert-GEMM pass
constexpr int kMoePassTokensWide = 16;  // when the experts average at least that many tokens
constexpr int kMoePassInts = 4 + kMoePassTokens;
constexpr int kMoeCtrInts = 96;
constexpr int kMoeCtrGateUp = 32, kMoeCtrDown = 64;  // counter offsets in ctr

// The single-token path's extra inputs (the gate/up kernel routes and quantizes the token itself).
struct MoeSingle {
  const float* logits;  // [E]
  const float* x;       // [H]
  int E, H;
  int32_t* sel_idx;     // [k]
  float* sel_w;         // [k]
};

struct MoeArgs {
  const float* x;       // [T][hidden]
  const float* logits;  // [T][E]
  int64_t T, E;
  int top_k;
  int gate_quant, up_quant, down_quant;
  const void* gate;  // stacked [E][ffn rows][hidden]
  const void* up;
  const void* down;  // stacked [E][hidden rows][ffn]
  int64_t hidden, ffn;
  float* y;          // [T][hidden]
  bool accumulate;   // y += the routed sum (y holds the values to add onto) instead of y =, in the
                     // reference's order: ((y + w0 e0) + w1 e1) + ...
  float* resid;      // null, or [T][hidden] the layer output is added to: resid += that sum (the
                     // decode step's residual, src/qwen_deepseek.rs:1301-1303), y not written
  int32_t* sel_idx;  // [T][k]
  float* sel_w;      // [T][k]
  // workspace carve-out (set by launch_moe)
  uint8_t* xq;
  float* act;
  float* yd;
  int max_active;
};

size_t moe_workspace_bytes(int64_t T, int64_t E, int top_k, int64_t hidden, int64_t ffn);
int check_moe_args(const MoeArgs& a, size_t gate_bytes, size_t up_bytes, size_t down_bytes);
int launch_moe(MoeArgs a, void* ws, hipStream_t s);

}  // namespace jero
