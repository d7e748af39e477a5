// moe.hip -- routed expert FFN (Qwen3-MoE) on gfx950.
//
// Replaces dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) for router logits already
// computed, with select_top_k_experts (src/gemma.rs:362-442), slice_or_lookup_expert on the
// stacked [hidden, ffn, n_experts] tensors (:729-746) and run_single_swiglu_expert (:748-771).
// The reference loops token by token and expert by expert; here the work is regrouped by
// expert so that each selected expert's weights stream from HBM once for all of its tokens:
//   1. route   (one workgroup): per token f32 softmax over all experts, top-k by (logit desc,
//              index asc) with non-finite logits ranked last, renormalised weights; then the
//              (token, slot) pairs are grouped by expert in ascending (token, slot) order, and
//              the ascending list of active experts is written.
//   2. quantize the T hidden vectors to Q8_K.
//   3. gate/up: one lane group per weight row; gate row f and up row f of an active expert
//              sit side by side in one wave, loaded once, and are dotted with every token routed
//              to that expert; act = silu(g) * u.
//   4. quantize act rows to Q8_K.
//   5. down:   one lane group per row of the expert's down matrix, dotted with each of its
//              tokens' act rows -> per-(token, slot) outputs.
//   6. combine y[t] = sum_j w[t][j] * out[t][j], j ascending as the reference accumulates.
// All integer partial sums are exact; every output element is reduced in a fixed order.
#include "moe.h"

#include "gemv_dot.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {

constexpr int kRouteThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 16;

__device__ __forceinline__ bool better(float a, int ia, float b, int ib) { return a > b || (a == b && ia < ib); }

__global__ void __launch_bounds__(kRouteThreads) moe_route_kernel(const float* __restrict__ logits, int T, int E,
                                                                  int k, int32_t* __restrict__ sel_idx,
                                                                  float* __restrict__ sel_w, MoeLists lists) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = kRouteThreads / 64;
  constexpr int PER = kMaxExperts / 64;
  __shared__ int s_count[kMaxExperts];
  // 1. routing, one wave per token
  for (int t = wv; t < T; t += nw) {
    const float* lt = logits + int64_t(t) * E;
    float key[PER], prob[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = lane + 64 * i;
      float l = e < E ? lt[e] : -INFINITY;
      bool fin = e < E && isfinite(l);
      key[i] = fin ? l : -INFINITY;
      if (fin) mx = fmaxf(mx, l);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = lane + 64 * i;
      bool fin = e < E && key[i] != -INFINITY;
      prob[i] = (fin && isfinite(mx)) ? expf(key[i] - mx) : 0.f;
      sum += prob[i];
    }
    sum = wave_sum(sum);
    const bool ok = sum > 0.f && isfinite(sum);
#pragma unroll
    for (int i = 0; i < PER; i++) prob[i] = ok ? prob[i] / sum : 1.0f / float(E);
    // top-k rounds; taken entries drop below every remaining key
    float ssum = 0.f;
    float wsel[kMaxTopK];
    int isel[kMaxTopK];
    bool taken[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) taken[i] = !(lane + 64 * i < E);
    for (int j = 0; j < k; j++) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      float bp = 0.f;
#pragma unroll
      for (int i = 0; i < PER; i++) {
        const int e = lane + 64 * i;
        if (!taken[i] && better(key[i], e, bv, bi)) {
          bv = key[i];
          bi = e;
          bp = prob[i];
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        float ov = __shfl_xor(bv, off, kWave);
        int oi = __shfl_xor(bi, off, kWave);
        float op = __shfl_xor(bp, off, kWave);
        if (better(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
          bp = op;
        }
      }
#pragma unroll
      for (int i = 0; i < PER; i++)
        if (lane + 64 * i == bi) taken[i] = true;
      isel[j] = bi;
      wsel[j] = bp;
      ssum += bp;
    }
    const bool sok = ssum > 0.f && isfinite(ssum);
    if (lane == 0) {
      for (int j = 0; j < k; j++) {
        sel_idx[t * k + j] = isel[j];
        sel_w[t * k + j] = sok ? wsel[j] / ssum : 1.0f / float(k);
      }
    }
  }
  // 2. group the (token, slot) pairs by expert
  for (int e = threadIdx.x; e < E; e += kRouteThreads) s_count[e] = 0;
  __threadfence_block();
  __syncthreads();
  const int n = T * k;
  for (int i = threadIdx.x; i < n; i += kRouteThreads) atomicAdd(&s_count[sel_idx[i]], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int off = 0, na = 0;
    for (int e = 0; e < E; e++) {
      lists.offset[e] = off;
      if (s_count[e] > 0) lists.active[na++] = e;
      off += s_count[e];
    }
    lists.offset[E] = off;
    *lists.n_active = na;
  }
  __syncthreads();
  // stable placement: thread e walks the pairs in order and keeps those routed to e
  for (int e = threadIdx.x; e < E; e += kRouteThreads) {
    if (s_count[e] == 0) continue;
    int pos = lists.offset[e];
    for (int i = 0; i < n; i++) {
      if (sel_idx[i] == e) {
        lists.entry[pos] = i;
        lists.inv[i] = pos;
        pos++;
      }
    }
  }
}

// gate/up + SwiGLU.  LPR <= 32: lane groups (2p, 2p+1) hold gate row and up row f0 + p.
template <int F, int LPR, int UPL>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(const uint8_t* __restrict__ gate,
                                                          const uint8_t* __restrict__ up, int64_t rb, int U, int Fdim,
                                                          int k, const uint8_t* __restrict__ xq, int64_t xq_rb,
                                                          MoeLists lists, float* __restrict__ act) {
  using Ut = Unit<F>;
  constexpr int G = kWave / LPR;
  constexpr int P = G / 2;  // (gate, up) row pairs per wave
  static_assert(P >= 1, "gate/up pairing needs two lane groups per wave");
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int waves_per_expert = (Fdim + P - 1) / P;
  const int slot = int(wave / waves_per_expert);
  if (slot >= *lists.n_active) return;
  const int e = lists.active[slot];
  const int g = lane / LPR, c = lane % LPR;
  const int f = int(wave % waves_per_expert) * P + g / 2;
  const bool is_up = g & 1;
  const bool row_ok = f < Fdim;
  const uint8_t* row = (is_up ? up : gate) + (int64_t(e) * Fdim + (row_ok ? f : 0)) * rb;
  typename Ut::W wt[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) {
    const int u = c + LPR * t;
    if (row_ok && u < U) Ut::load_w(wt[t], row, u);
  }
  const int i0 = lists.offset[e], i1 = lists.offset[e + 1];
  for (int i = i0; i < i1; i++) {
    const int tok = lists.entry[i] / k;
    const uint8_t* xt = xq + int64_t(tok) * xq_rb;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      if (row_ok && u < U) {
        typename Ut::Act a;
        Ut::load_act(a, xt, u);
        acc += Ut::dot(wt[t], a, nullptr);
      }
    }
    acc = group_sum_last<LPR>(acc);
    const float gv = __shfl(acc, lane - LPR, kWave);  // gate total, from the group below
    if (is_up && c == LPR - 1 && row_ok) {
      const float silu = gv / (1.0f + expf(-gv));
      act[int64_t(i) * Fdim + f] = silu * acc;
    }
  }
}

// down: one lane group per row h of the expert's down matrix, over the expert's entries.
template <int F, int LPR, int UPL>
__global__ void __launch_bounds__(256) moe_down_kernel(const uint8_t* __restrict__ down, int64_t rb, int U, int H,
                                                       const uint8_t* __restrict__ aq, int64_t aq_rb, MoeLists lists,
                                                       float* __restrict__ yd) {
  using Ut = Unit<F>;
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int waves_per_expert = (H + G - 1) / G;
  const int slot = int(wave / waves_per_expert);
  if (slot >= *lists.n_active) return;
  const int e = lists.active[slot];
  const int g = lane / LPR, c = lane % LPR;
  const int h = int(wave % waves_per_expert) * G + g;
  const bool row_ok = h < H;
  const uint8_t* row = down + (int64_t(e) * H + (row_ok ? h : 0)) * rb;
  typename Ut::W wt[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) {
    const int u = c + LPR * t;
    if (row_ok && u < U) Ut::load_w(wt[t], row, u);
  }
  const int i0 = lists.offset[e], i1 = lists.offset[e + 1];
  for (int i = i0; i < i1; i++) {
    const uint8_t* at = aq + int64_t(i) * aq_rb;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      if (row_ok && u < U) {
        typename Ut::Act a;
        Ut::load_act(a, at, u);
        acc += Ut::dot(wt[t], a, nullptr);
      }
    }
    acc = group_sum_last<LPR>(acc);
    if (c == LPR - 1 && row_ok) yd[int64_t(i) * H + h] = acc;
  }
}

__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ yd, const float* __restrict__ w,
                                                          const int32_t* __restrict__ inv, int T, int k, int H,
                                                          float* __restrict__ y) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= int64_t(T) * H) return;
  const int t = int(idx / H), h = int(idx % H);
  float acc = 0.f;
  for (int j = 0; j < k; j++) acc += w[t * k + j] * yd[int64_t(inv[t * k + j]) * H + h];
  y[idx] = acc;
}

// ---------------------------------------------------------------- launch plumbing

namespace {

int lpr_for(int U) { return U > 32 ? 64 : U > 16 ? 32 : U > 4 ? 16 : 4; }

template <int F, int LPR, int UPL>
void gate_up_one(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  constexpr int P = (kWave / LPR) / 2;
  const int U = units_per_row(F, a.hidden);
  int64_t waves = int64_t(a.max_active) * ((a.ffn + P - 1) / P);
  hipLaunchKernelGGL((moe_gate_up_kernel<F, LPR, UPL>), dim3(unsigned((waves + 3) / 4)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(a.gate), static_cast<const uint8_t*>(a.up),
                     row_bytes(F, a.hidden), U, int(a.ffn), a.top_k, a.xq, row_bytes(JERO_Q8_K, a.hidden), L, a.act);
}

template <int F>
int gate_up_fmt(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  const int U = units_per_row(F, a.hidden);
  switch (lpr_for(U)) {
    case 4: gate_up_one<F, 4, 1>(a, L, s); return JERO_OK;
    case 16: gate_up_one<F, 16, 1>(a, L, s); return JERO_OK;
    case 32: gate_up_one<F, 32, 1>(a, L, s); return JERO_OK;
    default:
      return fail(JERO_ERR_CAPABILITY_MISMATCH,
                  "moe: hidden " + std::to_string(a.hidden) + " above the gate/up pairing limit (2048 for K-quants)");
  }
}

template <int F, int LPR, int UPL>
void down_one(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  constexpr int G = kWave / LPR;
  const int U = units_per_row(F, a.ffn);
  int64_t waves = int64_t(a.max_active) * ((a.hidden + G - 1) / G);
  hipLaunchKernelGGL((moe_down_kernel<F, LPR, UPL>), dim3(unsigned((waves + 3) / 4)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(a.down), row_bytes(F, a.ffn), U, int(a.hidden), a.aq,
                     row_bytes(JERO_Q8_K, a.ffn), L, a.yd);
}

template <int F>
int down_fmt(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  const int U = units_per_row(F, a.ffn);
  const int lpr = lpr_for(U);
  const int upl = (U + lpr - 1) / lpr;
  if (lpr == 4) down_one<F, 4, 1>(a, L, s);
  else if (lpr == 16) down_one<F, 16, 1>(a, L, s);
  else if (lpr == 32) down_one<F, 32, 1>(a, L, s);
  else if (upl == 1) down_one<F, 64, 1>(a, L, s);
  else if (upl == 2) down_one<F, 64, 2>(a, L, s);
  else if (upl <= 4) down_one<F, 64, 4>(a, L, s);
  else
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: ffn " + std::to_string(a.ffn) + " above the down-proj limit");
  return JERO_OK;
}

}  // namespace

size_t moe_workspace_bytes(int64_t T, int64_t E, int top_k, int64_t hidden, int64_t ffn) {
  const int64_t n = T * top_k;
  size_t b = 0;
  auto add = [&](size_t x) { b += (x + 255) & ~size_t(255); };
  add(size_t(T) * size_t(row_bytes(JERO_Q8_K, hidden)));  // xq
  add(sizeof(int32_t) * size_t(E + 1));                    // offset
  add(sizeof(int32_t) * size_t(E));                        // active
  add(sizeof(int32_t));                                    // n_active
  add(sizeof(int32_t) * size_t(n) * 2);                    // entry, inv
  add(sizeof(float) * size_t(n) * size_t(ffn));            // act
  add(size_t(n) * size_t(row_bytes(JERO_Q8_K, ffn)));      // act_q
  add(sizeof(float) * size_t(n) * size_t(hidden));         // per-slot down outputs
  return b;
}

int launch_moe(MoeArgs a, void* ws, hipStream_t s) {
  const int64_t n = a.T * a.top_k;
  uint8_t* p = static_cast<uint8_t*>(ws);
  auto take = [&](size_t x) {
    uint8_t* r = p;
    p += (x + 255) & ~size_t(255);
    return r;
  };
  a.xq = take(size_t(a.T) * size_t(row_bytes(JERO_Q8_K, a.hidden)));
  MoeLists L;
  L.offset = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(a.E + 1)));
  L.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(a.E)));
  L.n_active = reinterpret_cast<int32_t*>(take(sizeof(int32_t)));
  int32_t* ei = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(n) * 2));
  L.entry = ei;
  L.inv = ei + n;
  a.act = reinterpret_cast<float*>(take(sizeof(float) * size_t(n) * size_t(a.ffn)));
  a.aq = take(size_t(n) * size_t(row_bytes(JERO_Q8_K, a.ffn)));
  a.yd = reinterpret_cast<float*>(take(sizeof(float) * size_t(n) * size_t(a.hidden)));
  a.max_active = int(n < a.E ? n : a.E);

  int rc = launch_quantize_act(JERO_Q8_K, a.x, a.T, a.hidden, a.xq, s);
  if (rc) return rc;
  hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(kRouteThreads), 0, s, a.logits, int(a.T), int(a.E), a.top_k,
                     a.sel_idx, a.sel_w, L);
  rc = check_launch("moe route");
  if (rc) return rc;
  rc = a.gate_quant == JERO_Q4_K ? gate_up_fmt<JERO_Q4_K>(a, L, s) : gate_up_fmt<JERO_Q6_K>(a, L, s);
  if (rc) return rc;
  rc = check_launch("moe gate/up");
  if (rc) return rc;
  rc = launch_quantize_act(JERO_Q8_K, a.act, n, a.ffn, const_cast<uint8_t*>(a.aq), s);
  if (rc) return rc;
  rc = a.down_quant == JERO_Q4_K ? down_fmt<JERO_Q4_K>(a, L, s) : down_fmt<JERO_Q6_K>(a, L, s);
  if (rc) return rc;
  rc = check_launch("moe down");
  if (rc) return rc;
  const int64_t total = a.T * a.hidden;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, a.yd, a.sel_w, L.inv,
                     int(a.T), a.top_k, int(a.hidden), a.y);
  return check_launch("moe combine");
}

int check_moe_args(const MoeArgs& a, size_t gate_bytes, size_t up_bytes, size_t down_bytes) {
  if (a.E <= 0 || a.top_k <= 0) return fail(JERO_ERR_ROUTING_UNAVAILABLE, "moe: no experts to route to");
  if (!a.x || !a.logits || !a.gate || !a.up || !a.down || !a.y || !a.sel_idx || !a.sel_w)
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe: null pointer");
  if (a.T <= 0 || a.hidden <= 0 || a.ffn <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "moe: empty input");
  if (a.top_k > a.E || a.top_k > kMaxTopK || a.E > kMaxExperts)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: top_k must be <= min(n_experts, 16), n_experts <= 1024");
  if (a.gate_quant != a.up_quant || (a.gate_quant != JERO_Q4_K && a.gate_quant != JERO_Q6_K) ||
      (a.down_quant != JERO_Q4_K && a.down_quant != JERO_Q6_K))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: gate/up must share a K-quant format; down Q4_K or Q6_K");
  int64_t rg = row_bytes(a.gate_quant, a.hidden), rd = row_bytes(a.down_quant, a.ffn);
  if (rg < 0 || rd < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "moe: hidden/ffn not multiples of 256");
  if (uint64_t(rg) * a.ffn * a.E > gate_bytes || uint64_t(rg) * a.ffn * a.E > up_bytes ||
      uint64_t(rd) * a.hidden * a.E > down_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "moe: stacked expert tensors smaller than [E][rows][cols]");
  if (!aligned4(a.gate) || !aligned4(a.up) || !aligned4(a.down) || (reinterpret_cast<uintptr_t>(a.x) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe: weights 4-byte and x 16-byte aligned");
  return JERO_OK;
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_moe_ffn(const float* x_dev, const float* router_logits_dev, int64_t n_tokens,
                                int64_t n_experts, int top_k, int gate_quant, const void* gate_dev, size_t gate_bytes,
                                int up_quant, const void* up_dev, size_t up_bytes, int down_quant,
                                const void* down_dev, size_t down_bytes, int64_t hidden, int64_t ffn, float* y_dev,
                                int32_t* sel_idx_dev, float* sel_w_dev, void* workspace_dev, size_t workspace_bytes,
                                void* stream) {
  MoeArgs a{};
  a.x = x_dev;
  a.logits = router_logits_dev;
  a.T = n_tokens;
  a.E = n_experts;
  a.top_k = top_k;
  a.gate_quant = gate_quant;
  a.up_quant = up_quant;
  a.down_quant = down_quant;
  a.gate = gate_dev;
  a.up = up_dev;
  a.down = down_dev;
  a.hidden = hidden;
  a.ffn = ffn;
  a.y = y_dev;
  a.sel_idx = sel_idx_dev;
  a.sel_w = sel_w_dev;
  int rc = check_moe_args(a, gate_bytes, up_bytes, down_bytes);
  if (rc) return rc;
  const size_t need = moe_workspace_bytes(n_tokens, n_experts, top_k, hidden, ffn);
  void* ws = workspace_dev;
  if (ws) {
    if (workspace_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "moe: workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
                                              std::to_string(need));
    if (reinterpret_cast<uintptr_t>(ws) & 255u)
      return fail(JERO_ERR_INVALID_ARGUMENT, "moe: workspace must be 256-byte aligned");
  } else {
    rc = workspace(need, &ws);
    if (rc) return rc;
  }
  return launch_moe(a, ws, static_cast<hipStream_t>(stream));
}

extern "C" size_t jero_hip_moe_workspace_bytes(int64_t n_tokens, int64_t n_experts, int top_k, int64_t hidden,
                                               int64_t ffn) {
  return moe_workspace_bytes(n_tokens, n_experts, top_k, hidden, ffn);
}
