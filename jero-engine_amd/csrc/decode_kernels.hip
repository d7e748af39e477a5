// decode_kernels.hip -- fused kernels of the batch-1 decode step (gfx950).
//
// The decode step of execute_token_standard_with_hidden (src/qwen_deepseek.rs:1239-1314) is
// a chain of GEMVs separated by small vector ops.  Here each GEMV absorbs its neighbours:
//   prologue: the workgroup turns the f32 input into the activation blocks the weight format
//             needs (ACT_Q8 or Q8_K) directly in LDS, optionally after RMSNorm
//             (rmsnorm_standard, :521-528) -- the weight loads of the first rows are already
//             in flight while it does so;
//   epilogue: plain store, residual add into the hidden state (:1086-1095, :1304-1306),
//             SwiGLU of paired gate/up rows (run_dense_swiglu_ffn, :696-727), or, for the
//             LM head, a per-workgroup (max, first index) for sample_greedy_argmax
//             (src/engine.rs:1873-1895).
// Token id and position are read from device memory, so one captured graph of the step can be
// replayed for consecutive tokens; the last kernel writes the greedy token and advances the
// position.
#include "decode.h"

#include <algorithm>

#include "dequant.h"
#include "gemv_dot.h"
#include "jero_common.h"
#include "runtime.h"

namespace jero {

// ---------------------------------------------------------------- prologue: f32 -> blocks in LDS

__device__ __forceinline__ float block_sum(float v, float* s_tmp) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) s_tmp[wv] = v;
  lds_barrier();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += s_tmp[i];
  return t;
}

// The workgroup's share of the f32 input, loaded before the weight rows so that the prologue
// only waits for these loads.  Q8_K: wave w takes blocks w, w+nw, ... (4 elements per lane,
// the quantizer's layout); ACT_Q8: half-wave h takes 32-element blocks h, h+2nw, ...
// Every load here and in the weight loads that follow is unconditional (block index clamped,
// a null norm pointer replaced by x): with a load under a branch the compiler cannot count
// the loads issued after the input, and the prologue would wait for the weights as well.
template <int ACT, int XB, bool NORM>
struct XRegs {
  float4 v[XB];
  float4 g[NORM ? XB : 1];  // RMSNorm weights (kernels that normalise their input)
};

template <int ACT, int XB, bool NORM>
__device__ __forceinline__ void load_x(XRegs<ACT, XB, NORM>& X, const float* __restrict__ x, const float* __restrict__ nw,
                                       int K) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  const float* g = nw ? nw : x;
#pragma unroll
  for (int i = 0; i < XB; i++) {
    if constexpr (ACT == JERO_Q8_K) {
      const int b = min(wv + nwv * i, K / 256 - 1);
      X.v[i] = reinterpret_cast<const float4*>(x + b * 256)[lane];
      if constexpr (NORM) X.g[i] = reinterpret_cast<const float4*>(g + b * 256)[lane];
    } else {
      const int b = min(2 * wv + (lane >> 5) + 2 * nwv * i, K / 32 - 1);
      X.v[i].x = x[b * 32 + (lane & 31)];
      if constexpr (NORM) X.g[i].x = g[b * 32 + (lane & 31)];
    }
  }
}

// Marks the input registers as used here.  Placed after the first weight loads: the compiler
// then cannot sink an input load into the prologue's per-block branch (where it would wait for
// every load in flight), and the wait for the input lands after the weight loads are issued.
__device__ __forceinline__ void pin4(float4& v) {
  float a = v.x, b = v.y, c = v.z, d = v.w;
  asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
  v = make_float4(a, b, c, d);
}
template <int ACT, int XB, bool NORM>
__device__ __forceinline__ void pin_x(XRegs<ACT, XB, NORM>& X) {
#pragma unroll
  for (int i = 0; i < XB; i++) {
    pin4(X.v[i]);
    if constexpr (NORM) pin4(X.g[i]);
  }
}

// Builds the activation blocks of x (or of rmsnorm(x) * nw) in LDS from the registers and
// returns the RMSNorm scale (1 without a norm).  It writes no global memory: a conditional store
// here would leave the compiler unable to count the weight loads still in flight, so it would
// make the first rows wait for loads issued after them (the trace is written afterwards,
// trace_xn).
template <int ACT, int XB, bool NORM>
__device__ float build_act_lds(XRegs<ACT, XB, NORM>& X, bool has_norm, float eps, int K, uint8_t* s_act,
                               float* s_tmp) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  float scale = 1.0f;
  if (has_norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < XB; i++) {
      if constexpr (ACT == JERO_Q8_K) {
        if (wv + nwv * i < K / 256)
          ss += X.v[i].x * X.v[i].x + X.v[i].y * X.v[i].y + X.v[i].z * X.v[i].z + X.v[i].w * X.v[i].w;
      } else {
        if (2 * wv + (lane >> 5) + 2 * nwv * i < K / 32) ss += X.v[i].x * X.v[i].x;
      }
    }
    ss = block_sum(ss, s_tmp);
    scale = 1.0f / sqrtf(ss / float(K) + eps);
  }
#pragma unroll
  for (int i = 0; i < XB; i++) {
    if constexpr (ACT == JERO_Q8_K) {
      const int b = wv + nwv * i;
      if (b < K / 256) {
        float e[4] = {X.v[i].x, X.v[i].y, X.v[i].z, X.v[i].w};
        if constexpr (NORM) {
          if (has_norm) {
            e[0] = e[0] * scale * X.g[i].x;
            e[1] = e[1] * scale * X.g[i].y;
            e[2] = e[2] * scale * X.g[i].z;
            e[3] = e[3] * scale * X.g[i].w;
          }
        }
        q8k_block_wave(e, lane, s_act + b * 292);
      }
    } else {
      const int b = 2 * wv + (lane >> 5) + 2 * nwv * i;
      if (b < K / 32) {
        const int l = lane & 31;
        float v = X.v[i].x;
        if constexpr (NORM) {
          if (has_norm) v = v * scale * X.g[i].x;
        }
        float a = fabsf(v);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, kWave));
        float d = a / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t* ob = s_act + b * 36;
        ob[4 + l] = uint8_t(int8_t(int(__builtin_rintf(v * id))));
        if (l == 0) *reinterpret_cast<float*>(ob) = d;
      }
    }
  }
  lds_barrier();
  return scale;
}

// Debug trace: the f32 values the prologue quantized, x[i] * scale * nw[i] (the same operations
// in the same order as build_act_lds, so the same bits), or x itself without a norm.
__device__ __forceinline__ void trace_xn(float* dst, const float* __restrict__ x, const float* __restrict__ nw,
                                         bool has_norm, float scale, int K) {
  for (int i = threadIdx.x; i < K; i += blockDim.x) dst[i] = has_norm ? x[i] * scale * nw[i] : x[i];
}

// Debug trace: the workgroup copies the activation blocks it built in LDS to global memory.
__device__ __forceinline__ void trace_act(uint8_t* dst, const uint8_t* s_act, int bytes) {
  for (int i = threadIdx.x; i < bytes / 4; i += blockDim.x)
    reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(s_act)[i];
}

// ---------------------------------------------------------------- fused GEMV

template <int F, int LPR, int UPL, int R, int OUT, int XB>
__global__ void __launch_bounds__(kDecodeThreads) dgemv_kernel(DGemvArgs a) {
  using Ut = Unit<F>;
  constexpr int ACT = (F == JERO_Q8_0 || F == JERO_Q4_0) ? JERO_ACT_Q8 : JERO_Q8_K;
  constexpr int G = kWave / LPR;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_mem[];
  float* s_tmp = reinterpret_cast<float*>(s_mem);  // 64 floats of scratch
  uint8_t* s_act = s_mem + 256;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t wave0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int64_t stride = int64_t(gridDim.x) * (blockDim.x / kWave);
  const int g = lane / LPR, c = lane % LPR;
  const int U = a.U;
  const int64_t N = a.N;
  const int64_t n_groups = a.n_groups;
  // the LM head streams its weights once; the layer GEMVs measured faster with the default policy
  constexpr bool NT = OUT == kOutArgmax && nt_capable(F);

  // row of (row group rg, row slot r, lane group g); SWIGLU pairs gate row f with up row half+f
  auto row_of = [&](int64_t rg, int r) -> int64_t {
    if constexpr (OUT == kOutSwiglu) {
      if constexpr (G == 1) {
        const int64_t f = rg * (R / 2) + r / 2;
        return (r & 1) ? a.half + f : f;
      } else {
        const int64_t f = (rg * R + r) * (G / 2) + g / 2;
        return (g & 1) ? a.half + f : f;
      }
    } else {
      return rg * (G * R) + int64_t(r) * G + g;
    }
  };
  auto row_valid = [&](int64_t rg, int r) -> bool {
    if constexpr (OUT == kOutSwiglu) {
      if constexpr (G == 1) {
        return rg * (R / 2) + r / 2 < a.half;
      } else {
        return (rg * R + r) * (G / 2) + g / 2 < a.half;
      }
    } else {
      return row_of(rg, r) < N;
    }
  };
  // Unconditional loads: a row past the end reads row 0, a unit past the row end reads the
  // row's last unit; neither reaches a result (row_valid and u < U mask them below).  The
  // residual epilogue's read of y rides with the weights: issued after them, a load of y would
  // make the wait for it a wait for everything issued before (loads complete in order).  Each
  // row of y is read and then written by the one wave that owns it.
  auto load_rows = [&](int64_t rg, typename Ut::W (&wt)[R][UPL], float (&yr)[R]) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const bool ok = rg < n_groups && row_valid(rg, r);
      const int64_t row = ok ? row_of(rg, r) : 0;
      if constexpr (OUT == kOutResid) yr[r] = a.y[row];
#pragma unroll
      for (int t = 0; t < UPL; t++) load_unit<F, NT>(wt[r][t], a.w, a.rb, N, U, row, min(c + LPR * t, U - 1));
    }
  };

  // 1. input loads, then the first row group's weight loads, then the prologue
  constexpr bool NORM = OUT != kOutResid;  // residual epilogues (Wo, down) take un-normalised input
  XRegs<ACT, XB, NORM> X;
  load_x<ACT, XB, NORM>(X, a.x, NORM ? a.norm_w : nullptr, a.K);
  // The next row group's weights are prefetched into the other of two register buffers, so
  // the wait before a group's math covers only that group's loads (reloading in place
  // instead, to fit two workgroups per CU on long rows, measured slower).
  typename Ut::W wa[R][UPL], wb[R][UPL];
  float ya[R], yb[R];
  load_rows(wave0, wa, ya);
  pin_x(X);
  // 2. activation blocks in LDS (every thread takes part)
  const bool tracing = blockIdx.x == 0 && a.tr_q8 != nullptr;
  const bool has_norm = NORM && a.norm_w != nullptr;
  const float xscale = build_act_lds<ACT, XB, NORM>(X, has_norm, a.eps, a.K, s_act, s_tmp);
  // The activation units stay in registers for all rows (re-reading them from LDS per row, to
  // fit two workgroups per CU on long rows, measured slower).
  typename Ut::Act act[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) Ut::load_act(act[t], s_act, min(c + LPR * t, U - 1));
  const bool last = c == LPR - 1;
  float best_v = -INFINITY;
  int64_t best_i = -1;
  // 3. row groups: reduce one group while the next one's loads are in flight
  auto process = [&](int64_t rg, const typename Ut::W (&cur)[R][UPL], const float (&yres)[R]) {
    float vals[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      float acc = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        const float d = Ut::dot(cur[r][t], act[t], nullptr);
        acc += (c + LPR * t < U) ? d : 0.f;
      }
      vals[r] = group_sum_last<LPR>(acc);
    }
    if constexpr (OUT == kOutSwiglu) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        if constexpr (G == 1) {
          if ((r & 1) && last && row_valid(rg, r)) {
            const float gv = vals[r - 1], uv = vals[r];
            const int64_t f = row_of(rg, r) - a.half;
            a.y[f] = gv / (1.0f + expf(-gv)) * uv;
            if (a.tr_gu) {
              a.tr_gu[f] = gv;
              a.tr_gu[a.half + f] = uv;
            }
          }
        } else {
          const float gv = __shfl(vals[r], lane - LPR, kWave);
          if ((g & 1) && last && row_valid(rg, r)) {
            const int64_t f = row_of(rg, r) - a.half;
            a.y[f] = gv / (1.0f + expf(-gv)) * vals[r];
            if (a.tr_gu) {
              a.tr_gu[f] = gv;
              a.tr_gu[a.half + f] = vals[r];
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int64_t row = row_of(rg, r);
        if (last && row < N) {
          if constexpr (OUT == kOutResid) {
            a.y[row] = yres[r] + vals[r];
          } else {
            a.y[row] = vals[r];
            if constexpr (OUT == kOutArgmax) {
              const float v = vals[r];
              if (!isnan(v) && (best_i < 0 || v > best_v)) {  // rows ascend: strict > keeps the first
                best_v = v;
                best_i = row;
              }
            }
          }
        }
      }
    }
  };
  // (sched_barrier: all of the next group's loads are issued before this group's math)
  for (int64_t rg = wave0; rg < n_groups; rg += 2 * stride) {
    load_rows(rg + stride, wb, yb);
    __builtin_amdgcn_sched_barrier(0);
    process(rg, wa, ya);
    if (rg + stride >= n_groups) break;
    load_rows(rg + 2 * stride, wa, ya);
    __builtin_amdgcn_sched_barrier(0);
    process(rg + stride, wb, yb);
  }
  // debug trace of the prologue (LDS is not written after it); stores before the rows would leave
  // the compiler unable to count the weight loads still in flight
  if (tracing) {
    trace_act(a.tr_q8, s_act, int(ACT == JERO_Q8_K ? a.K / 256 * 292 : a.K / 32 * 36));
    if (a.tr_xn) trace_xn(a.tr_xn, a.x, a.norm_w, has_norm, xscale, a.K);
  }
  if constexpr (OUT == kOutArgmax) {
    // (max, first index) over the workgroup's rows, NaN skipped
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float ov = __shfl_xor(best_v, off, kWave);
      int64_t oi = __shfl_xor(best_i, off, kWave);
      if (oi >= 0 && (best_i < 0 || ov > best_v || (ov == best_v && oi < best_i))) {
        best_v = ov;
        best_i = oi;
      }
    }
    __shared__ float s_bv[kDecodeThreads / 64];
    __shared__ int64_t s_bi[kDecodeThreads / 64];
    if (lane == 0) {
      s_bv[wv] = best_v;
      s_bi[wv] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int i = 1; i < int(blockDim.x >> 6); i++) {
        if (s_bi[i] >= 0 && (best_i < 0 || s_bv[i] > best_v || (s_bv[i] == best_v && s_bi[i] < best_i))) {
          best_v = s_bv[i];
          best_i = s_bi[i];
        }
      }
      a.amax_v[blockIdx.x] = best_v;
      a.amax_i[blockIdx.x] = best_i;
    }
  }
}

// ---------------------------------------------------------------- two tensors, one launch

// Loads of row r of a K-quant tensor for one wave (64 lanes), unconditional: a row past the end
// reads row 0 and a unit past the row end reads the row's last unit (masked in the dot).
template <int F, int UPL>
__device__ __forceinline__ void load_row_units(const uint8_t* __restrict__ w, int64_t rb, int U, int64_t N, int64_t r,
                                               typename Unit<F>::W (&wt)[UPL]) {
  const int c = threadIdx.x & 63;
  const int64_t row = r < N ? r : 0;
#pragma unroll
  for (int t = 0; t < UPL; t++) {
    const int u = min(c + 64 * t, U - 1);
    if constexpr (is_planar(F))
      Unit<F>::load_w_planar(wt[t], w, N, U, row, u);
    else
      Unit<F>::load_w(wt[t], w + row * rb, u);
  }
}

// Rows of one store segment for this wave: rows r_begin, r_begin + stride, ... below N of a
// K-quant tensor, one row per wave (64 lanes), dotted with the activation blocks in LDS.  `wa`
// holds the first row's weights, already issued; the next row's loads go into the other
// buffer before each row's math.
template <int F, int UPL>
__device__ __forceinline__ void store_segment(const uint8_t* __restrict__ w, int64_t rb, int U, int64_t N,
                                              int64_t r_begin, int64_t stride, const uint8_t* s_act, float* y,
                                              typename Unit<F>::W (&wa)[UPL]) {
  using Ut = Unit<F>;
  const int c = threadIdx.x & 63;
  typename Ut::Act act[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) Ut::load_act(act[t], s_act, min(c + 64 * t, U - 1));
  auto process = [&](int64_t r, const typename Ut::W (&cur)[UPL]) {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const float d = Ut::dot(cur[t], act[t], nullptr);
      acc += (c + 64 * t < U) ? d : 0.f;
    }
    acc = group_sum_last<64>(acc);
    if (c == 63) y[r] = acc;
  };
  typename Ut::W wb[UPL];
  for (int64_t r = r_begin; r < N; r += 2 * stride) {
    load_row_units<F, UPL>(w, rb, U, N, r + stride, wb);
    __builtin_amdgcn_sched_barrier(0);
    process(r, wa);
    if (r + stride >= N) break;
    load_row_units<F, UPL>(w, rb, U, N, r + 2 * stride, wa);
    __builtin_amdgcn_sched_barrier(0);
    process(r + stride, wb);
  }
}

// rmsnorm(x) . [W1; W2] for two K-quant tensors of different formats (the Q|K and V projections
// of a layer whose attn_v is Q6_K): rows [0, N) of W1 then rows [0, N2) of W2 into y[0, N + N2).
// One prologue (RMSNorm + Q8_K blocks in LDS) serves both; each wave runs its W1 rows, then its
// W2 rows, in the order of one persistent row index over both tensors.
template <int F1, int F2, int UPL, int XB>
__global__ void __launch_bounds__(kDecodeThreads) dgemv_dual_kernel(DGemvArgs a) {
  static_assert(F1 != JERO_Q8_0 && F1 != JERO_Q4_0 && F2 != JERO_Q8_0 && F2 != JERO_Q4_0, "K-quants only");
  extern __shared__ __attribute__((aligned(16))) uint8_t s_mem[];
  float* s_tmp = reinterpret_cast<float*>(s_mem);
  uint8_t* s_act = s_mem + 256;
  const int64_t wave0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int64_t stride = int64_t(gridDim.x) * (blockDim.x / kWave);
  const int64_t N1 = a.N, total = a.N + a.N2;
  // first row index of the wave in each segment (the persistent index runs over N1 + N2 rows)
  const int64_t r1 = wave0;
  const int64_t r2 = (wave0 >= N1 ? wave0 : wave0 + ((N1 - wave0 + stride - 1) / stride) * stride) - N1;
  XRegs<JERO_Q8_K, XB, true> X;
  load_x<JERO_Q8_K, XB, true>(X, a.x, a.norm_w, a.K);
  typename Unit<F1>::W c1[UPL];
  typename Unit<F2>::W c2[UPL];
  load_row_units<F1, UPL>(a.w, a.rb, a.U, N1, r1, c1);
  pin_x(X);
  const bool tracing = blockIdx.x == 0 && a.tr_q8 != nullptr;
  const float xscale = build_act_lds<JERO_Q8_K, XB, true>(X, a.norm_w != nullptr, a.eps, a.K, s_act, s_tmp);
  store_segment<F1, UPL>(a.w, a.rb, a.U, N1, r1, stride, s_act, a.y, c1);
  if (r2 + N1 < total) {
    load_row_units<F2, UPL>(a.w2, a.rb2, a.U, a.N2, r2, c2);
    store_segment<F2, UPL>(a.w2, a.rb2, a.U, a.N2, r2, stride, s_act, a.y + N1, c2);
  }
  if (tracing) {  // after the rows (see dgemv_kernel)
    trace_act(a.tr_q8, s_act, a.K / 256 * 292);
    if (a.tr_xn) trace_xn(a.tr_xn, a.x, a.norm_w, a.norm_w != nullptr, xscale, a.K);
  }
}

// ---------------------------------------------------------------- small kernels

// hidden = embed_token(*token) (src/qwen_deepseek.rs:558-582): row *token of token_embd's `rows`,
// or the deterministic row of a token past them (embed_value); -1 (the greedy token of all-NaN
// logits) embeds as zeros.
// Block 0 also writes the step's RoPE table: (cos, sin) of pos / theta^(2i/hd), the f32 angle
// of the reference's apply_rope_inplace (src/qwen_deepseek.rs:1056-1071).
__global__ void __launch_bounds__(256) embed_kernel(int quant, const uint8_t* __restrict__ w, int64_t rb, int H,
                                                    int64_t rows, const int32_t* __restrict__ token,
                                                    float* __restrict__ out, const int64_t* __restrict__ pos,
                                                    float theta, int hd, float* __restrict__ rope_cs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && threadIdx.x < hd / 2) {
    const float expo = float(2 * threadIdx.x) / float(hd);
    const float angle = float(*pos) / powf(theta, expo);
    float sn, cs;
    sincosf(angle, &sn, &cs);
    rope_cs[2 * threadIdx.x] = cs;
    rope_cs[2 * threadIdx.x + 1] = sn;
  }
  if (i >= H) return;
  out[i] = embed_value(quant, w, rb, rows, *token, i);
}

// (max, first index) merge of sample_greedy_argmax (src/engine.rs:1873-1895): NaN never wins,
// a larger value wins, an equal value keeps the lower index.  idx < 0 marks "no value yet".
__device__ __forceinline__ void argmax_merge(float& bv, int64_t& bi, float ov, int64_t oi) {
  if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
    bv = ov;
    bi = oi;
  }
}

// Workgroup-wide (max, first index) of per-thread candidates; the result is in thread 0.
__device__ __forceinline__ void argmax_block(float& bv, int64_t& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, kWave);
    const int64_t oi = __shfl_xor(bi, off, kWave);
    argmax_merge(bv, bi, ov, oi);
  }
  __shared__ float s_bv[16];
  __shared__ int64_t s_bi[16];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) {
    s_bv[wv] = bv;
    s_bi[wv] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int i = 1; i < int(blockDim.x >> 6); i++) argmax_merge(bv, bi, s_bv[i], s_bi[i]);
}

// Per-workgroup (max, first index) of a contiguous chunk of x (the standalone argmax_f32).
__global__ void __launch_bounds__(1024) argmax_partial_kernel(const float* __restrict__ x, int64_t n, int64_t chunk,
                                                              float* __restrict__ pv, int64_t* __restrict__ pi) {
  const int64_t b0 = int64_t(blockIdx.x) * chunk;
  const int64_t b1 = b0 + chunk < n ? b0 + chunk : n;
  float bv = -INFINITY;
  int64_t bi = -1;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) {  // ascending per thread
    const float v = x[i];
    if (!isnan(v) && (bi < 0 || v > bv)) {
      bv = v;
      bi = i;
    }
  }
  argmax_block(bv, bi);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = bv;
    pi[blockIdx.x] = bi;
  }
}

// The greedy token from n per-workgroup (max, index) pairs.
//   Decode step (pos != null): *token = the index and the position advances.  Logits that are
//   all NaN (or empty) leave no index: the reference's engine then fails closed
//   (src/engine.rs:636-641), so the step sets the sticky *status, stores token -1 and keeps the
//   position; while *status is set later steps store -1 and leave the position alone (the
//   host reads the status and must set a new position to go on).
//   Standalone argmax (pos == null): *out_idx = the index, -1 for none (Option::None).
__global__ void __launch_bounds__(1024) argmax_final_kernel(const float* __restrict__ v, const int64_t* __restrict__ idx,
                                                            int n, int32_t* __restrict__ token,
                                                            int64_t* __restrict__ pos, int32_t* __restrict__ status,
                                                            int64_t* __restrict__ out_idx) {
  float bv = -INFINITY;
  int64_t bi = -1;
  for (int i = threadIdx.x; i < n; i += blockDim.x) argmax_merge(bv, bi, v[i], idx[i]);
  argmax_block(bv, bi);
  if (threadIdx.x == 0) {
    if (pos == nullptr) {
      *out_idx = bi;
    } else if (*status != 0) {
      *token = -1;
    } else if (bi < 0) {
      *status = 1;
      *token = -1;
    } else {
      *token = int32_t(bi);
      *pos += 1;
    }
  }
}

// ---------------------------------------------------------------- long rows

// The fused decode GEMV for rows longer than the register-resident path takes (dgemv_max_k):
// the prologue loops over the activation blocks, building them in LDS (after RMSNorm: a first
// pass sums the squares), and each wave then reduces one row (SwiGLU: a gate row and its up
// row) at a time, loading UPL units per lane per step and the activation units from LDS.  The
// epilogues and the debug trace are the register-resident kernel's.
template <int F, int OUT>
__global__ void __launch_bounds__(kDecodeThreads) dgemv_long_kernel(DGemvArgs a) {
  using Ut = Unit<F>;
  constexpr int ACT = (F == JERO_Q8_0 || F == JERO_Q4_0) ? JERO_ACT_Q8 : JERO_Q8_K;
  constexpr int R = OUT == kOutSwiglu ? 2 : 1;
  constexpr int UPL = 4;
  constexpr bool NORM = OUT != kOutResid;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_mem[];
  float* s_tmp = reinterpret_cast<float*>(s_mem);
  uint8_t* s_act = s_mem + 256;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nwv = blockDim.x >> 6;
  const int K = a.K, U = a.U;
  const bool has_norm = NORM && a.norm_w != nullptr;
  const bool tracing = blockIdx.x == 0 && a.tr_q8 != nullptr;
  float* tr_xn = tracing ? a.tr_xn : nullptr;
  // 1. prologue
  float scale = 1.0f;
  if (has_norm) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) ss += a.x[i] * a.x[i];
    ss = block_sum(ss, s_tmp);
    scale = 1.0f / sqrtf(ss / float(K) + a.eps);
  }
  if constexpr (ACT == JERO_Q8_K) {
    for (int b = wv; b < K / 256; b += nwv) {
      const float4 xv = reinterpret_cast<const float4*>(a.x + b * 256)[lane];
      float e[4] = {xv.x, xv.y, xv.z, xv.w};
      if (has_norm) {
        const float4 g = reinterpret_cast<const float4*>(a.norm_w + b * 256)[lane];
        e[0] = e[0] * scale * g.x;
        e[1] = e[1] * scale * g.y;
        e[2] = e[2] * scale * g.z;
        e[3] = e[3] * scale * g.w;
      }
      if (tr_xn) reinterpret_cast<float4*>(tr_xn + b * 256)[lane] = make_float4(e[0], e[1], e[2], e[3]);
      q8k_block_wave(e, lane, s_act + b * 292);
    }
  } else {
    const int nb = K / 32, l = lane & 31;
    for (int p = wv; 2 * p < nb; p += nwv) {  // both half-waves take the same number of steps
      const int b = 2 * p + (lane >> 5);
      const bool ok = b < nb;
      const int bb = ok ? b : nb - 1;
      float v = a.x[bb * 32 + l];
      if (has_norm) v = v * scale * a.norm_w[bb * 32 + l];
      if (tr_xn && ok) tr_xn[b * 32 + l] = v;
      float am = fabsf(v);
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, kWave));
      const float d = am / 127.0f;
      const float id = d != 0.0f ? 1.0f / d : 0.0f;
      if (ok) {
        s_act[b * 36 + 4 + l] = uint8_t(int8_t(int(__builtin_rintf(v * id))));
        if (l == 0) *reinterpret_cast<float*>(s_act + b * 36) = d;
      }
    }
  }
  lds_barrier();
  if (tracing) trace_act(a.tr_q8, s_act, int(ACT == JERO_Q8_K ? K / 256 * 292 : K / 32 * 36));
  // 2. rows
  const int64_t wave0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int64_t stride = int64_t(gridDim.x) * nwv;
  const int64_t items = OUT == kOutSwiglu ? a.half : a.N;
  float best_v = -INFINITY;
  int64_t best_i = -1;
  for (int64_t it = wave0; it < items; it += stride) {
    int64_t rows[R];
    rows[0] = it;
    if constexpr (R == 2) rows[1] = a.half + it;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int u0 = 0; u0 < U; u0 += 64 * UPL) {
      typename Ut::W wt[R][UPL];
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < UPL; t++) {
          const int u = min(u0 + lane + 64 * t, U - 1);
          if constexpr (is_planar(F))
            Ut::load_w_planar(wt[r][t], a.w, a.N, U, rows[r], u);
          else
            Ut::load_w(wt[r][t], a.w + rows[r] * a.rb, u);
        }
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        const int u = u0 + lane + 64 * t;
        typename Ut::Act act;
        Ut::load_act(act, s_act, min(u, U - 1));
#pragma unroll
        for (int r = 0; r < R; r++) {
          const float d = Ut::dot(wt[r][t], act, nullptr);
          acc[r] += u < U ? d : 0.f;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = group_sum_last<64>(acc[r]);
    if (lane == 63) {
      if constexpr (OUT == kOutSwiglu) {
        const float gv = acc[0], uv = acc[1];
        a.y[it] = gv / (1.0f + expf(-gv)) * uv;
        if (a.tr_gu) {
          a.tr_gu[it] = gv;
          a.tr_gu[a.half + it] = uv;
        }
      } else if constexpr (OUT == kOutResid) {
        a.y[it] = a.y[it] + acc[0];
      } else {
        a.y[it] = acc[0];
        if constexpr (OUT == kOutArgmax) {
          if (!isnan(acc[0]) && (best_i < 0 || acc[0] > best_v)) {  // rows ascend per wave
            best_v = acc[0];
            best_i = it;
          }
        }
      }
    }
  }
  if constexpr (OUT == kOutArgmax) {
    argmax_block(best_v, best_i);
    if (threadIdx.x == 0) {
      a.amax_v[blockIdx.x] = best_v;
      a.amax_i[blockIdx.x] = best_i;
    }
  }
}

__global__ void set_state_kernel(int32_t* token, int64_t* pos, int32_t* status, int32_t t, int64_t p) {
  *token = t;
  *pos = p;
  *status = 0;
}

// ---------------------------------------------------------------- launchers

namespace {

// Workgroups of one dgemv instance that fit on a CU at once (registers and LDS); the
// persistent grid never exceeds what is resident, or a second batch of workgroups would
// start only after the first one drained.
template <int F, int LPR, int UPL, int R, int OUT, int XB>
int dgemv_fit() {
  static const int fit = [] {
    int nb = 0;
    const size_t shm = 256 + size_t(XB) * (kDecodeThreads / kWave) * 292 + 16;  // prologue LDS bound
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, dgemv_kernel<F, LPR, UPL, R, OUT, XB>, kDecodeThreads,
                                                     shm) != hipSuccess || nb < 1)
      nb = 1;
    return nb;
  }();
  return fit;
}

template <int F, int LPR, int UPL, int R, int OUT, int XB>
int dgemv_one(DGemvArgs a, int64_t rows_or_pairs, hipStream_t s) {
  constexpr int G = kWave / LPR;
  if constexpr (OUT == kOutSwiglu) {
    const int64_t per = G == 1 ? R / 2 : R * (G / 2);
    a.n_groups = (rows_or_pairs + per - 1) / per;
  } else {
    a.n_groups = (rows_or_pairs + G * R - 1) / (G * R);
  }
  const int64_t wpb = kDecodeThreads / kWave;
  int64_t blocks = (a.n_groups + wpb - 1) / wpb;
  const int per_cu = std::min(kDecodeBlocksPerCU, dgemv_fit<F, LPR, UPL, R, OUT, XB>());
  const int64_t cap = int64_t(device_info().cus) * per_cu;
  if (blocks > cap) blocks = cap;
  if (a.max_blocks > 0 && blocks > a.max_blocks) blocks = a.max_blocks;
  const size_t shm = 256 + size_t(row_bytes((F == JERO_Q8_0 || F == JERO_Q4_0) ? JERO_ACT_Q8 : JERO_Q8_K, a.K));
  hipLaunchKernelGGL((dgemv_kernel<F, LPR, UPL, R, OUT, XB>), dim3(unsigned(blocks)), dim3(kDecodeThreads),
                     (shm + 15) & ~size_t(15), s, a);
  return int(blocks);
}

// Activation blocks each wave builds in the prologue.
inline int xb_for(int F, int K) {
  const int waves = kDecodeThreads / kWave;
  const int per = (F == JERO_Q8_0 || F == JERO_Q4_0) ? (K / 32 + 2 * waves - 1) / (2 * waves)
                                                      : (K / 256 + waves - 1) / waves;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 6 ? 6 : 8;
}

template <int F, int LPR, int UPL, int OUT>
int dgemv_xb(const DGemvArgs& a, int64_t rows_or_pairs, hipStream_t s) {
  // one row per wave slot; SwiGLU with one row group per wave needs its gate/up pair in-wave
  constexpr int R = (OUT == kOutSwiglu && LPR == 64) ? 2 : 1;
  switch (xb_for(F, a.K)) {
    case 1: return dgemv_one<F, LPR, UPL, R, OUT, 1>(a, rows_or_pairs, s);
    case 2: return dgemv_one<F, LPR, UPL, R, OUT, 2>(a, rows_or_pairs, s);
    case 4: return dgemv_one<F, LPR, UPL, R, OUT, 4>(a, rows_or_pairs, s);
    case 6: return dgemv_one<F, LPR, UPL, R, OUT, 6>(a, rows_or_pairs, s);
    default: return dgemv_one<F, LPR, UPL, R, OUT, 8>(a, rows_or_pairs, s);
  }
}

// Returns the workgroups launched (> 0) or a negated status.
template <int F, int OUT>
int dgemv_fmt(const DGemvArgs& a, int64_t rows_or_pairs, hipStream_t s) {
  const int U = a.U;
  const int lpr = U > 32 ? 64 : U > 16 ? 32 : U > 4 ? 16 : 4;
  const int upl = (U + lpr - 1) / lpr;
  if (lpr == 4) return dgemv_xb<F, 4, 1, OUT>(a, rows_or_pairs, s);
  if (lpr == 16) return dgemv_xb<F, 16, 1, OUT>(a, rows_or_pairs, s);
  if (lpr == 32) return dgemv_xb<F, 32, 1, OUT>(a, rows_or_pairs, s);
  if (upl == 1) return dgemv_xb<F, 64, 1, OUT>(a, rows_or_pairs, s);
  if (upl == 2) return dgemv_xb<F, 64, 2, OUT>(a, rows_or_pairs, s);
  if (upl <= 3) return dgemv_xb<F, 64, 3, OUT>(a, rows_or_pairs, s);
  if (upl <= 4) return dgemv_xb<F, 64, 4, OUT>(a, rows_or_pairs, s);
  return -fail(JERO_ERR_CAPABILITY_MISMATCH, "decode: row of " + std::to_string(a.K) + " elements too long");
}

template <int F, int OUT>
int dgemv_long(DGemvArgs a, hipStream_t s) {
  const int64_t items = OUT == kOutSwiglu ? a.half : a.N;
  int64_t blocks = (items + kDecodeThreads / kWave - 1) / (kDecodeThreads / kWave);
  const int64_t cap = int64_t(device_info().cus) * kDecodeBlocksPerCU;
  if (blocks > cap) blocks = cap;
  if (a.max_blocks > 0 && blocks > a.max_blocks) blocks = a.max_blocks;
  const size_t shm = 256 + size_t(row_bytes((F == JERO_Q8_0 || F == JERO_Q4_0) ? JERO_ACT_Q8 : JERO_Q8_K, a.K));
  hipLaunchKernelGGL((dgemv_long_kernel<F, OUT>), dim3(unsigned(blocks)), dim3(kDecodeThreads), (shm + 15) & ~size_t(15),
                     s, a);
  return int(blocks);
}

template <int OUT>
int dgemv_out(int quant, const DGemvArgs& a, int64_t rows_or_pairs, hipStream_t s) {
  if (a.K > dgemv_max_k(quant)) {  // rows beyond the register-resident path
    switch (quant) {
      case JERO_Q4_K_R: return dgemv_long<JERO_Q4_K_R, OUT>(a, s);
      case JERO_Q6_K: return dgemv_long<JERO_Q6_K, OUT>(a, s);
      case JERO_Q6_K_R: return dgemv_long<JERO_Q6_K_R, OUT>(a, s);
      case JERO_Q8_0: return dgemv_long<JERO_Q8_0, OUT>(a, s);
      case JERO_Q4_0: return dgemv_long<JERO_Q4_0, OUT>(a, s);
    }
    return -fail(JERO_ERR_CAPABILITY_MISMATCH, "decode: unsupported weight quantization " + std::to_string(quant));
  }
  // K-quant matrices reach the decode step in their planar layouts (the model re-lays them out
  // at finalize); raw Q6_K remains for tensors the caller hands over unconverted
  switch (quant) {
    case JERO_Q4_K_R: return dgemv_fmt<JERO_Q4_K_R, OUT>(a, rows_or_pairs, s);
    case JERO_Q6_K: return dgemv_fmt<JERO_Q6_K, OUT>(a, rows_or_pairs, s);
    case JERO_Q6_K_R: return dgemv_fmt<JERO_Q6_K_R, OUT>(a, rows_or_pairs, s);
    case JERO_Q8_0: return dgemv_fmt<JERO_Q8_0, OUT>(a, rows_or_pairs, s);
    case JERO_Q4_0: return dgemv_fmt<JERO_Q4_0, OUT>(a, rows_or_pairs, s);
  }
  return -fail(JERO_ERR_CAPABILITY_MISMATCH, "decode: unsupported weight quantization " + std::to_string(quant));
}

}  // namespace

int launch_dgemv(int quant, int out_mode, const DGemvArgs& a, hipStream_t s, int* blocks) {
  int rc;
  switch (out_mode) {
    case kOutStore: rc = dgemv_out<kOutStore>(quant, a, a.N, s); break;
    case kOutResid: rc = dgemv_out<kOutResid>(quant, a, a.N, s); break;
    case kOutSwiglu: rc = dgemv_out<kOutSwiglu>(quant, a, a.half, s); break;
    case kOutArgmax: rc = dgemv_out<kOutArgmax>(quant, a, a.N, s); break;
    default: return fail(JERO_ERR_INVALID_ARGUMENT, "decode: bad output mode");
  }
  if (rc < 0) return -rc;
  if (blocks) *blocks = rc;
  return check_launch("decode gemv");
}

int launch_dgemv_dual(int quant1, int quant2, const DGemvArgs& a0, hipStream_t s) {
  if (a0.U > 64 || a0.K % 256 != 0)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "decode: two-tensor GEMV takes rows of at most 4096 K-quant elements");
  DGemvArgs a = a0;
  const int64_t wpb = kDecodeThreads / kWave;
  int64_t blocks = (a.N + a.N2 + wpb - 1) / wpb;
  const int64_t cap = int64_t(device_info().cus) * kDecodeBlocksPerCU;
  if (blocks > cap) blocks = cap;
  const size_t shm = (256 + size_t(row_bytes(JERO_Q8_K, a.K)) + 15) & ~size_t(15);
  const int xb = xb_for(JERO_Q4_K, a.K);
#define JERO_DUAL(Q1, Q2, XBV)                                                                            \
  hipLaunchKernelGGL((dgemv_dual_kernel<Q1, Q2, 1, XBV>), dim3(unsigned(blocks)), dim3(kDecodeThreads), shm, s, a)
  if (quant1 == JERO_Q4_K_R && quant2 == JERO_Q6_K_R) {
    if (xb <= 1) JERO_DUAL(JERO_Q4_K_R, JERO_Q6_K_R, 1);
    else JERO_DUAL(JERO_Q4_K_R, JERO_Q6_K_R, 2);
  } else if (quant1 == JERO_Q6_K_R && quant2 == JERO_Q4_K_R) {
    if (xb <= 1) JERO_DUAL(JERO_Q6_K_R, JERO_Q4_K_R, 1);
    else JERO_DUAL(JERO_Q6_K_R, JERO_Q4_K_R, 2);
  } else {
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "decode: no two-tensor GEMV for this format pair");
  }
#undef JERO_DUAL
  return check_launch("decode two-tensor gemv");
}

int dgemv_long_max_k(int quant) {
  // the activation blocks of a row live in LDS
  return (quant == JERO_Q8_0 || quant == JERO_Q4_0) ? (kDecodeMaxLongActBytes / 36) * 32
                                                    : (kDecodeMaxLongActBytes / 292) * 256;
}

int dgemv_max_k(int quant) {
  // UPL <= 4 units per lane, and the prologue's kDecodeMaxActBlocks blocks per wave
  return (quant == JERO_Q8_0 || quant == JERO_Q4_0) ? 32 * 2 * (kDecodeThreads / kWave) * kDecodeMaxActBlocks
                                                    : 256 * (kDecodeThreads / kWave) * kDecodeMaxActBlocks;
}

int launch_embed(int quant, const void* w, int64_t rb, int H, int64_t rows, const int32_t* token, float* out,
                 const int64_t* pos, float theta, int hd, float* rope_cs, hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel, dim3(unsigned((H + 255) / 256)), dim3(256), 0, s, quant,
                     static_cast<const uint8_t*>(w), rb, H, rows, token, out, pos, theta, hd, rope_cs);
  return check_launch("embed");
}

int launch_argmax_final(const float* v, const int64_t* idx, int n, int32_t* token, int64_t* pos, int32_t* status,
                        hipStream_t s) {
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, v, idx, n, token, pos, status, nullptr);
  return check_launch("argmax");
}

int argmax_partials(int64_t n) { return n <= 0 ? 0 : int(std::min<int64_t>(1024, (n + 8191) / 8192)); }

int launch_argmax(const float* x, int64_t n, int64_t* out_idx, float* pv, int64_t* pi, hipStream_t s) {
  const int nb = argmax_partials(n);
  if (nb > 0) {
    const int64_t chunk = (n + nb - 1) / nb;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(unsigned(nb)), dim3(1024), 0, s, x, n, chunk, pv, pi);
  }
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, s, pv, pi, nb, nullptr, nullptr, nullptr, out_idx);
  return check_launch("argmax");
}

// project_or_deterministic_slice's fallback (src/gemma.rs:841-860): y[i] = in[i % len] * scale for
// i < out_len, in = x, or RMSNorm(x) * norm_w when norm_w is set (each workgroup reduces the norm
// itself: len is a hidden size); RESID adds into y.  1024 outputs per workgroup; grid y is the
// row of a batch (x and y rows x_stride and y_stride floats apart).
__global__ void __launch_bounds__(256) det_proj_kernel(const float* __restrict__ x, int64_t len,
                                                        const float* __restrict__ norm_w, float eps, float scale,
                                                        float* __restrict__ y, int64_t out_len, int resid,
                                                        int64_t x_stride, int64_t y_stride) {
  __shared__ float s_tmp[4];
  x += blockIdx.y * x_stride;
  y += blockIdx.y * y_stride;
  float inv = 1.0f;
  if (norm_w) {
    float ss = 0.f;
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum(ss, s_tmp);
    inv = 1.0f / sqrtf(ss / float(len) + eps);
  }
  const int64_t end = min(out_len, int64_t(blockIdx.x + 1) * 1024);
  for (int64_t i = int64_t(blockIdx.x) * 1024 + threadIdx.x; i < end; i += blockDim.x) {
    const int64_t j = i % len;
    float v = x[j];
    if (norm_w) v = v * inv * norm_w[j];
    v *= scale;
    if (resid) y[i] += v;
    else y[i] = v;
  }
}

// SwiGLU of separately computed gate | up rows (the fused epilogue's formula): act[i] =
// silu(gu[i]) * gu[F + i].
__global__ void __launch_bounds__(256) swiglu_kernel(const float* __restrict__ gu, int64_t F, float* __restrict__ act) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= F) return;
  const float gv = gu[i], uv = gu[F + i];
  act[i] = gv / (1.0f + expf(-gv)) * uv;
}

// read_f32_weight_or_default (src/qwen_deepseek.rs:491-519) of a norm weight, out[len]: raw null
// (the tensor is absent) gives all ones; F32 keeps each finite stored value and gives 1.0 for a
// non-finite one and past the tensor's n_el elements; another format dequantizes its first len
// elements (row 0) when deq is set (at least len elements, len a whole number of blocks), else
// all ones.
__global__ void __launch_bounds__(256) norm_weight_kernel(int quant, const uint8_t* __restrict__ raw, int64_t n_el,
                                                           int64_t len, int deq, float* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= len) return;
  float v = 1.0f;
  if (raw != nullptr) {
    if (quant == JERO_F32) {
      if (i < n_el) {
        const float r = reinterpret_cast<const float*>(raw)[i];
        if (isfinite(r)) v = r;
      }
    } else if (deq) {
      v = dequant_elem(quant, raw, i);
    }
  }
  out[i] = v;
}

// The LM head's final RMSNorm of x into xn [H] (xn = x * (1 / sqrt(mean(x^2) + eps)) * nw, the
// head GEMV prologue's formula), for heads whose GEMV takes an f32 input (F32 / F16 / BF16 rows).
__global__ void __launch_bounds__(1024) head_norm_kernel(const float* __restrict__ x, const float* __restrict__ nw,
                                                          float eps, int64_t H, float* __restrict__ xn) {
  __shared__ float s_tmp[16];
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) ss += x[i] * x[i];
  ss = block_sum(ss, s_tmp);
  const float inv = 1.0f / sqrtf(ss / float(H) + eps);
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) xn[i] = x[i] * inv * nw[i];
}

// project_lm_head's logits that no head row gives (src/qwen_deepseek.rs:584-632), from the final
// hidden state x with xn = RMSNorm(x) * nw recomputed per workgroup:
//   mode 0, rows past a head of `start` rows (:614-616): logits[i] = xn[i % H] * 0.05;
//   mode 1, no usable head (:626-631): logits[i] = tanh(sum(xn) / 16) + xn[i % H] * 0.1 + (i % 13) * 0.01,
//   each operation rounded on its own as the reference computes it.
// Workgroup b covers [start + b kHeadTailRows, ...) and writes its (max, first index) at pv / pi[b]
// (pv null: none); workgroup 0 also writes xn to tr_xn (the trace's head input) when given.
__global__ void __launch_bounds__(256) head_tail_kernel(const float* __restrict__ x, const float* __restrict__ nw,
                                                         float eps, int64_t H, int mode, int64_t start, int64_t L,
                                                         float* __restrict__ logits, float* __restrict__ pv,
                                                         int64_t* __restrict__ pi, float* __restrict__ tr_xn) {
#pragma clang fp contract(off)
  __shared__ float s_tmp[4];
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += blockDim.x) ss += x[i] * x[i];
  ss = block_sum(ss, s_tmp);
  const float inv = 1.0f / sqrtf(ss / float(H) + eps);
  float base = 0.f;
  if (mode == 1) {
    float sx = 0.f;
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) sx += x[i] * inv * nw[i];
    __syncthreads();  // every wave has read s_tmp before it is reused
    sx = block_sum(sx, s_tmp);
    base = tanhf(sx / 16.0f);
  }
  if (tr_xn != nullptr && blockIdx.x == 0)
    for (int64_t i = threadIdx.x; i < H; i += blockDim.x) tr_xn[i] = x[i] * inv * nw[i];
  const int64_t b0 = start + int64_t(blockIdx.x) * kHeadTailRows;
  const int64_t b1 = b0 + kHeadTailRows < L ? b0 + kHeadTailRows : L;
  float bv = -INFINITY;
  int64_t bi = -1;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) {  // ascending per thread
    const int64_t j = i % H;
    const float xn = x[j] * inv * nw[j];
    const float v = mode == 0 ? xn * 0.05f : (base + xn * 0.1f) + float(i % 13) * 0.01f;  // no contraction
    logits[i] = v;
    if (!isnan(v) && (bi < 0 || v > bv)) {
      bv = v;
      bi = i;
    }
  }
  argmax_block(bv, bi);
  if (threadIdx.x == 0 && pv != nullptr) {
    pv[blockIdx.x] = bv;
    pi[blockIdx.x] = bi;
  }
}

int launch_norm_weight(int quant, const void* raw, int64_t n_el, int64_t len, bool deq, float* out, hipStream_t s) {
  hipLaunchKernelGGL(norm_weight_kernel, dim3(unsigned((len + 255) / 256)), dim3(256), 0, s, quant,
                     static_cast<const uint8_t*>(raw), n_el, len, deq ? 1 : 0, out);
  return check_launch("norm weight");
}

int launch_head_norm(const float* x, const float* nw, float eps, int64_t H, float* xn, hipStream_t s) {
  hipLaunchKernelGGL(head_norm_kernel, dim3(1), dim3(1024), 0, s, x, nw, eps, H, xn);
  return check_launch("head norm");
}

int head_tail_blocks(int64_t start, int64_t L) {
  return L > start ? int((L - start + kHeadTailRows - 1) / kHeadTailRows) : 0;
}

int launch_head_tail(const float* x, const float* nw, float eps, int64_t H, int mode, int64_t start, int64_t L,
                     float* logits, float* pv, int64_t* pi, float* tr_xn, hipStream_t s) {
  const int nb = head_tail_blocks(start, L);
  if (nb == 0) return JERO_OK;
  hipLaunchKernelGGL(head_tail_kernel, dim3(unsigned(nb)), dim3(256), 0, s, x, nw, eps, H, mode, start, L, logits, pv,
                     pi, tr_xn);
  return check_launch("head tail");
}

int launch_argmax_partials(const float* x, int64_t n, float* pv, int64_t* pi, hipStream_t s) {
  const int nb = argmax_partials(n);
  if (nb > 0) {
    const int64_t chunk = (n + nb - 1) / nb;
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(unsigned(nb)), dim3(1024), 0, s, x, n, chunk, pv, pi);
    if (check_launch("argmax partials")) return -1;
  }
  return nb;
}

int launch_det_proj(const float* x, int64_t len, const float* norm_w, float eps, float scale, float* y,
                    int64_t out_len, bool resid, hipStream_t s, int64_t rows, int64_t x_stride, int64_t y_stride) {
  hipLaunchKernelGGL(det_proj_kernel, dim3(unsigned((out_len + 1023) / 1024), unsigned(rows)), dim3(256), 0, s, x, len,
                     norm_w, eps, scale, y, out_len, resid ? 1 : 0, x_stride, y_stride);
  return check_launch("deterministic projection");
}

int launch_swiglu(const float* gu, int64_t F, float* act, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((F + 255) / 256)), dim3(256), 0, s, gu, F, act);
  return check_launch("swiglu");
}

int launch_set_state(int32_t* token, int64_t* pos, int32_t* status, int32_t t, int64_t p, hipStream_t s) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(1), 0, s, token, pos, status, t, p);
  return check_launch("set state");
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_argmax(const float* x_dev, int64_t n, int64_t* idx_dev, void* workspace_dev,
                               size_t workspace_bytes, void* stream) {
  if (!idx_dev || (n > 0 && !x_dev)) return fail(JERO_ERR_INVALID_ARGUMENT, "argmax: null pointer");
  if (n < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "argmax: negative length");
  if (reinterpret_cast<uintptr_t>(idx_dev) & 7u) return fail(JERO_ERR_INVALID_ARGUMENT, "argmax: index not 8-byte aligned");
  const int nb = argmax_partials(n);
  const size_t need = size_t(nb) * (sizeof(float) + sizeof(int64_t)) + 16;
  void* ws = workspace_dev;
  if (ws) {
    if (workspace_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "argmax: workspace of " + std::to_string(workspace_bytes) +
                                              " bytes, need " + std::to_string(need));
    if (reinterpret_cast<uintptr_t>(ws) & 7u)
      return fail(JERO_ERR_INVALID_ARGUMENT, "argmax: workspace must be 8-byte aligned");
  } else {
    const int rc = workspace(need, &ws);
    if (rc) return rc;
  }
  int64_t* pi = static_cast<int64_t*>(ws);
  float* pv = reinterpret_cast<float*>(pi + nb);
  return launch_argmax(x_dev, n, idx_dev, pv, pi, static_cast<hipStream_t>(stream));
}
