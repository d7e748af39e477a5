// gemv_float.hip -- GEMV over unquantized weight rows (F32, F16, BF16) on gfx950.
//
// Replaces matvec_f32 (src/gemma.rs:140-189, one dot_product_f32_scalar per row) and the
// vec_dot_f16 / vec_dot_bf16 arms of matvec_any_slice (src/gemma.rs:72-74), whose typical tensor
// on the hot path is a Qwen3-MoE router (ffn_gate_inp, F32 [hidden, n_experts]).  The input is the
// f32 vector itself (no activation quantization).  HBM-bound: LPR lanes share a row and walk it
// in 16-byte pieces, four pieces in flight per lane; products accumulate in f32 per lane (fma) and
// the row total is a DPP butterfly over the LPR lanes, so each row is reduced in one fixed order
// that depends only on n_in.  Rows that do not start 16-byte aligned (F16/BF16 with n_in not a
// multiple of 8, F32 with n_in not a multiple of 4) take an element-wise path with the same
// lane-to-element mapping at scalar width.  No row-length limit.
#include "gemv.h"

#include "jero_common.h"
#include "runtime.h"

namespace jero {

namespace {

constexpr int kFloatThreads = 256;
constexpr int kPieces = 4;  // 16-byte pieces in flight per lane

template <int Q>
__device__ __forceinline__ float widen(uint32_t bits16) {
  if constexpr (Q == JERO_BF16) return __uint_as_float(bits16 << 16);
  else return float(__builtin_bit_cast(_Float16, uint16_t(bits16)));
}

// Dot product of the 16 weight bytes v (4 f32 or 8 half-width values) with x[e0 ..).
template <int Q>
__device__ __forceinline__ float piece_dot(const u32x4 v, const float* __restrict__ x, int64_t e0, float acc) {
  if constexpr (Q == JERO_F32) {
    const float4 xv = *reinterpret_cast<const float4*>(x + e0);
    acc = fmaf(__uint_as_float(v.x), xv.x, acc);
    acc = fmaf(__uint_as_float(v.y), xv.y, acc);
    acc = fmaf(__uint_as_float(v.z), xv.z, acc);
    acc = fmaf(__uint_as_float(v.w), xv.w, acc);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(x + e0);
    const float4 b = *reinterpret_cast<const float4*>(x + e0 + 4);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      acc = fmaf(widen<Q>(w[i] & 0xFFFFu), xs[2 * i], acc);
      acc = fmaf(widen<Q>(w[i] >> 16), xs[2 * i + 1], acc);
    }
  }
  return acc;
}

// VEC: every row starts 16-byte aligned and K is a multiple of the piece width.
template <int Q, int LPR, bool VEC>
__global__ void __launch_bounds__(kFloatThreads) gemv_float_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                                   int64_t K, int64_t N, const float* __restrict__ x,
                                                                   float* __restrict__ y) {
  constexpr int ES = Q == JERO_F32 ? 4 : 2;  // bytes per element
  constexpr int EP = 16 / ES;                // elements per 16-byte piece
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x & 63, g = lane / LPR, c = lane % LPR;
  const int64_t row = ((int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave) * G + g;
  const int64_t rr = row < N ? row : N - 1;  // loads stay in bounds; the store is masked
  const uint8_t* wr = w + rr * rb;
  float acc = 0.f;
  if constexpr (VEC) {
    const int64_t pieces = K / EP;
    for (int64_t p0 = c; p0 < pieces; p0 += int64_t(LPR) * kPieces) {
      u32x4 v[kPieces];
#pragma unroll
      for (int i = 0; i < kPieces; i++) {
        const int64_t p = p0 + int64_t(LPR) * i;
        v[i] = *reinterpret_cast<const u32x4*>(wr + 16 * (p < pieces ? p : pieces - 1));
      }
#pragma unroll
      for (int i = 0; i < kPieces; i++) {
        const int64_t p = p0 + int64_t(LPR) * i;
        if (p < pieces) acc = piece_dot<Q>(v[i], x, p * EP, acc);
      }
    }
  } else {
    for (int64_t e = c; e < K; e += LPR) {
      float wv;
      if constexpr (Q == JERO_F32) wv = *reinterpret_cast<const float*>(wr + 4 * e);
      else wv = widen<Q>(*reinterpret_cast<const uint16_t*>(wr + 2 * e));
      acc = fmaf(wv, x[e], acc);
    }
  }
  acc = group_sum_last<LPR>(acc);
  if (c == LPR - 1 && row < N) y[row] = acc;
}

template <int Q, bool VEC>
void launch_q(const uint8_t* w, int64_t rb, int64_t K, int64_t N, const float* x, float* y, hipStream_t s) {
  constexpr int EP = 16 / (Q == JERO_F32 ? 4 : 2);
  const int64_t pieces = VEC ? K / EP : K;
  const int lpr = pieces >= 64 ? 64 : pieces >= 32 ? 32 : pieces >= 16 ? 16 : 4;
  const int64_t waves = (N + (kWave / lpr) - 1) / (kWave / lpr);
  const dim3 grid(unsigned((waves + kFloatThreads / kWave - 1) / (kFloatThreads / kWave)));
  switch (lpr) {
    case 64: hipLaunchKernelGGL((gemv_float_kernel<Q, 64, VEC>), grid, dim3(kFloatThreads), 0, s, w, rb, K, N, x, y); break;
    case 32: hipLaunchKernelGGL((gemv_float_kernel<Q, 32, VEC>), grid, dim3(kFloatThreads), 0, s, w, rb, K, N, x, y); break;
    case 16: hipLaunchKernelGGL((gemv_float_kernel<Q, 16, VEC>), grid, dim3(kFloatThreads), 0, s, w, rb, K, N, x, y); break;
    default: hipLaunchKernelGGL((gemv_float_kernel<Q, 4, VEC>), grid, dim3(kFloatThreads), 0, s, w, rb, K, N, x, y); break;
  }
}

template <int Q>
void launch_fq(const uint8_t* w, int64_t K, int64_t N, const float* x, float* y, hipStream_t s) {
  const int64_t rb = row_bytes(Q, K);
  const bool vec = (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && rb % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  if (vec) launch_q<Q, true>(w, rb, K, N, x, y, s);
  else launch_q<Q, false>(w, rb, K, N, x, y, s);
}

// The Qwen3-MoE FFN's first two steps in one launch (src/qwen_deepseek.rs:1278-1284, 882-892):
// xn = x * (1 / sqrt(mean(x^2) + eps)) * nw, then the router logits y = W xn over F32 rows of
// K elements (16-byte aligned, K % 4 == 0).  Every workgroup computes the norm itself (the same
// per-thread sums in the same order, so every workgroup holds the same xn bits) into LDS; the
// first also stores xn for the expert kernels.  The thread's elements of x and of the norm
// weights are loaded first, then each lane's first weight pieces, all unconditionally
// (clamped), so the norm waits for one round trip and overlaps the row fetch.
constexpr int kRouterPieces = 8;  // pieces per lane in flight: one pass over a 2048-wide row at LPR 64

template <int LPR, int PER>
__global__ void __launch_bounds__(kFloatThreads) router_norm_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                                    int64_t K, int64_t N, const float* __restrict__ x,
                                                                    const float* __restrict__ nw, float eps,
                                                                    float* __restrict__ xn, float* __restrict__ y) {
  extern __shared__ float s_x[];  // K floats
  __shared__ float s_tmp[kFloatThreads / kWave];
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x & 63, g = lane / LPR, c = lane % LPR;
  const int64_t row = ((int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave) * G + g;
  const int64_t rr = row < N ? row : N - 1;
  const uint8_t* wr = w + rr * rb;
  // the thread's elements i = tid + 256 j of x and of the norm weights, all loaded up front
  // (clamped), before the weights: the norm waits for one round trip and not for the weights
  float xv[PER], gv[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int64_t i = min<int64_t>(threadIdx.x + int64_t(kFloatThreads) * j, K - 1);
    xv[j] = x[i];
    gv[j] = nw[i];
  }
  const int64_t pieces = K / 4;
  u32x4 v[kRouterPieces];
#pragma unroll
  for (int i = 0; i < kRouterPieces; i++) {
    const int64_t p = c + int64_t(LPR) * i;
    v[i] = *reinterpret_cast<const u32x4*>(wr + 16 * (p < pieces ? p : pieces - 1));
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; j++)
    if (threadIdx.x + int64_t(kFloatThreads) * j < K) ss += xv[j] * xv[j];
  ss = wave_sum_dpp(ss);
  if (lane == 0) s_tmp[threadIdx.x >> 6] = ss;
  lds_barrier();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kFloatThreads / kWave; i++) t += s_tmp[i];
  const float inv = 1.0f / sqrtf(t / float(K) + eps);
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int64_t i = threadIdx.x + int64_t(kFloatThreads) * j;
    if (i < K) {
      const float e = xv[j] * inv * gv[j];
      s_x[i] = e;
      if (blockIdx.x == 0) xn[i] = e;
    }
  }
  lds_barrier();
  float acc = 0.f;
  for (int64_t p0 = c;; p0 += int64_t(LPR) * kRouterPieces) {
#pragma unroll
    for (int i = 0; i < kRouterPieces; i++) {
      const int64_t p = p0 + int64_t(LPR) * i;
      if (p < pieces) {
        const float4 xv = *reinterpret_cast<const float4*>(s_x + 4 * p);
        acc = fmaf(__uint_as_float(v[i].x), xv.x, acc);
        acc = fmaf(__uint_as_float(v[i].y), xv.y, acc);
        acc = fmaf(__uint_as_float(v[i].z), xv.z, acc);
        acc = fmaf(__uint_as_float(v[i].w), xv.w, acc);
      }
    }
    const int64_t next = p0 + int64_t(LPR) * kRouterPieces;
    if (next - c >= pieces) break;  // uniform across the wave: every lane's chunk start is p0 - c apart
#pragma unroll
    for (int i = 0; i < kRouterPieces; i++) {
      const int64_t p = next + int64_t(LPR) * i;
      v[i] = *reinterpret_cast<const u32x4*>(wr + 16 * (p < pieces ? p : pieces - 1));
    }
  }
  acc = group_sum_last<LPR>(acc);
  if (c == LPR - 1 && row < N) y[row] = acc;
}

// Y[t][n] = sum_k X[t][k] W[n][k] over F32 rows: the router logits of a batch of token rows (the
// batched prefill's form of matvec_f32 per token), on v_mfma_f32_16x16x4f32.  A workgroup owns one
// 16 x 16 tile (16 rows t, 16 rows n); its four waves take the four quarters of K (whole 64-wide
// chunks, the first waves one more when the chunk count is not a multiple of 4) and the tile is
// their sum, wave 0 + 1 + 2 + 3 in that order through LDS.  In a step, lane l supplies
// A[l % 16][l / 16] = X[t0 + l % 16][k] and B[l / 16][l % 16] = W[n0 + l % 16][k] with the same
// k = c + 4 (l / 16) + s for both; the lane reads 16 bytes of each row per 16 k, four of them per
// buffer, two buffers alternating.  D: lane l holds rows 4 (l / 16) + i of column l % 16.
// K % 64 == 0; rows past T or N are read clamped and not stored.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kRowsChunk = 64;

__global__ void __launch_bounds__(256) matmul_f32_rows_kernel(const float* __restrict__ w, int64_t K, int64_t N,
                                                              const float* __restrict__ x, int64_t T,
                                                              float* __restrict__ y, int64_t tiles_n) {
  __shared__ v4f s_part[3][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, r = lane & 15, q = lane >> 4;
  const int64_t tt = int64_t(blockIdx.x) / tiles_n, tn = int64_t(blockIdx.x) - tt * tiles_n;
  const int64_t chunks = K / kRowsChunk, per = chunks / 4, extra = chunks % 4;
  const int64_t c_lo = (wv * per + min<int64_t>(wv, extra)) * kRowsChunk;
  const int64_t c_hi = c_lo + (per + (wv < extra ? 1 : 0)) * kRowsChunk;  // this wave's K range
  const float* xr = x + min(tt * 16 + r, T - 1) * K + 4 * q;
  const float* wr = w + min(tn * 16 + r, N - 1) * K + 4 * q;
  auto load = [&](float4 (&xa)[4], float4 (&wa)[4], int64_t c) {
    c = min(c, K - kRowsChunk);  // past the end: the last chunk again (not used)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      xa[g] = *reinterpret_cast<const float4*>(xr + c + 16 * g);
      wa[g] = *reinterpret_cast<const float4*>(wr + c + 16 * g);
    }
  };
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  auto steps = [&](const float4 (&xa)[4], const float4 (&wa)[4]) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[g].x, wa[g].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[g].y, wa[g].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[g].z, wa[g].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[g].w, wa[g].w, acc, 0, 0, 0);
    }
  };
  if (c_lo < c_hi) {  // uniform over the wave
    float4 xa[4], wa[4], xb[4], wb[4];
    load(xa, wa, c_lo);
    for (int64_t c = c_lo;; c += 2 * kRowsChunk) {
      load(xb, wb, c + kRowsChunk);
      steps(xa, wa);
      if (c + kRowsChunk >= c_hi) break;
      load(xa, wa, c + 2 * kRowsChunk);
      steps(xb, wb);
      if (c + 2 * kRowsChunk >= c_hi) break;
    }
  }
  if (wv > 0) s_part[wv - 1][lane] = acc;
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int j = 0; j < 3; j++) acc += s_part[j][lane];
    const int64_t n = tn * 16 + r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int64_t t = tt * 16 + 4 * q + i;
      if (n < N && t < T) y[t * N + n] = acc[i];
    }
  }
}

}  // namespace

int launch_matmul_f32_rows(const void* w, int64_t n_in, int64_t n_out, const float* x, int64_t rows, float* y,
                           hipStream_t s) {
  if (n_in < kRowsChunk || n_in % kRowsChunk != 0 || n_out < 1 || rows < 1)
    return fail(JERO_ERR_TENSOR_BOUNDS, "router rows: n_in must be a positive multiple of 64");
  if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(x) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "router rows: weights and rows must be 16-byte aligned");
  const int64_t tiles_n = (n_out + 15) / 16, tiles = ((rows + 15) / 16) * tiles_n;
  hipLaunchKernelGGL(matmul_f32_rows_kernel, dim3(unsigned(tiles)), dim3(256), 0, s,
                     static_cast<const float*>(w), n_in, n_out, x, rows, y, tiles_n);
  return check_launch("router rows (F32)");
}

bool router_norm_fits(int quant, const void* w, int64_t n_in, const float* x, const float* xn) {
  return quant == JERO_F32 && n_in % 4 == 0 && n_in >= 4 && n_in <= kRouterMaxK &&
         (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
         (reinterpret_cast<uintptr_t>(xn) & 15u) == 0;
}

int launch_router_norm(const void* w, int64_t n_in, int64_t n_out, const float* x, const float* nw, float eps,
                       float* xn, float* y, hipStream_t s) {
  if (!router_norm_fits(JERO_F32, w, n_in, x, xn) || n_out < 1)
    return fail(JERO_ERR_INVALID_ARGUMENT, "router_norm: unsupported shape or alignment");
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  const int64_t rb = 4 * n_in, pieces = n_in / 4;
  const int lpr = pieces >= 64 ? 64 : pieces >= 32 ? 32 : pieces >= 16 ? 16 : 4;
  const int64_t waves = (n_out + (kWave / lpr) - 1) / (kWave / lpr);
  const dim3 grid(unsigned((waves + kFloatThreads / kWave - 1) / (kFloatThreads / kWave)));
  const size_t lds = sizeof(float) * size_t(n_in);
  const int per = int((n_in + kFloatThreads - 1) / kFloatThreads);  // elements per thread, <= 32
#define JERO_ROUTER(L, P)                                                                                 \
  hipLaunchKernelGGL((router_norm_kernel<L, P>), grid, dim3(kFloatThreads), lds, s, wb, rb, n_in, n_out, x, nw, \
                     eps, xn, y)
#define JERO_ROUTER_P(L)              \
  do {                                \
    if (per <= 8) JERO_ROUTER(L, 8);   \
    else if (per <= 16) JERO_ROUTER(L, 16); \
    else JERO_ROUTER(L, 32);          \
  } while (0)
  switch (lpr) {
    case 64: JERO_ROUTER_P(64); break;
    case 32: JERO_ROUTER_P(32); break;
    case 16: JERO_ROUTER_P(16); break;
    default: JERO_ROUTER_P(4); break;
  }
#undef JERO_ROUTER_P
#undef JERO_ROUTER
  return check_launch("router (norm + F32 rows)");
}

bool is_float_weight(int quant) { return quant == JERO_F32 || quant == JERO_F16 || quant == JERO_BF16; }

int launch_matvec_float(int quant, const void* w, int64_t n_in, int64_t n_out, const float* x, float* y,
                        hipStream_t s) {
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  switch (quant) {
    case JERO_F32: launch_fq<JERO_F32>(wb, n_in, n_out, x, y, s); break;
    case JERO_F16: launch_fq<JERO_F16>(wb, n_in, n_out, x, y, s); break;
    case JERO_BF16: launch_fq<JERO_BF16>(wb, n_in, n_out, x, y, s); break;
    default: return fail(JERO_ERR_CAPABILITY_MISMATCH, "matvec: not a float weight format");
  }
  return check_launch("matvec (float weights)");
}

}  // namespace jero
