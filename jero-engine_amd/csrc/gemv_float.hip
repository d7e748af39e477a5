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

}  // namespace

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
