// gemv.hip -- decode GEMV y = W x over GGUF weight bytes on gfx950.
//
// Replaces matvec_any (src/gemma.rs:100-138) and the vec_dot_* kernels it dispatches to
// (src/gemma.rs:66-95).  Design (activation-stationary, one wave = a group of rows):
//   * A row is cut into units (gemv_dot.h).  LPR lanes share one row; lane c of the row owns
//     units c, c+LPR, ..., up to UPL of them, and keeps their activation slice in registers
//     for the whole kernel, so the activation is read once per wave, never per row.
//   * 64/LPR rows are reduced side by side (one per lane group) and R such row groups per
//     wave: all R*UPL weight loads (16-byte, dword-aligned) are issued before any math so a
//     lane has R*UPL*48 bytes in flight.
//   * Integer partial sums per sub-block are exact (v_dot4_i32_i8); each lane folds its
//     units to one f32 and the row total is a butterfly over the LPR lanes.
// Each row is reduced by exactly one lane group: the result is independent of the grid, as
// matvec_any's results are independent of its row partitioning.
#include "gemv.h"

#include "gemv_dot.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {

template <int F, int LPR, int UPL, int R, bool PART>
__global__ void __launch_bounds__(256) gemv_kernel(const uint8_t* __restrict__ w, int64_t rb, int U, int64_t N,
                                                   const uint8_t* __restrict__ xq, float* __restrict__ y,
                                                   int32_t* __restrict__ part, int64_t ppr) {
  using Ut = Unit<F>;
  constexpr int G = kWave / LPR;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int g = lane / LPR, c = lane % LPR;
  const int64_t row0 = wave * (G * R);
  if (row0 >= N) return;

  typename Ut::W wt[R][UPL];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t row = row0 + r * G + g;
    const uint8_t* rp = w + (row < N ? row : 0) * rb;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      if (row < N && u < U) Ut::load_w(wt[r][t], rp, u);
    }
  }

  typename Ut::Act act[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) {
    const int u = c + LPR * t;
    if (u < U) Ut::load_act(act[t], xq, u);
  }

#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t row = row0 + r * G + g;
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      if (row < N && u < U) {
        if constexpr (PART) {
          int32_t p[Ut::kPartials];
          acc += Ut::dot(wt[r][t], act[t], p);
#pragma unroll
          for (int k = 0; k < Ut::kPartials; k++) part[row * ppr + Ut::part_index(u, k)] = p[k];
        } else {
          acc += Ut::dot(wt[r][t], act[t], nullptr);
        }
      }
    }
    acc = group_sum<LPR>(acc);
    if (c == 0 && row < N) y[row] = acc;
  }
}

namespace {

template <int F, int LPR, int UPL, int R, bool PART>
void launch_one(const uint8_t* w, int64_t rb, int U, int64_t N, const uint8_t* xq, float* y, int32_t* part,
                int64_t ppr, hipStream_t stream) {
  constexpr int G = kWave / LPR;
  int64_t waves = (N + G * R - 1) / (G * R);
  int64_t blocks = (waves + 3) / 4;
  hipLaunchKernelGGL((gemv_kernel<F, LPR, UPL, R, PART>), dim3(unsigned(blocks)), dim3(256), 0, stream, w, rb, U,
                     N, xq, y, part, ppr);
}

template <int F, int LPR, int UPL, bool PART>
void launch_r(int R, const uint8_t* w, int64_t rb, int U, int64_t N, const uint8_t* xq, float* y, int32_t* part,
              int64_t ppr, hipStream_t s) {
  if constexpr (PART) {
    launch_one<F, LPR, UPL, 1, true>(w, rb, U, N, xq, y, part, ppr, s);
  } else {
    if (R >= 4)
      launch_one<F, LPR, UPL, 4, false>(w, rb, U, N, xq, y, part, ppr, s);
    else if (R == 2)
      launch_one<F, LPR, UPL, 2, false>(w, rb, U, N, xq, y, part, ppr, s);
    else
      launch_one<F, LPR, UPL, 1, false>(w, rb, U, N, xq, y, part, ppr, s);
  }
}

template <int F, bool PART>
int launch_fmt(const uint8_t* w, int64_t k, int64_t N, const uint8_t* xq, float* y, int32_t* part,
               hipStream_t s) {
  const int64_t rb = row_bytes(F, k);
  const int U = units_per_row(F, k);
  const int64_t ppr = partials_per_row(F, k);
  int lpr = U > 32 ? 64 : U > 16 ? 32 : U > 4 ? 16 : 4;
  int upl = (U + lpr - 1) / lpr;
  int G = kWave / lpr;
  // Rows per wave: enough waves to cover ~8 per CU first, then deepen the per-lane queue.
  const int cus = device_info().cus;
  int64_t groups = (N + G - 1) / G;
  int R = groups >= int64_t(cus) * 8 * 4 ? 4 : groups >= int64_t(cus) * 8 * 2 ? 2 : 1;
  if (lpr == 4) {
    launch_r<F, 4, 1, PART>(R, w, rb, U, N, xq, y, part, ppr, s);
  } else if (lpr == 16) {
    launch_r<F, 16, 1, PART>(R, w, rb, U, N, xq, y, part, ppr, s);
  } else if (lpr == 32) {
    launch_r<F, 32, 1, PART>(R, w, rb, U, N, xq, y, part, ppr, s);
  } else {
    switch (upl) {
      case 1: launch_r<F, 64, 1, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      case 2: launch_r<F, 64, 2, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      case 3: launch_r<F, 64, 3, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      case 4: launch_r<F, 64, 4, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      case 5:
      case 6: launch_r<F, 64, 6, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      case 7:
      case 8: launch_r<F, 64, 8, PART>(R, w, rb, U, N, xq, y, part, ppr, s); break;
      default:
        return fail(JERO_ERR_CAPABILITY_MISMATCH,
                    "matvec: n_in=" + std::to_string(k) + " exceeds the register-resident activation limit (" +
                        std::to_string(64 * 8) + " units per row)");
    }
  }
  return check_launch("matvec");
}

}  // namespace

int max_gemv_k(int quant) { return 64 * 8 * ((quant == JERO_Q4_K || quant == JERO_Q6_K) ? 64 : 32); }

int check_matvec_args(int quant, const void* w, size_t w_bytes, int64_t n_in, int64_t n_out, const void* xq,
                      const float* y) {
  if (!is_weight_quant(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "unsupported weight quantization " + std::to_string(quant));
  if (!w || !xq || !y) return fail(JERO_ERR_INVALID_ARGUMENT, "matvec: null pointer");
  if (n_in <= 0 || n_out <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "matvec output and input cannot be empty");
  int64_t rb = row_bytes(quant, n_in);
  if (rb < 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "matvec: n_in=" + std::to_string(n_in) + " is not a multiple of the block");
  if (uint64_t(rb) * uint64_t(n_out) > w_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "matvec: tensor holds " + std::to_string(w_bytes) + " bytes, shape needs " +
                                            std::to_string(rb * n_out));
  if (n_in > max_gemv_k(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "matvec: n_in=" + std::to_string(n_in) + " above the supported " +
                                                  std::to_string(max_gemv_k(quant)));
  if (!aligned4(w) || !aligned4(xq) || !aligned4(y))
    return fail(JERO_ERR_INVALID_ARGUMENT, "matvec: weights, activations and output must be 4-byte aligned");
  return JERO_OK;
}

int launch_matvec(int quant, const void* w, int64_t n_in, int64_t n_out, const void* xq, float* y,
                  int32_t* part, hipStream_t s) {
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  const uint8_t* xb = static_cast<const uint8_t*>(xq);
  if (part) {
    switch (quant) {
      case JERO_Q4_K: return launch_fmt<JERO_Q4_K, true>(wb, n_in, n_out, xb, y, part, s);
      case JERO_Q6_K: return launch_fmt<JERO_Q6_K, true>(wb, n_in, n_out, xb, y, part, s);
      case JERO_Q8_0: return launch_fmt<JERO_Q8_0, true>(wb, n_in, n_out, xb, y, part, s);
      case JERO_Q4_0: return launch_fmt<JERO_Q4_0, true>(wb, n_in, n_out, xb, y, part, s);
    }
  } else {
    switch (quant) {
      case JERO_Q4_K: return launch_fmt<JERO_Q4_K, false>(wb, n_in, n_out, xb, y, nullptr, s);
      case JERO_Q6_K: return launch_fmt<JERO_Q6_K, false>(wb, n_in, n_out, xb, y, nullptr, s);
      case JERO_Q8_0: return launch_fmt<JERO_Q8_0, false>(wb, n_in, n_out, xb, y, nullptr, s);
      case JERO_Q4_0: return launch_fmt<JERO_Q4_0, false>(wb, n_in, n_out, xb, y, nullptr, s);
    }
  }
  return fail(JERO_ERR_CAPABILITY_MISMATCH, "unsupported weight quantization " + std::to_string(quant));
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_matvec(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                               const void* xq_dev, float* y_dev, void* stream) {
  int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, xq_dev, y_dev);
  if (rc) return rc;
  return launch_matvec(quant, w_dev, n_in, n_out, xq_dev, y_dev, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_matvec_partials(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                                        const void* xq_dev, float* y_dev, int32_t* partials_dev, void* stream) {
  int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, xq_dev, y_dev);
  if (rc) return rc;
  if (!partials_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "matvec_partials: null partials");
  return launch_matvec(quant, w_dev, n_in, n_out, xq_dev, y_dev, partials_dev, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_vec_dot(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                                const float* x_dev, float* y_dev, void* workspace_dev, size_t workspace_bytes,
                                void* stream) {
  int act = act_format(quant);
  int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, x_dev, y_dev);
  if (rc) return rc;
  if (reinterpret_cast<uintptr_t>(x_dev) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "vec_dot: input must be 16-byte aligned");
  size_t need = size_t(row_bytes(act, n_in));
  void* ws = workspace_dev;
  if (ws) {
    if (workspace_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "vec_dot: workspace of " + std::to_string(workspace_bytes) +
                                              " bytes, need " + std::to_string(need));
    if (!aligned4(ws)) return fail(JERO_ERR_INVALID_ARGUMENT, "vec_dot: workspace must be 4-byte aligned");
  } else {
    rc = workspace(need, &ws);
    if (rc) return rc;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = launch_quantize_act(act, x_dev, 1, n_in, ws, s);
  if (rc) return rc;
  return launch_matvec(quant, w_dev, n_in, n_out, ws, y_dev, nullptr, s);
}
