// gemv.hip -- decode GEMV y = W x over GGUF weight bytes on gfx950.
//
// Replaces matvec_any (src/gemma.rs:100-138) and the vec_dot_* kernels it dispatches to
// (src/gemma.rs:66-95).  Design (activation-stationary, one wave = a group of rows):
//   * A row is cut into units (gemv_dot.h).  LPR lanes share one row; lane c of the row owns
//     units c, c+LPR, ..., up to UPL of them, and keeps their activation slice in registers
//     for the whole kernel, so the activation is read once per wave, never per row.
//   * 64/LPR rows are reduced side by side (one per lane group) and R such row groups per
//     wave: all R*UPL weight loads (16-byte, dword-aligned) are issued before any math.
//   * For long rows (>= 8192 elements) the workgroup first copies the quantized activation
//     into LDS with 16-byte loads issued ahead of the weight loads, and each lane takes its
//     slice from LDS: one activation read per workgroup instead of one per wave.
//   * Integer partial sums per sub-block are exact (v_dot4_i32_i8); each lane folds its
//     units to one f32 and the row total is a DPP butterfly over the LPR lanes.
// Each row is reduced by exactly one lane group in a fixed order that depends only on n_in:
// the result is independent of the grid, as matvec_any's results are independent of its row
// partitioning.
#include "gemv.h"

#include <mutex>
#include <vector>

#include "gemv_dot.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {

constexpr int kGemvThreads = 256;

// NT: the launch reads every weight byte once (non-temporal weight loads).
template <int F, int LPR, int UPL, int R, bool PART, bool LDS_ACT, bool NT>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(const uint8_t* __restrict__ w, int64_t rb, int U,
                                                             int64_t N, const uint8_t* __restrict__ xq,
                                                             int act_bytes, float* __restrict__ y,
                                                             int32_t* __restrict__ part, int64_t ppr) {
  using Ut = Unit<F>;
  constexpr int G = kWave / LPR;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_act[];
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int g = lane / LPR, c = lane % LPR;
  const int64_t row0 = wave * (G * R);

  // 1. activation copy into registers first (its loads retire before the weight loads)
  constexpr int kMaxChunks = 10;  // 16-byte chunks per thread: up to 40 KB of activation
  u32x4 av[LDS_ACT ? kMaxChunks : 1];
  const int n16 = act_bytes >> 4;
  if constexpr (LDS_ACT) {
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) av[i] = ld4(xq + 16 * min(int(threadIdx.x) + kGemvThreads * i, n16 - 1));
  } else {
    if (row0 >= N) return;
  }

  // 2. weight loads for all rows of the wave, unconditional (row and unit clamped into the
  //    matrix, results of clamped lanes masked below): a load under a branch gets a wait of
  //    its own, and the activation's wait would become a wait for the weights as well
  typename Ut::W wt[R][UPL];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t row = min(row0 + r * G + g, N - 1);
#pragma unroll
    for (int t = 0; t < UPL; t++) load_unit<F, NT>(wt[r][t], w, rb, N, U, row, min(c + LPR * t, U - 1));
  }

  // 3. activation slice: from LDS (staged once per workgroup) or straight from global
  const uint8_t* act_src = xq;
  if constexpr (LDS_ACT) {
#pragma unroll
    for (int i = 0; i < kMaxChunks; i++) {
      const int ch = threadIdx.x + kGemvThreads * i;
      if (ch < n16) *reinterpret_cast<u32x4*>(s_act + 16 * ch) = av[i];
    }
    for (int d = 4 * n16 + threadIdx.x; d < act_bytes / 4; d += kGemvThreads)
      reinterpret_cast<uint32_t*>(s_act)[d] = reinterpret_cast<const uint32_t*>(xq)[d];
    lds_barrier();  // this wave's LDS writes only, not its weight loads
    if (row0 >= N) return;
    act_src = s_act;
  }
  typename Ut::Act act[UPL];
#pragma unroll
  for (int t = 0; t < UPL; t++) Ut::load_act(act[t], act_src, min(c + LPR * t, U - 1));

  // 4. per-row dot products, DPP reduction over the row's lanes
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int64_t row = row0 + r * G + g;
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      const bool ok = row < N && u < U;
      if constexpr (PART) {
        int32_t p[Ut::kPartials];
        const float d = Ut::dot(wt[r][t], act[t], p);
        acc += ok ? d : 0.0f;
        if (ok) {
#pragma unroll
          for (int k = 0; k < Ut::kPartials; k++) part[row * ppr + Ut::part_index(u, k)] = p[k];
        }
      } else {
        const float d = Ut::dot(wt[r][t], act[t], nullptr);
        acc += ok ? d : 0.0f;
      }
    }
    acc = group_sum_last<LPR>(acc);
    if (c == LPR - 1 && row < N) y[row] = acc;
  }
}

// Rows longer than the register-resident activation allows (no row-length limit): each wave
// reduces R rows, one per 64 lanes in turn; the workgroup stages the activation through LDS in
// chunks of whole blocks (kLongChunkBytes), every lane walks the chunk's units c, c + 64, ...
// with all R rows' loads of a step issued together, and the f32 accumulators carry across
// chunks.  Each row is reduced in an order that depends only on n_in.
constexpr int kLongChunkBytes = 32 * 1024;

template <int F, int R, bool PART>
__global__ void __launch_bounds__(kGemvThreads) gemv_long_kernel(const uint8_t* __restrict__ w, int64_t rb, int U,
                                                                  int64_t N, const uint8_t* __restrict__ xq,
                                                                  int64_t act_bytes, int act_block, int units_per_block,
                                                                  int chunk_blocks, float* __restrict__ y,
                                                                  int32_t* __restrict__ part, int64_t ppr) {
  using Ut = Unit<F>;
  __shared__ __attribute__((aligned(16))) uint8_t s_act[kLongChunkBytes];
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int64_t row0 = wave * R;
  const int64_t n_blocks = act_bytes / act_block;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.f;
  for (int64_t b0 = 0; b0 < n_blocks; b0 += chunk_blocks) {
    const int nb = int(n_blocks - b0 < chunk_blocks ? n_blocks - b0 : chunk_blocks);
    const int bytes = nb * act_block;  // a multiple of 4
    __syncthreads();                   // the previous chunk is no longer read
    for (int i = threadIdx.x; i < bytes / 4; i += kGemvThreads)
      reinterpret_cast<uint32_t*>(s_act)[i] = reinterpret_cast<const uint32_t*>(xq + b0 * act_block)[i];
    __syncthreads();
    const int u_first = int(b0) * units_per_block, u_count = nb * units_per_block;
    for (int j = lane; j < u_count; j += kWave) {
      const int u = u_first + j;
      typename Ut::W wt[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int64_t row = row0 + r < N ? row0 + r : N - 1;
        if constexpr (is_planar(F))
          Ut::load_w_planar(wt[r], w, N, U, row, u);
        else
          Ut::load_w(wt[r], w + row * rb, u);
      }
      typename Ut::Act a;
      Ut::load_act(a, s_act, j);  // chunks start on block boundaries: unit j of the chunk
#pragma unroll
      for (int r = 0; r < R; r++) {
        if constexpr (PART) {
          int32_t p[Ut::kPartials];
          acc[r] += Ut::dot(wt[r], a, p);
          if (row0 + r < N) {
#pragma unroll
            for (int k = 0; k < Ut::kPartials; k++) part[(row0 + r) * ppr + Ut::part_index(u, k)] = p[k];
          }
        } else {
          acc[r] += Ut::dot(wt[r], a, nullptr);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float v = group_sum_last<64>(acc[r]);
    if (lane == 63 && row0 + r < N) y[row0 + r] = v;
  }
}

namespace {

struct Launch {
  const uint8_t* w;
  int64_t rb;
  int U;
  int64_t N;
  const uint8_t* xq;
  int act_bytes;
  float* y;
  int32_t* part;
  int64_t ppr;
  hipStream_t s;
  bool nt;  // every weight byte read once: non-temporal loads where the format has them
};

template <int F, int LPR, int UPL, int R, bool PART, bool LDS>
void launch_one(const Launch& L) {
  constexpr int G = kWave / LPR;
  int64_t waves = (L.N + G * R - 1) / (G * R);
  int64_t blocks = (waves + kGemvThreads / kWave - 1) / (kGemvThreads / kWave);
  size_t shm = LDS ? size_t((L.act_bytes + 15) & ~15) : 0;
  if constexpr (nt_capable(F)) {
    if (L.nt) {
      hipLaunchKernelGGL((gemv_kernel<F, LPR, UPL, R, PART, LDS, true>), dim3(unsigned(blocks)), dim3(kGemvThreads),
                         shm, L.s, L.w, L.rb, L.U, L.N, L.xq, L.act_bytes, L.y, L.part, L.ppr);
      return;
    }
  }
  hipLaunchKernelGGL((gemv_kernel<F, LPR, UPL, R, PART, LDS, false>), dim3(unsigned(blocks)), dim3(kGemvThreads), shm,
                     L.s, L.w, L.rb, L.U, L.N, L.xq, L.act_bytes, L.y, L.part, L.ppr);
}

template <int F, int LPR, int UPL, bool PART, bool LDS>
void launch_r(int R, const Launch& L) {
  if constexpr (PART) {
    launch_one<F, LPR, UPL, 1, true, LDS>(L);
  } else {
    if (R >= 4)
      launch_one<F, LPR, UPL, 4, false, LDS>(L);
    else if (R == 2)
      launch_one<F, LPR, UPL, 2, false, LDS>(L);
    else
      launch_one<F, LPR, UPL, 1, false, LDS>(L);
  }
}

template <int F, int UPL, bool PART>
void launch_upl(int R, bool lds, const Launch& L) {
  if (lds)
    launch_r<F, 64, UPL, PART, true>(R, L);
  else
    launch_r<F, 64, UPL, PART, false>(R, L);
}

template <int F, bool PART>
int launch_fmt(const uint8_t* w, int64_t k, int64_t N, const uint8_t* xq, float* y, int32_t* part, hipStream_t s,
               bool once) {
  Launch L{w, row_bytes(F, k), units_per_row(F, k), N, xq, int(row_bytes(act_format(F), k)), y, part,
           partials_per_row(F, k), s, once};
  const int U = L.U;
  int lpr = U > 32 ? 64 : U > 16 ? 32 : U > 4 ? 16 : 4;
  int upl = (U + lpr - 1) / lpr;
  int G = kWave / lpr;
  // Rows per wave: measured on MI355X, two rows per wave is best up to ~12K rows of 4096
  // and four for the 150K-row output head.  Long rows (K >= 8192) of the GGUF layouts run one
  // row per wave with the activation staged in LDS; the planar layouts measured faster with
  // the same row count as short rows and the activation read straight from global
  // (12288->4096 Q4_K_R: 7.25 us against 8.08 us staged).
  const int cus = device_info().cus;
  int64_t groups = (N + G - 1) / G;
  int R = groups >= int64_t(cus) * 64 ? 4 : groups >= int64_t(cus) * 8 ? 2 : 1;
  bool lds = k >= 8192 && !is_planar(F);
  if (lds) R = 1;
  if (lpr == 4) {
    launch_r<F, 4, 1, PART, false>(R, L);
  } else if (lpr == 16) {
    launch_r<F, 16, 1, PART, false>(R, L);
  } else if (lpr == 32) {
    launch_r<F, 32, 1, PART, false>(R, L);
  } else {
    switch (upl) {
      case 1: launch_upl<F, 1, PART>(R, lds, L); break;
      case 2: launch_upl<F, 2, PART>(R, lds, L); break;
      case 3: launch_upl<F, 3, PART>(R, lds, L); break;
      case 4: launch_upl<F, 4, PART>(R, lds, L); break;
      case 5:
      case 6: launch_upl<F, 6, PART>(R, lds, L); break;
      case 7:
      case 8: launch_upl<F, 8, PART>(R, lds, L); break;
      default: {
        // rows beyond the register-resident activation: the K-looped kernel
        constexpr int act = (F == JERO_Q8_0 || F == JERO_Q4_0) ? JERO_ACT_Q8 : JERO_Q8_K;
        constexpr int ab = act == JERO_Q8_K ? 292 : 36;
        constexpr int upb = act == JERO_Q8_K ? 4 : 1;
        constexpr int RL = PART ? 1 : 2;
        const int64_t waves = (N + RL - 1) / RL;
        const int64_t blocks = (waves + kGemvThreads / kWave - 1) / (kGemvThreads / kWave);
        hipLaunchKernelGGL((gemv_long_kernel<F, RL, PART>), dim3(unsigned(blocks)), dim3(kGemvThreads), 0, s, w,
                           L.rb, U, N, xq, row_bytes(act, k), ab, upb, kLongChunkBytes / ab, y, part, L.ppr);
      }
    }
  }
  return check_launch("matvec");
}

// Regroups Q4_K blocks into the JERO_Q4_K_R row runs (one thread per block).
__global__ void __launch_bounds__(256) repack_q4k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         int64_t N, int nb) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N * nb) return;
  const int U = 4 * nb;
  const int b = int(t % nb);
  const uint8_t* s = src + t * 144;
  uint8_t* row = dst + (t / nb) * (int64_t(nb) * 144);
  for (int i = 0; i < 16; i++) row[U * 32 + b * 16 + i] = s[i];
  for (int q = 0; q < 4; q++) {
    const int u = 4 * b + q;
    for (int i = 0; i < 16; i++) {
      row[u * 16 + i] = s[16 + 32 * q + i];
      row[U * 16 + u * 16 + i] = s[32 + 32 * q + i];
    }
  }
}

// Regroups Q6_K blocks into the JERO_Q6_K_R planes (one thread per block).
__global__ void __launch_bounds__(256) repack_q6k_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         int64_t N, int nb) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N * nb) return;
  const int64_t r = t / nb;
  const int b = int(t % nb);
  const int U = 4 * nb;
  const int64_t plane = N * int64_t(U) * 16;
  const uint8_t* s = src + t * 210;
  uint8_t* lo = dst;
  uint8_t* hi = dst + plane;
  uint8_t* qh = dst + 2 * plane;
  uint8_t* sc = dst + 3 * plane;
  uint8_t* dd = sc + N * int64_t(U) * 4;
  for (int q = 0; q < 4; q++) {
    const int n = q >> 1, j = q & 1;
    const int64_t u = r * U + 4 * b + q;
    for (int i = 0; i < 16; i++) {
      lo[u * 16 + i] = s[64 * n + 16 * j + i];
      hi[u * 16 + i] = s[64 * n + 32 + 16 * j + i];
      qh[u * 16 + i] = s[128 + 32 * n + 16 * j + i];
    }
    for (int k = 0; k < 4; k++) sc[u * 4 + k] = s[192 + 8 * n + j + 2 * k];
  }
  dd[t * 2] = s[208];
  dd[t * 2 + 1] = s[209];
}

// Regroups Q4_K blocks into JERO_Q4_K_T pieces (one thread per block).
__global__ void __launch_bounds__(256) repack_q4k_tiled_kernel(const uint8_t* __restrict__ src,
                                                               uint8_t* __restrict__ dst, int64_t N, int nb) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N * nb) return;
  const int64_t r = t / nb;
  const int b = int(t % nb), c = int(r & 15);
  const uint8_t* s = src + t * 144;
  uint8_t* pc = dst + ((r >> 4) * nb + b) * 2304;
  for (int k = 0; k < 16; k++) pc[2048 + c * 16 + k] = s[k];
  for (int i = 0; i < 4; i++)
    for (int k = 0; k < 16; k++) {
      pc[((2 * i) * 16 + c) * 16 + k] = s[16 + 32 * i + k];
      pc[((2 * i + 1) * 16 + c) * 16 + k] = s[32 + 32 * i + k];
    }
}

// Regroups Q6_K blocks into JERO_Q6_K_T pieces (one thread per block).
__global__ void __launch_bounds__(256) repack_q6k_tiled_kernel(const uint8_t* __restrict__ src,
                                                               uint8_t* __restrict__ dst, int64_t N, int nb) {
  int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= N * nb) return;
  const int64_t r = t / nb;
  const int b = int(t % nb), c = int(r & 15);
  const uint8_t* s = src + t * 210;
  uint8_t* pc = dst + ((r >> 4) * nb + b) * 3360;
  for (int i = 0; i < 4; i++) {
    const int n = i >> 1, j = i & 1;
    for (int k = 0; k < 16; k++) {
      pc[((2 * i) * 16 + c) * 16 + k] = s[64 * n + 16 * j + k];
      pc[((2 * i + 1) * 16 + c) * 16 + k] = s[64 * n + 32 + 16 * j + k];
      pc[2048 + (i * 16 + c) * 16 + k] = s[128 + 32 * n + 16 * j + k];
    }
    for (int k = 0; k < 4; k++) pc[3072 + c * 16 + i * 4 + k] = s[192 + 8 * n + j + 2 * k];
  }
  pc[3328 + c * 2] = s[208];
  pc[3328 + c * 2 + 1] = s[209];
}

}  // namespace

int max_gemv_k(int quant) {
  return 64 * 8 * int(64 / units_per_row(quant, 64));  // 64 lanes x 8 units of 64 or 32 elements
}

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
  if (n_in > (int64_t(1) << 30) || n_out > (int64_t(1) << 40))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "matvec: n_in above 2^30 or n_out above 2^40");
  if (!aligned4(w) || !aligned4(xq) || !aligned4(y))
    return fail(JERO_ERR_INVALID_ARGUMENT, "matvec: weights, activations and output must be 4-byte aligned");
  if (is_planar(quant) && (reinterpret_cast<uintptr_t>(w) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "matvec: Q4_K_R / Q6_K_R planes must be 16-byte aligned");
  return JERO_OK;
}

int launch_matvec(int quant, const void* w, int64_t n_in, int64_t n_out, const void* xq, float* y, int32_t* part,
                  hipStream_t s, bool once) {
  if (is_float_weight(quant)) {
    if (part) return fail(JERO_ERR_CAPABILITY_MISMATCH, "matvec_partials: float weights have no integer partial sums");
    return launch_matvec_float(quant, w, n_in, n_out, static_cast<const float*>(xq), y, s);
  }
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  const uint8_t* xb = static_cast<const uint8_t*>(xq);
  if (part) {
    switch (quant) {
      case JERO_Q4_K: return launch_fmt<JERO_Q4_K, true>(wb, n_in, n_out, xb, y, part, s, once);
      case JERO_Q4_K_R: return launch_fmt<JERO_Q4_K_R, true>(wb, n_in, n_out, xb, y, part, s, once);
      case JERO_Q6_K: return launch_fmt<JERO_Q6_K, true>(wb, n_in, n_out, xb, y, part, s, once);
      case JERO_Q6_K_R: return launch_fmt<JERO_Q6_K_R, true>(wb, n_in, n_out, xb, y, part, s, once);
      case JERO_Q8_0: return launch_fmt<JERO_Q8_0, true>(wb, n_in, n_out, xb, y, part, s, once);
      case JERO_Q4_0: return launch_fmt<JERO_Q4_0, true>(wb, n_in, n_out, xb, y, part, s, once);
    }
  } else {
    switch (quant) {
      case JERO_Q4_K: return launch_fmt<JERO_Q4_K, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
      case JERO_Q4_K_R: return launch_fmt<JERO_Q4_K_R, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
      case JERO_Q6_K: return launch_fmt<JERO_Q6_K, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
      case JERO_Q6_K_R: return launch_fmt<JERO_Q6_K_R, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
      case JERO_Q8_0: return launch_fmt<JERO_Q8_0, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
      case JERO_Q4_0: return launch_fmt<JERO_Q4_0, false>(wb, n_in, n_out, xb, y, nullptr, s, once);
    }
  }
  return fail(JERO_ERR_CAPABILITY_MISMATCH, "unsupported weight quantization " + std::to_string(quant));
}

int launch_repack(int quant, const void* src, int64_t n_in, int64_t n_out, void* dst, int* dst_quant,
                  hipStream_t s) {
  if (quant != JERO_Q4_K && quant != JERO_Q6_K)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "repack: only Q4_K and Q6_K have a device layout (got " +
                                                  std::to_string(quant) + ")");
  int nb = int(n_in / 256);
  int64_t blocks = n_out * nb;
  const dim3 grid(unsigned((blocks + 255) / 256));
  if (quant == JERO_Q4_K)
    hipLaunchKernelGGL(repack_q4k_kernel, grid, dim3(256), 0, s, static_cast<const uint8_t*>(src),
                       static_cast<uint8_t*>(dst), n_out, nb);
  else
    hipLaunchKernelGGL(repack_q6k_kernel, grid, dim3(256), 0, s, static_cast<const uint8_t*>(src),
                       static_cast<uint8_t*>(dst), n_out, nb);
  if (dst_quant) *dst_quant = quant == JERO_Q4_K ? JERO_Q4_K_R : JERO_Q6_K_R;
  return check_launch("repack");
}

int launch_repack_experts(int quant, const void* src, int64_t n_in, int64_t n_rows, void* dst, int* dst_quant,
                          hipStream_t s) {
  if (quant != JERO_Q4_K && quant != JERO_Q6_K)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "repack_experts: only Q4_K and Q6_K have a tiled layout (got " +
                                                  std::to_string(quant) + ")");
  const int nb = int(n_in / 256);
  const int64_t blocks = n_rows * nb;
  const dim3 grid(unsigned((blocks + 255) / 256));
  if (quant == JERO_Q4_K)
    hipLaunchKernelGGL(repack_q4k_tiled_kernel, grid, dim3(256), 0, s, static_cast<const uint8_t*>(src),
                       static_cast<uint8_t*>(dst), n_rows, nb);
  else
    hipLaunchKernelGGL(repack_q6k_tiled_kernel, grid, dim3(256), 0, s, static_cast<const uint8_t*>(src),
                       static_cast<uint8_t*>(dst), n_rows, nb);
  if (dst_quant) *dst_quant = quant == JERO_Q4_K ? JERO_Q4_K_T : JERO_Q6_K_T;
  return check_launch("repack_experts");
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == JERO_F32) return launch_matvec(quant, w_dev, n_in, n_out, x_dev, y_dev, nullptr, s);  // unquantized
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
  rc = launch_quantize_act(act, x_dev, 1, n_in, ws, s);
  if (rc) return rc;
  return launch_matvec(quant, w_dev, n_in, n_out, ws, y_dev, nullptr, s);
}

// ---- the allocation-free vec_dot: activation staging in a static device array ----
// Every device holding the library holds its own copy of `scratch` until the process ends.  In
// host code the array's name is only a stand-in for it: its device address, per device, comes
// from hipGetSymbolAddress, taken once per device with that device current and kept here.
namespace {
constexpr size_t kVecDotScratchBytes = 128 * 1024;
}  // namespace
static __device__ __align__(256) uint8_t scratch[kVecDotScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device: the device address of `scratch`

int scratch_ptr(void** out) {
  int dev = 0;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (int(g_scratch_ptr.size()) <= dev) g_scratch_ptr.resize(size_t(dev) + 1, nullptr);
  if (!g_scratch_ptr[size_t(dev)]) {
    void* p = nullptr;
    rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "vec_dot_noalloc: hipGetSymbolAddress");
    if (rc) return rc;
    g_scratch_ptr[size_t(dev)] = p;
  }
  *out = g_scratch_ptr[size_t(dev)];
  return JERO_OK;
}
}  // namespace

extern "C" int jero_hip_vec_dot_noalloc(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                                        const float* x_dev, float* y_dev, void* stream) {
  const int act = act_format(quant);
  int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, x_dev, y_dev);
  if (rc) return rc;
  if (reinterpret_cast<uintptr_t>(x_dev) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "vec_dot_noalloc: input must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (act == JERO_F32) return launch_matvec(quant, w_dev, n_in, n_out, x_dev, y_dev, nullptr, s);  // no staging
  const size_t need = size_t(row_bytes(act, n_in));
  if (need > kVecDotScratchBytes)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "vec_dot_noalloc: n_in=" + std::to_string(n_in) + " needs " +
                                                  std::to_string(need) + " bytes of activation staging, above its " +
                                                  std::to_string(kVecDotScratchBytes) + "-byte static buffer");
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc) return rc;
  rc = launch_quantize_act(act, x_dev, 1, n_in, ws, s);
  if (rc) return rc;
  return launch_matvec(quant, w_dev, n_in, n_out, ws, y_dev, nullptr, s);
}

extern "C" int jero_hip_repack(int quant, const void* src_dev, size_t src_bytes, int64_t n_in, int64_t n_out,
                               void* dst_dev, int* dst_quant, void* stream) {
  if (!src_dev || !dst_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "repack: null pointer");
  if (n_in <= 0 || n_out <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "repack: empty tensor");
  int64_t rb = row_bytes(quant, n_in);
  if (rb < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "repack: n_in is not a multiple of the block");
  if (uint64_t(rb) * uint64_t(n_out) > src_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "repack: tensor holds " + std::to_string(src_bytes) + " bytes, shape needs " +
                                            std::to_string(rb * n_out));
  if (reinterpret_cast<uintptr_t>(dst_dev) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "repack: destination must be 16-byte aligned");
  const uint8_t* s0 = static_cast<const uint8_t*>(src_dev);
  const uint8_t* d0 = static_cast<const uint8_t*>(dst_dev);
  size_t n = size_t(rb) * size_t(n_out);
  if (s0 < d0 + n && d0 < s0 + n) return fail(JERO_ERR_INVALID_ARGUMENT, "repack: source and destination overlap");
  return launch_repack(quant, src_dev, n_in, n_out, dst_dev, dst_quant, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_repack_experts(int quant, const void* src_dev, size_t src_bytes, int64_t n_in,
                                       int64_t rows_per_expert, int64_t n_experts, void* dst_dev, int* dst_quant,
                                       void* stream) {
  if (!src_dev || !dst_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "repack_experts: null pointer");
  if (n_in <= 0 || rows_per_expert <= 0 || n_experts <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "repack_experts: empty tensor");
  if (rows_per_expert % 16)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "repack_experts: rows per expert must be a multiple of 16 (got " +
                                                  std::to_string(rows_per_expert) + ")");
  const int64_t rb = row_bytes(quant, n_in), n_rows = rows_per_expert * n_experts;
  if (rb < 0) return fail(JERO_ERR_TENSOR_BOUNDS, "repack_experts: n_in is not a multiple of the block");
  if (uint64_t(rb) * uint64_t(n_rows) > src_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "repack_experts: tensor holds " + std::to_string(src_bytes) +
                                            " bytes, shape needs " + std::to_string(rb * n_rows));
  if (reinterpret_cast<uintptr_t>(dst_dev) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "repack_experts: destination must be 16-byte aligned");
  const uint8_t* s0 = static_cast<const uint8_t*>(src_dev);
  const uint8_t* d0 = static_cast<const uint8_t*>(dst_dev);
  const size_t n = size_t(rb) * size_t(n_rows);
  if (s0 < d0 + n && d0 < s0 + n)
    return fail(JERO_ERR_INVALID_ARGUMENT, "repack_experts: source and destination overlap");
  return launch_repack_experts(quant, src_dev, n_in, n_rows, dst_dev, dst_quant, static_cast<hipStream_t>(stream));
}
