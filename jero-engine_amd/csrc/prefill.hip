// prefill.hip -- the row kernels of the batched prefill (jero_hip_model_prefill): the n prompt
// tokens go through each layer at once, as GEMMs over n activation rows, instead of
// run_prefill_with_hidden's token loop (src/qwen_deepseek.rs:2217-2316, loop :2298-2312).  Each
// kernel is the per-token arithmetic of the decode step applied to every row: the embedding row,
// RMSNorm, QK-norm and RoPE (the fused attention prologue's formulas), the K/V ring append,
// SwiGLU and the residual add.
#include "prefill.h"

#include "dequant.h"
#include "jero_common.h"
#include "runtime.h"

namespace jero {

namespace {

// X[t][i] = embed_token(tokens[t]) (a row of token_embd's `rows`, or the deterministic row);
// grid (ceil(H / 256), n).
__global__ void __launch_bounds__(256) embed_rows_kernel(int quant, const uint8_t* __restrict__ w, int64_t rb, int64_t rows,
                                                         int H, const int32_t* __restrict__ tokens,
                                                         float* __restrict__ X) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= H) return;
  X[int64_t(blockIdx.y) * H + i] = embed_value(quant, w, rb, rows, tokens[blockIdx.y], i);
}

__device__ __forceinline__ float block_sum256(float v, float* s_tmp) {
  v = wave_sum_dpp(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) s_tmp[wv] = v;
  __syncthreads();
  return s_tmp[0] + s_tmp[1] + s_tmp[2] + s_tmp[3];
}

// XN[t] = RMSNorm(X[t]) * w: x * (1 / sqrt(mean(x^2) + eps)) * w; one workgroup per row.
__global__ void __launch_bounds__(256) rmsnorm_rows_kernel(const float* __restrict__ X, int64_t H,
                                                           const float* __restrict__ w, float eps,
                                                           float* __restrict__ XN) {
  __shared__ float s_tmp[4];
  const float* x = X + int64_t(blockIdx.x) * H;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += 256) ss += x[i] * x[i];
  ss = block_sum256(ss, s_tmp);
  const float inv = 1.0f / sqrtf(ss / float(H) + eps);
  float* y = XN + int64_t(blockIdx.x) * H;
  for (int64_t i = threadIdx.x; i < H; i += 256) y[i] = x[i] * inv * w[i];
}

// One wave per token t = blockIdx.x and kRopeRowsPerWave head rows y from kRopeRowsPerWave *
// blockIdx.y on, their loads issued together: y < nq a q head, y < nq + nkv a k head (both:
// per-head RMSNorm when a norm is given, then RoPE at position pos0 + t with the decode step's
// table cos / sin of pos / theta^(2i / hd), written back in place; k also into its ring slot),
// otherwise a v head (into its ring slot).  Lane l holds pairs l and l + 64 (those below hd / 2:
// head_dim up to 256), pair i being dims (2i, 2i + 1).  Token t's table also goes to rope_cs[t][hd]
// (the trace of its step).
constexpr int kRopeRowsPerWave = 4;
constexpr int kRopePairsPerLane = 2;
template <typename KV>
__global__ void __launch_bounds__(64) qk_rope_rows_kernel(float* __restrict__ q, int64_t q_stride, float* __restrict__ k,
                                                          int64_t k_stride, const float* __restrict__ v,
                                                          int64_t v_stride, const float* __restrict__ v2, int nq,
                                                          int nkv, int hd,
                                                          const float* __restrict__ q_norm,
                                                          const float* __restrict__ k_norm, float eps, int64_t pos0,
                                                          float theta, float* __restrict__ rope_cs,
                                                          KV* __restrict__ k_ring, KV* __restrict__ v_ring,
                                                          int64_t capacity) {
  const int t = blockIdx.x, lane = threadIdx.x, ny = nq + 2 * nkv, y0 = kRopeRowsPerWave * int(blockIdx.y);
  const int64_t pos = pos0 + t;
  const int64_t slot = pos % capacity;
  const int64_t kvd = int64_t(nkv) * hd;
  constexpr int PL = kRopePairsPerLane;
  bool on[PL];
  int pr[PL];
#pragma unroll
  for (int c = 0; c < PL; c++) {
    on[c] = lane + 64 * c < hd / 2;
    pr[c] = on[c] ? lane + 64 * c : hd / 2 - 1;
  }
  // every row's loads first (rows past the last repeat it and are not used)
  float2 x[kRopeRowsPerWave][PL], g[kRopeRowsPerWave][PL], x2[kRopeRowsPerWave][PL];
#pragma unroll
  for (int j = 0; j < kRopeRowsPerWave; j++) {
    const int y = min(y0 + j, ny - 1);
    const bool isv = y >= nq + nkv;
    const float* row = y < nq ? q + t * q_stride + int64_t(y) * hd
                       : !isv ? k + t * k_stride + int64_t(y - nq) * hd
                              : v + t * v_stride + int64_t(y - nq - nkv) * hd;
    const float* nw = y < nq ? q_norm : !isv ? k_norm : nullptr;
    const float* row2 = isv && v2 ? v2 + t * v_stride + int64_t(y - nq - nkv) * hd : row;
#pragma unroll
    for (int c = 0; c < PL; c++) {
      x[j][c] = reinterpret_cast<const float2*>(row)[pr[c]];
      g[j][c] = reinterpret_cast<const float2*>(nw ? nw : row)[pr[c]];
      x2[j][c] = reinterpret_cast<const float2*>(row2)[pr[c]];
    }
  }
  float sn[PL], cn[PL];
#pragma unroll
  for (int c = 0; c < PL; c++) {
    const float expo = float(2 * pr[c]) / float(hd);
    sincosf(float(pos) / powf(theta, expo), &sn[c], &cn[c]);
    if (y0 == 0 && on[c]) {
      rope_cs[int64_t(t) * hd + 2 * pr[c]] = cn[c];
      rope_cs[int64_t(t) * hd + 2 * pr[c] + 1] = sn[c];
    }
  }
#pragma unroll
  for (int j = 0; j < kRopeRowsPerWave; j++) {
    const int y = y0 + j;
    if (y >= ny) break;  // uniform
    if (y >= nq + nkv) {  // v head: ring append only (the two halves' sum, when split)
#pragma unroll
      for (int c = 0; c < PL; c++) {
        if (!on[c]) continue;
        const float2 xv = v2 ? make_float2(x[j][c].x + x2[j][c].x, x[j][c].y + x2[j][c].y) : x[j][c];
        KV* dst = v_ring + slot * kvd + int64_t(y - nq - nkv) * hd + 2 * pr[c];
        dst[0] = KV(xv.x);
        dst[1] = KV(xv.y);
      }
      continue;
    }
    const bool isq = y < nq;
    float2 xv[PL];
#pragma unroll
    for (int c = 0; c < PL; c++) xv[c] = x[j][c];
    if (isq ? q_norm : k_norm) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < PL; c++) ss += on[c] ? xv[c].x * xv[c].x + xv[c].y * xv[c].y : 0.f;
      ss = wave_sum_dpp(ss);
      const float inv = 1.0f / sqrtf(ss / float(hd) + eps);
#pragma unroll
      for (int c = 0; c < PL; c++) {
        xv[c].x = xv[c].x * inv * g[j][c].x;
        xv[c].y = xv[c].y * inv * g[j][c].y;
      }
    }
#pragma unroll
    for (int c = 0; c < PL; c++) {
      if (!on[c]) continue;
      const float2 r = make_float2(xv[c].x * cn[c] - xv[c].y * sn[c], xv[c].x * sn[c] + xv[c].y * cn[c]);
      float* row = isq ? q + t * q_stride + int64_t(y) * hd : k + t * k_stride + int64_t(y - nq) * hd;
      reinterpret_cast<float2*>(row)[pr[c]] = r;
      if (!isq) {
        KV* dst = k_ring + slot * kvd + int64_t(y - nq) * hd + 2 * pr[c];
        dst[0] = KV(r.x);
        dst[1] = KV(r.y);
      }
    }
  }
}

// act[t][i] = silu(g[t][i]) * u[t][i] (the decode step's SwiGLU formula); grid (ceil(F / 256), n).
__global__ void __launch_bounds__(256) swiglu_rows_kernel(const float* __restrict__ g, int64_t g_stride,
                                                          const float* __restrict__ u, int64_t u_stride,
                                                          float* __restrict__ act, int64_t F) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= F) return;
  const int64_t t = blockIdx.y;
  const float gv = g[t * g_stride + i], uv = u[t * u_stride + i];
  act[t * F + i] = gv / (1.0f + expf(-gv)) * uv;
}

// The fused row step before a projection over Q8_K activations, one workgroup per row t:
// X[t] += D[t] (+ D2[t], added to D[t] first: the two K halves of a split projection) when D is
// given (the previous projection's residual, written back), XN[t] =
// RMSNorm(X[t]) * w as rmsnorm_rows_kernel computes it (the same per-thread strided sums, so the
// same bits), XN[t] also stored when XN is given, and Q[t] = the Q8_K blocks of XN[t] as
// quant_q8k_kernel makes them (a wave per 256-block from LDS).  H a multiple of 256, at most
// kFusedMaxH.
constexpr int kFusedMaxH = 8192;
__global__ void __launch_bounds__(256) add_rmsnorm_q8k_rows_kernel(float* __restrict__ X, const float* __restrict__ D,
                                                                   const float* __restrict__ D2, int64_t H,
                                                                   const float* __restrict__ w, float eps,
                                                                   float* __restrict__ XN, uint8_t* __restrict__ Q) {
  __shared__ float s_tmp[4];
  __shared__ __attribute__((aligned(16))) float s_xn[kFusedMaxH];
  float* x = X + int64_t(blockIdx.x) * H;
  const float* d = D ? D + int64_t(blockIdx.x) * H : x;
  const float* d2 = D2 ? D2 + int64_t(blockIdx.x) * H : x;
  const int per = int(H / 256);  // elements per thread: i = threadIdx.x + 256 k
  float ss = 0.f;
  // eight elements' loads in flight per batch, then the sums in the same order as the plain loop
  for (int k0 = 0; k0 < per; k0 += 8) {
    float v[8], e[8], e2[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int64_t i = threadIdx.x + 256 * int64_t(min(k0 + k, per - 1));
      v[k] = x[i];
      e[k] = d[i];
      e2[k] = d2[i];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      if (k0 + k < per) {
        const int64_t i = threadIdx.x + 256 * int64_t(k0 + k);
        float u = v[k];
        if (D) {
          u += D2 ? e[k] + e2[k] : e[k];
          x[i] = u;
        }
        s_xn[i] = u;
        ss += u * u;
      }
    }
  }
  ss = block_sum256(ss, s_tmp);
  const float inv = 1.0f / sqrtf(ss / float(H) + eps);
  float* y = XN ? XN + int64_t(blockIdx.x) * H : nullptr;
  for (int k0 = 0; k0 < per; k0 += 8) {
    float wk[8];
#pragma unroll
    for (int k = 0; k < 8; k++) wk[k] = w[threadIdx.x + 256 * int64_t(min(k0 + k, per - 1))];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      if (k0 + k < per) {
        const int64_t i = threadIdx.x + 256 * int64_t(k0 + k);
        const float u = s_xn[i] * inv * wk[k];
        s_xn[i] = u;
        if (y) y[i] = u;
      }
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint8_t* q = Q + int64_t(blockIdx.x) * (H / 256) * 292;
  for (int64_t j = wv; j < H / 256; j += 4) {
    const float4 v = reinterpret_cast<const float4*>(s_xn + 256 * j)[lane];
    const float e[4] = {v.x, v.y, v.z, v.w};
    q8k_block_wave(e, lane, q + j * 292);
  }
}

// add_rmsnorm_q8k_rows_kernel at H = 256 PER: the same element mapping, sums and products (the
// same bits), with every load of the row (X, D, D2 and the weights) issued before the first use,
// so a row costs one round trip instead of one per batch of eight.
template <int PER>
__global__ void __launch_bounds__(256) add_rmsnorm_q8k_rows_fixed_kernel(float* __restrict__ X,
                                                                         const float* __restrict__ D,
                                                                         const float* __restrict__ D2,
                                                                         const float* __restrict__ w, float eps,
                                                                         float* __restrict__ XN,
                                                                         uint8_t* __restrict__ Q) {
  constexpr int H = 256 * PER;
  __shared__ float s_tmp[4];
  __shared__ __attribute__((aligned(16))) float s_xn[H];
  float* x = X + int64_t(blockIdx.x) * H;
  const float* d = D ? D + int64_t(blockIdx.x) * H : x;
  const float* d2 = D2 ? D2 + int64_t(blockIdx.x) * H : x;
  float v[PER], e[PER], e2[PER], wk[PER];
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int i = threadIdx.x + 256 * k;
    v[k] = x[i];
    e[k] = d[i];
    e2[k] = d2[i];
    wk[k] = w[i];
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    float u = v[k];
    if (D) {
      u += D2 ? e[k] + e2[k] : e[k];
      x[threadIdx.x + 256 * k] = u;
    }
    v[k] = u;
    ss += u * u;
  }
  ss = block_sum256(ss, s_tmp);
  const float inv = 1.0f / sqrtf(ss / float(H) + eps);
  float* y = XN ? XN + int64_t(blockIdx.x) * H : nullptr;
#pragma unroll
  for (int k = 0; k < PER; k++) {
    const int i = threadIdx.x + 256 * k;
    const float u = v[k] * inv * wk[k];
    s_xn[i] = u;
    if (y) y[i] = u;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint8_t* q = Q + int64_t(blockIdx.x) * PER * 292;
  for (int j = wv; j < PER; j += 4) {
    const float4 f = reinterpret_cast<const float4*>(s_xn + 256 * j)[lane];
    const float ev[4] = {f.x, f.y, f.z, f.w};
    q8k_block_wave(ev, lane, q + j * 292);
  }
}

// act[t] = silu(g[t]) * u[t] as swiglu_rows_kernel computes it, stored when act is given, and its
// Q8_K blocks: a wave per kSwigluBlocksPerWave 256-blocks (4 elements per lane), their loads issued
// together, grid (ceil(F / (1024 kSwigluBlocksPerWave)), n).
constexpr int kSwigluBlocksPerWave = 2;
__global__ void __launch_bounds__(256) swiglu_q8k_rows_kernel(const float* __restrict__ g, int64_t g_stride,
                                                              const float* __restrict__ u, int64_t u_stride,
                                                              float* __restrict__ act, int64_t F,
                                                              uint8_t* __restrict__ Q) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t nblk = F / 256, j0 = (int64_t(blockIdx.x) * 4 + wv) * kSwigluBlocksPerWave, t = blockIdx.y;
  if (j0 >= nblk) return;
  float4 gv[kSwigluBlocksPerWave], uv[kSwigluBlocksPerWave];
#pragma unroll
  for (int b = 0; b < kSwigluBlocksPerWave; b++) {  // a block past the last repeats it, unused
    const int64_t j = min(j0 + b, nblk - 1);
    gv[b] = reinterpret_cast<const float4*>(g + t * g_stride + 256 * j)[lane];
    uv[b] = reinterpret_cast<const float4*>(u + t * u_stride + 256 * j)[lane];
  }
#pragma unroll
  for (int b = 0; b < kSwigluBlocksPerWave; b++) {
    const int64_t j = j0 + b;
    if (j >= nblk) break;  // uniform
    const float ga[4] = {gv[b].x, gv[b].y, gv[b].z, gv[b].w}, ua[4] = {uv[b].x, uv[b].y, uv[b].z, uv[b].w};
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; i++) e[i] = ga[i] / (1.0f + expf(-ga[i])) * ua[i];
    if (act) reinterpret_cast<float4*>(act + t * F + 256 * j)[lane] = make_float4(e[0], e[1], e[2], e[3]);
    q8k_block_wave(e, lane, Q + (t * nblk + j) * 292);
  }
}

// x[i] += d[i] (the residual of Wo and down).
__global__ void __launch_bounds__(256) add_rows_kernel(float* __restrict__ x, const float* __restrict__ d, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] += d[i];
}

}  // namespace

int launch_embed_rows(int quant, const void* w, int64_t rb, int64_t rows, int H, const int32_t* tokens, int64_t n,
                      float* X,
                      hipStream_t s) {
  hipLaunchKernelGGL(embed_rows_kernel, dim3(unsigned((H + 255) / 256), unsigned(n)), dim3(256), 0, s, quant,
                     static_cast<const uint8_t*>(w), rb, rows, H, tokens, X);
  return check_launch("prefill embed");
}

int launch_rmsnorm_rows(const float* X, int64_t n, int64_t H, const float* w, float eps, float* XN, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(unsigned(n)), dim3(256), 0, s, X, H, w, eps, XN);
  return check_launch("prefill rmsnorm");
}

int launch_qk_rope_rows(float* q, int64_t q_stride, float* k, int64_t k_stride, const float* v, int64_t v_stride,
                        const float* v2, int64_t n, int nq, int nkv, int hd, const float* q_norm, const float* k_norm, float eps,
                        int64_t pos0, float theta, float* rope_cs, void* k_ring, void* v_ring, bool kv_f16,
                        int64_t capacity, hipStream_t s) {
  const dim3 grid(unsigned(n), unsigned((nq + 2 * nkv + kRopeRowsPerWave - 1) / kRopeRowsPerWave));
  if (kv_f16)
    hipLaunchKernelGGL(qk_rope_rows_kernel<_Float16>, grid, dim3(64), 0, s, q, q_stride, k, k_stride, v, v_stride, v2, nq,
                       nkv, hd, q_norm, k_norm, eps, pos0, theta, rope_cs, static_cast<_Float16*>(k_ring),
                       static_cast<_Float16*>(v_ring), capacity);
  else
    hipLaunchKernelGGL(qk_rope_rows_kernel<float>, grid, dim3(64), 0, s, q, q_stride, k, k_stride, v, v_stride, v2, nq,
                       nkv, hd, q_norm, k_norm, eps, pos0, theta, rope_cs, static_cast<float*>(k_ring),
                       static_cast<float*>(v_ring), capacity);
  return check_launch("prefill qk-norm / rope");
}

int launch_swiglu_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* act, int64_t n,
                       int64_t F, hipStream_t s) {
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3(unsigned((F + 255) / 256), unsigned(n)), dim3(256), 0, s, g, g_stride,
                     u, u_stride, act, F);
  return check_launch("prefill swiglu");
}

int launch_add_rmsnorm_q8k_rows(float* X, const float* D, const float* D2, int64_t n, int64_t H, const float* w,
                                float eps, float* XN, void* Q, hipStream_t s) {
  if (H % 256 || H > kFusedMaxH) return fail(JERO_ERR_CAPABILITY_MISMATCH, "prefill: fused RMSNorm rows need H % 256 == 0, H <= 8192");
  uint8_t* q = static_cast<uint8_t*>(Q);
  const dim3 grid{unsigned(n)}, block{256u};
  switch (H / 256) {  // the hidden sizes of the Qwen3 family (and 512): one round trip per row
    case 2: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<2>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    case 4: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<4>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    case 8: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<8>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    case 10: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<10>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    case 16: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<16>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    case 20: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_fixed_kernel<20>, grid, block, 0, s, X, D, D2, w, eps, XN, q); break;
    default: hipLaunchKernelGGL(add_rmsnorm_q8k_rows_kernel, grid, block, 0, s, X, D, D2, H, w, eps, XN, q);
  }
  return check_launch("prefill rmsnorm + q8_k");
}

int launch_swiglu_q8k_rows(const float* g, int64_t g_stride, const float* u, int64_t u_stride, float* act, int64_t n,
                           int64_t F, void* Q, hipStream_t s) {
  if (F % 256 || (g_stride | u_stride) % 4)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "prefill: fused SwiGLU rows need F % 256 == 0");
  const int64_t per_wg = 4 * kSwigluBlocksPerWave;
  hipLaunchKernelGGL(swiglu_q8k_rows_kernel, dim3(unsigned((F / 256 + per_wg - 1) / per_wg), unsigned(n)), dim3(256), 0, s, g,
                     g_stride, u, u_stride, act, F, static_cast<uint8_t*>(Q));
  return check_launch("prefill swiglu + q8_k");
}

int launch_add_rows(float* x, const float* d, int64_t count, hipStream_t s) {
  hipLaunchKernelGGL(add_rows_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, s, x, d, count);
  return check_launch("prefill residual");
}

}  // namespace jero
