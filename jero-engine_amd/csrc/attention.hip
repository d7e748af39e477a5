// attention.hip -- GQA softmax attention of one decode token over the KV ring, gfx950.
//
// Replaces gqa_causal_attention_f32 (called at src/qwen_deepseek.rs:669-691) and, in its
// fused form, the rest of run_gqa_causal_with_cache_scaled (src/qwen_deepseek.rs:643-694) plus
// the QK-norm and RoPE of run_dense_attention_sublayer_scaled (:1039-1071).
//
// KV layout (the recipes' flat ring, src/qwen_deepseek.rs:643-694): per layer a K ring then a
// V ring, each [capacity][n_kv * head_dim], f32 (as the reference) or f16 (half the bytes).
//
// Split-K ("flash decoding"): workgroup (split s, kv head h) owns positions
// [s*64, s*64+64) of the active slots and all q heads of h's group.  It issues its K and V
// loads (16 bytes per lane, consecutive lanes on consecutive bytes) before anything else, so
// a workgroup has its whole 2 x 128 x head_dim tile in flight; then it scores, exponentiates
// against its local max and accumulates P V.  A second kernel merges the splits with the
// usual max/sum rescaling.  Fused mode: every workgroup rebuilds its q heads (per-head RMSNorm,
// interleaved RoPE, scale folded in); the workgroup whose range holds the new slot also
// normalises/rotates k, writes k and v into the ring and uses them for that slot.
#include "attention.h"

#include "jero_common.h"
#include "runtime.h"

namespace jero {

constexpr int kAttnThreads = 256;
// Positions per workgroup (64 measured fastest at 4096 positions, head_dim 128: 32 and 128
// were 17 % slower).  The 16-byte K/V tiling needs at least 64 positions at head_dim 32.
__host__ __device__ constexpr int attn_chunk(int /*hd*/) { return 64; }
constexpr int kMaxGroup = 8;    // q heads per kv head

template <typename T>
__device__ __forceinline__ void widen16(const u32x4 v, float* out);
template <>
__device__ __forceinline__ void widen16<_Float16>(const u32x4 v, float* out) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    out[2 * i] = float(__builtin_bit_cast(_Float16, uint16_t(w[i] & 0xFFFFu)));
    out[2 * i + 1] = float(__builtin_bit_cast(_Float16, uint16_t(w[i] >> 16)));
  }
}
template <>
__device__ __forceinline__ void widen16<float>(const u32x4 v, float* out) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) out[i] = __uint_as_float(w[i]);
}

template <typename T>
__device__ __forceinline__ T narrow(float x) {
  return T(x);
}

// RoPE angle of pair i at position pos: pos / theta^(2i/hd), in f32 as the reference computes it.
__device__ __forceinline__ float rope_angle(int i, int hd, int64_t pos, float theta) {
  float expo = float(2 * i) / float(hd);
  return float(pos) / powf(theta, expo);
}

// Per-head RMSNorm (weight pair nw, if has_norm) + interleaved RoPE of one head held as one
// pair per lane in a group of HD/2 lanes; cs = (cos, sin) of the pair's angle.
template <int HD>
__device__ __forceinline__ float2 norm_rope_pair(float x0, float x1, bool has_norm, float2 nw, float eps, float2 cs) {
  if (has_norm) {
    float ss = x0 * x0 + x1 * x1;
#pragma unroll
    for (int off = HD / 4; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    float inv = 1.0f / sqrtf(ss / float(HD) + eps);
    x0 = x0 * inv * nw.x;
    x1 = x1 * inv * nw.y;
  }
  return make_float2(x0 * cs.x - x1 * cs.y, x0 * cs.y + x1 * cs.x);
}

template <int HD, typename KV, bool FUSED, int MAXG>
__global__ void __launch_bounds__(kAttnThreads) attn_partial_kernel(AttnParams p) {
  constexpr int EPL = 16 / int(sizeof(KV));     // elements per 16-byte load
  constexpr int LPP = HD / EPL;                 // lanes per position (K rows)
  constexpr int PPW = kWave / LPP;              // positions per wave per step
  constexpr int CH = attn_chunk(HD);
  constexpr int KSTEPS = CH / (PPW * (kAttnThreads / kWave));
  constexpr int DPT = HD / EPL;                 // dim chunks per V row
  constexpr int NPS = kAttnThreads / DPT;       // position subsets in the PV phase
  constexpr int VSTEPS = CH / NPS;
  static_assert(KSTEPS >= 1 && VSTEPS >= 1, "tile shape");

  __shared__ float s_q[MAXG][HD];
  __shared__ float s_knew[HD];
  __shared__ float s_vnew[HD];
  __shared__ float s_p[MAXG][CH];
  __shared__ float s_red[kAttnThreads / kWave][MAXG * HD];
  __shared__ float s_m[MAXG], s_l[MAXG];

  const int split = blockIdx.x, kh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int group = p.group;
  const int64_t kvd = int64_t(p.nkv) * HD;
  const int S = gridDim.x;
  const int p0 = split * CH;

  // 0. this thread's q pairs (fused: also the new k), issued first so that waiting for them
  //    does not wait for the K/V tile behind them
  constexpr int HPW = 128 / HD;                         // heads per wave pass (HD/2 lanes per head)
  constexpr int HPP = (kAttnThreads / kWave) * HPW;     // heads per pass of the workgroup
  constexpr int NPASS = (MAXG + (FUSED ? 1 : 0) + HPP - 1) / HPP;
  const int pair = lane % (HD / 2), sub = lane / (HD / 2);
  float2 qx[NPASS];
  // Loads are unconditional, from clamped in-bounds addresses: a load under a branch gets its
  // own wait for completion, which would serialise the tile's round trips.
#pragma unroll
  for (int it = 0; it < NPASS; it++) {
    const int gi = wv * HPW + it * HPP + sub;
    const bool is_k = FUSED && gi == group;
    const float* src = is_k ? p.k_new + kh * HD : p.q + (int64_t(kh) * group + (gi < group ? gi : 0)) * HD;
    const float2 v = *reinterpret_cast<const float2*>(src + 2 * pair);
    qx[it] = (gi < group || is_k) ? v : make_float2(0.f, 0.f);
  }

  // Fused mode: the rest of what the prologue reads (position, RoPE table, norm weights, the
  // new v) goes out in the same batch.  A null pointer reads a valid stand-in (the q vector)
  // whose value is then ignored.
  const float* dummy = p.q;
  float2 cs_pre = make_float2(1.f, 0.f), qn_pre = cs_pre, kn_pre = cs_pre;
  float vnew_pre = 0.f;
  int64_t pos_pre = p.pos;
  if constexpr (FUSED) {
    pos_pre = *(p.pos_dev ? p.pos_dev : reinterpret_cast<const int64_t*>(p.k));
    cs_pre = *reinterpret_cast<const float2*>((p.rope_cs ? p.rope_cs : dummy) + 2 * pair);
    qn_pre = *reinterpret_cast<const float2*>((p.q_norm ? p.q_norm : dummy) + 2 * pair);
    kn_pre = *reinterpret_cast<const float2*>((p.k_norm ? p.k_norm : dummy) + 2 * pair);
    vnew_pre = p.v_new[kh * HD + tid % HD];
  }

  // 1. K and V tiles into registers.  With the position on the device the grid covers every
  //    ring slot, so slots [p0, p0 + 64) are inside the ring whatever the position; slots past
  //    the active range are loaded and then ignored.
  const int bound = p.pos_dev ? int(p.capacity) : p.active;
  const int pl = min(p0 + CH, bound);
  const KV* kb = static_cast<const KV*>(p.k) + kh * HD;
  const KV* vb = static_cast<const KV*>(p.v) + kh * HD;
  u32x4 kreg[KSTEPS], vreg[VSTEPS];
  const int kc = lane % LPP;
#pragma unroll
  for (int i = 0; i < KSTEPS; i++) {
    const int pos = min(p0 + (i * (kAttnThreads / kWave) + wv) * PPW + lane / LPP, pl - 1);
    kreg[i] = ld4(reinterpret_cast<const uint8_t*>(kb + int64_t(pos) * kvd + kc * EPL));
  }
  const int dc = tid % DPT, ps = tid / DPT;
#pragma unroll
  for (int i = 0; i < VSTEPS; i++) {
    const int pos = min(p0 + i * NPS + ps, pl - 1);
    vreg[i] = ld4(reinterpret_cast<const uint8_t*>(vb + int64_t(pos) * kvd + dc * EPL));
  }

  int active = p.active, slot = p.slot;
  int64_t pos_now = p.pos;
  if (p.pos_dev) {  // position kept on the device (graph-replayed decode)
    pos_now = pos_pre;
    slot = int(pos_now % p.capacity);
    active = int(pos_now + 1 < p.capacity ? pos_now + 1 : p.capacity);
  }
  if (p0 >= active) {  // empty split: contributes nothing to the merge
    if (tid < group) {
      const int h = kh * group + tid;
      p.part_ml[(int64_t(h) * S + split) * 2 + 0] = -INFINITY;
      p.part_ml[(int64_t(h) * S + split) * 2 + 1] = 0.f;
    }
    return;
  }
  const int p1 = min(p0 + CH, active);

  // 2. q heads of this group (and, fused, the new k/v) into LDS
  const bool own_slot = FUSED && slot >= p0 && slot < p1;
  {
    float2 cs = cs_pre;
    if (FUSED && !p.rope_cs) sincosf(rope_angle(pair, HD, pos_now, p.theta), &cs.y, &cs.x);
#pragma unroll
    for (int it = 0; it < NPASS; it++) {
      const int gi = wv * HPW + it * HPP + sub;
      const bool is_k = FUSED && gi == group;
      const bool ok = gi < group || is_k;
      float2 r;
      if constexpr (FUSED)
        r = norm_rope_pair<HD>(qx[it].x, qx[it].y, (is_k ? p.k_norm : p.q_norm) != nullptr, is_k ? kn_pre : qn_pre,
                               p.eps, cs);
      else
        r = qx[it];
      if (ok) {
        if (is_k) {
          s_knew[2 * pair] = r.x;
          s_knew[2 * pair + 1] = r.y;
        } else {
          s_q[gi][2 * pair] = r.x * p.scale;
          s_q[gi][2 * pair + 1] = r.y * p.scale;
        }
      }
    }
    if (own_slot && tid < HD) s_vnew[tid] = vnew_pre;
  }
  __syncthreads();
  if (own_slot) {  // append the new token's k, v to the ring
    KV* kw = static_cast<KV*>(p.k_write) + int64_t(slot) * kvd + kh * HD;
    KV* vw = static_cast<KV*>(p.v_write) + int64_t(slot) * kvd + kh * HD;
    for (int d = tid; d < HD; d += kAttnThreads) {
      kw[d] = narrow<KV>(s_knew[d]);
      vw[d] = narrow<KV>(s_vnew[d]);
    }
  }

  // 3. scores: 16-byte K slices against every q head of the group, reduced over LPP lanes
#pragma unroll
  for (int i = 0; i < KSTEPS; i++) {
    const int pos = p0 + (i * (kAttnThreads / kWave) + wv) * PPW + lane / LPP;
    float kf[EPL];
    if (pos < p1) {
      if (FUSED && pos == slot) {
#pragma unroll
        for (int e = 0; e < EPL; e++) kf[e] = s_knew[kc * EPL + e];
      } else {
        widen16<KV>(kreg[i], kf);
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPL; e++) kf[e] = 0.f;
    }
#pragma unroll
    for (int gi = 0; gi < MAXG; gi++) {
      if (gi < group) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) s += s_q[gi][kc * EPL + e] * kf[e];
        if constexpr (LPP <= 16) {
          s = group_sum_all<LPP>(s);  // DPP within a row of 16 lanes
          if (kc == 0 && pos < p1) s_p[gi][pos - p0] = s;
        } else {
          s = group_sum_last<LPP>(s);
          if (kc == LPP - 1 && pos < p1) s_p[gi][pos - p0] = s;
        }
      }
    }
  }
  __syncthreads();

  // 4. local softmax numerators per head (one wave per head)
  const int n = p1 - p0;
  for (int gi = wv; gi < group; gi += kAttnThreads / kWave) {
    float m = -INFINITY;
    for (int j = lane; j < n; j += kWave) m = fmaxf(m, s_p[gi][j]);
    m = wave_max_dpp(m);
    float l = 0.f;
    for (int j = lane; j < n; j += kWave) {
      float e = expf(s_p[gi][j] - m);
      s_p[gi][j] = e;
      l += e;
    }
    l = wave_sum_dpp(l);
    if (lane == 0) {
      s_m[gi] = m;
      s_l[gi] = l;
    }
  }
  __syncthreads();

  // 5. P V over this thread's position subset, then across subsets
  float acc[MAXG][EPL];
#pragma unroll
  for (int gi = 0; gi < MAXG; gi++)
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[gi][e] = 0.f;
#pragma unroll
  for (int i = 0; i < VSTEPS; i++) {
    const int pos = p0 + i * NPS + ps;
    if (pos < p1) {
      float vf[EPL];
      if (FUSED && pos == slot) {
#pragma unroll
        for (int e = 0; e < EPL; e++) vf[e] = s_vnew[dc * EPL + e];
      } else {
        widen16<KV>(vreg[i], vf);
      }
#pragma unroll
      for (int gi = 0; gi < MAXG; gi++) {
        if (gi < group) {
          const float pr = s_p[gi][pos - p0];
#pragma unroll
          for (int e = 0; e < EPL; e++) acc[gi][e] += pr * vf[e];
        }
      }
    }
  }
  // subsets of one wave sit DPT lanes apart
#pragma unroll
  for (int gi = 0; gi < MAXG; gi++) {
    if (gi < group) {
#pragma unroll
      for (int e = 0; e < EPL; e++) {
        float v = acc[gi][e];
#pragma unroll
        for (int off = DPT; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
        acc[gi][e] = v;
      }
    }
  }
  if (lane < DPT) {
#pragma unroll
    for (int gi = 0; gi < MAXG; gi++)
      if (gi < group)
#pragma unroll
        for (int e = 0; e < EPL; e++) s_red[wv][gi * HD + dc * EPL + e] = acc[gi][e];
  }
  __syncthreads();
  for (int idx = tid; idx < group * HD; idx += kAttnThreads) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnThreads / kWave; w++) v += s_red[w][idx];
    const int gi = idx / HD, d = idx % HD;
    const int h = kh * group + gi;
    p.part_o[(int64_t(h) * S + split) * HD + d] = v;
  }
  if (tid < group) {
    const int h = kh * group + tid;
    p.part_ml[(int64_t(h) * S + split) * 2 + 0] = s_m[tid];
    p.part_ml[(int64_t(h) * S + split) * 2 + 1] = s_l[tid];
  }
}

// Merge of the splits: one workgroup per q head.  Thread (q, g) owns float4 column q of the
// head and splits s = g (mod SG).  Its first CH partial rows are loaded at entry, before the
// split weights w_s = exp(m_s - M) are known, so the whole merge costs one round trip to the
// partials for up to SG * CH splits.  Empty splits (l = 0) never wrote their rows: their
// weight is 0 and the select keeps whatever those rows hold out of the sum.
constexpr int kMaxSplits = 2048;

template <int HD>
__global__ void __launch_bounds__(256) attn_combine_kernel(const float* __restrict__ part_o,
                                                           const float* __restrict__ part_ml, int S,
                                                           float* __restrict__ out) {
  constexpr int Q = HD / 4;    // float4 columns of a row
  constexpr int SG = 256 / Q;  // split groups
  constexpr int CH = 8;        // rows per thread per pass
  __shared__ float s_w[kMaxSplits];
  __shared__ float4 s_red[256];
  __shared__ float s_ml[8];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int q = tid % Q, g = tid / Q;
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + int64_t(h) * S;
  const float4* po = reinterpret_cast<const float4*>(part_o + int64_t(h) * S * HD) + q;
  // every load below is unconditional (clamped to split S - 1): a load under a branch would
  // wait for its own completion and serialise the round trips
  float4 ov[CH];
#pragma unroll
  for (int i = 0; i < CH; i++) ov[i] = po[int64_t(min(g + SG * i, S - 1)) * Q];
  constexpr int MLPT = kMaxSplits / 256;
  float2 e[MLPT];
#pragma unroll
  for (int i = 0; i < MLPT; i++) e[i] = ml[min(tid + 256 * i, S - 1)];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < MLPT; i++)
    if (tid + 256 * i < S && e[i].y > 0.f) m = fmaxf(m, e[i].x);
  m = wave_max_dpp(m);
  if (lane == 0) s_ml[wv] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_ml[0], s_ml[1]), fmaxf(s_ml[2], s_ml[3]));
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < MLPT; i++) {
    const int s = tid + 256 * i;
    const float w = (s < S && e[i].y > 0.f) ? expf(e[i].x - M) : 0.f;
    if (s < S) s_w[s] = w;
    l += w * e[i].y;
  }
  l = wave_sum_dpp(l);
  if (lane == 0) s_ml[4 + wv] = l;
  __syncthreads();
  const float L = s_ml[4] + s_ml[5] + s_ml[6] + s_ml[7];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int base = 0;;) {
#pragma unroll
    for (int i = 0; i < CH; i++) {
      const int s = base + g + SG * i;
      const float w = s < S ? s_w[s] : 0.f;
      const bool on = w != 0.f;
      acc.x += on ? w * ov[i].x : 0.f;
      acc.y += on ? w * ov[i].y : 0.f;
      acc.z += on ? w * ov[i].z : 0.f;
      acc.w += on ? w * ov[i].w : 0.f;
    }
    base += SG * CH;
    if (base >= S) break;
#pragma unroll
    for (int i = 0; i < CH; i++) ov[i] = po[int64_t(min(base + g + SG * i, S - 1)) * Q];
  }
  s_red[tid] = acc;
  __syncthreads();
  if (tid < Q) {
    float4 o = s_red[tid];
#pragma unroll
    for (int j = 1; j < SG; j++) {
      const float4 r = s_red[j * Q + tid];
      o.x += r.x;
      o.y += r.y;
      o.z += r.z;
      o.w += r.w;
    }
    const float inv = 1.0f / L;
    float* oh = out + int64_t(h) * HD + 4 * tid;
    oh[0] = o.x * inv;
    oh[1] = o.y * inv;
    oh[2] = o.z * inv;
    oh[3] = o.w * inv;
  }
}

int attn_splits(int active, int hd) { return (active + attn_chunk(hd) - 1) / attn_chunk(hd); }

size_t attn_workspace_bytes(int nq, int hd, int active) {
  const size_t S = size_t(attn_splits(active, hd));
  return size_t(nq) * S * (size_t(hd) + 2) * sizeof(float);
}

template <int HD, typename KV, bool FUSED>
static void launch_partial(const AttnParams& p, int S, hipStream_t s) {
  if (p.group <= 1)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 1>), dim3(S, p.nkv), dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 2)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 2>), dim3(S, p.nkv), dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 4)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 4>), dim3(S, p.nkv), dim3(kAttnThreads), 0, s, p);
  else
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 8>), dim3(S, p.nkv), dim3(kAttnThreads), 0, s, p);
}

template <int HD>
static void launch_combine(const AttnParams& p, int S, float* out, hipStream_t s) {
  const int nq = p.nkv * p.group;
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(nq), dim3(256), 0, s, p.part_o, p.part_ml, S, out);
}

int launch_attention(const AttnParams& p0, bool fused, float* out, hipStream_t s) {
  AttnParams p = p0;
  const int S = attn_splits(p.pos_dev ? int(p.capacity) : p.active, p.hd);
  p.part_ml = p.part_o + size_t(p.nkv) * p.group * S * p.hd;
#define JERO_ATTN_CASE(HDV)                                                                     \
  if (p.hd == HDV) {                                                                            \
    if (p.kv_dtype == JERO_KV_F16) {                                                            \
      if (fused) launch_partial<HDV, _Float16, true>(p, S, s);                                  \
      else launch_partial<HDV, _Float16, false>(p, S, s);                                       \
    } else {                                                                                    \
      if (fused) launch_partial<HDV, float, true>(p, S, s);                                     \
      else launch_partial<HDV, float, false>(p, S, s);                                          \
    }                                                                                           \
  }
  JERO_ATTN_CASE(32) else JERO_ATTN_CASE(64) else JERO_ATTN_CASE(128) else return fail(
      JERO_ERR_CAPABILITY_MISMATCH, "attention: head_dim " + std::to_string(p.hd) + " not in {32, 64, 128}");
#undef JERO_ATTN_CASE
  int rc = check_launch("attention partial");
  if (rc) return rc;
  if (p.hd == 32) launch_combine<32>(p, S, out, s);
  else if (p.hd == 64) launch_combine<64>(p, S, out, s);
  else launch_combine<128>(p, S, out, s);
  return check_launch("attention combine");
}

int check_attention_shape(int nq, int nkv, int hd, int64_t seq_len) {
  if (nq <= 0 || nkv <= 0 || hd <= 0 || seq_len <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "attention: empty heads or sequence");
  if (nq % nkv) return fail(JERO_ERR_TENSOR_BOUNDS, "attention: n_heads_q not a multiple of n_heads_kv");
  if (nq / nkv > kMaxGroup)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: more than " + std::to_string(kMaxGroup) +
                                                  " q heads per kv head");
  if (hd != 32 && hd != 64 && hd != 128)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: head_dim " + std::to_string(hd) + " not in {32, 64, 128}");
  if (seq_len > int64_t(kMaxSplits) * attn_chunk(hd))
    return fail(JERO_ERR_CONTEXT_LENGTH_EXCEEDED, "attention: more than " +
                                                      std::to_string(int64_t(kMaxSplits) * attn_chunk(hd)) + " positions");
  return JERO_OK;
}

}  // namespace jero

using namespace jero;

extern "C" int jero_hip_gqa_attention(float* out_dev, const float* q_dev, const void* k_dev, const void* v_dev,
                                      int kv_dtype, int n_heads_q, int n_heads_kv, int head_dim, int64_t seq_len,
                                      float scale, void* workspace_dev, size_t workspace_bytes, void* stream) {
  int rc = check_attention_shape(n_heads_q, n_heads_kv, head_dim, seq_len);
  if (rc) return rc;
  if (!out_dev || !q_dev || !k_dev || !v_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "attention: null pointer");
  if (kv_dtype != JERO_KV_F32 && kv_dtype != JERO_KV_F16)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: kv_dtype must be JERO_KV_F32 or JERO_KV_F16");
  if ((reinterpret_cast<uintptr_t>(k_dev) | reinterpret_cast<uintptr_t>(v_dev)) & 15u)
    return fail(JERO_ERR_INVALID_ARGUMENT, "attention: K and V must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(q_dev) & 7u) return fail(JERO_ERR_INVALID_ARGUMENT, "attention: q must be 8-byte aligned");
  size_t need = attn_workspace_bytes(n_heads_q, head_dim, int(seq_len));
  void* ws = workspace_dev;
  if (ws) {
    if (workspace_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "attention: workspace of " + std::to_string(workspace_bytes) +
                                              " bytes, need " + std::to_string(need));
    if (reinterpret_cast<uintptr_t>(ws) & 15u)
      return fail(JERO_ERR_INVALID_ARGUMENT, "attention: workspace must be 16-byte aligned");
  } else {
    rc = workspace(need, &ws);
    if (rc) return rc;
  }
  AttnParams p{};
  p.q = q_dev;
  p.k = k_dev;
  p.v = v_dev;
  p.kv_dtype = kv_dtype;
  p.nkv = n_heads_kv;
  p.group = n_heads_q / n_heads_kv;
  p.hd = head_dim;
  p.active = int(seq_len);
  p.scale = scale;
  p.slot = -1;
  p.part_o = static_cast<float*>(ws);
  return launch_attention(p, false, out_dev, static_cast<hipStream_t>(stream));
}
