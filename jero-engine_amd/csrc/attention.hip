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
// [s*64, s*64+64) of the active slots and all q heads of h's group, each of its four waves 16
// of them.  A wave issues all its loads first (its 2 x 16 x head_dim K/V rows, 16 bytes per
// lane), then scores, exponentiates against its own max and accumulates P V with DPP
// reductions only; one barrier merges the four waves.  A second kernel merges the splits with
// the usual max/sum rescaling.  Fused mode: every wave rebuilds its q heads (per-head RMSNorm,
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
constexpr int kFlashThreads = 512;  // the prefill's flash kernel: 8 waves

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

// exp(x) for the softmax and the split merges (x <= 0): 2^(x log2 e) with the hardware v_exp_f32,
// two instructions against ~12 for the range-reduced expf.  Relative error about |x| * 6e-8
// (the rounding of x log2 e) plus one ulp; arguments below -87 flush to 0, which the softmax
// would not distinguish anyway.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// Sum over aligned groups of W consecutive lanes (W a power of two up to 32); every lane of a
// group gets the total.  DPP within a row of 16 lanes, one swizzle across rows for W = 32.
template <int W>
__device__ __forceinline__ float lanes_sum(float v) {
  if constexpr (W >= 2) v = dpp_add<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v = dpp_add<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v = dpp_add<0x141, 0xF>(v);   // row_half_mirror
  if constexpr (W >= 16) v = dpp_add<0x140, 0xF>(v);  // row_mirror
  if constexpr (W >= 32) v += __shfl_xor(v, 16, kWave);
  return v;
}

// Per-head RMSNorm (weights nw, if has_norm) + interleaved RoPE of one head held as E
// consecutive elements per lane in a group of HD/E lanes; cs[j] = (cos, sin) of pair j.
template <int HD, int E>
__device__ __forceinline__ void norm_rope_chunk(float (&x)[E], bool has_norm, const float (&nw)[E], float eps,
                                                const float2 (&cs)[E / 2]) {
  if (has_norm) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; e++) ss += x[e] * x[e];
    ss = lanes_sum<HD / E>(ss);
    const float inv = 1.0f / sqrtf(ss / float(HD) + eps);
#pragma unroll
    for (int e = 0; e < E; e++) x[e] = x[e] * inv * nw[e];
  }
#pragma unroll
  for (int j = 0; j < E / 2; j++) {
    const float x0 = x[2 * j], x1 = x[2 * j + 1];
    x[2 * j] = x0 * cs[j].x - x1 * cs[j].y;
    x[2 * j + 1] = x0 * cs[j].y + x1 * cs[j].x;
  }
}

// n floats at an 8-byte aligned address (n even), as float2 loads.
template <int N>
__device__ __forceinline__ void ld_floats(float (&dst)[N], const float* __restrict__ src) {
#pragma unroll
  for (int j = 0; j < N / 2; j++) {
    const float2 v = reinterpret_cast<const float2*>(src)[j];
    dst[2 * j] = v.x;
    dst[2 * j + 1] = v.y;
  }
}

// Split-K partial of one decode token's attention.  Workgroup (split s, kv head h) owns the
// 64 slots [64 s, 64 s + 64) and every q head of h's group; each of its four waves treats 16 of
// those slots as a sub-split of its own and the workgroup merges the four at the end.
//   * All global loads go out first, unconditionally (clamped in-bounds addresses): the q
//     heads, the fused-mode extras and the wave's K and V rows, 16 bytes per lane.
//   * K layout: lane = (position kp, chunk kc); each position's CPR chunk lanes hold the q heads'
//     matching chunks, so scores are a DPP sum over CPR consecutive lanes.  In fused mode each q
//     head is normalised and rotated once per workgroup, by one wave in the same layout (the head's sum
//     of squares is the same DPP sum), and shared through LDS; that barrier waits for LDS only,
//     so the K/V rows stay in flight.
//   * The wave's softmax (max, exp, sum over its 16 positions) reduces across the position
//     groups only: a position's score is already in all of its chunk lanes.
//   * V layout: lane = (chunk vc, position vp) with the PPL positions of a load in consecutive
//     lanes, so P V sums over positions with DPP as well; the numerators move from the K
//     layout to the V layout through the wave's own LDS rows (no barrier).
//   * The four sub-splits merge with the usual max rescaling through LDS, one barrier.
template <int HD, typename KV, bool FUSED, int MAXG>
__global__ void __launch_bounds__(kAttnThreads) attn_partial_kernel(AttnParams p) {
  {  // token of a batch of queries (zero offsets for one query)
    const int t = blockIdx.z;
    p.q += t * p.q_stride;
    p.active += t;
    p.part_o += t * p.part_tok;
    p.part_ml += t * p.part_tok_ml;
  }
  constexpr int EPL = 16 / int(sizeof(KV));  // KV elements per 16-byte load
  constexpr int CPR = HD / EPL;              // 16-byte chunks per K/V row
  constexpr int PPL = kWave / CPR;           // positions per wave-wide load
  constexpr int NW = kAttnThreads / kWave;   // waves = sub-splits
  constexpr int CH = attn_chunk(HD);         // positions per workgroup
  constexpr int WPOS = CH / NW;              // positions per wave
  constexpr int NL = WPOS / PPL;             // K loads and V loads per lane
  constexpr int G4 = (MAXG + 3) / 4;         // float4s per position row of numerators
  static_assert(NL >= 1 && NL * PPL == WPOS && CPR <= 32, "tile shape");

  __shared__ float s_q[MAXG][HD];
  __shared__ float4 s_p[NW][WPOS][G4];
  __shared__ float s_o[NW][MAXG][HD];
  __shared__ float s_m[NW][MAXG], s_l[NW][MAXG];

  const int split = blockIdx.x, kh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int group = p.group;
  const int64_t kvd = int64_t(p.nkv) * HD;
  const int S = gridDim.x;
  const int p0 = split * CH;
  const int w0 = p0 + wv * WPOS;
  const int kc = lane % CPR, kp = lane / CPR;
  const int vp = lane % PPL, vc = lane / PPL;

  // 0. loads.  Fused: wave w prepares q heads w, w + NW, ... and the workgroup shares them
  //    through LDS; otherwise every wave loads all of its q heads (only the scale to apply).
  constexpr int HPW = FUSED ? (MAXG + NW - 1) / NW : MAXG;
  float qw[HPW][EPL];
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int h = FUSED ? wv + NW * j : j;
    ld_floats<EPL>(qw[j], p.q + (int64_t(kh) * group + min(h, group - 1)) * HD + kc * EPL);
  }
  int64_t pos_pre = p.pos;
  float kn[EPL], vn[EPL], qnw[EPL], knw[EPL], csr[EPL];
  if constexpr (FUSED) {
    // a null pointer reads a valid stand-in (the q vector) whose value is then ignored
    pos_pre = *(p.pos_dev ? p.pos_dev : reinterpret_cast<const int64_t*>(p.k));
    ld_floats<EPL>(kn, p.k_new + kh * HD + kc * EPL);
    ld_floats<EPL>(vn, p.v_new + kh * HD + vc * EPL);
    ld_floats<EPL>(qnw, (p.q_norm ? p.q_norm : p.q) + kc * EPL);
    ld_floats<EPL>(knw, (p.k_norm ? p.k_norm : p.q) + kc * EPL);
    ld_floats<EPL>(csr, (p.rope_cs ? p.rope_cs : p.q) + kc * EPL);
  }
  // With the position on the device the grid covers every ring slot, so slots [p0, p0 + 64)
  // are inside the ring whatever the position; slots past the active range are loaded and
  // then ignored.
  const int bound = p.pos_dev ? int(p.capacity) : p.active;
  const int pl = min(p0 + CH, bound);
  const KV* kb = static_cast<const KV*>(p.k) + kh * HD;
  const KV* vb = static_cast<const KV*>(p.v) + kh * HD;
  u32x4 kreg[NL], vreg[NL];
#pragma unroll
  for (int i = 0; i < NL; i++)
    kreg[i] = ld4(reinterpret_cast<const uint8_t*>(kb + int64_t(min(w0 + i * PPL + kp, pl - 1)) * kvd + kc * EPL));
#pragma unroll
  for (int i = 0; i < NL; i++)
    vreg[i] = ld4(reinterpret_cast<const uint8_t*>(vb + int64_t(min(w0 + i * PPL + vp, pl - 1)) * kvd + vc * EPL));

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

  // 1. q heads (fused: QK-norm and RoPE, also of the new k in the workgroup that holds its
  //    slot), scale folded into q; each head is prepared by one wave and shared through LDS
  if constexpr (FUSED) {
    float2 cs[EPL / 2];
#pragma unroll
    for (int j = 0; j < EPL / 2; j++) {
      if (p.rope_cs) {
        cs[j] = make_float2(csr[2 * j], csr[2 * j + 1]);
      } else {
        float sn, cn;
        sincosf(rope_angle(kc * (EPL / 2) + j, HD, pos_now, p.theta), &sn, &cn);
        cs[j] = make_float2(cn, sn);
      }
    }
#pragma unroll
    for (int j = 0; j < HPW; j++) norm_rope_chunk<HD, EPL>(qw[j], p.q_norm != nullptr, qnw, p.eps, cs);
    if (slot >= p0 && slot < p1) norm_rope_chunk<HD, EPL>(kn, p.k_norm != nullptr, knw, p.eps, cs);
    if (p.tr_q != nullptr && kp == 0) {  // debug trace
      if (split == 0) {
#pragma unroll
        for (int j = 0; j < HPW; j++) {
          const int h = wv + NW * j;
          if (h < group)
#pragma unroll
            for (int e = 0; e < EPL; e++) p.tr_q[(int64_t(kh) * group + h) * HD + kc * EPL + e] = qw[j][e];
        }
      }
      if (wv == 0 && slot >= p0 && slot < p1)
#pragma unroll
        for (int e = 0; e < EPL; e++) p.tr_k[int64_t(kh) * HD + kc * EPL + e] = kn[e];
    }
  }
  float q[MAXG][EPL];
  if constexpr (FUSED) {
#pragma unroll
    for (int j = 0; j < HPW; j++) {
      const int h = wv + NW * j;
      if (h < MAXG && kp == 0) {
#pragma unroll
        for (int e = 0; e < EPL; e++) s_q[h][kc * EPL + e] = qw[j][e] * p.scale;
      }
    }
    lds_barrier();  // LDS only: the K/V loads stay in flight
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) q[h][e] = s_q[h][kc * EPL + e];
  } else {
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) q[h][e] = qw[h][e] * p.scale;
  }

  // 2. scores of the wave's positions (K layout); masked slots score -inf
  float sc[NL][MAXG];
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int pos = w0 + i * PPL + kp;
    float kf[EPL];
    widen16<KV>(kreg[i], kf);
    if constexpr (FUSED) {
#pragma unroll
      for (int e = 0; e < EPL; e++) kf[e] = pos == slot ? kn[e] : kf[e];
    }
#pragma unroll
    for (int h = 0; h < MAXG; h++) {
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e++) s += q[h][e] * kf[e];
      s = lanes_sum<CPR>(s);
      sc[i][h] = pos < p1 ? s : -INFINITY;
    }
  }

  // 3. the wave's softmax numerators, max and sum per head (uniform across the wave).  A
  //    position's score is already in all CPR of its lanes, so only the position groups
  //    (lanes CPR apart) are reduced.
  float m[MAXG], l[MAXG];
#pragma unroll
  for (int h = 0; h < MAXG; h++) {
    float mx = sc[0][h];
#pragma unroll
    for (int i = 1; i < NL; i++) mx = fmaxf(mx, sc[i][h]);
#pragma unroll
    for (int off = CPR; off < kWave; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const float e = mx == -INFINITY ? 0.f : exp_fast(sc[i][h] - mx);
      sc[i][h] = e;
      sum += e;
    }
#pragma unroll
    for (int off = CPR; off < kWave; off <<= 1) sum += __shfl_xor(sum, off, kWave);
    m[h] = mx;
    l[h] = sum;
  }
  if (kc == 0) {
#pragma unroll
    for (int i = 0; i < NL; i++)
#pragma unroll
      for (int g4 = 0; g4 < G4; g4++) {
        float t[4];
#pragma unroll
        for (int k = 0; k < 4; k++) t[k] = 4 * g4 + k < MAXG ? sc[i][4 * g4 + k] : 0.f;
        s_p[wv][i * PPL + kp][g4] = make_float4(t[0], t[1], t[2], t[3]);
      }
  }

  // 4. P V over the wave's positions (V layout), summed over the PPL position lanes
  float acc[MAXG][EPL];
#pragma unroll
  for (int h = 0; h < MAXG; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[h][e] = 0.f;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int pos = w0 + i * PPL + vp;
    float pr[G4 * 4];
#pragma unroll
    for (int g4 = 0; g4 < G4; g4++) {
      const float4 t = s_p[wv][i * PPL + vp][g4];  // written by this wave above
      pr[4 * g4] = t.x;
      pr[4 * g4 + 1] = t.y;
      pr[4 * g4 + 2] = t.z;
      pr[4 * g4 + 3] = t.w;
    }
    float vf[EPL];
    widen16<KV>(vreg[i], vf);
#pragma unroll
    for (int e = 0; e < EPL; e++) {
      if constexpr (FUSED) vf[e] = pos == slot ? vn[e] : vf[e];
      vf[e] = pos < p1 ? vf[e] : 0.f;  // a stale slot past the active range may hold anything
    }
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) acc[h][e] += pr[h] * vf[e];
  }
#pragma unroll
  for (int h = 0; h < MAXG; h++)
#pragma unroll
    for (int e = 0; e < EPL; e++) acc[h][e] = lanes_sum<PPL>(acc[h][e]);

  // fused: the workgroup holding the new slot appends k, v to the ring
  if constexpr (FUSED) {
    if (slot >= p0 && slot < p1) {
      KV* kw = static_cast<KV*>(p.k_write) + int64_t(slot) * kvd + kh * HD;
      KV* vw = static_cast<KV*>(p.v_write) + int64_t(slot) * kvd + kh * HD;
#pragma unroll
      for (int i = 0; i < NL; i++) {
        if (w0 + i * PPL + kp == slot)
#pragma unroll
          for (int e = 0; e < EPL; e++) kw[kc * EPL + e] = narrow<KV>(kn[e]);
        if (w0 + i * PPL + vp == slot)
#pragma unroll
          for (int e = 0; e < EPL; e++) vw[vc * EPL + e] = narrow<KV>(vn[e]);
      }
    }
  }

  // 5. merge of the four sub-splits
  if (vp == 0) {
#pragma unroll
    for (int h = 0; h < MAXG; h++)
#pragma unroll
      for (int e = 0; e < EPL; e++) s_o[wv][h][vc * EPL + e] = acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < MAXG; h++) {
      s_m[wv][h] = m[h];
      s_l[wv][h] = l[h];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < group * HD; idx += kAttnThreads) {
    const int h = idx / HD, d = idx % HD;
    float M = s_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w][h]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float wt = s_m[w][h] == -INFINITY ? 0.f : exp_fast(s_m[w][h] - M);
      o += wt * s_o[w][h][d];
      L += wt * s_l[w][h];
    }
    const int64_t row = int64_t(kh * group + h) * S + split;
    p.part_o[row * HD + d] = o;
    if (d == 0) {
      p.part_ml[row * 2 + 0] = M;
      p.part_ml[row * 2 + 1] = L;
    }
  }
}

// ---------------------------------------------------------------- f16 rings on MFMA

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ h4_t h4_of(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(h4_t, (uint64_t(hi) << 32) | lo);
}

// The split-K partial for f16 rings on the matrix cores (v_mfma_f32_16x16x16_f16).  Workgroup
// (split s, kv head h) owns slots [64 s, 64 s + 64) and all (up to 16) q heads of h's group; wave w
// owns the 16 slots [64 s + 16 w, +16), one MFMA tile.
//   * Lane l loads 16-byte chunks 4j + l/16 (j < HD/32) of the K row and of the V row of slot
//     l % 16: a row's chunks come from four consecutive lanes, 64 contiguous bytes per load.
//   * Scores S^T[slot][head] = sum_d K[slot][d] q[head][d]: A = the K chunks as loaded (16-dim
//     tile i takes the lane's halves 4i .. 4i+3, i.e. dims 8(4(i/2) + l/16) + 4(i%2) + t), B = q in
//     the same dim order.  q is split into f16 hi + lo parts (q = hi + lo to 2^-22) and the K
//     values are exact f16, so two MFMAs per tile give the f32 scores.
//   * The result lands as lane l: head l % 16, slots 4(l/16) + r -- exactly the A layout of P V
//     (rows = heads, k = slots), so the softmax numerators p (split hi + lo as q) feed P V with no
//     data movement.  V needs the k = slot layout: one MFMA against the identity (A = the V chunks
//     as loaded, B = I) returns V^T tile by tile in that layout, exactly (one non-zero product).
//   * Slots past the active range score -inf and their V is zeroed before any product (a stale
//     slot may hold anything).  The softmax max and sum reduce over the 4 lanes of a head.
//   * Fused (decode step): the q heads are normalised and rotated once per workgroup into LDS (one
//     wave per head); the workgroup holding the new slot does the same for k, attends to the new
//     k and v rounded to f16 (the values the ring then holds) and appends them to the ring.
template <int HD, int MAXG, bool FUSED>
__global__ void __launch_bounds__(kAttnThreads) attn_mfma_kernel(AttnParams p) {
  // the score columns are the group's heads of query blockIdx.z (a batch of queries: one query
  // per grid z, each attending to its own first active + z slots)
  const int group = p.group;
  const int t0 = blockIdx.z;
  p.q += t0 * p.q_stride;
  p.active += t0;
  p.part_o += t0 * p.part_tok;
  p.part_ml += t0 * p.part_tok_ml;
  const int ncol = group;  // valid score columns
  constexpr int NCH = HD / 32;  // 16-byte chunks per lane per row
  constexpr int NT = HD / 16;   // 16-dim MFMA tiles
  constexpr int NW = kAttnThreads / kWave;
  constexpr int CH = 16 * NW;   // slots per workgroup
  constexpr int QC = MAXG;      // score columns with a q row
  static_assert(MAXG <= 16 && (HD == 64 || HD == 128), "tile shape");
  __shared__ __attribute__((aligned(16))) float s_q[16][HD];
  __shared__ __attribute__((aligned(16))) float s_kn[HD], s_vn[HD];
  __shared__ float s_o[NW][QC][HD];
  __shared__ float s_m[NW][16], s_l[NW][16];

  const int split = blockIdx.x, kh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t kvd = int64_t(p.nkv) * HD;
  const int S = gridDim.x;
  const int p0 = split * CH, w0 = p0 + wv * 16;
  const int kq = lane >> 4, col = lane & 15;

  // 0. small loads first (they complete before the K/V loads issued after them)
  int64_t pos_pre = p.pos;
  if constexpr (FUSED) pos_pre = *(p.pos_dev ? p.pos_dev : reinterpret_cast<const int64_t*>(p.k));
  // wave w prepares columns w, w + NW, ... as one pair of dims per lane (lanes < HD / 2)
  constexpr int HPW = (QC + NW - 1) / NW;
  const int pr = lane < HD / 2 ? lane : HD / 2 - 1;
  float2 qv[HPW];
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int c = min(wv + NW * j, ncol - 1);
    qv[j] = reinterpret_cast<const float2*>(p.q + (int64_t(kh) * group + c) * HD)[pr];
  }
  float2 knv = make_float2(0.f, 0.f), vnv = knv, qnw = knv, knw = knv, csv = knv;
  if constexpr (FUSED) {
    knv = reinterpret_cast<const float2*>(p.k_new + kh * HD)[pr];
    vnv = reinterpret_cast<const float2*>(p.v_new + kh * HD)[pr];
    qnw = reinterpret_cast<const float2*>(p.q_norm ? p.q_norm : p.q)[pr];
    knw = reinterpret_cast<const float2*>(p.k_norm ? p.k_norm : p.q)[pr];
    csv = reinterpret_cast<const float2*>(p.rope_cs ? p.rope_cs : p.q)[pr];
  }
  // 1. K and V loads: slot w0 + col, chunks 4j + kq (clamped in-bounds; masked below)
  const int act_hi = p.active;  // slots the query attends to
  const int bound = p.pos_dev ? int(p.capacity) : act_hi;
  const int pl = min(p0 + CH, bound);
  const int ps = min(w0 + col, pl - 1);
  const _Float16* kb = static_cast<const _Float16*>(p.k) + int64_t(kh) * HD + int64_t(ps) * kvd;
  const _Float16* vb = static_cast<const _Float16*>(p.v) + int64_t(kh) * HD + int64_t(ps) * kvd;
  u32x4 kr[NCH], vr[NCH];
#pragma unroll
  for (int j = 0; j < NCH; j++) kr[j] = ld4(reinterpret_cast<const uint8_t*>(kb + 8 * (4 * j + kq)));
#pragma unroll
  for (int j = 0; j < NCH; j++) vr[j] = ld4(reinterpret_cast<const uint8_t*>(vb + 8 * (4 * j + kq)));

  int active = act_hi, slot = p.slot;
  int64_t pos_now = p.pos;
  if (p.pos_dev) {
    pos_now = pos_pre;
    slot = int(pos_now % p.capacity);
    active = int(pos_now + 1 < p.capacity ? pos_now + 1 : p.capacity);
  }
  if (p0 >= active) {  // empty split: contributes nothing to the merge
    if (tid < ncol) {
      const int h = kh * group + tid;
      float* ml = p.part_ml;
      ml[(int64_t(h) * S + split) * 2 + 0] = -INFINITY;
      ml[(int64_t(h) * S + split) * 2 + 1] = 0.f;
    }
    return;
  }
  const int p1 = min(p0 + CH, active);
  const bool has_slot = FUSED && slot >= p0 && slot < p1;

  // 2. q heads (fused: QK-norm, RoPE), scaled, into LDS; rows past the group are zero
  float2 cs = csv;
  if constexpr (FUSED) {
    if (!p.rope_cs) {
      float sn, cn;
      sincosf(rope_angle(pr, HD, pos_now, p.theta), &sn, &cn);
      cs = make_float2(cn, sn);
    }
  }
  auto norm_rope = [&](float2 x, bool has_norm, float2 nw) -> float2 {
    if (has_norm) {
      const float ss = wave_sum_dpp(lane < HD / 2 ? x.x * x.x + x.y * x.y : 0.f);
      const float inv = 1.0f / sqrtf(ss / float(HD) + p.eps);
      x.x = x.x * inv * nw.x;
      x.y = x.y * inv * nw.y;
    }
    return make_float2(x.x * cs.x - x.y * cs.y, x.x * cs.y + x.y * cs.x);
  };
  // (the debug trace of q and k is written at the end: a conditional store here would leave the
  // compiler unable to count the K/V loads in flight, and the scores would wait for V as well)
  float2 q_tr[HPW], k_tr = make_float2(0.f, 0.f);
#pragma unroll
  for (int j = 0; j < HPW; j++) {
    const int h = wv + NW * j;
    float2 x = qv[j];
    if constexpr (FUSED) x = norm_rope(x, p.q_norm != nullptr, qnw);
    q_tr[j] = x;
    if (h < 16 && lane < HD / 2) {
      const bool real = h < ncol;
      reinterpret_cast<float2*>(s_q[h])[lane] = real ? make_float2(x.x * p.scale, x.y * p.scale) : make_float2(0.f, 0.f);
    }
  }
  for (int h = wv + NW * HPW; h < 16; h += NW)  // rows no wave prepared (MAXG < 16)
    if (lane < HD / 2) reinterpret_cast<float2*>(s_q[h])[lane] = make_float2(0.f, 0.f);
  if constexpr (FUSED) {
    if (has_slot && wv == 0) {
      k_tr = norm_rope(knv, p.k_norm != nullptr, knw);
      if (lane < HD / 2) {
        reinterpret_cast<float2*>(s_kn)[lane] = k_tr;
        reinterpret_cast<float2*>(s_vn)[lane] = vnv;
      }
    }
  }
  lds_barrier();  // LDS only: the K/V loads stay in flight

  // 3. B operands of the scores: q hi / lo in the lanes' dim order
  h4_t qhi[NT], qlo[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int d = 8 * (4 * (i / 2) + kq) + 4 * (i % 2);
    const float4 q = *reinterpret_cast<const float4*>(&s_q[col][d]);
    const float qa[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const _Float16 hi = _Float16(qa[t]);
      qhi[i][t] = hi;
      qlo[i][t] = _Float16(qa[t] - float(hi));
    }
  }
  // the new slot's k and v, as f16, replace the ring values in the lane that holds that slot
  const bool mine = has_slot && w0 + col == slot;
  if constexpr (FUSED) {
    if (mine) {
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        const int d = 8 * (4 * j + kq);
        const float* vn = s_vn + d;  // the new v, loaded at entry (a load here would sit under a branch)
        uint32_t kw[4], vw[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          kw[t] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(s_kn[d + 2 * t]))) |
                  (uint32_t(__builtin_bit_cast(uint16_t, _Float16(s_kn[d + 2 * t + 1]))) << 16);
          vw[t] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(vn[2 * t]))) |
                  (uint32_t(__builtin_bit_cast(uint16_t, _Float16(vn[2 * t + 1]))) << 16);
        }
        kr[j] = u32x4{kw[0], kw[1], kw[2], kw[3]};
        vr[j] = u32x4{vw[0], vw[1], vw[2], vw[3]};
      }
    }
  }
  // a slot past the active range may hold anything: its V row becomes zeros
  if (w0 + col >= p1) {
#pragma unroll
    for (int j = 0; j < NCH; j++) vr[j] = u32x4{0u, 0u, 0u, 0u};
  }

  // 4. scores: lane holds head col, slots w0 + 4 kq + r
  f4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const u32x4 c = kr[i / 2];
    const h4_t a = (i & 1) ? h4_of(c.z, c.w) : h4_of(c.x, c.y);
    sc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qhi[i], sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qlo[i], sc, 0, 0, 0);
  }
  // this lane's column attends to slots below lim (its token's count; none for an empty column)
  const int lim = p1;
  float s[4];
#pragma unroll
  for (int r = 0; r < 4; r++) s[r] = w0 + 4 * kq + r < lim ? sc[r] : -INFINITY;
  // 5. the wave's softmax per head: the 4 lanes col, col + 16, col + 32, col + 48
  float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  float e[4], sum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    e[r] = mx == -INFINITY ? 0.f : exp_fast(s[r] - mx);
    sum += e[r];
  }
  sum += __shfl_xor(sum, 16, kWave);
  sum += __shfl_xor(sum, 32, kWave);
  h4_t phi, plo;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const _Float16 hi = _Float16(e[r]);
    phi[r] = hi;
    plo[r] = _Float16(e[r] - float(hi));
  }
  // 6. P V: V^T tiles through the identity, then two MFMAs per tile
  h4_t ident;
#pragma unroll
  for (int t = 0; t < 4; t++) ident[t] = _Float16(4 * kq + t == col ? 1.0f : 0.0f);
  f4_t o[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const u32x4 c = vr[i / 2];
    const h4_t a = (i & 1) ? h4_of(c.z, c.w) : h4_of(c.x, c.y);
    const f4_t vt = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ident, f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    h4_t b;
#pragma unroll
    for (int t = 0; t < 4; t++) b[t] = _Float16(vt[t]);  // exact: the values are f16
    o[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, b, f4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    o[i] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, b, o[i], 0, 0, 0);
  }
  // o[i]: lane holds heads 4 kq + r, the dim of column col of tile i
  // 7. fused: the workgroup holding the new slot appends k and v to the ring (as f16)
  if constexpr (FUSED) {
    if (mine) {
      _Float16* kw = static_cast<_Float16*>(p.k_write) + int64_t(slot) * kvd + kh * HD;
      _Float16* vw = static_cast<_Float16*>(p.v_write) + int64_t(slot) * kvd + kh * HD;
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        *reinterpret_cast<u32x4*>(kw + 8 * (4 * j + kq)) = kr[j];
        *reinterpret_cast<u32x4*>(vw + 8 * (4 * j + kq)) = vr[j];
      }
    }
  }
  // 8. merge of the four waves
#pragma unroll
  for (int i = 0; i < NT; i++) {
    // column col of tile i holds dim 8 (4 (i/2) + col/4) + 4 (i%2) + col%4
    const int d = 8 * (4 * (i / 2) + (col >> 2)) + 4 * (i & 1) + (col & 3);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int h = 4 * kq + r;
      if (h < QC && h < ncol) s_o[wv][h][d] = o[i][r];
    }
  }
  if (lane < 16) {
    s_m[wv][lane] = mx;
    s_l[wv][lane] = sum;
  }
  __syncthreads();
  for (int idx = tid; idx < ncol * HD; idx += kAttnThreads) {
    const int h = idx / HD, d = idx % HD;  // h: the score column
    float M = s_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w][h]);
    float ov = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float wt = s_m[w][h] == -INFINITY ? 0.f : exp_fast(s_m[w][h] - M);
      ov += wt * s_o[w][h][d];
      L += wt * s_l[w][h];
    }
    const int64_t row = int64_t(kh * group + h) * S + split;
    p.part_o[row * HD + d] = ov;
    if (d == 0) {
      p.part_ml[row * 2 + 0] = M;
      p.part_ml[row * 2 + 1] = L;
    }
  }
  if constexpr (FUSED) {  // debug trace: q after QK-norm and RoPE (split 0), the new k (its slot's workgroup)
    if (split == 0 && p.tr_q != nullptr && lane < HD / 2) {
#pragma unroll
      for (int j = 0; j < HPW; j++) {
        const int h = wv + NW * j;
        if (h < 16 && h < ncol) reinterpret_cast<float2*>(p.tr_q + (int64_t(kh) * group + h) * HD)[lane] = q_tr[j];
      }
    }
    if (has_slot && wv == 0 && p.tr_k != nullptr && lane < HD / 2)
      reinterpret_cast<float2*>(p.tr_k + int64_t(kh) * HD)[lane] = k_tr;
  }
}

// Causal attention of a batch of consecutive queries (the prefill) over an f16 ring, flash
// style: grid (ceil(T / (4 tpw)), nkv) with tpw = 16 / group tokens per column set, the token
// blocks with the longest causal ranges first.  Eight waves: column set w % 4 holds the 16 score
// columns (token, head) of its tpw tokens, all heads of the group, and waves w and w + 4 share
// them, taking alternate 64-slot runs.  The workgroup walks the slots its tokens attend to
// (query t of the batch: the first active + t slots) 128 at a time, stages their K and V rows in
// LDS (V zero past the last attended slot; the next 128 rows are loaded into registers while
// the current ones are used; V transposed, [dim][slot]), and each wave takes its run 32 slots
// at a time through an online softmax (running max and sum per column over the 4 lanes that
// hold it, the accumulators rescaled per 32 slots).  The two waves' states of a column are
// merged through LDS at the end.  Per 32 slots: S^T = K q for two 16-slot chunks on
// v_mfma_f32_16x16x32_f16 (q split into f16 hi + lo, one accumulator each), P V on the same
// MFMA with K = the lane's 8 slots of both chunks, the B operand read straight from V^T (P
// split likewise).  No split partials: the rows
// o / l go through LDS and are written as f32 rows (out, when given) and, when q8k is given, as
// the Q8_K blocks of Wo's input (group * HD a multiple of 256: the group's heads fill whole
// blocks), quantized from the same f32 values.
template <int HD>
__global__ void __launch_bounds__(kFlashThreads) attn_flash_kernel(AttnParams p, float* __restrict__ out,
                                                                   int64_t out_stride, uint8_t* __restrict__ q8k) {
  constexpr int NCH = HD / 32, NT = HD / 16, NCS = 4, CH = 64, RS = 2 * CH;
  constexpr int NW = kFlashThreads / kWave;
  constexpr int KS = 2 * HD + 16;  // LDS bytes per staged K row: the f16 row and 16 bytes of padding
  constexpr int VTS = RS + 8;      // f16 per row of V^T (one row per dim)
  // K rows, then V^T.  After the runs: the second waves' partial states at the start, the
  // workgroup's output rows (4 (16 / group) tokens of group * HD floats: at most 256 HD bytes)
  // after RS K rows
  __shared__ __attribute__((aligned(16))) uint8_t s_kv[RS * KS + HD * VTS * 2];
  constexpr int PO_BYTES = NCS * NT * 4 * 64 * 4 + NCS * 16 * 2 * 4;
  static_assert(PO_BYTES <= RS * KS && RS * KS + 256 * HD <= RS * KS + HD * VTS * 2, "merge areas fit the staging");
  uint8_t* const s_k = s_kv;
  _Float16* const s_vt = reinterpret_cast<_Float16*>(s_kv + RS * KS);
  const int group = p.group, tpw = 16 / group;
  const int kh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, cs = wv & 3, rp = wv >> 2;
  const int col = lane & 15, kq = lane >> 4;
  const int64_t kvd = int64_t(p.nkv) * HD;
  const int tg0 = int(gridDim.x - 1 - blockIdx.x) * NCS * tpw;  // the workgroup's first token
  const int ntl = min(NCS * tpw, p.n_tok - tg0);                 // and its token count
  const int pl = p.active + tg0 + ntl - 1;                       // slots any of its tokens attends to
  const int nstep = (pl + RS - 1) / RS;
  const int tw0 = tg0 + cs * tpw;                                // this wave's first token
  const int ncol = max(0, min(tpw, p.n_tok - tw0)) * group;      // this wave's valid columns
  // staging: row r = tid / 4 of the 128 slots, a quarter of it per thread (K: dims qq HD / 4 + 8 j
  // + t; V: the 16-byte chunks 4 j + qq, dims 8 (4 j + qq) + t, so that the transposed stores of
  // the four quarters meet at most two to a bank)
  const int r = tid >> 2, qq = tid & 3;
  const uint8_t* const kb = static_cast<const uint8_t*>(p.k) + int64_t(kh) * HD * 2 + qq * (HD / 2);
  const uint8_t* const vb = static_cast<const uint8_t*>(p.v) + int64_t(kh) * HD * 2 + 16 * qq;
  u32x4 kr[HD / 32], vr[HD / 32];
  auto load_step = [&](int st) {
    const int64_t o = int64_t(min(st * RS + r, pl - 1)) * kvd * 2;
#pragma unroll
    for (int j = 0; j < HD / 32; j++) kr[j] = ld4(kb + o + 16 * j);
#pragma unroll
    for (int j = 0; j < HD / 32; j++) vr[j] = ld4(vb + o + 64 * j);
  };
  load_step(0);
  // this lane's q fragments for column col (token tw0 + col / group, head col % group), scaled
  const bool cvalid = col < ncol;
  const int ctl = cvalid ? col / group : 0, chd = cvalid ? col % group : 0;
  // (a wave past the last token reads the last token's row and uses none of it)
  const float* qrow = p.q + int64_t(min(tw0 + ctl, p.n_tok - 1)) * p.q_stride + (int64_t(kh) * group + chd) * HD;
  h8_t qhi[NCH], qlo[NCH];  // dims 32 j + 8 kq .. + 8, the K-row fragment's dims
#pragma unroll
  for (int j = 0; j < NCH; j++) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const float4 q = *reinterpret_cast<const float4*>(qrow + 32 * j + 8 * kq + 4 * h);
      const float qa[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const float v = cvalid ? qa[t] * p.scale : 0.f;
        const _Float16 hi = _Float16(v);
        qhi[j][4 * h + t] = hi;
        qlo[j][4 * h + t] = _Float16(v - float(hi));
      }
    }
  }
  const int lim = cvalid ? p.active + tw0 + ctl : 0;  // the column's slots: [0, lim)
  float m = -INFINITY, l = 0.f;
  f4_t o[NT];
#pragma unroll
  for (int i = 0; i < NT; i++) o[i] = f4_t{0.f, 0.f, 0.f, 0.f};
  for (int st = 0; st < nstep; st++) {
    const int p0 = st * RS + rp * CH;  // this wave's run
    if (st) lds_barrier();             // every wave is done with the previous rows
    const bool vz = st * RS + r >= pl;
    // V^T in dwords of two slots: rows r and r ^ 1 (lanes 4 apart) swap halves of their chunk,
    // the even row then stores dims 0..3 of the chunk for both slots, the odd row dims 4..7
    const bool odd = r & 1;
    uint32_t* const s_vt32 = reinterpret_cast<uint32_t*>(s_vt);
#pragma unroll
    for (int j = 0; j < HD / 32; j++) {
      *reinterpret_cast<u32x4*>(s_k + r * KS + qq * (HD / 2) + 16 * j) = kr[j];
      const u32x4 vv = vz ? u32x4{0u, 0u, 0u, 0u} : vr[j];
      const uint32_t r0 = __shfl_xor(odd ? vv.x : vv.z, 4, kWave), r1 = __shfl_xor(odd ? vv.y : vv.w, 4, kWave);
      const uint32_t a0 = odd ? vv.z : vv.x, a1 = odd ? vv.w : vv.y;  // this row's four dims
      // dword (slot even, slot odd): the even row's f16 in the low half
      const uint32_t lo0 = odd ? r0 : a0, hi0 = odd ? a0 : r0, lo1 = odd ? r1 : a1, hi1 = odd ? a1 : r1;
      const int d0 = 8 * (4 * j + qq) + (odd ? 4 : 0);
      uint32_t* dst = s_vt32 + (d0 * VTS + (r & ~1)) / 2;
      dst[0] = (lo0 & 0xFFFFu) | (hi0 << 16);
      dst[VTS / 2] = (lo0 >> 16) | (hi0 & 0xFFFF0000u);
      dst[VTS] = (lo1 & 0xFFFFu) | (hi1 << 16);
      dst[3 * (VTS / 2)] = (lo1 >> 16) | (hi1 & 0xFFFF0000u);
    }
    load_step(min(st + 1, nstep - 1));  // the next rows (the last step reloads itself: no branch)
    lds_barrier();
    for (int cp = 0; cp < 2; cp++) {  // 32 slots at a time: chunks A (c0 ..) and B (c0 + 16 ..)
      const int c0 = p0 + 32 * cp, sr = rp * CH + 32 * cp;  // sr: the staged row of slot c0
      if (c0 >= pl) break;  // uniform in the wave: no slot of these chunks is attended by any token
      // scores: lane holds column col, slots c0 + 4 kq + r (A) and c0 + 16 + 4 kq + r (B)
      f4_t ha = {0.f, 0.f, 0.f, 0.f}, la = ha, hb = ha, lb = ha;
#pragma unroll
      for (int j = 0; j < NCH; j++) {
        const h8_t ka = __builtin_bit_cast(h8_t, *reinterpret_cast<const u32x4*>(s_k + (sr + col) * KS + 16 * (4 * j + kq)));
        const h8_t kb8 = __builtin_bit_cast(h8_t, *reinterpret_cast<const u32x4*>(s_k + (sr + 16 + col) * KS +
                                                                                  16 * (4 * j + kq)));
        ha = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[j], ha, 0, 0, 0);
        la = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[j], la, 0, 0, 0);
        hb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb8, qhi[j], hb, 0, 0, 0);
        lb = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb8, qlo[j], lb, 0, 0, 0);
      }
      float s8[8];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        s8[rr] = c0 + 4 * kq + rr < lim ? ha[rr] + la[rr] : -INFINITY;
        s8[4 + rr] = c0 + 16 + 4 * kq + rr < lim ? hb[rr] + lb[rr] : -INFINITY;
      }
      float mx = s8[0];
#pragma unroll
      for (int rr = 1; rr < 8; rr++) mx = fmaxf(mx, s8[rr]);
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mn = fmaxf(m, mx);
      const float alpha = mn == -INFINITY ? 1.f : exp_fast(m - mn);
      float e[8], sum = 0.f;
#pragma unroll
      for (int rr = 0; rr < 8; rr++) {
        e[rr] = mn == -INFINITY ? 0.f : exp_fast(s8[rr] - mn);
        sum += e[rr];
      }
      sum += __shfl_xor(sum, 16, kWave);
      sum += __shfl_xor(sum, 32, kWave);
      l = l * alpha + sum;
      m = mn;
      // the accumulators hold columns 4 kq + rr: their factors from the lanes of those columns
      float ar[4];
#pragma unroll
      for (int rr = 0; rr < 4; rr++) ar[rr] = __shfl(alpha, 4 * kq + rr, kWave);
      // P as the A operand of a K = 32 MFMA: the lane's 8 K elements are its 8 slots above, and the
      // B operand (V) holds the same 8 slots for dim 16 i + col
      h8_t phi, plo;
#pragma unroll
      for (int rr = 0; rr < 8; rr++) {
        const _Float16 hi = _Float16(e[rr]);
        phi[rr] = hi;
        plo[rr] = _Float16(e[rr] - float(hi));
      }
#pragma unroll
      for (int i = 0; i < NT; i++) {
        const _Float16* vrow = s_vt + (16 * i + col) * VTS + sr + 4 * kq;
        const h4_t va = *reinterpret_cast<const h4_t*>(vrow), vb4 = *reinterpret_cast<const h4_t*>(vrow + 16);
        const h8_t bv = {va[0], va[1], va[2], va[3], vb4[0], vb4[1], vb4[2], vb4[3]};
#pragma unroll
        for (int rr = 0; rr < 4; rr++) o[i][rr] *= ar[rr];
        o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(phi, bv, o[i], 0, 0, 0);
        o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo, bv, o[i], 0, 0, 0);
      }
    }
  }
  // merge the two waves of each column set; o[i][rr] is column 4 kq + rr at dim 16 i + col
  float* const s_po = reinterpret_cast<float*>(s_kv);  // [set][i][rr][lane]
  float* const s_pml = s_po + NCS * NT * 4 * 64;       // [set][column][m, l]
  const int rowlen = group * HD;
  float* const s_row = reinterpret_cast<float*>(s_kv + RS * KS);  // [token of the workgroup][group * HD]
  lds_barrier();  // every wave is done with the staged rows
  if (rp == 1) {
#pragma unroll
    for (int i = 0; i < NT; i++)
#pragma unroll
      for (int rr = 0; rr < 4; rr++) s_po[((cs * NT + i) * 4 + rr) * 64 + lane] = o[i][rr];
    if (kq == 0) {
      s_pml[(cs * 16 + col) * 2] = m;
      s_pml[(cs * 16 + col) * 2 + 1] = l;
    }
  }
  lds_barrier();
  if (rp == 0) {
    const float m1 = s_pml[(cs * 16 + col) * 2], l1 = s_pml[(cs * 16 + col) * 2 + 1];
    const float M = fmaxf(m, m1);
    const float a0 = m == -INFINITY ? 0.f : exp_fast(m - M), a1 = m1 == -INFINITY ? 0.f : exp_fast(m1 - M);
    const float lt = l * a0 + l1 * a1;
    float f0[4], f1[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const float li = __shfl(lt, 4 * kq + rr, kWave);
      f0[rr] = __shfl(a0, 4 * kq + rr, kWave) / li;
      f1[rr] = __shfl(a1, 4 * kq + rr, kWave) / li;
    }
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int c = 4 * kq + rr;
      if (c < ncol) {
        float* dst = s_row + (cs * tpw + c / group) * rowlen + (c % group) * HD;
#pragma unroll
        for (int i = 0; i < NT; i++)
          dst[16 * i + col] = o[i][rr] * f0[rr] + s_po[((cs * NT + i) * 4 + rr) * 64 + lane] * f1[rr];
      }
    }
  }
  lds_barrier();
  if (out)
    for (int idx = 4 * tid; idx < ntl * rowlen; idx += 4 * kFlashThreads) {
      const int tl = idx / rowlen, e = idx - tl * rowlen;
      *reinterpret_cast<float4*>(out + int64_t(tg0 + tl) * out_stride + int64_t(kh) * rowlen + e) =
          *reinterpret_cast<const float4*>(s_row + idx);
    }
  if (q8k) {
    const int bpt = rowlen / 256;                      // the group's Q8_K blocks per token
    const int64_t rbq = int64_t(p.nkv) * bpt * 292;    // bytes of a token's Q8_K row
    for (int jb = wv; jb < ntl * bpt; jb += NW) {
      const int tl = jb / bpt, j = jb - tl * bpt;
      const float4 v = reinterpret_cast<const float4*>(s_row + tl * rowlen + 256 * j)[lane];
      const float ev[4] = {v.x, v.y, v.z, v.w};
      q8k_block_wave(ev, lane, q8k + int64_t(tg0 + tl) * rbq + (int64_t(kh) * bpt + j) * 292);
    }
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
                                                           float* __restrict__ out, int64_t tok_o, int64_t tok_ml,
                                                           int64_t tok_out) {
  part_o += blockIdx.y * tok_o;  // token of a batch of queries
  part_ml += blockIdx.y * tok_ml;
  out += blockIdx.y * tok_out;
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
    const float w = (s < S && e[i].y > 0.f) ? exp_fast(e[i].x - M) : 0.f;
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

// Merge for up to 256 splits (decode up to 16384 positions): one workgroup per q head, wave w
// takes splits w, w + 4, ... (at most 64, one per lane).  Every load goes out at entry -- the
// lane's (m, l) and, for each of the wave's splits, the partial rows' elements of the lane's
// dims -- so the merge costs one round trip; the wave's max and sum are DPP reductions, the
// split weights are broadcast with readlane, and one barrier merges the four waves.
constexpr int kCombineSmallSplits = 256;

template <int HD>
__global__ void __launch_bounds__(256) attn_combine_small_kernel(const float* __restrict__ part_o,
                                                                 const float* __restrict__ part_ml, int S,
                                                                 float* __restrict__ out, int64_t tok_o,
                                                                 int64_t tok_ml, int64_t tok_out) {
  part_o += blockIdx.y * tok_o;  // token of a batch of queries
  part_ml += blockIdx.y * tok_ml;
  out += blockIdx.y * tok_out;
  constexpr int DPL = HD >= 64 ? HD / 64 : 1;  // dims per lane
  constexpr int CHUNK = 16;                    // splits per batch of loads
  __shared__ float s_o[4][HD];
  __shared__ float s_ml[4][2];
  const int h = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int ns = (S - wv + 3) / 4;  // splits of this wave
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + int64_t(h) * S;
  const float* po = part_o + int64_t(h) * S * HD;
  const int s_lane = min(wv + 4 * lane, S - 1);
  const float2 e = ml[s_lane];
  float o[DPL];
#pragma unroll
  for (int t = 0; t < DPL; t++) o[t] = 0.f;
  // first batch of partial-row loads, issued before the (m, l) arithmetic
  float v[CHUNK][DPL];
#pragma unroll
  for (int jj = 0; jj < CHUNK; jj++)
#pragma unroll
    for (int t = 0; t < DPL; t++)
      v[jj][t] = po[int64_t(min(wv + 4 * jj, S - 1)) * HD + min(lane + 64 * t, HD - 1)];
  const bool ok = lane < ns && e.y > 0.f;
  const float M = wave_max_dpp(ok ? e.x : -INFINITY);
  const float wgt = ok ? exp_fast(e.x - M) : 0.f;
  const float L = wave_sum_dpp(wgt * e.y);
  for (int j0 = 0; j0 < ns; j0 += CHUNK) {
    if (j0 > 0) {
#pragma unroll
      for (int jj = 0; jj < CHUNK; jj++)
#pragma unroll
        for (int t = 0; t < DPL; t++)
          v[jj][t] = po[int64_t(min(wv + 4 * (j0 + jj), S - 1)) * HD + min(lane + 64 * t, HD - 1)];
    }
    // Empty splits never wrote their rows (the workspace holds whatever was there, possibly
    // NaN): their zero weight selects the row out of the sum instead of multiplying it.
#pragma unroll
    for (int jj = 0; jj < CHUNK; jj++) {
      const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), j0 + jj));
      const bool use = j0 + jj < ns && w != 0.f;
#pragma unroll
      for (int t = 0; t < DPL; t++) o[t] += use ? w * v[jj][t] : 0.f;
    }
  }
#pragma unroll
  for (int t = 0; t < DPL; t++)
    if (lane + 64 * t < HD) s_o[wv][lane + 64 * t] = o[t];
  if (lane == 0) {
    s_ml[wv][0] = M;
    s_ml[wv][1] = L;
  }
  __syncthreads();
  for (int d = threadIdx.x; d < HD; d += 256) {
    float Mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++)
      if (s_ml[w][1] > 0.f) Mx = fmaxf(Mx, s_ml[w][0]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const bool live = s_ml[w][1] > 0.f;
      const float c = live ? exp_fast(s_ml[w][0] - Mx) : 0.f;
      num += live ? c * s_o[w][d] : 0.f;
      den += c * s_ml[w][1];
    }
    out[int64_t(h) * HD + d] = num / den;
  }
}

// ---------------------------------------------------------------- any even head_dim up to 256
// gqa_causal_attention_f32 takes any even head_dim (even_head_dim, src/qwen_deepseek.rs:58-65) and
// any group size; the kernels above are built for head_dim 32 / 64 / 128 and up to 8 (16 on the
// matrix cores) q heads per kv head.  The others run these two: a split-K partial with a runtime
// head_dim and one q head per workgroup, and a merge with a runtime head_dim.  Workgroup (split s,
// q head h, query z) owns slots [64 s, 64 s + 64), 16 per wave; lane l holds dims l, l + 64,
// l + 128 and l + 192 (those below head_dim), so a slot's score is one whole-wave DPP sum.  Every
// K / V load of the wave goes out before the first score.  Fused mode: the workgroup normalises and
// rotates its q head (the RoPE partner of dim d, d ^ 1, sits one lane over) and, holding the new
// slot, k; the workgroup of the group's first q head appends k and v to the ring.
constexpr int kGenDims = 4;     // dims per lane: head_dim <= 256
constexpr int kGenSlots = 16;   // slots per wave
constexpr int kGenMaxHd = 64 * kGenDims;

template <typename KV, bool FUSED>
__global__ void __launch_bounds__(kAttnThreads) attn_generic_kernel(AttnParams p) {
  const int t0 = blockIdx.z;
  p.q += t0 * p.q_stride;
  p.active += t0;
  p.part_o += t0 * p.part_tok;
  p.part_ml += t0 * p.part_tok_ml;
  const int hd = p.hd, group = p.group;
  const int split = blockIdx.x, h = blockIdx.y, kh = h / group;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int S = gridDim.x;
  const int64_t kvd = int64_t(p.nkv) * hd;
  constexpr int CH = kGenSlots * (kAttnThreads / kWave);
  const int p0 = split * CH, w0 = p0 + wv * kGenSlots;
  __shared__ float s_o[kAttnThreads / kWave][kGenMaxHd];
  __shared__ float s_m[kAttnThreads / kWave], s_l[kAttnThreads / kWave];

  // small loads first, then every K / V row of the wave (clamped in-bounds; masked below)
  int64_t pos_now = p.pos;
  if (p.pos_dev) pos_now = *p.pos_dev;
  float q[kGenDims], kn[kGenDims], vn[kGenDims], qnw[kGenDims], knw[kGenDims];
#pragma unroll
  for (int t = 0; t < kGenDims; t++) {
    const int d = min(lane + 64 * t, hd - 1);
    q[t] = p.q[int64_t(h) * hd + d];
    kn[t] = vn[t] = qnw[t] = knw[t] = 0.f;
    if constexpr (FUSED) {
      kn[t] = p.k_new[int64_t(kh) * hd + d];
      vn[t] = p.v_new[int64_t(kh) * hd + d];
      qnw[t] = p.q_norm ? p.q_norm[d] : 0.f;
      knw[t] = p.k_norm ? p.k_norm[d] : 0.f;
    }
  }
  const int bound = p.pos_dev ? int(p.capacity) : p.active;
  const KV* kb = static_cast<const KV*>(p.k) + int64_t(kh) * hd;
  const KV* vb = static_cast<const KV*>(p.v) + int64_t(kh) * hd;
  KV kr[kGenSlots][kGenDims], vr[kGenSlots][kGenDims];
#pragma unroll
  for (int i = 0; i < kGenSlots; i++) {
    const int64_t ps = min(w0 + i, bound - 1);
#pragma unroll
    for (int t = 0; t < kGenDims; t++) {
      const int d = min(lane + 64 * t, hd - 1);
      kr[i][t] = kb[ps * kvd + d];
      vr[i][t] = vb[ps * kvd + d];
    }
  }
  int active = p.active, slot = p.slot;
  if (p.pos_dev) {
    slot = int(pos_now % p.capacity);
    active = int(pos_now + 1 < p.capacity ? pos_now + 1 : p.capacity);
  }
  float* ml = p.part_ml;
  if (p0 >= active) {  // empty split: contributes nothing to the merge
    if (threadIdx.x == 0) {
      ml[(int64_t(h) * S + split) * 2 + 0] = -INFINITY;
      ml[(int64_t(h) * S + split) * 2 + 1] = 0.f;
    }
    return;
  }
  const int p1 = min(p0 + CH, active);
  const bool has_slot = FUSED && slot >= p0 && slot < p1;
  if constexpr (FUSED) {
    // per-head RMSNorm, then RoPE of the pair (2i, 2i + 1) = dims (d & ~1, d | 1)
    float cs[kGenDims], sn[kGenDims];
#pragma unroll
    for (int t = 0; t < kGenDims; t++) {
      const int i = min(lane + 64 * t, hd - 1) >> 1;
      if (p.rope_cs) {
        cs[t] = p.rope_cs[2 * i];
        sn[t] = p.rope_cs[2 * i + 1];
      } else {
        sincosf(rope_angle(i, hd, pos_now, p.theta), &sn[t], &cs[t]);
      }
    }
    auto norm_rope = [&](float (&x)[kGenDims], bool has_norm, const float (&nw)[kGenDims]) {
      if (has_norm) {
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < kGenDims; t++) ss += lane + 64 * t < hd ? x[t] * x[t] : 0.f;
        ss = wave_sum_dpp(ss);
        const float inv = 1.0f / sqrtf(ss / float(hd) + p.eps);
#pragma unroll
        for (int t = 0; t < kGenDims; t++) x[t] = x[t] * inv * nw[t];
      }
      const bool odd = lane & 1;
#pragma unroll
      for (int t = 0; t < kGenDims; t++) {
        const float other = __shfl_xor(x[t], 1, kWave);
        const float x0 = odd ? other : x[t], x1 = odd ? x[t] : other;
        x[t] = odd ? x0 * sn[t] + x1 * cs[t] : x0 * cs[t] - x1 * sn[t];
      }
    };
    norm_rope(q, p.q_norm != nullptr, qnw);
    if (p.tr_q && split == 0 && wv == 0) {
#pragma unroll
      for (int t = 0; t < kGenDims; t++)
        if (lane + 64 * t < hd) p.tr_q[int64_t(h) * hd + lane + 64 * t] = q[t];
    }
    if (has_slot) {
      norm_rope(kn, p.k_norm != nullptr, knw);
      if (p.tr_k && h == kh * group && wv == 0) {
#pragma unroll
        for (int t = 0; t < kGenDims; t++)
          if (lane + 64 * t < hd) p.tr_k[int64_t(kh) * hd + lane + 64 * t] = kn[t];
      }
      // the ring holds the new k and v as KV values: attend to those
#pragma unroll
      for (int t = 0; t < kGenDims; t++) {
        kn[t] = float(KV(kn[t]));
        vn[t] = float(KV(vn[t]));
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kGenDims; t++) q[t] = lane + 64 * t < hd ? q[t] * p.scale : 0.f;

  // scores, the wave's softmax over its slots, P V
  float sc[kGenSlots];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kGenSlots; i++) {
    const int pos = w0 + i;
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < kGenDims; t++) {
      float kv = float(kr[i][t]);
      if constexpr (FUSED) kv = pos == slot ? kn[t] : kv;
      s += q[t] * kv;
    }
    s = wave_sum_dpp(s);
    sc[i] = pos < p1 ? s : -INFINITY;
    mx = fmaxf(mx, sc[i]);
  }
  float l = 0.f, acc[kGenDims];
#pragma unroll
  for (int t = 0; t < kGenDims; t++) acc[t] = 0.f;
#pragma unroll
  for (int i = 0; i < kGenSlots; i++) {
    const int pos = w0 + i;
    const float e = mx == -INFINITY ? 0.f : exp_fast(sc[i] - mx);
    l += e;
#pragma unroll
    for (int t = 0; t < kGenDims; t++) {
      float v = float(vr[i][t]);
      if constexpr (FUSED) v = pos == slot ? vn[t] : v;
      v = pos < p1 ? v : 0.f;  // a stale slot past the active range may hold anything
      acc[t] += e * v;
    }
  }
  // fused: the group's first q head's workgroup appends k and v to the ring
  if constexpr (FUSED) {
    if (has_slot && h == kh * group && wv == 0) {
      KV* kw = static_cast<KV*>(p.k_write) + int64_t(slot) * kvd + int64_t(kh) * hd;
      KV* vw = static_cast<KV*>(p.v_write) + int64_t(slot) * kvd + int64_t(kh) * hd;
#pragma unroll
      for (int t = 0; t < kGenDims; t++)
        if (lane + 64 * t < hd) {
          kw[lane + 64 * t] = KV(kn[t]);
          vw[lane + 64 * t] = KV(vn[t]);
        }
    }
  }
  // merge of the four waves
#pragma unroll
  for (int t = 0; t < kGenDims; t++)
    if (lane + 64 * t < hd) s_o[wv][lane + 64 * t] = acc[t];
  if (lane == 0) {
    s_m[wv] = mx;
    s_l[wv] = l;
  }
  __syncthreads();
  constexpr int NW = kAttnThreads / kWave;
  for (int d = threadIdx.x; d < hd; d += kAttnThreads) {
    float M = s_m[0];
#pragma unroll
    for (int w = 1; w < NW; w++) M = fmaxf(M, s_m[w]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float wt = s_m[w] == -INFINITY ? 0.f : exp_fast(s_m[w] - M);
      o += wt * s_o[w][d];
      L += wt * s_l[w];
    }
    const int64_t row = int64_t(h) * S + split;
    p.part_o[row * hd + d] = o;
    if (d == 0) {
      ml[row * 2 + 0] = M;
      ml[row * 2 + 1] = L;
    }
  }
}

// Merge of the generic kernel's splits, runtime head_dim: one workgroup per (q head, query).
// Splits with l = 0 (empty) never wrote their rows and are left out by select.
__global__ void __launch_bounds__(256) attn_combine_generic_kernel(const float* __restrict__ part_o,
                                                                   const float* __restrict__ part_ml, int S, int hd,
                                                                   float* __restrict__ out, int64_t tok_o,
                                                                   int64_t tok_ml, int64_t tok_out) {
  part_o += blockIdx.y * tok_o;
  part_ml += blockIdx.y * tok_ml;
  out += blockIdx.y * tok_out;
  __shared__ float s_red[4];
  const int h = blockIdx.x, lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + int64_t(h) * S;
  float m = -INFINITY;
  for (int s = threadIdx.x; s < S; s += 256) {
    const float2 e = ml[s];
    if (e.y > 0.f) m = fmaxf(m, e.x);
  }
  m = wave_max_dpp(m);
  if (lane == 0) s_red[wv] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  const float* po = part_o + int64_t(h) * S * hd;
  for (int d = threadIdx.x; d < hd; d += 256) {
    float num = 0.f, den = 0.f;
    for (int s = 0; s < S; s++) {
      const float2 e = ml[s];
      const bool live = e.y > 0.f;
      const float c = live ? exp_fast(e.x - M) : 0.f;
      num += live ? c * po[int64_t(s) * hd + d] : 0.f;
      den += c * e.y;
    }
    out[int64_t(h) * hd + d] = num / den;
  }
}

int attn_splits(int active, int hd) { return (active + attn_chunk(hd) - 1) / attn_chunk(hd); }

// head_dim and group sizes the head_dim-templated kernels take (the rest run the generic pair)
bool attn_templated(int hd, int group) { return (hd == 32 || hd == 64 || hd == 128) && group <= kMaxGroup; }

size_t attn_workspace_bytes(int nq, int hd, int active) {
  const size_t S = size_t(attn_splits(active, hd));
  return size_t(nq) * S * (size_t(hd) + 2) * sizeof(float);
}

template <int HD, typename KV, bool FUSED>
static void launch_partial(const AttnParams& p, int S, int T, hipStream_t s) {
  const dim3 grid(S, p.nkv, T);
  if (p.group <= 1)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 1>), grid, dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 2)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 2>), grid, dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 4)
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 4>), grid, dim3(kAttnThreads), 0, s, p);
  else
    hipLaunchKernelGGL((attn_partial_kernel<HD, KV, FUSED, 8>), grid, dim3(kAttnThreads), 0, s, p);
}

template <int HD, bool FUSED>
static void launch_mfma(const AttnParams& p, int S, int T, hipStream_t s) {
  const dim3 grid(S, p.nkv, T);
  if (p.group <= 1)
    hipLaunchKernelGGL((attn_mfma_kernel<HD, 1, FUSED>), grid, dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 2)
    hipLaunchKernelGGL((attn_mfma_kernel<HD, 2, FUSED>), grid, dim3(kAttnThreads), 0, s, p);
  else if (p.group <= 4)
    hipLaunchKernelGGL((attn_mfma_kernel<HD, 4, FUSED>), grid, dim3(kAttnThreads), 0, s, p);
  else
    hipLaunchKernelGGL((attn_mfma_kernel<HD, 8, FUSED>), grid, dim3(kAttnThreads), 0, s, p);
}

template <int HD>
static void launch_combine(const AttnParams& p, int S, int T, float* out, int64_t out_stride, hipStream_t s) {
  const int nq = p.nkv * p.group;
  const dim3 grid(nq, T);
  if (S <= kCombineSmallSplits)
    hipLaunchKernelGGL((attn_combine_small_kernel<HD>), grid, dim3(256), 0, s, p.part_o, p.part_ml, S, out,
                       p.part_tok, p.part_tok_ml, out_stride);
  else
    hipLaunchKernelGGL((attn_combine_kernel<HD>), grid, dim3(256), 0, s, p.part_o, p.part_ml, S, out, p.part_tok,
                       p.part_tok_ml, out_stride);
}

// The split-K partial kernel over S splits for T queries, then the merge.
static int attention_impl(AttnParams p, bool fused, int S, int T, float* out, int64_t out_stride, hipStream_t s) {
  const int64_t nq = int64_t(p.nkv) * p.group;
  p.part_tok = T > 1 ? nq * S * p.hd : 0;
  p.part_tok_ml = T > 1 ? nq * S * 2 : 0;
  p.part_ml = p.part_o + int64_t(T) * nq * S * p.hd;
  p.n_tok = T;
  if (!attn_templated(p.hd, p.group)) {  // any other even head_dim or group: one q head per workgroup
    const dim3 grid(S, unsigned(nq), T);
    if (p.kv_dtype == JERO_KV_F16) {
      if (fused) hipLaunchKernelGGL((attn_generic_kernel<_Float16, true>), grid, dim3(kAttnThreads), 0, s, p);
      else hipLaunchKernelGGL((attn_generic_kernel<_Float16, false>), grid, dim3(kAttnThreads), 0, s, p);
    } else {
      if (fused) hipLaunchKernelGGL((attn_generic_kernel<float, true>), grid, dim3(kAttnThreads), 0, s, p);
      else hipLaunchKernelGGL((attn_generic_kernel<float, false>), grid, dim3(kAttnThreads), 0, s, p);
    }
    int rc = check_launch("attention partial");
    if (rc) return rc;
    hipLaunchKernelGGL(attn_combine_generic_kernel, dim3(unsigned(nq), T), dim3(256), 0, s, p.part_o, p.part_ml, S,
                       p.hd, out, p.part_tok, p.part_tok_ml, out_stride);
    return check_launch("attention combine");
  }
#define JERO_ATTN_CASE(HDV)                                                                     \
  if (p.hd == HDV) {                                                                            \
    if (p.kv_dtype == JERO_KV_F16 && HDV >= 64) {                                               \
      if (fused) launch_mfma<(HDV >= 64 ? HDV : 64), true>(p, S, T, s);                         \
      else launch_mfma<(HDV >= 64 ? HDV : 64), false>(p, S, T, s);                              \
    } else if (p.kv_dtype == JERO_KV_F16) {                                                     \
      if (fused) launch_partial<HDV, _Float16, true>(p, S, T, s);                               \
      else launch_partial<HDV, _Float16, false>(p, S, T, s);                                    \
    } else {                                                                                    \
      if (fused) launch_partial<HDV, float, true>(p, S, T, s);                                  \
      else launch_partial<HDV, float, false>(p, S, T, s);                                       \
    }                                                                                           \
  }
  JERO_ATTN_CASE(32) else JERO_ATTN_CASE(64) else JERO_ATTN_CASE(128) else return fail(
      JERO_ERR_CAPABILITY_MISMATCH, "attention: head_dim " + std::to_string(p.hd) + " not in {32, 64, 128}");
#undef JERO_ATTN_CASE
  int rc = check_launch("attention partial");
  if (rc) return rc;
  if (p.hd == 32) launch_combine<32>(p, S, T, out, out_stride, s);
  else if (p.hd == 64) launch_combine<64>(p, S, T, out, out_stride, s);
  else launch_combine<128>(p, S, T, out, out_stride, s);
  return check_launch("attention combine");
}

int launch_attention(const AttnParams& p, bool fused, float* out, hipStream_t s) {
  return attention_impl(p, fused, attn_splits(p.pos_dev ? int(p.capacity) : p.active, p.hd), 1, out, 0, s);
}

bool attn_flash_ok(int kv_dtype, int hd, int n_tok, int group) {
  return kv_dtype == JERO_KV_F16 && (hd == 64 || hd == 128) && n_tok > 1 && group <= kMaxGroup;
}

bool attn_flash_q8k_ok(int group, int hd) { return (hd == 64 || hd == 128) && (group * hd) % 256 == 0; }

int launch_attention_tokens(const AttnParams& p0, int n_tok, int64_t q_stride, float* out, int64_t out_stride,
                            hipStream_t s, void* q8k) {
  if (n_tok <= 0 || n_tok > 65535) return fail(JERO_ERR_TENSOR_BOUNDS, "attention: query batch of 1..65535 tokens");
  AttnParams p = p0;
  p.q_stride = q_stride;
  p.n_tok = n_tok;
  if (attn_flash_ok(p.kv_dtype, p.hd, n_tok, p.group)) {
    if (q8k && !attn_flash_q8k_ok(p.group, p.hd))
      return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: no Q8_K rows for this head group");
    if (!out && !q8k) return fail(JERO_ERR_INVALID_ARGUMENT, "attention: no output");
    if (out && ((reinterpret_cast<uintptr_t>(out) & 15u) || out_stride % 4))
      return fail(JERO_ERR_INVALID_ARGUMENT, "attention: output rows must be 16-byte aligned");
    const int tpg = 4 * (16 / p.group);  // four column sets of 16 / group tokens
    const dim3 grid(unsigned((n_tok + tpg - 1) / tpg), unsigned(p.nkv));
    uint8_t* q = static_cast<uint8_t*>(q8k);
    if (p.hd == 64) hipLaunchKernelGGL(attn_flash_kernel<64>, grid, dim3(kFlashThreads), 0, s, p, out, out_stride, q);
    else hipLaunchKernelGGL(attn_flash_kernel<128>, grid, dim3(kFlashThreads), 0, s, p, out, out_stride, q);
    return check_launch("attention flash");
  }
  if (q8k) return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: Q8_K rows need an f16 ring, head_dim 64 or 128");
  return attention_impl(p, false, attn_splits(p.active + n_tok - 1, p.hd), n_tok, out, out_stride, s);
}

static_assert(int64_t(kMaxSplits) * attn_chunk(64) == JERO_MAX_ATTENTION_POSITIONS, "attention position limit");

int check_attention_shape(int nq, int nkv, int hd, int64_t seq_len) {
  if (nq <= 0 || nkv <= 0 || hd <= 0 || seq_len <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "attention: empty heads or sequence");
  if (nq % nkv) return fail(JERO_ERR_TENSOR_BOUNDS, "attention: n_heads_q not a multiple of n_heads_kv");
  if (hd % 2 || hd > kGenMaxHd)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "attention: head_dim " + std::to_string(hd) +
                                                  " must be even and at most " + std::to_string(kGenMaxHd));
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
