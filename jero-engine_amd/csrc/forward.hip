// forward.hip -- ForwardModel (src/forward.rs:834-1075), the synthetic all-int8 transformer, on gfx950.
//
// Exact integer arithmetic throughout, so the device pass is bit-identical to the reference:
// int32 dot products (v_dot4_i32_i8), requant (:345-350), the integer RMSNorm (:672-699, isqrt
// :747-758), the integer-weighted attention (:702-744), the i8 saturating residual adds (:817-821)
// and the greedy sample (:978-986).
//
// HBM layout: every matrix row-major int8 [n][k] (Matrix::rows, n padded to whole 8-row tiles with
// zero rows), generated on the device from the seed (splitmix / fill_small are integer hashes, so
// no weight bytes cross PCIe); per layer the K and V caches int8 [max_positions][512]; the residual
// rows x, the attention input / output rows and the FFN rows int8 [rows][width].
//
// One forward call over m tokens at start_pos, per layer:
//   qkv   : RMSNorm of x in the prologue (each workgroup normalises the rows it needs in LDS), the
//           three projections in one launch (blockIdx.y picks wq / wk / wv), k and v rows written
//           straight into the caches at start_pos
//   attn  : one workgroup per query row over cache rows 0..=start_pos + r; a one-row step below
//           kAttInMax positions computes it instead in the prologue of every wo workgroup (a
//           launch saved for npos KiB of cache reads per workgroup)
//   wo    : requant, then saturating add into x
//   up    : RMSNorm prologue, requant, relu
//   down  : requant, saturating add into x
// then the head (RMSNorm of the last row, int32 logits).  In evaluate, the next step's first launch
// samples the greedy token from those logits and embeds it in every workgroup's prologue (one
// workgroup also stores the token and the row): the decode loop never waits for the host.  Up to kMvRows rows the projections run on the matvec kernel below
// (one weight row per wave, the token rows in LDS); longer prompts run the int8 MFMA GEMM of
// gemm.hip with the same fused epilogues, after a row RMSNorm kernel.
#include <algorithm>
#include <string>
#include <vector>

#include "forward.h"
#include "jero_common.h"
#include "runtime.h"

namespace jero {

constexpr int kFwdDim = 512, kFwdFfn = 1024, kFwdLayers = 4, kFwdMats = 6;
constexpr int kMvRows = 64;     // token rows of one matvec launch (LDS: m x K bytes, 64 KiB at most)
constexpr int kMvWaves = 4;     // weight rows per matvec workgroup, one per wave
constexpr int kAttChunk = 4096;  // cache positions whose weights one attention pass keeps in LDS
constexpr int64_t kAttInMax = 128;  // one-row steps below this position compute attention in wo
constexpr int64_t kFwdMaxPositions = int64_t(1) << 22;

// splitmix (src/forward.rs:326-332): one SplitMix64 output for state x.
__host__ __device__ __forceinline__ uint64_t splitmix(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Element i of fill_small(seed, .) (src/forward.rs:335-343), in [-8, 7].
__device__ __forceinline__ int small_of(uint64_t seed, uint64_t i) {
  return int(splitmix(seed ^ (i * 0xA24BAED4963EE407ull)) & 0xFu) - 8;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_add_i(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}

// Integer sum over the wave with DPP; the total lands in lane 63.
__device__ __forceinline__ int wave_sum_last_i(int v) {
  v = dpp_add_i<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add_i<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_add_i<0x124, 0xF>(v);  // row_ror:4
  v = dpp_add_i<0x128, 0xF>(v);  // row_ror:8
  v = dpp_add_i<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v = dpp_add_i<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// Integer sum over each 16-lane DPP row, in every lane of the row.
__device__ __forceinline__ int row_sum_i(int v) {
  v = dpp_add_i<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v = dpp_add_i<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v = dpp_add_i<0x124, 0xF>(v);  // row_ror:4
  return dpp_add_i<0x128, 0xF>(v);  // row_ror:8
}

__device__ __forceinline__ int8_t clamp_i8(int v, int lo) { return int8_t(v < lo ? lo : v > 127 ? 127 : v); }

// isqrt (src/forward.rs:747-758) is floor(sqrt(v)); for v < 2^24 the hardware square root is
// within one of it, and one correction step each way makes it exact.
__device__ __forceinline__ uint32_t floor_sqrt_u24(uint32_t v) {
  uint32_t r = uint32_t(__builtin_amdgcn_sqrtf(float(v)));
  if (r * r > v) r--;
  if ((r + 1) * (r + 1) <= v) r++;
  return r;
}

// ForwardExec::rmsnorm (src/forward.rs:672-699) of one 512-byte row held by a wave, 8 bytes per
// lane: rms = max(isqrt(sum v^2 / 512), 1), y = clamp(v * 48 / rms, -127, 127) (division
// truncating toward zero).  |v * 48| <= 6144 and rms <= 128, so the quotient is the high word of
// |v * 48| * ceil(2^32 / rms), exact (division by an invariant integer, Granlund & Montgomery
// 1994: the error term stays below |v * 48| / 2^32 < 1 / rms).
__device__ __forceinline__ void rmsnorm_lane(uint32_t (&v)[2]) {
  int ss = dot4(v[0], v[0], dot4(v[1], v[1], 0));
  ss = __builtin_amdgcn_readlane(wave_sum_last_i(ss), 63);
  const uint32_t rms = max(floor_sqrt_u24(uint32_t(ss) / kFwdDim), 1u);
  const uint32_t mul = rms == 1 ? 0u : 0xFFFFFFFFu / rms + 1u;  // ceil(2^32 / rms) for rms > 1
#pragma unroll
  for (int d = 0; d < 2; d++) {
    uint32_t o = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int x = int(int8_t(byte_of(v[d], b))) * 48;
      const uint32_t ax = uint32_t(x < 0 ? -x : x);
      const int q = int(rms == 1 ? ax : __umulhi(ax, mul));
      o |= uint32_t(uint8_t(clamp_i8(x < 0 ? -q : q, -127))) << (8 * b);
    }
    v[d] = o;
  }
}

// ForwardExec::attention (src/forward.rs:702-744) for one query row at position npos - 1 over
// cache rows 0..npos-1, by the 256 threads of a workgroup: w_t = clamp(q . k_t >> 10, 0, 127) + 1,
// out = sum w_t v_t / sum w_t (int64, truncating).  Positions go in blocks of 64 whose k and v
// loads are all issued at once (one memory round trip per block): sixteen 16-lane groups score
// four keys each (32 bytes per lane) into LDS bytes, then eight groups of 32 threads each weigh
// every eighth value row, 16 columns per thread.  The int32 partials (exact: 128 * 127 * 4096 / 8
// per group) meet in LDS every kAttChunk positions and carry in int64, two columns per thread.
struct AttSmem {
  uint8_t wts[2][64];
  int part[8][kFwdDim];
  int tw[8];
};

__device__ __forceinline__ void attend_row(const int8_t* __restrict__ q, const int8_t* __restrict__ kc,
                                           const int8_t* __restrict__ vc, int64_t npos, int8_t* __restrict__ out,
                                           AttSmem& S) {
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6, g = lane >> 4, sub = lane & 15;
  const uint8_t* qr = reinterpret_cast<const uint8_t*>(q) + sub * 32;
  const u32x4 q0 = ld4(qr), q1 = ld4(qr + 16);
  const int grp = t >> 5, c16 = (t & 31) * 16, kj = wv * 4 + g;
  int64_t acc0 = 0, acc1 = 0, total = 0;
  int buf = 0;
  for (int64_t c0 = 0; c0 < npos; c0 += kAttChunk) {
    const int cn = int(std::min<int64_t>(kAttChunk, npos - c0));
    const uint8_t* kb = reinterpret_cast<const uint8_t*>(kc) + c0 * kFwdDim + sub * 32;
    const uint8_t* vb = reinterpret_cast<const uint8_t*>(vc) + c0 * kFwdDim + c16;
    int a[16] = {}, tw = 0;
    for (int b0 = 0; b0 < cn; b0 += 64) {
      u32x4 k[4][2], v[8];  // positions past the pass read its last row, weighted 0
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint8_t* kr = kb + int64_t(min(b0 + kj + 16 * u, cn - 1)) * kFwdDim;
        k[u][0] = ld4(kr), k[u][1] = ld4(kr + 16);
      }
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = ld4(vb + int64_t(min(b0 + grp + 8 * i, cn - 1)) * kFwdDim);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        int sc = 0;
#pragma unroll
        for (int d = 0; d < 4; d++) sc = dot4(q0[d], k[u][0][d], dot4(q1[d], k[u][1][d], sc));
        sc = row_sum_i(sc);
        const int sh = sc >> 10;
        if (sub == 0) S.wts[buf][kj + 16 * u] = uint8_t((sh < 0 ? 0 : sh > 127 ? 127 : sh) + 1);
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int j = grp + 8 * i;
        const int w = b0 + j < cn ? int(S.wts[buf][j]) : 0;
#pragma unroll
        for (int b = 0; b < 16; b++) a[b] += w * int(int8_t(byte_of(v[i][b >> 2], b & 3)));
        tw += w;
      }
      buf ^= 1;  // the next block's scores go to the other buffer: no second barrier
    }
#pragma unroll
    for (int b = 0; b < 16; b += 4) *reinterpret_cast<int4*>(&S.part[grp][c16 + b]) = int4{a[b], a[b + 1], a[b + 2], a[b + 3]};
    if ((t & 31) == 0) S.tw[grp] = tw;
    __syncthreads();
    int s0 = 0, s1 = 0, st = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int2 pr = *reinterpret_cast<const int2*>(&S.part[i][2 * t]);
      s0 += pr.x, s1 += pr.y, st += S.tw[i];
    }
    acc0 += s0, acc1 += s1, total += st;
    __syncthreads();
  }
  if (total <= INT32_MAX && acc0 >= -INT32_MAX && acc0 <= INT32_MAX && acc1 >= -INT32_MAX && acc1 <= INT32_MAX) {
    out[2 * t] = int8_t(int(acc0) / int(total));  // the same truncating quotient in 32 bits
    out[2 * t + 1] = int8_t(int(acc1) / int(total));
  } else {
    out[2 * t] = int8_t(acc0 / total);
    out[2 * t + 1] = int8_t(acc1 / total);
  }
}

// embed (src/forward.rs:918-926) of one token into a 512-byte row by the calling workgroup:
// fill_small(seed ^ token * 0x9E3779B9) * 8.
__device__ __forceinline__ void embed_row(uint64_t seed, uint32_t token, int8_t* __restrict__ x) {
  const uint64_t s = seed ^ (uint64_t(token) * 0x9E3779B9ull);
  for (int i = threadIdx.x; i < kFwdDim; i += blockDim.x) x[i] = int8_t(small_of(s, uint64_t(i)) * 8);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_min_i(int v) {
  return min(v, __builtin_amdgcn_update_dpp(INT32_MAX, v, CTRL, ROW_MASK, 0xF, false));
}

// Whole-wave integer max / min with DPP, returned to every lane (read from lane 63).
__device__ __forceinline__ int wave_max_i(int v) { return wave_max_i32_dpp(v); }
__device__ __forceinline__ int wave_min_i(int v) {
  v = dpp_min_i<0xB1, 0xF>(v);
  v = dpp_min_i<0x4E, 0xF>(v);
  v = dpp_min_i<0x124, 0xF>(v);
  v = dpp_min_i<0x128, 0xF>(v);
  v = dpp_min_i<0x142, 0xA>(v);
  v = dpp_min_i<0x143, 0xC>(v);
  return __builtin_amdgcn_readlane(v, 63);
}

// ForwardModel::sample (src/forward.rs:978-986) by the calling workgroup of 256 threads: the
// first index of the largest of logits[0, max(vocab, 1)), returned to every thread.  Each thread
// keeps the first maximum of its strided share; per wave the largest value, then the smallest
// index holding it; the four waves meet in LDS.
__device__ __forceinline__ uint32_t sample_block(const int32_t* __restrict__ logits, int64_t vocab) {
  __shared__ int sv[kMvWaves], si[kMvWaves];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int n = int(vocab > 1 ? vocab : 1);
  int bv = INT32_MIN, bi = INT32_MAX;
  for (int i = t; i < n; i += 256) {
    const int v = logits[i];
    if (bi == INT32_MAX || v > bv) bv = v, bi = i;
  }
  const int wmax = wave_max_i(bi == INT32_MAX ? INT32_MIN : bv);
  const int widx = wave_min_i(bi != INT32_MAX && bv == wmax ? bi : INT32_MAX);
  if (lane == 0) sv[wv] = wmax, si[wv] = widx;
  __syncthreads();
  int v = sv[0], idx = si[0];
#pragma unroll
  for (int w = 1; w < kMvWaves; w++)
    if (si[w] != INT32_MAX && (idx == INT32_MAX || sv[w] > v || (sv[w] == v && si[w] < idx))) v = sv[w], idx = si[w];
  return uint32_t(idx);
}

// Up to three projections of one launch (same shape and shift); blockIdx.y picks one.
struct MvProj {
  const int8_t* w;
  void* out;
};
// Where the matvec's input rows come from.
enum { kInRows = 0, kInAttention = 1, kInSample = 2 };
struct MvArgs {
  MvProj p[3];
  const int8_t* x;  // kInRows: token rows [m][K]; kInSample: where workgroup (0, 0) stores the row
  int m, N, shift;
  // kInAttention (m == 1): the attention of q over the npos cache rows, computed by every
  // workgroup for itself
  const int8_t *q, *kc, *vc;
  int64_t npos;
  // kInSample (m == 1): the embedding of the greedy token of the previous step's logits, computed
  // by every workgroup for itself; workgroup (0, 0) also stores the token at *tok and the row at x
  const int32_t* logits;
  int64_t vocab;
  uint32_t* tok;
  uint64_t seed;
};

// out[r][n] = EPI(sum_k x[r][k] w[n][k]) for r < m <= kMvRows: each wave's R weight rows (K / 64
// bytes per lane each) are loaded first, while the input rows are staged in LDS (RMSNorm-ed if
// NORM, K = 512); then one DPP reduction per (weight row, token row), lane 63 writes.  The
// one-row inputs kInAttention and kInSample are computed by each workgroup itself, so that
// attention shares the wo launch and the sample the next step's first launch; every workgroup
// repeats that small step (npos KiB of cache reads, or the scan of the logits) instead of a
// launch boundary and a round trip through memory.
template <int K, int EPI, bool NORM, int IN, int R>
__global__ void __launch_bounds__(kMvWaves * 64) fwd_matvec_kernel(MvArgs a) {
  static_assert(K == kFwdDim || K == kFwdFfn, "row width");
  static_assert(!NORM || K == kFwdDim, "RMSNorm rows are model rows");
  static_assert(IN != kInAttention || (!NORM && K == kFwdDim), "attention rows are model rows");
  static_assert(IN != kInSample || (NORM && K == kFwdDim), "the sampled row feeds a normed projection");
  constexpr int D = K / 256;  // dwords per lane
  extern __shared__ uint32_t xs[];  // [m][K / 4]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * kMvWaves + wv) * R;
  const MvProj p = a.p[blockIdx.y];
  uint32_t w[R][D];
#pragma unroll
  for (int i = 0; i < R; i++) {
    const uint8_t* wr = reinterpret_cast<const uint8_t*>(p.w) + int64_t(min(n0 + i, a.N - 1)) * K + lane * 4 * D;
    if constexpr (D == 2) {
      const u32x2 t = ld2(wr);
      w[i][0] = t[0], w[i][1] = t[1];
    } else {
      const u32x4 t = ld4(wr);
      w[i][0] = t[0], w[i][1] = t[1], w[i][2] = t[2], w[i][3] = t[3];
    }
  }
  if constexpr (IN == kInAttention) {
    __shared__ AttSmem S;
    attend_row(a.q, a.kc, a.vc, a.npos, reinterpret_cast<int8_t*>(xs), S);
  } else if constexpr (IN == kInSample) {
    const uint32_t tok = sample_block(a.logits, a.vocab);
    if (wv == 0) {
      const uint64_t sd = a.seed ^ (uint64_t(tok) * 0x9E3779B9ull);
      uint32_t v[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; e++)
        v[e >> 2] |= uint32_t(uint8_t(int8_t(small_of(sd, uint64_t(lane * 8 + e)) * 8))) << (8 * (e & 3));
      if (blockIdx.x == 0 && blockIdx.y == 0) {
        *reinterpret_cast<u32x2*>(const_cast<int8_t*>(a.x) + lane * 8) = u32x2{v[0], v[1]};
        if (lane == 0) *a.tok = tok;
      }
      rmsnorm_lane(v);
      xs[lane * 2] = v[0], xs[lane * 2 + 1] = v[1];
    }
  } else {
    for (int r = wv; r < a.m; r += kMvWaves) {
      uint32_t v[D];
      const uint8_t* src = reinterpret_cast<const uint8_t*>(a.x) + int64_t(r) * K + lane * 4 * D;
      if constexpr (D == 2) {
        const u32x2 t = ld2(src);
        v[0] = t[0], v[1] = t[1];
      } else {
        const u32x4 t = ld4(src);
        v[0] = t[0], v[1] = t[1], v[2] = t[2], v[3] = t[3];
      }
      if constexpr (NORM) rmsnorm_lane(v);
#pragma unroll
      for (int d = 0; d < D; d++) xs[r * (K / 4) + lane * D + d] = v[d];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < R; i++) {
    const int n = n0 + i;
    if (n >= a.N) return;
    for (int r = 0; r < a.m; r++) {
      int acc = 0;
#pragma unroll
      for (int d = 0; d < D; d++) acc = dot4(w[i][d], xs[r * (K / 4) + lane * D + d], acc);
      acc = wave_sum_last_i(acc);
      if (lane == 63) {
        const int64_t o = int64_t(r) * a.N + n;
        if constexpr (EPI == kI8OutI32) {
          static_cast<int32_t*>(p.out)[o] = acc;
        } else {
          const int q = int(int32_t(uint32_t(acc) + (uint32_t(1) << (a.shift - 1))) >> a.shift);
          const int8_t rq = clamp_i8(q, -127);
          int8_t* dst = static_cast<int8_t*>(p.out) + o;
          if constexpr (EPI == kI8OutRequant) *dst = rq;
          else if constexpr (EPI == kI8OutRequantRelu) *dst = rq < 0 ? int8_t(0) : rq;
          else *dst = clamp_i8(int(*dst) + int(rq), -128);
        }
      }
    }
  }
}

// The greedy token of the head's logits into *tok (sample_block): one workgroup.
__global__ void __launch_bounds__(256) fwd_sample_kernel(const int32_t* __restrict__ logits, int64_t vocab,
                                                         uint32_t* __restrict__ tok) {
  const uint32_t t = sample_block(logits, vocab);
  if (threadIdx.x == 0) *tok = t;
}

// RMSNorm of m rows (the MFMA path's projection input): one wave per row.
__global__ void __launch_bounds__(64) fwd_rmsnorm_rows_kernel(const int8_t* __restrict__ x, int8_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  const u32x2 t = ld2(reinterpret_cast<const uint8_t*>(x) + r * kFwdDim + lane * 8);
  uint32_t v[2] = {t[0], t[1]};
  rmsnorm_lane(v);
  *reinterpret_cast<u32x2*>(out + r * kFwdDim + lane * 8) = u32x2{v[0], v[1]};
}

// Attention of query rows r = blockIdx.x at positions start_pos + r (the prefill's m rows).
__global__ void __launch_bounds__(256) fwd_attention_kernel(const int8_t* __restrict__ q, const int8_t* __restrict__ kc,
                                                            const int8_t* __restrict__ vc, int64_t start_pos,
                                                            int8_t* __restrict__ out) {
  __shared__ AttSmem S;
  const int64_t r = blockIdx.x;
  attend_row(q + r * kFwdDim, kc, vc, start_pos + r + 1, out + r * kFwdDim, S);
}

// embed of token rows tok[0, m), one workgroup per row.
__global__ void __launch_bounds__(256) fwd_embed_kernel(uint64_t seed, const uint32_t* __restrict__ tok,
                                                        int8_t* __restrict__ x) {
  embed_row(seed, tok[blockIdx.x], x + int64_t(blockIdx.x) * kFwdDim);
}

// Matrix::random (src/forward.rs:364-377): fill_small(seed, n k) then zero padding rows.
__global__ void __launch_bounds__(256) fwd_fill_kernel(uint64_t seed, int64_t valid, int64_t total,
                                                       int8_t* __restrict__ w) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x)
    w[i] = i < valid ? int8_t(small_of(seed, uint64_t(i))) : int8_t(0);
}

}  // namespace jero

using namespace jero;

struct jero_forward_model {
  int device = -1;
  uint64_t seed = 0;
  int64_t vocab = 0, head_rows = 0, cap = 0, len = 0;
  int8_t* w[kFwdLayers][kFwdMats] = {};
  int8_t* head = nullptr;
  int8_t* kc[kFwdLayers] = {};
  int8_t* vc[kFwdLayers] = {};
  int8_t *x = nullptr, *h = nullptr, *q = nullptr, *att = nullptr, *up = nullptr;  // [cap] rows
  int32_t* logits = nullptr;                                                        // [head_rows]
  uint32_t* tokens = nullptr;  // [cap]: the call's token rows, or evaluate's generated tokens
  std::vector<void*> owned;
  // evaluate's decode steps as a HIP graph for one (prompt length, max_tokens), replayed on gs
  hipStream_t gs = nullptr;
  hipGraphExec_t graph = nullptr;
  int64_t graph_n = -1, graph_max = -1;
};

namespace {

const int64_t kMatRows[kFwdMats] = {kFwdDim, kFwdDim, kFwdDim, kFwdDim, kFwdFfn, kFwdDim};
const int64_t kMatCols[kFwdMats] = {kFwdDim, kFwdDim, kFwdDim, kFwdDim, kFwdDim, kFwdFfn};
int mat_shift(int which) { return which == 5 ? 7 : 6; }

int fwd_alloc(jero_forward_model* f, size_t bytes, void** p) {
  if (hipMalloc(p, bytes < 256 ? 256 : bytes) != hipSuccess)
    return fail(JERO_ERR_INSUFFICIENT_MEMORY, "forward_model: hipMalloc of " + std::to_string(bytes) + " bytes failed");
  f->owned.push_back(*p);
  return JERO_OK;
}

void fwd_release(jero_forward_model* f) {
  if (f->graph) (void)hipGraphExecDestroy(f->graph);
  if (f->gs) (void)hipStreamDestroy(f->gs);
  for (void* p : f->owned) (void)hipFree(p);
  delete f;
}

int gen_matrix(uint64_t seed, int64_t n, int64_t k, int8_t* dst) {
  const int64_t total = (n + 7) / 8 * 8 * k;
  hipLaunchKernelGGL(fwd_fill_kernel, dim3(unsigned(std::min<int64_t>((total + 255) / 256, 4096))), dim3(256), 0, 0,
                     seed, n * k, total, dst);
  return check_launch("forward_model weights");
}

// m token rows (m <= kMvRows) through up to three same-shaped projections, R weight rows a wave.
template <int K, int EPI, bool NORM, int IN = kInRows, int R = 1>
int mv(const MvArgs& a, int n_proj, hipStream_t s) {
  const int per_wg = kMvWaves * R;
  const dim3 grid(unsigned((a.N + per_wg - 1) / per_wg), unsigned(n_proj));
  hipLaunchKernelGGL((fwd_matvec_kernel<K, EPI, NORM, IN, R>), grid, dim3(kMvWaves * 64), size_t(a.m) * K, s, a);
  return check_launch("forward matvec");
}

MvArgs mv_args(const int8_t* x, int64_t m, int64_t N, int shift) {
  MvArgs a{};
  a.x = x;
  a.m = int(m);
  a.N = int(N);
  a.shift = shift;
  return a;
}

int embed_tokens(jero_forward_model* f, int64_t m, hipStream_t s) {
  hipLaunchKernelGGL(fwd_embed_kernel, dim3(unsigned(m)), dim3(256), 0, s, f->seed, f->tokens, f->x);
  return check_launch("forward embed");
}

// ForwardModel::forward (src/forward.rs:930-976) over m token rows whose embeddings are in f->x,
// or, with sampled set (m == 1), over the greedy token of the previous step's logits in f->logits
// (ForwardModel::sample, src/forward.rs:978-986), which goes to *sampled and its embedding to f->x.
int forward_rows(jero_forward_model* f, int64_t m, int64_t start_pos, int32_t* logits, uint32_t* sampled,
                 hipStream_t s) {
  const int64_t D = kFwdDim;
  int rc;
  const bool small = m <= kMvRows;
  for (int l = 0; l < kFwdLayers; l++) {
    int8_t* const* W = f->w[l];
    int8_t* kdst = f->kc[l] + start_pos * D;
    int8_t* vdst = f->vc[l] + start_pos * D;
    if (small) {
      MvArgs a = mv_args(f->x, m, D, 6);
      a.p[0] = {W[0], f->q};
      a.p[1] = {W[1], kdst};
      a.p[2] = {W[2], vdst};
      if (l == 0 && sampled) {
        a.logits = f->logits, a.vocab = f->vocab, a.tok = sampled, a.seed = f->seed;
        rc = mv<kFwdDim, kI8OutRequant, true, kInSample>(a, 3, s);
      } else {
        rc = mv<kFwdDim, kI8OutRequant, true>(a, 3, s);
      }
      if (rc) return rc;
    } else {
      hipLaunchKernelGGL(fwd_rmsnorm_rows_kernel, dim3(unsigned(m)), dim3(64), 0, s, f->x, f->h);
      if ((rc = check_launch("forward rmsnorm")) ||
          (rc = launch_gemm_i8_epi(kI8OutRequant, f->h, m, D, W[0], D, f->q, 6, s)) ||
          (rc = launch_gemm_i8_epi(kI8OutRequant, f->h, m, D, W[1], D, kdst, 6, s)) ||
          (rc = launch_gemm_i8_epi(kI8OutRequant, f->h, m, D, W[2], D, vdst, 6, s)))
        return rc;
    }
    const bool att_in = m == 1 && start_pos < kAttInMax;
    if (!att_in) {
      hipLaunchKernelGGL(fwd_attention_kernel, dim3(unsigned(m)), dim3(256), 0, s, f->q, f->kc[l], f->vc[l],
                         start_pos, f->att);
      if ((rc = check_launch("forward attention"))) return rc;
    }
    if (small) {
      MvArgs a = mv_args(f->att, m, D, 6);
      a.p[0] = {W[3], f->x};
      if (att_in) {
        a.q = f->q, a.kc = f->kc[l], a.vc = f->vc[l], a.npos = start_pos + 1;
        rc = mv<kFwdDim, kI8OutRequantSatAdd, false, kInAttention>(a, 1, s);
      } else {
        rc = mv<kFwdDim, kI8OutRequantSatAdd, false>(a, 1, s);
      }
      if (rc) return rc;
      a = mv_args(f->x, m, kFwdFfn, 6);
      a.p[0] = {W[4], f->up};
      if ((rc = mv<kFwdDim, kI8OutRequantRelu, true>(a, 1, s))) return rc;
      a = mv_args(f->up, m, D, 7);
      a.p[0] = {W[5], f->x};
      if ((rc = mv<kFwdFfn, kI8OutRequantSatAdd, false>(a, 1, s))) return rc;
    } else {
      if ((rc = launch_gemm_i8_epi(kI8OutRequantSatAdd, f->att, m, D, W[3], D, f->x, 6, s))) return rc;
      hipLaunchKernelGGL(fwd_rmsnorm_rows_kernel, dim3(unsigned(m)), dim3(64), 0, s, f->x, f->h);
      if ((rc = check_launch("forward rmsnorm")) ||
          (rc = launch_gemm_i8_epi(kI8OutRequantRelu, f->h, m, D, W[4], kFwdFfn, f->up, 6, s)) ||
          (rc = launch_gemm_i8_epi(kI8OutRequantSatAdd, f->up, m, kFwdFfn, W[5], D, f->x, 7, s)))
        return rc;
    }
  }
  MvArgs a = mv_args(f->x + (m - 1) * D, 1, f->head_rows, 0);
  a.p[0] = {f->head, logits};
  return mv<kFwdDim, kI8OutI32, true>(a, 1, s);
}

// Records evaluate's decode steps for a prompt of n tokens and max_tokens >= 1 generated ones into
// f->graph: step i (1 <= i < max_tokens) samples tokens[i - 1] from the previous logits in its
// first launch and runs it at position n + i - 1; then the last sample into tokens[max_tokens - 1].
int capture_decode(jero_forward_model* f, int64_t n, int64_t max_tokens) {
  if (f->graph) {
    (void)hipGraphExecDestroy(f->graph);
    f->graph = nullptr;
  }
  f->graph_n = f->graph_max = -1;
  int rc = check_hip(hipStreamBeginCapture(f->gs, hipStreamCaptureModeThreadLocal), "forward capture");
  if (rc) return rc;
  uint32_t* const toks = f->tokens;
  for (int64_t i = 1; i < max_tokens && !rc; i++) rc = forward_rows(f, 1, n + i - 1, f->logits, toks + i - 1, f->gs);
  if (!rc) {
    hipLaunchKernelGGL(fwd_sample_kernel, dim3(1), dim3(256), 0, f->gs, f->logits, f->vocab, toks + max_tokens - 1);
    rc = check_launch("forward sample");
  }
  hipGraph_t g = nullptr;
  const int rc_end = check_hip(hipStreamEndCapture(f->gs, &g), "forward capture end");
  if (!rc) rc = rc_end;
  if (!rc) rc = check_hip(hipGraphInstantiate(&f->graph, g, nullptr, nullptr, 0), "forward graph instantiate");
  if (g) (void)hipGraphDestroy(g);
  if (rc) {
    f->graph = nullptr;
    return rc;
  }
  f->graph_n = n, f->graph_max = max_tokens;
  return JERO_OK;
}

int check_model(const jero_forward_model* f, const char* who) {
  if (!f) return fail(JERO_ERR_INVALID_ARGUMENT, std::string(who) + ": null model");
  int dev = -1;
  int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (rc) return rc;
  if (dev != f->device)
    return fail(JERO_ERR_INVALID_ARGUMENT, std::string(who) + ": the model lives on device " +
                                               std::to_string(f->device) + ", not the current one");
  return JERO_OK;
}

}  // namespace

extern "C" int jero_hip_forward_model_create(uint64_t seed, int64_t vocab, int64_t max_positions,
                                             jero_forward_model** out) {
  if (!out) return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_create: null pointer");
  *out = nullptr;
  if (vocab < 0 || vocab > (int64_t(1) << 24))
    return fail(JERO_ERR_TENSOR_BOUNDS, "forward_model_create: vocab must be in 0..2^24");
  if (max_positions < 1 || max_positions > kFwdMaxPositions)
    return fail(JERO_ERR_TENSOR_BOUNDS, "forward_model_create: max_positions must be in 1..2^22");
  auto* f = new jero_forward_model();
  int rc = check_hip(hipGetDevice(&f->device), "hipGetDevice");
  if (rc) {
    delete f;
    return rc;
  }
  f->seed = seed;
  f->vocab = vocab;
  f->cap = max_positions;
  f->head_rows = (std::max<int64_t>(vocab, 1) + 7) / 8 * 8;
  const size_t cap = size_t(max_positions);
  void* p;
  for (int l = 0; l < kFwdLayers && !rc; l++) {
    for (int j = 0; j < kFwdMats && !rc; j++)
      if (!(rc = fwd_alloc(f, size_t(kMatRows[j] * kMatCols[j]), &p))) f->w[l][j] = static_cast<int8_t*>(p);
    if (!rc && !(rc = fwd_alloc(f, cap * kFwdDim, &p))) f->kc[l] = static_cast<int8_t*>(p);
    if (!rc && !(rc = fwd_alloc(f, cap * kFwdDim, &p))) f->vc[l] = static_cast<int8_t*>(p);
  }
  int8_t** rows[5] = {&f->x, &f->h, &f->q, &f->att, &f->up};
  for (int i = 0; i < 5 && !rc; i++)
    if (!(rc = fwd_alloc(f, cap * (i == 4 ? kFwdFfn : kFwdDim), &p))) *rows[i] = static_cast<int8_t*>(p);
  if (!rc && !(rc = fwd_alloc(f, size_t(f->head_rows) * kFwdDim, &p))) f->head = static_cast<int8_t*>(p);
  if (!rc && !(rc = fwd_alloc(f, size_t(f->head_rows) * sizeof(int32_t), &p))) f->logits = static_cast<int32_t*>(p);
  if (!rc && !(rc = fwd_alloc(f, cap * sizeof(uint32_t), &p))) f->tokens = static_cast<uint32_t*>(p);
  // ForwardModel::new (src/forward.rs:879-903): layer l's matrices from splitmix(seed ^ (16 l + j)),
  // j = 1..6 for wq wk wv wo up down; the head from splitmix(seed ^ 0xFFFF), max(vocab, 1) rows.
  for (int l = 0; l < kFwdLayers && !rc; l++)
    for (int j = 0; j < kFwdMats && !rc; j++)
      rc = gen_matrix(splitmix(seed ^ (uint64_t(l) * 16 + uint64_t(j) + 1)), kMatRows[j], kMatCols[j], f->w[l][j]);
  if (!rc) rc = gen_matrix(splitmix(seed ^ 0xFFFFull), std::max<int64_t>(vocab, 1), kFwdDim, f->head);
  if (!rc) rc = check_hip(hipDeviceSynchronize(), "forward_model_create");
  if (rc) {
    fwd_release(f);
    return rc;
  }
  *out = f;
  return JERO_OK;
}

extern "C" int jero_hip_forward_model_destroy(jero_forward_model* f) {
  if (!f) return JERO_OK;
  (void)hipDeviceSynchronize();
  fwd_release(f);
  return JERO_OK;
}

extern "C" int64_t jero_hip_forward_model_head_rows(const jero_forward_model* f) { return f ? f->head_rows : -1; }

extern "C" int64_t jero_hip_forward_model_positions(const jero_forward_model* f) { return f ? f->len : -1; }

extern "C" int jero_hip_forward_model_reset(jero_forward_model* f) {
  if (!f) return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_reset: null model");
  f->len = 0;
  return JERO_OK;
}

extern "C" int jero_hip_forward_model_weight(const jero_forward_model* f, int layer, int which, const int8_t** w_dev,
                                             int64_t* n, int64_t* k, int* shift) {
  if (!f || !w_dev || !n || !k || !shift) return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_weight: null pointer");
  if (layer == -1) {
    *w_dev = f->head, *n = f->head_rows, *k = kFwdDim, *shift = 6;
    return JERO_OK;
  }
  if (layer < 0 || layer >= kFwdLayers || which < 0 || which >= kFwdMats)
    return fail(JERO_ERR_TENSOR_BOUNDS, "forward_model_weight: layer must be -1 (head) or 0..3, which 0..5");
  *w_dev = f->w[layer][which], *n = kMatRows[which], *k = kMatCols[which], *shift = mat_shift(which);
  return JERO_OK;
}

extern "C" int jero_hip_forward_model_forward(jero_forward_model* f, const uint32_t* tokens, int64_t m,
                                              int64_t start_pos, int32_t* logits_dev, void* stream) {
  int rc = check_model(f, "forward_model_forward");
  if (rc) return rc;
  if (!tokens || !logits_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_forward: null pointer");
  if (m < 1) return fail(JERO_ERR_TENSOR_BOUNDS, "forward_model_forward: no tokens");
  if (start_pos != f->len)
    return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_forward: start_pos " + std::to_string(start_pos) +
                                               " is not the cached position count " + std::to_string(f->len));
  if (m > f->cap - start_pos)
    return fail(JERO_ERR_CONTEXT_LENGTH_EXCEEDED, "forward_model_forward: " + std::to_string(start_pos + m) +
                                                      " positions exceed the capacity " + std::to_string(f->cap));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if ((rc = check_hip(hipMemcpyAsync(f->tokens, tokens, size_t(m) * sizeof(uint32_t), hipMemcpyHostToDevice, s),
                      "forward tokens")) ||
      (rc = embed_tokens(f, m, s)) || (rc = forward_rows(f, m, start_pos, logits_dev, nullptr, s)))
    return rc;
  f->len = start_pos + m;
  return JERO_OK;
}

extern "C" int jero_hip_forward_model_evaluate(jero_forward_model* f, const uint32_t* prompt, int64_t n,
                                               int64_t max_tokens, uint32_t* generated, float* timing_ms,
                                               void* stream) {
  int rc = check_model(f, "forward_model_evaluate");
  if (rc) return rc;
  if (!prompt || (max_tokens > 0 && !generated))
    return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_evaluate: null pointer");
  if (n < 1) return fail(JERO_ERR_CAPABILITY_MISMATCH, "forward_model_evaluate: prompt token sequence cannot be empty");
  if (max_tokens < 0) return fail(JERO_ERR_INVALID_ARGUMENT, "forward_model_evaluate: negative max_tokens");
  const int64_t need = n + (max_tokens > 0 ? max_tokens - 1 : 0);
  if (n > f->cap || need > f->cap)
    return fail(JERO_ERR_CONTEXT_LENGTH_EXCEEDED, "forward_model_evaluate: " + std::to_string(need) +
                                                      " positions exceed the capacity " + std::to_string(f->cap));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipEvent_t ev[3] = {};
  for (int i = 0; i < 3 && !rc; i++) rc = check_hip(hipEventCreate(&ev[i]), "forward_model_evaluate events");
  f->len = 0;
  // Prefill: the prompt rows, then its sample lands in tokens[0]; decode step i runs tokens[i-1]
  // at position n + i - 1 and samples into tokens[i] (evaluate, src/forward.rs:1016-1038).
  if (!rc) rc = check_hip(hipMemcpyAsync(f->tokens, prompt, size_t(n) * sizeof(uint32_t), hipMemcpyHostToDevice, s),
                          "forward prompt");
  if (!rc) rc = check_hip(hipEventRecord(ev[0], s), "event");
  if (!rc) rc = embed_tokens(f, n, s);
  uint32_t* const toks = f->tokens;
  if (!rc) rc = forward_rows(f, n, 0, f->logits, nullptr, s);
  if (!rc) rc = check_hip(hipEventRecord(ev[1], s), "event");
  // The decode steps run as one graph on the model's stream gs, after the prefill: the steps are
  // the same launches for every evaluate of this (n, max_tokens), so they are captured once and
  // replayed (the host then enqueues one graph instead of ~17 launches per token).
  if (!rc && !f->gs) rc = check_hip(hipStreamCreateWithFlags(&f->gs, hipStreamNonBlocking), "forward stream");
  if (!rc) rc = check_hip(hipStreamWaitEvent(f->gs, ev[1], 0), "forward stream order");
  if (!rc && max_tokens > 0 && (f->graph_n != n || f->graph_max != max_tokens || !f->graph))
    rc = capture_decode(f, n, max_tokens);
  if (!rc && max_tokens > 0) rc = check_hip(hipGraphLaunch(f->graph, f->gs), "forward decode graph");
  if (!rc) rc = check_hip(hipEventRecord(ev[2], f->gs), "event");
  if (!rc && max_tokens > 0)
    rc = check_hip(hipMemcpyAsync(generated, toks, size_t(max_tokens) * sizeof(uint32_t), hipMemcpyDeviceToHost,
                                  f->gs),
                   "forward generated");
  if (!rc) rc = check_hip(hipStreamSynchronize(f->gs), "forward_model_evaluate");
  if (!rc && timing_ms) {
    rc = check_hip(hipEventElapsedTime(&timing_ms[0], ev[0], ev[1]), "event time");
    if (!rc) rc = check_hip(hipEventElapsedTime(&timing_ms[1], ev[1], ev[2]), "event time");
  }
  for (hipEvent_t e : ev)
    if (e) (void)hipEventDestroy(e);
  if (!rc) f->len = need;
  return rc;
}
