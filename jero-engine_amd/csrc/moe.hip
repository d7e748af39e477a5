// moe.hip -- routed expert FFN (Qwen3-MoE) on gfx950.
//
// Replaces dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) for router logits already
// computed, with select_top_k_experts (src/gemma.rs:362-442), slice_or_lookup_expert on the
// stacked [hidden, ffn, n_experts] tensors (:729-746) and run_single_swiglu_expert (:748-771).
// The reference loops token by token and expert by expert; here the work is regrouped by
// expert so that each selected expert's weights stream from HBM once for all of its tokens:
//   1. route:  per token (one wave) f32 softmax over all experts, top-k by (logit desc, index
//              asc) with non-finite logits ranked last, renormalised weights; the T hidden
//              vectors are quantized to Q8_K alongside.
//   2. group:  the (token, slot) pairs are grouped by expert in ascending (token, slot) order and
//              the ascending list of active experts is written (one workgroup).  Few tokens run
//              1 and 2 in one workgroup; many spread 1 over the GPU and group in a second launch.
//   3. gate/up: one lane group per weight row; gate row f and up row f of an active expert
//              sit side by side in one wave, loaded once, and are dotted with every token routed
//              to that expert; act = silu(g) * u.
//   4. quantize act rows to Q8_K.
//   5. down:   one lane group per row of the expert's down matrix, dotted with each of its
//              tokens' act rows -> per-(token, slot) outputs.
//   6. combine y[t] = sum_j w[t][j] * out[t][j], j ascending as the reference accumulates.
// All integer partial sums are exact; every output element is reduced in a fixed order.
#include "moe.h"

#include <algorithm>
#include <type_traits>

#include "gemv_dot.h"
#include "quantize.h"
#include "runtime.h"

namespace jero {

constexpr int kRouteThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 16;
constexpr int kRouteLdsPairs = 8192;  // (token, slot) pairs grouped from LDS (keys hold 13 bits)
constexpr int kGroupSortPairs = 1024;  // above this many pairs, grouping sorts instead of ranking

// Activations are quantized in 256-element groups, one wave per group (four consecutive elements
// per lane), to the format of the weights they meet: one Q8_K block (292 bytes) for the K-quants,
// eight ACT_Q8 blocks (288 bytes) for Q8_0 / Q4_0.  A row keeps the Q8_K row's stride either way.
__host__ __device__ constexpr bool act_is_q8(int f) { return f == JERO_Q8_0 || f == JERO_Q4_0; }
__host__ __device__ constexpr int act_group_bytes(bool aq8) { return aq8 ? 288 : 292; }
__device__ __forceinline__ void act_group_wave(const float e[4], int lane, uint8_t* ob, bool aq8) {
  if (aq8) actq8_blocks_wave(e, lane, ob);
  else q8k_block_wave(e, lane, ob);
}

// Routes token t in one wave (PER = expert columns per lane, E <= 64 * PER): f32 softmax over
// all experts, top-k by (logit desc, index asc) with non-finite logits last, renormalised
// weights -> sel_idx / sel_w (and s_sel when given).
template <int PER>
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int t, int E, int k,
                                            int32_t* __restrict__ sel_idx, float* __restrict__ sel_w, int* s_sel) {
  const int lane = threadIdx.x & 63;
  const float* lt = logits + int64_t(t) * E;
  float key[PER], prob[PER];
  // all loads first, unconditional (clamped), then branch-free selects: a branch on a loaded
  // value makes the load wait by itself
  float lv[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) lv[i] = lt[min(lane + 64 * i, E - 1)];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const bool fin = (lane + 64 * i < E) & (fabsf(lv[i]) <= 3.402823466e38f);  // finite, not NaN
    key[i] = fin ? lv[i] : -INFINITY;
    mx = fmaxf(mx, key[i]);
  }
  mx = wave_max_dpp(mx);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const bool fin = lane + 64 * i < E && key[i] != -INFINITY;
    prob[i] = (fin && isfinite(mx)) ? expf(key[i] - mx) : 0.f;
    sum += prob[i];
  }
  sum = wave_sum_dpp(sum);
  const bool ok = sum > 0.f && isfinite(sum);
#pragma unroll
  for (int i = 0; i < PER; i++) prob[i] = ok ? prob[i] / sum : 1.0f / float(E);
  // top-k rounds: the wave-wide best remaining key (DPP max), then its lowest expert index
  // (the first column i, then the lowest lane, whose entry holds it); taken entries drop out.
  // Keys are compared as f32::total_cmp orders them (src/gemma.rs:417), i.e. as signed integers
  // of the sign-folded bits, so +0.0 ranks above -0.0.
  int tkey[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) tkey[i] = total_order_key(key[i]);
  float ssum = 0.f;
  int my_i = 0;  // lane j keeps selection j
  float my_w = 0.f;
  bool taken[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) taken[i] = !(lane + 64 * i < E);
  for (int j = 0; j < k; j++) {
    int lb = int(0x80000000u);
#pragma unroll
    for (int i = 0; i < PER; i++) lb = taken[i] ? lb : max(lb, tkey[i]);
    const int best = wave_max_i32_dpp(lb);
    int bi = -1;
    float bp = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const uint64_t hit = __ballot(!taken[i] && tkey[i] == best);
      if (bi < 0 && hit != 0) {
        const int src = __builtin_ctzll(hit);
        bi = src + 64 * i;
        bp = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, prob[i]), src));
        taken[i] = taken[i] || lane == src;
      }
    }
    my_i = lane == j ? bi : my_i;
    my_w = lane == j ? bp : my_w;
    ssum += bp;
  }
  const bool sok = ssum > 0.f && isfinite(ssum);
  if (lane < k) {
    sel_idx[t * k + lane] = my_i;
    sel_w[t * k + lane] = sok ? my_w / ssum : 1.0f / float(k);
    if (s_sel && t * k + lane < kRouteLdsPairs) s_sel[t * k + lane] = my_i;
  }
}

// LDS of the grouping step.
struct GroupLds {
  int count[kMaxExperts];
  int off[kMaxExperts];
  int fill[kMaxExperts];
  int active[kMaxExperts];
  int poff[kMaxExperts];  // first pass of each expert (pass descriptors)
  int wsum[3 * (kRouteThreads / 64)];
  int n_active;
  __attribute__((aligned(16))) int sel[kRouteLdsPairs + 4];  // the selections, when they fit
  int list[kRouteLdsPairs];                                   // pairs grouped by expert, atomic order
  int entry[kRouteLdsPairs];                                  // the final list (descriptors' tokens)
};

// Zeroes the per-expert counters (before a barrier that precedes group_pairs).
__device__ __forceinline__ void group_init(GroupLds& g, int E) {
  for (int e = threadIdx.x; e < E; e += kRouteThreads) {
    g.count[e] = 0;
    g.fill[e] = 0;
  }
}

// Groups the n (token, slot) pairs by expert, in ascending pair order within an expert, and
// writes the ascending list of active experts; with lists.pass, also the pass descriptors, their
// number and zeroed work counters (n must then fit in LDS).  The selections are in g.sel when n
// fits, else in sel_idx.  One workgroup of kRouteThreads threads; starts and ends with a barrier.
__device__ void group_pairs(GroupLds& g, const int32_t* __restrict__ sel_idx, int n, int E, int k, MoeLists lists) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = kRouteThreads / 64;
  const int PT = lists.pass_tokens == kMoePassTokensWide ? kMoePassTokensWide : kMoePassTokens;
  if (threadIdx.x < 4 && n + int(threadIdx.x) < kRouteLdsPairs + 4) g.sel[n + threadIdx.x] = -1;
  __syncthreads();
  const bool in_lds = n <= kRouteLdsPairs;
  for (int i = threadIdx.x; i < n; i += kRouteThreads) atomicAdd(&g.count[in_lds ? g.sel[i] : sel_idx[i]], 1);
  __syncthreads();
  {
    // exclusive scans of the counts (offsets), of the active flags (active list) and of the
    // pass counts, one thread per expert: wave scans, then the 16 wave totals
    const int e = threadIdx.x;
    const int c = e < E ? g.count[e] : 0, f = c > 0 ? 1 : 0, np = (c + PT - 1) / PT;
    int ic = c, jf = f, kp = np;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int oc = __shfl_up(ic, off, kWave), of = __shfl_up(jf, off, kWave), op = __shfl_up(kp, off, kWave);
      if (lane >= off) {
        ic += oc;
        jf += of;
        kp += op;
      }
    }
    if (lane == 63) {
      g.wsum[wv] = ic;
      g.wsum[nw + wv] = jf;
      g.wsum[2 * nw + wv] = kp;
    }
    __syncthreads();
    int bc = 0, bf = 0, bp = 0;
    for (int w = 0; w < wv; w++) {
      bc += g.wsum[w];
      bf += g.wsum[nw + w];
      bp += g.wsum[2 * nw + w];
    }
    if (e < E) {
      const int off_e = bc + ic - c;
      g.off[e] = off_e;
      g.poff[e] = bp + kp - np;
      lists.offset[e] = off_e;
      if (f) {
        lists.active[bf + jf - 1] = e;
        g.active[bf + jf - 1] = e;
      }
      if (e == E - 1) {
        lists.offset[E] = off_e + c;
        *lists.n_active = bf + jf;
        g.n_active = bf + jf;
        if (lists.pass) {
          lists.ctr[0] = bp + kp;
          lists.ctr[kMoeCtrGateUp] = 0;
          lists.ctr[kMoeCtrDown] = 0;
        }
      }
    }
  }
  __syncthreads();
  const int nt = n / k, words = (nt + 31) / 32;  // tokens (pairs t * k + j) and their bitmask words
  if (in_lds && n > kGroupSortPairs && n % k == 0 && E * words <= kRouteLdsPairs / 2) {
    // many pairs: token t's k selections are distinct experts, so pair (t, j)'s rank among its
    // expert's pairs is the number of tokens before t that selected that expert; from per-expert
    // token bitmasks and the prefix counts of their words (both in g.list), in one pass
    uint32_t* bits = reinterpret_cast<uint32_t*>(g.list);
    int* pre = g.list + E * words;
    for (int i = threadIdx.x; i < E * words; i += kRouteThreads) bits[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kRouteThreads) {
      const int t = i / k;
      atomicOr(&bits[g.sel[i] * words + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += kRouteThreads) {
      int run = 0;
      for (int w = 0; w < words; w++) {
        pre[e * words + w] = run;
        run += __popc(bits[e * words + w]);
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kRouteThreads) {
      const int t = i / k, e = g.sel[i], wd = e * words + (t >> 5);
      const int q = g.off[e] + pre[wd] + __popc(bits[wd] & ((1u << (t & 31)) - 1u));
      lists.entry[q] = i;
      lists.inv[i] = q;
      g.entry[q] = i;
    }
  } else if (in_lds && n > kGroupSortPairs) {
    // many pairs: sort the unique keys (expert << 13 | pair) ascending in LDS (bitonic network,
    // padded to a power of two): expert e's pairs land at [off[e], off[e] + count[e]) in
    // ascending pair order, the placement below without its per-pair scan of the segment
    int P = 1;
    while (P < n) P <<= 1;
    for (int i = threadIdx.x; i < P; i += kRouteThreads) g.list[i] = i < n ? (g.sel[i] << 13) | i : 0x7FFFFFFF;
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = threadIdx.x; t < P / 2; t += kRouteThreads) {
          const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
          const int a = g.list[lo], b = g.list[hi];
          if ((a > b) == ((lo & size) == 0)) {
            g.list[lo] = b;
            g.list[hi] = a;
          }
        }
        __syncthreads();
      }
    }
    for (int q = threadIdx.x; q < n; q += kRouteThreads) {
      const int i = g.list[q] & 8191;
      lists.entry[q] = i;
      lists.inv[i] = q;
      g.entry[q] = i;
    }
  } else if (in_lds) {
    // stable placement in two parallel steps: each pair takes a slot of its expert's segment by
    // an LDS atomic, then its final place is its rank among the segment's pairs (pairs ascend)
    for (int i = threadIdx.x; i < n; i += kRouteThreads) {
      const int e = g.sel[i];
      g.list[g.off[e] + atomicAdd(&g.fill[e], 1)] = i;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kRouteThreads) {
      const int e = g.sel[i], o = g.off[e], c = g.count[e];
      int r = 0;
      for (int q = 0; q < c; q++) r += g.list[o + q] < i ? 1 : 0;
      lists.entry[o + r] = i;
      lists.inv[i] = o + r;
      g.entry[o + r] = i;
    }
  }
  if (in_lds) {
    if (lists.pass) {
      // per pass of an expert: expert, first list position, count, and its tokens (the last
      // one repeated past the count); one thread per pass, whose expert is the last one with
      // poff[e] <= pass (an expert with no pairs has the poff of the next, so is passed over)
      __syncthreads();
      const int passes = g.poff[E - 1] + (g.count[E - 1] + PT - 1) / PT;
      for (int pi = threadIdx.x; pi < passes; pi += kRouteThreads) {
        int lo = 0, hi = E - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (g.poff[mid] <= pi) lo = mid;
          else hi = mid - 1;
        }
        const int e = lo, o = g.off[e], b = (pi - g.poff[e]) * PT, m = min(PT, g.count[e] - b);
        int32_t* pd = lists.pass + int64_t(pi) * (4 + PT);
        pd[0] = e;
        pd[1] = o + b;
        pd[2] = m;
        pd[3] = 0;
        for (int j = 0; j < PT; j++) pd[4 + j] = g.entry[o + b + min(j, m - 1)] / k;
      }
    }
  } else {
    // more pairs than LDS holds: thread e walks the selections in order and keeps those routed to e
    for (int e = threadIdx.x; e < E; e += kRouteThreads) {
      int pos = g.off[e];
      for (int i = 0; i < n; i++) {
        if (sel_idx[i] == e) {
          lists.entry[pos] = i;
          lists.inv[i] = pos;
          pos++;
        }
      }
    }
  }
}

// Few tokens: one workgroup quantizes the hidden vectors (when xq is given; one wave per
// 256-element group; aq8: the ACT_Q8 blocks of Q8_0 / Q4_0 gate/up weights, else Q8_K), routes
// (one wave per token) and groups.
template <int PER>
__global__ void __launch_bounds__(kRouteThreads) moe_route_kernel(const float* __restrict__ logits, int T, int E,
                                                                  int k, int32_t* __restrict__ sel_idx,
                                                                  float* __restrict__ sel_w, MoeLists lists,
                                                                  const float* __restrict__ x, int H,
                                                                  uint8_t* __restrict__ xq, int64_t xq_rb, int aq8) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = kRouteThreads / 64;
  __shared__ GroupLds g;
  if (xq) {
    const int bpr = H / 256, nblk = T * bpr, gb = act_group_bytes(aq8);
    for (int blk = wv; blk < nblk; blk += nw) {
      const int t = blk / bpr, j = blk - t * bpr;
      const float4 v = reinterpret_cast<const float4*>(x + int64_t(t) * H + int64_t(j) * 256)[lane];
      const float e[4] = {v.x, v.y, v.z, v.w};
      act_group_wave(e, lane, xq + int64_t(t) * xq_rb + int64_t(j) * gb, aq8);
    }
  }
  group_init(g, E);
  for (int t = wv; t < T; t += nw) route_token<PER>(logits, t, E, k, sel_idx, sel_w, g.sel);
  group_pairs(g, sel_idx, T * k, E, k, lists);
}

// Many tokens, first step: workgroups [0, n_quant_wg) quantize the hidden vectors (one wave per
// 256-element group, in the format aq8 names as above), the others route one token per wave.  Spreading the routing over
// many CUs matters: a single workgroup is bound by one CU's VALU issue at a few dozen tokens.
template <int PER>
__global__ void __launch_bounds__(256) moe_prep_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                       int32_t* __restrict__ sel_idx, float* __restrict__ sel_w,
                                                       const float* __restrict__ x, int H, uint8_t* __restrict__ xq,
                                                       int64_t xq_rb, int n_quant_wg, int aq8) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (int(blockIdx.x) < n_quant_wg) {
    const int bpr = H / 256, nblk = T * bpr, gb = act_group_bytes(aq8);
    for (int blk = int(blockIdx.x) * 4 + wv; blk < nblk; blk += n_quant_wg * 4) {
      const int t = blk / bpr, j = blk - t * bpr;
      const float4 v = reinterpret_cast<const float4*>(x + int64_t(t) * H + int64_t(j) * 256)[lane];
      const float e[4] = {v.x, v.y, v.z, v.w};
      act_group_wave(e, lane, xq + int64_t(t) * xq_rb + int64_t(j) * gb, aq8);
    }
  } else {
    const int t = (int(blockIdx.x) - n_quant_wg) * 4 + wv;
    if (t < T) route_token<PER>(logits, t, E, k, sel_idx, sel_w, nullptr);
  }
}

// Many tokens, second step: one workgroup groups the selections.
__global__ void __launch_bounds__(kRouteThreads) moe_group_kernel(const int32_t* __restrict__ sel_idx, int n, int E,
                                                                  int k, MoeLists lists) {
  __shared__ GroupLds g;
  group_init(g, E);
  if (n <= kRouteLdsPairs)
    for (int i = threadIdx.x; i < n; i += kRouteThreads) g.sel[i] = sel_idx[i];
  group_pairs(g, sel_idx, n, E, k, lists);
}

constexpr int kMoeTokChunk = 8;          // activation rows of one expert staged in LDS per pass
constexpr int64_t kMoeStageBytes = 49152;  // LDS for them

// Waits for every global load in flight.  Ends a staging loop whose last LDS writes sit under a
// lane condition: without it the loads feeding them look outstanding to the compiler on the path
// that skips those writes, and it then waits at the next reuse of their registers (inside the
// weight pipeline) instead.
__device__ __forceinline__ void vm_settle() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Makes v opaque to the optimizer at this point (it waits for v's load here): a value picked by
// lane from loaded registers is otherwise turned back into a load of its own, a second trip.
__device__ __forceinline__ void pin(u32x4& v) { asm volatile("" : "+v"(v)); }


// Unit u of row `row` of a stacked expert tensor of n_rows rows: GGUF bytes (rb per row) or a
// planar layout (Q4_K_R / Q6_K_R, as written by jero_hip_repack over all n_rows rows).
template <int F>
__device__ __forceinline__ void load_unit(typename Unit<F>::W& w, const uint8_t* __restrict__ base, int64_t n_rows,
                                          int U, int64_t rb, int64_t row, int u) {
  if constexpr (is_planar(F))
    Unit<F>::load_w_planar(w, base, n_rows, U, row, u);
  else
    Unit<F>::load_w(w, base + row * rb, u);
}

// Copies `n` activation rows of `rb` bytes (dword multiples) into LDS: row j comes from
// src + rows[j] * rb, with rows[] already in LDS.  Eight unconditional (clamped) loads per thread
// are in flight at a time.  Ends with a barrier on LDS traffic (global loads issued before
// the staging complete first anyway: their counter drains in order).
__device__ __forceinline__ void stage_rows(uint32_t* __restrict__ dst, const uint8_t* __restrict__ src, int64_t rb,
                                           int n, const int* __restrict__ rows) {
  const int words = int(rb / 4), total = n * words;
  for (int idx0 = threadIdx.x; idx0 < total; idx0 += 8 * int(blockDim.x)) {
    uint32_t v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int idx = min(idx0 + q * int(blockDim.x), total - 1);
      const int j = idx / words, w = idx - j * words;
      v[q] = reinterpret_cast<const uint32_t*>(src + int64_t(rows[j]) * rb)[w];
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int idx = idx0 + q * int(blockDim.x);
      if (idx < total) dst[idx] = v[q];
    }
  }
  vm_settle();
  lds_barrier();
}

// Quantizes n consecutive f32 rows (src rows row0 .. row0 + n, `cols` floats each) to activation
// rows of `qrb` bytes in LDS (aq8: ACT_Q8, else Q8_K), one wave per 256-element group; each wave
// loads four groups before quantizing them.  Ends with a barrier on LDS traffic.
__device__ __forceinline__ void stage_quant_rows(uint8_t* __restrict__ dst, const float* __restrict__ src, int cols,
                                                 int64_t qrb, int n, int row0, bool aq8) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = int(blockDim.x) >> 6;
  const int bpr = cols / 256, total = n * bpr;
  for (int b0 = wv; b0 < total; b0 += 4 * nw) {
    float4 v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int b = min(b0 + q * nw, total - 1), j = b / bpr, jb = b - j * bpr;
      v[q] = reinterpret_cast<const float4*>(src + int64_t(row0 + j) * cols + int64_t(jb) * 256)[lane];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int b = b0 + q * nw;  // uniform over the wave
      if (b < total) {
        const int j = b / bpr, jb = b - j * bpr;
        const float e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
        act_group_wave(e, lane, dst + int64_t(j) * qrb + int64_t(jb) * act_group_bytes(aq8), aq8);
      }
    }
  }
  vm_settle();
  lds_barrier();
}

// gate/up + SwiGLU.  A workgroup takes one active expert and 4 * ppw * P of its (gate, up) row
// pairs: lane groups (2p, 2p+1) of a wave hold gate row and up row f.  The expert's token
// activations are staged in LDS (`chunk` rows per pass), so each weight row is read from HBM once
// and each activation once per workgroup.  Two register buffers alternate: the next row pair's
// weights are in flight while the current one is reduced over the tokens.  The loads are kept
// where they are issued by three rules: no buffer is copied into the other (a copy waits for the
// load), every path through the token loop uses the weights (the loop runs at least once, and
// units past the row end are dotted clamped and then dropped by a select, never skipped by a
// branch), and barriers wait on LDS only.
template <int F, int LPR, int UPL, int SPER>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(const uint8_t* __restrict__ gate,
                                                          const uint8_t* __restrict__ up, int64_t n_rows, int64_t rb,
                                                          int U, int Fdim,
                                                          int k, const uint8_t* __restrict__ xq, int64_t xq_rb,
                                                          MoeLists lists, float* __restrict__ act, int ppw,
                                                          int wg_per_expert, int chunk, MoeSingle one) {
  using Ut = Unit<F>;
  using W = typename Ut::W;
  constexpr int G = kWave / LPR;
  constexpr int P = G / 2;  // (gate, up) row pairs per wave pass
  static_assert(P >= 1, "gate/up pairing needs two lane groups per wave");
  extern __shared__ uint32_t s_x[];
  __shared__ int s_rows[kMoeTokChunk];
  __shared__ int s_sel[kMaxTopK];
  const int slot = int(blockIdx.x) / wg_per_expert, part = int(blockIdx.x) % wg_per_expert;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int e, i0, cnt;
  if constexpr (SPER > 0) {
    // one token (SPER expert columns per lane): every workgroup routes it (wave 0; the selections
    // are written out too, by all workgroups alike) and quantizes it to a Q8_K row in LDS (the
    // other waves); slot j is the token's j-th selection, its act row j
    if (wv == 0) {
      route_token<SPER>(one.logits, 0, one.E, k, one.sel_idx, one.sel_w, s_sel);
    } else {
      for (int blk = wv - 1; blk < one.H / 256; blk += 3) {
        const float4 v = reinterpret_cast<const float4*>(one.x + int64_t(blk) * 256)[lane];
        const float ev[4] = {v.x, v.y, v.z, v.w};
        act_group_wave(ev, lane, reinterpret_cast<uint8_t*>(s_x) + blk * act_group_bytes(act_is_q8(F)), act_is_q8(F));
      }
    }
    __syncthreads();
    e = s_sel[slot];
    i0 = slot;
    cnt = 1;
  } else {
    if (slot >= *lists.n_active) return;  // uniform over the workgroup
    e = lists.active[slot];
    i0 = lists.offset[e];
    cnt = lists.offset[e + 1] - i0;
  }
  const int g = lane / LPR, c = lane % LPR;
  const bool is_up = g & 1;
  const int rows_wg = 4 * ppw * P, fbase = part * rows_wg;  // the workgroup's row pairs
  const int r0 = wv * ppw * P + g / 2;                       // this lane group's first, in them
  const int f0 = fbase + r0;
  // results go to LDS and leave in one coalesced pass per token chunk: a global store inside the
  // pipeline would count with the weight loads, and waiting for the weights would wait for it
  float* s_out = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(s_x) + int64_t(chunk) * xq_rb);
  auto load_pair = [&](int it, W (&wt)[UPL]) {
    const int f = min(f0 + it * P, Fdim - 1);
#pragma unroll
    for (int t = 0; t < UPL; t++)
      load_unit<F>(wt[t], is_up ? up : gate, n_rows, U, rb, int64_t(e) * Fdim + f, min(c + LPR * t, U - 1));
  };
  auto process = [&](int it, W (&wt)[UPL], int nch) {
    typename Ut::Prep pr[UPL];  // unpacked once for all the tokens
#pragma unroll
    for (int t = 0; t < UPL; t++) Ut::prep(pr[t], wt[t], min(c + LPR * t, U - 1));
    int j = 0;
    do {  // nch >= 1
      const uint8_t* xt = reinterpret_cast<const uint8_t*>(s_x) + int64_t(j) * xq_rb;
      float accv = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        const int u = c + LPR * t;
        typename Ut::Act a;
        Ut::load_act(a, xt, min(u, U - 1));
        const float d = Ut::dot_prep(pr[t], a);
        accv += u < U ? d : 0.f;
      }
      accv = group_sum_last<LPR>(accv);
      const float gv = __shfl(accv, lane - LPR, kWave);  // gate total, from the group below
      if (is_up && c == LPR - 1) {
        const float silu = gv / (1.0f + expf(-gv));
        s_out[j * rows_wg + r0 + it * P] = silu * accv;
      }
    } while (++j < nch);
  };
  W wa[UPL], wb[UPL];
  for (int base = 0; base < cnt; base += chunk) {
    const int nch = min(chunk, cnt - base);
    load_pair(0, wa);  // in flight while the activations are staged
    if constexpr (SPER == 0) {  // (one token: its row is in LDS already)
      lds_barrier();            // the previous pass's readers are done
      if (int(threadIdx.x) < nch) s_rows[threadIdx.x] = lists.entry[i0 + base + threadIdx.x] / k;
      lds_barrier();
      stage_rows(s_x, xq, xq_rb, nch, s_rows);
    }
    // ppw is even: the loop's only exit is at the bottom, so no path leaves wb in flight
    for (int it = 0;; it += 2) {
      load_pair(it + 1, wb);
      __builtin_amdgcn_sched_barrier(0);
      process(it, wa, nch);
      load_pair(min(it + 2, ppw - 1), wa);  // the last one is redundant
      __builtin_amdgcn_sched_barrier(0);
      process(it + 1, wb, nch);
      if (it + 2 >= ppw) break;
    }
    lds_barrier();
    for (int idx = threadIdx.x; idx < nch * rows_wg; idx += 256) {
      const int j = idx / rows_wg, r = idx - j * rows_wg;
      if (fbase + r < Fdim) act[int64_t(i0 + base + j) * Fdim + fbase + r] = s_out[idx];
    }
  }
}

// down: a workgroup takes one active expert and 4 * rpw * G rows h of its down matrix (one lane
// group per row); the expert's act rows (contiguous, entries i0 .. i1, f32) are quantized to Q8_K
// straight into LDS.  Weights alternate between two register buffers under the rules of gate/up.
template <int F, int LPR, int UPL>
__global__ void __launch_bounds__(256) moe_down_kernel(const uint8_t* __restrict__ down, int64_t n_rows, int64_t rb,
                                                       int U, int H,
                                                       const float* __restrict__ act, int ffn, int64_t aq_rb,
                                                       MoeLists lists, float* __restrict__ yd, int rpw,
                                                       int wg_per_expert, int chunk) {
  using Ut = Unit<F>;
  using W = typename Ut::W;
  constexpr int G = kWave / LPR;
  extern __shared__ uint32_t s_x[];
  const int slot = int(blockIdx.x) / wg_per_expert, part = int(blockIdx.x) % wg_per_expert;
  if (slot >= *lists.n_active) return;
  const int e = lists.active[slot];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / LPR, c = lane % LPR;
  const int i0 = lists.offset[e], cnt = lists.offset[e + 1] - i0;
  const int rows_wg = 4 * rpw * G, hbase = part * rows_wg;  // the workgroup's rows
  const int r0 = wv * rpw * G + g;                          // this lane group's first, in them
  const int h0 = hbase + r0;
  // results leave through LDS, as in gate/up
  float* s_out = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(s_x) + int64_t(chunk) * aq_rb);
  auto load_row = [&](int it, W (&wt)[UPL]) {
    const int h = min(h0 + it * G, H - 1);
#pragma unroll
    for (int t = 0; t < UPL; t++)
      load_unit<F>(wt[t], down, n_rows, U, rb, int64_t(e) * H + h, min(c + LPR * t, U - 1));
  };
  auto process = [&](int it, W (&wt)[UPL], int nch) {
    typename Ut::Prep pr[UPL];  // unpacked once for all the tokens
#pragma unroll
    for (int t = 0; t < UPL; t++) Ut::prep(pr[t], wt[t], min(c + LPR * t, U - 1));
    int j = 0;
    do {  // nch >= 1
      const uint8_t* at = reinterpret_cast<const uint8_t*>(s_x) + int64_t(j) * aq_rb;
      float accv = 0.f;
#pragma unroll
      for (int t = 0; t < UPL; t++) {
        const int u = c + LPR * t;
        typename Ut::Act a;
        Ut::load_act(a, at, min(u, U - 1));
        const float d = Ut::dot_prep(pr[t], a);
        accv += u < U ? d : 0.f;
      }
      accv = group_sum_last<LPR>(accv);
      if (c == LPR - 1) s_out[j * rows_wg + r0 + it * G] = accv;
    } while (++j < nch);
  };
  W wa[UPL], wb[UPL];
  for (int base = 0; base < cnt; base += chunk) {
    const int nch = min(chunk, cnt - base);
    load_row(0, wa);  // in flight while the activations are staged
    lds_barrier();    // the previous pass's readers are done
    stage_quant_rows(reinterpret_cast<uint8_t*>(s_x), act, ffn, aq_rb, nch, i0 + base, act_is_q8(F));
    for (int it = 0;; it += 2) {  // rpw is even, as ppw in gate/up
      load_row(it + 1, wb);
      __builtin_amdgcn_sched_barrier(0);
      process(it, wa, nch);
      load_row(min(it + 2, rpw - 1), wa);
      __builtin_amdgcn_sched_barrier(0);
      process(it + 1, wb, nch);
      if (it + 2 >= rpw) break;
    }
    lds_barrier();
    for (int idx = threadIdx.x; idx < nch * rows_wg; idx += 256) {
      const int j = idx / rows_wg, r = idx - j * rows_wg;
      if (hbase + r < H) yd[int64_t(i0 + base + j) * H + hbase + r] = s_out[idx];
    }
  }
}

// Logical workgroup of physical workgroup b (of n) when groups of m consecutive logical
// workgroups read the same 128-byte lines (the rows of one 16-row tile).  Workgroups go to the 8
// XCDs round-robin and each XCD has its own L2, so in every run of 8m physical workgroups the m
// members of a group are given physical indices 8 apart (one XCD), and the lines are fetched
// from HBM once instead of once per XCD.  A tail shorter than 8m keeps the identity order.
__device__ __forceinline__ int xcd_grouped(int b, int n, int m) {
  const int chunk = 8 * m;
  if (m <= 1 || b >= n / chunk * chunk) return b;
  const int c = b / chunk, r = b - c * chunk;
  return c * chunk + (r & 7) * m + (r >> 3);
}

// One token, down and combine in one: a workgroup takes RW rows h of the output, and for each its
// k selected experts' down rows (units (slot j, row r), lane group per unit); the token's act rows
// (act row j = selection j) are quantized to Q8_K in LDS.  The dots land in LDS and the workgroup
// then writes y[h] = sum over j ascending of w_j * dot_j, the reference's combine order.
// PRE: the k act rows hold at most 4 * kDown1PreBlocks 256-blocks; each wave loads its blocks into
// registers at entry, beside the selections (they do not depend on them), and quantizes them while
// the first weights are in flight; else they are staged after the first weight loads.
constexpr int kDown1PreBlocks = 8;

template <int F, int LPR, int UPL, bool PRE>
__global__ void __launch_bounds__(256) moe1_down_kernel(const uint8_t* __restrict__ down, int64_t n_rows, int64_t rb,
                                                        int U, int H, const float* __restrict__ act, int ffn,
                                                        int64_t aq_rb, int k, const int32_t* __restrict__ sel_idx,
                                                        const float* __restrict__ sel_w, float* __restrict__ y, int RW,
                                                        int upg, int accumulate, float* __restrict__ resid) {
  using Ut = Unit<F>;
  using W = typename Ut::W;
  constexpr int G = kWave / LPR;
  extern __shared__ uint32_t s_x[];  // k Q8_K act rows, then dots [k][RW]
  __shared__ int s_sel[kMaxTopK];
  __shared__ float s_w[kMaxTopK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int g = lane / LPR, c = lane % LPR;
  const int lg = wv * G + g, n_lg = 4 * G;  // lane group and their number
  // Q6_K_T / Q4_K_T rows come in 16-row tiles; the 16 / RW workgroups of a tile share its lines
  constexpr bool kTiled = F == JERO_Q6_K_T || F == JERO_Q4_K_T;
  const int share = kTiled && RW < 16 && 16 % RW == 0 ? 16 / RW : 1;
  const int hbase = xcd_grouped(int(blockIdx.x), int(gridDim.x), share) * RW, n_units = RW * k;
  float* s_dot = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(s_x) + int64_t(k) * aq_rb);
  const int nbk = ffn / 256, total_blk = k * nbk;
  float4 av[PRE ? kDown1PreBlocks : 1];
  if constexpr (PRE) {  // unconditional (clamped) loads of the wave's act blocks
#pragma unroll
    for (int q = 0; q < kDown1PreBlocks; q++) {
      const int b = min(wv + 4 * q, total_blk - 1), j = b / nbk, jb = b - j * nbk;
      av[q] = reinterpret_cast<const float4*>(act + int64_t(j) * ffn + int64_t(jb) * 256)[lane];
    }
  }
  if (threadIdx.x < kMaxTopK) {
    const int j = min(int(threadIdx.x), k - 1);
    s_sel[threadIdx.x] = sel_idx[j];
    s_w[threadIdx.x] = sel_w[j];
  }
  __syncthreads();
  // unit i of this lane group: q = lg + n_lg * i -> (slot j, row r), clamped past the end
  auto unit = [&](int i, int& j, int& r) {
    const int q = min(lg + n_lg * i, n_units - 1);
    j = q / RW;
    r = q - j * RW;
  };
  auto load_unit_w = [&](int i, W (&wt)[UPL]) {
    int j, r;
    unit(i, j, r);
    const int h = min(hbase + r, H - 1);
#pragma unroll
    for (int t = 0; t < UPL; t++)
      load_unit<F>(wt[t], down, n_rows, U, rb, int64_t(s_sel[j]) * H + h, min(c + LPR * t, U - 1));
  };
  auto process = [&](int i, W (&wt)[UPL]) {
    int j, r;
    unit(i, j, r);
    typename Ut::Prep pr[UPL];
#pragma unroll
    for (int t = 0; t < UPL; t++) Ut::prep(pr[t], wt[t], min(c + LPR * t, U - 1));
    const uint8_t* at = reinterpret_cast<const uint8_t*>(s_x) + int64_t(j) * aq_rb;
    float accv = 0.f;
#pragma unroll
    for (int t = 0; t < UPL; t++) {
      const int u = c + LPR * t;
      typename Ut::Act a;
      Ut::load_act(a, at, min(u, U - 1));
      const float d = Ut::dot_prep(pr[t], a);
      accv += u < U ? d : 0.f;
    }
    accv = group_sum_last<LPR>(accv);
    if (c == LPR - 1 && lg + n_lg * i < n_units) s_dot[j * RW + r] = accv;
  };
  W wa[UPL], wb[UPL];
  load_unit_w(0, wa);  // in flight while the act rows are quantized
  if constexpr (PRE) {
    // blocks past the last one quantize into a dummy block after the dots (no branch skips a wait)
    uint8_t* dummy = reinterpret_cast<uint8_t*>(s_dot + k * RW);
#pragma unroll
    for (int q = 0; q < kDown1PreBlocks; q++) {
      const int b = wv + 4 * q, j = b / nbk, jb = b - j * nbk;
      const float e[4] = {av[q].x, av[q].y, av[q].z, av[q].w};
      act_group_wave(e, lane,
                     b < total_blk ? reinterpret_cast<uint8_t*>(s_x) + int64_t(j) * aq_rb + act_group_bytes(act_is_q8(F)) * jb
                                   : dummy,
                     act_is_q8(F));
    }
    lds_barrier();
  } else {
    stage_quant_rows(reinterpret_cast<uint8_t*>(s_x), act, ffn, aq_rb, k, 0, act_is_q8(F));
  }
  for (int i = 0;; i += 2) {  // upg is even: the loop's only exit is at the bottom
    load_unit_w(i + 1, wb);
    __builtin_amdgcn_sched_barrier(0);
    process(i, wa);
    load_unit_w(min(i + 2, upg - 1), wa);  // the last one is redundant
    __builtin_amdgcn_sched_barrier(0);
    process(i + 1, wb);
    if (i + 2 >= upg) break;
  }
  lds_barrier();
  for (int r = threadIdx.x; r < RW; r += 256) {
    if (hbase + r >= H) continue;
    float acc = accumulate ? y[hbase + r] : 0.f;
    for (int j = 0; j < k; j++) acc += s_w[j] * s_dot[j * RW + r];
    if (resid) resid[hbase + r] += acc;
    else y[hbase + r] = acc;
  }
}

// ---------------------------------------------------------------- expert GEMMs on MFMA
// Several tokens per expert: v_mfma_i32_16x16x64_i8 over one 64-weight unit at a time.  Lane l
// supplies A row l % 16 and B column l % 16 (a weight row) over K [16 (l / 16), +16) and receives
// C rows 4 (l / 16) .. +4 of column l % 16.  Two forms, both exact in integers per block:
//   * Q4_K in 16-token passes (plane form): the A rows are 16 tokens.  A lane's 16 weights of a unit lie in one
//     sub-block, whose 6-bit scale splits as sc = 8a + b: the lane feeds the MFMA the planes
//     a q4 and b q4 (<= 105), so 8 Ta + Tb over the block's four units is the block's sum of
//     sc q4 q8 per (token, row), and the mins sum over the 16 bsums is one f16 MFMA.
//   * Q6_K, and Q4_K in 8-token passes (segment form): a unit has SEG integer-scaled segments
//     (Q4_K: 2 sub-blocks of 32; Q6_K: 4 groups of 16).  The 16 A rows are (token, segment)
//     pairs, each holding its token's activations only in the K range of its segment (zeros
//     elsewhere), so one MFMA yields the exact integer sum of every segment for 16 / SEG tokens;
//     the segment scales (and Q4_K mins) come from the lane's own weight row and are applied
//     in-lane, in integers.
// The block's float scales then apply once per block, dx * (d * isum - dmin * msum) as the
// reference's block dot.  Activations are staged in LDS as Q8_K rows (rows of 16-byte multiples,
// one more row of zeros for the A lanes outside their group).

typedef int v4i __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int mfma_seg(int f) { return is_q6k(f) ? 4 : 2; }
// LDS bytes per staged token row: its Q8_K row rounded up to 16 bytes, plus 16, made an odd number
// of 16-byte units so that the rows of the 8 tokens start 4 banks apart: a wave's A reads (one
// 16-byte piece from each of up to 8 rows at the same offset) then hit distinct banks.
__host__ __device__ inline int act_row_stride(int nb) {
  const int s = ((nb * 292 + 15) & ~15) + 16;
  return (s / 16) % 2 ? s : s + 16;
}
// Tokens staged per pass (PT: NT = PT / TPT token tiles): a pass descriptor's worth.

// The weights of block b (units 4b .. 4b + 3: one step) of one weight row for lane group kg, as
// loaded.  A step takes a whole block so that every cache line it fetches is used up within
// the step: lines shared between steps were evicted from L2 between their uses (the step
// working set of all resident waves exceeds an XCD's L2), costing 1.45x the HBM bytes.  A Cur
// holds the lane's pointers into its weight row of tile 0 (one per region of the layout); a step
// adds its tile's and block's offsets, which are uniform.
template <int F>
struct MfmaPiece;
template <>
struct MfmaPiece<JERO_Q4_K_R> {
  u32x4 q[4];  // q0 (kg even) or q1 (kg odd) run of each unit: 16 bytes of qs
  u32x4 h;     // the block header (d, dmin, 12 scale bytes)
  struct Cur {
    const uint8_t *q, *h;
    int64_t tile;  // bytes per 16 rows
  };
  static __device__ __forceinline__ Cur cursor(const uint8_t* __restrict__ base, int64_t /*n_rows*/, int U,
                                               int64_t /*rb*/, int64_t row, int kg) {
    const uint8_t* rp = base + row * (int64_t(U) * 36);
    return {rp + (kg & 1) * U * 16, rp + U * 32, int64_t(16) * U * 36};
  }
  static __device__ __forceinline__ void load(MfmaPiece& p, const Cur& cu, int tile, int b) {
    const int64_t o = tile * cu.tile;
#pragma unroll
    for (int x = 0; x < 4; x++) p.q[x] = ld4(cu.q + o + (4 * b + x) * 16);
    p.h = ld4(cu.h + o + b * 16);
  }
};
template <>
struct MfmaPiece<JERO_Q4_K> : MfmaPiece<JERO_Q4_K_R> {
  static __device__ __forceinline__ Cur cursor(const uint8_t* __restrict__ base, int64_t /*n_rows*/, int /*U*/,
                                               int64_t rb, int64_t row, int kg) {
    const uint8_t* rp = base + row * rb;
    return {rp + 16 + 16 * (kg & 1), rp, 16 * rb};
  }
  static __device__ __forceinline__ void load(MfmaPiece& p, const Cur& cu, int tile, int b) {
    const int64_t o = tile * cu.tile + b * 144;
#pragma unroll
    for (int x = 0; x < 4; x++) p.q[x] = ld4(cu.q + o + 32 * x);
    p.h = ld4(cu.h + o);
  }
};
template <>
struct MfmaPiece<JERO_Q6_K_R> {
  u32x4 x[4], qh[4];  // ql run (lo for even kg, hi for odd) and qh run of each unit
  u32x4 sc;           // the units' int8 group scales, one dword per unit
  uint32_t dw, dsh;   // the block's f16 d: its dword and shift
  struct Cur {
    const uint8_t *x, *qh, *sc, *d;
    int U;
  };
  static __device__ __forceinline__ Cur cursor(const uint8_t* __restrict__ base, int64_t n_rows, int U,
                                               int64_t /*rb*/, int64_t row, int kg) {
    const int64_t plane = n_rows * int64_t(U) * 16;
    return {base + (kg & 1) * plane + row * U * 16, base + 2 * plane + row * U * 16, base + 3 * plane + row * U * 4,
            base + 3 * plane + n_rows * int64_t(U) * 4 + row * (U / 4) * 2, U};
  }
  static __device__ __forceinline__ void load(MfmaPiece& p, const Cur& cu, int tile, int b) {
    const int64_t gu = int64_t(tile) * 16 * cu.U + 4 * b;  // the step's first unit, from the row's
#pragma unroll
    for (int x = 0; x < 4; x++) {
      p.x[x] = ld4(cu.x + (gu + x) * 16);
      p.qh[x] = ld4(cu.qh + (gu + x) * 16);
    }
    p.sc = ld4(cu.sc + gu * 4);
    const uint8_t* dp = cu.d + (int64_t(tile) * 16 * (cu.U / 4) + b) * 2;
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(dp) & 3u);
    p.dw = ld1(dp - sh);
    p.dsh = 8u * sh;
  }
};

// The 16-row tiled layouts: a step reads whole contiguous pieces (one per tile and block).
template <>
struct MfmaPiece<JERO_Q4_K_T> : MfmaPiece<JERO_Q4_K_R> {
  static __device__ __forceinline__ Cur cursor(const uint8_t* __restrict__ base, int64_t /*n_rows*/, int U,
                                               int64_t /*rb*/, int64_t row, int kg) {
    const int64_t tile = int64_t(U / 4) * 2304;  // bytes per 16 rows
    const uint8_t* pc = base + (row >> 4) * tile;
    const int c = int(row & 15);
    return {pc + ((kg & 1) * 16 + c) * 16, pc + 2048 + c * 16, tile};
  }
  static __device__ __forceinline__ void load(MfmaPiece& p, const Cur& cu, int tile, int b) {
    const int64_t o = tile * cu.tile + b * 2304;
#pragma unroll
    for (int x = 0; x < 4; x++) p.q[x] = ld4(cu.q + o + 512 * x);
    p.h = ld4(cu.h + o);
  }
};
template <>
struct MfmaPiece<JERO_Q6_K_T> : MfmaPiece<JERO_Q6_K_R> {
  struct Cur {
    const uint8_t *x, *qh, *sc, *d;
    int64_t tile;   // bytes per 16 rows
    uint32_t dsh;   // the f16 d's shift in its dword (rows alternate halves)
  };
  static __device__ __forceinline__ Cur cursor(const uint8_t* __restrict__ base, int64_t /*n_rows*/, int U,
                                               int64_t /*rb*/, int64_t row, int kg) {
    const int64_t tile = int64_t(U / 4) * 3360;
    const uint8_t* pc = base + (row >> 4) * tile;
    const int c = int(row & 15);
    return {pc + ((kg & 1) * 16 + c) * 16, pc + 2048 + c * 16, pc + 3072 + c * 16, pc + 3328 + (c & ~1) * 2, tile,
            16u * uint32_t(c & 1)};
  }
  static __device__ __forceinline__ void load(MfmaPiece& p, const Cur& cu, int tile, int b) {
    const int64_t o = tile * cu.tile + b * 3360;
#pragma unroll
    for (int x = 0; x < 4; x++) {
      p.x[x] = ld4(cu.x + o + 512 * x);
      p.qh[x] = ld4(cu.qh + o + 256 * x);
    }
    p.sc = ld4(cu.sc + o);
    p.dw = ld1(cu.d + o);
    p.dsh = cu.dsh;
  }
};

// 6-bit scale and min of Q4_K sub-block `sb` (0..7) from the block header h.
__device__ __forceinline__ void q4k_scale_min(const u32x4& h, int sb, int& sc, int& m) {
  const uint32_t jj = uint32_t(sb & 3);
  const uint32_t a = byte_of(h.y, jj), bb = byte_of(h.z, jj), c = byte_of(h.w, jj);
  sc = int(sb < 4 ? a & 63u : (c & 15u) | ((a >> 6) << 4));
  m = int(sb < 4 ? bb & 63u : (c >> 4) | ((bb >> 6) << 4));
}

constexpr int kStageChunks = 8;  // Q8_K staging: 16-byte chunks per thread in one batch
constexpr int kStageBlocks = 8;  // f32 staging: 256-element blocks per wave in one batch

// Work items: (pass, row block) -- one pass descriptor's tokens (up to PT of one expert) against 64 * tiles weight rows of that expert (tiles tiles of 16 per wave, one after
// the other), numbered pass-major.  The grid is persistent (what fits on the GPU at once) and
// each workgroup takes the next item from a counter until none is left.  The next item's number
// is fetched while the current one runs.  Each tile's results go to LDS when its last block is
// done and leave in one coalesced pass.  GU: gate (w0) and up (w1) rows from the tokens' Q8_K
// rows, out = silu(gate) * up per (list entry, row); else down (w0) rows from the f32 act rows
// (quantized here), out = the dot per (list entry, row).  An item makes two dependent trips to
// memory before its first MFMA: the pass descriptor, then the activations (batches of 8 rows) with the
// first weights behind them; the load counter drains in order, so nothing small waits behind
// weights.  R is a multiple of 64 * tiles: no row is clamped.
// Workgroups per CU the register budget is cut for: three (168 VGPRs), except Q6_K gate/up, whose
// two tensors' pieces need more registers than that without spilling, and the 16-token passes
// (twice the accumulators) of Q6_K down: two.  (Q6_K gate/up takes no 16-token passes: they spill
// at any budget.)  Q4_K's 16-token passes take the plane form, one tile in 160 VGPRs.
__host__ __device__ constexpr int mfma_min_wgs(int f, bool gu, int pt) {
  return mfma_seg(f) == 4 && (gu || pt > kMoePassTokens) ? 2 : 3;
}

// Four bytes times s (<= 7) as two 16-bit lanes: no carry between bytes, each product <= 105.
__device__ __forceinline__ uint32_t bytes_times(uint32_t x, uint32_t s) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, x) * u16x2{uint16_t(s), uint16_t(s)});
}

template <int F, bool GU, int PT>
__global__ void __launch_bounds__(256, mfma_min_wgs(F, GU, PT)) moe_mfma_kernel(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                                       int64_t n_rows, int64_t rb, int U, int R, int tiles,
                                                       const uint8_t* __restrict__ xq, int64_t xq_rb,
                                                       const float* __restrict__ act_in, MoeLists lists,
                                                       float* __restrict__ out, int wg_per_expert, int ctr_off) {
  // Q4_K in 16-token passes: the plane form.  A rows are 16 tokens over the whole K range; a
  // lane's B bytes lie in one sub-block, whose scale sc = 8a + b splits them into the exact int8
  // planes a q4 and b q4 (<= 105), so two MFMAs per unit sum the scales in and T = 8 Ta + Tb is
  // the block's integer sum of sc q4 q8 per (token, row); the mins sum over the 16 bsums is one
  // f16 MFMA (exact: |bsum| <= 2032, m <= 63, sums below 2^24).  The VALU only expands the planes
  // and applies the block's float scales.  Q6_K, and Q4_K in 8-token passes (which would leave
  // half of a 16-token tile empty): the segment form (below).
  constexpr int SEG = mfma_seg(F);
  constexpr bool PLANE = SEG == 2 && PT > kMoePassTokens;
  constexpr int TPT = PLANE ? 16 : 16 / SEG, NT = PLANE ? (PT + 15) / 16 : PT / TPT, LT = PLANE ? 4 : 4 / SEG;
  constexpr int NW = GU ? 2 : 1;  // weight tensors per wave
  using Piece = MfmaPiece<F>;
  using Cur = typename Piece::Cur;
  extern __shared__ __attribute__((aligned(16))) uint8_t s_act[];
  __shared__ int s_tok[PT];
  __shared__ int s_item;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = lane & 15, kg = lane >> 4;
  const int nb = U / 4, stride = act_row_stride(nb);
  const int zrow = PT * stride, dummy = zrow + stride;  // the zero row, then a dummy area
  const int steps = tiles * nb;
  float* s_out = reinterpret_cast<float*>(s_act + dummy + 304);  // [tiles][PT][64 rows]
  for (int i = threadIdx.x; i < stride / 16; i += 256) *reinterpret_cast<u32x4*>(s_act + zrow + 16 * i) = u32x4{};
  // the counter is bumped by atomicInc (with no wrap): the compiler turns a single-lane atomicAdd
  // into a wave-aggregated one whose result it waits for at once
  unsigned* const ctr = reinterpret_cast<unsigned*>(lists.ctr + ctr_off);
  const int n_items = lists.ctr[0] * wg_per_expert;
  if (threadIdx.x == 0) s_item = int(atomicInc(ctr, 0xFFFFFFFFu));
  __syncthreads();
  const uint8_t* wt[2] = {w0, GU ? w1 : w0};
  // A operand lanes: virtual row vr = (token, segment); K group kg belongs to segment kg / (4 / SEG)
  const int vr = lane & 15, a_tok = PLANE ? vr : vr / SEG, kg_seg = kg / (4 / SEG);
  const bool a_on = PLANE || vr % SEG == kg_seg;
  const int a_lane = SEG == 2 ? 4 + 16 * kg : 4 + 32 * kg;  // the lane's K group in a unit's bytes
  const uint32_t nsh = (kg & 2) ? 4u : 0u;                    // its nibble: low for kg < 2
  static_assert(PT % 4 == 0, "a pass descriptor is 1 + PT / 4 16-byte loads");
  for (int item = s_item; item < n_items;) {  // item is uniform over the workgroup
    const int pi = item / wg_per_expert, part = item - pi * wg_per_expert;
    // the pass descriptor in one trip: expert, first list position, token count, 0, tokens
    const uint8_t* pd = reinterpret_cast<const uint8_t*>(lists.pass) + int64_t(pi) * ((4 + PT) * 4);
    u32x4 ph = ld4(pd), ptv[PT / 4];
#pragma unroll
    for (int i = 0; i < PT / 4; i++) {
      ptv[i] = ld4(pd + 16 + 16 * i);
      pin(ptv[i]);  // held in registers: else a thread's token is loaded again once the header is in
    }
    const int e = int(ph.x), i0 = int(ph.y), nch = int(ph.z);
    uint32_t tj[PT];
#pragma unroll
    for (int i = 0; i < PT / 4; i++) {
      tj[4 * i] = ptv[i].x;
      tj[4 * i + 1] = ptv[i].y;
      tj[4 * i + 2] = ptv[i].z;
      tj[4 * i + 3] = ptv[i].w;
    }
    const int row0 = (part * 4 + wv) * tiles * 16 + c;  // this lane's weight row (B column) in tile 0
    Cur cur[NW];
#pragma unroll
    for (int t = 0; t < NW; t++) cur[t] = Piece::cursor(wt[t], n_rows, U, rb, int64_t(e) * R + row0, kg);
    // step s: block s % nb of tile s / nb (steps past the end clamp to the last)
    auto load = [&](int s_, Piece (&p)[NW]) {
      const int sc = min(s_, steps - 1), tile = sc / nb;
#pragma unroll
      for (int t = 0; t < NW; t++) Piece::load(p[t], cur[t], tile, sc - tile * nb);
    };
    // the lane's LDS rows: its A row's token (or the zero row), and the tokens of its C rows
    int a_base[NT], e_base[NT][LT], r_base[NT];
#pragma unroll
    for (int tl = 0; tl < NT; tl++) {
      r_base[tl] = min(tl * TPT + a_tok, nch - 1) * stride;  // the A row's token (plane form: its bsums)
      a_base[tl] = (a_on ? r_base[tl] : zrow) + a_lane;
#pragma unroll
      for (int q = 0; q < LT; q++) e_base[tl][q] = min(tl * TPT + kg * LT + q, nch - 1) * stride;
    }
    if (threadIdx.x < PT) s_tok[threadIdx.x] = int(tj[threadIdx.x]);
    lds_barrier();  // s_tok
    // Q6_K: the block's sum over its 16 groups of scale x bsum, per (token, row), comes from one f16
    // MFMA (exact: |sum| < 2^23): K slot 4 kg' + t is group 8n + j + 2t of unit kg' = 2n + j (the
    // unit's scale byte t), and A row 4 kg + i holds token 4 i + kg, so that C[tl] of lane (c, kg)
    // is token 4 tl + kg, as in the int8 MFMA.  The lane's A row: its token's bsums of groups 8n + j
    // + 2t, t = 0..3, the halves j of four dwords.
    const int fb_base = min((vr & 3) * 4 + (vr >> 2), nch - 1) * stride + 260 + 16 * (kg >> 1);
    const uint32_t fb_sh = 16u * uint32_t(kg & 1);
    const uint32_t qh_rot = uint32_t(2 * kg - 4) & 31u;  // rotates the lane's 2 high bits to bits 4..5
    // the K loop over NTA token tiles (NTA = NT; one instance: a second one for passes of at most
    // TPT tokens, whose buffers and staging would have to be its own, spilled registers)
    auto kloop = [&](auto nta) {
      constexpr int NTA = decltype(nta)::value;
      Piece pa[NW], pb[NW];
      // staging in batches: a batch's loads all issued, (after the first batch's) the first
      // weights, then the batch's LDS writes (out-of-range slots write a dummy area: no branch
      // may skip a wait); one batch holds 8 Q8_K rows of up to 4096 or 8 f32 rows of up to 1024
      if constexpr (GU) {
        const int chunks = int(xq_rb / 16), total = nch * chunks;  // 16-byte chunks of a (padded) Q8_K row
        auto batch = [&](int base, bool first) {
          u32x4 v[kStageChunks];
#pragma unroll
          for (int q = 0; q < kStageChunks; q++) {
            const int idx = min(base + int(threadIdx.x) + 256 * q, total - 1), j = idx / chunks;
            v[q] = ld4(xq + int64_t(s_tok[j]) * xq_rb + (idx - j * chunks) * 16);
          }
          if (first) load(0, pa);
#pragma unroll
          for (int q = 0; q < kStageChunks; q++) {
            const int idx = base + int(threadIdx.x) + 256 * q, j = idx / chunks;
            *reinterpret_cast<u32x4*>(s_act + (idx < total ? j * stride + (idx - j * chunks) * 16 : dummy)) = v[q];
          }
        };
        batch(0, true);
        for (int base = 256 * kStageChunks; base < total; base += 256 * kStageChunks) batch(base, false);
      } else {
        const int cols = U * 64, total = nch * nb;
        auto batch = [&](int base, bool first) {
          float4 v[kStageBlocks];
#pragma unroll
          for (int q = 0; q < kStageBlocks; q++) {
            const int b = min(base + wv + 4 * q, total - 1), j = b / nb, jb = b - j * nb;
            v[q] = reinterpret_cast<const float4*>(act_in + int64_t(i0 + j) * cols + int64_t(jb) * 256)[lane];
          }
          if (first) load(0, pa);
#pragma unroll
          for (int q = 0; q < kStageBlocks; q++) {
            const int b = base + wv + 4 * q, j = b / nb, jb = b - j * nb;
            const float ev[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
            q8k_block_wave(ev, lane, s_act + (b < total ? j * stride + 292 * jb : dummy));
          }
        };
        batch(0, true);
        for (int base = 4 * kStageBlocks; base < total; base += 4 * kStageBlocks) batch(base, false);
      }
      lds_barrier();
      // the next item's number, fetched behind the first weights: its wait comes after the K loop
      unsigned nxt = 0;
      if (threadIdx.x == 0) nxt = atomicInc(ctr, 0xFFFFFFFFu);
      float acc[NW][NT][LT];
#pragma unroll
      for (int t = 0; t < NW; t++)
#pragma unroll
        for (int tl = 0; tl < NT; tl++)
#pragma unroll
          for (int q = 0; q < LT; q++) acc[t][tl][q] = 0.f;
      // one step: block b (units 4b .. 4b + 3) of one tile; a step past the last (steps odd) is a
      // padding step: clamped loads, nothing accumulated
      auto process = [&](int s_, Piece (&p)[NW]) {
        const bool live = s_ < steps;
        const int sc_ = min(s_, steps - 1), tile = sc_ / nb, b = sc_ - tile * nb, bo = 292 * b;
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        typedef float f4 __attribute__((ext_vector_type(4)));
        if constexpr (PLANE) {
          v4i Ca[NW][NTA], Cb[NW][NTA];  // the a and b planes' integer sums over the block
#pragma unroll
          for (int x = 0; x < 4; x++) {
            v4i A[NTA];
#pragma unroll
            for (int tl = 0; tl < NTA; tl++) {
              const uint32_t* ap = reinterpret_cast<const uint32_t*>(s_act + a_base[tl] + bo + 64 * x);  // 4-byte aligned
              A[tl] = v4i{int(ap[0]), int(ap[1]), int(ap[2]), int(ap[3])};
            }
#pragma unroll
            for (int t = 0; t < NW; t++) {
              // B: this lane's 16 weights of unit x (sub-block 2x + kg / 2) times a and b
              int sc, mn;
              q4k_scale_min(p[t].h, 2 * x + (kg >> 1), sc, mn);
              const uint32_t sa = uint32_t(sc) >> 3, sb = uint32_t(sc) & 7u;
              const u32x4 q = p[t].q[x];
              const uint32_t qd[4] = {q.x, q.y, q.z, q.w};
              v4i Ba, Bb;
#pragma unroll
              for (int w = 0; w < 4; w++) {
                const uint32_t nib = (qd[w] >> nsh) & 0x0F0F0F0Fu;
                Ba[w] = int(bytes_times(nib, sa));
                Bb[w] = int(bytes_times(nib, sb));
              }
#pragma unroll
              for (int tl = 0; tl < NTA; tl++) {
                Ca[t][tl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[tl], Ba, x == 0 ? v4i{0, 0, 0, 0} : Ca[t][tl], 0, 0, 0);
                Cb[t][tl] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[tl], Bb, x == 0 ? v4i{0, 0, 0, 0} : Cb[t][tl], 0, 0, 0);
              }
            }
          }
          // the mins: A row = the A token's 16 bsums (this lane: 4 kg .. 4 kg + 3), B column = the
          // lane's weight row, K slot k taking the min of sub-block k / 2
          h4 Ab[NTA];
#pragma unroll
          for (int tl = 0; tl < NTA; tl++) {
            const uint32_t* bp = reinterpret_cast<const uint32_t*>(s_act + r_base[tl] + bo + 260 + 8 * kg);
            const uint32_t b0 = bp[0], b1 = bp[1];
            Ab[tl] = h4{_Float16(int(int16_t(b0 & 0xFFFFu))), _Float16(int(int16_t(b0 >> 16))),
                        _Float16(int(int16_t(b1 & 0xFFFFu))), _Float16(int(int16_t(b1 >> 16)))};
          }
#pragma unroll
          for (int t = 0; t < NW; t++) {
            int s0, m0, s1, m1;
            q4k_scale_min(p[t].h, 2 * kg, s0, m0);
            q4k_scale_min(p[t].h, 2 * kg + 1, s1, m1);
            const h4 Bm = h4{_Float16(m0), _Float16(m0), _Float16(m1), _Float16(m1)};
            const float dw = h2f(p[t].h.x), dm = h2f(p[t].h.x >> 16);
#pragma unroll
            for (int tl = 0; tl < NTA; tl++) {
              const f4 Mn = __builtin_amdgcn_mfma_f32_16x16x16f16(Ab[tl], Bm, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
              // the block's float scales, once per (tensor, token): dx (d sum sc S - dmin sum m bsum)
#pragma unroll
              for (int q = 0; q < LT; q++) {
                const float dx = *reinterpret_cast<const float*>(s_act + e_base[tl][q] + bo);
                const int T = (Ca[t][tl][q] << 3) + Cb[t][tl][q];
                const float term = dx * (dw * float(T) - dm * Mn[q]);
                acc[t][tl][q] += live ? term : 0.f;
              }
            }
          }
        } else {  // the segment form: (token, segment) rows, the segment scales in integers
          int isum[NW][NT][LT], msum[NW][NT][LT];  // the block's integer sums (msum: Q4_K mins)
#pragma unroll
          for (int x = 0; x < 4; x++) {
            v4i A[NTA];
#pragma unroll
            for (int tl = 0; tl < NTA; tl++) {
              const int xo = SEG == 2 ? 64 * x : 128 * (x >> 1) + 16 * (x & 1);
              const uint32_t* ap = reinterpret_cast<const uint32_t*>(s_act + a_base[tl] + bo + xo);  // 4-byte aligned
              A[tl] = v4i{int(ap[0]), int(ap[1]), int(ap[2]), int(ap[3])};
            }
#pragma unroll
            for (int t = 0; t < NW; t++) {
              // B: this lane's weight row over K group kg, as non-negative int8
              v4i B;
              int sc[SEG], mn[SEG];
              if constexpr (SEG == 2) {
                const u32x4 q = p[t].q[x];
                const uint32_t qd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int w = 0; w < 4; w++) B[w] = int((qd[w] >> nsh) & 0x0F0F0F0Fu);
#pragma unroll
                for (int sg = 0; sg < 2; sg++) q4k_scale_min(p[t].h, 2 * x + sg, sc[sg], mn[sg]);
              } else {
                const uint32_t xd[4] = {p[t].x[x].x, p[t].x[x].y, p[t].x[x].z, p[t].x[x].w};
                const uint32_t hd[4] = {p[t].qh[x].x, p[t].qh[x].y, p[t].qh[x].z, p[t].qh[x].w};
#pragma unroll
                for (int w = 0; w < 4; w++)
                  B[w] = int(((xd[w] >> nsh) & 0x0F0F0F0Fu) |
                             (__builtin_amdgcn_alignbit(hd[w], hd[w], qh_rot) & 0x30303030u));
                const uint32_t scd[4] = {p[t].sc.x, p[t].sc.y, p[t].sc.z, p[t].sc.w};
#pragma unroll
                for (int g = 0; g < 4; g++) sc[g] = int(int8_t(scd[x] >> (8 * g)));
              }
#pragma unroll
              for (int tl = 0; tl < NTA; tl++) {
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[tl], B, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int q = 0; q < LT; q++) {
                  if constexpr (SEG == 2) {
                    const int16_t* bs = reinterpret_cast<const int16_t*>(s_act + e_base[tl][q] + bo + 260);
                    const int bsa = int(bs[4 * x]) + int(bs[4 * x + 1]), bsb = int(bs[4 * x + 2]) + int(bs[4 * x + 3]);
                    // 24-bit products: |C| < 2^16 for a 32-weight sub-block, scales and mins < 64
                    const int is = __mul24(sc[0], C[SEG * q]) + __mul24(sc[1], C[SEG * q + 1]);
                    const int ms = __mul24(mn[0], bsa) + __mul24(mn[1], bsb);
                    isum[t][tl][q] = x == 0 ? is : isum[t][tl][q] + is;
                    msum[t][tl][q] = x == 0 ? ms : msum[t][tl][q] + ms;
                  } else {
                    int is = 0;  // the q6 offset of 32 is taken off once per block, below
#pragma unroll
                    for (int g = 0; g < 4; g++) is += __mul24(sc[g], C[g]);  // |C| < 2^17
                    isum[t][tl][q] = x == 0 ? is : isum[t][tl][q] + is;
                  }
                }
              }
            }
          }
          if constexpr (SEG == 4) {
            const uint32_t* bp = reinterpret_cast<const uint32_t*>(s_act + fb_base + bo);
            h4 Ab;
#pragma unroll
            for (int t4 = 0; t4 < 4; t4++) Ab[t4] = _Float16(int(int16_t(bp[t4] >> fb_sh)));
#pragma unroll
            for (int t = 0; t < NW; t++) {
              pin(p[t].sc);  // in registers already: else the lane's pick becomes a load of its own
              const uint32_t sdw = kg == 0 ? p[t].sc.x : kg == 1 ? p[t].sc.y : kg == 2 ? p[t].sc.z : p[t].sc.w;
              h4 Bb;
#pragma unroll
              for (int t4 = 0; t4 < 4; t4++) Bb[t4] = _Float16(int(int8_t(sdw >> (8 * t4))));
              const f4 Cb = __builtin_amdgcn_mfma_f32_16x16x16f16(Ab, Bb, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
              for (int tl = 0; tl < NTA; tl++) isum[t][tl][0] -= 32 * int(Cb[tl]);
            }
          }
          // the block's float scales, once per (tensor, token)
#pragma unroll
          for (int t = 0; t < NW; t++)
#pragma unroll
            for (int tl = 0; tl < NTA; tl++)
#pragma unroll
              for (int q = 0; q < LT; q++) {
                const float dx = *reinterpret_cast<const float*>(s_act + e_base[tl][q] + bo);
                float term;
                if constexpr (SEG == 2)
                  term = dx * (h2f(p[t].h.x) * float(isum[t][tl][q]) - h2f(p[t].h.x >> 16) * float(msum[t][tl][q]));
                else
                  term = dx * (h2f(p[t].dw >> p[t].dsh) * float(isum[t][tl][q]));
                acc[t][tl][q] += live ? term : 0.f;
              }
        }
        if (b == nb - 1) {  // the tile's last block: its results to LDS, accumulators reset
#pragma unroll
          for (int tl = 0; tl < NTA; tl++)
#pragma unroll
            for (int q = 0; q < LT; q++) {
              float v;
              if constexpr (GU) {
                const float g = acc[0][tl][q];
                v = g / (1.0f + expf(-g)) * acc[1][tl][q];
              } else {
                v = acc[0][tl][q];
              }
              const int t_loc = tl * TPT + kg * LT + q;  // past PT: a plane-form tile's rows of no token
              if (live && t_loc < PT) s_out[(tile * PT + t_loc) * 64 + 16 * wv + c] = v;
#pragma unroll
              for (int t = 0; t < NW; t++) acc[t][tl][q] = 0.f;
            }
        }
      };
      // an even number of steps (a padding step when odd): the loop's only exit is at the bottom
      for (int s_ = 0;; s_ += 2) {
        load(s_ + 1, pb);
        __builtin_amdgcn_sched_barrier(0);
        process(s_, pa);
        load(s_ + 2, pa);  // the last one is redundant (clamped)
        __builtin_amdgcn_sched_barrier(0);
        process(s_ + 1, pb);
        if (s_ + 2 >= steps) break;
      }
      // the next item's number goes out before the flush's stores: its wait then waits for no store
      if (threadIdx.x == 0) s_item = int(nxt);
    };
    kloop(std::integral_constant<int, NT>{});
    lds_barrier();  // s_out and s_item; every thread read the item's s_tok and s_item long ago
    item = s_item;
    // no barrier after the flush: the next item writes s_tok and s_act before its staging
    // barrier and s_out only after it, and nobody reads those here
    for (int idx = threadIdx.x; idx < tiles * nch * 64; idx += 256) {
      const int tile = idx / (nch * 64), rem = idx - tile * nch * 64, t = rem / 64, w = (rem / 16) & 3, cc = rem & 15;
      const int row = (part * 4 + w) * tiles * 16 + 16 * tile + cc;
      out[int64_t(i0 + t) * R + row] = s_out[(tile * PT + t) * 64 + 16 * w + cc];
    }
  }
}

__global__ void __launch_bounds__(256) moe_combine_kernel(const float* __restrict__ yd, const float* __restrict__ w,
                                                          const int32_t* __restrict__ inv, int T, int k, int H,
                                                          float* __restrict__ y, int accumulate,
                                                          float* __restrict__ resid) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= int64_t(T) * H) return;
  const int t = int(idx / H), h = int(idx % H);
  float acc = accumulate ? y[idx] : 0.f;
  for (int j = 0; j < k; j++) acc += w[t * k + j] * yd[int64_t(inv[t * k + j]) * H + h];
  if (resid) resid[idx] += acc;
  else y[idx] = acc;
}

// ---------------------------------------------------------------- launch plumbing

// Passes of pt tokens over n (token, slot) pairs among E experts: at most one partial pass per
// active expert.
int64_t moe_max_passes(int64_t n, int64_t E, int pt) { return (n + (pt - 1) * std::min(n, E)) / pt; }
// Descriptor ints for either pass size.
int64_t moe_pass_area(int64_t n, int64_t E) {
  return std::max(moe_max_passes(n, E, kMoePassTokens) * (4 + kMoePassTokens),
                  moe_max_passes(n, E, kMoePassTokensWide) * (4 + kMoePassTokensWide));
}

// Bytes between the tokens' Q8_K rows in the workspace: a row rounded up to 16 bytes, so that the
// expert GEMMs stage them in 16-byte pieces.
int64_t moe_xq_rb(int64_t hidden) { return (row_bytes(JERO_Q8_K, hidden) + 15) & ~int64_t(15); }

namespace {

int lpr_for(int U) { return U > 32 ? 64 : U > 16 ? 32 : U > 4 ? 16 : 4; }

// Work per wave: an even number of row pairs (2 .. 16), enough that the grid is about 4096 waves.
template <int F, int LPR, int UPL, int SPER>
void gate_up_one(const MoeArgs& a, const MoeLists& L, const MoeSingle& one, hipStream_t s) {
  constexpr int P = (kWave / LPR) / 2;
  const int U = units_per_row(F, a.hidden);
  const int64_t pairs = int64_t(a.max_active) * a.ffn;
  const int ppw = 2 * int(std::min<int64_t>(8, std::max<int64_t>(1, pairs / (int64_t(P) * 8192))));  // even
  const int wg_per_expert = int((a.ffn + 4 * P * ppw - 1) / (4 * P * ppw));
  const int64_t xrb = moe_xq_rb(a.hidden);
  // an expert holds at most T of the (token, slot) pairs: size the LDS stage for no more
  const int chunk = int(std::max<int64_t>(1, std::min<int64_t>({kMoeTokChunk, kMoeStageBytes / xrb, a.T})));
  hipLaunchKernelGGL((moe_gate_up_kernel<F, LPR, UPL, SPER>), dim3(unsigned(int64_t(a.max_active) * wg_per_expert)),
                     dim3(256), size_t(chunk) * size_t(xrb + 4 * 4 * P * ppw), s, static_cast<const uint8_t*>(a.gate),
                     static_cast<const uint8_t*>(a.up), a.E * a.ffn, row_bytes(F, a.hidden), U, int(a.ffn), a.top_k,
                     a.xq, xrb, L, a.act, ppw, wg_per_expert, chunk, one);
}

// SPER > 0: the single-token path (the kernel routes with SPER expert columns per lane).
template <int F, int SPER = 0>
int gate_up_fmt(const MoeArgs& a, const MoeLists& L, hipStream_t s, const MoeSingle& one = MoeSingle{}) {
  const int U = units_per_row(F, a.hidden);
  // a gate row and its up row share a wave: at most 32 lanes per row, more units per lane beyond
  switch (lpr_for(U)) {
    case 4: gate_up_one<F, 4, 1, SPER>(a, L, one, s); return JERO_OK;
    case 16: gate_up_one<F, 16, 1, SPER>(a, L, one, s); return JERO_OK;
    case 32: gate_up_one<F, 32, 1, SPER>(a, L, one, s); return JERO_OK;
    default:
      if (U <= 64) {
        gate_up_one<F, 32, 2, SPER>(a, L, one, s);
        return JERO_OK;
      }
      if (U <= 128) {
        gate_up_one<F, 32, 4, SPER>(a, L, one, s);
        return JERO_OK;
      }
      return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: hidden " + std::to_string(a.hidden) +
                                                    " above the gate/up pairing limit (8192 for K-quants, 4096 for "
                                                    "Q8_0 / Q4_0)");
  }
}

template <int F, int LPR, int UPL>
void down_one(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  constexpr int G = kWave / LPR;
  const int U = units_per_row(F, a.ffn);
  const int64_t rows = int64_t(a.max_active) * a.hidden;
  const int rpw = 2 * int(std::min<int64_t>(8, std::max<int64_t>(1, rows / (int64_t(G) * 8192))));  // even
  const int wg_per_expert = int((a.hidden + 4 * G * rpw - 1) / (4 * G * rpw));
  const int64_t arb = row_bytes(JERO_Q8_K, a.ffn);
  const int chunk = int(std::max<int64_t>(1, std::min<int64_t>({kMoeTokChunk, kMoeStageBytes / arb, a.T})));
  hipLaunchKernelGGL((moe_down_kernel<F, LPR, UPL>), dim3(unsigned(int64_t(a.max_active) * wg_per_expert)),
                     dim3(256), size_t(chunk) * size_t(arb + 4 * 4 * G * rpw), s, static_cast<const uint8_t*>(a.down),
                     a.E * a.hidden,
                     row_bytes(F, a.ffn), U, int(a.hidden), a.act, int(a.ffn), arb, L, a.yd, rpw, wg_per_expert, chunk);
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

// One token: down rows of all k selected experts per workgroup, combined in selection order.
// Each lane group takes an even number (2) of (slot, row) units; RW rows per workgroup.
template <int F, int LPR, int UPL>
void down1_one(const MoeArgs& a, hipStream_t s) {
  constexpr int G = kWave / LPR;
  const int U = units_per_row(F, a.ffn), upg = 2;
  const int RW = std::max(1, 4 * G * upg / a.top_k);
  const int64_t arb = row_bytes(JERO_Q8_K, a.ffn);
  const size_t lds = size_t(a.top_k) * size_t(arb) + sizeof(float) * size_t(a.top_k) * RW + 292;  // + dummy block
  const bool pre = a.top_k * (a.ffn / 256) <= 4 * kDown1PreBlocks;
  hipLaunchKernelGGL((pre ? moe1_down_kernel<F, LPR, UPL, true> : moe1_down_kernel<F, LPR, UPL, false>),
                     dim3(unsigned((a.hidden + RW - 1) / RW)), dim3(256), lds, s,
                     static_cast<const uint8_t*>(a.down), a.E * a.hidden, row_bytes(F, a.ffn), U, int(a.hidden), a.act,
                     int(a.ffn), arb, a.top_k, a.sel_idx, a.sel_w, a.y, RW, upg, int(a.accumulate), a.resid);
}

template <int F>
int down1_fmt(const MoeArgs& a, hipStream_t s) {
  const int U = units_per_row(F, a.ffn);
  const int lpr = lpr_for(U);
  const int upl = (U + lpr - 1) / lpr;
  if (lpr == 4) down1_one<F, 4, 1>(a, s);
  else if (lpr == 16) down1_one<F, 16, 1>(a, s);
  else if (lpr == 32) down1_one<F, 32, 1>(a, s);
  else if (upl == 1) down1_one<F, 64, 1>(a, s);
  else if (upl == 2) down1_one<F, 64, 2>(a, s);
  else if (upl <= 4) down1_one<F, 64, 4>(a, s);
  else
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: ffn " + std::to_string(a.ffn) + " above the down-proj limit");
  return JERO_OK;
}

// Expert GEMMs on MFMA (several tokens per expert): formats with a piece loader.
bool mfma_format(int f) { return f == JERO_Q4_K || f == JERO_Q4_K_R || f == JERO_Q4_K_T || f == JERO_Q6_K_R || f == JERO_Q6_K_T; }

// Workgroups of the persistent expert-GEMM grid per CU, at most (fewer when registers or LDS
// allow fewer): enough waves to keep each CU's share of HBM busy, few enough that each item is
// short, as the kernel's tail is about one item long.
constexpr int kMfmaWgPerCu = 3;

// 16-row tiles per wave of an expert GEMM item (R, the weight rows per expert, a multiple of 64):
// gate/up (K = hidden, long rows) two, down (K = ffn, short rows) four, where they divide R.
int mfma_tiles(bool gu, int64_t R) {
  if (R % 256 == 0 && !gu) return 4;
  return R % 128 == 0 ? 2 : 1;
}

size_t mfma_lds(int nb, int tiles, int pt) {
  return size_t(pt + 1) * size_t(act_row_stride(nb)) + 304 +  // + zero row, dummy area
         sizeof(float) * size_t(tiles) * size_t(pt) * 64;     // + the results
}

template <int F, bool GU, int PT>
void mfma_one_pt(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  const int64_t K = GU ? a.hidden : a.ffn, R = GU ? a.ffn : a.hidden;
  const int U = units_per_row(F, K), nb = U / 4, tiles = mfma_tiles(GU, R);
  const int wg_per_expert = int(R / (64 * tiles));
  const size_t lds = mfma_lds(nb, tiles, PT);
  int fit = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, moe_mfma_kernel<F, GU, PT>, 256, lds) != hipSuccess || fit < 1)
    fit = 1;
  const int64_t items = moe_max_passes(a.T * a.top_k, a.E, PT) * wg_per_expert;
  const int64_t grid = std::min<int64_t>(items, int64_t(std::min(fit, kMfmaWgPerCu)) * device_info().cus);
  const uint8_t* w0 = static_cast<const uint8_t*>(GU ? a.gate : a.down);
  const uint8_t* w1 = static_cast<const uint8_t*>(GU ? a.up : a.down);
  hipLaunchKernelGGL((moe_mfma_kernel<F, GU, PT>), dim3(unsigned(grid)), dim3(256), lds, s, w0, w1, a.E * R,
                     row_bytes(F, K), U, int(R), tiles, a.xq, moe_xq_rb(a.hidden), a.act, L, GU ? a.act : a.yd,
                     wg_per_expert, GU ? kMoeCtrGateUp : kMoeCtrDown);
}

template <int F, bool GU>
void mfma_one(const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  if constexpr (GU && mfma_seg(F) == 4) {
    mfma_one_pt<F, GU, kMoePassTokens>(a, L, s);  // launch_moe gives Q6_K gate/up no wide passes
  } else {
    if (L.pass_tokens == kMoePassTokensWide) mfma_one_pt<F, GU, kMoePassTokensWide>(a, L, s);
    else mfma_one_pt<F, GU, kMoePassTokens>(a, L, s);
  }
}

template <bool GU>
void mfma_fmt(int f, const MoeArgs& a, const MoeLists& L, hipStream_t s) {
  switch (f) {
    case JERO_Q4_K: mfma_one<JERO_Q4_K, GU>(a, L, s); break;
    case JERO_Q4_K_R: mfma_one<JERO_Q4_K_R, GU>(a, L, s); break;
    case JERO_Q4_K_T: mfma_one<JERO_Q4_K_T, GU>(a, L, s); break;
    case JERO_Q6_K_T: mfma_one<JERO_Q6_K_T, GU>(a, L, s); break;
    default: mfma_one<JERO_Q6_K_R, GU>(a, L, s); break;
  }
}

}  // namespace

size_t moe_workspace_bytes(int64_t T, int64_t E, int top_k, int64_t hidden, int64_t ffn) {
  const int64_t n = T * top_k;
  size_t b = 0;
  auto add = [&](size_t x) { b += (x + 255) & ~size_t(255); };
  add(size_t(T) * size_t(moe_xq_rb(hidden)));             // xq
  add(sizeof(int32_t) * size_t(E + 1));                    // offset
  add(sizeof(int32_t) * size_t(E));                        // active
  add(sizeof(int32_t));                                    // n_active
  add(sizeof(int32_t) * size_t(n) * 2);                    // entry, inv
  add(sizeof(int32_t) * size_t(moe_pass_area(n, E)));  // pass descriptors
  add(sizeof(int32_t) * kMoeCtrInts);                                   // pass count, work counters
  add(sizeof(float) * size_t(n) * size_t(ffn));            // act
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
  const int64_t xq_rb = moe_xq_rb(a.hidden);
  a.xq = take(size_t(a.T) * size_t(xq_rb));
  MoeLists L{};
  L.offset = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(a.E + 1)));
  L.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(a.E)));
  L.n_active = reinterpret_cast<int32_t*>(take(sizeof(int32_t)));
  int32_t* ei = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(n) * 2));
  L.entry = ei;
  L.inv = ei + n;
  int32_t* pass = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(moe_pass_area(n, a.E))));
  int32_t* ctr = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * kMoeCtrInts));
  a.act = reinterpret_cast<float*>(take(sizeof(float) * size_t(a.ffn) * size_t(n)));
  a.yd = reinterpret_cast<float*>(take(sizeof(float) * size_t(n) * size_t(a.hidden)));
  a.max_active = int(n < a.E ? n : a.E);
  // several tokens per expert on average: the MFMA expert GEMMs (a token's dot products come
  // out of the matrix cores instead of one cross-lane reduction per token and row); they start
  // from the pass descriptors and work counters, written by the grouping step
  const bool mfma = a.T * a.top_k >= 2 * a.E && n <= kRouteLdsPairs && mfma_format(a.gate_quant) &&
                    mfma_format(a.down_quant) && a.hidden % 64 == 0 && a.ffn % 64 == 0 &&  // whole 64-row items
                    kMoePassTokens * (xq_rb / 16) <= kStageChunks * 256 &&                   // a batch: 8 rows
                    kMoePassTokens * (a.ffn / 256) <= 4 * kStageBlocks;
  // passes of 16 tokens when the experts average at least 16 (each expert's weights are then read
  // half as often) and the staged rows leave LDS for two workgroups per CU
  const int64_t nb_gu = a.hidden / 256, nb_dn = a.ffn / 256;
  const bool wide = mfma && a.T * a.top_k >= int64_t(kMoePassTokensWide) * a.E && mfma_seg(a.gate_quant) == 2 &&
                    std::max(mfma_lds(int(nb_gu), mfma_tiles(true, a.ffn), kMoePassTokensWide),
                             mfma_lds(int(nb_dn), mfma_tiles(false, a.hidden), kMoePassTokensWide)) <= 80 * 1024;
  L.pass = mfma ? pass : nullptr;
  L.pass_tokens = wide ? kMoePassTokensWide : kMoePassTokens;
  L.ctr = ctr;

  // one token among at most 128 experts: two launches.  Gate/up routes and quantizes the token
  // itself (every workgroup alike), down takes all k selected experts' rows per workgroup and
  // sums them in selection order: no grouping, no combine.
  if (a.T == 1 && a.E <= 128) {
    const MoeSingle one{a.logits, a.x, int(a.E), int(a.hidden), a.sel_idx, a.sel_w};
    int rc;
    switch (a.gate_quant) {
      case JERO_Q4_K: rc = gate_up_fmt<JERO_Q4_K, 2>(a, L, s, one); break;
      case JERO_Q4_K_R: rc = gate_up_fmt<JERO_Q4_K_R, 2>(a, L, s, one); break;
      case JERO_Q4_K_T: rc = gate_up_fmt<JERO_Q4_K_T, 2>(a, L, s, one); break;
      case JERO_Q6_K_T: rc = gate_up_fmt<JERO_Q6_K_T, 2>(a, L, s, one); break;
      case JERO_Q6_K: rc = gate_up_fmt<JERO_Q6_K, 2>(a, L, s, one); break;
      case JERO_Q8_0: rc = gate_up_fmt<JERO_Q8_0, 2>(a, L, s, one); break;
      case JERO_Q4_0: rc = gate_up_fmt<JERO_Q4_0, 2>(a, L, s, one); break;
      default: rc = gate_up_fmt<JERO_Q6_K_R, 2>(a, L, s, one); break;
    }
    if (rc) return rc;
    rc = check_launch("moe gate/up");
    if (rc) return rc;
    switch (a.down_quant) {
      case JERO_Q4_K: rc = down1_fmt<JERO_Q4_K>(a, s); break;
      case JERO_Q4_K_R: rc = down1_fmt<JERO_Q4_K_R>(a, s); break;
      case JERO_Q4_K_T: rc = down1_fmt<JERO_Q4_K_T>(a, s); break;
      case JERO_Q6_K_T: rc = down1_fmt<JERO_Q6_K_T>(a, s); break;
      case JERO_Q6_K: rc = down1_fmt<JERO_Q6_K>(a, s); break;
      case JERO_Q8_0: rc = down1_fmt<JERO_Q8_0>(a, s); break;
      case JERO_Q4_0: rc = down1_fmt<JERO_Q4_0>(a, s); break;
      default: rc = down1_fmt<JERO_Q6_K_R>(a, s); break;
    }
    if (rc) return rc;
    return check_launch("moe down");
  }

  // few tokens: one workgroup quantizes, routes and groups; many: quantize and route over many
  // workgroups, then group in one
  const bool single = a.T * (a.hidden / 256) <= 2 * (kRouteThreads / kWave);
  const int per = a.E <= 128 ? 2 : a.E <= 256 ? 4 : a.E <= 512 ? 8 : 16;
  const int n_quant_wg = int(std::min<int64_t>(1024, (a.T * (a.hidden / 256) + 3) / 4));
  const unsigned prep_grid = unsigned(n_quant_wg + (a.T + 3) / 4);
  const int aq8 = act_is_q8(a.gate_quant);  // the hidden rows' activation format: the gate/up weights'
#define JERO_ROUTE(P)                                                                                            \
  do {                                                                                                           \
    if (single)                                                                                                  \
      hipLaunchKernelGGL(moe_route_kernel<P>, dim3(1), dim3(kRouteThreads), 0, s, a.logits, int(a.T), int(a.E),  \
                         a.top_k, a.sel_idx, a.sel_w, L, a.x, int(a.hidden), a.xq, xq_rb, aq8);                 \
    else                                                                                                         \
      hipLaunchKernelGGL(moe_prep_kernel<P>, dim3(prep_grid), dim3(256), 0, s, a.logits, int(a.T), int(a.E),     \
                         a.top_k, a.sel_idx, a.sel_w, a.x, int(a.hidden), a.xq, xq_rb, n_quant_wg, aq8);        \
  } while (0)
  if (per == 2) JERO_ROUTE(2);
  else if (per == 4) JERO_ROUTE(4);
  else if (per == 8) JERO_ROUTE(8);
  else JERO_ROUTE(16);
#undef JERO_ROUTE
  int rc = check_launch("moe route");
  if (rc) return rc;
  if (!single) {
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(kRouteThreads), 0, s, a.sel_idx, int(n), int(a.E), a.top_k, L);
    rc = check_launch("moe group");
    if (rc) return rc;
  }
  if (mfma) {
    mfma_fmt<true>(a.gate_quant, a, L, s);
    rc = check_launch("moe gate/up");
    if (rc) return rc;
    mfma_fmt<false>(a.down_quant, a, L, s);
    rc = check_launch("moe down");
    if (rc) return rc;
  } else {
  switch (a.gate_quant) {
    case JERO_Q4_K: rc = gate_up_fmt<JERO_Q4_K>(a, L, s); break;
    case JERO_Q4_K_R: rc = gate_up_fmt<JERO_Q4_K_R>(a, L, s); break;
    case JERO_Q4_K_T: rc = gate_up_fmt<JERO_Q4_K_T>(a, L, s); break;
    case JERO_Q6_K_T: rc = gate_up_fmt<JERO_Q6_K_T>(a, L, s); break;
    case JERO_Q6_K: rc = gate_up_fmt<JERO_Q6_K>(a, L, s); break;
    case JERO_Q8_0: rc = gate_up_fmt<JERO_Q8_0>(a, L, s); break;
    case JERO_Q4_0: rc = gate_up_fmt<JERO_Q4_0>(a, L, s); break;
    default: rc = gate_up_fmt<JERO_Q6_K_R>(a, L, s); break;
  }
  if (rc) return rc;
  rc = check_launch("moe gate/up");
  if (rc) return rc;
  switch (a.down_quant) {
    case JERO_Q4_K: rc = down_fmt<JERO_Q4_K>(a, L, s); break;
    case JERO_Q4_K_R: rc = down_fmt<JERO_Q4_K_R>(a, L, s); break;
    case JERO_Q4_K_T: rc = down_fmt<JERO_Q4_K_T>(a, L, s); break;
    case JERO_Q6_K_T: rc = down_fmt<JERO_Q6_K_T>(a, L, s); break;
    case JERO_Q6_K: rc = down_fmt<JERO_Q6_K>(a, L, s); break;
    case JERO_Q8_0: rc = down_fmt<JERO_Q8_0>(a, L, s); break;
    case JERO_Q4_0: rc = down_fmt<JERO_Q4_0>(a, L, s); break;
    default: rc = down_fmt<JERO_Q6_K_R>(a, L, s); break;
  }
  if (rc) return rc;
  rc = check_launch("moe down");
  if (rc) return rc;
  }
  const int64_t total = a.T * a.hidden;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, a.yd, a.sel_w, L.inv,
                     int(a.T), a.top_k, int(a.hidden), a.y, int(a.accumulate), a.resid);
  return check_launch("moe combine");
}

int check_moe_args(const MoeArgs& a, size_t gate_bytes, size_t up_bytes, size_t down_bytes) {
  if (a.E <= 0 || a.top_k <= 0) return fail(JERO_ERR_ROUTING_UNAVAILABLE, "moe: no experts to route to");
  if (!a.x || !a.logits || !a.gate || !a.up || !a.down || !a.y || !a.sel_idx || !a.sel_w)
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe: null pointer");
  if (a.T <= 0 || a.hidden <= 0 || a.ffn <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "moe: empty input");
  if (a.top_k > a.E || a.top_k > kMaxTopK || a.E > kMaxExperts)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: top_k must be <= min(n_experts, 16), n_experts <= 1024");
  auto expert_format = [](int f) { return is_kquant(f) || act_is_q8(f); };
  if (a.gate_quant != a.up_quant || !expert_format(a.gate_quant) || !expert_format(a.down_quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "moe: gate/up must share one format; gate/up and down each Q4_K or "
                                              "Q6_K (GGUF, repacked _R or tiled _T layouts), Q8_0 or Q4_0");
  int64_t rg = row_bytes(a.gate_quant, a.hidden), rd = row_bytes(a.down_quant, a.ffn);
  // (the activations are quantized in 256-element groups, whatever the format)
  if (rg < 0 || rd < 0 || a.hidden % 256 || a.ffn % 256)
    return fail(JERO_ERR_TENSOR_BOUNDS, "moe: hidden/ffn not multiples of 256");
  if (uint64_t(rg) * a.ffn * a.E > gate_bytes || uint64_t(rg) * a.ffn * a.E > up_bytes ||
      uint64_t(rd) * a.hidden * a.E > down_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "moe: stacked expert tensors smaller than [E][rows][cols]");
  if (!aligned4(a.gate) || !aligned4(a.up) || !aligned4(a.down) || (reinterpret_cast<uintptr_t>(a.x) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe: weights 4-byte and x 16-byte aligned");
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if ((is_planar(a.gate_quant) && (!a16(a.gate) || !a16(a.up))) || (is_planar(a.down_quant) && !a16(a.down)))
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe: repacked (_R, _T) expert tensors must be 16-byte aligned");
  return JERO_OK;
}

}  // namespace jero

using namespace jero;

namespace {
int moe_entry(const float* x_dev, const float* router_logits_dev, int64_t n_tokens, int64_t n_experts, int top_k,
              int gate_quant, const void* gate_dev, size_t gate_bytes, int up_quant, const void* up_dev,
              size_t up_bytes, int down_quant, const void* down_dev, size_t down_bytes, int64_t hidden, int64_t ffn,
              float* y_dev, int32_t* sel_idx_dev, float* sel_w_dev, void* workspace_dev, size_t workspace_bytes,
              void* stream, bool accumulate) {
  MoeArgs a{};
  a.accumulate = accumulate;
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
}  // namespace

extern "C" int jero_hip_moe_ffn(const float* x_dev, const float* router_logits_dev, int64_t n_tokens,
                                int64_t n_experts, int top_k, int gate_quant, const void* gate_dev, size_t gate_bytes,
                                int up_quant, const void* up_dev, size_t up_bytes, int down_quant,
                                const void* down_dev, size_t down_bytes, int64_t hidden, int64_t ffn, float* y_dev,
                                int32_t* sel_idx_dev, float* sel_w_dev, void* workspace_dev, size_t workspace_bytes,
                                void* stream) {
  return moe_entry(x_dev, router_logits_dev, n_tokens, n_experts, top_k, gate_quant, gate_dev, gate_bytes, up_quant,
                   up_dev, up_bytes, down_quant, down_dev, down_bytes, hidden, ffn, y_dev, sel_idx_dev, sel_w_dev,
                   workspace_dev, workspace_bytes, stream, false);
}

extern "C" int jero_hip_moe_ffn_acc(const float* x_dev, const float* router_logits_dev, int64_t n_tokens,
                                    int64_t n_experts, int top_k, int gate_quant, const void* gate_dev,
                                    size_t gate_bytes, int up_quant, const void* up_dev, size_t up_bytes,
                                    int down_quant, const void* down_dev, size_t down_bytes, int64_t hidden,
                                    int64_t ffn, float* y_dev, int32_t* sel_idx_dev, float* sel_w_dev,
                                    void* workspace_dev, size_t workspace_bytes, void* stream) {
  return moe_entry(x_dev, router_logits_dev, n_tokens, n_experts, top_k, gate_quant, gate_dev, gate_bytes, up_quant,
                   up_dev, up_bytes, down_quant, down_dev, down_bytes, hidden, ffn, y_dev, sel_idx_dev, sel_w_dev,
                   workspace_dev, workspace_bytes, stream, true);
}

extern "C" int jero_hip_moe_trace_view(void* workspace_dev, int64_t n_tokens, int64_t n_experts, int top_k,
                                       int64_t hidden, int64_t ffn, float** act_dev, int32_t** pair_row_dev,
                                       int* identity) {
  if (!workspace_dev || !act_dev || !pair_row_dev || !identity)
    return fail(JERO_ERR_INVALID_ARGUMENT, "moe_trace_view: null pointer");
  if (n_tokens <= 0 || n_experts <= 0 || top_k <= 0 || hidden <= 0 || ffn <= 0)
    return fail(JERO_ERR_TENSOR_BOUNDS, "moe_trace_view: empty shape");
  // the carve-out of launch_moe, in the same order
  const int64_t n = n_tokens * top_k;
  uint8_t* p = static_cast<uint8_t*>(workspace_dev);
  auto take = [&](size_t x) {
    uint8_t* r = p;
    p += (x + 255) & ~size_t(255);
    return r;
  };
  take(size_t(n_tokens) * size_t(moe_xq_rb(hidden)));
  take(sizeof(int32_t) * size_t(n_experts + 1));
  take(sizeof(int32_t) * size_t(n_experts));
  take(sizeof(int32_t));
  int32_t* ei = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * size_t(n) * 2));
  take(sizeof(int32_t) * size_t(moe_pass_area(n, n_experts)));
  take(sizeof(int32_t) * kMoeCtrInts);
  *act_dev = reinterpret_cast<float*>(take(sizeof(float) * size_t(ffn) * size_t(n)));
  *pair_row_dev = ei + n;
  *identity = (n_tokens == 1 && n_experts <= 128) ? 1 : 0;  // the one-token path keeps rows in selection order
  return JERO_OK;
}

extern "C" size_t jero_hip_moe_workspace_bytes(int64_t n_tokens, int64_t n_experts, int top_k, int64_t hidden,
                                               int64_t ffn) {
  return moe_workspace_bytes(n_tokens, n_experts, top_k, hidden, ffn);
}
