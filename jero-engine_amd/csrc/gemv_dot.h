// gemv_dot.h -- per-format "unit" dot products of the GEMV kernels.
//
// A unit is the slice of one weight row that one lane reduces per step:
//   Q4_K : 64 elements = one (super-block b, 64-element group i): the 16-byte block header
//          (d, dmin, 12 scale bytes) and the 32 bytes qs[32i, 32i+32) -> sub-blocks 2i, 2i+1
//   Q6_K : 64 elements = (block b, half n, 16-lane group j): ql[64n+16j..+16], ql[64n+32+16j..+16],
//          qh[32n+16j..+16], four int8 scales sc[8n+j+2t], d -> four 16-element groups
//   Q8_0 : 32 elements = one block (f16 d + 32 int8)
//   Q4_0 : 32 elements = one block (f16 d + 16 nibble bytes)
// Act<F> holds the matching activation slice (ACT_Q8 or Q8_K) in registers; it is loaded
// once per wave and reused for every row the wave reduces (activation-stationary GEMV).
// Integer partial sums are exact (v_dot4_i32_i8); the float combine follows the block
// formulas: Q4_K d_x (d sum sc S - dmin sum m bsum), Q6_K d_x d sum sc S, Q8_0/Q4_0 d_w d_x S.
#pragma once

#include "jero_common.h"

namespace jero {

template <int F>
struct Unit;

// ---------------------------------------------------------------- Q4_K x Q8_K
template <>
struct Unit<JERO_Q4_K> {
  static constexpr int kElems = 64;
  static constexpr int kPartials = 2;  // two 32-element sub-blocks
  // index of partial t of unit u within the row's partial sums (one per 32 elements)
  static __device__ __forceinline__ int part_index(int u, int t) { return 2 * u + t; }

  struct Act {
    uint32_t a[16];
    float dx;
    int bsa, bsb;
    uint32_t jj0, hi;  // scale byte index of sub-block 2i (mod 4), and i >= 2
  };
  struct W {
    u32x4 h, q0, q1;
  };

  static __device__ __forceinline__ void load_act(Act& A, const uint8_t* __restrict__ xq, int u) {
    int b = u >> 2, i = u & 3;
    const uint8_t* blk = xq + int64_t(b) * 292;
    A.dx = *reinterpret_cast<const float*>(blk);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      u32x4 v = ld4(blk + 4 + 64 * i + 16 * t);
      A.a[4 * t + 0] = v.x;
      A.a[4 * t + 1] = v.y;
      A.a[4 * t + 2] = v.z;
      A.a[4 * t + 3] = v.w;
    }
    u32x2 bs = ld2(blk + 260 + 8 * i);
    A.bsa = int(int16_t(bs.x & 0xFFFFu)) + int(int16_t(bs.x >> 16));
    A.bsb = int(int16_t(bs.y & 0xFFFFu)) + int(int16_t(bs.y >> 16));
    A.jj0 = uint32_t((2 * i) & 3);
    A.hi = uint32_t(i >= 2);
  }

  template <bool NT = false>  // NT: non-temporal loads (the weights of a single-pass GEMV)
  static __device__ __forceinline__ void load_w(W& w, const uint8_t* __restrict__ row, int u) {
    int b = u >> 2, i = u & 3;
    const uint8_t* blk = row + int64_t(b) * 144;
    w.h = ldx4<NT>(blk);
    w.q0 = ldx4<NT>(blk + 16 + 32 * i);
    w.q1 = ldx4<NT>(blk + 32 + 32 * i);
  }

  // 6-bit scale and min of sub-block with scale byte index jj (see get_scale_min_k4).
  static __device__ __forceinline__ void scale_min(const W& w, uint32_t jj, uint32_t hi, int& sc, int& m) {
    uint32_t a = byte_of(w.h.y, jj), bb = byte_of(w.h.z, jj), c = byte_of(w.h.w, jj);
    uint32_t sc_lo = a & 63u, m_lo = bb & 63u;
    uint32_t sc_hi = (c & 15u) | ((a >> 6) << 4), m_hi = (c >> 4) | ((bb >> 6) << 4);
    sc = int(hi ? sc_hi : sc_lo);
    m = int(hi ? m_hi : m_lo);
  }

  static __device__ __forceinline__ float dot(const W& w, const Act& A, int32_t* part) {
    uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    int sa = 0, sb = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      sa = dot4(q[t] & 0x0F0F0F0Fu, A.a[t], sa);
      sb = dot4((q[t] >> 4) & 0x0F0F0F0Fu, A.a[8 + t], sb);
    }
    if (part) {
      part[0] = sa;
      part[1] = sb;
    }
    int sca, ma, scb, mb;
    scale_min(w, A.jj0, A.hi, sca, ma);
    scale_min(w, A.jj0 + 1u, A.hi, scb, mb);
    int isum = sca * sa + scb * sb;
    int msum = ma * A.bsa + mb * A.bsb;
    float d = h2f(w.h.x), dmin = h2f(w.h.x >> 16);
    return A.dx * (d * float(isum) - dmin * float(msum));
  }

  // The unit unpacked once for dot products with several activation vectors (the same integer
  // sums and float operations as dot, so the same bits).
  struct Prep {
    uint32_t v[16];  // nibbles of sub-block 2i (v[0..8)) and 2i+1 (v[8..16))
    int sca, scb, ma, mb;
    float d, dmin;
  };
  static __device__ __forceinline__ void prep(Prep& p, const W& w, int u) {
    const uint32_t q[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
#pragma unroll
    for (int t = 0; t < 8; t++) {
      p.v[t] = q[t] & 0x0F0F0F0Fu;
      p.v[8 + t] = (q[t] >> 4) & 0x0F0F0F0Fu;
    }
    const int i = u & 3;
    scale_min(w, uint32_t((2 * i) & 3), uint32_t(i >= 2), p.sca, p.ma);
    scale_min(w, uint32_t((2 * i) & 3) + 1u, uint32_t(i >= 2), p.scb, p.mb);
    p.d = h2f(w.h.x);
    p.dmin = h2f(w.h.x >> 16);
  }
  static __device__ __forceinline__ float dot_prep(const Prep& p, const Act& A) {
    int sa = 0, sb = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      sa = dot4(p.v[t], A.a[t], sa);
      sb = dot4(p.v[8 + t], A.a[8 + t], sb);
    }
    const int isum = p.sca * sa + p.scb * sb;
    const int msum = p.ma * A.bsa + p.mb * A.bsb;
    return A.dx * (p.d * float(isum) - p.dmin * float(msum));
  }
};

// ---------------------------------------------------------------- Q4_K, planar device layout
// JERO_Q4_K_R keeps each row of a Q4_K tensor (nb blocks, U = 4 nb units of 64 elements) in
// its own 144 nb bytes, regrouped into three runs, so that each 16-byte load instruction of a
// wave reads one contiguous kilobyte (the GGUF layout spreads a wave's loads over every line
// of its blocks) while a row stays one contiguous range:
//   row = q0 [U][16] | q1 [U][16] | h [nb][16]
//   q0[u] = qs[32i .. 32i+16), q1[u] = qs[32i+16 .. 32i+32) of block b (unit u = 4b+i);
//   h[b] = d, dmin, scales[12] (the block's first 16 bytes).
// Same size as the GGUF tensor; the dot product is Unit<Q4_K>'s.
template <>
struct Unit<JERO_Q4_K_R> : Unit<JERO_Q4_K> {
  template <bool NT = false>
  static __device__ __forceinline__ void load_w_planar(W& w, const uint8_t* __restrict__ base, int64_t /*N*/, int U,
                                                       int64_t row, int u) {
    const uint8_t* rp = base + row * (int64_t(U) * 36);
    w.q0 = ldx4<NT>(rp + u * 16);
    w.q1 = ldx4<NT>(rp + U * 16 + u * 16);
    w.h = ldx4<NT>(rp + U * 32 + (u >> 2) * 16);
  }
};

// ---------------------------------------------------------------- Q4_K, 16-row tiles (experts)
// JERO_Q4_K_T holds a Q4_K tensor of N rows (N a multiple of 16) as pieces of 2304 bytes, one per
// (tile of 16 rows, block column b), tiles in row order and, within a tile, b ascending:
//   piece = q [4 units i][2 runs][16 rows][16] | h [16 rows][16]
//   q[i][0][c] = qs[32i .. 32i+16), q[i][1][c] = qs[32i+16 .. 32i+32) of row c's block b;
//   h[c] = that block's first 16 bytes (d, dmin, scales).
// A wave's loads of one 16-row block column then read whole contiguous pieces: the expert GEMMs
// step over 16 rows block by block, and the per-row runs of Q4_K_R would have them touch 64 bytes
// in each of 32 places (measured 3.1 against 5.5 TB/s for the same bytes read contiguously).
template <>
struct Unit<JERO_Q4_K_T> : Unit<JERO_Q4_K> {
  static __device__ __forceinline__ void load_w_planar(W& w, const uint8_t* __restrict__ base, int64_t /*N*/, int U,
                                                       int64_t row, int u) {
    const int c = int(row & 15), i = u & 3;
    const uint8_t* pc = base + ((row >> 4) * (U / 4) + (u >> 2)) * 2304;
    w.q0 = ld4(pc + ((2 * i) * 16 + c) * 16);
    w.q1 = ld4(pc + ((2 * i + 1) * 16 + c) * 16);
    w.h = ld4(pc + 2048 + c * 16);
  }
};

// ---------------------------------------------------------------- Q6_K x Q8_K
template <>
struct Unit<JERO_Q6_K> {
  static constexpr int kElems = 64;
  static constexpr int kPartials = 4;  // four 16-element groups
  // group index (one per 16 elements) of partial t of unit u = 4b + 2n + j: 16b + 8n + j + 2t
  static __device__ __forceinline__ int part_index(int u, int t) {
    return 16 * (u >> 2) + 8 * ((u >> 1) & 1) + (u & 1) + 2 * t;
  }

  struct Act {
    uint32_t a[16];  // a[4t + k]: q8 of group t, dword k
    float dx;
    int bs32[4];     // 32 * bsum of group t
  };
  // d stays as the loaded dword and the shift of its f16 (converted in dot): converting at
  // the load would make the compiler wait for the load wherever it places the conversion.
  struct W {
    u32x4 lo, hi, qh;
    uint32_t sc;  // the unit's four int8 scales sc[8n+j+2t], t = 0..3, one per byte
    uint32_t dw, dsh;
  };
  // f16 at a 2-byte aligned address: the dword holding it and its bit shift.
  static __device__ __forceinline__ void load_d(W& w, const uint8_t* __restrict__ p) {
    const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
    w.dw = ld1(p - s);
    w.dsh = 8u * s;
  }

  static __device__ __forceinline__ void load_act(Act& A, const uint8_t* __restrict__ xq, int u) {
    int b = u >> 2, n = (u >> 1) & 1, j = u & 1;
    const uint8_t* blk = xq + int64_t(b) * 292;
    A.dx = *reinterpret_cast<const float*>(blk);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      u32x4 v = ld4(blk + 4 + 128 * n + 16 * j + 32 * t);
      A.a[4 * t + 0] = v.x;
      A.a[4 * t + 1] = v.y;
      A.a[4 * t + 2] = v.z;
      A.a[4 * t + 3] = v.w;
    }
    u32x4 bs = ld4(blk + 260 + 16 * n);  // bsums[8n .. 8n+8)
    uint32_t dw[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
    for (int t = 0; t < 4; t++) A.bs32[t] = 32 * int(int16_t((dw[t] >> (16 * j)) & 0xFFFFu));
  }

  // Raw GGUF layout: block b of the row, pieces of unit (n, j); 2-byte aligned reads.
  static __device__ __forceinline__ void load_w(W& w, const uint8_t* __restrict__ row, int u) {
    int b = u >> 2, n = (u >> 1) & 1, j = u & 1;
    const uint8_t* blk = row + int64_t(b) * 210;
    w.lo = ld16_a2(blk + 64 * n + 16 * j);
    w.hi = ld16_a2(blk + 64 * n + 32 + 16 * j);
    w.qh = ld16_a2(blk + 128 + 32 * n + 16 * j);
    u32x2 sc = ld8_a2(blk + 192 + 8 * n);
    uint32_t sh = 8u * uint32_t(j);
    w.sc = ((sc.x >> sh) & 0xFFu) | (((sc.x >> (sh + 16u)) & 0xFFu) << 8) | (((sc.y >> sh) & 0xFFu) << 16) |
           (((sc.y >> (sh + 16u)) & 0xFFu) << 24);
    load_d(w, blk + 208);
  }

  static __device__ __forceinline__ float dot(const W& w, const Act& A, int32_t* part) {
    uint32_t lo[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
    uint32_t hi[4] = {w.hi.x, w.hi.y, w.hi.z, w.hi.w};
    uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
    int s0 = 0, s1 = 0, s2 = 0, s3 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      uint32_t v0 = (lo[k] & 0x0F0F0F0Fu) | ((qh[k] & 0x03030303u) << 4);
      uint32_t v1 = (hi[k] & 0x0F0F0F0Fu) | ((qh[k] & 0x0C0C0C0Cu) << 2);
      uint32_t v2 = ((lo[k] >> 4) & 0x0F0F0F0Fu) | (qh[k] & 0x30303030u);
      uint32_t v3 = ((hi[k] >> 4) & 0x0F0F0F0Fu) | ((qh[k] >> 2) & 0x30303030u);
      s0 = dot4(v0, A.a[0 + k], s0);
      s1 = dot4(v1, A.a[4 + k], s1);
      s2 = dot4(v2, A.a[8 + k], s2);
      s3 = dot4(v3, A.a[12 + k], s3);
    }
    s0 -= A.bs32[0];
    s1 -= A.bs32[1];
    s2 -= A.bs32[2];
    s3 -= A.bs32[3];
    if (part) {
      part[0] = s0;
      part[1] = s1;
      part[2] = s2;
      part[3] = s3;
    }
    int c0 = int(int8_t(w.sc)), c1 = int(int8_t(w.sc >> 8));
    int c2 = int(int8_t(w.sc >> 16)), c3 = int(int8_t(w.sc >> 24));
    int isum = c0 * s0 + c1 * s1 + c2 * s2 + c3 * s3;
    return A.dx * h2f(w.dw >> w.dsh) * float(isum);
  }

  // The unit unpacked once for dot products with several activation vectors (same bits as dot).
  struct Prep {
    uint32_t v[16];  // v[4g + k]: 6-bit values of group g, dword k
    int c[4];
    float d;
  };
  static __device__ __forceinline__ void prep(Prep& p, const W& w, int /*u*/) {
    const uint32_t lo[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
    const uint32_t hi[4] = {w.hi.x, w.hi.y, w.hi.z, w.hi.w};
    const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      p.v[0 + k] = (lo[k] & 0x0F0F0F0Fu) | ((qh[k] & 0x03030303u) << 4);
      p.v[4 + k] = (hi[k] & 0x0F0F0F0Fu) | ((qh[k] & 0x0C0C0C0Cu) << 2);
      p.v[8 + k] = ((lo[k] >> 4) & 0x0F0F0F0Fu) | (qh[k] & 0x30303030u);
      p.v[12 + k] = ((hi[k] >> 4) & 0x0F0F0F0Fu) | ((qh[k] >> 2) & 0x30303030u);
    }
#pragma unroll
    for (int g = 0; g < 4; g++) p.c[g] = int(int8_t(w.sc >> (8 * g)));
    p.d = h2f(w.dw >> w.dsh);
  }
  static __device__ __forceinline__ float dot_prep(const Prep& p, const Act& A) {
    int sg[4] = {0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int g = 0; g < 4; g++) sg[g] = dot4(p.v[4 * g + k], A.a[4 * g + k], sg[g]);
    int isum = 0;
#pragma unroll
    for (int g = 0; g < 4; g++) isum += p.c[g] * (sg[g] - A.bs32[g]);
    return A.dx * p.d * float(isum);
  }
};

// ---------------------------------------------------------------- Q6_K, planar device layout
// JERO_Q6_K_R holds the bytes of a Q6_K tensor of N rows and nb blocks per row (U = 4 nb
// units per row) as five planes, so that every load is 16-byte aligned and consecutive lanes
// read consecutive bytes:
//   lo [N][U][16] = ql[64n+16j .. +16]      hi [N][U][16] = ql[64n+32+16j .. +16]
//   qh [N][U][16] = qh[32n+16j .. +16]      sc [N][U][4]  = sc[8n+j+2t], t = 0..3
//   d  [N][nb] f16
// Same size as the GGUF tensor (210 bytes per block); the dot product is Unit<Q6_K>'s.
template <>
struct Unit<JERO_Q6_K_R> : Unit<JERO_Q6_K> {
  template <bool NT = false>
  static __device__ __forceinline__ void load_w_planar(W& w, const uint8_t* __restrict__ base, int64_t N, int U,
                                                       int64_t row, int u) {
    const int64_t plane = N * int64_t(U) * 16;
    const int64_t gu = row * U + u;
    w.lo = ldx4<NT>(base + gu * 16);
    w.hi = ldx4<NT>(base + plane + gu * 16);
    w.qh = ldx4<NT>(base + 2 * plane + gu * 16);
    w.sc = ldx1<NT>(base + 3 * plane + gu * 4);
    load_d(w, base + 3 * plane + N * int64_t(U) * 4 + (row * (U / 4) + (u >> 2)) * 2);
  }
};

// ---------------------------------------------------------------- Q6_K, 16-row tiles (experts)
// JERO_Q6_K_T holds a Q6_K tensor of N rows (N a multiple of 16) as pieces of 3360 bytes, one per
// (tile of 16 rows, block column b), in the order of Q4_K_T; with units u = 4b + i, i = 2n + j:
//   piece = ql [4 i][2 halves][16 rows][16] | qh [4 i][16 rows][16] | sc [16 rows][4 i][4] | d [16 rows] f16
//   ql[i][0][c] = ql[64n+16j .. +16], ql[i][1][c] = ql[64n+32+16j .. +16], qh[i][c] = qh[32n+16j .. +16],
//   sc[c][i] = sc[8n+j+2t], t = 0..3 (the Q6_K_R pieces of row c, regrouped by tile).
template <>
struct Unit<JERO_Q6_K_T> : Unit<JERO_Q6_K> {
  static __device__ __forceinline__ void load_w_planar(W& w, const uint8_t* __restrict__ base, int64_t /*N*/, int U,
                                                       int64_t row, int u) {
    const int c = int(row & 15), i = u & 3;
    const uint8_t* pc = base + ((row >> 4) * (U / 4) + (u >> 2)) * 3360;
    w.lo = ld4(pc + ((2 * i) * 16 + c) * 16);
    w.hi = ld4(pc + ((2 * i + 1) * 16 + c) * 16);
    w.qh = ld4(pc + 2048 + (i * 16 + c) * 16);
    w.sc = ld1(pc + 3072 + c * 16 + i * 4);
    load_d(w, pc + 3328 + c * 2);
  }
};

// ---------------------------------------------------------------- Q8_0 x ACT_Q8
template <>
struct Unit<JERO_Q8_0> {
  static constexpr int kElems = 32;
  static constexpr int kPartials = 1;
  static __device__ __forceinline__ int part_index(int u, int) { return u; }

  struct Act {
    uint32_t a[8];
    float dx;
  };
  struct W {
    uint32_t D[9];
    uint32_t s;  // byte offset of the block inside D[0] (0 or 2)
  };

  static __device__ __forceinline__ void load_act(Act& A, const uint8_t* __restrict__ xq, int u) {
    const uint8_t* blk = xq + int64_t(u) * 36;
    A.dx = *reinterpret_cast<const float*>(blk);
    u32x4 v0 = ld4(blk + 4), v1 = ld4(blk + 20);
    A.a[0] = v0.x; A.a[1] = v0.y; A.a[2] = v0.z; A.a[3] = v0.w;
    A.a[4] = v1.x; A.a[5] = v1.y; A.a[6] = v1.z; A.a[7] = v1.w;
  }

  // The 34-byte block is read as the nine dwords from the dword-aligned address at or below
  // it: each holds at least one byte of the block.
  static __device__ __forceinline__ void load_w(W& w, const uint8_t* __restrict__ row, int u) {
    const uint8_t* p = row + int64_t(u) * 34;
    w.s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t* base = p - w.s;  // pointer arithmetic keeps the global address space
    u32x4 v0 = ld4(base), v1 = ld4(base + 16);
    w.D[0] = v0.x; w.D[1] = v0.y; w.D[2] = v0.z; w.D[3] = v0.w;
    w.D[4] = v1.x; w.D[5] = v1.y; w.D[6] = v1.z; w.D[7] = v1.w;
    w.D[8] = ld1(base + 32);
  }

  static __device__ __forceinline__ float dot(const W& w, const Act& A, int32_t* part) {
    int s = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      uint32_t q = w.s ? w.D[t + 1] : funnel(w.D[t], w.D[t + 1], 2u);
      s = dot4(q, A.a[t], s);
    }
    if (part) part[0] = s;
    float d = h2f(w.D[0] >> (8u * w.s));
    return d * A.dx * float(s);
  }

  // the many-token form of the expert kernels: nothing to unpack ahead of the token loop
  using Prep = W;
  static __device__ __forceinline__ void prep(Prep& p, const W& w, int /*u*/) { p = w; }
  static __device__ __forceinline__ float dot_prep(const Prep& p, const Act& A) { return dot(p, A, nullptr); }
};

// ---------------------------------------------------------------- Q4_0 x ACT_Q8
template <>
struct Unit<JERO_Q4_0> {
  static constexpr int kElems = 32;
  static constexpr int kPartials = 1;
  static __device__ __forceinline__ int part_index(int u, int) { return u; }

  struct Act {
    uint32_t a[8];
    float dx;
    int asum8;  // 8 * sum of the block's q8
  };
  struct W {
    uint32_t D[5];
    uint32_t s;
  };

  static __device__ __forceinline__ void load_act(Act& A, const uint8_t* __restrict__ xq, int u) {
    const uint8_t* blk = xq + int64_t(u) * 36;
    A.dx = *reinterpret_cast<const float*>(blk);
    u32x4 v0 = ld4(blk + 4), v1 = ld4(blk + 20);
    A.a[0] = v0.x; A.a[1] = v0.y; A.a[2] = v0.z; A.a[3] = v0.w;
    A.a[4] = v1.x; A.a[5] = v1.y; A.a[6] = v1.z; A.a[7] = v1.w;
    int s = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) s = dot4(A.a[t], 0x01010101u, s);
    A.asum8 = 8 * s;
  }

  // The 18-byte block is read as the five dwords from the dword-aligned address at or below it.
  static __device__ __forceinline__ void load_w(W& w, const uint8_t* __restrict__ row, int u) {
    const uint8_t* p = row + int64_t(u) * 18;
    w.s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint8_t* base = p - w.s;  // pointer arithmetic keeps the global address space
    u32x4 v0 = ld4(base);
    w.D[0] = v0.x; w.D[1] = v0.y; w.D[2] = v0.z; w.D[3] = v0.w;
    w.D[4] = ld1(base + 16);
  }

  static __device__ __forceinline__ float dot(const W& w, const Act& A, int32_t* part) {
    int s = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      uint32_t q = w.s ? w.D[t + 1] : funnel(w.D[t], w.D[t + 1], 2u);
      s = dot4(q & 0x0F0F0F0Fu, A.a[t], s);
      s = dot4((q >> 4) & 0x0F0F0F0Fu, A.a[4 + t], s);
    }
    s -= A.asum8;
    if (part) part[0] = s;
    float d = h2f(w.D[0] >> (8u * w.s));
    return d * A.dx * float(s);
  }

  using Prep = W;
  static __device__ __forceinline__ void prep(Prep& p, const W& w, int /*u*/) { p = w; }
  static __device__ __forceinline__ float dot_prep(const Prep& p, const Act& A) { return dot(p, A, nullptr); }
};

// Units per row and partial sums per row of a weight format.  "Planar": a device layout read
// through Unit<F>::load_w_planar (16-byte aligned).
__host__ __device__ constexpr bool is_planar(int f) {
  return f == JERO_Q4_K_R || f == JERO_Q6_K_R || f == JERO_Q4_K_T || f == JERO_Q6_K_T;
}
// Formats whose weight loads have a non-temporal variant (16-byte pieces that no other load of
// the launch touches).
__host__ __device__ constexpr bool nt_capable(int f) { return f == JERO_Q4_K || f == JERO_Q4_K_R || f == JERO_Q6_K_R; }

// Loads the weights of unit u of a row through Unit<F>'s loader (non-temporal when NT).
template <int F, bool NT>
__device__ __forceinline__ void load_unit(typename Unit<F>::W& w, const uint8_t* __restrict__ base, int64_t rb,
                                          int64_t N, int U, int64_t row, int u) {
  static_assert(!NT || nt_capable(F), "no non-temporal loader for this format");
  if constexpr (is_planar(F)) {
    if constexpr (NT) Unit<F>::template load_w_planar<true>(w, base, N, U, row, u);
    else Unit<F>::load_w_planar(w, base, N, U, row, u);
  } else {
    if constexpr (NT) Unit<F>::template load_w<true>(w, base + row * rb, u);
    else Unit<F>::load_w(w, base + row * rb, u);
  }
}

__host__ __device__ constexpr bool is_q6k(int f) { return f == JERO_Q6_K || f == JERO_Q6_K_R || f == JERO_Q6_K_T; }
__host__ __device__ constexpr bool is_kquant(int f) {
  return f == JERO_Q4_K || f == JERO_Q4_K_R || f == JERO_Q4_K_T || is_q6k(f);
}
__host__ __device__ constexpr int units_per_row(int f, int64_t k) { return int(k / (is_kquant(f) ? 64 : 32)); }
__host__ __device__ constexpr int64_t partials_per_row(int f, int64_t k) { return is_q6k(f) ? k / 16 : k / 32; }

}  // namespace jero
