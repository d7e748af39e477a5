// gemm.hip -- prefill GEMM over GGUF Q4_K weights and the exact int8 GEMM, on gfx950 int8 MFMA.
//
// Q4_K x Q8_K (many tokens at once).  Row m of Y is the GEMV of x_m (the reference's prefill runs
// matvec_any token by token, src/qwen_deepseek.rs:2298-2312), so per 256-element block b:
//   y[m][n] += d_x[m,b] * (d_w[n,b] * T - dmin[n,b] * Mn),
//   T  = sum_k sc_{j(k)}[n] * q4[n][k] * q8[m][k]      (j = 32-element sub-block)
//   Mn = sum_{i<16} m_{i/2}[n] * bsum16[m][i]
// T needs the 6-bit sub-block scale inside the sum.  sc = 8a + b with a, b in 0..7 splits it
// into two int8 planes a*q4 and b*q4 (both <= 105), so T = 8 * (plane-a product) + (plane-b
// product): 16 v_mfma_i32_32x32x32_i8 per 32x32 tile and block, accumulated in one int32
// register set (shifted left by 3 between the planes), exact.  Mn is one
// v_mfma_f32_32x32x16_f16 over the 16 bsums (|bsum| <= 2032 and m <= 63 are exact in f16, the
// sums stay below 2^24).  The scales are applied once per block in f32.
//
// Tiling: a workgroup of 8 waves (two per SIMD) owns a 128 (tokens) x 128 (weight rows) tile;
// each wave a 64 x 32 piece of 2 x 1 MFMA tiles.  Per block, the 128 activation rows (int8 +
// bsums + d) and the 128 weight rows as raw Q4_K bytes are staged in LDS, double-buffered: the
// global loads of block b+1 are in flight while block b runs.  Each lane expands its own weight
// fragments to the two int8 planes and decodes its row's scales in registers.  Workgroups are
// mapped so that the ones sharing a weight tile run on one XCD (one L2).
//
// int8 x int8 -> int32 (ForwardExec::matmul, src/forward.rs:555-655, 763-811): a workgroup of
// 4 waves on the same 128 x 128 tile (each wave a 64 x 64 quadrant of 2 x 2 MFMA tiles),
// 256-wide K steps, one v_mfma_i32_32x32x32_i8 per 32 K.  The operands are row-major or in the
// packed tile layout of jero_hip_pack_tiles (read in place: the loader computes each 16-byte
// piece's address); the epilogue writes int32 rows, int8 rows requantized as forward.rs's
// `requant` (:345-350) does, or tile-major 8 x 8 blocks for gemm_i8_ime's callback (:779-796).
#include <algorithm>
#include <string>

#include "forward.h"
#include "gemv.h"
#include "jero_common.h"
#include "runtime.h"

namespace jero {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kGemmThreads = 256;  // int8 kernel
constexpr int kGemmBM = 128;       // tokens (rows of x) per workgroup tile
constexpr int kGemmBN = 128;       // weight rows per workgroup tile
constexpr int kPlaneStride = 272;  // LDS bytes per 256-byte row: 16-byte reads of 16 rows hit distinct banks
constexpr int kQ4Threads = 512;    // Q4_K kernel: 8 waves, two per SIMD

// One block (256 K-elements) of the workgroup's 128 activation rows and 128 weight rows, as
// plain copies: the weight rows stay raw Q4_K (each lane expands its fragments to the int8
// planes and decodes its row's scale fields in registers).
struct __attribute__((aligned(16))) Q4kStage {
  int8_t a[kGemmBM][kPlaneStride];  // q8 of the activation block
  uint8_t w[kGemmBN][144];          // raw Q4_K blocks (144 = 9 x 16: rows stay 16-byte aligned)
  int16_t bs[kGemmBM][16];          // activation bsums (raw)
  float dx[kGemmBM];
};

// Global data of one block for this thread: a quarter of an activation row and of a weight row.
struct Q4kRegs {
  u32x4 aq[4];  // 64 bytes of the activation row's q8
  u32x4 ax;     // quarter 0: d in .x; quarters 1, 2: bsums 0..7, 8..15
  u32x4 wc[3];  // weight row chunks q, q + 4 and (quarter 0) chunk 8
};

// Workgroup -> (weight tile, token tile): workgroup w runs on XCD w % 8; each XCD takes a
// contiguous range of tiles, which runs every token tile of one weight tile back to back.
__device__ __forceinline__ void gemm_tile_of(int wg, int n_wg, int n_tiles_m, int& tm, int& tn) {
  int l = wg;
  if ((n_wg & 7) == 0) l = (wg & 7) * (n_wg >> 3) + (wg >> 3);  // a bijection when 8 divides the grid
  tn = l / n_tiles_m;
  tm = l % n_tiles_m;
}

// Every load is unconditional (rows past M read row M-1 and are never stored).  PLANAR: the weight
// rows are in the Q4_K_R layout (each row's q0 run of U = 4 nb 16-byte pieces, its q1 run, then
// its nb block headers); the chunks land in LDS as the same raw Q4_K block, so the rest of the
// kernel, and its results, do not depend on the layout.
template <bool PLANAR>
__device__ __forceinline__ void q4k_load(Q4kRegs& R, const uint8_t* __restrict__ x, int64_t xrb, int m0, int M,
                                         const uint8_t* __restrict__ w, int64_t wrb, int n0, int b, int nb) {
  const int t = threadIdx.x, r = t >> 2, q = t & 3;
  const int m = min(m0 + r, M - 1);
  const uint8_t* xa = x + int64_t(m) * xrb + int64_t(b) * 292;
#pragma unroll
  for (int i = 0; i < 4; i++) R.aq[i] = ld4(xa + 4 + 64 * q + 16 * i);
  R.ax = ld4(xa + (q == 1 ? 260 : q == 2 ? 276 : 0));
  const uint8_t* rp = w + int64_t(n0 + r) * wrb;
  // 16-byte chunk c of the row's block b: 0 = header, 1 + i = qs bytes [16 i, 16 i + 16)
  auto chunk = [&](int c) -> const uint8_t* {
    if constexpr (!PLANAR) {
      return rp + int64_t(b) * 144 + 16 * c;
    } else {
      const int U = 4 * nb, i = c - 1;
      return c == 0 ? rp + U * 32 + b * 16 : rp + (i & 1) * U * 16 + (4 * b + (i >> 1)) * 16;
    }
  };
  R.wc[0] = ld4(chunk(q));
  R.wc[1] = ld4(chunk(q + 4));
  R.wc[2] = ld4(chunk(q == 0 ? 8 : q));
}

__device__ __forceinline__ void q4k_store(const Q4kRegs& R, Q4kStage& S) {
  const int t = threadIdx.x, r = t >> 2, q = t & 3;
#pragma unroll
  for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4*>(&S.a[r][64 * q + 16 * i]) = R.aq[i];
  *reinterpret_cast<u32x4*>(&S.w[r][16 * q]) = R.wc[0];
  *reinterpret_cast<u32x4*>(&S.w[r][16 * (q + 4)]) = R.wc[1];
  // quarter 0 writes chunk 8; the others rewrite their chunk q with the same bytes
  *reinterpret_cast<u32x4*>(&S.w[r][q == 0 ? 128 : 16 * q]) = R.wc[2];
  if (q == 0) S.dx[r] = __uint_as_float(R.ax.x);
  if (q == 1 || q == 2) *reinterpret_cast<u32x4*>(&S.bs[r][8 * (q - 1)]) = R.ax;
}

// Byte i (0..11) of the 12 packed scale bytes held in three dwords.
__device__ __forceinline__ uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
  const uint32_t w = i < 4 ? s0 : i < 8 ? s1 : s2;
  return (w >> (8 * (i & 3))) & 0xFFu;
}

__device__ __forceinline__ uint32_t pk_mul(uint32_t x, uint32_t s) {
  // four bytes times s (<= 7): per 16-bit half b0*s + (b1*s << 8), no carry since b*s <= 105
  const u16x2 r = __builtin_bit_cast(u16x2, x) * u16x2{uint16_t(s), uint16_t(s)};
  return __builtin_bit_cast(uint32_t, r);
}

template <bool PLANAR>
__global__ void __launch_bounds__(kQ4Threads) gemm_q4k_kernel(const uint8_t* __restrict__ w, int64_t wrb,
                                                               const uint8_t* __restrict__ x, int64_t xrb, int M,
                                                               int N, int nb, float* __restrict__ y) {
  __shared__ Q4kStage S[2];
  const int n_tiles_m = (M + kGemmBM - 1) / kGemmBM;
  int tm, tn;
  gemm_tile_of(blockIdx.x, gridDim.x, n_tiles_m, tm, tn);
  const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv >> 2, wn = wv & 3;  // wave tile: rows 64 wm .. +64, weight rows 32 wn .. +32
  const int lr = lane & 31, lh = lane >> 5;
  const int nl = 32 * wn + lr;

  v16f acc[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[i][v] = 0.f;

  Q4kRegs R;
  q4k_load<PLANAR>(R, x, xrb, m0, M, w, wrb, n0, 0, nb);
  q4k_store(R, S[0]);
  __syncthreads();
  for (int b = 0; b < nb; b++) {
    const Q4kStage& T = S[b & 1];
    if (b + 1 < nb) q4k_load<PLANAR>(R, x, xrb, m0, M, w, wrb, n0, b + 1, nb);
    // this lane's weight row: header d, dmin and the 6-bit scales / mins (GGUF Q4_K packing)
    const u32x4 hd = *reinterpret_cast<const u32x4*>(&T.w[nl][0]);
    uint32_t scv[8], mvv[4];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      scv[j] = j < 4 ? sbyte(hd.y, hd.z, hd.w, j) & 63u
                     : (sbyte(hd.y, hd.z, hd.w, j + 4) & 15u) | ((sbyte(hd.y, hd.z, hd.w, j - 4) >> 6) << 4);
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {  // mins of sub-blocks 4 lh + jj (this lane's half of the bsums)
      const int j = 4 * lh + jj;
      mvv[jj] = j < 4 ? sbyte(hd.y, hd.z, hd.w, j + 4) & 63u
                      : (sbyte(hd.y, hd.z, hd.w, j + 4) >> 4) | ((sbyte(hd.y, hd.z, hd.w, j) >> 6) << 4);
    }
    v16i Ca[2], Cb[2];  // plane a (sc >> 3) and plane b (sc & 7) products
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // qs bytes 32 i + 16 lh .. +16: low nibbles are sub-block 2i, high nibbles 2i + 1, at
      // K-elements 16 lh .. +16 of each (the MFMA fragment of this lane)
      const u32x4 raw = *reinterpret_cast<const u32x4*>(&T.w[nl][16 + 32 * i + 16 * lh]);
      const uint32_t s0 = scv[2 * i], s1 = scv[2 * i + 1];
      v4i pa0, pb0, pa1, pb1;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t ql = raw[e] & 0x0F0F0F0Fu, qh = (raw[e] >> 4) & 0x0F0F0F0Fu;
        pa0[e] = int(pk_mul(ql, s0 >> 3));
        pb0[e] = int(pk_mul(ql, s0 & 7u));
        pa1[e] = int(pk_mul(qh, s1 >> 3));
        pb1[e] = int(pk_mul(qh, s1 & 7u));
      }
#pragma unroll
      for (int mt = 0; mt < 2; mt++) {
        const v4i af0 = *reinterpret_cast<const v4i*>(&T.a[64 * wm + 32 * mt + lr][64 * i + 16 * lh]);
        const v4i af1 = *reinterpret_cast<const v4i*>(&T.a[64 * wm + 32 * mt + lr][64 * i + 32 + 16 * lh]);
        if (i == 0) {
          const v16i z = {};
          Ca[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pa0, z, 0, 0, 0);
          Cb[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pb0, z, 0, 0, 0);
        } else {
          Ca[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pa0, Ca[mt], 0, 0, 0);
          Cb[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pb0, Cb[mt], 0, 0, 0);
        }
        Ca[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, pa1, Ca[mt], 0, 0, 0);
        Cb[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, pb1, Cb[mt], 0, 0, 0);
      }
    }
    // mins (bsums . m over the 16 bsum groups), then the block's scales:
    // column n = lane % 32 of the tile, rows (v/4)*8 + (lane/32)*4 + v%4
    v8h mnf;
#pragma unroll
    for (int i = 0; i < 8; i++) mnf[i] = _Float16(float(mvv[i >> 1]));
    const float dw = float(__builtin_bit_cast(_Float16, uint16_t(hd.x & 0xFFFFu)));
    const float dm = float(__builtin_bit_cast(_Float16, uint16_t(hd.x >> 16)));
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
      const u32x4 braw = *reinterpret_cast<const u32x4*>(&T.bs[64 * wm + 32 * mt + lr][8 * lh]);
      v8h bsf;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        bsf[2 * i] = _Float16(float(int16_t(braw[i] & 0xFFFFu)));
        bsf[2 * i + 1] = _Float16(float(int16_t(braw[i] >> 16)));
      }
      const v16f z = {};
      const v16f Mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsf, mnf, z, 0, 0, 0);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 dx = *reinterpret_cast<const float4*>(&T.dx[64 * wm + 32 * mt + 8 * g + 4 * lh]);
        const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int v = 4 * g + e;
          const int tv = (Ca[mt][v] << 3) + Cb[mt][v];
          acc[mt][v] = fmaf(dxv[e], dw * float(tv) - dm * Mn[v], acc[mt][v]);
        }
      }
    }
    // stage b + 1 goes to the buffer every wave finished reading before the last barrier
    if (b + 1 < nb) q4k_store(R, S[(b + 1) & 1]);
    __syncthreads();
  }
  // store: for each v, the 32 lanes of a half-wave write 32 consecutive floats of one row
  const int n = n0 + nl;
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = m0 + 64 * wm + 32 * mt + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (m < M) y[int64_t(m) * N + n] = acc[mt][v];
    }
}

// ---------------------------------------------------------------- int8 x int8 -> int32

struct __attribute__((aligned(16))) I8Stage {
  int8_t a[kGemmBM][kPlaneStride];
  int8_t b[kGemmBN][kPlaneStride];
};

// Packed tile layout (jero_hip_pack_tiles): element (r, c) of a [rows][K] int8 matrix, rows
// padded with zero rows to whole tiles of kTileRows, K a multiple of kTileK, sits at byte
//   ((r / kTileRows * (K / kTileK) + c / kTileK) * kTileRows + r % kTileRows) * kTileK + c % kTileK
// i.e. tile by tile, each tile's K chunks in order, each chunk its rows' kTileK bytes in order.
constexpr int kTileRows = 8, kTileK = 32;

__device__ __forceinline__ int64_t packed_offset(int r, int c, int K) {
  return ((int64_t(r / kTileRows) * (K / kTileK) + c / kTileK) * kTileRows + r % kTileRows) * kTileK + c % kTileK;
}

// 256 K-bytes of a row of 128 rows, 2 threads per row: 8 loads of 16 bytes each.  Chunks at or
// past k are zero; rows past `rows` read row rows-1.
template <bool PACKED>
__device__ __forceinline__ void i8_load(u32x4 (&r)[8], const int8_t* __restrict__ p, int64_t ld, int row0, int rows,
                                        int k0, int K) {
  const int t = threadIdx.x, rr = t >> 1, h = t & 1;
  const int row = min(row0 + rr, rows - 1);
  const uint8_t* base = reinterpret_cast<const uint8_t*>(p) + (PACKED ? 0 : int64_t(row) * ld);
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int kk = k0 + 128 * h + 16 * i;
    const int kc = min(kk, K - 16);
    const u32x4 v = ld4(base + (PACKED ? packed_offset(row, kc, K) : kc));
    r[i] = kk < K ? v : u32x4{0u, 0u, 0u, 0u};
  }
}

// forward.rs's requant (:345-350): (v + 2^(shift-1)) >> shift, clamped to [-127, 127]; the add
// wraps as two's complement (the reference's release build), the shift is arithmetic.
__device__ __forceinline__ int8_t requant_i8(int32_t v, int shift) {
  const int32_t r = int32_t(uint32_t(v) + (uint32_t(1) << (shift - 1))) >> shift;
  return int8_t(r < -127 ? -127 : r > 127 ? 127 : r);
}

// kI8OutRequantRelu and kI8OutRequantSatAdd (forward.h) are the two fused epilogues of
// ForwardModel::forward (src/forward.rs:963-968): max(requant, 0) for the up projection, and the
// i8 saturating add of the requantized result into the residual rows (sat_add, :817-821) for wo
// and down.

__device__ __forceinline__ void i8_store(const u32x4 (&r)[8], int8_t (*dst)[kPlaneStride]) {
  const int t = threadIdx.x, rr = t >> 1, h = t & 1;
#pragma unroll
  for (int i = 0; i < 8; i++) *reinterpret_cast<u32x4*>(&dst[rr][128 * h + 16 * i]) = r[i];
}

// EPI kI8OutI32: out int32 [M][N]; kI8OutRequant: out int8 [M][N], requant_i8(., shift);
// kI8OutTiles: out int32 blocks [M / 8][N / 8][8 * 8], block (m / 8, n / 8) element (m % 8) * 8 + n % 8.
template <bool PACKED, int EPI>
__global__ void __launch_bounds__(kGemmThreads) gemm_i8_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ w,
                                                                int M, int N, int K, void* __restrict__ out, int shift) {
  __shared__ I8Stage S;
  const int n_tiles_m = (M + kGemmBM - 1) / kGemmBM;
  int tm, tn;
  gemm_tile_of(blockIdx.x, gridDim.x, n_tiles_m, tm, tn);
  const int m0 = tm * kGemmBM, n0 = tn * kGemmBN;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int lr = lane & 31, lh = lane >> 5;
  v16i C[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
      for (int v = 0; v < 16; v++) C[i][k][v] = 0;
  u32x4 ra[8], rb[8];
  i8_load<PACKED>(ra, x, K, m0, M, 0, K);
  i8_load<PACKED>(rb, w, K, n0, N, 0, K);
  i8_store(ra, S.a);
  i8_store(rb, S.b);
  __syncthreads();
  for (int k0 = 0; k0 < K; k0 += 256) {
    const bool more = k0 + 256 < K;
    if (more) {
      i8_load<PACKED>(ra, x, K, m0, M, k0 + 256, K);
      i8_load<PACKED>(rb, w, K, n0, N, k0 + 256, K);
    }
    const int steps = min(8, (K - k0 + 31) / 32);
    for (int j = 0; j < steps; j++) {
      v4i af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        af[i] = *reinterpret_cast<const v4i*>(&S.a[64 * wm + 32 * i + lr][32 * j + 16 * lh]);
        bf[i] = *reinterpret_cast<const v4i*>(&S.b[64 * wn + 32 * i + lr][32 * j + 16 * lh]);
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int k = 0; k < 2; k++) C[i][k] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[k], C[i][k], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      i8_store(ra, S.a);
      i8_store(rb, S.b);
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int n = n0 + 64 * wn + 32 * k + lr;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * lh + (v & 3);
        if (m < M && n < N) {
          if constexpr (EPI == kI8OutI32) {
            static_cast<int32_t*>(out)[int64_t(m) * N + n] = C[i][k][v];
          } else if constexpr (EPI == kI8OutRequant) {
            static_cast<int8_t*>(out)[int64_t(m) * N + n] = requant_i8(C[i][k][v], shift);
          } else if constexpr (EPI == kI8OutRequantRelu) {
            const int8_t r = requant_i8(C[i][k][v], shift);
            static_cast<int8_t*>(out)[int64_t(m) * N + n] = r < 0 ? int8_t(0) : r;
          } else if constexpr (EPI == kI8OutRequantSatAdd) {
            int8_t* o = static_cast<int8_t*>(out) + int64_t(m) * N + n;
            const int t = int(*o) + int(requant_i8(C[i][k][v], shift));
            *o = int8_t(t < -128 ? -128 : t > 127 ? 127 : t);
          } else {
            const int64_t blk = int64_t(m / kTileRows) * (N / kTileRows) + n / kTileRows;
            static_cast<int32_t*>(out)[blk * kTileRows * kTileRows + (m % kTileRows) * kTileRows + n % kTileRows] =
                C[i][k][v];
          }
        }
      }
    }
}

// K not a multiple of 16: one output per thread, byte loads (EPI: kI8OutI32 or kI8OutRequant).
template <int EPI>
__global__ void __launch_bounds__(256) gemm_i8_small_kernel(const int8_t* __restrict__ x, const int8_t* __restrict__ w,
                                                             int M, int N, int K, void* __restrict__ out, int shift) {
  const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= int64_t(M) * N) return;
  const int m = int(idx / N), n = int(idx % N);
  const int8_t* xa = x + int64_t(m) * K;
  const int8_t* wb = w + int64_t(n) * K;
  int32_t s = 0;
  for (int k = 0; k < K; k++) s += int32_t(xa[k]) * int32_t(wb[k]);
  if constexpr (EPI == kI8OutI32) static_cast<int32_t*>(out)[idx] = s;
  else static_cast<int8_t*>(out)[idx] = requant_i8(s, shift);
}

__global__ void __launch_bounds__(256) requant_kernel(const int32_t* __restrict__ raw, int64_t n, int shift,
                                                       int8_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = requant_i8(raw[i], shift);
}

// One thread per byte of the packed matrix: the byte of element (r, c), or 0 for padding rows.
__global__ void __launch_bounds__(256) pack_tiles_kernel(const int8_t* __restrict__ src, int64_t rows, int K,
                                                          int64_t total, int8_t* __restrict__ dst) {
  const int64_t o = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (o >= total) return;
  const int kk = int(o % kTileK);
  const int64_t q = o / kTileK;
  const int i = int(q % kTileRows);
  const int64_t tc = q / kTileRows;
  const int kc = int(tc % (K / kTileK));
  const int64_t r = (tc / (K / kTileK)) * kTileRows + i;
  dst[o] = r < rows ? src[r * K + int64_t(kc) * kTileK + kk] : int8_t(0);
}

int gemm_tiles(int64_t M, int64_t N) { return int(((M + kGemmBM - 1) / kGemmBM) * ((N + kGemmBN - 1) / kGemmBN)); }

// Shared argument checks of the int8 products: sizes within 32-bit tile indexing and no int32
// sum able to overflow (|x w| <= 128 * 128 per term).
static int check_i8_args(const void* x, int64_t m, int64_t k, const void* w, int64_t n, const void* out,
                         const char* who) {
  if (!x || !w || !out) return fail(JERO_ERR_INVALID_ARGUMENT, std::string(who) + ": null pointer");
  if (m <= 0 || n <= 0 || k <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, std::string(who) + ": empty operand");
  if (m > (int64_t(1) << 24) || n > (int64_t(1) << 24) || k > (int64_t(1) << 24))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string(who) + ": m, n, k above 2^24");
  if (k * 128 * 128 > INT32_MAX)
    return fail(JERO_ERR_CAPABILITY_MISMATCH, std::string(who) + ": k=" + std::to_string(k) + " could overflow int32 sums");
  return JERO_OK;
}

template <int EPI>
static int launch_gemm_i8(const int8_t* x, int64_t m, int64_t k, const int8_t* w, int64_t n, void* out, int shift,
                          hipStream_t s) {
  int rc = check_i8_args(x, m, k, w, n, out, "gemm_i8");
  if (rc) return rc;
  if (k % 16 == 0 && aligned4(x) && aligned4(w)) {
    hipLaunchKernelGGL((gemm_i8_kernel<false, EPI>), dim3(unsigned(gemm_tiles(m, n))), dim3(kGemmThreads), 0, s, x, w,
                       int(m), int(n), int(k), out, shift);
    return check_launch("gemm i8");
  }
  const int64_t total = m * n;
  hipLaunchKernelGGL((gemm_i8_small_kernel<EPI>), dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, x, w, int(m),
                     int(n), int(k), out, shift);
  return check_launch("gemm i8 (small k)");
}

// The forward pass's projections: the MFMA kernel with one of the int8 epilogues.
int launch_gemm_i8_epi(int epi, const int8_t* x, int64_t m, int64_t k, const int8_t* w, int64_t n, int8_t* out,
                       int shift, hipStream_t s) {
  int rc = check_i8_args(x, m, k, w, n, out, "gemm_i8 (forward)");
  if (rc) return rc;
  if (k % 16 || !aligned4(x) || !aligned4(w)) return fail(JERO_ERR_INVALID_ARGUMENT, "gemm_i8 (forward): k % 16");
  const dim3 grid(unsigned(gemm_tiles(m, n))), block(kGemmThreads);
  if (epi == kI8OutRequant)
    hipLaunchKernelGGL((gemm_i8_kernel<false, kI8OutRequant>), grid, block, 0, s, x, w, int(m), int(n), int(k), out,
                       shift);
  else if (epi == kI8OutRequantRelu)
    hipLaunchKernelGGL((gemm_i8_kernel<false, kI8OutRequantRelu>), grid, block, 0, s, x, w, int(m), int(n), int(k),
                       out, shift);
  else if (epi == kI8OutRequantSatAdd)
    hipLaunchKernelGGL((gemm_i8_kernel<false, kI8OutRequantSatAdd>), grid, block, 0, s, x, w, int(m), int(n), int(k),
                       out, shift);
  else
    return fail(JERO_ERR_INVALID_ARGUMENT, "gemm_i8 (forward): epilogue");
  return check_launch("gemm i8 (forward)");
}

}  // namespace jero

using namespace jero;

namespace jero {

int launch_gemm(int quant, const void* w_dev, int64_t n_in, int64_t n_out, const void* xq_dev, int64_t m, float* y_dev,
                hipStream_t s) {
  const int act = act_format(quant);
  const int64_t xrb = row_bytes(act, n_in);
  if ((quant == JERO_Q4_K || quant == JERO_Q4_K_R) && n_out % kGemmBN == 0) {
    const int tiles = gemm_tiles(m, n_out);
    if (quant == JERO_Q4_K)
      hipLaunchKernelGGL(gemm_q4k_kernel<false>, dim3(unsigned(tiles)), dim3(kQ4Threads), 0, s,
                         static_cast<const uint8_t*>(w_dev), row_bytes(quant, n_in),
                         static_cast<const uint8_t*>(xq_dev), xrb, int(m), int(n_out), int(n_in / 256), y_dev);
    else
      hipLaunchKernelGGL(gemm_q4k_kernel<true>, dim3(unsigned(tiles)), dim3(kQ4Threads), 0, s,
                         static_cast<const uint8_t*>(w_dev), row_bytes(quant, n_in),
                         static_cast<const uint8_t*>(xq_dev), xrb, int(m), int(n_out), int(n_in / 256), y_dev);
    return check_launch("gemm q4_k");
  }
  // other formats and shapes: one GEMV per activation row (each row is matvec_any of x_m)
  for (int64_t r = 0; r < m; r++) {
    const int rc = launch_matvec(quant, w_dev, n_in, n_out, static_cast<const uint8_t*>(xq_dev) + r * xrb,
                                 y_dev + r * n_out, nullptr, s, false);  // every row re-reads the matrix
    if (rc) return rc;
  }
  return JERO_OK;
}

}  // namespace jero

extern "C" int jero_hip_gemm(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                             const void* xq_dev, int64_t m, float* y_dev, void* stream) {
  int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, xq_dev, y_dev);
  if (rc) return rc;
  if (m <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "gemm: no activation rows");
  if (m > (int64_t(1) << 24) || n_out > (int64_t(1) << 30))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "gemm: m or n_out beyond the 32-bit tile indexing");
  return launch_gemm(quant, w_dev, n_in, n_out, xq_dev, m, y_dev, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_gemm_i8(const int8_t* x_dev, int64_t m, int64_t k, const int8_t* w_dev, int64_t n,
                                int32_t* out_dev, void* stream) {
  return launch_gemm_i8<kI8OutI32>(x_dev, m, k, w_dev, n, out_dev, 0, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_gemm_i8_requant(const int8_t* x_dev, int64_t m, int64_t k, const int8_t* w_dev, int64_t n,
                                        int shift, int8_t* out_dev, void* stream) {
  if (shift < 1 || shift > 31) return fail(JERO_ERR_INVALID_ARGUMENT, "gemm_i8_requant: shift must be in 1..31");
  return launch_gemm_i8<kI8OutRequant>(x_dev, m, k, w_dev, n, out_dev, shift, static_cast<hipStream_t>(stream));
}

extern "C" int jero_hip_requant_i8(const int32_t* raw_dev, int64_t n, int shift, int8_t* out_dev, void* stream) {
  if (!raw_dev || !out_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "requant_i8: null pointer");
  if (shift < 1 || shift > 31) return fail(JERO_ERR_INVALID_ARGUMENT, "requant_i8: shift must be in 1..31");
  if (n <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "requant_i8: empty input");
  hipLaunchKernelGGL(requant_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     raw_dev, n, shift, out_dev);
  return check_launch("requant_i8");
}

extern "C" int64_t jero_hip_tile_count(int64_t rows) { return rows <= 0 ? 0 : (rows + kTileRows - 1) / kTileRows; }

extern "C" int jero_hip_pack_tiles(const int8_t* src_dev, int64_t rows, int64_t k, int8_t* dst_dev, void* stream) {
  if (!src_dev || !dst_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "pack_tiles: null pointer");
  if (rows <= 0 || k <= 0) return fail(JERO_ERR_TENSOR_BOUNDS, "pack_tiles: empty matrix");
  if (k % kTileK) return fail(JERO_ERR_TENSOR_BOUNDS, "pack_tiles: k not a multiple of " + std::to_string(kTileK));
  if (rows > (int64_t(1) << 24) || k > (int64_t(1) << 24))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "pack_tiles: rows or k above 2^24");
  const int64_t total = jero_hip_tile_count(rows) * kTileRows * k;
  hipLaunchKernelGGL(pack_tiles_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src_dev, rows, int(k), total, dst_dev);
  return check_launch("pack_tiles");
}

extern "C" int jero_hip_gemm_i8_tiles(const int8_t* a_packed_dev, int64_t m_tiles, const int8_t* w_packed_dev,
                                      int64_t tile_begin, int64_t tile_end, int64_t k_chunks, int32_t* c_dev,
                                      void* stream) {
  if (!a_packed_dev || !w_packed_dev || !c_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "gemm_i8_tiles: null pointer");
  if (m_tiles <= 0 || k_chunks <= 0 || tile_begin < 0 || tile_end <= tile_begin)
    return fail(JERO_ERR_TENSOR_BOUNDS, "gemm_i8_tiles: empty tile range");
  if (!aligned4(a_packed_dev) || !aligned4(w_packed_dev))
    return fail(JERO_ERR_INVALID_ARGUMENT, "gemm_i8_tiles: packed operands must be 4-byte aligned");
  const int64_t m = m_tiles * kTileRows, n = (tile_end - tile_begin) * kTileRows, k = k_chunks * kTileK;
  int rc = check_i8_args(a_packed_dev, m, k, w_packed_dev, n, c_dev, "gemm_i8_tiles");
  if (rc) return rc;
  const int8_t* w0 = w_packed_dev + tile_begin * k_chunks * kTileRows * kTileK;
  hipLaunchKernelGGL((gemm_i8_kernel<true, kI8OutTiles>), dim3(unsigned(gemm_tiles(m, n))), dim3(kGemmThreads), 0,
                     static_cast<hipStream_t>(stream), a_packed_dev, w0, int(m), int(n), int(k),
                     static_cast<void*>(c_dev), 0);
  return check_launch("gemm_i8_tiles");
}
