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

// SPLIT: the grid holds two workgroups per tile, each over one half of the K blocks, adding its
// partial tile into y (zeroed before the launch): two addends, so the sum is the same in either
// order, bit for bit.
template <bool PLANAR, bool SPLIT>
__global__ void __launch_bounds__(kQ4Threads) gemm_q4k_kernel(const uint8_t* __restrict__ w, int64_t wrb,
                                                               const uint8_t* __restrict__ x, int64_t xrb, int M,
                                                               int N, int nb, float* __restrict__ y) {
  __shared__ Q4kStage S[2];
  const int n_tiles_m = (M + kGemmBM - 1) / kGemmBM;
  int tm, tn;
  const int half = SPLIT ? int(blockIdx.x & 1) : 0;
  gemm_tile_of(SPLIT ? int(blockIdx.x >> 1) : int(blockIdx.x), SPLIT ? int(gridDim.x >> 1) : int(gridDim.x),
               n_tiles_m, tm, tn);
  const int b0 = SPLIT ? half * ((nb + 1) / 2) : 0, b1 = SPLIT ? (half ? nb : (nb + 1) / 2) : nb;
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
  q4k_load<PLANAR>(R, x, xrb, m0, M, w, wrb, n0, b0, nb);
  q4k_store(R, S[0]);
  __syncthreads();
  for (int b = b0; b < b1; b++) {
    const Q4kStage& T = S[(b - b0) & 1];
    if (b + 1 < b1) q4k_load<PLANAR>(R, x, xrb, m0, M, w, wrb, n0, b + 1, nb);
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
    if (b + 1 < b1) q4k_store(R, S[(b + 1 - b0) & 1]);
    __syncthreads();
  }
  // store: for each v, the 32 lanes of a half-wave write 32 consecutive floats of one row
  const int n = n0 + nl;
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = m0 + 64 * wm + 32 * mt + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (m < M) {
        if constexpr (SPLIT) atomicAdd(&y[int64_t(m) * N + n], acc[mt][v]);
        else y[int64_t(m) * N + n] = acc[mt][v];
      }
    }
}

__global__ void __launch_bounds__(256) zero_f32_kernel(float* __restrict__ y, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    y[i] = 0.f;
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

// ---------------------------------------------------------------- GEMM layouts: Q4_K_G and Q6_K_P

int gemm_tiles(int64_t M, int64_t N);

// Two load-time layouts feed one kernel structure (a workgroup of four waves owns 64 tokens x 128
// weight rows, each wave one 32-row tile, its weight fragments loaded straight into registers in
// 1 KB runs, the activations shared through LDS):
//   JERO_Q4_K_G: the Q4_K quants regrouped per (32-row tile, block) in the order of the MFMA
//     fragments, with the block headers' 6-bit scales and mins unpacked to bytes (11 % more than
//     the Q4_K bytes); the kernel expands each fragment in registers to the two exact int8 planes
//     of the sub-block scale sc = 8 a + b (a, b in 0..7): a * q4 and b * q4, both <= 105.
//   JERO_Q6_K_P: a Q6_K weight is d * sc * (q6 - 32) with the int8 sub-block scale sc and q6 in
//     0..63, so w = sc * (q6 - 32) is an exact integer in [-4064, 4096]; w = 128 hi + lo with
//     hi = (w + 64) >> 7 in [-32, 32] and lo in [-64, 63] gives two int8 planes stored expanded
//     (2 bytes per weight): 6-bit weights with signed int8 scales cost more to expand per use
//     than to read.  Per 256-block the int8 products add up exactly: 128 (hi . q8) + (lo . q8) =
//     w . q8 and |w . q8| <= 256 * 4096 * 128 < 2^31.
// Both are built once per tensor (GGUF bytes or the _R device layouts) and rows past n_out are
// zero (n_out is padded to a multiple of 32).

// Address of byte `off` (0..209, GGUF block order: ql[128] qh[64] scales[16] d) of block
// (r, b), in the GGUF bytes or the JERO_Q6_K_R planes.  A 16-byte run of ql or qh starting at a
// multiple of 16 stays contiguous in both.
__device__ __forceinline__ const uint8_t* q6k_at(const uint8_t* __restrict__ p, bool planar, int64_t N, int nb,
                                                 int64_t r, int b, int off) {
  if (!planar) return p + (r * nb + b) * 210 + off;
  const int U = 4 * nb;
  const int64_t plane = N * int64_t(U) * 16;
  const int64_t u0 = r * U + 4 * b;
  if (off < 128) {  // ql: lo plane (bytes 0..31 of each 64), hi plane (32..63)
    const int n = off >> 6, rem = off & 63, which = rem >> 5, j = (rem >> 4) & 1, i = rem & 15;
    return p + which * plane + (u0 + 2 * n + j) * 16 + i;
  }
  if (off < 192) {  // qh
    const int o = off - 128, n = o >> 5, j = (o >> 4) & 1, i = o & 15;
    return p + 2 * plane + (u0 + 2 * n + j) * 16 + i;
  }
  if (off < 208) {  // scales: byte 8 n + j + 2 k -> unit 2 n + j, byte k
    const int o = off - 192, n = o >> 3, j = o & 1, k = (o & 7) >> 1;
    return p + 3 * plane + (u0 + 2 * n + j) * 4 + k;
  }
  return p + 3 * plane + N * int64_t(U) * 4 + (r * nb + b) * 2 + (off - 208);
}

// Scale and min of sub-block sb from a Q4_K block header h (d | dmin, then the 12 packed scale
// bytes, GGUF packing): sub-blocks 0..3 in the low 6 bits of bytes sb and sb + 4, sub-blocks 4..7
// from the nibbles of byte sb + 4 and the top bits of bytes sb - 4 and sb.
__device__ __forceinline__ void q4k_scale_min_of(const u32x4& h, int sb, int& sc, int& m) {
  const uint32_t jj = uint32_t(sb & 3);
  const uint32_t a = byte_of(h.y, jj), bb = byte_of(h.z, jj), c = byte_of(h.w, jj);
  sc = int(sb < 4 ? a & 63u : (c & 15u) | ((a >> 6) << 4));
  m = int(sb < 4 ? bb & 63u : (c >> 4) | ((bb >> 6) << 4));
}

// ---- JERO_Q4_K_G.  A record (5120 bytes, one 32-row tile and one block):
//   qs [4 pairs i][64 lanes][16 bytes]: lane (r, h) holds qs bytes 32 i + 16 h .. + 16 of row r of
//     the tile: its low nibbles are elements 16 h .. + 16 of sub-block 2 i, its high nibbles the
//     same elements of sub-block 2 i + 1 (one lane's B fragment of both, before scaling);
//   headers [2 halves h][32 rows][16 bytes]: d and dmin (the block's f16 pair), the 8 sub-block
//     scales as bytes, then the mins of sub-blocks 4 h .. 4 h + 3 as bytes (what lane (r, h) needs).
constexpr int kQ4gRec = 4 * 1024 + 32 * 32;

// ---- JERO_Q6_K_P.  A record (16 512 bytes, one 32-row tile and one block):
//   planes [8 K steps s][2: hi, lo][64 lanes][16 bytes]: lane (r, h) holds row r of the tile at
//     elements 32 s + 16 h .. + 16 of the block (the B operand of v_mfma_i32_32x32x32_i8);
//   d [32] f32.
constexpr int kQ6pPlanes = 8 * 2 * 64 * 16;
constexpr int kQ6pRec = kQ6pPlanes + 32 * 4;

static bool is_q4k(int quant) { return quant == JERO_Q4_K || quant == JERO_Q4_K_R; }
static bool is_q6k(int quant) { return quant == JERO_Q6_K || quant == JERO_Q6_K_R; }

size_t gemm_layout_bytes(int quant, int64_t n_in, int64_t n_out) {
  if (!is_q4k(quant) && !is_q6k(quant)) return 0;
  return size_t((n_out + 31) / 32) * size_t(n_in / 256) * size_t(is_q4k(quant) ? kQ4gRec : kQ6pRec);
}

// One thread per 16-byte piece of a Q4_K_G record (320 per record: 256 qs pieces, 64 headers).
__global__ void __launch_bounds__(256) q4kg_kernel(const uint8_t* __restrict__ src, int planar, int64_t N,
                                                   int64_t tiles, int nb, uint8_t* __restrict__ dst) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= tiles * nb * 320) return;
  const int c = int(t % 320);
  const int64_t tb = t / 320;
  const int b = int(tb % nb);
  const int U = 4 * nb;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (c < 256) {  // qs piece p = 2 i + h of row r (Q4_K_R: run p & 1, unit 4 b + p / 2)
    const int i = c >> 6, lane = c & 63, h = lane >> 5, p = 2 * i + h;
    const int64_t r = (tb / nb) * 32 + (lane & 31);
    if (r < N) {
      const uint8_t* rp = src + r * int64_t(nb) * 144;
      v = ld4(planar ? rp + (p & 1) * U * 16 + (4 * b + (p >> 1)) * 16 : rp + int64_t(b) * 144 + 16 + 16 * p);
    }
  } else {  // header half h of row r, at lane r + 32 h
    const int h = (c - 256) >> 5;
    const int64_t r = (tb / nb) * 32 + ((c - 256) & 31);
    if (r < N) {
      const uint8_t* rp = src + r * int64_t(nb) * 144;
      const u32x4 hd = ld4(planar ? rp + U * 32 + b * 16 : rp + int64_t(b) * 144);
      uint32_t sc[2] = {0u, 0u}, mn = 0u;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        int s_, m_;
        q4k_scale_min_of(hd, j, s_, m_);
        sc[j >> 2] |= uint32_t(s_) << (8 * (j & 3));
        if ((j >> 2) == h) mn |= uint32_t(m_) << (8 * (j & 3));
      }
      v = u32x4{hd.x, sc[0], sc[1], mn};
    }
  }
  *reinterpret_cast<u32x4*>(dst + tb * kQ4gRec + int64_t(c) * 16) = v;
}

// One thread per Q6_K_P lane fragment: thread (tile, block b, K step s, lane (i, h)) expands the
// 16 consecutive weights 16 g .. + 16, g = 2 s + h, of row 32 tile + i into its 16-byte piece of
// each plane, so a wave writes 1 KB runs; the threads of step 0 and h = 0 also write the row's d.
// The element order is ggml's: element 128 n + 32 k + l is the low (k < 2) or high nibble of
// ql[64 n + l + 32 (k & 1)] with bits 2 k of qh[32 n + l], scale 8 n + l / 16 + 2 k.  GGUF Q6_K
// blocks are only 2-byte aligned, so their runs are read as bytes.
__global__ void __launch_bounds__(256) q6kp_kernel(const uint8_t* __restrict__ src, int planar, int64_t N,
                                                   int64_t tiles, int nb, uint8_t* __restrict__ dst) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= tiles * nb * 512) return;
  const int lane = int(t & 63), s = int((t >> 6) & 7);
  const int64_t tb = t >> 9;
  const int64_t r = (tb / nb) * 32 + (lane & 31);
  const int b = int(tb % nb), h = lane >> 5, g = 2 * s + h;
  uint8_t* rec = dst + tb * int64_t(kQ6pRec);
  uint32_t ph[4] = {0u, 0u, 0u, 0u}, pl[4] = {0u, 0u, 0u, 0u};
  float d = 0.f;
  if (r < N) {
    const int e0 = 16 * g, n = e0 >> 7, quarter = (e0 & 127) >> 5, l0 = e0 & 31;
    const int sc = int(int8_t(*q6k_at(src, planar, N, nb, r, b, 192 + 8 * n + l0 / 16 + 2 * quarter)));
    const uint8_t* qlp = q6k_at(src, planar, N, nb, r, b, 64 * n + l0 + (quarter & 1) * 32);
    const uint8_t* qhp = q6k_at(src, planar, N, nb, r, b, 128 + 32 * n + l0);
    uint32_t ql[4], qh[4];
    if (planar) {
      const u32x4 a = ld4(qlp), c = ld4(qhp);
      ql[0] = a.x, ql[1] = a.y, ql[2] = a.z, ql[3] = a.w;
      qh[0] = c.x, qh[1] = c.y, qh[2] = c.z, qh[3] = c.w;
    } else {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        ql[k] = uint32_t(qlp[4 * k]) | (uint32_t(qlp[4 * k + 1]) << 8) | (uint32_t(qlp[4 * k + 2]) << 16) |
                (uint32_t(qlp[4 * k + 3]) << 24);
        qh[k] = uint32_t(qhp[4 * k]) | (uint32_t(qhp[4 * k + 1]) << 8) | (uint32_t(qhp[4 * k + 2]) << 16) |
                (uint32_t(qhp[4 * k + 3]) << 24);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t qlb = byte_of(ql[k], e), qhb = byte_of(qh[k], e);
        const int q6 = int(((quarter >= 2 ? qlb >> 4 : qlb) & 15u) | (((qhb >> (2 * quarter)) & 3u) << 4));
        const int w = sc * (q6 - 32);
        const int hh = (w + 64) >> 7;
        ph[k] |= uint32_t(uint8_t(int8_t(hh))) << (8 * e);
        pl[k] |= uint32_t(uint8_t(int8_t(w - 128 * hh))) << (8 * e);
      }
    if (s == 0 && h == 0) {
      const uint8_t* dp = q6k_at(src, planar, N, nb, r, b, 208);
      d = float(__builtin_bit_cast(_Float16, uint16_t(uint32_t(dp[0]) | (uint32_t(dp[1]) << 8))));
    }
  }
  *reinterpret_cast<u32x4*>(rec + ((2 * s) * 64 + lane) * 16) = u32x4{ph[0], ph[1], ph[2], ph[3]};
  *reinterpret_cast<u32x4*>(rec + ((2 * s + 1) * 64 + lane) * 16) = u32x4{pl[0], pl[1], pl[2], pl[3]};
  if (s == 0 && h == 0) reinterpret_cast<float*>(rec + kQ6pPlanes)[lane] = d;
}

constexpr int kGpThreads = 256;  // 4 waves, one 32-row weight tile each
constexpr int kGpBM = 64;        // tokens per workgroup tile
constexpr int kGpBN = 128;       // weight rows per workgroup tile

// One block of the workgroup's 64 activation rows (the weights do not pass through LDS).
struct __attribute__((aligned(16))) GpStage {
  int8_t a[kGpBM][kPlaneStride];  // q8 (16-byte reads of 16 rows hit distinct banks)
  _Float16 bs[kGpBM][16];         // Q4_K: the 16 bsums, as f16 (exact: |bsum| <= 2048)
  float dx[kGpBM];
};

// A thread's share of one activation block: a quarter of row t / 4 (64 q8 bytes) and, by quarter,
// the row's d (quarter 0) or half of its bsums (quarters 1, 2).
struct GpAct {
  u32x4 q[4];
  u32x4 tail;
};

__device__ __forceinline__ void gp_load_act(GpAct& A, const uint8_t* __restrict__ xq, int64_t xrb, int m0, int M,
                                            int b) {
  const int t = threadIdx.x, r = t >> 2, q = t & 3;
  const uint8_t* xa = xq + int64_t(min(m0 + r, M - 1)) * xrb + int64_t(b) * 292;
#pragma unroll
  for (int i = 0; i < 4; i++) A.q[i] = ld4(xa + 4 + 64 * q + 16 * i);
  A.tail = ld4(xa + (q == 1 ? 260 : q == 2 ? 276 : 0));
}

template <bool BSUMS>
__device__ __forceinline__ void gp_store_act(const GpAct& A, GpStage& S) {
  const int t = threadIdx.x, r = t >> 2, q = t & 3;
#pragma unroll
  for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4*>(&S.a[r][64 * q + 16 * i]) = A.q[i];
  if (q == 0) S.dx[r] = __uint_as_float(A.tail.x);
  if constexpr (BSUMS) {
    if (q == 1 || q == 2) {
      const uint32_t bw[4] = {A.tail.x, A.tail.y, A.tail.z, A.tail.w};
      uint32_t hw[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        hw[i] = uint32_t(__builtin_bit_cast(uint16_t, _Float16(float(int16_t(bw[i] & 0xFFFFu))))) |
                (uint32_t(__builtin_bit_cast(uint16_t, _Float16(float(int16_t(bw[i] >> 16))))) << 16);
      *reinterpret_cast<u32x4*>(&S.bs[r][8 * (q - 1)]) = u32x4{hw[0], hw[1], hw[2], hw[3]};
    }
  }
}

// Y[m][n] = sum_b dx[m,b] (d[n,b] T[m,n,b] - dmin[n,b] (m . bsums)[m,n,b]) over the 256-blocks
// (Q6_K: no dmin term), row m of Y equal to the GEMV of x_m, with T the block's exact integer
// sum of w . q8.  A workgroup of four waves owns a 64 (tokens) x 128 (weight rows) tile, each wave
// the 64 tokens x one 32-row record tile (read by that wave only), as two 32-token MFMA halves.
// Per block a wave loads its record into registers while the previous block runs (Q6_K_P: step
// by step, each step's two 1 KB plane runs as soon as its MFMAs have read the registers), the
// activations of the next block go through LDS (double-buffered, one barrier per block), and
// the block's integer sums are scaled into f32 accumulators.  Q4_K_G: per K pair the lane's
// fragment is expanded to the planes a * q4, b * q4 of both sub-blocks and T = 8 Ta + Tb; the
// mins term is one v_mfma_f32_32x32x16_f16 over the 16 bsums (|bsum| <= 2048 and m <= 63 are
// exact in f16, sums below 2^24).  Q6_K_P: T = 128 Th + Tl.  Two workgroups share a CU.  SPLIT:
// two workgroups per tile, one per half of the blocks, adding into the zeroed output (two
// addends: the same sum in either order).
template <bool Q4, bool SPLIT>
__global__ void __launch_bounds__(kGpThreads, 2) gemm_laid_kernel(const uint8_t* __restrict__ xq, int64_t xrb,
                                                                   const uint8_t* __restrict__ wg, int M, int N,
                                                                   int nb, float* __restrict__ y,
                                                                   float* __restrict__ y2) {
  __shared__ GpStage S[2];
  constexpr int REC = Q4 ? kQ4gRec : kQ6pRec;
  const int n_tiles_m = (M + kGpBM - 1) / kGpBM;
  int tm, tn;
  const int half = SPLIT ? int(blockIdx.x & 1) : 0;
  gemm_tile_of(SPLIT ? int(blockIdx.x >> 1) : int(blockIdx.x), SPLIT ? int(gridDim.x >> 1) : int(gridDim.x),
               n_tiles_m, tm, tn);
  const int b0 = SPLIT ? half * ((nb + 1) / 2) : 0, b1 = SPLIT ? (half ? nb : (nb + 1) / 2) : nb;
  const int m0 = tm * kGpBM;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int lr = lane & 31, lh = lane >> 5;
  // this wave's record tile (clamped: a tile past N computes rows that are never stored)
  const int t32 = min(4 * tn + wv, (N + 31) / 32 - 1);
  const uint8_t* wt = wg + int64_t(t32) * nb * REC;
  const uint8_t* wl = wt + 16 * lane;                                  // this lane's fragments
  const uint8_t* wr = wt + (Q4 ? 4096 + 16 * lane : kQ6pPlanes + 4 * lr);  // its row's header half / d

  float acc[2][16];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[mt][v] = 0.f;

  GpAct A;
  constexpr int NW = Q4 ? 4 : 16;  // 16-byte fragment loads per lane and block
  u32x4 W[NW];
  u32x4 H = {0u, 0u, 0u, 0u};  // Q4_K_G: the row's header
  float dq = 0.f;              // Q6_K_P: the row's d
  auto load_w = [&](u32x4 (&Wd)[NW], int64_t o) {
#pragma unroll
    for (int i = 0; i < NW; i++) Wd[i] = ld4(wl + o + 1024 * i);
  };
  gp_load_act(A, xq, xrb, m0, M, b0);
  load_w(W, int64_t(b0) * REC);
  if constexpr (Q4) H = ld4(wr + int64_t(b0) * REC);
  else dq = __uint_as_float(ld1(wr + int64_t(b0) * REC));
  gp_store_act<Q4>(A, S[0]);
  __syncthreads();
  for (int b = b0; b < b1; b++) {
    const GpStage& T = S[(b - b0) & 1];
    const int bn = min(b + 1, b1 - 1);  // the last block reloads itself: every load unconditional
    const int64_t on = int64_t(bn) * REC;
    gp_load_act(A, xq, xrb, m0, M, bn);
    float dw, dm = 0.f;
    v8h mnf = {};
    v16i Ch[2], Cl[2];  // Q4_K_G: the a and b planes; Q6_K_P: hi and lo
    if constexpr (Q4) {
      const u32x4 Hc = H;
      H = ld4(wr + on);
      __builtin_amdgcn_sched_barrier(0);  // the activation and header loads are issued here
#pragma unroll
      for (int jj = 0; jj < 4; jj++)  // the mins of this lane's half of the bsum groups
        mnf[2 * jj] = mnf[2 * jj + 1] = _Float16(float(byte_of(Hc.w, jj)));
      dw = float(__builtin_bit_cast(_Float16, uint16_t(Hc.x & 0xFFFFu)));
      dm = float(__builtin_bit_cast(_Float16, uint16_t(Hc.x >> 16)));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t sw = i < 2 ? Hc.y : Hc.z;
        const uint32_t s0 = byte_of(sw, 2 * (i & 1)), s1 = byte_of(sw, 2 * (i & 1) + 1);
        const uint32_t raw[4] = {W[i].x, W[i].y, W[i].z, W[i].w};
        W[i] = ld4(wl + on + 1024 * i);  // the next block's fragment, as soon as this one is read
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
          const v4i af0 = *reinterpret_cast<const v4i*>(&T.a[32 * mt + lr][64 * i + 16 * lh]);
          const v4i af1 = *reinterpret_cast<const v4i*>(&T.a[32 * mt + lr][64 * i + 32 + 16 * lh]);
          const v16i z = {};
          Ch[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pa0, i == 0 ? z : Ch[mt], 0, 0, 0);
          Cl[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af0, pb0, i == 0 ? z : Cl[mt], 0, 0, 0);
          Ch[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, pa1, Ch[mt], 0, 0, 0);
          Cl[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af1, pb1, Cl[mt], 0, 0, 0);
        }
      }
    } else {
      __builtin_amdgcn_sched_barrier(0);  // the activation loads ahead of the weight loads
      dw = dq;
#pragma unroll
      for (int s = 0; s < 8; s++) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
          const v4i af = *reinterpret_cast<const v4i*>(&T.a[32 * mt + lr][32 * s + 16 * lh]);
          const v16i z = {};
          Ch[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, __builtin_bit_cast(v4i, W[2 * s]), s == 0 ? z : Ch[mt],
                                                         0, 0, 0);
          Cl[mt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, __builtin_bit_cast(v4i, W[2 * s + 1]),
                                                         s == 0 ? z : Cl[mt], 0, 0, 0);
        }
        W[2 * s] = ld4(wl + on + (2 * s) * 1024);
        W[2 * s + 1] = ld4(wl + on + (2 * s + 1) * 1024);
        // the step's loads are issued here: left to itself the scheduler sinks them all to the
        // end of the block, and the next block's first MFMAs then wait for a full round trip
        __builtin_amdgcn_sched_barrier(0);
      }
      dq = __uint_as_float(ld1(wr + on));
    }
    // block b + 1 goes to the buffer every wave finished reading before the last barrier
    gp_store_act<Q4>(A, S[(b - b0 + 1) & 1]);
    // the block's scales: column n = lane % 32 of the tile, token rows 8 (v / 4) + 4 (lane / 32) + v % 4
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
      v16f Mn = {};
      if constexpr (Q4) {
        const v8h bsf = *reinterpret_cast<const v8h*>(&T.bs[32 * mt + lr][8 * lh]);
        Mn = __builtin_amdgcn_mfma_f32_32x32x16_f16(bsf, mnf, Mn, 0, 0, 0);
      }
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 dx = *reinterpret_cast<const float4*>(&T.dx[32 * mt + 8 * g + 4 * lh]);
        const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int v = 4 * g + e;
          const float tv = float(Q4 ? (Ch[mt][v] << 3) + Cl[mt][v] : Ch[mt][v] * 128 + Cl[mt][v]);
          acc[mt][v] = fmaf(dxv[e], Q4 ? dw * tv - dm * Mn[v] : dw * tv, acc[mt][v]);
        }
      }
    }
    __syncthreads();
  }
  // store: for each v, the 32 lanes of a half-wave write 32 consecutive floats of one row
  const int n = 32 * (4 * tn + wv) + lr;
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int m = m0 + 32 * mt + 8 * (v >> 2) + 4 * lh + (v & 3);
      if (m < M && n < N) {
        if constexpr (SPLIT) {
          if (y2) (half ? y2 : y)[int64_t(m) * N + n] = acc[mt][v];
          else atomicAdd(&y[int64_t(m) * N + n], acc[mt][v]);
        } else {
          y[int64_t(m) * N + n] = acc[mt][v];
        }
      }
    }
}

int launch_gemm_layout(int quant, const void* w, int64_t n_in, int64_t n_out, void* dst, hipStream_t s) {
  if (!is_q4k(quant) && !is_q6k(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "gemm layout: weights must be Q4_K, Q4_K_R, Q6_K or Q6_K_R");
  const int nb = int(n_in / 256);
  const int64_t tiles = (n_out + 31) / 32;
  const int planar = quant == JERO_Q4_K_R || quant == JERO_Q6_K_R;
  const uint8_t* src = static_cast<const uint8_t*>(w);
  uint8_t* d = static_cast<uint8_t*>(dst);
  if (is_q4k(quant)) {
    const int64_t threads = tiles * nb * 320;
    hipLaunchKernelGGL(q4kg_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, src, planar, n_out, tiles,
                       nb, d);
  } else {
    const int64_t threads = tiles * nb * 512;
    hipLaunchKernelGGL(q6kp_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, src, planar, n_out, tiles,
                       nb, d);
  }
  return check_launch("gemm layout");
}

int launch_gemm_laid(int laid, const void* w, int64_t n_in, int64_t n_out, const void* xq, int64_t m, float* y,
                     hipStream_t s, float* y2, bool* split_out) {
  const int nb = int(n_in / 256);
  const int64_t tiles = ((m + kGpBM - 1) / kGpBM) * ((n_out + kGpBN - 1) / kGpBN);
  // two workgroups per CU: a grid that fills at most half of that splits K in two
  const bool split = nb >= 2 && tiles <= device_info().cus;
  if (split_out) *split_out = split && y2;
  const uint8_t* xb = static_cast<const uint8_t*>(xq);
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  const int64_t xrb = row_bytes(JERO_Q8_K, n_in);
  const dim3 grid(unsigned(split ? 2 * tiles : tiles)), block(kGpThreads);
  if (split) {
    if (!y2) {  // both halves add into the zeroed output
      hipLaunchKernelGGL(zero_f32_kernel, dim3(unsigned(std::min<int64_t>((m * n_out + 255) / 256, 4096))), dim3(256),
                         0, s, y, m * n_out);
      int rc = check_launch("gemm zero");
      if (rc) return rc;
    }
    if (laid == JERO_Q4_K_G)
      hipLaunchKernelGGL((gemm_laid_kernel<true, true>), grid, block, 0, s, xb, xrb, wb, int(m), int(n_out), nb, y, y2);
    else
      hipLaunchKernelGGL((gemm_laid_kernel<false, true>), grid, block, 0, s, xb, xrb, wb, int(m), int(n_out), nb, y, y2);
  } else if (laid == JERO_Q4_K_G) {
    hipLaunchKernelGGL((gemm_laid_kernel<true, false>), grid, block, 0, s, xb, xrb, wb, int(m), int(n_out), nb, y, y2);
  } else {
    hipLaunchKernelGGL((gemm_laid_kernel<false, false>), grid, block, 0, s, xb, xrb, wb, int(m), int(n_out), nb, y, y2);
  }
  return check_launch(laid == JERO_Q4_K_G ? "gemm q4_k_g" : "gemm q6_k_p");
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
                hipStream_t s, const void* laid, float* y2, bool* split_out) {
  if (split_out) *split_out = false;
  const int act = act_format(quant);
  const int64_t xrb = row_bytes(act, n_in);
  if (quant == JERO_Q4_K_G || quant == JERO_Q6_K_P) return launch_gemm_laid(quant, w_dev, n_in, n_out, xq_dev, m, y_dev, s);
  if ((is_q4k(quant) || is_q6k(quant)) && laid)
    return launch_gemm_laid(is_q4k(quant) ? JERO_Q4_K_G : JERO_Q6_K_P, laid, n_in, n_out, xq_dev, m, y_dev, s, y2,
                            split_out);
  if (is_q6k(quant) && m >= kLaidMinRows) {  // the Q6_K_P planes built into the library workspace for this call
    void* ws = nullptr;
    int rc = workspace(gemm_layout_bytes(quant, n_in, n_out), &ws);
    if (!rc) rc = launch_gemm_layout(quant, w_dev, n_in, n_out, ws, s);
    if (rc) return rc;
    return launch_gemm_laid(JERO_Q6_K_P, ws, n_in, n_out, xq_dev, m, y_dev, s);
  }
  if ((quant == JERO_Q4_K || quant == JERO_Q4_K_R) && n_out % kGemmBN == 0) {
    const int tiles = gemm_tiles(m, n_out);
    const int nb = int(n_in / 256);
    // at most half the CUs busy (one 115 KB workgroup per CU): two workgroups per tile, one per
    // half of K, adding into a zeroed output
    const bool split = nb >= 2 && 2 * tiles <= device_info().cus;
    const uint8_t* wb = static_cast<const uint8_t*>(w_dev);
    const uint8_t* xb = static_cast<const uint8_t*>(xq_dev);
    const int64_t wrb = row_bytes(quant, n_in);
    if (split) {
      hipLaunchKernelGGL(zero_f32_kernel, dim3(unsigned(std::min<int64_t>((m * n_out + 255) / 256, 4096))), dim3(256),
                         0, s, y_dev, m * n_out);
      int rc = check_launch("gemm q4_k zero");
      if (rc) return rc;
      if (quant == JERO_Q4_K)
        hipLaunchKernelGGL((gemm_q4k_kernel<false, true>), dim3(unsigned(2 * tiles)), dim3(kQ4Threads), 0, s, wb, wrb,
                           xb, xrb, int(m), int(n_out), nb, y_dev);
      else
        hipLaunchKernelGGL((gemm_q4k_kernel<true, true>), dim3(unsigned(2 * tiles)), dim3(kQ4Threads), 0, s, wb, wrb,
                           xb, xrb, int(m), int(n_out), nb, y_dev);
    } else if (quant == JERO_Q4_K) {
      hipLaunchKernelGGL((gemm_q4k_kernel<false, false>), dim3(unsigned(tiles)), dim3(kQ4Threads), 0, s, wb, wrb, xb,
                         xrb, int(m), int(n_out), nb, y_dev);
    } else {
      hipLaunchKernelGGL((gemm_q4k_kernel<true, false>), dim3(unsigned(tiles)), dim3(kQ4Threads), 0, s, wb, wrb, xb,
                         xrb, int(m), int(n_out), nb, y_dev);
    }
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

extern "C" size_t jero_hip_gemm_layout_bytes(int quant, int64_t n_in, int64_t n_out) {
  if (n_in <= 0 || n_out <= 0 || n_in % 256 || n_in > (int64_t(1) << 30) || n_out > (int64_t(1) << 30)) return 0;
  return jero::gemm_layout_bytes(quant, n_in, n_out);
}

extern "C" int jero_hip_repack_gemm(int quant, const void* src_dev, size_t src_bytes, int64_t n_in, int64_t n_out,
                                    void* dst_dev, size_t dst_bytes, int* dst_quant, void* stream) {
  if (!jero::is_q4k(quant) && !jero::is_q6k(quant))
    return fail(JERO_ERR_CAPABILITY_MISMATCH, "repack_gemm: weights must be Q4_K, Q4_K_R, Q6_K or Q6_K_R");
  if (!src_dev || !dst_dev || !dst_quant) return fail(JERO_ERR_INVALID_ARGUMENT, "repack_gemm: null pointer");
  const size_t need = jero_hip_gemm_layout_bytes(quant, n_in, n_out);
  if (!need) return fail(JERO_ERR_TENSOR_BOUNDS, "repack_gemm: n_in a multiple of 256, sizes within 2^30");
  if (uint64_t(jero::row_bytes(quant, n_in)) * uint64_t(n_out) > src_bytes)
    return fail(JERO_ERR_TENSOR_BOUNDS, "repack_gemm: source holds fewer bytes than the shape");
  if (dst_bytes < need)
    return fail(JERO_ERR_TENSOR_BOUNDS, "repack_gemm: destination holds " + std::to_string(dst_bytes) +
                                            " bytes, the layout needs " + std::to_string(need));
  if ((reinterpret_cast<uintptr_t>(src_dev) & 15u) || (reinterpret_cast<uintptr_t>(dst_dev) & 15u))
    return fail(JERO_ERR_INVALID_ARGUMENT, "repack_gemm: source and destination must be 16-byte aligned");
  const int rc = jero::launch_gemm_layout(quant, src_dev, n_in, n_out, dst_dev, static_cast<hipStream_t>(stream));
  if (!rc) *dst_quant = jero::is_q4k(quant) ? JERO_Q4_K_G : JERO_Q6_K_P;
  return rc;
}

extern "C" int jero_hip_gemm(int quant, const void* w_dev, size_t w_bytes, int64_t n_in, int64_t n_out,
                             const void* xq_dev, int64_t m, float* y_dev, void* stream) {
  if (quant == JERO_Q4_K_G || quant == JERO_Q6_K_P) {
    const int base = quant == JERO_Q4_K_G ? JERO_Q4_K : JERO_Q6_K;
    if (!w_dev || !xq_dev || !y_dev) return fail(JERO_ERR_INVALID_ARGUMENT, "gemm: null pointer");
    const size_t need = jero_hip_gemm_layout_bytes(base, n_in, n_out);
    if (!need) return fail(JERO_ERR_TENSOR_BOUNDS, "gemm: the GEMM layouts need n_in a multiple of 256, sizes within 2^30");
    if (w_bytes < need)
      return fail(JERO_ERR_TENSOR_BOUNDS, "gemm: the layout holds " + std::to_string(w_bytes) +
                                              " bytes, the shape needs " + std::to_string(need));
    if ((reinterpret_cast<uintptr_t>(w_dev) & 15u) || !jero::aligned4(xq_dev) || !jero::aligned4(y_dev))
      return fail(JERO_ERR_INVALID_ARGUMENT, "gemm: layout 16-byte aligned, activations and output 4-byte aligned");
  } else {
    int rc = check_matvec_args(quant, w_dev, w_bytes, n_in, n_out, xq_dev, y_dev);
    if (rc) return rc;
  }
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
