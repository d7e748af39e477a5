// jero_common.h -- device-side helpers shared by the gfx950 kernels of libjero_hip.
//
// Block formats (GGUF/ggml, little endian) read by the kernels:
//   Q8_0   34 B : f16 d | i8 q[32]
//   Q4_0   18 B : f16 d | u8 qs[16]            (q - 8, low nibbles first)
//   Q4_K  144 B : f16 d | f16 dmin | u8 sc[12] | u8 qs[128]
//   Q6_K  210 B : u8 ql[128] | u8 qh[64] | i8 sc[16] | f16 d
//   Q8_K  292 B : f32 d | i8 q[256] | i16 bsums[16]      (activation for Q4_K / Q6_K)
//   ACT_Q8 36 B : f32 d | i8 q[32]                       (activation for Q8_0 / Q4_0)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jero_hip.h"

namespace jero {

constexpr int kWave = 64;

struct FmtInfo {
  int block_elems;
  int block_bytes;
};

__host__ __device__ constexpr FmtInfo fmt_info(int q) {
  return q == JERO_Q8_0     ? FmtInfo{32, 34}
         : q == JERO_Q4_0   ? FmtInfo{32, 18}
         : q == JERO_Q4_K   ? FmtInfo{256, 144}
         : q == JERO_Q4_K_R ? FmtInfo{256, 144}
         : q == JERO_Q4_K_T ? FmtInfo{256, 144}
         : q == JERO_Q6_K   ? FmtInfo{256, 210}
         : q == JERO_Q6_K_R ? FmtInfo{256, 210}
         : q == JERO_Q6_K_T ? FmtInfo{256, 210}
         : q == JERO_Q8_K   ? FmtInfo{256, 292}
         : q == JERO_ACT_Q8 ? FmtInfo{32, 36}
         : q == JERO_F32    ? FmtInfo{1, 4}
         : q == JERO_F16    ? FmtInfo{1, 2}
         : q == JERO_BF16   ? FmtInfo{1, 2}
                            : FmtInfo{0, 0};
}

// 16-byte vector with 4-byte alignment: selects global_load_dwordx4 on any dword address.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ u32x4 ld4(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x2 ld2(const uint8_t* p) { return *reinterpret_cast<const u32x2*>(p); }
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Weight bytes that a launch reads exactly once: non-temporal loads (global_load ... nt).  A pure
// read of 9-28 MB runs 8-11 % faster with them than with the default policy; where bytes are
// re-read (rows of a prefill GEMV, neighbouring workgroups sharing lines, overlapping dword reads
// of 2-byte aligned blocks) they measured slower, and the default policy stays.
__device__ __forceinline__ u32x4 ldw4(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ uint32_t ldw1(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}
template <bool NT>
__device__ __forceinline__ u32x4 ldx4(const uint8_t* p) {
  if constexpr (NT) return ldw4(p);
  else return ld4(p);
}
template <bool NT>
__device__ __forceinline__ uint32_t ldx1(const uint8_t* p) {
  if constexpr (NT) return ldw1(p);
  else return ld1(p);
}

// Bytes [s, s+4) of the 8-byte little-endian pair (lo, hi), s in 0..3.
__device__ __forceinline__ uint32_t funnel(uint32_t lo, uint32_t hi, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// 16 bytes starting at an address that is only 2-byte aligned.  Reads the five dwords that
// cover them from the dword-aligned address below: every dword read holds at least one byte
// of [p, p+16), so the read never leaves the pages that hold the requested bytes.  At an
// aligned address the fifth read repeats the fourth dword (funnel ignores it): every load is
// issued unconditionally, since a load under a branch gets a wait for completion of its own.
__device__ __forceinline__ u32x4 ld16_a2(const uint8_t* p) {
  const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint8_t* base = p - s;  // pointer arithmetic keeps the global address space
  u32x4 w = ld4(base);
  uint32_t w4 = ld1(base + (s != 0u ? 16 : 12));
  u32x4 r;
  r.x = funnel(w.x, w.y, s);
  r.y = funnel(w.y, w.z, s);
  r.z = funnel(w.z, w.w, s);
  r.w = funnel(w.w, w4, s);
  return r;
}

// 4 bytes at a 2-byte aligned address (same page argument as ld16_a2).
__device__ __forceinline__ uint32_t ld4_a2(const uint8_t* p) {
  const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint8_t* base = p - s;  // pointer arithmetic keeps the global address space
  uint32_t w0 = ld1(base);
  uint32_t w1 = ld1(base + (s != 0u ? 4 : 0));
  return funnel(w0, w1, s);
}

// 8 bytes at a 2-byte aligned address.
__device__ __forceinline__ u32x2 ld8_a2(const uint8_t* p) {
  const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint8_t* base = p - s;  // pointer arithmetic keeps the global address space
  u32x2 w = ld2(base);
  uint32_t w2 = ld1(base + (s != 0u ? 8 : 4));
  u32x2 r;
  r.x = funnel(w.x, w.y, s);
  r.y = funnel(w.y, w2, s);
  return r;
}

// 2-byte f16 at a 2-byte aligned address -> f32.
__device__ __forceinline__ float ldh_a2(const uint8_t* p) {
  const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
  uint32_t w = ld1(p - s);
  uint16_t h = uint16_t(w >> (8u * s));
  return float(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return float(__builtin_bit_cast(_Float16, uint16_t(bits16 & 0xFFFFu)));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, uint32_t i) { return __builtin_amdgcn_ubfe(w, 8u * i, 8u); }

// Sum over groups of `width` consecutive lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <int WIDTH>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// DPP add of a lane permutation (quad_perm / row_ror / row_bcast controls); lanes outside
// row_mask add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
  int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false);
  return v + __builtin_bit_cast(float, o);
}

// Sum over groups of WIDTH (4, 16, 32 or 64) consecutive lanes with DPP; the group total
// lands in the group's last lane (lane % WIDTH == WIDTH - 1).
template <int WIDTH>
__device__ __forceinline__ float group_sum_last(float v) {
  static_assert(WIDTH == 4 || WIDTH == 16 || WIDTH == 32 || WIDTH == 64, "group width");
  v = dpp_add<0xB1, 0xF>(v);  // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);  // quad_perm [2,3,0,1]
  if constexpr (WIDTH >= 16) {
    v = dpp_add<0x124, 0xF>(v);  // row_ror:4
    v = dpp_add<0x128, 0xF>(v);  // row_ror:8
  }
  if constexpr (WIDTH >= 32) v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  if constexpr (WIDTH >= 64) v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for its
// outstanding global loads (which __syncthreads' fence would also drain).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Sum over aligned groups of WIDTH (4, 8 or 16) lanes; every lane of a group gets the total.
template <int WIDTH>
__device__ __forceinline__ float group_sum_all(float v) {
  static_assert(WIDTH == 4 || WIDTH == 8 || WIDTH == 16, "group width");
  v = dpp_add<0xB1, 0xF>(v);                            // quad_perm [1,0,3,2]
  v = dpp_add<0x4E, 0xF>(v);                            // quad_perm [2,3,0,1]
  if constexpr (WIDTH >= 8) v = dpp_add<0x141, 0xF>(v);   // row_half_mirror
  if constexpr (WIDTH >= 16) v = dpp_add<0x140, 0xF>(v);  // row_mirror
  return v;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max(float v) {
  int o = __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, -INFINITY), __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                      0xF, false);
  return fmaxf(v, __builtin_bit_cast(float, o));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_max_i32(int v) {
  const int o = __builtin_amdgcn_update_dpp(int(0x80000000u), v, CTRL, ROW_MASK, 0xF, false);
  return max(v, o);
}

// f32::total_cmp as a signed integer key: a negative float has every bit but the sign flipped,
// so the keys order -inf < ... < -0.0 < +0.0 < ... < +inf (NaNs at the two ends by sign).
__host__ __device__ __forceinline__ int total_order_key(float f) {
  const int b = __builtin_bit_cast(int, f);
  return b ^ int(uint32_t(b >> 31) >> 1);
}

// Whole-wave reductions with DPP; the result is returned uniformly (read from lane 63).
__device__ __forceinline__ int wave_max_i32_dpp(int v) {
  v = dpp_max_i32<0xB1, 0xF>(v);
  v = dpp_max_i32<0x4E, 0xF>(v);
  v = dpp_max_i32<0x124, 0xF>(v);
  v = dpp_max_i32<0x128, 0xF>(v);
  v = dpp_max_i32<0x142, 0xA>(v);
  v = dpp_max_i32<0x143, 0xC>(v);
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = group_sum_last<64>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = dpp_max<0xB1, 0xF>(v);
  v = dpp_max<0x4E, 0xF>(v);
  v = dpp_max<0x124, 0xF>(v);
  v = dpp_max<0x128, 0xF>(v);
  v = dpp_max<0x142, 0xA>(v);
  v = dpp_max<0x143, 0xC>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Q8_K block of 256 elements from one wave, four consecutive elements per lane, written as its
// three fields: 256 int8 at qs, 16 int16 bsums at bs, the f32 scale at d (LDS or global memory,
// 4-byte aligned).  ggml's rule: the first element (lowest index) of largest magnitude is `max`;
// iscale = -127 / max, q = min(127, rint(iscale * x)), d = 1 / iscale, bsums over 16-element
// groups; an all-zero block stores zeros.
__device__ __forceinline__ void q8k_block_wave_split(const float e[4], int lane, uint8_t* qs, uint8_t* bs, uint8_t* d) {
  float am = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; t++) am = fmaxf(am, fabsf(e[t]));
  am = wave_max_dpp(am);  // uniform block max |x|
  if (am == 0.0f) {
    reinterpret_cast<uint32_t*>(qs)[lane] = 0u;
    if (lane < 16) reinterpret_cast<int16_t*>(bs)[lane] = 0;
    if (lane == 0) *reinterpret_cast<float*>(d) = 0.0f;
    return;
  }
  // the first element (lowest index) with |x| == max sets the sign: lowest lane, lowest t
  int mine = 4;
#pragma unroll
  for (int t = 3; t >= 0; t--)
    if (fabsf(e[t]) == am) mine = t;
  const uint64_t hit = __ballot(mine < 4);
  const int src = __builtin_ctzll(hit);
  const int t_src = __builtin_amdgcn_readlane(mine, src);
  const float mxv = __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t_src == 0 ? e[0] : t_src == 1 ? e[1]
                                                               : t_src == 2 ? e[2] : e[3]),
                                       src));
  float iscale = -127.0f / mxv;
  int s = 0;
  uint32_t packed = 0;
#pragma unroll
  for (int t = 0; t < 4; t++) {
    int qv = int(__builtin_rintf(iscale * e[t]));
    qv = qv < 127 ? qv : 127;
    s += qv;
    packed |= (uint32_t(qv) & 0xFFu) << (8 * t);
  }
  reinterpret_cast<uint32_t*>(qs)[lane] = packed;
  s = int(group_sum_all<4>(float(s)));  // |s| <= 508: exact in f32
  if ((lane & 3) == 0) reinterpret_cast<int16_t*>(bs)[lane >> 2] = int16_t(s);
  if (lane == 0) *reinterpret_cast<float*>(d) = 1.0f / iscale;
}

// The same block written as one 292-byte Q8_K block at ob.
__device__ __forceinline__ void q8k_block_wave(const float e[4], int lane, uint8_t* ob) {
  q8k_block_wave_split(e, lane, ob + 4, ob + 260, ob);
}

// The same 256 elements as eight ACT_Q8 blocks (the activations of Q8_0 / Q4_0 weights) at
// ob + 36 j, block j from lanes 8j .. 8j + 7: f32 d = amax / 127, q = rint(x * (1 / d)) (0 for an
// all-zero block), the operations of the ACT_Q8 quantizer kernel.  ob is 4-byte aligned.
__device__ __forceinline__ void actq8_blocks_wave(const float e[4], int lane, uint8_t* ob) {
  float a = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; t++) a = fmaxf(a, fabsf(e[t]));
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) a = fmaxf(a, __shfl_xor(a, off, kWave));
  const float d = a / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint32_t packed = 0;
#pragma unroll
  for (int t = 0; t < 4; t++) packed |= (uint32_t(int(__builtin_rintf(e[t] * id))) & 0xFFu) << (8 * t);
  uint8_t* blk = ob + 36 * (lane >> 3);
  *reinterpret_cast<uint32_t*>(blk + 4 + 4 * (lane & 7)) = packed;
  if ((lane & 7) == 0) *reinterpret_cast<float*>(blk) = d;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

}  // namespace jero
