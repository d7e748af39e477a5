// dequant.h -- row dequantization launcher.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "jero_common.h"

namespace jero {

// Element `col` of a GGUF row (f32/f16/Q8_0/Q4_0/Q4_K/Q6_K), as dequantize_token_row computes it.
__device__ __forceinline__ float dequant_elem(int quant, const uint8_t* __restrict__ row, int64_t col) {
  switch (quant) {
    case JERO_F32: return reinterpret_cast<const float*>(row)[col];
    case JERO_F16: return ldh_a2(row + 2 * col);
    case JERO_BF16: {
      const uint8_t* p = row + 2 * col;
      const uint32_t s = uint32_t(reinterpret_cast<uintptr_t>(p) & 3u);
      return __uint_as_float(((ld1(p - s) >> (8u * s)) & 0xFFFFu) << 16);
    }
    case JERO_Q8_0: {
      const uint8_t* b = row + (col / 32) * 34;
      return ldh_a2(b) * float(int8_t(b[2 + col % 32]));
    }
    case JERO_Q4_0: {
      const uint8_t* b = row + (col / 32) * 18;
      int j = int(col % 32);
      int q = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
      return ldh_a2(b) * float(q - 8);
    }
    case JERO_Q4_K: {
      const uint8_t* b = row + (col / 256) * 144;
      int e = int(col % 256), i = e / 64, hi = (e / 32) & 1, l = e % 32, j = e / 32;
      const uint8_t* s = b + 4;
      int sc, m;
      if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
      } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
      }
      int q = hi ? (b[16 + 32 * i + l] >> 4) : (b[16 + 32 * i + l] & 15);
      return ldh_a2(b) * float(sc) * float(q) - ldh_a2(b + 2) * float(m);
    }
    case JERO_Q6_K: {
      const uint8_t* b = row + (col / 256) * 210;
      int e = int(col % 256), n = e / 128, r = e % 128, t = r / 32, l = r % 32;
      uint8_t ql = b[64 * n + l + (t & 1) * 32];
      int lo4 = (t & 2) ? (ql >> 4) : (ql & 15);
      int h2 = (b[128 + 32 * n + l] >> (2 * t)) & 3;
      int q = (lo4 | (h2 << 4)) - 32;
      int sc = int(int8_t(b[192 + e / 16]));
      return ldh_a2(b + 208) * float(sc) * float(q);
    }
    default: return 0.0f;
  }
}

// embed_token (src/qwen_deepseek.rs:558-582), element i of the embedding of token t: row t of the
// token_embd tensor (rows of `rb` bytes, `rows` of them; w null when absent) when it has that row,
// else the deterministic row ((t % 31) * 0.05 + 0.25) + (i % 7) * 0.01 in f32, each operation
// rounded on its own as the reference computes it: contraction into fused multiply-adds is off
// for these operators (the pragma reaches only operators written in this function, not those
// inside __fmul_rn / __fadd_rn, which the compiler would still fuse).  t < 0 marks no token
// (the greedy token of a step that failed closed) and embeds as zeros.
__device__ __forceinline__ float embed_value(int quant, const uint8_t* __restrict__ w, int64_t rb, int64_t rows,
                                             int64_t t, int64_t i) {
#pragma clang fp contract(off)
  if (t < 0) return 0.0f;
  if (t < rows) return dequant_elem(quant, w + t * rb, i);
  const float seed = float(uint32_t(t) % 31u) * 0.05f + 0.25f;
  const float off = float(i % 7) * 0.01f;
  return seed + off;
}

int launch_dequant_rows(int quant, const void* w, int64_t n_in, int64_t row0, int64_t n_rows, float* out,
                        hipStream_t s);

}  // namespace jero
