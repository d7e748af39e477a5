// forward.h -- the int8 product epilogues shared by the exact int8 GEMM and the int8 forward pass.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jero {

// kI8OutI32: int32 [M][N]; kI8OutRequant: int8 [M][N] = requant(acc, shift); kI8OutTiles: int32
// 8 x 8 blocks; kI8OutRequantRelu: max(requant, 0); kI8OutRequantSatAdd: out = sat_i8(out + requant).
enum { kI8OutI32 = 0, kI8OutRequant = 1, kI8OutTiles = 2, kI8OutRequantRelu = 3, kI8OutRequantSatAdd = 4 };

// x int8 [m][k] times row-major w int8 [n][k] on the int8 MFMA kernel, written through epilogue
// epi (kI8OutRequant, kI8OutRequantRelu or kI8OutRequantSatAdd) into out int8 [m][n].
int launch_gemm_i8_epi(int epi, const int8_t* x, int64_t m, int64_t k, const int8_t* w, int64_t n, int8_t* out,
                       int shift, hipStream_t s);

}  // namespace jero
