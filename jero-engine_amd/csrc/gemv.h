// gemv.h -- GEMV launchers shared by the entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace jero {

// F32 / F16 / BF16 weight rows (their "activation" is the f32 input itself).
bool is_float_weight(int quant);
// Enqueues y = W x for unquantized weight rows (any n_in).
int launch_matvec_float(int quant, const void* w, int64_t n_in, int64_t n_out, const float* x, float* y,
                        hipStream_t s);
// Largest n_in the register-resident activation layout supports for a weight format (longer
// rows run the K-looped kernel).
int max_gemv_k(int quant);
// Validates a matvec call (shape, bytes, alignment); records the error and returns its code.
int check_matvec_args(int quant, const void* w, size_t w_bytes, int64_t n_in, int64_t n_out, const void* xq,
                      const float* y);
// Enqueues y = W xq (and the int32 partial sums when part != nullptr).  once: the launch is the
// only reader of these weights for a while (a single GEMV, not one of a batch of rows over the
// same matrix), so its weight loads may bypass the caches (non-temporal).
int launch_matvec(int quant, const void* w, int64_t n_in, int64_t n_out, const void* xq, float* y, int32_t* part,
                  hipStream_t s, bool once = true);
// Y[m][n_out] for m activation rows (jero_hip_gemm after its checks): the int8-MFMA kernel for
// Q4_K and Q4_K_R with n_out a multiple of 128; for Q6_K and Q6_K_R from kQ6PlanesMinRows rows
// (or whenever q6_planes is given) the int8-MFMA kernel over the tensor's two int8 planes
// (q6_planes: built by launch_q6k_planes; null: built for this call in the library workspace);
// one GEMV per row otherwise.
constexpr int64_t kQ6PlanesMinRows = 8;
int launch_gemm(int quant, const void* w, int64_t n_in, int64_t n_out, const void* xq, int64_t m, float* y,
                hipStream_t s, const void* q6_planes = nullptr);
// The int8 planes of a Q6_K / Q6_K_R tensor for the MFMA GEMM (planes: q6k_planes_bytes bytes).
size_t q6k_planes_bytes(int64_t n_in, int64_t n_out);
int launch_q6k_planes(int quant, const void* w, int64_t n_in, int64_t n_out, void* planes, hipStream_t s);
// Enqueues the Q4_K -> Q4_K_R or Q6_K -> Q6_K_R re-layout (dst: 16-byte aligned, same size).
int launch_repack(int quant, const void* src, int64_t n_in, int64_t n_out, void* dst, int* dst_quant, hipStream_t s);
int launch_repack_experts(int quant, const void* src, int64_t n_in, int64_t n_rows, void* dst, int* dst_quant,
                          hipStream_t s);

}  // namespace jero
