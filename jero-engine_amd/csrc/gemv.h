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
// xn = RMSNorm(x) * nw (eps) and y = W xn over F32 rows in one launch, for inputs router_norm_fits
// accepts (F32, n_in % 4 == 0 and <= kRouterMaxK, w / x / xn 16-byte aligned); xn is written too.
constexpr int64_t kRouterMaxK = 8192;  // xn staged in 32 KB of LDS
bool router_norm_fits(int quant, const void* w, int64_t n_in, const float* x, const float* xn);
int launch_router_norm(const void* w, int64_t n_in, int64_t n_out, const float* x, const float* nw, float eps,
                       float* xn, float* y, hipStream_t s);
// Y[rows][n_out] = X[rows][n_in] W^T over F32 weight rows (n_out rows of n_in floats), one launch on
// the f32 MFMA; n_in a multiple of 64, w and x 16-byte aligned.
int launch_matmul_f32_rows(const void* w, int64_t n_in, int64_t n_out, const float* x, int64_t rows, float* y,
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
// Y[m][n_out] for m activation rows (jero_hip_gemm after its checks): JERO_Q4_K_G / JERO_Q6_K_P
// (w in that GEMM layout), or Q4_K / Q4_K_R / Q6_K / Q6_K_R with their GEMM layout given
// (laid), run the int8-MFMA kernel over the layout; Q6_K / Q6_K_R from kLaidMinRows rows build
// the Q6_K_P planes into the library workspace for the call; Q4_K / Q4_K_R with n_out a multiple
// of 128 run the int8-MFMA kernel over the Q4_K bytes; one GEMV per row otherwise.  With y2 given,
// a layout GEMM whose grid splits K in two writes one half's sums to y and the other's to y2
// (*split_out true; the product is y + y2, the same bits as the one-output form) instead of adding
// both into a zeroed y.
constexpr int64_t kLaidMinRows = 8;
int launch_gemm(int quant, const void* w, int64_t n_in, int64_t n_out, const void* xq, int64_t m, float* y,
                hipStream_t s, const void* laid = nullptr, float* y2 = nullptr, bool* split_out = nullptr);
// The GEMM layout of a Q4_K / Q4_K_R tensor (JERO_Q4_K_G) or Q6_K / Q6_K_R tensor (JERO_Q6_K_P):
// gemm_layout_bytes bytes, 16-byte aligned (0 for other formats); and the GEMM over it.
size_t gemm_layout_bytes(int quant, int64_t n_in, int64_t n_out);
int launch_gemm_layout(int quant, const void* w, int64_t n_in, int64_t n_out, void* dst, hipStream_t s);
int launch_gemm_laid(int laid, const void* w, int64_t n_in, int64_t n_out, const void* xq, int64_t m, float* y,
                     hipStream_t s, float* y2 = nullptr, bool* split_out = nullptr);
// Enqueues the Q4_K -> Q4_K_R or Q6_K -> Q6_K_R re-layout (dst: 16-byte aligned, same size).
int launch_repack(int quant, const void* src, int64_t n_in, int64_t n_out, void* dst, int* dst_quant, hipStream_t s);
int launch_repack_experts(int quant, const void* src, int64_t n_in, int64_t n_rows, void* dst, int* dst_quant,
                          hipStream_t s);

}  // namespace jero
