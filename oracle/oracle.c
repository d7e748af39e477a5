/*
 * oracle.c -- CPU restatement of jero-engine's quantized-matmul hot path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py; the product library never links it.
 * The functions, their reference citations and their pins are listed in oracle.h.
 *
 * Plain C99 + pthreads, scalar, no intrinsics: built -O3 -march=native it is also the
 * "C restatement of the reference's portable CPU path" that bench.py times.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float jo_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        e++;
        mant <<= 1;
      } while ((mant & 0x400u) == 0);
      mant &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Round-to-nearest-even float -> half (IEEE 754 conversion). */
uint16_t jo_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7FFFFFFFu;
  if (absx >= 0x7F800000u) { /* inf or nan */
    return (uint16_t)(sign | 0x7C00u | (absx > 0x7F800000u ? 0x200u : 0u));
  }
  if (absx >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7C00u);
  }
  if (absx < 0x38800000u) { /* result is subnormal or zero in half */
    /* value = absx as float; half subnormal unit = 2^-24 */
    float af;
    memcpy(&af, &absx, 4);
    float scaled = af * 16777216.0f; /* exact: multiply by 2^24 */
    /* rint with round-half-even in the default FP environment */
    uint32_t m = (uint32_t)nearbyintf(scaled);
    return (uint16_t)(sign | m);
  }
  uint32_t mant = absx & 0x7FFFFFu;
  uint32_t exp = (absx >> 23) - 127 + 15;
  uint32_t h = (exp << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carries into exponent correctly */
  return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------ formats */

int64_t jo_block_elems(int quant) {
  switch (quant) {
    case JO_F32:
    case JO_F16:
    case JO_BF16: return 1;
    case JO_Q4_0:
    case JO_Q8_0:
    case JO_ACT_Q8: return 32;
    case JO_Q4_K:
    case JO_Q6_K:
    case JO_Q8_K: return 256;
    default: return 0;
  }
}

int64_t jo_block_bytes(int quant) {
  switch (quant) {
    case JO_F32: return 4;
    case JO_F16:
    case JO_BF16: return 2;
    case JO_Q4_0: return 18;
    case JO_Q8_0: return 34;
    case JO_ACT_Q8: return 36;
    case JO_Q4_K: return 144;
    case JO_Q6_K: return 210;
    case JO_Q8_K: return 292;
    default: return 0;
  }
}

int64_t jo_row_bytes(int quant, int64_t n) {
  int64_t be = jo_block_elems(quant);
  if (be <= 0 || n < 0 || n % be) return -1;
  return (n / be) * jo_block_bytes(quant);
}

int jo_act_format(int weight_quant) {
  switch (weight_quant) {
    case JO_Q4_0:
    case JO_Q8_0: return JO_ACT_Q8;
    case JO_Q4_K:
    case JO_Q6_K: return JO_Q8_K;
    case JO_F32:
    case JO_F16:
    case JO_BF16: return JO_F32; /* the f32 input itself (matvec_f32, vec_dot_f16/bf16) */
    default: return -1;
  }
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline float rdf32(const uint8_t *p) {
  float f;
  memcpy(&f, p, 4);
  return f;
}
static inline int16_t rdi16(const uint8_t *p) { return (int16_t)rd16(p); }

/* Q4_K 6-bit scale/min of sub-block j (ggml get_scale_min_k4). */
static inline void q4k_scale_min(int j, const uint8_t *s, int *sc, int *m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* Unpack one Q6_K block to 256 signed values in [-32, 31] and return the 16 scales. */
static void q6k_unpack(const uint8_t *b, int8_t q[256], int8_t sc[16]) {
  const uint8_t *ql = b, *qh = b + 128;
  for (int n = 0; n < 2; n++) {
    for (int l = 0; l < 32; l++) {
      q[128 * n + l] = (int8_t)(((ql[64 * n + l] & 0xF) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32);
      q[128 * n + l + 32] = (int8_t)(((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32);
      q[128 * n + l + 64] = (int8_t)(((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32);
      q[128 * n + l + 96] = (int8_t)(((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32);
    }
  }
  memcpy(sc, b + 192, 16);
}

int jo_dequantize_row(int quant, const void *row, int64_t n, float *out) {
  const uint8_t *p = (const uint8_t *)row;
  int64_t be = jo_block_elems(quant), bb = jo_block_bytes(quant);
  if (be <= 0 || n % be) return -1;
  int64_t nb = n / be;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t *blk = p + b * bb;
    float *y = out + b * be;
    switch (quant) {
      case JO_F32: y[0] = rdf32(blk); break;
      case JO_F16: y[0] = jo_f16_to_f32(rd16(blk)); break;
      case JO_BF16: {
        uint32_t bits = (uint32_t)rd16(blk) << 16;
        memcpy(&y[0], &bits, 4);
      } break;
      case JO_Q8_0: {
        float d = jo_f16_to_f32(rd16(blk));
        for (int j = 0; j < 32; j++) y[j] = d * (float)(int8_t)blk[2 + j];
      } break;
      case JO_Q4_0: {
        float d = jo_f16_to_f32(rd16(blk));
        for (int j = 0; j < 16; j++) {
          y[j] = d * (float)((blk[2 + j] & 0xF) - 8);
          y[j + 16] = d * (float)((blk[2 + j] >> 4) - 8);
        }
      } break;
      case JO_ACT_Q8: {
        float d = rdf32(blk);
        for (int j = 0; j < 32; j++) y[j] = d * (float)(int8_t)blk[4 + j];
      } break;
      case JO_Q4_K: {
        float d = jo_f16_to_f32(rd16(blk)), dmin = jo_f16_to_f32(rd16(blk + 2));
        const uint8_t *s = blk + 4, *qs = blk + 16;
        for (int i = 0; i < 4; i++) {
          int sc1, m1, sc2, m2;
          q4k_scale_min(2 * i, s, &sc1, &m1);
          q4k_scale_min(2 * i + 1, s, &sc2, &m2);
          float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
          float d2 = d * (float)sc2, mm2 = dmin * (float)m2;
          for (int l = 0; l < 32; l++) {
            y[64 * i + l] = d1 * (float)(qs[32 * i + l] & 0xF) - mm1;
            y[64 * i + 32 + l] = d2 * (float)(qs[32 * i + l] >> 4) - mm2;
          }
        }
      } break;
      case JO_Q6_K: {
        int8_t q[256], sc[16];
        q6k_unpack(blk, q, sc);
        float d = jo_f16_to_f32(rd16(blk + 208));
        for (int l = 0; l < 256; l++) y[l] = d * (float)sc[l / 16] * (float)q[l];
      } break;
      case JO_Q8_K: {
        float d = rdf32(blk);
        for (int j = 0; j < 256; j++) y[j] = d * (float)(int8_t)blk[4 + j];
      } break;
      default: return -1;
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ activation quantizers */

/* QuantizedActQ8 block: {f32 d; i8 q[32]}.  d = amax/127 stays f32 (an f16 d misses the
 * golden llama logits by 0.19; the f32 d matches them to 8e-7).  q = round-half-even(x * (1/d)). */
void jo_quantize_act_q8(const float *x, int64_t m, int64_t k, void *out) {
  uint8_t *o = (uint8_t *)out;
  int64_t nb = k / 32;
  for (int64_t r = 0; r < m; r++) {
    for (int64_t b = 0; b < nb; b++) {
      const float *xb = x + r * k + b * 32;
      uint8_t *ob = o + (r * nb + b) * 36;
      float amax = 0.0f;
      for (int j = 0; j < 32; j++) {
        float a = fabsf(xb[j]);
        if (a > amax) amax = a;
      }
      float d = amax / 127.0f;
      float id = d != 0.0f ? 1.0f / d : 0.0f;
      memcpy(ob, &d, 4);
      for (int j = 0; j < 32; j++) {
        float v = xb[j] * id;
        ob[4 + j] = (uint8_t)(int8_t)(int)nearbyintf(v);
      }
    }
  }
}

/* Q8_K block: {f32 d; i8 qs[256]; i16 bsums[16]} (ggml quantize_row_q8_K_ref). The signed
 * element of largest magnitude (first one on ties) sets iscale = -127/max; q = min(127,
 * round-half-even(iscale*x)); d = 1/iscale; bsums are sums of 16 consecutive q. */
void jo_quantize_q8_k(const float *x, int64_t m, int64_t k, void *out) {
  uint8_t *o = (uint8_t *)out;
  int64_t nb = k / 256;
  for (int64_t r = 0; r < m; r++) {
    for (int64_t b = 0; b < nb; b++) {
      const float *xb = x + r * k + b * 256;
      uint8_t *ob = o + (r * nb + b) * 292;
      float amax = 0.0f, mx = 0.0f;
      for (int j = 0; j < 256; j++) {
        float a = fabsf(xb[j]);
        if (a > amax) {
          amax = a;
          mx = xb[j];
        }
      }
      if (amax == 0.0f) {
        memset(ob, 0, 292);
        continue;
      }
      float iscale = -127.0f / mx;
      int8_t q[256];
      for (int j = 0; j < 256; j++) {
        int v = (int)nearbyintf(iscale * xb[j]);
        q[j] = (int8_t)(v < 127 ? v : 127);
      }
      float d = 1.0f / iscale;
      memcpy(ob, &d, 4);
      memcpy(ob + 4, q, 256);
      for (int g = 0; g < 16; g++) {
        int s = 0;
        for (int l = 0; l < 16; l++) s += q[16 * g + l];
        int16_t s16 = (int16_t)s;
        memcpy(ob + 260 + 2 * g, &s16, 2);
      }
    }
  }
}

void jo_quantize_act(int act_quant, const float *x, int64_t m, int64_t k, void *out) {
  if (act_quant == JO_F32) { /* unquantized input of the float weight formats */
    memcpy(out, x, (size_t)(m * k) * 4);
    return;
  }
  if (act_quant == JO_Q8_K)
    jo_quantize_q8_k(x, m, k, out);
  else
    jo_quantize_act_q8(x, m, k, out);
}

/* ------------------------------------------------------------------ dot products */

int64_t jo_partials_per_row(int quant, int64_t k) {
  switch (quant) {
    case JO_Q8_0:
    case JO_Q4_0: return k / 32;
    case JO_Q4_K: return k / 32;
    case JO_Q6_K: return k / 16;
    default: return 0;
  }
}

double jo_vec_dot_row(int quant, const void *wrow, int64_t k, const void *xq, int32_t *partials) {
  const uint8_t *w = (const uint8_t *)wrow, *a = (const uint8_t *)xq;
  double acc = 0.0;
  switch (quant) {
    case JO_Q8_0: /* y = sum_b f16(d_w) * d_x * sum_32 q_w q_x */
      for (int64_t b = 0; b < k / 32; b++) {
        const uint8_t *wb = w + b * 34, *ab = a + b * 36;
        int32_t s = 0;
        for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)wb[2 + j] * (int32_t)(int8_t)ab[4 + j];
        if (partials) partials[b] = s;
        acc += (double)jo_f16_to_f32(rd16(wb)) * (double)rdf32(ab) * (double)s;
      }
      break;
    case JO_Q4_0: /* y = sum_b f16(d_w) * d_x * sum_32 (q4 - 8) q_x */
      for (int64_t b = 0; b < k / 32; b++) {
        const uint8_t *wb = w + b * 18, *ab = a + b * 36;
        int32_t s = 0;
        for (int j = 0; j < 16; j++) {
          s += ((wb[2 + j] & 0xF) - 8) * (int32_t)(int8_t)ab[4 + j];
          s += ((wb[2 + j] >> 4) - 8) * (int32_t)(int8_t)ab[4 + j + 16];
        }
        if (partials) partials[b] = s;
        acc += (double)jo_f16_to_f32(rd16(wb)) * (double)rdf32(ab) * (double)s;
      }
      break;
    case JO_Q4_K: /* y = sum_b d_x (d sum_j sc_j S_j - dmin sum_j m_j sum(q8 in j)) */
      for (int64_t b = 0; b < k / 256; b++) {
        const uint8_t *wb = w + b * 144, *ab = a + b * 292;
        const uint8_t *s = wb + 4, *qs = wb + 16;
        const int8_t *q8 = (const int8_t *)(ab + 4);
        int64_t isum = 0, msum = 0;
        for (int j = 0; j < 8; j++) {
          int sc, mn;
          q4k_scale_min(j, s, &sc, &mn);
          int i = j / 2, hi = j & 1;
          int32_t S = 0, qsum = 0;
          for (int l = 0; l < 32; l++) {
            int q4 = hi ? (qs[32 * i + l] >> 4) : (qs[32 * i + l] & 0xF);
            S += q4 * q8[32 * j + l];
            qsum += q8[32 * j + l];
          }
          if (partials) partials[b * 8 + j] = S;
          isum += (int64_t)sc * S;
          msum += (int64_t)mn * qsum;
        }
        double dx = rdf32(ab);
        acc += dx * ((double)jo_f16_to_f32(rd16(wb)) * (double)isum -
                     (double)jo_f16_to_f32(rd16(wb + 2)) * (double)msum);
      }
      break;
    case JO_F32:
    case JO_F16:
    case JO_BF16: /* matvec_f32 / vec_dot_f16 / vec_dot_bf16 (src/gemma.rs:72-74,140-189): the row
                     widened to f32 dotted with the f32 input, accumulated in f64 here */
      for (int64_t i = 0; i < k; i++) {
        float wv;
        jo_dequantize_row(quant, w + i * jo_block_bytes(quant), 1, &wv);
        acc += (double)wv * (double)rdf32(a + 4 * i);
      }
      break;
    case JO_Q6_K: /* y = sum_b d_x d sum_i sc_i sum_16 (q6 - 32) q8 */
      for (int64_t b = 0; b < k / 256; b++) {
        const uint8_t *wb = w + b * 210, *ab = a + b * 292;
        const int8_t *q8 = (const int8_t *)(ab + 4);
        int8_t q[256], sc[16];
        q6k_unpack(wb, q, sc);
        int64_t isum = 0;
        for (int g = 0; g < 16; g++) {
          int32_t S = 0;
          for (int l = 0; l < 16; l++) S += q[16 * g + l] * q8[16 * g + l];
          if (partials) partials[b * 16 + g] = S;
          isum += (int64_t)sc[g] * S;
        }
        acc += (double)rdf32(ab) * (double)jo_f16_to_f32(rd16(wb + 208)) * (double)isum;
      }
      break;
    default: break;
  }
  return acc;
}

/* ------------------------------------------------------------------ threaded row loops */

typedef struct {
  int quant;
  const uint8_t *w;
  int64_t k, n, row_bytes, act_row_bytes, chunk;
  const uint8_t *xq;
  int64_t m; /* activation rows (GEMM) */
  float *y;
  int tid, threads;
} jo_job;

static void *jo_worker(void *arg) {
  jo_job *j = (jo_job *)arg;
  int64_t nchunks = (j->n + j->chunk - 1) / j->chunk;
  for (int64_t c = j->tid; c < nchunks; c += j->threads) {
    int64_t r0 = c * j->chunk, r1 = r0 + j->chunk < j->n ? r0 + j->chunk : j->n;
    for (int64_t mm = 0; mm < j->m; mm++)
      for (int64_t r = r0; r < r1; r++)
        j->y[mm * j->n + r] =
            (float)jo_vec_dot_row(j->quant, j->w + r * j->row_bytes, j->k, j->xq + mm * j->act_row_bytes, NULL);
  }
  return NULL;
}

static int jo_run_rows(int quant, const void *w, int64_t k, int64_t n, const void *xq, int64_t m, float *y,
                       int threads) {
  int act = jo_act_format(quant);
  if (act < 0 || k <= 0 || n <= 0 || jo_row_bytes(quant, k) < 0) return -1;
  if (threads < 1) threads = 1;
  if (n < 64) threads = 1; /* matvec_any runs short outputs on the caller thread */
  int64_t chunk = (n + threads - 1) / threads;
  if (chunk < 16) chunk = 16;
  if (chunk > 2048) chunk = 2048;
  jo_job jobs[256];
  pthread_t th[256];
  if (threads > 256) threads = 256;
  for (int t = 0; t < threads; t++) {
    jobs[t] = (jo_job){quant, (const uint8_t *)w, k, n, jo_row_bytes(quant, k), jo_row_bytes(act, k), chunk,
                       (const uint8_t *)xq, m, y, t, threads};
  }
  if (threads == 1) {
    jo_worker(&jobs[0]);
    return 0;
  }
  for (int t = 0; t < threads; t++) pthread_create(&th[t], NULL, jo_worker, &jobs[t]);
  for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
  return 0;
}

int jo_matvec(int quant, const void *w, int64_t k, int64_t n, const void *xq, float *y, int threads) {
  return jo_run_rows(quant, w, k, n, xq, 1, y, threads);
}

int jo_gemm(int quant, const void *w, int64_t k, int64_t n, const void *xq, int64_t m, float *y, int threads) {
  return jo_run_rows(quant, w, k, n, xq, m, y, threads);
}

int jo_vec_dot(int quant, const void *w, int64_t k, int64_t n, const float *x, float *y, int threads) {
  int act = jo_act_format(quant);
  if (act < 0 || jo_row_bytes(act, k) < 0) return -1;
  void *xq = malloc((size_t)jo_row_bytes(act, k));
  if (!xq) return -1;
  jo_quantize_act(act, x, 1, k, xq);
  int rc = jo_matvec(quant, w, k, n, xq, y, threads);
  free(xq);
  return rc;
}

int jo_matvec_dequant_f64(int quant, const void *w, int64_t k, int64_t n, const void *xq, double *y) {
  int act = jo_act_format(quant);
  int64_t rb = jo_row_bytes(quant, k);
  if (act < 0 || rb < 0) return -1;
  float *wr = (float *)malloc((size_t)k * 4), *xr = (float *)malloc((size_t)k * 4);
  if (!wr || !xr) {
    free(wr);
    free(xr);
    return -1;
  }
  jo_dequantize_row(act, xq, k, xr);
  for (int64_t r = 0; r < n; r++) {
    jo_dequantize_row(quant, (const uint8_t *)w + r * rb, k, wr);
    double s = 0.0;
    for (int64_t i = 0; i < k; i++) s += (double)wr[i] * (double)xr[i];
    y[r] = s;
  }
  free(wr);
  free(xr);
  return 0;
}

int jo_matvec_partials(int quant, const void *w, int64_t k, int64_t n, const void *xq, int32_t *partials) {
  int64_t rb = jo_row_bytes(quant, k), pp = jo_partials_per_row(quant, k);
  if (rb < 0 || pp <= 0) return -1;
  for (int64_t r = 0; r < n; r++) jo_vec_dot_row(quant, (const uint8_t *)w + r * rb, k, xq, partials + r * pp);
  return 0;
}

void jo_gemm_i8(const int8_t *x, int64_t m, const int8_t *w, int64_t n, int64_t k, int32_t *out) {
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      int32_t s = 0;
      for (int64_t t = 0; t < k; t++) s += (int32_t)x[i * k + t] * (int32_t)w[j * k + t];
      out[i * n + j] = s;
    }
}

/* ------------------------------------------------------------------ elementwise + attention */

void jo_rmsnorm(float *out, const float *x, const float *w, int64_t n, float eps) {
  double ss = 0.0;
  for (int64_t i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
  double scale = 1.0 / sqrt(ss / (double)n + (double)eps);
  for (int64_t i = 0; i < n; i++) out[i] = (float)((double)x[i] * scale * (double)w[i]);
}

void jo_rope_inplace(float *x, int64_t len, int hd, int64_t pos, float theta) {
  for (int64_t h = 0; h < len / hd; h++) {
    float *v = x + h * hd;
    for (int i = 0; i < hd / 2; i++) {
      float expo = (float)(2 * i) / (float)hd;
      float angle = (float)pos / powf(theta, expo); /* f32 angle, as the scalar reference */
      double c = cos((double)angle), s = sin((double)angle);
      double x0 = v[2 * i], x1 = v[2 * i + 1];
      v[2 * i] = (float)(x0 * c - x1 * s);
      v[2 * i + 1] = (float)(x0 * s + x1 * c);
    }
  }
}

void jo_swiglu(float *out, const float *gate, const float *up, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    double g = gate[i];
    out[i] = (float)(g / (1.0 + exp(-g)) * (double)up[i]);
  }
}

int64_t jo_argmax(const float *x, int64_t n) {
  int64_t best = -1;
  float bv = -INFINITY;
  for (int64_t i = 0; i < n; i++) {
    if (isnan(x[i])) continue;
    if (best < 0 || x[i] > bv) {
      bv = x[i];
      best = i;
    }
  }
  return best;
}

int jo_gqa_attention(float *out, const float *q, const float *k, const float *v, int nq, int nkv, int hd,
                     int64_t seq_len, float scale) {
  if (nq <= 0 || nkv <= 0 || hd <= 0 || nq % nkv || seq_len <= 0) return -1;
  int group = nq / nkv;
  int64_t kvd = (int64_t)nkv * hd;
  double *sc = (double *)malloc((size_t)seq_len * sizeof(double));
  double *acc = (double *)malloc((size_t)hd * sizeof(double));
  if (!sc || !acc) {
    free(sc);
    free(acc);
    return -1;
  }
  for (int h = 0; h < nq; h++) {
    int kh = h / group;
    const float *qh = q + (int64_t)h * hd;
    double mx = -INFINITY;
    for (int64_t t = 0; t < seq_len; t++) {
      const float *kt = k + t * kvd + (int64_t)kh * hd;
      double s = 0.0;
      for (int d = 0; d < hd; d++) s += (double)qh[d] * (double)kt[d];
      s *= (double)scale;
      sc[t] = s;
      if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (int64_t t = 0; t < seq_len; t++) {
      sc[t] = exp(sc[t] - mx);
      sum += sc[t];
    }
    for (int d = 0; d < hd; d++) acc[d] = 0.0;
    for (int64_t t = 0; t < seq_len; t++) {
      const float *vt = v + t * kvd + (int64_t)kh * hd;
      double p = sc[t] / sum;
      for (int d = 0; d < hd; d++) acc[d] += p * (double)vt[d];
    }
    for (int d = 0; d < hd; d++) out[(int64_t)h * hd + d] = (float)acc[d];
  }
  free(sc);
  free(acc);
  return 0;
}

/* f32::total_cmp as a signed integer key: for a negative float every bit but the sign is
 * flipped, so the keys order -inf < ... < -0.0 < +0.0 < ... < +inf as signed integers. */
static int32_t jo_total_key(float f) {
  int32_t b;
  memcpy(&b, &f, 4);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

/* select_top_k_experts (src/gemma.rs:362-442): f32 softmax over all experts, stable order
 * by logit descending under f32::total_cmp (:417; non-finite logits rank as -inf, +0.0 above
 * -0.0) with the lower index first, take k, renormalise the chosen probabilities when
 * normalize != 0. */
int jo_select_top_k(const float *logits, int64_t n, int top_k, int normalize, int32_t *idx, float *w) {
  if (n <= 0 || top_k <= 0) return 0;
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; i++)
    if (isfinite(logits[i]) && logits[i] > mx) mx = logits[i];
  float *p = (float *)malloc((size_t)n * 4);
  int64_t *ord = (int64_t *)malloc((size_t)n * 8);
  if (!p || !ord) {
    free(p);
    free(ord);
    return 0;
  }
  float sum = 0.0f;
  for (int64_t i = 0; i < n; i++) {
    p[i] = (isfinite(logits[i]) && isfinite(mx)) ? expf(logits[i] - mx) : 0.0f;
    sum += p[i];
  }
  if (sum > 0.0f && isfinite(sum)) {
    for (int64_t i = 0; i < n; i++) p[i] /= sum;
  } else {
    for (int64_t i = 0; i < n; i++) p[i] = 1.0f / (float)n;
  }
  /* insertion order by (logit desc, index asc) */
  for (int64_t i = 0; i < n; i++) ord[i] = i;
  for (int64_t i = 1; i < n; i++) {
    int64_t cur = ord[i];
    int32_t lc = jo_total_key(isfinite(logits[cur]) ? logits[cur] : -INFINITY);
    int64_t j = i - 1;
    while (j >= 0) {
      int32_t lj = jo_total_key(isfinite(logits[ord[j]]) ? logits[ord[j]] : -INFINITY);
      if (lj < lc) {
        ord[j + 1] = ord[j];
        j--;
      } else {
        break;
      }
    }
    ord[j + 1] = cur;
  }
  int k = top_k < n ? top_k : (int)n;
  float ssum = 0.0f;
  for (int i = 0; i < k; i++) {
    idx[i] = (int32_t)ord[i];
    w[i] = p[ord[i]];
    ssum += w[i];
  }
  if (normalize) {
    if (ssum > 0.0f && isfinite(ssum)) {
      for (int i = 0; i < k; i++) w[i] /= ssum;
    } else {
      for (int i = 0; i < k; i++) w[i] = 1.0f / (float)k;
    }
  }
  free(p);
  free(ord);
  return k;
}

/* ------------------------------------------------------------------ MoE */

static int jo_matvec_f32in(int quant, const void *w, int64_t k, int64_t n, const float *x, float *y, int threads) {
  return jo_vec_dot(quant, w, k, n, x, y, threads);
}

int jo_swiglu_expert(int gate_quant, const void *gate, int up_quant, const void *up, int down_quant,
                     const void *down, int64_t hidden, int64_t ffn, const float *x, float *y) {
  float *g = (float *)malloc((size_t)ffn * 4), *u = (float *)malloc((size_t)ffn * 4);
  float *a = (float *)malloc((size_t)ffn * 4);
  int rc = (!g || !u || !a) ? -1 : 0;
  if (!rc) rc = jo_matvec_f32in(gate_quant, gate, hidden, ffn, x, g, 1);
  if (!rc) rc = jo_matvec_f32in(up_quant, up, hidden, ffn, x, u, 1);
  if (!rc) {
    jo_swiglu(a, g, u, ffn);
    rc = jo_matvec_f32in(down_quant, down, ffn, hidden, a, y, 1);
  }
  free(g);
  free(u);
  free(a);
  return rc;
}

typedef struct {
  const float *router_logits;
  int64_t t0, t1, n_experts;
  int top_k, gq, uq, dq;
  const uint8_t *gate, *up, *down;
  int64_t hidden, ffn;
  const float *x;
  float *y;
  int32_t *sel_idx;
  float *sel_w;
  int rc;
} jo_moe_job;

static void *jo_moe_worker(void *arg) {
  jo_moe_job *j = (jo_moe_job *)arg;
  int64_t gstride = jo_row_bytes(j->gq, j->hidden) * j->ffn;
  int64_t ustride = jo_row_bytes(j->uq, j->hidden) * j->ffn;
  int64_t dstride = jo_row_bytes(j->dq, j->ffn) * j->hidden;
  float *tmp = (float *)malloc((size_t)j->hidden * 4);
  if (!tmp) {
    j->rc = -1;
    return NULL;
  }
  for (int64_t t = j->t0; t < j->t1; t++) {
    int32_t *idx = j->sel_idx + t * j->top_k;
    float *w = j->sel_w + t * j->top_k;
    int k = jo_select_top_k(j->router_logits + t * j->n_experts, j->n_experts, j->top_k, 1, idx, w);
    float *yt = j->y + t * j->hidden;
    for (int64_t i = 0; i < j->hidden; i++) yt[i] = 0.0f;
    for (int s = 0; s < k; s++) {
      int64_t e = idx[s];
      if (jo_swiglu_expert(j->gq, j->gate + e * gstride, j->uq, j->up + e * ustride, j->dq, j->down + e * dstride,
                           j->hidden, j->ffn, j->x + t * j->hidden, tmp)) {
        j->rc = -1;
        break;
      }
      for (int64_t i = 0; i < j->hidden; i++) yt[i] += w[s] * tmp[i];
    }
  }
  free(tmp);
  return NULL;
}

int jo_moe_ffn(const float *router_logits, int64_t t, int64_t n_experts, int top_k, int gate_quant,
               const void *gate, int up_quant, const void *up, int down_quant, const void *down, int64_t hidden,
               int64_t ffn, const float *x, float *y, int32_t *sel_idx, float *sel_w, int threads) {
  if (t <= 0 || n_experts <= 0 || top_k <= 0 || top_k > n_experts) return -1;
  if (threads < 1) threads = 1;
  if (threads > t) threads = (int)t;
  if (threads > 256) threads = 256;
  jo_moe_job jobs[256];
  pthread_t th[256];
  int64_t per = (t + threads - 1) / threads;
  for (int i = 0; i < threads; i++) {
    int64_t t0 = i * per, t1 = t0 + per < t ? t0 + per : t;
    jobs[i] = (jo_moe_job){router_logits, t0, t1, n_experts, top_k, gate_quant, up_quant, down_quant,
                           (const uint8_t *)gate, (const uint8_t *)up, (const uint8_t *)down, hidden, ffn, x, y,
                           sel_idx, sel_w, 0};
  }
  for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, jo_moe_worker, &jobs[i]);
  int rc = 0;
  for (int i = 0; i < threads; i++) {
    pthread_join(th[i], NULL);
    if (jobs[i].rc) rc = jobs[i].rc;
  }
  return rc;
}

/* ------------------------------------------------------------------ decode step */

static void jo_head_rmsnorm(float *x, int64_t len, int hd, const float *w, float eps) {
  float *tmp = (float *)malloc((size_t)hd * 4);
  for (int64_t h = 0; h < len / hd; h++) {
    jo_rmsnorm(tmp, x + h * hd, w, hd, eps);
    memcpy(x + h * hd, tmp, (size_t)hd * 4);
  }
  free(tmp);
}

/* y = W . x for an f32 x: x quantized to W's activation format (written to q8 when given),
 * then jo_matvec. */
static int jo_matvec_q(int quant, const void *w, int64_t k, int64_t n, const float *x, float *y, int threads,
                       void *q8) {
  int act = jo_act_format(quant);
  int64_t qb = jo_row_bytes(act, k);
  if (act < 0 || qb < 0) return -1;
  void *xq = malloc((size_t)qb);
  if (!xq) return -1;
  jo_quantize_act(act, x, 1, k, xq);
  if (q8) memcpy(q8, xq, (size_t)qb);
  int rc = jo_matvec(quant, w, k, n, xq, y, threads);
  free(xq);
  return rc;
}

/* project_or_deterministic_slice (src/gemma.rs:841-860): the projection when the tensor is present
 * (its element count out_len * in_len is checked when the model is built), else the deterministic
 * slice out[i] = in[i % in_len] * scale.  A fallback leaves the activation-block trace untouched. */
static int proj_or_det(const jo_tensor *w, int64_t in_len, int64_t out_len, const float *in, float *out, float scale,
                       int threads, void *q8_trace) {
  if (!w->data) {
    for (int64_t i = 0; i < out_len; i++) out[i] = in[i % in_len] * scale;
    return 0;
  }
  return jo_matvec_q(w->quant, w->data, in_len, out_len, in, out, threads, q8_trace);
}

/* The attention sublayer of layer L (src/qwen_deepseek.rs:1262-1275 with
 * run_dense_attention_sublayer_scaled :984-1097): x += Wo(attention(RMSNorm(x))); writes K/V of
 * `pos` into layer L's rings. */
int jo_decode_attn(const jo_model *M, float *kv, int64_t L, float *x, int64_t pos, int threads,
                   const jo_layer_trace *tr) {
  const int64_t H = M->hidden, qd = (int64_t)M->nq * M->hd, kvd = (int64_t)M->nkv * M->hd;
  const int64_t cap = M->kv_capacity;
  /* the attention sublayer and QK-norm use rms_eps as given */
  const float eps_attn = M->eps;
  static const jo_layer_trace none;
  if (!tr) tr = &none;
  if (L < 0 || L >= M->n_layers || cap <= 0 || pos < 0) return -1;
  const jo_layer *ly = &M->layers[L];
  float *xn = (float *)malloc((size_t)H * 4), *qkv = (float *)malloc((size_t)(qd + 2 * kvd) * 4);
  float *att = (float *)malloc((size_t)qd * 4), *proj = (float *)malloc((size_t)H * 4);
  int rc = (!xn || !qkv || !att || !proj) ? -1 : 0;
  float *q = qkv, *k = qkv + qd, *v = qkv + qd + kvd;
  if (!rc) {
    jo_rmsnorm(xn, x, ly->attn_norm, H, eps_attn);
    if (tr->xn_attn) memcpy(tr->xn_attn, xn, (size_t)H * 4);
    /* scales of the fallback: q 0.5, k 0.25, v 0.125 (src/qwen_deepseek.rs:1011-1031) */
    rc |= proj_or_det(&ly->wq, H, qd, xn, q, 0.5f, threads, tr->q8_attn);
    rc |= proj_or_det(&ly->wk, H, kvd, xn, k, 0.25f, threads, NULL);
    rc |= proj_or_det(&ly->wv, H, kvd, xn, v, 0.125f, threads, NULL);
  }
  if (!rc) {
    if (tr->qkv) memcpy(tr->qkv, qkv, (size_t)(qd + 2 * kvd) * 4);
    /* QK-norm before RoPE (:1039-1071) */
    if (ly->q_norm) jo_head_rmsnorm(q, qd, M->hd, ly->q_norm, eps_attn);
    if (ly->k_norm) jo_head_rmsnorm(k, kvd, M->hd, ly->k_norm, eps_attn);
    jo_rope_inplace(q, qd, M->hd, pos, M->theta);
    jo_rope_inplace(k, kvd, M->hd, pos, M->theta);
    if (tr->q_rope) memcpy(tr->q_rope, q, (size_t)qd * 4);
    if (tr->k_rope) memcpy(tr->k_rope, k, (size_t)kvd * 4);
    float *kring = kv + L * 2 * cap * kvd, *vring = kring + cap * kvd;
    int64_t slot = pos % cap, active = pos + 1 < cap ? pos + 1 : cap;
    memcpy(kring + slot * kvd, k, (size_t)kvd * 4);
    memcpy(vring + slot * kvd, v, (size_t)kvd * 4);
    if (M->kv_f16) /* an f16 ring: the new row as the ring holds it, before it is attended */
      for (int64_t i = 0; i < kvd; i++) {
        kring[slot * kvd + i] = jo_f16_to_f32(jo_f32_to_f16(kring[slot * kvd + i]));
        vring[slot * kvd + i] = jo_f16_to_f32(jo_f32_to_f16(vring[slot * kvd + i]));
      }
    rc |= jo_gqa_attention(att, q, kring, vring, M->nq, M->nkv, M->hd, active, 1.0f / sqrtf((float)M->hd));
  }
  if (!rc) {
    if (tr->attn) memcpy(tr->attn, att, (size_t)qd * 4);
    rc |= proj_or_det(&ly->wo, qd, H, att, proj, 0.25f, threads, tr->q8_wo); /* :1086-1092 */
    for (int64_t i = 0; i < H; i++) x[i] += proj[i];
    if (tr->x_mid) memcpy(tr->x_mid, x, (size_t)H * 4);
  }
  free(xn);
  free(qkv);
  free(att);
  free(proj);
  return rc;
}

int jo_decode_layer(const jo_model *M, float *kv, int64_t L, float *x, int64_t pos, int threads,
                    const jo_layer_trace *tr) {
  const int64_t H = M->hidden, F = M->ffn;
  /* the FFN norm uses rms_eps.max(1e-6) (:1251) */
  const float eps_ffn = M->eps > 1e-6f ? M->eps : 1e-6f;
  static const jo_layer_trace none;
  if (!tr) tr = &none;
  int rc = jo_decode_attn(M, kv, L, x, pos, threads, tr);
  if (rc) return rc;
  const jo_layer *ly = &M->layers[L];
  float *xn = (float *)malloc((size_t)H * 4), *proj = (float *)malloc((size_t)H * 4);
  float *gu = (float *)malloc((size_t)F * 8), *a = (float *)malloc((size_t)F * 4);
  rc = (!xn || !proj || !gu || !a) ? -1 : 0;
  if (!rc) {
    jo_rmsnorm(xn, x, ly->ffn_norm, H, eps_ffn);
    if (tr->xn_ffn) memcpy(tr->xn_ffn, xn, (size_t)H * 4);
    /* run_dense_swiglu_ffn (:696-725): gate 0.5, up 0.25, down 0.125 */
    rc |= proj_or_det(&ly->w_gate, H, F, xn, gu, 0.5f, threads, tr->q8_ffn);
    rc |= proj_or_det(&ly->w_up, H, F, xn, gu + F, 0.25f, threads, NULL);
  }
  if (!rc) {
    if (tr->gu) memcpy(tr->gu, gu, (size_t)F * 8);
    jo_swiglu(a, gu, gu + F, F);
    if (tr->act) memcpy(tr->act, a, (size_t)F * 4);
    rc |= proj_or_det(&ly->w_down, F, H, a, proj, 0.125f, threads, tr->q8_down);
    for (int64_t i = 0; i < H; i++) x[i] += proj[i];
  }
  free(xn);
  free(proj);
  free(gu);
  free(a);
  return rc;
}

void jo_read_f32_weight_or_default(int quant, const void *data, int64_t n_elements, int64_t len, float def,
                                   float *out) {
  for (int64_t i = 0; i < len; i++) out[i] = def;
  if (!data || len <= 0) return;
  if (quant == JO_F32) { /* :499-509: stored finite values, `def` elsewhere */
    const uint8_t *raw = (const uint8_t *)data;
    for (int64_t i = 0; i < len && i < n_elements; i++) {
      float v = rdf32(raw + 4 * i);
      if (isfinite(v)) out[i] = v;
    }
    return;
  }
  if (n_elements < len) return; /* :510 */
  float *deq = (float *)malloc((size_t)len * 4);
  if (!deq) return;
  if (jo_dequantize_row(quant, data, len, deq) == 0) memcpy(out, deq, (size_t)len * 4); /* row 0, :511-514 */
  free(deq);
}

int64_t jo_logits_len(int64_t vocab, int has_head, int64_t head_rows) {
  if (has_head && head_rows > vocab && head_rows % 64 == 0 && head_rows - vocab <= 1024) return head_rows;
  return vocab;
}

/* The reference rounds each f32 operation of the deterministic rows on its own: no contraction
 * into fused multiply-adds here (nor in jo_decode_head's fallback). */
__attribute__((optimize("fp-contract=off"))) int jo_embed_token(const jo_model *M, uint32_t token, float *x) {
  const int64_t H = M->hidden;
  if (M->tok_embd.data && (int64_t)token < M->embd_rows)
    return jo_dequantize_row(M->tok_embd.quant,
                             (const uint8_t *)M->tok_embd.data + (int64_t)token * jo_row_bytes(M->tok_embd.quant, H), H,
                             x);
  const float seed = (float)(token % 31u) * 0.05f + 0.25f; /* :574-580 */
  for (int64_t i = 0; i < H; i++) x[i] = seed + (float)(i % 7) * 0.01f;
  return 0;
}

static int64_t model_logits_len(const jo_model *M) { return M->logits_len > 0 ? M->logits_len : M->vocab; }

__attribute__((optimize("fp-contract=off"))) int jo_decode_head(const jo_model *M, const float *x, float *logits,
                                                                int threads, float *xn_head, void *q8_head) {
  const int64_t H = M->hidden, L = model_logits_len(M);
  const float eps = M->eps > 1e-6f ? M->eps : 1e-6f; /* :1305-1306 */
  float *xn = (float *)malloc((size_t)H * 4);
  if (!xn) return -1;
  jo_rmsnorm(xn, x, M->output_norm, H, eps);
  if (xn_head) memcpy(xn_head, xn, (size_t)H * 4);
  int rc = 0;
  const int64_t rows = M->output.data ? M->out_rows : 0;
  if (rows > 0 && M->out_in == H) {
    /* the head's first min(L, rows) rows (slice_rows), the rest a slice of xn (:607-618) */
    const int64_t target = L < rows ? L : rows;
    rc = jo_matvec_q(M->output.quant, M->output.data, H, target, xn, logits, threads, q8_head);
    for (int64_t i = target; i < L; i++) logits[i] = xn[i % H] * 0.05f;
  } else if (rows > 0 && M->out_in * rows == L * H) {
    /* the same elements read as L rows of H (:620-623) */
    rc = jo_matvec_q(M->output.quant, M->output.data, H, L, xn, logits, threads, q8_head);
  } else {
    /* no usable head (:626-631): the sum in element order, as the iterator sums it */
    float sum = 0.0f;
    for (int64_t i = 0; i < H; i++) sum += xn[i];
    const float base = tanhf(sum / 16.0f);
    for (int64_t i = 0; i < L; i++) {
      const float t = base + xn[i % H] * 0.1f;
      logits[i] = t + (float)(i % 13) * 0.01f;
    }
  }
  free(xn);
  return rc;
}

int jo_decode_step(const jo_model *M, float *kv, int32_t token, int64_t pos, float *logits, int threads) {
  const int64_t H = M->hidden;
  if (token < 0 || M->kv_capacity <= 0) return -1;
  float *x = (float *)malloc((size_t)H * 4);
  if (!x) return -1;
  int rc = jo_embed_token(M, (uint32_t)token, x);
  for (int64_t L = 0; L < M->n_layers && !rc; L++) rc = jo_decode_layer(M, kv, L, x, pos, threads, NULL);
  if (!rc) rc = jo_decode_head(M, x, logits, threads, NULL, NULL);
  free(x);
  return rc;
}

/* ------------------------------------------------------------------ synthetic int8 ForwardModel */

/* splitmix (src/forward.rs:326-332): one SplitMix64 output for state x. */
uint64_t jo_splitmix(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* fill_small (src/forward.rs:335-343): out[i] = (splitmix(seed ^ i * C) & 15) - 8. */
void jo_fill_small(uint64_t seed, int64_t len, int8_t *out) {
  for (int64_t i = 0; i < len; i++)
    out[i] = (int8_t)((int)(jo_splitmix(seed ^ ((uint64_t)i * 0xA24BAED4963EE407ull)) & 0xF) - 8);
}

/* isqrt (src/forward.rs:747-758): Newton's iteration from x = v, y = ceil(v / 2), stopping when y
 * no longer decreases; the midpoint is floor((x + v / x) / 2) without overflow. */
uint64_t jo_isqrt(uint64_t v) {
  if (v < 2) return v;
  uint64_t x = v, y = v / 2 + (v & 1);
  while (y < x) {
    x = y;
    const uint64_t b = v / x;
    y = (x & b) + ((x ^ b) >> 1);
  }
  return x;
}

/* ForwardExec::rmsnorm (src/forward.rs:672-699): per row, rms = max(isqrt(sum v^2 / DIM), 1),
 * y = clamp(v * 48 / rms, -127, 127) with division truncating toward zero. */
void jo_fwd_rmsnorm(const int8_t *x, int64_t m, int8_t *out) {
  for (int64_t r = 0; r < m; r++) {
    const int8_t *row = x + r * JO_FWD_DIM;
    uint64_t ms = 0;
    for (int i = 0; i < JO_FWD_DIM; i++) ms += (uint64_t)((int32_t)row[i] * (int32_t)row[i]);
    uint64_t rq = jo_isqrt(ms / JO_FWD_DIM);
    int32_t rms = rq > INT32_MAX ? INT32_MAX : (int32_t)rq;
    if (rms < 1) rms = 1;
    for (int i = 0; i < JO_FWD_DIM; i++) {
      int32_t y = (int32_t)row[i] * 48 / rms;
      out[r * JO_FWD_DIM + i] = (int8_t)(y < -127 ? -127 : y > 127 ? 127 : y);
    }
  }
}

/* ForwardExec::attention (src/forward.rs:702-744): query row r sits at position start_pos + r and
 * attends to cache rows 0..=start_pos + r with integer weights w = clamp(q.k >> 10, 0, 127) + 1;
 * out = sum(w v) / sum(w), int64 division truncating toward zero. */
void jo_fwd_attention(const int8_t *q, const int8_t *k_cache, const int8_t *v_cache, int64_t m, int64_t start_pos,
                      int8_t *out) {
  int64_t acc[JO_FWD_DIM];
  for (int64_t r = 0; r < m; r++) {
    const int64_t pos = start_pos + r;
    const int8_t *qrow = q + r * JO_FWD_DIM;
    memset(acc, 0, sizeof acc);
    int64_t total = 0;
    for (int64_t t = 0; t <= pos; t++) {
      const int8_t *krow = k_cache + t * JO_FWD_DIM, *vrow = v_cache + t * JO_FWD_DIM;
      int32_t s = 0;
      for (int i = 0; i < JO_FWD_DIM; i++) s += (int32_t)qrow[i] * (int32_t)krow[i];
      int32_t sh = s >> 10;
      const int64_t w = (int64_t)(sh < 0 ? 0 : sh > 127 ? 127 : sh) + 1;
      total += w;
      for (int i = 0; i < JO_FWD_DIM; i++) acc[i] += w * vrow[i];
    }
    for (int i = 0; i < JO_FWD_DIM; i++) out[r * JO_FWD_DIM + i] = (int8_t)(acc[i] / total);
  }
}

/* requant (src/forward.rs:345-350) over a buffer; relu != 0 then clamps below at 0 (the up
 * projection, :963-966). */
static void fwd_requant(const int32_t *raw, int64_t n, int shift, int relu, int8_t *out) {
  for (int64_t i = 0; i < n; i++) {
    int32_t r = (int32_t)((uint32_t)raw[i] + (1u << (shift - 1))) >> shift;
    r = r < -127 ? -127 : r > 127 ? 127 : r;
    if (relu && r < 0) r = 0;
    out[i] = (int8_t)r;
  }
}

/* sat_add (src/forward.rs:817-821): i8 saturating add in place. */
static void fwd_sat_add(int8_t *a, const int8_t *b, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    int s = (int)a[i] + (int)b[i];
    a[i] = (int8_t)(s < -128 ? -128 : s > 127 ? 127 : s);
  }
}

typedef struct jo_fwd_mat {
  int64_t n, k; /* n padded to whole 8-row tiles (Matrix::random, src/forward.rs:364-377) */
  int shift;
  int8_t *rows;
} jo_fwd_mat;

typedef struct fwd_pool fwd_pool;

struct jo_fwd_model {
  uint64_t seed;
  int64_t vocab, cap, len;
  int threads;
  fwd_pool *pool; /* threads - 1 persistent workers (NULL: one thread) */
  jo_fwd_mat w[JO_FWD_LAYERS][6];
  jo_fwd_mat head;
  int8_t *kc[JO_FWD_LAYERS], *vc[JO_FWD_LAYERS];
};

static void fwd_pool_free(fwd_pool *p);

static int fwd_mat(jo_fwd_mat *m, uint64_t seed, int64_t n, int64_t k, int shift) {
  const int64_t n_pad = (n + 7) / 8 * 8;
  m->n = n_pad;
  m->k = k;
  m->shift = shift;
  m->rows = (int8_t *)calloc((size_t)(n_pad * k), 1);
  if (!m->rows) return -1;
  jo_fill_small(seed, n * k, m->rows);
  return 0;
}

void jo_fwd_free(jo_fwd_model *f) {
  if (!f) return;
  for (int l = 0; l < JO_FWD_LAYERS; l++) {
    for (int j = 0; j < 6; j++) free(f->w[l][j].rows);
    free(f->kc[l]);
    free(f->vc[l]);
  }
  free(f->head.rows);
  fwd_pool_free(f->pool);
  free(f);
}

/* ForwardModel::new (src/forward.rs:879-903): layer l's matrices from seeds
 * splitmix(seed ^ (16 l + 1..6)) in the order wq wk wv wo up down, shifts 6 (down: 7); the LM
 * head from splitmix(seed ^ 0xFFFF) with max(vocab, 1) rows. */
jo_fwd_model *jo_fwd_new(uint64_t seed, int64_t vocab, int64_t max_positions) {
  if (vocab < 0 || max_positions < 1) return NULL;
  jo_fwd_model *f = (jo_fwd_model *)calloc(1, sizeof *f);
  if (!f) return NULL;
  f->seed = seed;
  f->vocab = vocab;
  f->cap = max_positions;
  f->threads = 1;
  int bad = 0;
  for (int l = 0; l < JO_FWD_LAYERS; l++) {
    const uint64_t s = (uint64_t)l * 16;
    const int64_t shape[6][2] = {{JO_FWD_DIM, JO_FWD_DIM}, {JO_FWD_DIM, JO_FWD_DIM}, {JO_FWD_DIM, JO_FWD_DIM},
                                 {JO_FWD_DIM, JO_FWD_DIM}, {JO_FWD_FFN, JO_FWD_DIM}, {JO_FWD_DIM, JO_FWD_FFN}};
    for (int j = 0; j < 6; j++)
      bad |= fwd_mat(&f->w[l][j], jo_splitmix(seed ^ (s + 1 + (uint64_t)j)), shape[j][0], shape[j][1], j == 5 ? 7 : 6);
    f->kc[l] = (int8_t *)malloc((size_t)(max_positions * JO_FWD_DIM));
    f->vc[l] = (int8_t *)malloc((size_t)(max_positions * JO_FWD_DIM));
    bad |= !f->kc[l] || !f->vc[l];
  }
  bad |= fwd_mat(&f->head, jo_splitmix(seed ^ 0xFFFFull), vocab > 1 ? vocab : 1, JO_FWD_DIM, 6);
  if (bad) {
    jo_fwd_free(f);
    return NULL;
  }
  return f;
}

int64_t jo_fwd_head_rows(const jo_fwd_model *f) { return f->head.n; }
int64_t jo_fwd_len(const jo_fwd_model *f) { return f->len; }
void jo_fwd_reset(jo_fwd_model *f) { f->len = 0; }

const int8_t *jo_fwd_weight(const jo_fwd_model *f, int layer, int which, int64_t *n, int64_t *k, int *shift) {
  const jo_fwd_mat *m;
  if (layer == -1) m = &f->head;
  else if (layer >= 0 && layer < JO_FWD_LAYERS && which >= 0 && which < 6) m = &f->w[layer][which];
  else return NULL;
  *n = m->n;
  *k = m->k;
  *shift = m->shift;
  return m->rows;
}

/* embed (src/forward.rs:918-926): fill_small(seed ^ token * 0x9E3779B9, DIM) * 8. */
void jo_fwd_embed(uint64_t seed, uint32_t token, int8_t *out) {
  jo_fill_small(seed ^ ((uint64_t)token * 0x9E3779B9ull), JO_FWD_DIM, out);
  for (int i = 0; i < JO_FWD_DIM; i++) out[i] = (int8_t)(out[i] * 8);
}

/* Splits [0, n) into contiguous ranges, one per thread (the checker's speed only: every range
 * computes the same integers as a single pass).  The threads are a persistent pool whose workers
 * spin on a job generation counter, as the reference's WorkerPool does under its default Spin
 * coordination profile (src/affinity.rs:1991-2030); a worker that finds no job for a while yields
 * its core between polls. */
typedef void (*fwd_range_fn)(void *ctx, int64_t lo, int64_t hi);

#define FWD_MAX_THREADS 64

typedef struct {
  fwd_pool *pool;
  int idx; /* range idx + 1 of a job (range 0 is the caller's) */
} fwd_worker_arg;

struct fwd_pool {
  int workers;
  pthread_t th[FWD_MAX_THREADS - 1];
  fwd_worker_arg args[FWD_MAX_THREADS - 1];
  uint64_t gen;  /* incremented (release) once a job's fields are written */
  int stop;
  int remaining; /* workers that have not finished the current job */
  fwd_range_fn fn;
  void *ctx;
  int64_t n;
  int parts;
};

static void fwd_range_of(int64_t n, int parts, int part, int64_t *lo, int64_t *hi) {
  const int64_t chunk = (n + parts - 1) / parts;
  *lo = part * chunk < n ? part * chunk : n;
  *hi = (part + 1) * chunk < n ? (part + 1) * chunk : n;
}

static void *fwd_pool_worker(void *arg) {
  fwd_worker_arg *a = (fwd_worker_arg *)arg;
  fwd_pool *p = a->pool;
  uint64_t seen = 0;
  for (;;) {
    uint64_t g;
    long idle = 0;
    while ((g = __atomic_load_n(&p->gen, __ATOMIC_ACQUIRE)) == seen) {
      if (__atomic_load_n(&p->stop, __ATOMIC_ACQUIRE)) return NULL;
      if (++idle > (1L << 16)) sched_yield();
    }
    seen = g;
    if (a->idx < p->parts) {
      int64_t lo, hi;
      fwd_range_of(p->n, p->parts, a->idx, &lo, &hi);
      if (lo < hi) p->fn(p->ctx, lo, hi);
    }
    __atomic_sub_fetch(&p->remaining, 1, __ATOMIC_RELEASE);
  }
}

static void fwd_pool_free(fwd_pool *p) {
  if (!p) return;
  __atomic_store_n(&p->stop, 1, __ATOMIC_RELEASE);
  for (int t = 0; t < p->workers; t++) pthread_join(p->th[t], NULL);
  free(p);
}

static fwd_pool *fwd_pool_new(int threads) {
  fwd_pool *p = (fwd_pool *)calloc(1, sizeof *p);
  if (!p) return NULL;
  for (int t = 0; t < threads - 1; t++) {
    p->args[t].pool = p;
    p->args[t].idx = t + 1;
    if (pthread_create(&p->th[t], NULL, fwd_pool_worker, &p->args[t])) break;
    p->workers++;
  }
  return p;
}

void jo_fwd_set_threads(jo_fwd_model *f, int threads) {
  if (threads < 1) threads = 1;
  if (threads > FWD_MAX_THREADS) threads = FWD_MAX_THREADS;
  fwd_pool_free(f->pool);
  f->pool = threads > 1 ? fwd_pool_new(threads) : NULL;
  f->threads = f->pool ? f->pool->workers + 1 : 1;
}

static void fwd_par(const jo_fwd_model *f, int64_t n, fwd_range_fn fn, void *ctx) {
  fwd_pool *p = f->pool;
  int parts = p ? p->workers + 1 : 1;
  if (parts > n) parts = (int)n;
  if (parts <= 1) {
    fn(ctx, 0, n);
    return;
  }
  p->fn = fn, p->ctx = ctx, p->n = n, p->parts = parts;
  __atomic_store_n(&p->remaining, p->workers, __ATOMIC_RELAXED);
  __atomic_add_fetch(&p->gen, 1, __ATOMIC_RELEASE);
  int64_t lo, hi;
  fwd_range_of(n, parts, 0, &lo, &hi);
  fn(ctx, lo, hi);
  while (__atomic_load_n(&p->remaining, __ATOMIC_ACQUIRE) != 0) {
  }
}

typedef struct {
  const int8_t *x, *w;
  int64_t m, n, k;
  int32_t *out;
} fwd_gemm_ctx;

/* out[i][j] = sum_t x[i][t] w[j][t] for weight rows j in [lo, hi). */
static void fwd_gemm_range(void *p, int64_t lo, int64_t hi) {
  const fwd_gemm_ctx *c = (const fwd_gemm_ctx *)p;
  for (int64_t j = lo; j < hi; j++) {
    const int8_t *wr = c->w + j * c->k;
    for (int64_t i = 0; i < c->m; i++) {
      const int8_t *xr = c->x + i * c->k;
      int32_t s = 0;
      for (int64_t t = 0; t < c->k; t++) s += (int32_t)xr[t] * (int32_t)wr[t];
      c->out[i * c->n + j] = s;
    }
  }
}

typedef struct {
  const int8_t *q, *kc, *vc;
  int64_t start_pos;
  int8_t *out;
} fwd_att_ctx;

static void fwd_att_range(void *p, int64_t lo, int64_t hi) {
  const fwd_att_ctx *c = (const fwd_att_ctx *)p;
  jo_fwd_attention(c->q + lo * JO_FWD_DIM, c->kc, c->vc, hi - lo, c->start_pos + lo, c->out + lo * JO_FWD_DIM);
}

static void fwd_proj(const jo_fwd_model *f, const jo_fwd_mat *w, const int8_t *x, int64_t m, int relu, int32_t *raw,
                     int8_t *out) {
  fwd_gemm_ctx c = {x, w->rows, m, w->n, w->k, raw};
  fwd_par(f, w->n, fwd_gemm_range, &c);
  fwd_requant(raw, m * w->n, w->shift, relu, out);
}

/* ForwardModel::forward (src/forward.rs:930-976): the tokens at positions start_pos.., which must
 * equal the positions already cached; logits [head rows] of the last token. */
int jo_fwd_forward(jo_fwd_model *f, const uint32_t *tokens, int64_t m, int64_t start_pos, int32_t *logits) {
  if (m < 1 || start_pos != f->len || start_pos + m > f->cap) return -1;
  const int64_t D = JO_FWD_DIM;
  int8_t *x = (int8_t *)malloc((size_t)(m * D)), *h = (int8_t *)malloc((size_t)(m * D));
  int8_t *q = (int8_t *)malloc((size_t)(m * D)), *a = (int8_t *)malloc((size_t)(m * D));
  int8_t *o = (int8_t *)malloc((size_t)(m * D)), *up = (int8_t *)malloc((size_t)(m * JO_FWD_FFN));
  int32_t *raw = (int32_t *)malloc((size_t)(m * JO_FWD_FFN) * sizeof(int32_t));
  int rc = (x && h && q && a && o && up && raw) ? 0 : -2;
  if (!rc) {
    for (int64_t r = 0; r < m; r++) jo_fwd_embed(f->seed, tokens[r], x + r * D);
    for (int l = 0; l < JO_FWD_LAYERS; l++) {
      const jo_fwd_mat *W = f->w[l];
      jo_fwd_rmsnorm(x, m, h);
      fwd_proj(f, &W[0], h, m, 0, raw, q);
      fwd_proj(f, &W[1], h, m, 0, raw, f->kc[l] + start_pos * D);
      fwd_proj(f, &W[2], h, m, 0, raw, f->vc[l] + start_pos * D);
      fwd_att_ctx ac = {q, f->kc[l], f->vc[l], start_pos, a};
      fwd_par(f, m, fwd_att_range, &ac);
      fwd_proj(f, &W[3], a, m, 0, raw, o);
      fwd_sat_add(x, o, m * D);
      jo_fwd_rmsnorm(x, m, h);
      fwd_proj(f, &W[4], h, m, 1, raw, up);
      fwd_proj(f, &W[5], up, m, 0, raw, o);
      fwd_sat_add(x, o, m * D);
    }
    jo_fwd_rmsnorm(x + (m - 1) * D, 1, h);
    fwd_gemm_ctx hc = {h, f->head.rows, 1, f->head.n, D, logits};
    fwd_par(f, f->head.n, fwd_gemm_range, &hc);
    f->len = start_pos + m;
  }
  free(x), free(h), free(q), free(a), free(o), free(up), free(raw);
  return rc;
}

/* ForwardModel::sample (src/forward.rs:978-986): the first index of the largest of the first
 * vocab logits (0 when vocab <= 1). */
uint32_t jo_fwd_sample(const int32_t *logits, int64_t vocab) {
  int64_t best = 0;
  for (int64_t i = 1; i < vocab; i++)
    if (logits[i] > logits[best]) best = i;
  return (uint32_t)best;
}

/* ForwardModel::evaluate's token loop (src/forward.rs:1000-1043): a fresh cache, the prompt's
 * forward, then greedy steps until max_tokens tokens are generated. */
int jo_fwd_evaluate(jo_fwd_model *f, const uint32_t *prompt, int64_t n, int64_t max_tokens, uint32_t *generated) {
  if (n < 1 || max_tokens < 0) return -1;
  if (n + (max_tokens > 0 ? max_tokens - 1 : 0) > f->cap) return -1;
  int32_t *logits = (int32_t *)malloc((size_t)f->head.n * sizeof(int32_t));
  if (!logits) return -2;
  f->len = 0;
  int rc = jo_fwd_forward(f, prompt, n, 0, logits);
  if (!rc && max_tokens > 0) {
    uint32_t tok = jo_fwd_sample(logits, f->vocab);
    generated[0] = tok;
    for (int64_t i = 1; i < max_tokens && !rc; i++) {
      rc = jo_fwd_forward(f, &tok, 1, n + i - 1, logits);
      tok = jo_fwd_sample(logits, f->vocab);
      generated[i] = tok;
    }
  }
  free(logits);
  return rc;
}
