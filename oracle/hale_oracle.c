/*
 * hale_oracle.c -- CPU restatement of Hale-Token's quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and timed CPU baseline); see the
 * header for who may load it.  Build: oracle/Makefile, which compiles with
 * -O3 -ffp-contract=off -fno-fast-math so that, as in Rust, no multiply-add is
 * ever fused and no floating-point expression is reassociated.
 *
 * Reference citations are Hale-Token paths (file:line).
 */
#include "hale_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ------------------------------------------------------------------------ */
/* Block geometry: src/tensor/dtype.rs:32-61                                */
/* ------------------------------------------------------------------------ */

size_t orc_block_len(int dtype) {
  return (dtype == ORC_Q8_0 || dtype == ORC_Q4_0) ? ORC_QK : 1;
}

size_t orc_block_bytes(int dtype) {
  switch (dtype) {
  case ORC_F32: return 4;
  case ORC_F16:
  case ORC_BF16: return 2;
  case ORC_Q8_0: return 2 + ORC_QK;
  case ORC_Q4_0: return 2 + ORC_QK / 2;
  default: return 0;
  }
}

long long orc_row_bytes(int dtype, size_t cols) {
  size_t bl = orc_block_len(dtype);
  if (orc_block_bytes(dtype) == 0 || cols % bl != 0) return -1;
  return (long long)(cols / bl * orc_block_bytes(dtype));
}

/* ------------------------------------------------------------------------ */
/* Scalar conversions                                                       */
/* ------------------------------------------------------------------------ */

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even, subnormals
 * kept, overflow to infinity.  This is the rounding half 2.7.1's
 * f16::from_f32 performs (src/tensor/quant.rs:299,316); NaN keeps its sign and
 * top payload bits with the quiet bit set. */
uint16_t orc_f32_to_f16(float v) {
  uint32_t x = f2u(v);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) {
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13));
  }
  int e = (int)exp - 127; /* unbiased exponent of v */
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    /* normal half: keep 10 mantissa bits, round the 13 dropped ones */
    uint32_t q = ((uint32_t)(e + 15) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry to inf */
    return (uint16_t)(sign | q);
  }
  /* f32 zeros and subnormals (< 2^-126) are far below half's smallest
   * subnormal (2^-24) and round to a signed zero. */
  if (exp == 0) return (uint16_t)sign;
  /* subnormal half: value = m * 2^(e-23) in units of 2^-24 is m >> -(e+1) */
  uint32_t m = man | 0x800000u;
  int s = -(e + 1); /* 14 .. */
  if (s > 24) return (uint16_t)sign; /* below 2^-25: rounds to zero */
  uint32_t q = m >> s;
  uint32_t rem = m & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

void orc_f32_to_f16_range(uint32_t lo, size_t n, uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < (long long)n; i++) out[i] = orc_f32_to_f16(u2f(lo + (uint32_t)i));
}

/* binary16 -> binary32 is exact (half::f16::to_f32, src/tensor/quant.rs:44-46). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t m = (uint32_t)h & 0x3ffu;
  if (e == 0) {
    float mag = (float)m * 0x1p-24f; /* exact: m < 2^10 */
    return u2f(f2u(mag) | sign);
  }
  if (e == 31) /* inf, or a NaN: payload kept, quiet bit set (F16C, fcvtl, half's fallback) */
    return u2f(sign | 0x7f800000u | (m ? 0x400000u : 0u) | (m << 13));
  return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* binary32 -> bfloat16, round to nearest even (half::bf16::from_f32). */
uint16_t orc_f32_to_bf16(float v) {
  uint32_t x = f2u(v);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  uint32_t q = x >> 16;
  uint32_t rem = x & 0xffffu;
  if (rem > 0x8000u || (rem == 0x8000u && (q & 1u))) q++;
  return (uint16_t)q;
}

/* Rust `as` casts from f32 saturate and send NaN to 0. */
int8_t orc_sat_i8(float v) {
  if (isnan(v)) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int8_t)v; /* truncation toward zero, in range */
}

int32_t orc_sat_i32(float v) {
  if (isnan(v)) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v <= -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

/* f32::exp compiles to a call of libm's expf on x86_64 Linux. */
float orc_expf(float v) { return expf(v); }

static inline float read_f16(const uint8_t *b) {
  return orc_f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
}

/* ------------------------------------------------------------------------ */
/* Encode: src/tensor/quant.rs:274-321                                      */
/* ------------------------------------------------------------------------ */

/* encode_block_q8_0, src/tensor/quant.rs:295-305 */
static void encode_block_q8_0(const float *block, uint8_t *out) {
  float amax = 0.0f;
  for (int j = 0; j < ORC_QK; j++) amax = fmaxf(amax, fabsf(block[j]));
  float scale = amax / 127.0f;
  float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  uint16_t h = orc_f32_to_f16(scale);
  out[0] = (uint8_t)(h & 0xff);
  out[1] = (uint8_t)(h >> 8);
  for (int j = 0; j < ORC_QK; j++) {
    float r = roundf(block[j] * inv);
    /* f32::clamp(-127, 127) leaves NaN as NaN; `as i8` then maps it to 0 */
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    out[2 + j] = (uint8_t)orc_sat_i8(r);
  }
}

/* encode_block_q4_0, src/tensor/quant.rs:309-321 */
static void encode_block_q4_0(const float *block, uint8_t *out) {
  float extreme = 0.0f;
  for (int j = 0; j < ORC_QK; j++)
    if (fabsf(block[j]) > fabsf(extreme)) extreme = block[j];
  float scale = extreme / -8.0f;
  float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
  uint16_t h = orc_f32_to_f16(scale);
  out[0] = (uint8_t)(h & 0xff);
  out[1] = (uint8_t)(h >> 8);
  for (int j = 0; j < ORC_QK / 2; j++) {
    int32_t lo = orc_sat_i32(block[j] * inv + 8.5f);
    int32_t hi = orc_sat_i32(block[j + ORC_QK / 2] * inv + 8.5f);
    lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
    hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
    out[2 + j] = (uint8_t)(lo | (hi << 4));
  }
}

/* encode_row, src/tensor/quant.rs:274-292 */
void orc_encode_row(int dtype, const float *values, size_t n, uint8_t *out) {
  switch (dtype) {
  case ORC_F32:
    memcpy(out, values, n * 4);
    break;
  case ORC_F16:
    for (size_t i = 0; i < n; i++) {
      uint16_t h = orc_f32_to_f16(values[i]);
      out[2 * i] = (uint8_t)(h & 0xff);
      out[2 * i + 1] = (uint8_t)(h >> 8);
    }
    break;
  case ORC_BF16:
    for (size_t i = 0; i < n; i++) {
      uint16_t h = orc_f32_to_bf16(values[i]);
      out[2 * i] = (uint8_t)(h & 0xff);
      out[2 * i + 1] = (uint8_t)(h >> 8);
    }
    break;
  case ORC_Q8_0:
    for (size_t b = 0; b < n / ORC_QK; b++)
      encode_block_q8_0(values + b * ORC_QK, out + b * 34);
    break;
  case ORC_Q4_0:
    for (size_t b = 0; b < n / ORC_QK; b++)
      encode_block_q4_0(values + b * ORC_QK, out + b * 18);
    break;
  default:
    break;
  }
}

/* decode_row, src/tensor/quant.rs:236-269 */
void orc_decode_row(int dtype, const uint8_t *row, float *out, size_t n) {
  switch (dtype) {
  case ORC_F32:
    memcpy(out, row, n * 4);
    break;
  case ORC_F16:
    for (size_t i = 0; i < n; i++) out[i] = read_f16(row + 2 * i);
    break;
  case ORC_BF16:
    for (size_t i = 0; i < n; i++)
      out[i] = u2f(((uint32_t)row[2 * i + 1] << 24) | ((uint32_t)row[2 * i] << 16));
    break;
  case ORC_Q8_0:
    for (size_t b = 0; b < n / ORC_QK; b++) {
      const uint8_t *blk = row + b * 34;
      float scale = read_f16(blk);
      for (int j = 0; j < ORC_QK; j++)
        out[b * ORC_QK + j] = scale * (float)(int8_t)blk[2 + j];
    }
    break;
  case ORC_Q4_0:
    for (size_t b = 0; b < n / ORC_QK; b++) {
      const uint8_t *blk = row + b * 18;
      float scale = read_f16(blk);
      for (int j = 0; j < ORC_QK / 2; j++) {
        out[b * ORC_QK + j] = scale * ((float)(blk[2 + j] & 0x0f) - 8.0f);
        out[b * ORC_QK + j + ORC_QK / 2] = scale * ((float)(blk[2 + j] >> 4) - 8.0f);
      }
    }
    break;
  default:
    break;
  }
}

/* ------------------------------------------------------------------------ */
/* Activation quantization: Q8Activations::quantize, quant.rs:77-93         */
/* ------------------------------------------------------------------------ */

void orc_q8_quantize(const float *x, size_t n, float *scales, int8_t *quants) {
  for (size_t b = 0; b < n / ORC_QK; b++) {
    const float *blk = x + b * ORC_QK;
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK; j++) amax = fmaxf(amax, fabsf(blk[j]));
    float scale = amax / 127.0f; /* kept as f32, not rounded to f16 */
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    scales[b] = scale;
    for (int j = 0; j < ORC_QK; j++)
      quants[b * ORC_QK + j] = orc_sat_i8(roundf(blk[j] * inv)); /* no clamp */
  }
}

/* ------------------------------------------------------------------------ */
/* Dot products                                                             */
/* ------------------------------------------------------------------------ */

/* dot_q8_0, src/tensor/quant.rs:115-127:
 *   total += read_f16(block) * x_scale * isum as f32
 * Rust evaluates a*b*c as (a*b)*c, then total + that. */
float orc_dot_q8_0(const uint8_t *row, size_t nb, const float *xs,
                   const int8_t *xq, int32_t *isums) {
  float total = 0.0f;
  for (size_t b = 0; b < nb; b++) {
    const uint8_t *blk = row + b * 34;
    const int8_t *q = xq + b * ORC_QK;
    int32_t isum = 0;
    for (int j = 0; j < ORC_QK; j++) isum += (int32_t)(int8_t)blk[2 + j] * (int32_t)q[j];
    if (isums) isums[b] = isum;
    float d = read_f16(blk) * xs[b];
    float t = d * (float)isum;
    total = total + t;
  }
  return total;
}

/* dot_q4_0, src/tensor/quant.rs:129-144: byte j pairs its low nibble with
 * xq[j] and its high nibble with xq[j+16]; both are offset by 8. */
float orc_dot_q4_0(const uint8_t *row, size_t nb, const float *xs,
                   const int8_t *xq, int32_t *isums) {
  float total = 0.0f;
  for (size_t b = 0; b < nb; b++) {
    const uint8_t *blk = row + b * 18;
    const int8_t *q = xq + b * ORC_QK;
    int32_t isum = 0;
    for (int j = 0; j < ORC_QK / 2; j++) {
      int32_t lo = (int32_t)(blk[2 + j] & 0x0f) - 8;
      int32_t hi = (int32_t)(blk[2 + j] >> 4) - 8;
      isum += lo * (int32_t)q[j] + hi * (int32_t)q[j + ORC_QK / 2];
    }
    if (isums) isums[b] = isum;
    float d = read_f16(blk) * xs[b];
    float t = d * (float)isum;
    total = total + t;
  }
  return total;
}

/* reduce, src/tensor/quant.rs:37-41 */
static inline float reduce8(const float *a) {
  float s0 = (a[0] + a[4]) + (a[1] + a[5]);
  float s1 = (a[2] + a[6]) + (a[3] + a[7]);
  return s0 + s1;
}

/* dot_lanes, src/tensor/quant.rs:152-160.  The tail is an f32
 * Iterator::sum, whose fold starts at -0.0 (x + -0.0 == x for every x). */
static float dot_lanes(const float *w, const float *x, size_t n, float *acc) {
  size_t done = n / 8 * 8;
  for (size_t i = 0; i < done; i += 8)
    for (int l = 0; l < 8; l++) acc[l] = acc[l] + w[i + l] * x[i + l];
  float tail = -0.0f;
  for (size_t i = done; i < n; i++) tail = tail + w[i] * x[i];
  return tail;
}

/* dot_f32 aligned path, src/tensor/quant.rs:186-194 (the unaligned path
 * gives the same bits: quant.rs:400-420). */
float orc_dot_f32(const float *w, const float *x, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float tail = dot_lanes(w, x, n, acc);
  return reduce8(acc) + tail;
}

/* dot_decoded, src/tensor/quant.rs:166-184 (f16 / bf16 rows) */
static float dot_decoded(int dtype, const uint8_t *row, const float *x, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float tail = 0.0f;
  float buf[64];
  for (size_t c = 0; c < n; c += 64) {
    size_t len = n - c < 64 ? n - c : 64;
    orc_decode_row(dtype, row + c * 2, buf, len);
    tail = tail + dot_lanes(buf, x + c, len, acc);
  }
  return reduce8(acc) + tail;
}

/* dot, src/tensor/quant.rs:59-66 */
float orc_dot(int dtype, const uint8_t *row, const float *x, size_t n) {
  switch (dtype) {
  case ORC_F32: {
    float *w = (float *)malloc(n * 4 + 4);
    memcpy(w, row, n * 4);
    float r = orc_dot_f32(w, x, n);
    free(w);
    return r;
  }
  case ORC_F16:
  case ORC_BF16:
    return dot_decoded(dtype, row, x, n);
  case ORC_Q8_0:
  case ORC_Q4_0: {
    size_t nb = n / ORC_QK;
    float *xs = (float *)malloc(nb * 4 + 4);
    int8_t *xq = (int8_t *)malloc(n + 1);
    orc_q8_quantize(x, n, xs, xq);
    float r = dtype == ORC_Q8_0 ? orc_dot_q8_0(row, nb, xs, xq, NULL)
                                : orc_dot_q4_0(row, nb, xs, xq, NULL);
    free(xs);
    free(xq);
    return r;
  }
  default:
    return NAN;
  }
}

/* ------------------------------------------------------------------------ */
/* Matvec: src/tensor/matrix.rs:115-143                                     */
/* ------------------------------------------------------------------------ */

#define ROWS_PER_TASK 32 /* src/tensor/matrix.rs:11 */

static inline float row_dot_q(int dtype, const uint8_t *row, size_t nb,
                              const float *xs, const int8_t *xq) {
  return dtype == ORC_Q8_0 ? orc_dot_q8_0(row, nb, xs, xq, NULL)
                           : orc_dot_q4_0(row, nb, xs, xq, NULL);
}

int orc_matvec(int dtype, size_t rows, size_t cols, const uint8_t *data,
               const float *x, float *out, int nthreads) {
  long long rb = orc_row_bytes(dtype, cols);
  if (rb < 0) return -1;
  size_t row_bytes = (size_t)rb;
  if (dtype == ORC_Q8_0 || dtype == ORC_Q4_0) {
    size_t nb = cols / ORC_QK;
    float *xs = (float *)malloc(nb * 4 + 4);
    int8_t *xq = (int8_t *)malloc(cols + 1);
    orc_q8_quantize(x, cols, xs, xq); /* once per matvec, shared by every row */
    if (nthreads <= 1) {
      for (size_t r = 0; r < rows; r++)
        out[r] = row_dot_q(dtype, data + r * row_bytes, nb, xs, xq);
    } else {
      long long ntasks = (long long)((rows + ROWS_PER_TASK - 1) / ROWS_PER_TASK);
#pragma omp parallel for num_threads(nthreads) schedule(static)
      for (long long t = 0; t < ntasks; t++) {
        size_t r0 = (size_t)t * ROWS_PER_TASK;
        size_t r1 = r0 + ROWS_PER_TASK < rows ? r0 + ROWS_PER_TASK : rows;
        for (size_t r = r0; r < r1; r++)
          out[r] = row_dot_q(dtype, data + r * row_bytes, nb, xs, xq);
      }
    }
    free(xs);
    free(xq);
  } else if (dtype == ORC_F32) {
    /* rows of an aligned f32 matrix are read in place */
    const float *w = (const float *)(const void *)data;
#pragma omp parallel for num_threads(nthreads > 1 ? nthreads : 1) schedule(static)
    for (long long r = 0; r < (long long)rows; r++)
      out[r] = orc_dot_f32(w + (size_t)r * cols, x, cols);
  } else {
#pragma omp parallel for num_threads(nthreads > 1 ? nthreads : 1) schedule(static)
    for (long long r = 0; r < (long long)rows; r++)
      out[r] = orc_dot(dtype, data + (size_t)r * row_bytes, x, cols);
  }
  return 0;
}

int orc_matvec_block_sums(int dtype, size_t rows, size_t cols,
                          const uint8_t *data, const float *x, int32_t *isums) {
  long long rb = orc_row_bytes(dtype, cols);
  if (rb < 0 || (dtype != ORC_Q8_0 && dtype != ORC_Q4_0)) return -1;
  size_t nb = cols / ORC_QK;
  float *xs = (float *)malloc(nb * 4 + 4);
  int8_t *xq = (int8_t *)malloc(cols + 1);
  orc_q8_quantize(x, cols, xs, xq);
  for (size_t r = 0; r < rows; r++) {
    const uint8_t *row = data + r * (size_t)rb;
    if (dtype == ORC_Q8_0)
      orc_dot_q8_0(row, nb, xs, xq, isums + r * nb);
    else
      orc_dot_q4_0(row, nb, xs, xq, isums + r * nb);
  }
  free(xs);
  free(xq);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Ops: src/ops/activation.rs, src/ops/topk.rs                              */
/* ------------------------------------------------------------------------ */

/* silu, src/ops/activation.rs:5-7 */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* softmax_in_place, src/ops/activation.rs:11-21 */
void orc_softmax_in_place(float *x, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - max);
    sum = sum + x[i];
  }
  for (size_t i = 0; i < n; i++) x[i] = x[i] / sum;
}

/* argmax, src/ops/activation.rs:24-32 */
size_t orc_argmax(const float *x, size_t n) {
  size_t best = 0;
  for (size_t i = 0; i < n; i++)
    if (x[i] > x[best]) best = i;
  return best;
}

/* f32::total_cmp key: flip the magnitude bits of negatives. */
static inline int32_t total_key(float v) {
  int32_t b = (int32_t)f2u(v);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

/* a ranks before b: higher total_cmp score, then lower index
 * (the Worst ordering of src/ops/topk.rs:27-40). */
static inline int better(int32_t ka, size_t ia, int32_t kb, size_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

/* top_k, src/ops/topk.rs:44-61: the bounded heap keeps the k minimal
 * elements under a total order, so keeping a sorted list of the k best
 * gives the same set in the same (best-first) order. */
size_t orc_top_k(const float *scores, size_t n, size_t k, uint32_t *index,
                 float *score) {
  if (k > n) k = n;
  if (k == 0) return 0;
  size_t cnt = 0;
  int32_t *keys = (int32_t *)malloc(k * sizeof(int32_t));
  for (size_t i = 0; i < n; i++) {
    int32_t key = total_key(scores[i]);
    if (cnt == k && !better(key, i, keys[k - 1], index[k - 1])) continue;
    size_t pos = cnt < k ? cnt : k - 1;
    while (pos > 0 && better(key, i, keys[pos - 1], index[pos - 1])) {
      keys[pos] = keys[pos - 1];
      index[pos] = index[pos - 1];
      score[pos] = score[pos - 1];
      pos--;
    }
    keys[pos] = key;
    index[pos] = (uint32_t)i;
    score[pos] = scores[i];
    if (cnt < k) cnt++;
  }
  free(keys);
  return cnt;
}

/* ------------------------------------------------------------------------ */
/* Norms, RoPE and attention: src/ops/norm.rs, src/ops/rope.rs,              */
/* src/model/attention.rs                                                   */
/* ------------------------------------------------------------------------ */

/* inverse_rms, src/ops/norm.rs:25-28: the squares summed in order
 * (Iterator::sum, from -0.0), divided by n as f32, then 1 / sqrt(. + eps). */
static float inverse_rms(const float *x, size_t n, float eps) {
  float s = -0.0f;
  for (size_t i = 0; i < n; i++) s = s + x[i] * x[i];
  const float mean_sq = s / (float)n;
  return 1.0f / sqrtf(mean_sq + eps);
}

/* rms_norm, src/ops/norm.rs:7-14: `v * scale * w` associates left. */
void orc_rms_norm(const float *x, const float *w, size_t n, float eps, float *out) {
  const float scale = inverse_rms(x, n, eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

/* rms_norm_in_place, src/ops/norm.rs:17-23: `*v *= scale * w`. */
void orc_rms_norm_in_place(float *x, const float *w, size_t n, float eps) {
  const float scale = inverse_rms(x, n, eps);
  for (size_t i = 0; i < n; i++) x[i] = x[i] * (scale * w[i]);
}

/* Rope::apply, src/ops/rope.rs:36-44 */
void orc_rope_apply(float *head, size_t hd, const float *cos, const float *sin) {
  const size_t half = hd / 2;
  for (size_t i = 0; i < half; i++) {
    const float a = head[i], b = head[half + i];
    head[i] = a * cos[i] - b * sin[i];
    head[half + i] = b * cos[i] + a * sin[i];
  }
}

/* Attention::forward, src/model/attention.rs:31-86 */
void orc_attention_forward(const orc_attention *a, const float *x, size_t position,
                           const float *cos, const float *sin, float *keys,
                           float *values, float *out) {
  const size_t hd = a->head_dim, nh = a->num_heads, nkv = a->num_kv_heads;
  const size_t kv_dim = nkv * hd;
  float *q = (float *)calloc(nh * hd, 4);
  float *k = keys + position * kv_dim;   /* cache.push(&k, &v) */
  float *v = values + position * kv_dim;
  orc_matvec(a->dtype, nh * hd, a->hidden, a->q_proj, x, q, 1);
  orc_matvec(a->dtype, kv_dim, a->hidden, a->k_proj, x, k, 1);
  orc_matvec(a->dtype, kv_dim, a->hidden, a->v_proj, x, v, 1);
  for (size_t h = 0; h < nh; h++) {  /* QK-norm, then RoPE, per head */
    if (a->q_norm) orc_rms_norm_in_place(q + h * hd, a->q_norm, hd, a->norm_eps);
    orc_rope_apply(q + h * hd, hd, cos, sin);
  }
  for (size_t h = 0; h < nkv; h++) {
    if (a->k_norm) orc_rms_norm_in_place(k + h * hd, a->k_norm, hd, a->norm_eps);
    orc_rope_apply(k + h * hd, hd, cos, sin);
  }
  const size_t seq_len = position + 1;
  const size_t group = nh / nkv;
  const float scale = 1.0f / sqrtf((float)hd);
  float *context = (float *)calloc(nh * hd, 4);
  float *scores = (float *)malloc(seq_len * 4);
  for (size_t h = 0; h < nh; h++) {
    const size_t kv_offset = (h / group) * hd;
    const float *qh = q + h * hd;
    for (size_t t = 0; t < seq_len; t++) {
      const float *key = keys + t * kv_dim + kv_offset;
      float s = -0.0f;  /* Iterator::sum */
      for (size_t j = 0; j < hd; j++) s = s + qh[j] * key[j];
      scores[t] = s * scale;
    }
    orc_softmax_in_place(scores, seq_len);
    float *ctx = context + h * hd;
    for (size_t t = 0; t < seq_len; t++) {
      const float p = scores[t];
      const float *val = values + t * kv_dim + kv_offset;
      for (size_t c = 0; c < hd; c++) ctx[c] = ctx[c] + p * val[c];
    }
  }
  orc_matvec(a->dtype, a->hidden, nh * hd, a->o_proj, context, out, 1);
  free(q);
  free(context);
  free(scores);
}

/* ------------------------------------------------------------------------ */
/* Expert and MoE layer                                                     */
/* ------------------------------------------------------------------------ */

/* Expert::forward, src/expert/mod.rs:91-103: gate and up matvecs (rayon::join
 * in the reference; one parallel loop over both here, same bits), then
 * h = silu(g) * u, then down.matvec(h). */
void orc_expert_forward(int dtype, size_t hidden, size_t inter,
                        const uint8_t *gate, const uint8_t *up,
                        const uint8_t *down, const float *x, float *out,
                        int nthreads) {
  size_t hb = (size_t)orc_row_bytes(dtype, hidden);
  size_t nbh = hidden / ORC_QK;
  float *g = (float *)malloc(2 * inter * sizeof(float));
  float *u = g + inter;
  float *xs = (float *)malloc(nbh * 4 + 4);
  int8_t *xq = (int8_t *)malloc(hidden + 1);
  orc_q8_quantize(x, hidden, xs, xq);
  long long tasks = (long long)((2 * inter + ROWS_PER_TASK - 1) / ROWS_PER_TASK);
#pragma omp parallel for num_threads(nthreads > 1 ? nthreads : 1) schedule(static)
  for (long long t = 0; t < tasks; t++) {
    size_t r0 = (size_t)t * ROWS_PER_TASK;
    size_t r1 = r0 + ROWS_PER_TASK < 2 * inter ? r0 + ROWS_PER_TASK : 2 * inter;
    for (size_t r = r0; r < r1; r++) {
      const uint8_t *row = r < inter ? gate + r * hb : up + (r - inter) * hb;
      g[r] = row_dot_q(dtype, row, nbh, xs, xq); /* g[inter + i] is u[i] */
    }
  }
  for (size_t i = 0; i < inter; i++) g[i] = orc_silu(g[i]) * u[i];
  orc_matvec(dtype, hidden, inter, down, g, out, nthreads);
  free(g);
  free(xs);
  free(xq);
}

/* MoeLayer::route, src/model/moe.rs:36-53 */
size_t orc_moe_route(const orc_moe_layer *L, const float *x,
                     const float *logits, uint32_t *index, float *weight) {
  size_t E = L->num_experts;
  float *probs = (float *)malloc(E * sizeof(float));
  if (logits)
    memcpy(probs, logits, E * sizeof(float));
  else
    for (size_t e = 0; e < E; e++) probs[e] = orc_dot_f32(L->router + e * L->hidden, x, L->hidden);
  orc_softmax_in_place(probs, E);
  size_t k = orc_top_k(probs, E, L->top_k, index, weight);
  float norm = 1.0f;
  if (L->normalize_topk) {
    norm = -0.0f; /* Iterator::sum::<f32>, best-first order */
    for (size_t i = 0; i < k; i++) norm = norm + weight[i];
  }
  for (size_t i = 0; i < k; i++) weight[i] = weight[i] / norm;
  free(probs);
  return k;
}

/* MoeLayer::forward, src/model/moe.rs:56-70: out = 0, then for each route in
 * best-first order out_i = out_i + w * expert(x)_i. */
int orc_moe_forward(const orc_moe_layer *L, const float *x,
                    const float *logits, float *out, uint32_t *index,
                    float *weight, int nthreads) {
  size_t H = L->hidden;
  uint32_t *idx = index;
  float *w = weight;
  uint32_t idx_local[256];
  float w_local[256];
  if (L->top_k > 256) return -1;
  if (!idx) idx = idx_local;
  if (!w) w = w_local;
  size_t k = orc_moe_route(L, x, logits, idx, w);
  float *tmp = (float *)malloc(H * sizeof(float));
  for (size_t i = 0; i < H; i++) out[i] = 0.0f;
  for (size_t r = 0; r < k; r++) {
    size_t e = idx[r];
    orc_expert_forward(L->dtype, H, L->inter, L->gate[e], L->up[e], L->down[e],
                       x, tmp, nthreads);
    for (size_t i = 0; i < H; i++) out[i] = out[i] + w[r] * tmp[i];
  }
  free(tmp);
  return 0;
}

/* Token-at-a-time prefill, src/model/transformer.rs:231-239: token t's
 * output is MoeLayer::forward(x_t), independent of every other token, so
 * with several threads the tokens are shared among them (each token's own
 * forward then runs on one thread: the bits do not depend on threads). */
int orc_moe_prefill(const orc_moe_layer *L, size_t tokens, const float *x,
                    const float *logits, float *out, uint32_t *index,
                    float *weight, int nthreads) {
  int rc = 0;
  const int tok_par = nthreads > 1 && tokens > 1;
#pragma omp parallel for num_threads(tok_par ? nthreads : 1) schedule(dynamic, 1) reduction(|| : rc)
  for (size_t t = 0; t < tokens; t++) {
    rc = rc || orc_moe_forward(L, x + t * L->hidden,
                               logits ? logits + t * L->num_experts : NULL,
                               out + t * L->hidden,
                               index ? index + t * L->top_k : NULL,
                               weight ? weight + t * L->top_k : NULL, tok_par ? 1 : nthreads);
  }
  return rc ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* Seeded synthetic inputs                                                  */
/* ------------------------------------------------------------------------ */

/* XorShift64::next_u64, src/generate/sampler.rs:135-140 */
uint64_t orc_xorshift64star(uint64_t *s) {
  *s ^= *s >> 12;
  *s ^= *s << 25;
  *s ^= *s >> 27;
  return *s * 0x2545F4914F6CDD1DULL;
}

void orc_fill_normal(uint64_t seed, float mean, float std, float *out, size_t n) {
  uint64_t s = seed ? seed : 1; /* XorShift64::new: seed.max(1) */
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    double u1 = (double)((orc_xorshift64star(&s) >> 11) + 1) * 0x1p-53; /* (0,1] */
    double u2 = (double)(orc_xorshift64star(&s) >> 11) * 0x1p-53;       /* [0,1) */
    double rad = sqrt(-2.0 * log(u1));
    out[i] = (float)((double)mean + (double)std * rad * cos(two_pi * u2));
    if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std * rad * sin(two_pi * u2));
  }
}

/* values(n, seed), src/tensor/quant.rs:328-338 */
void orc_test_values(size_t n, uint32_t seed, float *out) {
  uint32_t s = seed * 2654435761u;
  if (s < 1) s = 1;
  for (size_t i = 0; i < n; i++) {
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    out[i] = ((float)s / (float)UINT32_MAX) * 2.0f - 1.0f;
  }
}

void orc_make_experts(int dtype, size_t hidden, size_t inter, size_t experts,
                      uint64_t seed, float std, uint8_t *gate, uint8_t *up,
                      uint8_t *down, int nthreads) {
  size_t gbytes = inter * (size_t)orc_row_bytes(dtype, hidden);
  size_t dbytes = hidden * (size_t)orc_row_bytes(dtype, inter);
  size_t hrb = (size_t)orc_row_bytes(dtype, hidden);
  size_t irb = (size_t)orc_row_bytes(dtype, inter);
#pragma omp parallel for num_threads(nthreads > 1 ? nthreads : 1) schedule(dynamic, 1)
  for (long long e = 0; e < (long long)experts; e++) {
    float *buf = (float *)malloc(hidden * inter * sizeof(float));
    uint64_t base = seed + 3 * (uint64_t)e;
    orc_fill_normal(base + 0, 0.0f, std, buf, hidden * inter);
    for (size_t r = 0; r < inter; r++)
      orc_encode_row(dtype, buf + r * hidden, hidden, gate + (size_t)e * gbytes + r * hrb);
    orc_fill_normal(base + 1, 0.0f, std, buf, hidden * inter);
    for (size_t r = 0; r < inter; r++)
      orc_encode_row(dtype, buf + r * hidden, hidden, up + (size_t)e * gbytes + r * hrb);
    orc_fill_normal(base + 2, 0.0f, std, buf, hidden * inter);
    for (size_t r = 0; r < hidden; r++)
      orc_encode_row(dtype, buf + r * inter, inter, down + (size_t)e * dbytes + r * irb);
    free(buf);
  }
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
