/*
 * hale_oracle.h -- CPU restatement of Hale-Token's quantized MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the CPU baseline that is timed beside it.  Only tests/, the
 * smoke() entry point and bench.py's cpu_baseline leg may load it; the
 * product library never links, calls or falls back to it.
 *
 * Every function restates the reference Rust code it names (file:line in the
 * Hale-Token tree) with the same arithmetic order, rounding and saturation:
 *   - no fused multiply-add anywhere (built with -ffp-contract=off),
 *   - roundf (half away from zero) == Rust f32::round,
 *   - saturating float->int casts == Rust `as i8` / `as i32` (NaN -> 0),
 *   - f32 -> f16 round-to-nearest-even == half 2.7.1 f16::from_f32,
 *   - expf is glibc's, which is what Rust's f32::exp calls on Linux.
 *
 * Parity pins (what checks each function against something other than
 * itself) are listed per function in tests/test_oracle.py.  Functions with no
 * such check would be marked "parity unpinned" here; at present the only
 * unpinned behaviour is NaN payload handling in f32->f16 (half's software
 * fallback vs F16C) and Iterator::sum's neutral element for an all -0.0
 * sum, neither reachable with the configured input distributions.
 */
#ifndef HALE_ORACLE_H
#define HALE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType discriminants, same order as src/tensor/dtype.rs:15-25. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_Q8_0 = 3, ORC_Q4_0 = 4 };
#define ORC_QK 32 /* src/tensor/dtype.rs:28 */

/* ---- block geometry: src/tensor/dtype.rs:32-61 ---- */
size_t orc_block_len(int dtype);
size_t orc_block_bytes(int dtype);
/* Returns -1 when cols is not a multiple of the block length. */
long long orc_row_bytes(int dtype, size_t cols);

/* ---- scalar conversions ---- */
uint16_t orc_f32_to_f16(float v);   /* half::f16::from_f32 (RNE)          */
float orc_f16_to_f32(uint16_t h);   /* half::f16::to_f32 (exact)          */
uint16_t orc_f32_to_bf16(float v);  /* half::bf16::from_f32 (RNE)         */
/* orc_f32_to_f16 over bit patterns lo .. lo+n-1 (exhaustive tests) */
void orc_f32_to_f16_range(uint32_t lo, size_t n, uint16_t *out);
int8_t orc_sat_i8(float v);         /* Rust `v as i8`                      */
int32_t orc_sat_i32(float v);       /* Rust `v as i32`                     */
float orc_expf(float v);            /* Rust f32::exp on Linux = glibc expf */

/* ---- encode / decode: src/tensor/quant.rs:236-321 ---- */
void orc_encode_row(int dtype, const float *values, size_t n, uint8_t *out);
void orc_decode_row(int dtype, const uint8_t *row, float *out, size_t n);

/* ---- activations: src/tensor/quant.rs:77-93 ---- */
void orc_q8_quantize(const float *x, size_t n, float *scales, int8_t *quants);

/* ---- dot products: src/tensor/quant.rs:59-66,107-144,152-194 ---- */
float orc_dot_q8_0(const uint8_t *row, size_t nb, const float *xs,
                   const int8_t *xq, int32_t *isums);
float orc_dot_q4_0(const uint8_t *row, size_t nb, const float *xs,
                   const int8_t *xq, int32_t *isums);
float orc_dot_f32(const float *w, const float *x, size_t n);
float orc_dot(int dtype, const uint8_t *row, const float *x, size_t n);

/* ---- matvec: src/tensor/matrix.rs:115-143 ----
 * nthreads <= 1 runs the serial loop (matvec_serial); otherwise rows are
 * split into 32-row tasks over nthreads threads (matvec).  Returns 0, or -1
 * on a shape error (the reference panics).  isums, when non-NULL, receives
 * the per-block i32 sums [rows][cols/32] of a quantized matrix. */
int orc_matvec(int dtype, size_t rows, size_t cols, const uint8_t *data,
               const float *x, float *out, int nthreads);
int orc_matvec_block_sums(int dtype, size_t rows, size_t cols,
                          const uint8_t *data, const float *x, int32_t *isums);

/* ---- ops: src/ops/activation.rs:5-32, src/ops/topk.rs:27-61 ---- */
float orc_silu(float x);
void orc_softmax_in_place(float *x, size_t n);
size_t orc_argmax(const float *x, size_t n);
size_t orc_top_k(const float *scores, size_t n, size_t k, uint32_t *index,
                 float *score);

/* ---- expert and MoE layer: src/expert/mod.rs:91-103, src/model/moe.rs ---- */
void orc_expert_forward(int dtype, size_t hidden, size_t inter,
                        const uint8_t *gate, const uint8_t *up,
                        const uint8_t *down, const float *x, float *out,
                        int nthreads);

typedef struct {
  int dtype;            /* expert weight dtype (Q8_0 or Q4_0)            */
  size_t hidden;        /* H                                              */
  size_t inter;         /* I                                              */
  size_t num_experts;   /* E                                              */
  size_t top_k;         /* experts_per_token                              */
  int normalize_topk;   /* MoeLayer::normalize_topk                       */
  const float *router;  /* [E][H] f32, or NULL when logits are supplied  */
  const uint8_t *const *gate; /* E pointers, each [I][H] encoded          */
  const uint8_t *const *up;   /* E pointers, each [I][H] encoded          */
  const uint8_t *const *down; /* E pointers, each [H][I] encoded          */
} orc_moe_layer;

/* MoeLayer::route (src/model/moe.rs:36-53).  `logits` may be NULL, in which
 * case the router matvec computes them; otherwise they are used as given
 * (the router matvec output).  Returns the number of routes written. */
size_t orc_moe_route(const orc_moe_layer *layer, const float *x,
                     const float *logits, uint32_t *index, float *weight);
/* MoeLayer::forward (src/model/moe.rs:56-70) for one token. */
int orc_moe_forward(const orc_moe_layer *layer, const float *x,
                    const float *logits, float *out, uint32_t *index,
                    float *weight, int nthreads);
/* Prefill: Transformer::prefill feeds tokens one at a time
 * (src/model/transformer.rs:231-239), so at the MoE layer token t's output
 * is MoeLayer::forward(x_t).  x and out are [T][H]; logits [T][E] or NULL;
 * index/weight [T][top_k]. */
int orc_moe_prefill(const orc_moe_layer *layer, size_t tokens,
                    const float *x, const float *logits, float *out,
                    uint32_t *index, float *weight, int nthreads);

/* ---- around the MoE block: src/ops/norm.rs, src/ops/rope.rs,
 * src/model/attention.rs ---- */
/* rms_norm (norm.rs:7-14): out[i] = x[i] * scale * w[i] with
 * scale = 1 / sqrt(sum(x^2) / n + eps), the sum taken in order. */
void orc_rms_norm(const float *x, const float *w, size_t n, float eps, float *out);
/* rms_norm_in_place (norm.rs:17-23): x[i] = x[i] * (scale * w[i]). */
void orc_rms_norm_in_place(float *x, const float *w, size_t n, float eps);
/* Rope::apply (rope.rs:36-44): rotate-half over one head of hd values. */
void orc_rope_apply(float *head, size_t hd, const float *cos, const float *sin);

typedef struct {
  int dtype;               /* dtype of the four projections             */
  size_t hidden;           /* H                                          */
  size_t num_heads;        /* query heads                                */
  size_t num_kv_heads;     /* key/value heads (GQA)                      */
  size_t head_dim;         /* hd (even)                                  */
  float norm_eps;          /* eps of the per-head QK-norm                */
  const uint8_t *q_proj;   /* [num_heads*hd][H] encoded rows             */
  const uint8_t *k_proj;   /* [num_kv_heads*hd][H]                       */
  const uint8_t *v_proj;   /* [num_kv_heads*hd][H]                       */
  const uint8_t *o_proj;   /* [H][num_heads*hd]                          */
  const float *q_norm;     /* [hd] QK-norm weights, or NULL              */
  const float *k_norm;     /* [hd], or NULL                              */
} orc_attention;

/* Attention::forward (attention.rs:31-86) for the token at `position`.
 * keys / values are the layer's cache, [position + 1][kv_dim] f32: rows
 * 0 .. position-1 hold earlier tokens, row `position` receives this token's
 * key (after QK-norm and RoPE) and value.  cos / sin: [hd/2]. */
void orc_attention_forward(const orc_attention *a, const float *x, size_t position,
                           const float *cos, const float *sin, float *keys,
                           float *values, float *out);

/* ---- seeded synthetic inputs ----
 * xorshift64* as in src/generate/sampler.rs:128-146 (shifts 12/25/27,
 * multiplier 0x2545F4914F6CDD1D, seed max(1)); normals by Box-Muller in
 * f64, rounded to f32.  `values` is the xorshift32 helper of the quant.rs
 * unit tests (src/tensor/quant.rs:328-338). */
uint64_t orc_xorshift64star(uint64_t *state);
void orc_fill_normal(uint64_t seed, float mean, float std, float *out,
                     size_t n);
void orc_test_values(size_t n, uint32_t seed, float *out);

/* Encodes `experts` SwiGLU experts with N(0, std^2) weights drawn from
 * seed, expert e using seed + e.  gate/up/down are [E][rows*row_bytes]. */
void orc_make_experts(int dtype, size_t hidden, size_t inter, size_t experts,
                      uint64_t seed, float std, uint8_t *gate, uint8_t *up,
                      uint8_t *down, int nthreads);

/* Number of host threads OpenMP would use by default. */
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
