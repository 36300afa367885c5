// kernels_attn.hip -- the steps on either side of the MoE block on gfx950:
// RMSNorm (src/ops/norm.rs) and one-token grouped-query attention with
// QK-norm, RoPE and a KV cache (src/model/attention.rs, src/ops/rope.rs,
// src/model/kv_cache.rs).
//
// Every sum keeps the reference's order, so every result is bit-identical:
//   - RMSNorm's sum of squares runs in order from -0.0 (Iterator::sum), then
//     1 / sqrt(sum / n + eps), then x * scale * w (rms_norm) or
//     x * (scale * w) (rms_norm_in_place);
//   - a score is the in-order sum q[0]k[0] + q[1]k[1] + ... from -0.0,
//     times 1 / sqrt(hd); softmax is softmax_in_place (max, glibc exp, an
//     in-order sum from 0.0, one division per score);
//   - a context element is 0 + p_0 v_0 + p_1 v_1 + ... in position order.
// The products and the exponentials are computed in parallel; each
// sequential sum runs in one lane.
#pragma clang fp contract(off)

#include "hale_device.h"
#include "kernels.h"

namespace hale {

constexpr int NORM_MAX = 8192;     // elements one RMSNorm work-group holds in LDS
constexpr int HEAD_MAX = 1024;     // largest head_dim
constexpr int PCHUNK = 1024;       // probabilities staged in LDS per context pass

// inverse_rms (src/ops/norm.rs:25-28) of n values whose squares are in
// sq[0, n) of LDS; every thread gets the scale.
__device__ __forceinline__ float block_inverse_rms(const float* sq, int n, float eps, float* bcast) {
  if (threadIdx.x == 0) {
    const float s = lds_sum_in_order(sq, n, -0.0f);
    bcast[0] = 1.0f / sqrtf(s / (float)n + eps);
  }
  __syncthreads();
  return bcast[0];
}

// One work-group per row: out = rms_norm(x + delta, w) with x updated to
// x + delta first when delta is given (add_in_place, then rms_norm).
// (out may be x itself: each thread reads an element before writing it.)
__global__ __launch_bounds__(256) void k_rms_norm(float* x, const float* __restrict__ delta,
                                                  const float* __restrict__ w, int n, float eps,
                                                  float* out) {
  __shared__ __attribute__((aligned(16))) float sq[NORM_MAX];
  __shared__ float bcast[1];
  float* xr = x + (size_t)blockIdx.x * n;
  const float* dr = delta ? delta + (size_t)blockIdx.x * n : nullptr;
  float* orow = out + (size_t)blockIdx.x * n;
  for (int i = threadIdx.x; i < n; i += 256) {
    float v = xr[i];
    if (dr) {
      v = v + dr[i];
      xr[i] = v;
    }
    sq[i] = v * v;
  }
  __syncthreads();
  const float scale = block_inverse_rms(sq, n, eps, bcast);
  for (int i = threadIdx.x; i < n; i += 256) orow[i] = xr[i] * scale * w[i];
}

// QK-norm and RoPE of every query and key head, then the cache push.
// Work-group h < nh: query head h (in place in q).  nh <= h < nh + nkv: key
// head h - nh, written to keys[pos]; the same work-group copies value head
// h - nh to values[pos].
__global__ __launch_bounds__(64) void k_qk_norm_rope(float* __restrict__ q, const float* __restrict__ k,
                                                     const float* __restrict__ v, int nh, int hd,
                                                     const float* __restrict__ q_norm,
                                                     const float* __restrict__ k_norm, float eps,
                                                     const float* __restrict__ cos,
                                                     const float* __restrict__ sin,
                                                     float* __restrict__ keys_pos,
                                                     float* __restrict__ values_pos) {
  __shared__ __attribute__((aligned(16))) float head[HEAD_MAX];
  __shared__ __attribute__((aligned(16))) float sq[HEAD_MAX];
  __shared__ float bcast[1];
  const int hb = blockIdx.x;
  const bool is_q = hb < nh;
  const int h = is_q ? hb : hb - nh;
  const float* src = is_q ? q + (size_t)h * hd : k + (size_t)h * hd;
  float* dst = is_q ? q + (size_t)h * hd : keys_pos + (size_t)h * hd;
  const float* wn = is_q ? q_norm : k_norm;
  for (int i = threadIdx.x; i < hd; i += 64) {
    const float a = src[i];
    head[i] = a;
    sq[i] = a * a;
  }
  if (!is_q)
    for (int i = threadIdx.x; i < hd; i += 64) values_pos[(size_t)h * hd + i] = v[(size_t)h * hd + i];
  __syncthreads();
  if (wn) {  // rms_norm_in_place: x = x * (scale * w)
    const float scale = block_inverse_rms(sq, hd, eps, bcast);
    for (int i = threadIdx.x; i < hd; i += 64) head[i] = head[i] * (scale * wn[i]);
    __syncthreads();
  }
  const int half = hd / 2;  // Rope::apply (src/ops/rope.rs:36-44)
  for (int i = threadIdx.x; i < half; i += 64) {
    const float a = head[i], b = head[half + i];
    dst[i] = a * cos[i] - b * sin[i];
    dst[half + i] = b * cos[i] + a * sin[i];
  }
}

// scores[h][t] = (q_h . key_t) * scale for t < seq, one thread per t.
__global__ __launch_bounds__(256) void k_attn_scores(const float* __restrict__ q,
                                                     const float* __restrict__ keys, int hd,
                                                     int kv_dim, int group, int seq, int ld,
                                                     float scale, float* __restrict__ scores) {
  __shared__ __attribute__((aligned(16))) float qh[HEAD_MAX];
  const int h = blockIdx.y;
  const int kvo = (h / group) * hd;
  for (int i = threadIdx.x; i < hd; i += 256) qh[i] = q[(size_t)h * hd + i];
  __syncthreads();
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= seq) return;
  const f32x4* key = (const f32x4*)(keys + (size_t)t * kv_dim + kvo);
  float s = -0.0f;  // Iterator::sum
  for (int j = 0; j < hd / 4; j++) {
    const f32x4 kv = key[j];
    s = s + qh[4 * j] * kv.x;
    s = s + qh[4 * j + 1] * kv.y;
    s = s + qh[4 * j + 2] * kv.z;
    s = s + qh[4 * j + 3] * kv.w;
  }
  scores[(size_t)h * ld + t] = s * scale;
}

// softmax_in_place over the head's scores, then the context
// ctx[c] = 0 + p_0 v_0[c] + p_1 v_1[c] + ... (one thread per c).
__global__ __launch_bounds__(256) void k_attn_softmax_ctx(float* __restrict__ scores,
                                                          const float* __restrict__ values, int hd,
                                                          int kv_dim, int group, int seq, int ld,
                                                          float* __restrict__ ctx) {
  __shared__ __attribute__((aligned(16))) float pbuf[PCHUNK];
  __shared__ float red[4];
  __shared__ float bcast[1];
  const int h = blockIdx.x;
  const int kvo = (h / group) * hd;
  float* sc = scores + (size_t)h * ld;
  const int tid = threadIdx.x;
  // max: fold(-inf, f32::max); order-free (a NaN is skipped either way)
  float m = -INFINITY;
  for (int t = tid; t < seq; t += 256) m = fmaxf(m, sc[t]);
  m = wave_max_f32(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  for (int t = tid; t < seq; t += 256) sc[t] = hale_expf(sc[t] - m);
  __syncthreads();
  if (tid == 0) {  // sum += v, in order from 0.0
    float sum = 0.0f;
    for (int t = 0; t < seq; t++) sum = sum + sc[t];
    bcast[0] = sum;
  }
  __syncthreads();
  const float sum = bcast[0];
  for (int t = tid; t < seq; t += 256) sc[t] = sc[t] / sum;
  __syncthreads();
  // context, PCHUNK probabilities at a time through LDS
  float acc[HEAD_MAX / 256];
#pragma unroll
  for (int i = 0; i < HEAD_MAX / 256; i++) acc[i] = 0.0f;
  for (int t0 = 0; t0 < seq; t0 += PCHUNK) {
    const int n = min(PCHUNK, seq - t0);
    for (int t = tid; t < n; t += 256) pbuf[t] = sc[t0 + t];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < HEAD_MAX / 256; i++) {
      const int c = tid + 256 * i;
      if (c < hd) {
        const float* vc = values + (size_t)t0 * kv_dim + kvo + c;
        float a = acc[i];
        for (int t = 0; t < n; t++) a = a + pbuf[t] * vc[(size_t)t * kv_dim];
        acc[i] = a;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < HEAD_MAX / 256; i++) {
    const int c = tid + 256 * i;
    if (c < hd) ctx[(size_t)h * hd + c] = acc[i];
  }
}

hipError_t launch_rms_norm(float* x, const float* delta, const float* w, size_t rows, size_t n,
                           float eps, float* out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (n == 0 || n > (size_t)NORM_MAX || rows > 0x7fffffffu) return hipErrorInvalidValue;
  return launch(k_rms_norm, (unsigned)rows, 256, 0, st, x, delta, w, (int)n, eps, out);
}

hipError_t launch_attention_core(const AttnArgs& a, hipStream_t st) {
  if (a.hd < 4 || a.hd > HEAD_MAX || a.hd % 4 || a.nh < 1 || a.nkv < 1 || a.nh % a.nkv || a.seq < 1 ||
      a.seq > a.ld)
    return hipErrorInvalidValue;
  const int kv_dim = a.nkv * a.hd;
  hipError_t e = launch(k_qk_norm_rope, (unsigned)(a.nh + a.nkv), 64, 0, st, a.q, a.k, a.v, a.nh, a.hd,
                        a.q_norm, a.k_norm, a.eps, a.cos, a.sin, a.keys + (size_t)(a.seq - 1) * kv_dim,
                        a.values + (size_t)(a.seq - 1) * kv_dim);
  if (e != hipSuccess) return e;
  const float scale = 1.0f / sqrtf((float)a.hd);
  dim3 gs((unsigned)((a.seq + 255) / 256), (unsigned)a.nh);
  e = launch(k_attn_scores, gs, 256, 0, st, (const float*)a.q, (const float*)a.keys, a.hd, kv_dim,
             a.nh / a.nkv, a.seq, a.ld, scale, a.scores);
  if (e != hipSuccess) return e;
  return launch(k_attn_softmax_ctx, (unsigned)a.nh, 256, 0, st, a.scores, (const float*)a.values, a.hd,
                kv_dim, a.nh / a.nkv, a.seq, a.ld, a.ctx);
}

}  // namespace hale
