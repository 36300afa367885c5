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
  // 32 key values per batch in two alternating register sets: the loads of
  // batch b + 1 are in flight while batch b is added (hd is a multiple of 16)
  const int nb = hd / 32;
  f32x4 A[8], B[8];
  auto ld8 = [&](f32x4* d, int b) {
#pragma unroll
    for (int u = 0; u < 8; u++) d[u] = key[8 * b + u];
  };
  auto add8 = [&](const f32x4* d, int b) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int j = 32 * b + 4 * u;
      s = s + qh[j] * d[u].x;
      s = s + qh[j + 1] * d[u].y;
      s = s + qh[j + 2] * d[u].z;
      s = s + qh[j + 3] * d[u].w;
    }
  };
  if (nb > 0) ld8(A, 0);
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    ld8(B, b + 1);
    add8(A, b);
    if (b + 2 < nb) ld8(A, b + 2);
    add8(B, b + 1);
  }
  if (b < nb) add8(A, b);
  for (int j = 32 * nb; j < hd; j += 4) {  // a 16-value remainder
    const f32x4 kv = key[j / 4];
    s = s + qh[j] * kv.x;
    s = s + qh[j + 1] * kv.y;
    s = s + qh[j + 2] * kv.z;
    s = s + qh[j + 3] * kv.w;
  }
  scores[(size_t)h * ld + t] = s * scale;
}

// softmax_in_place over each head's scores (one work-group per head): the
// max in any order, the exponentials in parallel, their sum in order by one
// thread (through LDS in chunks, several reads in flight), then one division
// per score.  The probabilities replace the scores.
constexpr int SM_CHUNK = 12288;  // exponentials per LDS chunk (48 KB)

__global__ __launch_bounds__(256) void k_attn_softmax(float* __restrict__ scores, int seq, int ld) {
  __shared__ __attribute__((aligned(16))) float buf[SM_CHUNK];
  __shared__ float red[4];
  __shared__ float bcast[1];
  float* sc = scores + (size_t)blockIdx.x * ld;
  const int tid = threadIdx.x;
  // max: fold(-inf, f32::max); order-free (a NaN is skipped either way)
  // up to SM_CHUNK scores stay in LDS from the first read to the division
  const bool resident = seq <= SM_CHUNK;
  float m = -INFINITY;
  for (int t = tid; t < seq; t += 256) {
    const float v = sc[t];
    m = fmaxf(m, v);
    if (resident) buf[t] = v;
  }
  m = wave_max_f32(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (resident) {
    for (int t = tid; t < seq; t += 256) buf[t] = hale_expf(buf[t] - m);
    __syncthreads();
    if (tid == 0) bcast[0] = lds_sum_in_order(buf, seq, 0.0f);
    __syncthreads();
    const float sum = bcast[0];
    for (int t = tid; t < seq; t += 256) sc[t] = buf[t] / sum;
    return;
  }
  float sum = 0.0f;  // sum += v from 0.0, carried by thread 0
  for (int c0 = 0; c0 < seq; c0 += SM_CHUNK) {
    const int n = min(SM_CHUNK, seq - c0);
    for (int t = tid; t < n; t += 256) {
      const float e = hale_expf(sc[c0 + t] - m);
      sc[c0 + t] = e;
      buf[t] = e;
    }
    __syncthreads();
    if (tid == 0) sum = lds_sum_in_order(buf, n, sum);
    __syncthreads();
  }
  if (tid == 0) bcast[0] = sum;
  __syncthreads();
  sum = bcast[0];
  for (int t = tid; t < seq; t += 256) sc[t] = sc[t] / sum;
}

// The context ctx[h][c] = 0 + p_0 v_0[c] + p_1 v_1[c] + ... in position
// order.  A work-group takes one key/value head and 16 of its columns for
// every query head of its group (thread (query head, column) < group x 16
// folds one chain; all 256 threads load), so each value is read once.  Values and
// probabilities stream through two LDS tiles of T positions, staged through
// registers: tile i + 1 loads while the chains add tile i.
constexpr int CTX_COLS = 16;
constexpr int CTX_LDS = 6144;  // floats per tile (values T x 16 + probabilities group x T)

__global__ __launch_bounds__(256) void k_attn_ctx(const float* __restrict__ probs,
                                                  const float* __restrict__ values, int hd,
                                                  int kv_dim, int group, int seq, int ld,
                                                  float* __restrict__ ctx) {
  __shared__ __attribute__((aligned(16))) float tile[2][CTX_LDS];
  const int g = blockIdx.x;                 // key/value head
  const int c0 = blockIdx.y * CTX_COLS;     // first column
  constexpr int nthr = 256;
  const int tid = threadIdx.x;
  const bool chain = tid < group * CTX_COLS;
  const int hq = tid / CTX_COLS, c = tid % CTX_COLS;
  // positions per tile: a multiple of 4 with T * 16 + group * (T + 4) <=
  // CTX_LDS; probability rows are T + 4 floats apart, so the query heads of
  // a wave read distinct banks
  const int T = (CTX_LDS - 4 * group) / (CTX_COLS + group) / 4 * 4;
  const int PP = T + 4;                     // probability row pitch
  const int nv4 = T * (CTX_COLS / 4);       // float4 of values per tile
  const int np4 = group * (T / 4);          // float4 of probabilities per tile
  const int ntiles = (seq + T - 1) / T;
  constexpr int MAXL = CTX_LDS / 4 / nthr;  // float4 loads per thread
  const float* vbase = values + (size_t)g * hd + c0;
  const float* pbase = probs + (size_t)g * group * ld;
  // NST register stages: tiles ti + 2 .. ti + NST are in flight while tile
  // ti is added from LDS and tile ti + 1 waits in the other LDS buffer
  constexpr int NST = 4;
  f32x4 r[NST][MAXL];
  auto load = [&](f32x4* R, int ti) {
    if (ti >= ntiles) return;
    const int t0 = ti * T, n = min(T, seq - t0);
#pragma unroll
    for (int j = 0; j < MAXL; j++) {
      const int i = tid + nthr * j;
      if (i < nv4) {
        const int t = i / (CTX_COLS / 4), q = i % (CTX_COLS / 4);
        if (t < n) R[j] = *(const f32x4*)(vbase + (size_t)(t0 + t) * kv_dim + 4 * q);
      } else if (i < nv4 + np4) {
        const int k = i - nv4, hh = k / (T / 4), t = 4 * (k % (T / 4));
        if (t < n) R[j] = *(const f32x4*)(pbase + (size_t)hh * ld + t0 + t);
      }
    }
  };
  auto store = [&](const f32x4* R, int b) {
#pragma unroll
    for (int j = 0; j < MAXL; j++) {
      const int i = tid + nthr * j;
      if (i < nv4) {
        *(f32x4*)&tile[b][4 * i] = R[j];
      } else if (i < nv4 + np4) {
        const int k = i - nv4, hh = k / (T / 4), t = 4 * (k % (T / 4));
        *(f32x4*)&tile[b][T * CTX_COLS + hh * PP + t] = R[j];
      }
    }
  };
  float acc = 0.0f;
  auto fold = [&](int ti) {
    const int n = min(T, seq - ti * T);
    const float* vt = tile[ti & 1];
    const float* pt = tile[ti & 1] + T * CTX_COLS + hq * PP;
    // products of FB positions at a time in two alternating register sets:
    // batch k + 1's LDS reads are in flight while batch k is added (FB adds
    // overlap the next batch's reads)
    constexpr int FB = 8;
    float PA[FB], PB[FB];
    auto prod = [&](float* d, int t) {
#pragma unroll
      for (int u = 0; u < FB; u++) d[u] = pt[t + u] * vt[(t + u) * CTX_COLS + c];
    };
    auto add = [&](const float* d) {
#pragma unroll
      for (int u = 0; u < FB; u++) acc = acc + d[u];
    };
    const int nbk = n / FB;
    if (nbk > 0) prod(PA, 0);
    int k = 0;
    for (; k + 1 < nbk; k += 2) {
      prod(PB, FB * (k + 1));
      add(PA);
      if (k + 2 < nbk) prod(PA, FB * (k + 2));
      add(PB);
    }
    if (k < nbk) add(PA);
    for (int t = FB * nbk; t < n; t++) acc = acc + pt[t] * vt[t * CTX_COLS + c];
  };
#pragma unroll
  for (int j = 0; j < NST; j++) load(r[j], j);
  if (ntiles > 0) store(r[0], 0);
  __syncthreads();
  for (int ti0 = 0; ti0 < ntiles; ti0 += NST) {
#pragma unroll
    for (int j = 0; j < NST; j++) {
      const int ti = ti0 + j;  // stage j holds tile ti (stored), stage j + 1 tile ti + 1
      if (ti < ntiles) {
        if (chain) fold(ti);
        if (ti + 1 < ntiles) store(r[(j + 1) % NST], (ti + 1) & 1);
        load(r[(j + 1) % NST], ti + 1 + NST);  // the stage just stored takes tile ti + 1 + NST
        __syncthreads();
      }
    }
  }
  if (chain) ctx[(size_t)(g * group + hq) * hd + c0 + c] = acc;
}

hipError_t launch_rms_norm(float* x, const float* delta, const float* w, size_t rows, size_t n,
                           float eps, float* out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (n == 0 || n > (size_t)NORM_MAX || rows > 0x7fffffffu) return hipErrorInvalidValue;
  return launch(k_rms_norm, (unsigned)rows, 256, 0, st, x, delta, w, (int)n, eps, out);
}

hipError_t launch_attention_core(const AttnArgs& a, hipStream_t st) {
  // head_dim a multiple of 16 (context column blocks), GQA group <= 16
  // (work-groups of group x 16 threads), score rows 16-byte aligned
  if (a.hd < 16 || a.hd > HEAD_MAX || a.hd % CTX_COLS || a.nh < 1 || a.nkv < 1 || a.nh % a.nkv ||
      a.nh / a.nkv > 16 || a.seq < 1 || a.seq > a.ld || a.ld % 4)
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
  e = launch(k_attn_softmax, (unsigned)a.nh, 256, 0, st, a.scores, a.seq, a.ld);
  if (e != hipSuccess) return e;
  dim3 gc((unsigned)a.nkv, (unsigned)(a.hd / CTX_COLS));
  return launch(k_attn_ctx, gc, 256, 0, st, (const float*)a.scores,
                (const float*)a.values, a.hd, kv_dim, a.nh / a.nkv, a.seq, a.ld, a.ctx);
}

}  // namespace hale
