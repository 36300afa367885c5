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
// x + delta first when delta is given (add_in_place, then rms_norm).  The
// row and the weights are read once, all loads in flight together, and
// stay in registers through the in-order sum of the squares.  (out may be x
// itself: every element is read before any is written.)
constexpr int NORM_PER = NORM_MAX / 256;  // elements per thread

__global__ __launch_bounds__(256) void k_rms_norm(float* x, const float* __restrict__ delta,
                                                  const float* __restrict__ w, int n, float eps,
                                                  float* out) {
  __shared__ __attribute__((aligned(16))) float sq[NORM_MAX];
  __shared__ float bcast[1];
  float* xr = x + (size_t)blockIdx.x * n;
  const float* dr = delta ? delta + (size_t)blockIdx.x * n : nullptr;
  float* orow = out + (size_t)blockIdx.x * n;
  const int tid = threadIdx.x;
  float xv[NORM_PER], wv[NORM_PER];
#pragma unroll
  for (int j = 0; j < NORM_PER; j++) {
    const int i = tid + 256 * j;
    if (i < n) {
      xv[j] = xr[i];
      wv[j] = w[i];
    }
  }
  if (dr) {
#pragma unroll
    for (int j = 0; j < NORM_PER; j++) {
      const int i = tid + 256 * j;
      if (i < n) {
        xv[j] = xv[j] + dr[i];
        xr[i] = xv[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NORM_PER; j++) {
    const int i = tid + 256 * j;
    if (i < n) sq[i] = xv[j] * xv[j];
  }
  __syncthreads();
  const float scale = block_inverse_rms(sq, n, eps, bcast);
#pragma unroll
  for (int j = 0; j < NORM_PER; j++) {
    const int i = tid + 256 * j;
    if (i < n) orow[i] = xv[j] * scale * wv[j];
  }
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

// scores[h][t] = (q_h . key_t) * scale for t < seq: the dot product in
// index order from -0.0 (Iterator::sum), then one multiply.  A work-group
// takes SC_POS positions of one key/value head for up to SC_HEADS query
// heads of its group (thread (query head, position) carries one chain), so
// every key row is read once per group.  Keys and the queries stream
// through LDS in chunks of SC_W dimensions: coalesced 16-byte loads (four
// lanes per 64-byte row piece), chunk c + 1 in registers while chunk c is
// added, and each chain reads its 4 key and 4 query values per 16-byte read.
constexpr int SC_POS = 32;
constexpr int SC_HEADS = 8;
constexpr int SC_W = 16;
constexpr int SC_KP = SC_W + 4;  // key row pitch in LDS

__global__ __launch_bounds__(256) void k_attn_scores(const float* __restrict__ q,
                                                     const float* __restrict__ keys, int hd,
                                                     int kv_dim, int group, int seq, int ld,
                                                     float scale, float* __restrict__ scores) {
  __shared__ __attribute__((aligned(16))) float kt[2][SC_POS * SC_KP];
  __shared__ __attribute__((aligned(16))) float qt[2][SC_HEADS * SC_W];
  const int g = blockIdx.y;                // key/value head
  const int h0 = blockIdx.z * SC_HEADS;    // first query head within the group
  const int nhq = min(SC_HEADS, group - h0);
  // work-group x runs on XCD x % 8: give each XCD a contiguous run of
  // position blocks, so each score row is written in long runs per XCD
  const int nbx = gridDim.x;
  const int bx = nbx % 8 ? (int)blockIdx.x : (int)(blockIdx.x % 8) * (nbx / 8) + (int)blockIdx.x / 8;
  const int t0 = bx * SC_POS;
  const int tid = threadIdx.x;
  const int hq = tid / SC_POS, tp = tid % SC_POS;
  const bool chain = hq < nhq && t0 + tp < seq;
  const int nc = hd / SC_W;
  // loads of one chunk: threads 0-127 a float4 of the keys (row tid / 4,
  // part tid % 4), threads 128 .. 128 + 4 nhq a float4 of the queries
  const int kr = tid / 4, kq = tid % 4;
  const bool kload = tid < SC_POS * 4 && t0 + kr < seq;
  const int qi = tid - SC_POS * 4, qh = qi / 4, qq = qi % 4;
  const bool qload = qi >= 0 && qh < nhq;
  const float* krow = keys + (size_t)(t0 + kr) * kv_dim + g * hd + 4 * kq;
  const float* qrow = q + (size_t)(g * group + h0 + qh) * hd + 4 * qq;
  f32x4 reg = {};
  auto load = [&](int c) {
    if (kload) reg = *(const f32x4*)(krow + SC_W * c);
    if (qload) reg = *(const f32x4*)(qrow + SC_W * c);
  };
  auto store = [&](int b) {
    if (kload) *(f32x4*)&kt[b][kr * SC_KP + 4 * kq] = reg;
    if (qload) *(f32x4*)&qt[b][qh * SC_W + 4 * qq] = reg;
  };
  float s = -0.0f;  // Iterator::sum
  load(0);
  store(0);
  if (nc > 1) load(1);
  __syncthreads();
  for (int c = 0; c < nc; c++) {
    if (chain) {
      const f32x4* kk = (const f32x4*)&kt[c & 1][tp * SC_KP];
      const f32x4* qv = (const f32x4*)&qt[c & 1][hq * SC_W];
#pragma unroll
      for (int u = 0; u < SC_W / 4; u++) {
        const f32x4 a = qv[u], b = kk[u];
        s = s + a.x * b.x;
        s = s + a.y * b.y;
        s = s + a.z * b.z;
        s = s + a.w * b.w;
      }
    }
    if (c + 1 < nc) {
      store((c + 1) & 1);  // that buffer was last read in iteration c - 1
      if (c + 2 < nc) load(c + 2);
    }
    __syncthreads();
  }
  if (chain) scores[(size_t)(g * group + h0 + hq) * ld + t0 + tp] = s * scale;
}

// softmax_in_place over each head's scores (one work-group per head): the
// max in any order, the exponentials in parallel, their sum in order by one
// thread, then one division per score.  The probabilities replace the
// scores.  Up to SM_CHUNK scores stay in LDS from the first read to the
// division, and there the in-order sum (about 10 cycles per dependent add)
// runs in lane 0 of wave 0 while waves 1-3 form the exponentials of the
// next SM_PIPE positions.  Longer rows go through global memory in chunks
// of SM_CHUNK.
constexpr int SM_CHUNK = 12288;  // exponentials per LDS chunk (48 KB)
constexpr int SM_PIPE = 512;     // positions per step of the pipelined sum

__global__ __launch_bounds__(256) void k_attn_softmax(float* __restrict__ scores, int seq, int ld) {
  __shared__ __attribute__((aligned(16))) float buf[SM_CHUNK];
  __shared__ float red[4];
  __shared__ float bcast[1];
  float* sc = scores + (size_t)blockIdx.x * ld;
  const int tid = threadIdx.x;
  // max: fold(-inf, f32::max); order-free (a NaN is skipped either way)
  const bool resident = seq <= SM_CHUNK;
  // 16 loads per thread in flight before they are reduced
  float m = -INFINITY;
  for (int t0 = tid; t0 < seq; t0 += 256 * 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int t = t0 + 256 * j;
      v[j] = t < seq ? sc[t] : -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int t = t0 + 256 * j;
      m = fmaxf(m, v[j]);
      if (resident && t < seq) buf[t] = v[j];
    }
  }
  m = wave_max_f32(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (resident) {
    // step k: waves 1-3 exponentiate block k + 1 while lane 0 adds block k
    const int nblk = (seq + SM_PIPE - 1) / SM_PIPE;
    auto expo = [&](int k) {
      const int e = min(seq, (k + 1) * SM_PIPE);
      for (int t = k * SM_PIPE + tid - 64; t < e; t += 192) buf[t] = hale_expf(buf[t] - m);
    };
    float sum = 0.0f;  // sum += exp(v - max), index order
    if (tid >= 64) expo(0);
    __syncthreads();
    for (int k = 0; k < nblk; k++) {
      if (tid == 0) sum = lds_sum_in_order_a16(buf + k * SM_PIPE, min(SM_PIPE, seq - k * SM_PIPE), sum);
      else if (tid >= 64 && k + 1 < nblk) expo(k + 1);
      __syncthreads();
    }
    if (tid == 0) bcast[0] = sum;
    __syncthreads();
    sum = bcast[0];
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
// order.  A work-group takes one key/value head, 16 of its columns and up
// to CTX_HEADS query heads of its group; thread (query head, column) of the
// first wave carries one chain.  A dependent f32 add costs about 10 cycles
// on one wave, and one wave issues about one instruction per 6 cycles, so
// the chains only read products and add them: one 16-byte LDS read per 4
// positions from their own row of a product tile [head x 16 + column][T].
// Waves 1-3 fill the product tile of tile i + 1 while the chains add tile
// i.  Their items are 4 columns of one position's values (16 bytes, kept in
// registers) and 4 positions of one head's probabilities (16 bytes), which
// go to a small LDS tile one iteration before the products that use them,
// so the probabilities that the softmax kernel has just written arrive in
// few, wide loads.  NST register stages of items are in flight.
constexpr int CTX_COLS = 16;
constexpr int CTX_HEADS = 2;       // query heads per work-group (32 chains)
constexpr int CTX_T = 256;         // positions per tile
constexpr int CTX_RP = CTX_T + 4;  // row pitch: rows 4 banks apart modulo 64
constexpr int CTX_ITEMS = (CTX_T * CTX_COLS / 4 + 191) / 192;  // value items per loading thread
static_assert(CTX_HEADS * CTX_T / 4 <= 192, "one probability item per loading thread");

__global__ __launch_bounds__(256) void k_attn_ctx(const float* __restrict__ probs,
                                                  const float* __restrict__ values, int hd,
                                                  int kv_dim, int group, int seq, int ld,
                                                  float* __restrict__ ctx) {
  constexpr int T = CTX_T, RP = CTX_RP;
  __shared__ __attribute__((aligned(16))) float prod[2][CTX_HEADS * CTX_COLS * RP];
  __shared__ __attribute__((aligned(16))) float pbuf[2][CTX_HEADS * T];
  const int g = blockIdx.x;               // key/value head
  const int c0 = blockIdx.y * CTX_COLS;   // first column
  const int h0 = blockIdx.z * CTX_HEADS;  // first query head within the group
  const int nh = min(CTX_HEADS, group - h0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ntiles = (seq + T - 1) / T;
  auto tile_n = [&](int ti) { return min(T, seq - ti * T); };

  if (wave == 0) {
    // the chains: two barriers before the first tile, then one per tile
    float acc = 0.0f;
    __syncthreads();
    __syncthreads();
    for (int ti = 0; ti < ntiles; ti++) {
      if (tid < nh * CTX_COLS) acc = lds_sum_in_order_a16(&prod[ti & 1][tid * RP], tile_n(ti), acc);
      __syncthreads();
    }
    if (tid < nh * CTX_COLS)
      ctx[(size_t)(g * group + h0 + tid / CTX_COLS) * hd + c0 + tid % CTX_COLS] = acc;
    return;
  }

  // waves 1-3: value item i = lt + 192 j of a tile is position i / 4,
  // columns 4q .. 4q + 3 with q = i % 4; probability item lt is head
  // lt / (T / 4), positions 4 (lt % (T / 4)) .. + 3
  constexpr int NLOAD = 192;
  const int lt = tid - 64;
  const float* vbase = values + (size_t)g * hd + c0;
  const float* pbase = probs + ((size_t)g * group + h0) * ld;
  const bool pitem = lt < nh * (T / 4);
  const int ph = lt / (T / 4), pt = 4 * (lt % (T / 4));
  struct Stage {
    f32x4 v[CTX_ITEMS];
    f32x4 p;
  };
  constexpr int NST = 4;
  Stage r[NST];
  auto load = [&](Stage& R, int ti) {
    if (ti >= ntiles) return;
    const int t0 = ti * T, n = tile_n(ti);
    const float* vb = vbase + (size_t)t0 * kv_dim;
#pragma unroll
    for (int j = 0; j < CTX_ITEMS; j++) {
      const int i = lt + NLOAD * j, t = i / 4, q = i % 4;
      if (i < T * 4 && t < n) R.v[j] = *(const f32x4*)(vb + (size_t)t * kv_dim + 4 * q);
    }
    // reads up to 3 past n stay inside the row: ld is a multiple of 4
    if (pitem && pt < n) R.p = *(const f32x4*)(pbase + (size_t)ph * ld + t0 + pt);
  };
  auto store_p = [&](const Stage& R, int b) {
    if (pitem) *(f32x4*)&pbuf[b][ph * T + pt] = R.p;
  };
  // products of the items into product buffer b (positions past the tile's
  // end are not written; the chains never read them)
  auto multiply = [&](const Stage& R, int b, int n) {
#pragma unroll
    for (int j = 0; j < CTX_ITEMS; j++) {
      const int i = lt + NLOAD * j, t = i / 4, q = i % 4;
      if (i < T * 4 && t < n) {
#pragma unroll
        for (int hh = 0; hh < CTX_HEADS; hh++) {
          if (hh < nh) {
            const float p = pbuf[b][hh * T + t];
            float* d = &prod[b][(hh * CTX_COLS + 4 * q) * RP + t];
            d[0] = p * R.v[j].x;
            d[RP] = p * R.v[j].y;
            d[2 * RP] = p * R.v[j].z;
            d[3 * RP] = p * R.v[j].w;
          }
        }
      }
    }
  };
  // Stage s holds the tiles ti with ti % NST == s.  Tile ti's probabilities
  // go to LDS at iteration ti - 2, its products form at iteration ti - 1,
  // and its stage is refilled at iteration ti (each step a barrier after
  // the previous one, so no load waits for a store of the same registers).
#pragma unroll
  for (int j = 0; j < NST; j++) load(r[j], j);
  if (ntiles > 0) store_p(r[0], 0);
  __syncthreads();
  if (ntiles > 0) multiply(r[0], 0, tile_n(0));
  if (ntiles > 1) store_p(r[1], 1);
  __syncthreads();
  for (int ti0 = 0; ti0 < ntiles; ti0 += NST) {
#pragma unroll
    for (int j = 0; j < NST; j++) {
      const int ti = ti0 + j;  // the chains add tile ti
      if (ti < ntiles) {
        if (ti + 1 < ntiles) multiply(r[(j + 1) % NST], (ti + 1) & 1, tile_n(ti + 1));
        if (ti + 2 < ntiles) store_p(r[(j + 2) % NST], ti & 1);
        load(r[j], ti + NST);
        __syncthreads();
      }
    }
  }
}

// softmax_in_place and the context in one kernel for score rows up to
// SMC_MAX positions: work-group (key/value head, 16 columns, 2 query heads)
// as in k_attn_ctx.  It reads its heads' scores into LDS, takes each head's
// max, then lanes 0 and 1 of wave 0 carry the two heads' in-order sums of
// the exp values while waves 1-3 form the exponentials SM_PIPE positions
// ahead.  The context follows as in k_attn_ctx, except that a product's
// probability is formed where it is used (exp value / sum, the reference's
// division), and the first value tiles are loaded before the softmax
// starts.  The eight work-groups of a head pair each repeat its softmax;
// that work hides under the sum chain, and no probability goes back to
// memory.
constexpr int SMC_MAX = 8192;

__global__ __launch_bounds__(256) void k_attn_softmax_ctx(const float* __restrict__ scores,
                                                          const float* __restrict__ values, int hd,
                                                          int kv_dim, int group, int seq, int ld,
                                                          float* __restrict__ ctx) {
  constexpr int T = CTX_T, RP = CTX_RP;
  __shared__ __attribute__((aligned(16))) float ebuf[CTX_HEADS][SMC_MAX];
  __shared__ __attribute__((aligned(16))) float prod[2][CTX_HEADS * CTX_COLS * RP];
  __shared__ float red[CTX_HEADS][4];
  __shared__ float s_sum[CTX_HEADS];
  const int g = blockIdx.x;               // key/value head
  const int c0 = blockIdx.y * CTX_COLS;   // first column
  const int h0 = blockIdx.z * CTX_HEADS;  // first query head within the group
  const int nh = min(CTX_HEADS, group - h0);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int ntiles = (seq + T - 1) / T;
  auto tile_n = [&](int ti) { return min(T, seq - ti * T); };
  const float* srow = scores + ((size_t)g * group + h0) * ld;

  // value items of waves 1-3 (as in k_attn_ctx); the first NST tiles go out
  // before the softmax
  constexpr int NLOAD = 192;
  const int lt = tid - 64;
  const float* vbase = values + (size_t)g * hd + c0;
  constexpr int NST = 4;
  f32x4 r[NST][CTX_ITEMS];
  auto load = [&](f32x4* R, int ti) {
    if (ti >= ntiles || lt < 0) return;
    const int t0 = ti * T, n = tile_n(ti);
    const float* vb = vbase + (size_t)t0 * kv_dim;
#pragma unroll
    for (int j = 0; j < CTX_ITEMS; j++) {
      const int i = lt + NLOAD * j, t = i / 4, q = i % 4;
      if (i < T * 4 && t < n) R[j] = *(const f32x4*)(vb + (size_t)t * kv_dim + 4 * q);
    }
  };
#pragma unroll
  for (int j = 0; j < NST; j++) load(r[j], j);

  // softmax: each head's max (order-free; both heads' loads in flight
  // together), exp values in place, in-order sum
  float mx[CTX_HEADS];
  {
    float m[CTX_HEADS];
#pragma unroll
    for (int hh = 0; hh < CTX_HEADS; hh++) m[hh] = -INFINITY;
    for (int t0 = tid; t0 < seq; t0 += 256 * 16) {
      float v[CTX_HEADS][16];
#pragma unroll
      for (int hh = 0; hh < CTX_HEADS; hh++)
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const int t = t0 + 256 * j;
          v[hh][j] = hh < nh && t < seq ? srow[(size_t)hh * ld + t] : -INFINITY;
        }
#pragma unroll
      for (int hh = 0; hh < CTX_HEADS; hh++)
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const int t = t0 + 256 * j;
          m[hh] = fmaxf(m[hh], v[hh][j]);
          if (hh < nh && t < seq) ebuf[hh][t] = v[hh][j];
        }
    }
#pragma unroll
    for (int hh = 0; hh < CTX_HEADS; hh++) {
      const float mw = wave_max_f32(m[hh]);
      if (lane == 0) red[hh][wave] = mw;
    }
  }
  __syncthreads();
#pragma unroll
  for (int hh = 0; hh < CTX_HEADS; hh++)
    mx[hh] = fmaxf(fmaxf(red[hh][0], red[hh][1]), fmaxf(red[hh][2], red[hh][3]));
  // blocks of the sum: a short first block (the chains start sooner), then
  // SM_PIPE positions each
  constexpr int FIRST = 128;
  auto bstart = [&](int k) { return k == 0 ? 0 : min(seq, FIRST + (k - 1) * SM_PIPE); };
  const int nblk = 1 + (max(0, seq - FIRST) + SM_PIPE - 1) / SM_PIPE;
  auto expo = [&](int k) {  // waves 1-3: the exp values of block k of every head
    const int b0 = bstart(k), len = bstart(k + 1) - b0;
    for (int i = lt; i < nh * len; i += NLOAD) {
      const int hh = i / len, t = b0 + i % len;
      ebuf[hh][t] = hale_expf(ebuf[hh][t] - (hh ? mx[1] : mx[0]));
    }
  };
  float sum = 0.0f;  // lane hh of wave 0: sum += exp(v - max), index order
  if (lt >= 0) expo(0);
  __syncthreads();
  for (int k = 0; k < nblk; k++) {
    if (wave == 0) {
      if (lane < nh) sum = lds_sum_in_order_a16(&ebuf[lane][bstart(k)], bstart(k + 1) - bstart(k), sum);
    } else if (k + 1 < nblk) {
      expo(k + 1);
    }
    __syncthreads();
  }
  if (wave == 0 && lane < nh) s_sum[lane] = sum;
  __syncthreads();
  float sm[CTX_HEADS];
#pragma unroll
  for (int hh = 0; hh < CTX_HEADS; hh++) sm[hh] = hh < nh ? s_sum[hh] : 1.0f;

  // context: products p_t v_t[c] with p_t = e_t / sum, tile i + 1 formed
  // while the chains add tile i
  auto multiply = [&](const f32x4* R, int ti, int b) {
    if (lt < 0) return;
    const int t0 = ti * T, n = tile_n(ti);
#pragma unroll
    for (int j = 0; j < CTX_ITEMS; j++) {
      const int i = lt + NLOAD * j, t = i / 4, q = i % 4;
      if (i < T * 4 && t < n) {
#pragma unroll
        for (int hh = 0; hh < CTX_HEADS; hh++) {
          if (hh < nh) {
            const float pr = ebuf[hh][t0 + t] / sm[hh];
            float* d = &prod[b][(hh * CTX_COLS + 4 * q) * RP + t];
            d[0] = pr * R[j].x;
            d[RP] = pr * R[j].y;
            d[2 * RP] = pr * R[j].z;
            d[3 * RP] = pr * R[j].w;
          }
        }
      }
    }
  };
  const bool chain = tid < nh * CTX_COLS;
  float acc = 0.0f;
  if (ntiles > 0) multiply(r[0], 0, 0);
  __syncthreads();
  for (int ti0 = 0; ti0 < ntiles; ti0 += NST) {
#pragma unroll
    for (int j = 0; j < NST; j++) {
      const int ti = ti0 + j;  // the chains add tile ti
      if (ti < ntiles) {
        if (chain) acc = lds_sum_in_order_a16(&prod[ti & 1][tid * RP], tile_n(ti), acc);
        if (ti + 1 < ntiles) multiply(r[(j + 1) % NST], ti + 1, (ti + 1) & 1);
        load(r[j], ti + NST);  // its products went to LDS one iteration ago
        __syncthreads();
      }
    }
  }
  if (chain) ctx[(size_t)(g * group + h0 + tid / CTX_COLS) * hd + c0 + tid % CTX_COLS] = acc;
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
  const int group = a.nh / a.nkv;
  dim3 gs((unsigned)((a.seq + SC_POS - 1) / SC_POS), (unsigned)a.nkv,
          (unsigned)((group + SC_HEADS - 1) / SC_HEADS));
  e = launch(k_attn_scores, gs, 256, 0, st, (const float*)a.q, (const float*)a.keys, a.hd, kv_dim,
             a.nh / a.nkv, a.seq, a.ld, scale, a.scores);
  if (e != hipSuccess) return e;
  dim3 gc((unsigned)a.nkv, (unsigned)(a.hd / CTX_COLS), (unsigned)((group + CTX_HEADS - 1) / CTX_HEADS));
  if (a.seq <= SMC_MAX)
    return launch(k_attn_softmax_ctx, gc, 256, 0, st, (const float*)a.scores,
                  (const float*)a.values, a.hd, kv_dim, group, a.seq, a.ld, a.ctx);
  e = launch(k_attn_softmax, (unsigned)a.nh, 256, 0, st, a.scores, a.seq, a.ld);
  if (e != hipSuccess) return e;
  return launch(k_attn_ctx, gc, 256, 0, st, (const float*)a.scores,
                (const float*)a.values, a.hd, kv_dim, group, a.seq, a.ld, a.ctx);
}

}  // namespace hale
