// kernels_decode.hip -- gfx950 kernels for the quantized matvec and the
// batch-1 MoE layer (Hale-Token src/tensor/quant.rs, src/tensor/matrix.rs,
// src/expert/mod.rs, src/model/moe.rs).
//
// Bit-exactness: every f32 result equals the reference's.  The reference
// sums the per-block terms of a row strictly left to right
// (dot_q8_0 / dot_q4_0, src/tensor/quant.rs:115-144), so the kernels compute
// the block terms in parallel, park them in LDS and fold each row in block
// order in one lane.
#pragma clang fp contract(off)

#include <atomic>

#include "hale_device.h"
#include "kernels.h"

namespace hale {

// ===========================================================================
// Layout conversion: reference block layout <-> HBM tile planes
// ===========================================================================

// One thread per (row, block) of the padded matrix; padding rows get zero
// codes and zero scales, so every plane byte is written.
template <int DT>
__global__ __launch_bounds__(256) void k_repack(const uint8_t* __restrict__ aos, size_t rows,
                                                int nb, size_t prow, uint8_t* __restrict__ codes,
                                                uint16_t* __restrict__ scales) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int BB = DT == Q8_0 ? 34 : 18;
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= prow * (size_t)nb) return;
  size_t row = id / nb;
  int b = (int)(id % nb);
  size_t tile = row / TILE;
  int r = (int)(row % TILE);
  uint8_t buf[32];
  uint16_t sc = 0;
  if (row < rows) {
    const uint8_t* src = aos + (row * nb + b) * BB;
    sc = (uint16_t)(src[0] | (src[1] << 8));
#pragma unroll
    for (int j = 0; j < CH * 16; j++) buf[j] = src[2 + j];
  } else {
#pragma unroll
    for (int j = 0; j < CH * 16; j++) buf[j] = 0;
  }
  scales[(tile * nb + b) * TILE + r] = sc;
#pragma unroll
  for (int c = 0; c < CH; c++) {
    uint8_t* dst = codes + (((tile * nb + b) * CH + c) * TILE + r) * 16;
    u32x4 v;
    __builtin_memcpy(&v, buf + 16 * c, 16);
    *(u32x4*)dst = v;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void k_unpack(const uint8_t* __restrict__ codes,
                                                const uint16_t* __restrict__ scales, size_t rows,
                                                int nb, uint8_t* __restrict__ aos) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int BB = DT == Q8_0 ? 34 : 18;
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * (size_t)nb) return;
  size_t row = id / nb;
  int b = (int)(id % nb);
  size_t tile = row / TILE;
  int r = (int)(row % TILE);
  uint8_t* dst = aos + (row * nb + b) * BB;
  uint16_t sc = scales[(tile * nb + b) * TILE + r];
  dst[0] = (uint8_t)(sc & 0xff);
  dst[1] = (uint8_t)(sc >> 8);
  for (int c = 0; c < CH; c++) {
    const uint8_t* src = codes + (((tile * nb + b) * CH + c) * TILE + r) * 16;
    for (int j = 0; j < 16; j++) dst[2 + 16 * c + j] = src[j];
  }
}

// ===========================================================================
// Weight quantization: encode_row (src/tensor/quant.rs:274-321)
// ===========================================================================

// One thread per block; writes the reference layout.
template <int DT>
__global__ __launch_bounds__(256) void k_encode(const float* __restrict__ values, size_t nblocks,
                                                uint8_t* __restrict__ out) {
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= nblocks) return;
  const f32x4* src = (const f32x4*)(values + id * QK);
  float v[QK];
#pragma unroll
  for (int i = 0; i < QK / 4; i++) {
    f32x4 f = src[i];
    v[4 * i] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  if constexpr (DT == Q8_0) {
    // encode_block_q8_0, quant.rs:295-305
    uint8_t* dst = out + id * 34;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(v[j]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    uint16_t h = f2h(scale);
    dst[0] = (uint8_t)(h & 0xff);
    dst[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int j = 0; j < QK; j++) {
      float r = roundf(v[j] * inv);
      r = r < -127.0f ? -127.0f : r;  // f32::clamp keeps NaN, `as i8` maps it to 0
      r = r > 127.0f ? 127.0f : r;
      dst[2 + j] = (uint8_t)(int8_t)sat_i8(r);
    }
  } else {
    // encode_block_q4_0, quant.rs:309-321
    uint8_t* dst = out + id * 18;
    float extreme = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; j++)
      if (fabsf(v[j]) > fabsf(extreme)) extreme = v[j];
    float scale = extreme / -8.0f;
    float inv = scale != 0.0f ? 1.0f / scale : 0.0f;
    uint16_t h = f2h(scale);
    dst[0] = (uint8_t)(h & 0xff);
    dst[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int j = 0; j < QK / 2; j++) {
      int lo = sat_i32(v[j] * inv + 8.5f);
      int hi = sat_i32(v[j + QK / 2] * inv + 8.5f);
      lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
      hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
      dst[2 + j] = (uint8_t)(lo | (hi << 4));
    }
  }
}

// ===========================================================================
// Activation quantization: Q8Activations::quantize (quant.rs:77-93)
// ===========================================================================

// x [ntok][n] -> act [ntok][n/32], any alignment of x: each 32-lane group
// quantizes one block.
__global__ __launch_bounds__(256) void k_act_quant_any(const float* __restrict__ x, size_t nblocks,
                                                       ActBlock* __restrict__ act) {
  size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) / 32;
  int j = threadIdx.x & 31;
  if (blk >= nblocks) return;  // uniform across the 32-lane group
  float v = x[blk * QK + j];
  float scale;
  int qsum;
  int q = quant_block_lane(v, &scale, &qsum);
  act[blk].q[j] = (int8_t)q;
  if (j == 0) {
    act[blk].scale = scale;
    act[blk].qsum = qsum;
  }
}

// The same for 16-byte aligned x; each 8-lane group quantizes one block
// from one 16-byte load per lane.  The block maximum and the code sum are
// order-free (max and integer sums), and scale, reciprocal and codes are
// the expressions of quant_block_lane.
__global__ __launch_bounds__(256) void k_act_quant(const float* __restrict__ x, size_t nblocks,
                                                   ActBlock* __restrict__ act) {
  const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) / 8;
  const int j = threadIdx.x & 7;
  if (blk >= nblocks) return;  // uniform across the 8-lane group
  const f32x4 v = *(const f32x4*)(x + blk * QK + 4 * j);
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = fmaxf(amax, HALE_DPP_F32(amax, 0xB1));   // lane ^ 1
  amax = fmaxf(amax, HALE_DPP_F32(amax, 0x4E));   // lane ^ 2
  amax = fmaxf(amax, HALE_DPP_F32(amax, 0x141));  // mirror within 8 lanes
  const float scale = amax / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  const int q0 = sat_i8(roundf(v.x * inv)), q1 = sat_i8(roundf(v.y * inv));
  const int q2 = sat_i8(roundf(v.z * inv)), q3 = sat_i8(roundf(v.w * inv));
  int qs = q0 + q1 + q2 + q3;
  qs += __builtin_amdgcn_update_dpp(0, qs, 0xB1, 0xF, 0xF, false);
  qs += __builtin_amdgcn_update_dpp(0, qs, 0x4E, 0xF, 0xF, false);
  qs += __builtin_amdgcn_update_dpp(0, qs, 0x141, 0xF, 0xF, false);
  *(unsigned*)(act[blk].q + 4 * j) = (unsigned)(q0 & 0xff) | (unsigned)(q1 & 0xff) << 8 |
                                     (unsigned)(q2 & 0xff) << 16 | (unsigned)(q3 & 0xff) << 24;
  if (j == 0) {
    act[blk].scale = scale;
    act[blk].qsum = qs;
  }
}

// ===========================================================================
// Router: MoeLayer::route (src/model/moe.rs:36-53)
// ===========================================================================
//
// Two parts.  k_route_logits (grid (E, T), 64 threads) computes logit e of
// token t with the 8-lane f32 order of dot_f32 (quant.rs:37-41,152-194) and
// quantizes a share of token t's activation blocks.  route_select (one
// wave) turns E logits into the top-k experts and their weights; the
// gate/up kernel runs it in every work-group's prologue, so no work-group
// ever waits for another.

constexpr int ROUTE_MAX_H = 8192;
constexpr int ROUTE_MAX_E = 1024;
constexpr int GEMV_MAX_NB = 512;  // blocks per row the GEMV stages in LDS

constexpr int ROUTE_THREADS = 256;
constexpr int ROUTE_VPT = ROUTE_MAX_H / 4 / ROUTE_THREADS;  // float4 of w (and of x) per thread

__global__ __launch_bounds__(ROUTE_THREADS) void k_route_logits(const float* __restrict__ router,
                                                                const float* __restrict__ x, int H,
                                                                int E, ActBlock* __restrict__ act,
                                                                float* __restrict__ logits) {
  __shared__ __attribute__((aligned(16))) float prod[ROUTE_MAX_H + 32];  // chain-major
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int t = blockIdx.y;
  const int gx = gridDim.x;
  const int e = blockIdx.x;
  const float* xt = x + (size_t)t * H;
  const int nb = H / QK;
  const float* w = router + (size_t)e * H;
  const int steps = H / 8;
  const int nvec = steps * 2;  // float4 chunks covering the 8-lane part

  // every load of the row and of x first
  f32x4 wv[ROUTE_VPT], xv[ROUTE_VPT];
#pragma unroll
  for (int j = 0; j < ROUTE_VPT; j++) {
    const int c = tid + j * ROUTE_THREADS;
    if (c < nvec) {
      wv[j] = *(const f32x4*)(w + 4 * c);
      xv[j] = *(const f32x4*)(xt + 4 * c);
    }
  }

  // activation quantization share: half-wave hw takes blocks hw + 8 (e + gx i)
  for (int bb = (tid >> 5) + 8 * e; bb < nb; bb += 8 * gx) {
    float v = xt[bb * QK + (lane & 31)];
    float scale;
    int qsum;
    int q = quant_block_lane(v, &scale, &qsum);
    ActBlock* ab = act + (size_t)t * nb + bb;
    ab->q[lane & 31] = (int8_t)q;
    if ((lane & 31) == 0) {
      ab->scale = scale;
      ab->qsum = qsum;
    }
  }

  // products w[i]*x[i] (each one rounding, order free) into chain-major LDS:
  // chain l holds i = 8s + l at prod[l * stride + s]
  const int stride = steps + 4;  // 16 B aligned rows, chains on distinct banks
#pragma unroll
  for (int j = 0; j < ROUTE_VPT; j++) {
    const int c = tid + j * ROUTE_THREADS;
    if (c < nvec) {
      const int sidx = c >> 1, l0 = (c & 1) * 4;
      prod[(l0 + 0) * stride + sidx] = wv[j].x * xv[j].x;
      prod[(l0 + 1) * stride + sidx] = wv[j].y * xv[j].y;
      prod[(l0 + 2) * stride + sidx] = wv[j].z * xv[j].z;
      prod[(l0 + 3) * stride + sidx] = wv[j].w * xv[j].w;
    }
  }
  __syncthreads();
  if (tid >= 64) return;
  // acc[l] += w[8i+l]*x[8i+l] in order of i
  float acc = 0.0f;
  if (lane < 8) acc = lds_sum_in_order_a16(prod + lane * stride, steps, acc);
  float a0 = __shfl(acc, 0), a1 = __shfl(acc, 1), a2 = __shfl(acc, 2), a3 = __shfl(acc, 3);
  float a4 = __shfl(acc, 4), a5 = __shfl(acc, 5), a6 = __shfl(acc, 6), a7 = __shfl(acc, 7);
  if (lane == 0) {
    float tail = -0.0f;  // Iterator::sum over the H % 8 leftover products
    for (int i = steps * 8; i < H; i++) tail = tail + w[i] * xt[i];
    float s0v = (a0 + a4) + (a1 + a5);
    float s1v = (a2 + a6) + (a3 + a7);
    logits[(size_t)t * E + e] = (s0v + s1v) + tail;
  }
}

// softmax_in_place (src/ops/activation.rs:11-21), top_k (src/ops/topk.rs:
// 44-61) and the renormalisation of MoeLayer::route, run by one whole wave
// (all 64 lanes active).  Element i lives in lane i % 64, slot i / 64.
//   - the sum of exp(l_i - max) is taken strictly in index order by lane 0,
//     reading the next 16 values from LDS while it adds the current 16;
//   - top-k: each probability gets its total_cmp key as an order-preserving
//     u32; in each of k rounds the wave's largest untaken key is found and
//     the lowest untaken index holding it wins (ties go to the lower index,
//     as in the reference), so the experts come out best first;
//   - norm = sum of the chosen probabilities in that order, then w = p / norm.
// The k chosen experts and renormalised weights go to sel_idx / sel_w
// (LDS), best first.  rs is LDS scratch of ROUTE_MAX_E + 4*64 words.
// k rounds over order-preserving u32 keys (element lane + 64 m in key[m],
// present where bit m of live is set): the wave's largest untaken key is
// the next best and the lowest untaken index holding it wins, so lane r
// ends with the r-th best index and its probability (decoded from the key)
// for r < k.  Taken keys are set to 0, no larger than any real key, so the
// wave maximum is the largest untaken key; the live mask keeps a real key of
// 0 apart from a taken one.  norm: the chosen probabilities summed best
// first from -0.0 (Iterator::sum), or 1 without renormalisation.
template <int PER>
__device__ __forceinline__ void topk_rounds(unsigned* key, unsigned& live, int k, int normalize,
                                            int* my_idx, float* my_p, float* norm_out) {
  const int lane = threadIdx.x & 63;
  float norm = normalize ? -0.0f : 1.0f;
  for (int r = 0; r < k; r++) {
    unsigned loc = key[0];
#pragma unroll
    for (int m = 1; m < PER; m++) loc = key[m] > loc ? key[m] : loc;
    const unsigned best = wave_max_u32(loc);
    int widx = -1;
#pragma unroll
    for (int m = 0; m < PER; m++) {
      const unsigned long long msk = __ballot(((live >> m) & 1u) && key[m] == best);
      if (widx < 0 && msk) widx = 64 * m + (int)__builtin_ctzll(msk);
    }
#pragma unroll
    for (int m = 0; m < PER; m++) {
      if (64 * m + lane == widx) {
        key[m] = 0u;
        live &= ~(1u << m);
      }
    }
    const float pw = key_value(best);
    if (normalize) norm = norm + pw;
    if (lane == r) {
      *my_idx = widx;
      *my_p = pw;
    }
  }
  *norm_out = norm;
}

constexpr int RS_SCRATCH = 2 * ROUTE_MAX_E + 4 * 64;

template <int PER>  // elements per lane: E <= 64 * PER
__device__ __forceinline__ void route_select_t(const float* lg, int E, int k, int normalize,
                                               int* sel_idx, float* sel_w, const ExpTable& tab,
                                               float* rs) {
  const int lane = threadIdx.x & 63;
  float* e_lds = rs;
  float v[PER];
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    v[m] = (i < E) ? lg[i] : -__builtin_huge_valf();
    mx = fmaxf(mx, v[m]);
  }
  mx = wave_max_f32(mx);  // max is order independent
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    v[m] = wave_expf(v[m] - mx, tab);
    if (i < E) e_lds[i] = v[m];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float sum = 0.0f;  // sum += exp(v - max), index order
  if (lane == 0) sum = lds_sum_in_order(e_lds, E, sum);
  sum = lane_value(sum, 0);
  unsigned key[PER];
  unsigned live = 0;  // bit m: element lane + 64 m exists and is not taken
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    key[m] = 0u;
    if (i < E) {
      key[m] = order_key(v[m] / sum);
      live |= 1u << m;
    }
  }
  int my_idx = 0;
  float my_p = 0.0f, norm = 0.0f;
  topk_rounds<PER>(key, live, k, normalize, &my_idx, &my_p, &norm);
  if (lane < k) {
    sel_idx[lane] = my_idx;
    sel_w[lane] = my_p / norm;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void route_select(const float* lg, int E, int k, int normalize,
                                             int* sel_idx, float* sel_w, const ExpTable& tab,
                                             float* rs) {
  if (E <= 64)
    route_select_t<1>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (E <= 128)
    route_select_t<2>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (E <= 256)
    route_select_t<4>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (E <= 512)
    route_select_t<8>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else
    route_select_t<16>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
}

// The same selection split over waves 0 and 1 of a work-group, for the
// gate/up prologue (every wave of the work-group passes the two barriers
// inside).  Ranking by logit gives the reference's order unless rounding
// makes two
// probabilities equal (the map logit -> exp(logit - max) -> probability is
// non-decreasing).  Wave 0 ranks by logit while wave 1 takes the max, the
// exp values, the in-order sum and the probability keys; then wave 0 checks
// the ranking against the probabilities: each chosen pair, and the last
// chosen against every unchosen element, must be in (probability desc,
// index asc) order.  If a check fails it ranks again by probability.
// Either way the result is the reference's.  rs: RS_SCRATCH words of LDS.
template <int PER>
__device__ __forceinline__ void route_select_pair_t(const float* lg, int E, int k, int normalize,
                                                    int* sel_idx, float* sel_w, const ExpTable& tab,
                                                    float* rs, int wave) {
  const int lane = threadIdx.x & 63;
  float* e_lds = rs;                                  // [E] exp values
  unsigned* pkey = (unsigned*)(rs + ROUTE_MAX_E);     // [E] probability keys
  float v[PER];
  unsigned key[PER];
  unsigned live = 0;
  int my_idx = 0;
  if (wave <= 1) {
#pragma unroll
    for (int m = 0; m < PER; m++) {
      const int i = lane + 64 * m;
      v[m] = (i < E) ? lg[i] : -__builtin_huge_valf();
    }
    if (wave == 1) {
      float mx = v[0];
#pragma unroll
      for (int m = 1; m < PER; m++) mx = fmaxf(mx, v[m]);
      mx = wave_max_f32(mx);
#pragma unroll
      for (int m = 0; m < PER; m++) v[m] = wave_expf(v[m] - mx, tab);
#pragma unroll
      for (int m = 0; m < PER; m++)
        if (lane + 64 * m < E) e_lds[lane + 64 * m] = v[m];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float sum = 0.0f;  // sum += exp(v - max), index order
      if (lane == 0) sum = lds_sum_in_order(e_lds, E, sum);
      sum = lane_value(sum, 0);
#pragma unroll
      for (int m = 0; m < PER; m++)
        if (lane + 64 * m < E) pkey[lane + 64 * m] = order_key(v[m] / sum);
    } else {
#pragma unroll
      for (int m = 0; m < PER; m++) {
        key[m] = 0u;
        if (lane + 64 * m < E) {
          key[m] = order_key(v[m]);
          live |= 1u << m;
        }
      }
      float unused_p, unused_norm;
      topk_rounds<PER>(key, live, k, 0, &my_idx, &unused_p, &unused_norm);
    }
  }
  __syncthreads();
  if (wave == 0) {
    // lane r < k checks chosen r against chosen r + 1.  Every unchosen
    // element ranks after the last chosen by logit, hence normally no higher
    // by probability; the ranking fails if one has a larger probability key,
    // or an equal one at a lower index.  live: unchosen existing elements of
    // this lane.
    const int next = __shfl(my_idx, lane + 1);
    const int last = __shfl(my_idx, k - 1);
    const unsigned klast = pkey[last];
    bool bad = false;
    if (lane + 1 < k) {
      const unsigned ka = pkey[my_idx], kb = pkey[next];
      bad = !(ka > kb || (ka == kb && my_idx < next));
    }
    unsigned pk[PER];
#pragma unroll
    for (int m = 0; m < PER; m++) {
      const int i = lane + 64 * m;
      pk[m] = (i < E) ? pkey[i] : 0u;
      if ((live >> m) & 1u) bad = bad || pk[m] > klast || (pk[m] == klast && i < last);
    }
    float my_p = 0.0f, norm = 1.0f;
    if (__ballot(bad) == 0ull) {
      my_p = lane < k ? key_value(pkey[my_idx]) : 0.0f;
      if (normalize) {
        norm = -0.0f;  // Iterator::sum in best-first order
        for (int r = 0; r < k; r++) norm = norm + lane_value(my_p, r);
      }
    } else {  // a tie the exp values did not show: rank by probability
      unsigned live2 = 0;
#pragma unroll
      for (int m = 0; m < PER; m++)
        if (lane + 64 * m < E) live2 |= 1u << m;
      topk_rounds<PER>(pk, live2, k, normalize, &my_idx, &my_p, &norm);
    }
    if (lane < k) {
      sel_idx[lane] = my_idx;
      sel_w[lane] = my_p / norm;
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void route_select_pair(const float* lg, int E, int k, int normalize,
                                                  int* sel_idx, float* sel_w, const ExpTable& tab,
                                                  float* rs, int wave) {
  if (E <= 64)
    route_select_pair_t<1>(lg, E, k, normalize, sel_idx, sel_w, tab, rs, wave);
  else if (E <= 128)
    route_select_pair_t<2>(lg, E, k, normalize, sel_idx, sel_w, tab, rs, wave);
  else if (E <= 256)
    route_select_pair_t<4>(lg, E, k, normalize, sel_idx, sel_w, tab, rs, wave);
  else if (E <= 512)
    route_select_pair_t<8>(lg, E, k, normalize, sel_idx, sel_w, tab, rs, wave);
  else
    route_select_pair_t<16>(lg, E, k, normalize, sel_idx, sel_w, tab, rs, wave);
}

// Standalone routing (MoeLayer::route without the experts, and the grouped
// path): one wave per token.
__global__ __launch_bounds__(64) void k_route_select(const float* __restrict__ logits, int E, int k,
                                                     int normalize, int* __restrict__ route_idx,
                                                     float* __restrict__ route_w,
                                                     unsigned long long* __restrict__ stats) {
  __shared__ int sel_idx[64];
  __shared__ float sel_w[64];
  __shared__ __attribute__((aligned(16))) float rs[RS_SCRATCH];
  const int t = blockIdx.x;
  ExpTable tab;
  tab.load();
  route_select(logits + (size_t)t * E, E, k, normalize, sel_idx, sel_w, tab, rs);
  __syncthreads();
  const int lane = threadIdx.x;
  if (lane < k) {
    route_idx[(size_t)t * k + lane] = sel_idx[lane];
    route_w[(size_t)t * k + lane] = sel_w[lane];
    if (stats) atomicAdd(&stats[sel_idx[lane]], 1ull);
  }
}

// ===========================================================================
// Exact tile GEMV
// ===========================================================================
//
// A work-group of 4 waves owns a group of 64 output rows (two 32-row tiles)
// and loops over the rows' quantization blocks in chunks: in a chunk wave w
// takes blocks w, w+4, w+8, ... and issues all of their loads at once (16
// per lane, 16 B each).  For one block a wave reads 2 x 512 B of codes
// (q4_0) or 2 x 1 KB (q8_0), every lane uses the same activation block
// (scalar loads), and lane l forms the block term (d_w * d_x) * isum of row
// l.  Terms go to LDS; wave 0 adds them to its 64 running row sums in block
// order, so each total is the reference's left-to-right sum.  The next
// chunk's loads are issued before the fold, and two LDS buffers let the
// other waves fill chunk c+1 while wave 0 folds chunk c.
//
// Epilogues:
//   EPI_PLAIN    out[row] = total                      (WeightMatrix::matvec)
//   EPI_GATE_UP  rows 0-31 gate, 32-63 up of one I-tile; h = silu(g)*u is
//                quantized to its q8 block for the down projection
//                (Expert::forward, src/expert/mod.rs:95-102).  With router
//                logits given, the prologue selects the slot's expert.

template <int DT>
__device__ __forceinline__ float block_term(const u32x4* c, uint16_t sc, const ActBlock* ab) {
  const int* aq = (const int*)ab->q;
  int isum = 0;
  if constexpr (DT == Q8_0) {
    isum = __builtin_amdgcn_sdot4((int)c[0].x, aq[0], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[0].y, aq[1], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[0].z, aq[2], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[0].w, aq[3], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[1].x, aq[4], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[1].y, aq[5], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[1].z, aq[6], isum, false);
    isum = __builtin_amdgcn_sdot4((int)c[1].w, aq[7], isum, false);
  } else {
    const unsigned m = 0x0f0f0f0fu;
    // raw nibbles (0..15) are non-negative as i8, so sdot4 sums n_j * x_j;
    // subtracting 8 * sum(x) applies the offset of 8
    isum = __builtin_amdgcn_sdot4((int)(c[0].x & m), aq[0], isum, false);
    isum = __builtin_amdgcn_sdot4((int)(c[0].y & m), aq[1], isum, false);
    isum = __builtin_amdgcn_sdot4((int)(c[0].z & m), aq[2], isum, false);
    isum = __builtin_amdgcn_sdot4((int)(c[0].w & m), aq[3], isum, false);
    isum = __builtin_amdgcn_sdot4((int)((c[0].x >> 4) & m), aq[4], isum, false);
    isum = __builtin_amdgcn_sdot4((int)((c[0].y >> 4) & m), aq[5], isum, false);
    isum = __builtin_amdgcn_sdot4((int)((c[0].z >> 4) & m), aq[6], isum, false);
    isum = __builtin_amdgcn_sdot4((int)((c[0].w >> 4) & m), aq[7], isum, false);
    isum -= 8 * ab->qsum;
  }
  float d = h2f(sc) * ab->scale;
  return d * (float)isum;
}

template <int DT>
__device__ __forceinline__ int block_isum(const u32x4* c, const ActBlock* ab) {
  const int* aq = (const int*)ab->q;
  int isum = 0;
  if constexpr (DT == Q8_0) {
    const unsigned* w = (const unsigned*)c;
    for (int i = 0; i < 8; i++) isum = __builtin_amdgcn_sdot4((int)w[i], aq[i], isum, false);
  } else {
    const unsigned* w = (const unsigned*)c;
    for (int i = 0; i < 4; i++) {
      isum = __builtin_amdgcn_sdot4((int)(w[i] & 0x0f0f0f0fu), aq[i], isum, false);
      isum = __builtin_amdgcn_sdot4((int)((w[i] >> 4) & 0x0f0f0f0fu), aq[4 + i], isum, false);
    }
    isum -= 8 * ab->qsum;
  }
  return isum;
}

// NW waves per work-group: four for plain rows; eight for gate/up (the
// terms of a one-token layer are spread over twice the waves, so they take
// half as long after the loads land), sixteen for q4_0 gate/up rows that
// fit one chunk (H <= 2048; with more chunks four loads in flight per lane
// pipeline worse).
template <int DT, int EPI, int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv(GemvArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int UPW = 64 / NW / CH;      // blocks per wave per chunk (64 / NW loads in flight)
  constexpr int CB = UPW * NW;           // blocks per chunk
  static_assert(UPW % 4 == 0, "terms go in groups of four blocks");
  __shared__ float terms[2][CB][GROUP];
  __shared__ ActBlock s_act[GEMV_MAX_NB];
  __shared__ int sel_idx[64];
  __shared__ float sel_w[64];
  __shared__ __attribute__((aligned(16))) float rs[EPI == EPI_GATE_UP ? RS_SCRATCH : 4];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  const int slot = blockIdx.y;
  const int nb = a.nb;

  // The activation blocks of this slot go to LDS.  With routing in the
  // prologue, waves 0 and 1 select the experts from the first instruction on
  // while the other waves stage the activations (wave 1 joins them after its
  // part of the selection); otherwise every wave stages and the
  // weight loads are issued before the staging stores.
  const bool routing = EPI == EPI_GATE_UP && a.logits != nullptr;
  const int nstage = routing ? 64 * (NW - 1) : 64 * NW;  // staging threads
  const int stid = routing ? (int)threadIdx.x - 64 : (int)threadIdx.x;
  constexpr int APER = (GEMV_MAX_NB * 3 + 64 * (NW - 1) - 1) / (64 * (NW - 1));
  u32x4 av[APER];
  if (stid >= 0) {
    const u32x4* src = (const u32x4*)(a.act + (size_t)slot * a.act_stride);
#pragma unroll
    for (int j = 0; j < APER; j++) {
      const int i = stid + j * nstage;
      if (i < nb * 3) av[j] = src[i];
    }
  }
  auto stage_act = [&]() {
    if (stid < 0) return;
    u32x4* dst = (u32x4*)s_act;
#pragma unroll
    for (int j = 0; j < APER; j++) {
      const int i = stid + j * nstage;
      if (i < nb * 3) dst[i] = av[j];
    }
  };
  ExpTable tab;
  if constexpr (EPI == EPI_GATE_UP) tab.load();
  int expert = a.route_idx ? a.route_idx[slot] : 0;
  if constexpr (EPI == EPI_GATE_UP) {
    if (routing) {  // choose this token's experts from the router logits
      if (wave >= 2) stage_act();
      route_select_pair(a.logits, a.E, a.slots, a.normalize, sel_idx, sel_w, tab, rs, wave);
      if (wave == 1) stage_act();
      if (g == 0 && threadIdx.x == 0) {  // one work-group per slot publishes it
        a.route_out_idx[slot] = sel_idx[slot];
        a.route_out_w[slot] = sel_w[slot];
        if (a.stats) atomicAdd(&a.stats[sel_idx[slot]], 1ull);
      }
      __syncthreads();
      expert = sel_idx[slot];
    }
  }

  // tile and matrix of this lane's row
  const uint8_t* cbase;
  const uint16_t* sbase;
  size_t tile;
  if constexpr (EPI == EPI_GATE_UP) {
    tile = g;
    cbase = (lane < 32 ? a.codes : a.codes2) + (size_t)expert * a.codes_stride;
    sbase = (lane < 32 ? a.scales : a.scales2) + (size_t)expert * a.scales_stride;
  } else {
    tile = 2 * (size_t)g + (lane >> 5);
    cbase = a.codes + (size_t)expert * a.codes_stride;
    sbase = a.scales + (size_t)expert * a.scales_stride;
  }
  const int r = lane & 31;
  const uint8_t* crow = cbase + (tile * nb * CH * TILE + r) * 16;
  const uint16_t* srow = sbase + tile * nb * TILE + r;
  const ActBlock* act = s_act;

  u32x4 cw[UPW][CH];
  uint16_t sw[UPW];
  // Blocks past the end of the row are clamped to the last block (an
  // in-bounds load whose term is never stored), so the chunk loop has no
  // branches and all of its loads are in flight together.
  auto load_block = [&](int ch, int s) {
    const int b = min(ch * CB + wave + NW * s, nb - 1);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[s][c] = __builtin_nontemporal_load((const u32x4*)(crow + ((size_t)b * CH + c) * TILE * 16));
    sw[s] = srow[(size_t)b * TILE];
  };
  auto load_chunk = [&](int ch) {
#pragma unroll
    for (int s = 0; s < UPW; s++) load_block(ch, s);
  };

  float total = 0.0f;
  const int nchunks = (nb + CB - 1) / CB;
  load_chunk(0);
  if (!routing) {
    stage_act();
    __syncthreads();
  }
  for (int ch = 0; ch < nchunks; ch++) {
    const int b0 = ch * CB;
    const int bend = min(nb, b0 + CB);
    float(*tb)[GROUP] = terms[ch & 1];
    // Terms in groups of four blocks; each group's registers take the next
    // chunk's loads as soon as its terms are done.  The scheduling barriers
    // keep the activation reads of one group live at a time, so the kernel
    // keeps few VGPRs (83-134: two work-groups per CU).
    float tv[UPW];
    const bool more = ch + 1 < nchunks;
#pragma unroll
    for (int s0 = 0; s0 < UPW; s0 += 4) {
#pragma unroll
      for (int s = s0; s < s0 + 4; s++)
        tv[s] = block_term<DT>(cw[s], sw[s], act + min(b0 + wave + NW * s, nb - 1));
#pragma unroll
      for (int s = s0; s < s0 + 4; s++) asm volatile("" : "+v"(tv[s]));  // computed here, not at the store
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
#pragma unroll
        for (int s = s0; s < s0 + 4; s++) load_block(ch + 1, s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // Rows past the end of the row's blocks take the clamped terms and are
    // never folded; an unconditional store keeps each term's computation
    // where it is written (a conditional one would be sunk into the store's
    // branch, keeping every input live until then).
#pragma unroll
    for (int s = 0; s < UPW; s++) tb[wave + NW * s][lane] = tv[s];
    __syncthreads();
    if (wave == 0) total = lds_sum_strided<GROUP>(&tb[0][lane], bend - b0, total);
  }
  if (wave != 0) return;

  if constexpr (EPI == EPI_PLAIN) {
    size_t row = tile * TILE + r;
    if (row < (size_t)a.rows) a.out[row] = total;
  } else if constexpr (EPI == EPI_GATE_UP) {
    float u = __shfl(total, lane + 32);
    float h = wave_silu(total, tab) * u;  // lanes 0-31: *g = silu(*g) * u
    float scale;
    int qsum;
    int q = quant_block_lane(h, &scale, &qsum);
    if (lane < 32) {
      ActBlock* hb = a.hact + (size_t)slot * a.hact_stride + g;
      hb->q[lane] = (int8_t)q;
      if (lane == 0) {
        hb->scale = scale;
        hb->qsum = qsum;
      }
    }
  }
}

// ===========================================================================
// Down projection and combine in one work-group per row group
// ===========================================================================
//
// MoeLayer::forward (src/model/moe.rs:63-68) for one token: out = 0, then
// for each route in best-first order out = out + w_s * down_s(h_s).  A
// work-group owns DR = 8 output rows for every slot, so the combine needs no
// other work-group, and the launch has H / 8 work-groups (256 at H = 2048).
// Its units are the (slot, block) pairs in slot-major order.  One wave-load
// covers 8 units x 8 rows: 8 segments of 128 B, each one cache line of the
// tile layout.  A chunk of CB units is loaded at once (UPW loads in flight
// per lane) together with its activation blocks; terms go to LDS.  The fold
// runs on 64 lanes, one per (row, slot): each adds its slot's block terms in
// block order, which is the reference's per-expert dot product, and the
// combine then takes the slots in route order.

// u / n for 0 <= u < 2^20 from a float reciprocal, corrected to the exact
// quotient (below 2^20 the float estimate is off by at most one)
__device__ __forceinline__ int div_small(int u, int n, float inv_n) {
  int q = (int)((float)u * inv_n);
  if (q * n > u) q--;
  else if ((q + 1) * n <= u) q++;
  return q;
}

constexpr int DR = DOWN_ROWS;   // rows per work-group of k_down_combine
// Waves per work-group of k_down_combine: 8 when the row groups fit the
// CUs one work-group each (the terms after the loads land are spread over
// twice the waves: 7.4 -> 6.2 us at H 2048), else 4, which keeps two
// work-groups per CU (8 waves need 167 VGPRs: at H 4096, 512 row groups
// would run in two rounds).
constexpr int DOWN_MAX_SLOTS = 64;

template <int DT, int NW>
__global__ __launch_bounds__(64 * NW) void k_down_combine(DownArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int J = 64 / DR;        // units side by side in one wave-load
  constexpr int UPW = 64 / NW / CH;  // loads of 16 B in flight per lane
  constexpr int CB = NW * J * UPW;   // units per chunk: 512 (q4_0), 256 (q8_0)
  static_assert(UPW % 4 == 0, "terms go in groups of four wave-loads");
  constexpr int AQ = (CB * 3 + 64 * NW - 1) / (64 * NW);
  constexpr int SPL = DOWN_MAX_SLOTS / 8;  // slots per fold lane
  // terms of row r at [r][unit]: a fold lane reads its slot's terms from
  // consecutive addresses (16-byte reads, several in flight); the row pitch
  // CB + 8 puts the 64 lanes of a term store in distinct banks
  __shared__ __attribute__((aligned(16))) float terms[DR][CB + 8];
  __shared__ ActBlock s_act[CB];
  __shared__ float s_tot[DOWN_MAX_SLOTS][DR];
  __shared__ int s_exp[DOWN_MAX_SLOTS];
  __shared__ float s_w[DOWN_MAX_SLOTS];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  const int nb = a.nb;
  const int slots = a.slots;
  const int nunits = slots * nb;
  const float inv_nb = 1.0f / (float)nb;
  if (threadIdx.x < slots) {
    s_exp[threadIdx.x] = a.route_idx[threadIdx.x];
    s_w[threadIdx.x] = a.route_w[threadIdx.x];
  }

  const int r = lane % DR;          // row within the group
  const int jl = lane / DR;         // unit within the wave-load
  // The four 8-row groups of a 32-row tile share its scale lines; work-group
  // g runs on XCD g % 8, so when the grid is a multiple of 32 the groups of
  // one tile get ids of one residue class: XCD x takes tiles x, x + 8, ...
  // (all four groups of each), a permutation of the row groups.
  size_t row0 = (size_t)g * DR;
  if ((gridDim.x & 31) == 0) {
    const int gx = g & 7, gj = g >> 3;
    row0 = (size_t)(gx + 8 * (gj >> 2)) * TILE + (size_t)(gj & 3) * DR;
  }
  const size_t tile = row0 / TILE;
  const int rt = (int)(row0 % TILE) + r;  // row within its 32-row tile
  const size_t row_off = (tile * nb * CH * TILE + rt) * 16;
  const size_t srow_off = tile * nb * TILE + rt;

  u32x4 cw[UPW][CH];
  uint16_t sw[UPW];
  u32x4 av[AQ];
  // unit of load s in the chunk at u0 (past the end: clamped to the last
  // unit, loaded and never stored)
  auto unit_of = [&](int u0, int s) { return min(u0 + (s * NW + wave) * J + jl, nunits - 1); };
  // wave-load s of the chunk at u0 holds at least one unit (wave-uniform)
  auto live = [&](int u0, int s) { return (s * NW + wave) * J < nunits - u0; };
  // The expert of each lane's unit comes from LDS; the lookups of a batch of
  // wave-loads are issued together (and pinned there) before its loads.
  int ex[UPW];
  auto lookup = [&](int u0, int s0, int n) {
#pragma unroll
    for (int s = s0; s < s0 + n; s++) ex[s] = s_exp[div_small(unit_of(u0, s), nb, inv_nb)];
#pragma unroll
    for (int s = s0; s < s0 + n; s++) asm volatile("" : "+v"(ex[s]));
  };
  auto load_unit = [&](int u0, int s) {
    const int u = unit_of(u0, s);
    const int sl = div_small(u, nb, inv_nb), b = u - sl * nb;
    const size_t e = (size_t)ex[s];
    const uint8_t* c0 = a.codes + e * a.codes_stride + row_off;
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[s][c] = __builtin_nontemporal_load((const u32x4*)(c0 + ((size_t)b * CH + c) * TILE * 16));
    sw[s] = a.scales[e * a.scales_stride + srow_off + (size_t)b * TILE];
  };
  auto load_act = [&](int u0) {
#pragma unroll
    for (int q = 0; q < AQ; q++) {
      const int i = threadIdx.x + q * 64 * NW;
      const int u = u0 + i / 3;
      if (i < CB * 3 && u < nunits) {
        const int sl = div_small(u, nb, inv_nb), b = u - sl * nb;
        av[q] = ((const u32x4*)(a.hact + (size_t)sl * a.hact_stride + b))[i % 3];
      }
    }
  };

  // fold lane (row r, slot group jl): slots jl, jl + 8, ...; running sums of
  // the current slot are kept per slot because a chunk may end mid-slot
  float tot[SPL];
#pragma unroll
  for (int i = 0; i < SPL; i++) tot[i] = 0.0f;

  load_act(0);      // the activation blocks do not depend on the routes
  __syncthreads();  // s_exp / s_w
  lookup(0, 0, UPW);
#pragma unroll
  for (int s = 0; s < UPW; s++)
    if (live(0, s)) load_unit(0, s);
  for (int u0 = 0; u0 < nunits; u0 += CB) {
#pragma unroll
    for (int q = 0; q < AQ; q++) {
      const int i = threadIdx.x + q * 64 * NW;
      if (i < CB * 3 && u0 + i / 3 < nunits) ((u32x4*)s_act)[i] = av[q];
    }
    __syncthreads();
    // Terms in groups of four wave-loads; each group's registers take the
    // next chunk's loads as soon as its terms are done (the asm statements
    // and scheduling barriers keep that order and the register count low).
    const bool more = u0 + CB < nunits;
    float tv[UPW];
#pragma unroll
    for (int s0 = 0; s0 < UPW; s0 += 4) {
#pragma unroll
      for (int s = s0; s < s0 + 4; s++)
        if (live(u0, s)) tv[s] = block_term<DT>(cw[s], sw[s], s_act + (unit_of(u0, s) - u0));
#pragma unroll
      for (int s = s0; s < s0 + 4; s++)
        if (live(u0, s)) asm volatile("" : "+v"(tv[s]));
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
        lookup(u0 + CB, s0, 4);
#pragma unroll
        for (int s = s0; s < s0 + 4; s++)
          if (live(u0 + CB, s)) load_unit(u0 + CB, s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (more) load_act(u0 + CB);
    // (s * NW + wave) * J + jl < CB: every store is in the chunk; units past
    // the end of a live wave-load hold clamped terms that the fold never reads
#pragma unroll
    for (int s = 0; s < UPW; s++)
      if (live(u0, s)) terms[r][(s * NW + wave) * J + jl] = tv[s];
    __syncthreads();
    if (wave == 0) {
      const int uend = min(nunits, u0 + CB);
#pragma unroll
      for (int i = 0; i < SPL; i++) {
        const int sl = jl + 8 * i;
        if (sl < slots) {
          // this slot's units inside the chunk, in block order
          const int ua = max(u0, sl * nb), ub = min(uend, (sl + 1) * nb);
          if (ub > ua) tot[i] = lds_sum_in_order(&terms[r][ua - u0], ub - ua, tot[i]);
        }
      }
    }
    __syncthreads();  // terms and s_act are rewritten by the next chunk
  }
  if (wave != 0) return;
#pragma unroll
  for (int i = 0; i < SPL; i++) {
    const int sl = jl + 8 * i;
    if (sl < slots) s_tot[sl][r] = tot[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < DR) {
    float acc = 0.0f;  // out.fill(0.0), then out = out + w * y in route order
    for (int sl = 0; sl < slots; sl++) acc = acc + s_w[sl] * s_tot[sl][lane];
    const size_t row = row0 + lane;
    if (row < (size_t)a.rows) a.out[row] = acc;
  }
}

// Per-block i32 sums of every row (the `isum` of dot_q8_0 / dot_q4_0), one
// thread per (row, block).  Parity instrumentation, not a hot path.
template <int DT>
__global__ __launch_bounds__(256) void k_block_sums(const uint8_t* __restrict__ codes,
                                                    const ActBlock* __restrict__ act, size_t rows,
                                                    int nb, int32_t* __restrict__ isums) {
  constexpr int CH = Layout<DT>::CH;
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= rows * (size_t)nb) return;
  size_t row = id / nb;
  int b = (int)(id % nb);
  size_t tile = row / TILE;
  int r = (int)(row % TILE);
  u32x4 c[2] = {};
  for (int ci = 0; ci < CH; ci++)
    c[ci] = *(const u32x4*)(codes + (((tile * nb + b) * CH + ci) * TILE + r) * 16);
  isums[id] = block_isum<DT>(c, act + b);
}

// Counter-based N(mean, std^2) generator for synthetic inputs: splitmix64 of
// (seed, pair index) gives two uniforms, Box-Muller gives two normals.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_fill_normal(float* __restrict__ out, size_t n, uint64_t seed,
                                                     float mean, float std) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t j = 2 * i;
  if (j >= n) return;
  uint64_t h = splitmix64(seed * 0xD1342543DE82EF95ull + i);
  float u1 = (float)((uint32_t)(h >> 40) + 1u) * 0x1p-24f;  // (0, 1]
  float u2 = (float)((uint32_t)(h >> 8) & 0xffffffu) * 0x1p-24f;
  float r = sqrtf(-2.0f * logf(u1));
  float sn, cs;
  sincosf(6.28318530717958647692f * u2, &sn, &cs);
  out[j] = mean + std * (r * cs);
  if (j + 1 < n) out[j + 1] = mean + std * (r * sn);
}

__global__ void k_fill(float* __restrict__ p, size_t n, float v) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// dst[i] = src[i] for n16 16-byte units: one read and one write of every
// byte, the yardstick for the HBM traffic counters
__global__ __launch_bounds__(256) void k_copy(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                              size_t n16) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// ===========================================================================
// Launchers
// ===========================================================================

static inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_repack(int dtype, const uint8_t* aos, size_t rows, size_t cols, uint8_t* codes,
                         uint16_t* scales, hipStream_t st) {
  int nb = (int)(cols / QK);
  size_t prow = padded_rows(rows);
  size_t n = prow * nb;
  if (n == 0) return hipSuccess;
  if (dtype == Q8_0) return launch(k_repack<Q8_0>, blocks_for(n, 256), 256, 0, st, aos, rows, nb, prow, codes, scales);
  return launch(k_repack<Q4_0>, blocks_for(n, 256), 256, 0, st, aos, rows, nb, prow, codes, scales);
}

hipError_t launch_unpack(int dtype, const uint8_t* codes, const uint16_t* scales, size_t rows,
                         size_t cols, uint8_t* aos, hipStream_t st) {
  int nb = (int)(cols / QK);
  size_t n = rows * nb;
  if (n == 0) return hipSuccess;
  if (dtype == Q8_0) return launch(k_unpack<Q8_0>, blocks_for(n, 256), 256, 0, st, codes, scales, rows, nb, aos);
  return launch(k_unpack<Q4_0>, blocks_for(n, 256), 256, 0, st, codes, scales, rows, nb, aos);
}

hipError_t launch_encode(int dtype, const float* values, size_t nblocks, uint8_t* out,
                         hipStream_t st) {
  if (nblocks == 0) return hipSuccess;
  if (dtype == Q8_0) return launch(k_encode<Q8_0>, blocks_for(nblocks, 256), 256, 0, st, values, nblocks, out);
  return launch(k_encode<Q4_0>, blocks_for(nblocks, 256), 256, 0, st, values, nblocks, out);
}

hipError_t launch_act_quant(const float* x, size_t nblocks, ActBlock* act, hipStream_t st) {
  if (nblocks == 0) return hipSuccess;
  if ((uintptr_t)x % 16)
    return launch(k_act_quant_any, blocks_for(nblocks * 32, 256), 256, 0, st, x, nblocks, act);
  return launch(k_act_quant, blocks_for(nblocks * 8, 256), 256, 0, st, x, nblocks, act);
}

hipError_t launch_route_logits(const float* router, const float* x, int H, int E, int T,
                               ActBlock* act, float* logits, hipStream_t st) {
  if (H > ROUTE_MAX_H || E > ROUTE_MAX_E || H % QK || E < 1 || T < 1) return hipErrorInvalidValue;
  dim3 grid(E, T);
  return launch(k_route_logits, grid, ROUTE_THREADS, 0, st, router, x, H, E, act, logits);
}

hipError_t launch_route_select(const float* logits, int E, int k, int normalize, int T,
                               int* route_idx, float* route_w, unsigned long long* stats,
                               hipStream_t st) {
  if (E > ROUTE_MAX_E || k > 64 || k > E || k < 1 || T < 1) return hipErrorInvalidValue;
  return launch(k_route_select, T, 64, 0, st, logits, E, k, normalize, route_idx, route_w, stats);
}

hipError_t launch_gemv(int dtype, int epi, const GemvArgs& a, int groups, int slots,
                       hipStream_t st) {
  if (groups == 0 || slots == 0) return hipSuccess;
  if (a.nb < 1 || a.nb > GEMV_MAX_NB) return hipErrorInvalidValue;
  if (a.logits && (epi != EPI_GATE_UP || a.E > ROUTE_MAX_E || slots > 64 || slots > a.E))
    return hipErrorInvalidValue;
  dim3 grid(groups, slots);
#define HALE_GEMV_CASE(D, E, W)                               \
  if (dtype == D && epi == E) {                               \
    return launch(k_gemv<D, E, W>, grid, 64 * W, 0, st, a);   \
  }
  HALE_GEMV_CASE(Q8_0, EPI_PLAIN, 4)
  HALE_GEMV_CASE(Q8_0, EPI_GATE_UP, 8)
  HALE_GEMV_CASE(Q4_0, EPI_PLAIN, 4)
  if (a.nb <= 64) HALE_GEMV_CASE(Q4_0, EPI_GATE_UP, 16)
  HALE_GEMV_CASE(Q4_0, EPI_GATE_UP, 8)
#undef HALE_GEMV_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_down_combine(int dtype, const DownArgs& a, hipStream_t st) {
  const unsigned groups = (unsigned)(padded_rows((size_t)a.rows) / DR);
  if (groups == 0) return hipSuccess;
  if (a.nb < 1 || a.slots < 1 || a.slots > DOWN_MAX_SLOTS) return hipErrorInvalidValue;
  // CUs of the current device, looked up once per device
  static std::atomic<int> cu_count[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  int cus = dev < 64 ? cu_count[dev].load(std::memory_order_relaxed) : 0;
  if (cus == 0) {
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    if (dev < 64) cu_count[dev].store(cus, std::memory_order_relaxed);
  }
  if (groups <= (unsigned)cus) {
    if (dtype == Q8_0) return launch(k_down_combine<Q8_0, 8>, groups, 512, 0, st, a);
    if (dtype == Q4_0) return launch(k_down_combine<Q4_0, 8>, groups, 512, 0, st, a);
  }
  if (dtype == Q8_0) return launch(k_down_combine<Q8_0, 4>, groups, 256, 0, st, a);
  if (dtype == Q4_0) return launch(k_down_combine<Q4_0, 4>, groups, 256, 0, st, a);
  return hipErrorInvalidValue;
}

hipError_t launch_block_sums(int dtype, const uint8_t* codes, const ActBlock* act, size_t rows,
                             size_t cols, int32_t* isums, hipStream_t st) {
  int nb = (int)(cols / QK);
  size_t n = rows * nb;
  if (n == 0) return hipSuccess;
  if (dtype == Q8_0) return launch(k_block_sums<Q8_0>, blocks_for(n, 256), 256, 0, st, codes, act, rows, nb, isums);
  return launch(k_block_sums<Q4_0>, blocks_for(n, 256), 256, 0, st, codes, act, rows, nb, isums);
}

hipError_t launch_fill_normal(float* p, size_t n, uint64_t seed, float mean, float std,
                              hipStream_t st) {
  if (n == 0) return hipSuccess;
  return launch(k_fill_normal, blocks_for((n + 1) / 2, 256), 256, 0, st, p, n, seed, mean, std);
}

hipError_t launch_fill(float* p, size_t n, float v, hipStream_t st) {
  if (n == 0) return hipSuccess;
  return launch(k_fill, blocks_for(n, 256), 256, 0, st, p, n, v);
}

hipError_t launch_copy(void* dst, const void* src, size_t n16, hipStream_t st) {
  if (!n16) return hipSuccess;
  const unsigned grid = (unsigned)std::min<size_t>(blocks_for(n16, 256), 256 * 64);
  return launch(k_copy, grid, 256, 0, st, (u32x4*)dst, (const u32x4*)src, n16);
}

}  // namespace hale
