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

// x [ntok][n] -> act [ntok][n/32]; each 32-lane group quantizes one block.
__global__ __launch_bounds__(256) void k_act_quant(const float* __restrict__ x, size_t nblocks,
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

// ===========================================================================
// Router: MoeLayer::route (src/model/moe.rs:36-53)
// ===========================================================================
//
// grid (gx, T), 64 threads.  With a router matrix gx == E and work-group e
// computes logit e of token t with the 8-lane f32 order of dot_f32
// (quant.rs:37-41,152-194); otherwise the logits are given and gx == 1.
// Every work-group also quantizes a share of token t's activation blocks.
// The last work-group of a token (counter) runs softmax, top-k and the
// renormalisation in one wave and resets the counter for the next launch.

constexpr int ROUTE_MAX_H = 8192;
constexpr int ROUTE_MAX_E = 1024;

__global__ __launch_bounds__(64) void k_route(const float* __restrict__ router,
                                              const float* __restrict__ logits_in,
                                              const float* __restrict__ x, int H, int E, int k,
                                              int normalize, ActBlock* __restrict__ act,
                                              float* __restrict__ logits, unsigned* counters,
                                              int* __restrict__ route_idx,
                                              float* __restrict__ route_w,
                                              unsigned long long* __restrict__ stats) {
  __shared__ __attribute__((aligned(16))) float prod[ROUTE_MAX_H + 32];  // products, chain-major
  __shared__ float sm[ROUTE_MAX_E];
  __shared__ int last_flag;
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  const int gx = gridDim.x;
  const int e = blockIdx.x;
  const float* xt = x + (size_t)t * H;
  const int nb = H / QK;

  // ---- activation quantization share: half-wave h takes block 2*(e+gx*i)+h
  for (int bb = 2 * e + (lane >> 5); bb < nb; bb += 2 * gx) {
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

  if (router != nullptr) {
    // ---- logit e: 8 accumulators, acc[l] += w[8i+l]*x[8i+l] in order of i
    const float* w = router + (size_t)e * H;
    const int steps = H / 8;
    const int stride = steps + 4;  // keeps 16 B alignment, spreads banks
    for (int i = lane; i < steps * 8; i += 64) prod[(i & 7) * stride + (i >> 3)] = w[i] * xt[i];
    __syncthreads();
    float acc = 0.0f;
    if (lane < 8) {
      const float* p = prod + lane * stride;
      int s = 0;
      for (; s + 4 <= steps; s += 4) {
        f32x4 q = *(const f32x4*)(p + s);
        acc = acc + q.x;
        acc = acc + q.y;
        acc = acc + q.z;
        acc = acc + q.w;
      }
      for (; s < steps; s++) acc = acc + p[s];
    }
    float a0 = __shfl(acc, 0), a1 = __shfl(acc, 1), a2 = __shfl(acc, 2), a3 = __shfl(acc, 3);
    float a4 = __shfl(acc, 4), a5 = __shfl(acc, 5), a6 = __shfl(acc, 6), a7 = __shfl(acc, 7);
    if (lane == 0) {
      float tail = -0.0f;  // Iterator::sum over the H % 8 leftover products
      for (int i = steps * 8; i < H; i++) tail = tail + w[i] * xt[i];
      float s0 = (a0 + a4) + (a1 + a5);
      float s1 = (a2 + a6) + (a3 + a7);
      logits[(size_t)t * E + e] = (s0 + s1) + tail;
    }
  }

  // ---- completion: the last work-group of token t continues
  const float* lg = logits_in ? logits_in + (size_t)t * E : logits + (size_t)t * E;
  if (gx > 1) {
    __threadfence();
    if (lane == 0) last_flag = (atomicAdd(&counters[t], 1u) == (unsigned)(gx - 1));
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    if (lane == 0) counters[t] = 0u;
  } else {
    __threadfence();
    __syncthreads();  // lane 0's logit store is visible to the whole group
  }

  // ---- softmax_in_place (src/ops/activation.rs:11-21)
  float mx = -__builtin_huge_valf();
  for (int i = lane; i < E; i += 64) {
    float v = __builtin_nontemporal_load(lg + i);
    sm[i] = v;
    mx = fmaxf(mx, v);
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  __syncthreads();
  for (int i = lane; i < E; i += 64) sm[i] = hale_expf(sm[i] - mx);
  __syncthreads();
  float sum = 0.0f;
  if (lane == 0)
    for (int i = 0; i < E; i++) sum = sum + sm[i];
  sum = __shfl(sum, 0);
  for (int i = lane; i < E; i += 64) sm[i] = sm[i] / sum;
  __syncthreads();

  // ---- top_k (src/ops/topk.rs:44-61): best total_cmp score, ties to lower index
  unsigned long long taken = 0;  // bit m: element lane + 64*m already chosen
  float norm = -0.0f;
  float chosen_score = 0.0f;
  int chosen_idx = 0;
  for (int r = 0; r < k; r++) {
    int bk = (int)0x80000000u, bi = 0x7fffffff;
    for (int m = 0, i = lane; i < E; m++, i += 64) {
      if (taken >> m & 1ull) continue;
      int key = total_key(sm[i]);
      if (key > bk || (key == bk && i < bi)) {
        bk = key;
        bi = i;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      int ok = __shfl_xor(bk, o), oi = __shfl_xor(bi, o);
      if (ok > bk || (ok == bk && oi < bi)) {
        bk = ok;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1ull << (bi >> 6);
    float sc = sm[bi];
    if (lane == r) {
      chosen_idx = bi;
      chosen_score = sc;
    }
    norm = norm + sc;  // Iterator::sum in best-first order (every lane)
  }
  if (!normalize) norm = 1.0f;
  if (lane < k) {
    route_idx[(size_t)t * k + lane] = chosen_idx;
    route_w[(size_t)t * k + lane] = chosen_score / norm;
    if (stats) atomicAdd(&stats[chosen_idx], 1ull);
  }
}

// ===========================================================================
// Exact tile GEMV
// ===========================================================================
//
// A work-group of 4 waves owns a group of 64 output rows (two 32-row tiles)
// and loops over the row's quantization blocks: wave w takes blocks
// w, w+4, w+8, ...  For one block a wave reads 2 x 512 B of codes (q4_0)
// or 2 x 1 KB (q8_0), all lanes use the same activation block (scalar
// loads), and lane l produces the term (d_w * d_x) * isum of row l.  Terms
// go to LDS in chunks of CB blocks; wave 0 folds each chunk into its 64
// running row sums in block order, so the total is the reference's
// left-to-right sum.  Two LDS buffers let the other waves fill chunk c+1
// while wave 0 folds chunk c.
//
// Epilogues:
//   EPI_PLAIN    out[row] = total                      (WeightMatrix::matvec)
//   EPI_GATE_UP  rows 0-31 gate, 32-63 up of one I-tile; h = silu(g)*u is
//                quantized to its q8 block for the down projection
//                (Expert::forward, src/expert/mod.rs:95-102)
//   EPI_COMBINE  per-slot results to ytmp; the last slot's work-group of the
//                row group adds them in route order: out = 0, then
//                out = out + w_s * y_s (MoeLayer::forward, moe.rs:63-68)

constexpr int CB = 32;  // blocks per LDS chunk

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

template <int DT, int EPI>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
  constexpr int CH = Layout<DT>::CH;
  __shared__ float terms[2][CB][GROUP];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  const int slot = blockIdx.y;
  const int nb = a.nb;
  const int expert = a.route_idx ? a.route_idx[slot] : 0;

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
  const ActBlock* act = a.act + (size_t)slot * a.act_stride;

  float total = 0.0f;
  const int nchunks = (nb + CB - 1) / CB;
  for (int ch = 0; ch < nchunks; ch++) {
    const int b0 = ch * CB;
    const int bend = min(nb, b0 + CB);
    float(*tb)[GROUP] = terms[ch & 1];
    // issue every load of this wave's share of the chunk, then compute
    u32x4 cw[CB / 4][CH];
    uint16_t sw[CB / 4];
#pragma unroll
    for (int s = 0; s < CB / 4; s++) {
      const int b = b0 + wave + 4 * s;
      if (b < bend) {
#pragma unroll
        for (int c = 0; c < CH; c++)
          cw[s][c] = __builtin_nontemporal_load((const u32x4*)(crow + ((size_t)b * CH + c) * TILE * 16));
        sw[s] = srow[(size_t)b * TILE];
      }
    }
#pragma unroll
    for (int s = 0; s < CB / 4; s++) {
      const int b = b0 + wave + 4 * s;
      if (b < bend) tb[b - b0][lane] = block_term<DT>(cw[s], sw[s], act + b);
    }
    __syncthreads();
    if (wave == 0)
      for (int b = 0; b < bend - b0; b++) total = total + tb[b][lane];
  }
  if (wave != 0) return;

  if constexpr (EPI == EPI_PLAIN) {
    size_t row = tile * TILE + r;
    if (row < (size_t)a.rows) a.out[row] = total;
  } else if constexpr (EPI == EPI_GATE_UP) {
    float u = __shfl(total, lane + 32);
    float h = silu(total) * u;  // lanes 0-31: *g = silu(*g) * u
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
  } else {  // EPI_COMBINE
    const size_t prow = padded_rows((size_t)a.rows);
    const size_t row = tile * TILE + r;
    a.ytmp[(size_t)slot * prow + row] = total;
    __threadfence();
    unsigned old = 0;
    if (lane == 0) old = atomicAdd(&a.counters[g], 1u);
    old = __shfl(old, 0);
    if (old != (unsigned)(a.slots - 1)) return;
    __threadfence();
    if (lane == 0) a.counters[g] = 0u;
    float acc = 0.0f;
    for (int s = 0; s < a.slots; s++)
      acc = acc + a.route_w[s] * __builtin_nontemporal_load(a.ytmp + (size_t)s * prow + row);
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
  if (dtype == Q8_0)
    k_repack<Q8_0><<<blocks_for(n, 256), 256, 0, st>>>(aos, rows, nb, prow, codes, scales);
  else
    k_repack<Q4_0><<<blocks_for(n, 256), 256, 0, st>>>(aos, rows, nb, prow, codes, scales);
  return hipGetLastError();
}

hipError_t launch_unpack(int dtype, const uint8_t* codes, const uint16_t* scales, size_t rows,
                         size_t cols, uint8_t* aos, hipStream_t st) {
  int nb = (int)(cols / QK);
  size_t n = rows * nb;
  if (n == 0) return hipSuccess;
  if (dtype == Q8_0)
    k_unpack<Q8_0><<<blocks_for(n, 256), 256, 0, st>>>(codes, scales, rows, nb, aos);
  else
    k_unpack<Q4_0><<<blocks_for(n, 256), 256, 0, st>>>(codes, scales, rows, nb, aos);
  return hipGetLastError();
}

hipError_t launch_encode(int dtype, const float* values, size_t nblocks, uint8_t* out,
                         hipStream_t st) {
  if (nblocks == 0) return hipSuccess;
  if (dtype == Q8_0)
    k_encode<Q8_0><<<blocks_for(nblocks, 256), 256, 0, st>>>(values, nblocks, out);
  else
    k_encode<Q4_0><<<blocks_for(nblocks, 256), 256, 0, st>>>(values, nblocks, out);
  return hipGetLastError();
}

hipError_t launch_act_quant(const float* x, size_t nblocks, ActBlock* act, hipStream_t st) {
  if (nblocks == 0) return hipSuccess;
  k_act_quant<<<blocks_for(nblocks * 32, 256), 256, 0, st>>>(x, nblocks, act);
  return hipGetLastError();
}

hipError_t launch_route(const float* router, const float* logits_in, const float* x, int H, int E,
                        int k, int normalize, int T, ActBlock* act, float* logits,
                        unsigned* counters, int* route_idx, float* route_w,
                        unsigned long long* stats, hipStream_t st) {
  if (H > ROUTE_MAX_H || E > ROUTE_MAX_E || k > 64 || k > E || H % QK) return hipErrorInvalidValue;
  dim3 grid(router ? E : 1, T);
  k_route<<<grid, 64, 0, st>>>(router, logits_in, x, H, E, k, normalize, act, logits, counters,
                               route_idx, route_w, stats);
  return hipGetLastError();
}

hipError_t launch_gemv(int dtype, int epi, const GemvArgs& a, int groups, int slots,
                       hipStream_t st) {
  if (groups == 0 || slots == 0) return hipSuccess;
  dim3 grid(groups, slots);
#define HALE_GEMV_CASE(D, E)                                  \
  if (dtype == D && epi == E) {                               \
    k_gemv<D, E><<<grid, 256, 0, st>>>(a);                    \
    return hipGetLastError();                                 \
  }
  HALE_GEMV_CASE(Q8_0, EPI_PLAIN)
  HALE_GEMV_CASE(Q8_0, EPI_GATE_UP)
  HALE_GEMV_CASE(Q8_0, EPI_COMBINE)
  HALE_GEMV_CASE(Q4_0, EPI_PLAIN)
  HALE_GEMV_CASE(Q4_0, EPI_GATE_UP)
  HALE_GEMV_CASE(Q4_0, EPI_COMBINE)
#undef HALE_GEMV_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_block_sums(int dtype, const uint8_t* codes, const ActBlock* act, size_t rows,
                             size_t cols, int32_t* isums, hipStream_t st) {
  int nb = (int)(cols / QK);
  size_t n = rows * nb;
  if (n == 0) return hipSuccess;
  if (dtype == Q8_0)
    k_block_sums<Q8_0><<<blocks_for(n, 256), 256, 0, st>>>(codes, act, rows, nb, isums);
  else
    k_block_sums<Q4_0><<<blocks_for(n, 256), 256, 0, st>>>(codes, act, rows, nb, isums);
  return hipGetLastError();
}

hipError_t launch_fill_normal(float* p, size_t n, uint64_t seed, float mean, float std,
                              hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_fill_normal<<<blocks_for((n + 1) / 2, 256), 256, 0, st>>>(p, n, seed, mean, std);
  return hipGetLastError();
}

hipError_t launch_fill(float* p, size_t n, float v, hipStream_t st) {
  if (n == 0) return hipSuccess;
  k_fill<<<blocks_for(n, 256), 256, 0, st>>>(p, n, v);
  return hipGetLastError();
}

}  // namespace hale
