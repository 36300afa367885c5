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
#include <type_traits>
#include <utility>

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
// Decoding: decode_row (src/tensor/quant.rs:236-269), WeightMatrix::to_f32
// ===========================================================================

// half's f16::to_f32 (F16C, fcvtl or its software path alike): exact; a NaN
// keeps its sign and payload and gets the quiet bit.
__device__ __forceinline__ float h2f_quiet(uint16_t h) {
  if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu))
    return __uint_as_float(((unsigned)(h & 0x8000u) << 16) | 0x7fc00000u | ((unsigned)(h & 0x3ffu) << 13));
  return h2f(h);
}

// little-endian u16 from two byte loads (any alignment)
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// decode_row over n values of reference-layout rows laid end to end (a row's
// blocks follow the previous row's, so value i is block i / 32, position
// i % 32 of the run).  One thread per value.  A: the base is aligned to the
// dtype's element or scale size, so values and scales load whole;
// otherwise by bytes, as the reference's unaligned fallback reads them.
template <int DT, bool A>
__global__ __launch_bounds__(256) void k_decode_ref(const uint8_t* __restrict__ src, size_t n,
                                                    float* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float v;
  if constexpr (DT == F32) {
    const uint8_t* p = src + 4 * i;
    const unsigned u = A ? *(const unsigned*)p
                         : (unsigned)p[0] | (unsigned)p[1] << 8 | (unsigned)p[2] << 16 | (unsigned)p[3] << 24;
    v = __uint_as_float(u);
  } else if constexpr (DT == F16) {
    v = h2f_quiet(A ? ((const uint16_t*)src)[i] : ld_u16(src + 2 * i));
  } else if constexpr (DT == BF16) {
    v = __uint_as_float((unsigned)(A ? ((const uint16_t*)src)[i] : ld_u16(src + 2 * i)) << 16);
  } else {
    constexpr int BB = DT == Q8_0 ? 34 : 18;
    const uint8_t* blk = src + (i / QK) * BB;
    const int j = (int)(i % QK);
    const float scale = h2f_quiet(A ? *(const uint16_t*)blk : ld_u16(blk));
    if constexpr (DT == Q8_0) {
      v = scale * (float)(int8_t)blk[2 + j];
    } else {
      const unsigned byte = blk[2 + (j & 15)];
      v = scale * ((float)(j < 16 ? byte & 15u : byte >> 4) - 8.0f);
    }
  }
  out[i] = v;
}

// The same values read from the HBM tile planes: rows row0 .. row0 + nrows - 1
// of a q8_0 / q4_0 matrix into out[nrows][nb * 32].  One thread per value.
template <int DT>
__global__ __launch_bounds__(256) void k_decode_tiles(const uint8_t* __restrict__ codes,
                                                      const uint16_t* __restrict__ scales,
                                                      size_t row0, size_t nrows, int nb,
                                                      float* __restrict__ out) {
  constexpr int CH = Layout<DT>::CH;
  const size_t cols = (size_t)nb * QK;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nrows * cols) return;
  const size_t row = row0 + i / cols;
  const int c = (int)(i % cols), b = c / QK, j = c % QK;
  const size_t tile = row / TILE;
  const int r = (int)(row % TILE);
  const float scale = h2f_quiet(scales[(tile * nb + b) * TILE + r]);
  const uint8_t* piece = codes + (((tile * nb + b) * CH + (CH == 2 ? j / 16 : 0)) * TILE + r) * 16;
  float v;
  if constexpr (DT == Q8_0) {
    v = scale * (float)(int8_t)piece[j % 16];
  } else {
    const unsigned byte = piece[j & 15];
    v = scale * ((float)(j < 16 ? byte & 15u : byte >> 4) - 8.0f);
  }
  out[i] = v;
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

// One q8 block from an aligned group of 8 lanes, lane j holding elements
// 4j..4j+3 as v.  The block maximum and the code sum are order-free (max
// and integer sums), and scale, reciprocal and codes are the expressions of
// quant_block_lane.  All 8 lanes of the group must be active.
__device__ __forceinline__ void quant_block8(f32x4 v, int j, ActBlock* dst) {
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
  *(unsigned*)(dst->q + 4 * j) = (unsigned)(q0 & 0xff) | (unsigned)(q1 & 0xff) << 8 |
                                 (unsigned)(q2 & 0xff) << 16 | (unsigned)(q3 & 0xff) << 24;
  if (j == 0) {
    dst->scale = scale;
    dst->qsum = qs;
  }
}

// The same for 16-byte aligned x; each 8-lane group quantizes one block
// from one 16-byte load per lane.
__global__ __launch_bounds__(256) void k_act_quant(const float* __restrict__ x, size_t nblocks,
                                                   ActBlock* __restrict__ act) {
  const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) / 8;
  const int j = threadIdx.x & 7;
  if (blk >= nblocks) return;  // uniform across the 8-lane group
  quant_block8(*(const f32x4*)(x + blk * QK + 4 * j), j, act + blk);
}

// ===========================================================================
// Router: MoeLayer::route (src/model/moe.rs:36-53)
// ===========================================================================
//
// Two parts.  k_route_logits (grid (E, T), 64 threads) computes logit e of
// token t with the 8-lane f32 order of dot_f32 (quant.rs:37-41,152-194) and
// quantizes a share of token t's activation blocks.  route_select (one
// wave) turns E logits into the top-k experts and their weights.  On the
// decode path the gate/up kernel selects by itself: every work-group ranks
// the logits to find its slot's expert, and one extra work-group runs
// route_select and publishes the routes, so no work-group waits for
// another.  k_route_select runs it for standalone routing and the grouped
// path, one wave per token.

constexpr int ROUTE_MAX_H = 8192;
constexpr int ROUTE_MAX_E = 1024;
constexpr int GEMV_MAX_NB = 512;  // blocks per row the GEMV stages in LDS

constexpr int ROUTE_THREADS = 256;

// VPT: float4 of w (and of x) per thread, so H <= 4 VPT ROUTE_THREADS.  The
// launcher takes the smallest of 2, 4 and 8 that covers H: registers and
// LDS sized for H = 8192 held four work-groups per CU, and a 16-token call
// of a 128-expert layer (2,048 work-groups) then ran in two rounds.
template <int VPT>
__global__ __launch_bounds__(ROUTE_THREADS) void k_route_logits(const float* __restrict__ router,
                                                                const float* __restrict__ x, int H,
                                                                int E, ActBlock* __restrict__ act,
                                                                float* __restrict__ logits) {
  __shared__ __attribute__((aligned(16))) float prod[4 * VPT * ROUTE_THREADS + 32];  // chain-major
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
  f32x4 wv[VPT], xv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; j++) {
    const int c = tid + j * ROUTE_THREADS;
    if (c < nvec) {
      wv[j] = *(const f32x4*)(w + 4 * c);
      xv[j] = *(const f32x4*)(xt + 4 * c);
    }
  }

  // activation quantization share, done by waves 1-3 while wave 0 runs the
  // fold chains: half-wave hw (0..5) of work-group e takes blocks
  // e + gx (hw + 6 i), so the blocks spread over all work-groups (one each
  // while nb <= E) rather than loading the first few; the first block's
  // value loads with the row
  const int hw = (tid >> 5) - 2;
  const int bb0 = e + gx * hw;
  float v0 = 0.0f;
  if (hw >= 0 && bb0 < nb) v0 = xt[bb0 * QK + (lane & 31)];

  // products w[i]*x[i] (each one rounding, order free) into chain-major LDS:
  // chain l holds i = 8s + l at prod[l * stride + s]
  const int stride = steps + 4;  // 16 B aligned rows, chains on distinct banks
#pragma unroll
  for (int j = 0; j < VPT; j++) {
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
  if (tid >= 64) {
    for (int bb = bb0; bb < nb; bb += 6 * gx) {
      const float v = bb == bb0 ? v0 : xt[bb * QK + (lane & 31)];
      float scale;
      int qsum;
      const int q = quant_block_lane(v, &scale, &qsum);
      ActBlock* ab = act + (size_t)t * nb + bb;
      ab->q[lane & 31] = (int8_t)q;
      if ((lane & 31) == 0) {
        ab->scale = scale;
        ab->qsum = qsum;
      }
    }
    return;
  }
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

// The router logits of many tokens (T >= ROUTE_TILED_MIN_T): work-group
// (eg, tg) computes experts RT_E eg .. RT_E eg + RT_E - 1 (RT_E = 16 or 8)
// for tokens 8 tg .. 8 tg + 7, one wave per expert.  Lane 8t + l of wave e
// carries chain l of logit (e, t):
// acc = acc + w_e[8s + l] * x_t[8s + l] in order of s, each product rounded
// before it is added (dot_f32's 8-lane order, quant.rs:152-194).  The
// RT_E + 8 rows (router rows, then tokens) stream through LDS chain-major in chunks
// of RT_K steps, two buffers, so chunk c + 1 loads while chunk c is added,
// and every staged row serves 8 or RT_E logits.  The eight chains of a logit
// are reduced in the one-token kernel's fixed order, so each logit has its
// bits.  Then the work-groups quantize the token tile's activation blocks
// (as k_act_quant does), each taking its share: block q of the tile goes to
// the work-group of expert column q % gridDim.x.
constexpr int RT_T = 8, RT_K = 64;
constexpr int RT_STRIDE = RT_K + 4;                 // floats per chain row (16-byte aligned)
// From 48 tokens.  Against one work-group per (expert, token) sized for
// the row length (eight per CU), per layer, graph replay, row-chain
// grouped path: Qwen3-30B-A3B q4_0 at 32 / 40 / 48 / 64 / 76 tokens 89.1 /
// 95.6 / 102.7 / 112.5 / 120 us with the tiles against 87.0 / 93.9 / 101.9 /
// 114.1 / 122.7 without; Qwen3-235B-A22B at 32 / 48 / 60: 294 / 315 / 352
// against 289 / 316 / 356.
constexpr int ROUTE_TILED_MIN_T = 48;

template <int RT_E>  // experts per work-group: one wave each
__global__ __launch_bounds__(64 * RT_E) void k_route_logits_tiled(const float* __restrict__ router,
                                                                  const float* __restrict__ x, int H,
                                                                  int E, int T,
                                                                  float* __restrict__ logits,
                                                                  ActBlock* __restrict__ act) {
  constexpr int NT = 64 * RT_E;                          // threads
  constexpr int RT_BUF = (RT_E + RT_T) * 8 * RT_STRIDE;  // floats per buffer
  __shared__ __attribute__((aligned(16))) float buf[2][RT_BUF];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int e0 = blockIdx.x * RT_E, t0 = blockIdx.y * RT_T;
  const int steps = H / 8;
  const int nchunk = (steps + RT_K - 1) / RT_K;
  // Chunk c of row r: elements [8 RT_K c, 8 RT_K (c + 1)), 2 RT_K float4;
  // thread q moves float4 pieces q, q + NT, q + 2 NT, ... of the rows.  Rows
  // past E or T repeat the last one and pieces past H the last piece
  // (in-bounds loads; their chains are not written).
  constexpr int PPR = 2 * RT_K;                       // float4 pieces per row and chunk
  constexpr int PPT = (RT_E + RT_T) * PPR / NT;       // pieces per thread
  static_assert((RT_E + RT_T) * PPR % NT == 0, "whole pieces per thread");
  auto load_chunk = [&](f32x4* v, int c) {
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const int idx = tid + NT * j, row = idx / PPR, piece = idx % PPR;
      const float* src = row < RT_E ? router + (size_t)min(e0 + row, E - 1) * H
                                    : x + (size_t)min(t0 + row - RT_E, T - 1) * H;
      const int elem = min(c * 8 * RT_K + 4 * piece, H - 4);
      v[j] = *(const f32x4*)(src + elem);
    }
  };
  auto store_chunk = [&](const f32x4* v, float* b) {
#pragma unroll
    for (int j = 0; j < PPT; j++) {
      const int idx = tid + NT * j, row = idx / PPR, piece = idx % PPR;
      float* r = b + (row * 8 + (piece & 1) * 4) * RT_STRIDE + (piece >> 1);
      r[0] = v[j].x;
      r[RT_STRIDE] = v[j].y;
      r[2 * RT_STRIDE] = v[j].z;
      r[3 * RT_STRIDE] = v[j].w;
    }
  };
  const int t = lane >> 3, l = lane & 7;
  const int wrow = (wave * 8 + l) * RT_STRIDE, xrow = ((RT_E + t) * 8 + l) * RT_STRIDE;
  f32x4 v[PPT];
  load_chunk(v, 0);
  store_chunk(v, buf[0]);
  __syncthreads();
  float acc = 0.0f;
  for (int c = 0; c < nchunk; c++) {
    if (c + 1 < nchunk) load_chunk(v, c + 1);  // in flight while chunk c is added
    const float* b = buf[c & 1];
    const int kc = min(RT_K, steps - c * RT_K);  // a multiple of 4 (H % 32 == 0)
    for (int s4 = 0; s4 < kc; s4 += 4) {
      const f32x4 wv = *(const f32x4*)(b + wrow + s4);
      const f32x4 xv = *(const f32x4*)(b + xrow + s4);
      acc = acc + wv.x * xv.x;
      acc = acc + wv.y * xv.y;
      acc = acc + wv.z * xv.z;
      acc = acc + wv.w * xv.w;
    }
    if (c + 1 < nchunk) store_chunk(v, buf[(c + 1) & 1]);
    __syncthreads();  // chunk c + 1 staged; every wave is done with chunk c
  }
  const int base = lane & ~7;
  const float a0 = __shfl(acc, base + 0), a1 = __shfl(acc, base + 1), a2 = __shfl(acc, base + 2),
              a3 = __shfl(acc, base + 3);
  const float a4 = __shfl(acc, base + 4), a5 = __shfl(acc, base + 5), a6 = __shfl(acc, base + 6),
              a7 = __shfl(acc, base + 7);
  const int e = e0 + wave, tok = t0 + t;
  if (l == 0 && e < E && tok < T) {
    const float tail = -0.0f;  // Iterator::sum over the H % 8 leftover products: none (H % 32 == 0)
    const float s0v = (a0 + a4) + (a1 + a5);
    const float s1v = (a2 + a6) + (a3 + a7);
    logits[(size_t)tok * E + e] = (s0v + s1v) + tail;
  }
  // this work-group's share of the tile's activation blocks, 8 lanes per
  // block, 128 blocks per pass (the bound is uniform per 8-lane group)
  const int nb = H / QK;
  const int nq = min(RT_T, T - t0) * nb;
  for (int q = blockIdx.x + gridDim.x * (tid >> 3); q < nq; q += gridDim.x * (NT / 8)) {
    const int tk = q / nb, b = q - tk * nb;
    const size_t blk = (size_t)(t0 + tk) * nb + b;
    quant_block8(*(const f32x4*)(x + blk * QK + 4 * (tid & 7)), tid & 7, act + blk);
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

constexpr int RS_SCRATCH = ROUTE_MAX_E + 4 * 64;

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

// E <= ME
template <int ME = ROUTE_MAX_E>
__device__ __forceinline__ void route_select(const float* lg, int E, int k, int normalize,
                                             int* sel_idx, float* sel_w, const ExpTable& tab,
                                             float* rs) {
  if (E <= 64)
    route_select_t<1>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (E <= 128)
    route_select_t<2>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (ME <= 256 || E <= 256)
    route_select_t<(ME < 256 ? 2 : 4)>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else if (E <= 512)
    route_select_t<8>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
  else
    route_select_t<16>(lg, E, k, normalize, sel_idx, sel_w, tab, rs);
}

// Selection in the gate/up prologue.
//
// A work-group of slot s needs the expert of rank s in the reference's
// order (probability desc, index asc).  Ranking by logit gives that order
// unless rounding makes two probabilities of different logits equal: the
// map logit -> exp(logit - max) -> probability never swaps two logits but
// may merge them.  So every wave of a work-group, on its own and from
// registers only (no LDS, no barrier), finds X, the element of logit rank s
// (select_slot_by_logit), and checks that no rounding can merge X's
// probability with that of an element of a different logit.  Then X's
// probability rank equals its logit rank, so X is the reference's choice
// for slot s, and the wave issues X's weight loads at once.  Otherwise (a
// near-tie around X, a NaN or an infinity among the logits, all rare) the
// work-group runs the reference's selection first and takes its slot s.
// One work-group of the launch publishes the reference's routes and
// weights for the down projection.

// Selection state in LDS, used only when the logit ranking is not safe.
template <int ME>
struct SelLds {
  float e[ME];        // scratch of route_select
  int sel_idx[64];    // the reference's choice, best first
  float sel_w[64];    // and its renormalised weights
};

// Element X of rank `slot` in (logit total order desc, index asc) among the
// E logits lg (E <= 64 PER), by one whole wave; element i is held by lane
// i % 64 in register i / 64.  The wave walks the distinct order keys from
// the top, one wave maximum per key (each below the last), counting each
// key's elements with ballots, until the count passes `slot`: X then has
// key K, the last one visited, and is the (slot - #keys above K)-th element
// of key K in index order.  At most slot + 2 maxima.  *safe (wave-uniform)
// tells whether X is certainly the reference's choice for this slot:
//   - no logit is NaN (a NaN makes every probability NaN) and the largest,
//     L0, is finite;
//   - L_X - L0 >= -60, and L_X is finite;
//   - the next larger logit a (if any) has a - L_X > 2^-13;
//   - the next smaller logit b (if any) is finite, b - L0 >= -60 and
//     L_X - b > 2^-13.
// For a pair of logits u > v with u - v > 2^-13 (computed in f32), v - L0
// >= -60 and both finite, x = fl(v - L0) errs by at most 2^-18, glibc expf by
// under one ulp and the division by half an ulp, so p_u / p_v >=
// exp(2^-13 - 2^-17)(1 - 3 * 2^-23) > 1.  That orders X strictly against a
// and b and, by the non-decreasing map, against every element beyond them
// (for those below -60 as well: their exp stays below exp(-60)(1 + 2^-23),
// under X's); elements of X's own logit have X's probability and keep index
// order.  So the probability rank of X is its logit rank.
template <int PER>
__device__ __forceinline__ int select_slot_by_logit(const float* __restrict__ lg, int E, int slot,
                                                    bool* safe) {
  const int lane = threadIdx.x & 63;
  unsigned key[PER];
  bool has[PER];
  bool nan = false;
#pragma unroll
  for (int m = 0; m < PER; m++) {
    const int i = lane + 64 * m;
    has[m] = i < E;
    const float v = has[m] ? lg[i] : 0.0f;
    key[m] = order_key(v);
    nan = nan || (has[m] && v != v);
  }
  // the largest key below `bound` (any key when `all`), 0 when there is none
  auto max_below = [&](unsigned bound, bool all) {
    unsigned loc = 0u;
#pragma unroll
    for (int m = 0; m < PER; m++)
      if (has[m] && (all || key[m] < bound)) loc = max(loc, key[m]);
    return wave_max_u32(loc);
  };
  auto count_eq = [&](unsigned k) {
    int c = 0;
#pragma unroll
    for (int m = 0; m < PER; m++) c += (int)__popcll(__ballot(has[m] && key[m] == k));
    return c;
  };
  const unsigned top = max_below(0u, true);
  unsigned K = top, above = 0u;
  int n_above = 0;  // elements with keys above K
  bool ok = true;
  for (int it = 0;; it++) {
    const int c = count_eq(K);
    if (n_above + c > slot) break;
    if (it > slot) {  // cannot happen with E > slot; keeps the loop bounded
      ok = false;
      break;
    }
    n_above += c;
    above = K;
    K = max_below(K, false);
  }
  int j = slot - n_above;  // X's place among the elements of key K
  int x = 0;
  bool found = false, any_below = false;
#pragma unroll
  for (int m = 0; m < PER; m++) {
    unsigned long long eq = __ballot(has[m] && key[m] == K);
    const int c = (int)__popcll(eq);
    if (!found) {
      if (j < c) {
        for (int q = 0; q < j; q++) eq &= eq - 1;
        x = 64 * m + (int)__builtin_ctzll(eq);
        found = true;
      } else {
        j -= c;
      }
    }
    any_below = any_below || __ballot(has[m] && key[m] < K) != 0ull;
  }
  const float l0 = key_value(top), lx = key_value(K);
  ok = ok && found && __ballot(nan) == 0ull && fabsf(l0) <= 3.0e38f && fabsf(lx) <= 3.0e38f &&
       lx - l0 >= -60.0f;
  if (n_above > 0) ok = ok && key_value(above) - lx > 0x1p-13f;
  if (any_below) {
    const float lb = key_value(max_below(K, false));
    ok = ok && fabsf(lb) <= 3.0e38f && lb - l0 >= -60.0f && lx - lb > 0x1p-13f;
  }
  *safe = ok;
  return __builtin_amdgcn_readfirstlane(x);
}

// E <= ME
template <int ME>
__device__ __forceinline__ int select_slot(const float* lg, int E, int slot, bool* safe) {
  if (E <= 64) return select_slot_by_logit<1>(lg, E, slot, safe);
  if (E <= 128) return select_slot_by_logit<2>(lg, E, slot, safe);
  if (ME <= 256 || E <= 256) return select_slot_by_logit<(ME < 256 ? 2 : 4)>(lg, E, slot, safe);
  return select_slot_by_logit<ME / 64>(lg, E, slot, safe);
}

// Standalone routing (MoeLayer::route without the experts, and the grouped
// path): one wave per token.
__device__ __forceinline__ void route_select_token(const float* __restrict__ logits, int E, int k,
                                                   int normalize, int t, int* __restrict__ route_idx,
                                                   float* __restrict__ route_w,
                                                   unsigned long long* __restrict__ stats) {
  __shared__ int sel_idx[64];
  __shared__ float sel_w[64];
  __shared__ __attribute__((aligned(16))) float rs[RS_SCRATCH];
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

__global__ __launch_bounds__(64) void k_route_select(const float* __restrict__ logits, int E, int k,
                                                     int normalize, int* __restrict__ route_idx,
                                                     float* __restrict__ route_w,
                                                     unsigned long long* __restrict__ stats) {
  route_select_token(logits, E, k, normalize, blockIdx.x, route_idx, route_w, stats);
}

// The routes of T tokens from given logits and the quantization of their
// activations in one launch (the two are independent): work-groups 0..T-1
// select token t's routes as k_route_select does, the others quantize 8
// activation blocks each as k_act_quant does (x 16-byte aligned).
__global__ __launch_bounds__(64) void k_route_select_quant(const float* __restrict__ logits, int E,
                                                           int k, int normalize, int T,
                                                           int* __restrict__ route_idx,
                                                           float* __restrict__ route_w,
                                                           const float* __restrict__ x,
                                                           size_t nblocks,
                                                           ActBlock* __restrict__ act) {
  const int g = blockIdx.x;
  if (g >= T) {  // work-group-uniform
    const size_t blk = (size_t)(g - T) * 8 + (threadIdx.x >> 3);
    const int j = threadIdx.x & 7;
    if (blk < nblocks) quant_block8(*(const f32x4*)(x + blk * QK + 4 * j), j, act + blk);
    return;
  }
  route_select_token(logits, E, k, normalize, g, route_idx, route_w, nullptr);
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
//                logits given, the prologue selects the slot's expert; grid
//                row y is slot y % k of token y / k when several tokens are
//                decoded in one launch.

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
// pipeline worse) when the layer has at most 256 experts.
// NT: non-temporal weight loads (ordinary ones when many tokens share the
// experts).
template <int DT, int EPI, int NW, int ME = 256, bool NT = true>  // ME: most experts the routed form selects among
__global__ __launch_bounds__(64 * NW) void k_gemv(GemvArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int UPW = 64 / NW / CH;      // blocks per wave per chunk (64 / NW loads in flight)
  constexpr int CB = UPW * NW;           // blocks per chunk
  static_assert(UPW % 4 == 0, "terms go in groups of four blocks");
  __shared__ float terms[2][CB][GROUP];
  __shared__ ActBlock s_act[GEMV_MAX_NB];
  struct NoSel {};
  __shared__ __attribute__((aligned(16)))
  typename std::conditional<EPI == EPI_GATE_UP, SelLds<ME>, NoSel>::type sel;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  // grid row y: slot y % slots of token y / slots (one token: slot y)
  const int tok = a.tokens > 1 ? (int)blockIdx.y / a.slots : 0;
  const int slot = (int)blockIdx.y - tok * a.slots;
  if (tok > 0) {
    a.act += (size_t)tok * a.act_tstride;
    a.logits += (size_t)tok * a.E;
    a.route_out_idx += (size_t)tok * a.slots;
    a.route_out_w += (size_t)tok * a.slots;
    a.hact += (size_t)tok * a.slots * a.hact_stride;
  }
  const int nb = a.nb;

  // Wave w takes blocks w UPW .. w UPW + UPW - 1 of every chunk of CB
  // blocks.  The activation blocks of this slot go to LDS, each wave staging the
  // blocks it reads itself, so no work-group barrier stands between the
  // staging and the terms.  Loads are issued first and stored once the
  // first weight loads are in flight.
  constexpr int WNB = (GEMV_MAX_NB + NW - 1) / NW;    // blocks per wave, at most
  constexpr int APER = (WNB * 3 + 63) / 64;          // 16-byte pieces per lane
  // block of the wave's t-th block (chunk t / UPW, position t % UPW)
  auto wave_block = [&](int t) { return (t / UPW) * CB + wave * UPW + t % UPW; };
  // With x given (gate/up of one expert, 16-byte aligned, at most 16 blocks
  // per wave: the launcher's check), the activation blocks are quantized
  // here, each wave its own blocks, 8 lanes per block, instead of read from
  // a.act: one launch less.
  constexpr int XPER = 2;  // f32x4 per lane: 16 blocks per wave
  const bool from_x = EPI == EPI_GATE_UP && a.x != nullptr;  // uniform
  const int nbw = (nb + CB - 1) / CB * UPW;                  // the wave's blocks (some past nb)
  u32x4 av[APER];
  f32x4 xv[XPER];
  if (from_x) {
#pragma unroll
    for (int m = 0; m < XPER; m++) {
      const int t = (lane >> 3) + 8 * m, b = wave_block(t);
      if (t < nbw && b < nb) xv[m] = *(const f32x4*)(a.x + (size_t)b * QK + 4 * (lane & 7));
    }
  } else {
    const u32x4* src = (const u32x4*)(a.act + (size_t)slot * a.act_stride);
#pragma unroll
    for (int j = 0; j < APER; j++) {
      const int p = lane + 64 * j;  // piece p % 3 of the wave's block p / 3
      const int b = wave_block(p / 3);
      if (p < WNB * 3 && b < nb) av[j] = src[b * 3 + p % 3];
    }
  }
  auto stage_act = [&]() {
    if (from_x) {
#pragma unroll
      for (int m = 0; m < XPER; m++) {
        const int t = (lane >> 3) + 8 * m, b = wave_block(t);
        if (t < nbw && b < nb) quant_block8(xv[m], lane & 7, s_act + b);  // uniform per 8 lanes
      }
    } else {
      u32x4* dst = (u32x4*)s_act;
#pragma unroll
      for (int j = 0; j < APER; j++) {
        const int p = lane + 64 * j;
        const int b = wave_block(p / 3);
        if (p < WNB * 3 && b < nb) dst[b * 3 + p % 3] = av[j];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  ExpTable tab;
  if constexpr (EPI == EPI_GATE_UP) tab.load();
  int expert = a.route_idx ? a.route_idx[slot] : 0;
  // With router logits given, every wave selects this slot's expert on its
  // own (select_slot); a work-group whose choice is not certain runs the
  // reference's selection first.  The last column of work-groups holds the
  // selector: its first work-group runs the reference's selection (softmax,
  // top-k, renormalisation) and publishes the routes and their weights for
  // the down projection, beside the rows' work.
  const bool routing = EPI == EPI_GATE_UP && a.logits != nullptr;
  if constexpr (EPI == EPI_GATE_UP) {
    if (routing && g == (int)gridDim.x - 1) {
      if (slot != 0 || wave != 0) return;
      route_select<ME>(a.logits, a.E, a.slots, a.normalize, sel.sel_idx, sel.sel_w, tab, sel.e);
      if (lane < a.slots) {
        a.route_out_idx[lane] = sel.sel_idx[lane];
        a.route_out_w[lane] = sel.sel_w[lane];
        if (a.stats) atomicAdd(&a.stats[sel.sel_idx[lane]], 1ull);
      }
      return;
    }
    if (routing) {
      bool safe;
      expert = select_slot<ME>(a.logits, a.E, slot, &safe);
      if (!safe) {  // every wave decided alike: uniform over the work-group
        if (wave == 0) route_select<ME>(a.logits, a.E, a.slots, a.normalize, sel.sel_idx, sel.sel_w, tab, sel.e);
        __syncthreads();
        expert = sel.sel_idx[slot];
      }
    }
  }

  // Wave 0's outputs of one item from its row totals: the plain rows, or
  // gate/up's h = silu(g) * u requantized.
  const int r = lane & 31;
  auto finish = [&](int tile, float total) {
    if constexpr (EPI == EPI_PLAIN) {
      const size_t row = (2 * (size_t)g + (lane >> 5)) * TILE + r;
      if (row < (size_t)a.rows) a.out[row] = total;
    } else if constexpr (EPI == EPI_GATE_UP) {
      float u = __shfl(total, lane + 32);
      float h = wave_silu(total, tab) * u;  // lanes 0-31: *g = silu(*g) * u
      float scale;
      int qsum;
      int q = quant_block_lane(h, &scale, &qsum);
      if (lane < 32) {
        ActBlock* hb = a.hact + (size_t)slot * a.hact_stride + tile;
        hb->q[lane] = (int8_t)q;
        if (lane == 0) {
          hb->scale = scale;
          hb->qsum = qsum;
        }
      }
    }
  };

  // The items of this work-group: gate/up tiles t0 .. t0 + nit - 1 (one
  // slot, so one expert and one activation), or the plain rows' 64-row
  // group g.  Their chunks run as one sequence: the loads of chunk c + 1,
  // the next item's first chunk included, are issued while chunk c's terms
  // are formed, and wave 0 folds each item's chunks in block order and
  // writes its outputs after its last one.
  const int ipw = EPI == EPI_GATE_UP ? a.ipw : 1;
  const int t0 = g * ipw;
  const int nit = EPI == EPI_GATE_UP ? min(ipw, a.tiles - t0) : 1;
  {
    const int ex = expert;
    // planes of this lane's matrix
    const uint8_t* cbase;
    const uint16_t* sbase;
    if constexpr (EPI == EPI_GATE_UP) {
      cbase = (lane < 32 ? a.codes : a.codes2) + (size_t)ex * a.codes_stride;
      sbase = (lane < 32 ? a.scales : a.scales2) + (size_t)ex * a.scales_stride;
    } else {
      cbase = a.codes + (size_t)ex * a.codes_stride;
      sbase = a.scales + (size_t)ex * a.scales_stride;
    }
    auto tile_of = [&](int it) -> size_t {
      return EPI == EPI_GATE_UP ? (size_t)(t0 + it) : 2 * (size_t)g + (lane >> 5);
    };
    auto crow_of = [&](int it) { return cbase + (tile_of(it) * nb * CH * TILE + r) * 16; };
    auto srow_of = [&](int it) { return sbase + tile_of(it) * nb * TILE + r; };
    const ActBlock* act = s_act;

    u32x4 cw[UPW][CH];
    uint16_t sw[UPW];
    // Blocks past the end of the row are clamped to the last block (an
    // in-bounds load whose term is never stored; the same goes for groups),
    // so the chunk loop has no branches and all of its loads are in flight
    // together.  (A clamped block's activation may be another wave's: it
    // only feeds that discarded term.)
    auto block_of = [&](int ch, int s) { return min(ch * CB + wave * UPW + s, nb - 1); };
    auto load_block = [&](const uint8_t* crow, const uint16_t* srow, int ch, int s) {
      const int b = block_of(ch, s);
#pragma unroll
      for (int c = 0; c < CH; c++)
        cw[s][c] = load_weights<NT>((const u32x4*)(crow + ((size_t)b * CH + c) * TILE * 16));
      sw[s] = srow[(size_t)b * TILE];
    };

    float total = 0.0f;
    const int nchunks = (nb + CB - 1) / CB;
    const int nc = nit * nchunks;
    {
      const uint8_t* crow = crow_of(0);
      const uint16_t* srow = srow_of(0);
#pragma unroll
      for (int s = 0; s < UPW; s++) load_block(crow, srow, 0, s);
    }
    stage_act();
    for (int c = 0; c < nc; c++) {
      const int it = c / nchunks, ch = c - it * nchunks;
      const int b0 = ch * CB;
      const int bend = min(nb, b0 + CB);
      float(*tb)[GROUP] = terms[c & 1];
      // Terms in groups of four blocks; each group's registers take the next
      // chunk's loads as soon as its terms are done.  The scheduling barriers
      // keep the activation reads of one group live at a time, so the kernel
      // keeps few VGPRs.
      float tv[UPW];
      const bool more = c + 1 < nc;
      const int itn = (c + 1) / nchunks, chn = c + 1 - itn * nchunks;
      const uint8_t* crn = crow_of(itn);
      const uint16_t* srn = srow_of(itn);
#pragma unroll
      for (int s0 = 0; s0 < UPW; s0 += 4) {
#pragma unroll
        for (int s = s0; s < s0 + 4; s++)
          tv[s] = block_term<DT>(cw[s], sw[s], act + block_of(ch, s));
#pragma unroll
        for (int s = s0; s < s0 + 4; s++) asm volatile("" : "+v"(tv[s]));  // computed here, not at the store
        __builtin_amdgcn_sched_barrier(0);
        if (more) {
#pragma unroll
          for (int s = s0; s < s0 + 4; s++) load_block(crn, srn, chn, s);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // Blocks past the end of the row take the clamped terms and are never
      // folded; an unconditional store keeps each term's computation where it
      // is written (a conditional one would be sunk into the store's branch,
      // keeping every input live until then).
#pragma unroll
      for (int s = 0; s < UPW; s++) tb[wave * UPW + s][lane] = tv[s];
      __syncthreads();
      if (wave == 0) {  // the fold chains first when the SIMD has several ready waves
        __builtin_amdgcn_s_setprio(3);
        total = lds_sum_strided<GROUP>(&tb[0][lane], bend - b0, total);
        __builtin_amdgcn_s_setprio(0);
        if (ch == nchunks - 1) {
          finish(t0 + it, total);
          total = 0.0f;
        }
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
//
// Units are (slot, block) pairs, taken in groups of eight consecutive blocks
// of one slot: pair p is block group p / slots of slot p % slots.  One
// wave-load covers one pair for the group's 8 rows: 8 segments of 128 B,
// each a cache line of the tile layout.  A chunk is CP consecutive pairs,
// so every slot's blocks advance in every chunk, and with them all 8 x slots
// fold chains.  Loads run two chunks ahead: chunk c + 2 is issued as soon
// as chunk c's terms are computed, while chunk c + 1 is in flight.  Each
// wave stages the activation blocks of its own units in LDS, so only the
// terms cross waves.  Wave 0 folds chunk c (64 lanes, one per (row, slot)
// chain, adding its slot's blocks in order: the reference's per-expert dot
// product) while the other waves compute chunk c + 1; the combine then
// takes the slots in route order.

// u / n for 0 <= u < 2^20 from a float reciprocal, corrected to the exact
// quotient (below 2^20 the float estimate is off by at most one)
__device__ __forceinline__ int div_small(int u, int n, float inv_n) {
  int q = (int)((float)u * inv_n);
  if (q * n > u) q--;
  else if ((q + 1) * n <= u) q++;
  return q;
}

constexpr int DR = DOWN_ROWS;   // rows per work-group of k_down_combine
constexpr int DOWN_MAX_SLOTS = 64;

template <int DT, int NW>
__global__ __launch_bounds__(64 * NW) void k_down_combine(DownArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int UPW = 4 / CH;        // pairs per wave and chunk (4 loads of 16 B per lane)
  constexpr int CP = NW * UPW;       // pairs per chunk
  constexpr int CU = CP * 8;         // units per chunk
  constexpr int APL = (UPW * 24 + 63) / 64;  // 16-byte activation pieces per lane and chunk
  constexpr int SPL = DOWN_MAX_SLOTS / 8;    // slots per fold lane
  // terms of row r at [r][unit]; the row pitch CU + 4 spreads the rows of a
  // term store over the banks
  __shared__ __attribute__((aligned(16))) float terms[2][DR][CU + 4];
  __shared__ ActBlock s_act[NW][UPW * 8];  // each wave's activation blocks of its current chunk
  __shared__ u32x4 s_scl[NW][UPW * 8];     // and its scales: [pair][block] x 8 rows
  __shared__ float s_tot[DOWN_MAX_SLOTS][DR];
  __shared__ int s_exp[DOWN_MAX_SLOTS];
  __shared__ float s_w[DOWN_MAX_SLOTS];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  const int nb = a.nb;
  const int slots = a.slots;
  if (blockIdx.y > 0) {  // token blockIdx.y of a few-token decode
    a.route_idx += (size_t)blockIdx.y * slots;
    a.route_w += (size_t)blockIdx.y * slots;
    a.hact += (size_t)blockIdx.y * slots * a.hact_stride;
    a.out += (size_t)blockIdx.y * a.rows;
  }
  const int nbg = (nb + 7) / 8;
  const int npairs = slots * nbg;
  const int nchunks = (npairs + CP - 1) / CP;
  const float inv_slots = 1.0f / (float)slots;
  if (threadIdx.x < slots) {
    s_exp[threadIdx.x] = a.route_idx[threadIdx.x];
    s_w[threadIdx.x] = a.route_w[threadIdx.x];
  }

  const int r = lane % DR;  // row within the group
  const int j = lane / DR;  // block within the pair's group of eight
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
  // the scales of the group's 8 rows for block b: 16 bytes at
  // srow_off + b * TILE elements
  const size_t srow_off = tile * nb * TILE + row0 % TILE;

  struct Buf {
    u32x4 cw[UPW][CH];
    u32x4 sv;  // lanes < UPW * 8: the group's 8 rows' scales of one block of one pair
    u32x4 av[APL];
  };
  // pair of wave-load s in chunk c (wave-uniform)
  auto pair_of = [&](int c, int s) { return c * CP + s * NW + wave; };
  // Issues chunk c's loads into B: every live wave-load's codes and scales,
  // and the activation blocks of the wave's units.  Blocks past the end of
  // the row are clamped to the last block (in-bounds; their terms are never
  // folded).
  auto issue = [&](Buf& B, int c) {
#pragma unroll
    for (int s = 0; s < UPW; s++) {
      const int p = pair_of(c, s);
      if (p < npairs) {  // wave-uniform
        const int bg = div_small(p, slots, inv_slots), sl = p - bg * slots;
        const int b = min(bg * 8 + j, nb - 1);
        const size_t e = (size_t)s_exp[sl];
        const uint8_t* c0 = a.codes + e * a.codes_stride + row_off;
#pragma unroll
        for (int q = 0; q < CH; q++)
          B.cw[s][q] = __builtin_nontemporal_load((const u32x4*)(c0 + ((size_t)b * CH + q) * TILE * 16));
      }
    }
    {  // lane l < UPW * 8: block l % 8 of pair l / 8 (clamped like the codes)
      const int s = lane / 8, p = pair_of(c, s);
      if (lane < UPW * 8 && p < npairs) {
        const int bg = div_small(p, slots, inv_slots), sl = p - bg * slots;
        const int b = min(bg * 8 + lane % 8, nb - 1);
        const size_t e = (size_t)s_exp[sl];
        B.sv = *(const u32x4*)(a.scales + e * a.scales_stride + srow_off + (size_t)b * TILE);
      }
    }
#pragma unroll
    for (int m = 0; m < APL; m++) {
      const int q = lane + 64 * m;  // piece q % 3 of unit q / 3 of the wave's units
      const int s = q / 24, u = (q % 24) / 3;
      const int p = pair_of(c, s);
      if (q < UPW * 24 && p < npairs) {
        const int bg = div_small(p, slots, inv_slots), sl = p - bg * slots;
        const int b = min(bg * 8 + u, nb - 1);
        B.av[m] = ((const u32x4*)(a.hact + (size_t)sl * a.hact_stride + b))[q % 3];
      }
    }
  };

  // fold lane (row r, slot group j): slots j, j + 8, ...
  float tot[SPL];
#pragma unroll
  for (int i = 0; i < SPL; i++) tot[i] = 0.0f;

  // Chunk c from B: stage the wave's activation blocks, the block terms,
  // chunk c + 2's loads into B, the terms to LDS; then wave 0 folds them.
  auto process = [&](Buf& B, int c) {
    float(*tb)[CU + 4] = terms[c & 1];
#pragma unroll
    for (int m = 0; m < APL; m++) {
      const int q = lane + 64 * m;
      if (q < UPW * 24 && pair_of(c, q / 24) < npairs) ((u32x4*)s_act[wave])[q] = B.av[m];
    }
    if (lane < UPW * 8 && pair_of(c, lane / 8) < npairs) s_scl[wave][lane] = B.sv;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float tv[UPW];
#pragma unroll
    for (int s = 0; s < UPW; s++)
      if (pair_of(c, s) < npairs)
        tv[s] = block_term<DT>(B.cw[s], ((const uint16_t*)&s_scl[wave][s * 8 + j])[r], &s_act[wave][s * 8 + j]);
#pragma unroll
    for (int s = 0; s < UPW; s++)
      if (pair_of(c, s) < npairs) asm volatile("" : "+v"(tv[s]));  // computed here, not at the store
    __builtin_amdgcn_sched_barrier(0);
    if (c + 2 < nchunks) issue(B, c + 2);
#pragma unroll
    for (int s = 0; s < UPW; s++)
      if (pair_of(c, s) < npairs) tb[r][(s * NW + wave) * 8 + j] = tv[s];
    __syncthreads();  // chunk c's terms are in; wave 0 has folded chunk c - 1
    if (wave == 0) {
      // The fold chains are the critical path of the chunk: their wave goes
      // first when the SIMD has several ready waves (the others fill its gaps)
      __builtin_amdgcn_s_setprio(3);
      const int pbeg = c * CP, pend = min(npairs, pbeg + CP);
#pragma unroll
      for (int i = 0; i < SPL; i++) {
        const int sl = j + 8 * i;
        if (sl < slots) {
          // this slot's pairs in the chunk, in block order: p = sl + q slots,
          // block group q; each pair's eight terms are read while the
          // previous pair's are added
          const int q0 = (pbeg - sl + slots - 1) / slots;
          const int p0 = sl + q0 * slots;
          const int np = p0 < pend ? (pend - p0 + slots - 1) / slots : 0;
          const float* t = &tb[r][(p0 - pbeg) * 8];
          const int ts = slots * 8;
          float acc = tot[i];
          f32x4 x0, x1;
          if (np > 0) {
            x0 = *(const f32x4*)t;
            x1 = *(const f32x4*)(t + 4);
          }
          for (int m = 0; m < np; m++) {
            f32x4 y0 = x0, y1 = x1;
            if (m + 1 < np) {
              y0 = *(const f32x4*)(t + (m + 1) * ts);
              y1 = *(const f32x4*)(t + (m + 1) * ts + 4);
            }
            const int n = nb - 8 * (q0 + m);  // blocks of this group inside the row
            if (n >= 8) {
              acc = acc + x0.x;
              acc = acc + x0.y;
              acc = acc + x0.z;
              acc = acc + x0.w;
              acc = acc + x1.x;
              acc = acc + x1.y;
              acc = acc + x1.z;
              acc = acc + x1.w;
            } else {  // the row's last, partial group
              const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
              for (int k = 0; k < n; k++) acc = acc + v[k];
            }
            x0 = y0;
            x1 = y1;
          }
          tot[i] = acc;
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  };

  __syncthreads();  // s_exp / s_w
  Buf A, B;
  issue(A, 0);
  if (nchunks > 1) issue(B, 1);
  for (int c = 0; c < nchunks; c += 2) {
    process(A, c);
    if (c + 1 < nchunks) process(B, c + 1);
  }
  if (wave != 0) return;
#pragma unroll
  for (int i = 0; i < SPL; i++) {
    const int sl = j + 8 * i;
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

// The same projection and combine with whole fold chains per wave, used
// for 3 routes over rows of 129-512 blocks, or in calls of CACHED_LOAD_TOKENS
// tokens or more, when every slot's activation blocks fit in LDS (the rest
// of one to three routes take k_down_tile below).  A
// work-group owns RG output rows for every slot (RG = 16 for 2 or 3 slots,
// 32 for 1); wave w takes the chain (RPW rows, slot) of row subgroup
// w / slots and slot w % slots.  Lane LPR r + j (LPR = 64 / RPW) holds row
// r and block LPR q + j of group q, so a wave-load reads, per block, the
// RPW rows' 16-byte chunks of the tile layout.  D groups are in flight; each
// group's terms join the row's running sum in block order by DPP shifts
// within the row's lanes, so no other wave or barrier is waited for until
// the combine.  (The launcher takes eight rows per wave.)  The chain's scales are
// staged in LDS first, one piece per block (its RPW rows' scales), loaded
// before the ring (loads return in order, so the staging barrier waits for
// them and the activations, not for the ring).
constexpr int DOWN_ACT_MAX = 1024;  // activation blocks staged in LDS (48 KB)
constexpr int DOWN_SCL_MAX = 4096;  // 16-byte scale pieces staged in LDS (64 KB): waves x blocks
constexpr int DOWN_CHAIN_MAX_NB = 512;  // blocks per row: one scale piece per lane and 64 blocks

__host__ __device__ inline int down_chain_rows(int slots) { return slots >= 4 ? 8 : (slots >= 2 ? 16 : 32); }
__host__ __device__ inline int down_chain_waves(int slots, int rpw) {
  return down_chain_rows(slots) / rpw * (slots < 8 ? slots : 8);
}
// bytes of k_down_chain's staging (its dynamic LDS)
static inline size_t down_chain_lds(int slots, int nb, int rpw) {
  return (size_t)slots * nb * 48 + (size_t)down_chain_waves(slots, rpw) * nb * 2 * rpw;
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// acc + the terms of lanes L + 1 .. L + K of the lane's DPP row, in lane
// order (a comma fold runs left to right); the _n form adds only lanes
// L + k with k < n.
template <int K>
__device__ __forceinline__ float row_term(float t) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x100 + K, 0xF, 0xF, false));
}
template <int... K>
__device__ __forceinline__ float row_fold(float acc, float t, std::integer_sequence<int, K...>) {
  ((acc = acc + row_term<K + 1>(t)), ...);
  return acc;
}
template <int... K>
__device__ __forceinline__ float row_fold_n(float acc, float t, int n, std::integer_sequence<int, K...>) {
  ((acc = K + 1 < n ? acc + row_term<K + 1>(t) : acc), ...);
  return acc;
}

template <int DT, int RPW, int D>  // D: groups in flight per wave, a multiple of 4
__global__ __launch_bounds__(512) void k_down_chain(DownArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int LPR = 64 / RPW;
  static_assert(D % 4 == 0, "groups go in batches of four");
  static_assert(RPW == 8 || RPW == 4, "a row's lanes lie in one DPP row");
  typedef typename std::conditional<RPW == 8, u32x4, u32x2>::type Piece;
  // LDS sized at launch (down_chain_lds): every slot's activation blocks
  // (slot s at [s * nb]), then each wave's scale pieces, one per block,
  // wave w at [w * nb, (w + 1) * nb)
  extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn_chain[];
  ActBlock* s_act = (ActBlock*)s_dyn_chain;
  Piece* s_scl = (Piece*)(s_dyn_chain + (size_t)a.slots * a.nb * 3);
  __shared__ float s_tot[3][32];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x;
  const int nb = a.nb, slots = a.slots;  // slots <= 3: one chain per wave
  if (blockIdx.y > 0) {  // token blockIdx.y of a few-token decode
    a.route_idx += (size_t)blockIdx.y * slots;
    a.route_w += (size_t)blockIdx.y * slots;
    a.hact += (size_t)blockIdx.y * slots * a.hact_stride;
    a.out += (size_t)blockIdx.y * a.rows;
  }
  const int nbg = (nb + LPR - 1) / LPR;
  const int rg = down_chain_rows(slots);
  const int sub = wave / slots, sl = wave % slots;
  // every slot's activation blocks (independent of the routes): loads
  // issued first, stored after the first weight loads.  The launcher takes
  // D = 4 only for rows of at most 4 LPR blocks and q4_0 D = 8 for at most
  // 8 LPR, so those variants hold at most 3 x LPR D blocks; the others up
  // to DOWN_ACT_MAX.  (Sizing them all for DOWN_ACT_MAX spilled the pieces.)
  constexpr int MAXB = (D == 4 || (DT == Q4_0 && D == 8)) ? 3 * LPR * D : DOWN_ACT_MAX;
  constexpr int APT = (MAXB * 3 + 255) / 256;  // pieces per thread, at most (256+ threads)
  const int npieces = slots * nb * 3;
  u32x4 av[APT];
#pragma unroll
  for (int m = 0; m < APT; m++) {
    const int i = threadIdx.x + m * blockDim.x;
    if (i < npieces) {
      const int sl = i / (nb * 3), rem = i - sl * nb * 3;
      av[m] = ((const u32x4*)(a.hact + (size_t)sl * a.hact_stride))[rem];
    }
  }
  // The row groups of a 32-row tile share its scale lines; work-group g runs
  // on XCD g % 8, so when the grid allows the groups of one tile get ids of
  // one residue class (a permutation of the row groups).
  const int per_tile = 32 / rg;
  size_t row0 = (size_t)g * rg;
  if (per_tile > 1 && gridDim.x % (8 * per_tile) == 0) {
    const int gx = g & 7, gj = g >> 3;
    row0 = (size_t)(gx + 8 * (gj / per_tile)) * TILE + (size_t)(gj % per_tile) * rg;
  }
  const int r = lane / LPR, j = lane % LPR;
  const size_t rowg = row0 + (size_t)sub * RPW;
  const size_t tile = rowg / TILE;
  const int rt = (int)(rowg % TILE) + r;
  const size_t row_off = (tile * nb * CH * TILE + rt) * 16;

  u32x4 cw[D][CH];
  const size_t e = (size_t)__builtin_amdgcn_readfirstlane(a.route_idx[sl]);
  const uint8_t* cbase = a.codes + e * a.codes_stride + row_off;
  // group q's codes into ring slot d (groups past the end are clamped to
  // the last: in-bounds loads that are never used)
  auto load = [&](int d, int q) {
    const int b = min(min(q, nbg - 1) * LPR + j, nb - 1);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[d][c] = __builtin_nontemporal_load((const u32x4*)(cbase + ((size_t)b * CH + c) * TILE * 16));
  };
  // The chain's scales: the RPW rows' scales of a block are contiguous in
  // the tile's scale line, so a lane loads whole pieces (blocks lane,
  // lane + 64, ...) and parks them in LDS; a per-block 2-byte load per lane
  // would touch a line per row group for a few useful bytes.  The pieces
  // (at most 512: the launcher keeps nb <= 512) are loaded before the
  // ring's codes: loads return in order, so they and the activation pieces
  // can be parked while the codes are still in flight, and the staging
  // barrier does not wait for the ring.
  Piece* scl = s_scl + wave * nb;
  const Piece* sp = (const Piece*)(a.scales + e * a.scales_stride + tile * nb * TILE + (rowg % TILE));
  {
    Piece v[8];
#pragma unroll
    for (int m = 0; m < 8; m++)
      if (lane + 64 * m < nb) v[m] = sp[(size_t)(lane + 64 * m) * (TILE * 2 / sizeof(Piece))];
#pragma unroll
    for (int d = 0; d < D; d++) load(d, d);
#pragma unroll
    for (int m = 0; m < 8; m++)
      if (lane + 64 * m < nb) scl[lane + 64 * m] = v[m];
  }
#pragma unroll
  for (int m = 0; m < APT; m++) {
    const int i = threadIdx.x + m * blockDim.x;
    if (i < npieces) ((u32x4*)s_act)[i] = av[m];
  }
  const uint16_t* scl16 = (const uint16_t*)scl;
  __syncthreads();  // s_act, s_scl

  {
    const ActBlock* act = s_act + (size_t)sl * nb;
    float acc = 0.0f;  // row r's dot product (valid in lane LPR r)
#pragma unroll 1
    for (int q0 = 0; q0 < nbg; q0 += D) {
#pragma unroll
      for (int d0 = 0; d0 < D; d0 += 4) {
        const int qb = q0 + d0;
        if (qb < nbg) {  // wave-uniform; the batch's four terms, then their sums in order
          float t[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int b = min((qb + i) * LPR + j, nb - 1);
            t[i] = block_term<DT>(cw[d0 + i], scl16[b * RPW + r], act + b);
          }
          if (qb + 4 <= nb / LPR) {  // four whole groups (wave-uniform): plain adds in block order
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc = row_fold(acc + t[i], t[i], std::make_integer_sequence<int, LPR - 1>{});
          } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
              // groups past the row's end have n <= 0 and add nothing
              const int n = nb - (qb + i) * LPR;  // blocks of the group inside the row
              acc = n > 0 ? acc + t[i] : acc;
              acc = row_fold_n(acc, t[i], n, std::make_integer_sequence<int, LPR - 1>{});
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) load(d0 + i, qb + i + D);
      }
    }
    if (j == 0) s_tot[sl][sub * RPW + r] = acc;
  }
  __syncthreads();
  if ((int)threadIdx.x < rg) {
    float acc = 0.0f;  // out.fill(0.0), then out = out + w * y in route order
    for (int s2 = 0; s2 < slots; s2++) acc = acc + a.route_w[s2] * s_tot[s2][threadIdx.x];
    const size_t row = row0 + threadIdx.x;
    if (row < (size_t)a.rows) a.out[row] = acc;
  }
}

// ===========================================================================
// Down projection and combine with block terms spread over the waves
// ===========================================================================
//
// MoeLayer::forward's combine (src/model/moe.rs:63-68) for S = 1 to 8
// routes, with each row's block terms spread over the work-group's waves
// (the k_gemv scheme) instead of one wave per chain.  A work-group owns RW
// output rows (32: one tile; 16 or 8: part of one) of every slot.  The
// slots go in pairs: lane l of a wave works for slot 2 q + l / 32 of the
// wave's pair q (waves w of one pair: w / (NW / (S / 2)) = q); within the
// half, lane RW p + r holds row r and block p of each group of 32 / RW
// consecutive blocks (one route: the whole wave works for it, lane RW p + r
// holding block p of each group of 64 / RW; for odd S the last pair's second
// half repeats the last slot's loads, the same lines in the same wave-load,
// and its chains are never combined).  So one wave-load reads, per slot, RW
// rows of consecutive blocks: 512 contiguous bytes of the tile layout per 16-byte
// chunk for RW = 32 (two 256-byte pieces for 16), where a wave per chain
// reads eight 128-byte lines spread over 4 KB.  Blocks go to the waves in
// chunks of CB per slot; the next chunk's loads are issued while a chunk's
// terms are formed.  Terms go to LDS; the first S RW / 64 waves add them to
// the running sums of the S x RW chains (chain RW s + r: slot s, row r) in
// block order, the reference's left-to-right sum; then
// out = (((0 + w_0 y_0) + w_1 y_1) + ...) in route order.  The launcher takes
// sixteen waves with two 16-byte code loads per lane in flight per chunk
// (q4_0; one 32-byte block for q8_0).  Measured (q4_0, one token): Mixtral-
// 8x7B-shaped down 11.8 us against 11.8-12.0 with eight waves and four
// loads, 13.5 with eight waves and two, 15.1 with four waves and four;
// Qwen3-235B-shaped, 16-row groups: 6.4-7.5 us with two loads, 6.6-6.7
// with three, 7.7 with four.
constexpr int DOWN_TILE_MAX_NB = 512;  // blocks per row: two slots' activations in 48 KB of LDS

static inline size_t down_tile_lds(int slots, int nb) { return (size_t)slots * nb * sizeof(ActBlock); }

// PLAIN: WeightMatrix::matvec (src/tensor/matrix.rs:115-143) of one matrix
// (S = 1, no routes): out[row] is the row's sum; x, when given, is
// quantized into the staging by the work-group (the expressions of
// k_act_quant, so the same q8 blocks).
template <int DT, int S, int NW, int RW, int UPW, bool PLAIN = false>
__global__ __launch_bounds__(64 * NW) void k_down_tile(DownArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int LPS = S == 1 ? 64 : 32;  // lanes per slot
  constexpr int BPL = LPS / RW;       // blocks per slot and wave-load
  constexpr int SP = S == 1 ? 1 : (S + 1) / 2;  // slot pairs (one route: one slot; odd S: a ghost)
  constexpr int WPP = NW / SP;        // waves per slot pair
  constexpr int CB = WPP * UPW * BPL; // blocks per chunk
  constexpr int NCH = (S == 1 ? 1 : 2 * SP) * RW;  // fold chains (a ghost slot's are never combined)
  constexpr int FW = (NCH + 63) / 64; // folding waves
  // terms per group (the largest of 4, 3, 2, 1 that divides UPW); the next
  // chunk's loads follow each group
  constexpr int GS = UPW % 4 == 0 ? 4 : (UPW % 3 == 0 ? 3 : (UPW % 2 == 0 ? 2 : 1));
  static_assert(S >= 1 && S <= 8, "at most eight routes");
  static_assert(NW % SP == 0, "whole waves per slot pair");
  static_assert(RW == 32 || RW == 16 || RW == 8, "a half-wave covers 1, 2 or 4 blocks of RW rows");
  static_assert(UPW % GS == 0, "wave-loads go in whole groups");
  static_assert(FW <= NW, "enough waves to fold");
  static_assert(!PLAIN || S == 1, "a plain matvec is one matrix");
  __shared__ float terms[2][CB][NCH];
  __shared__ float s_tot[NCH];
  // every slot's activation blocks, sized at launch (down_tile_lds): slot s at [s * nb]
  extern __shared__ __attribute__((aligned(16))) u32x4 s_dyn_tile[];
  ActBlock* s_act = (ActBlock*)s_dyn_tile;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = a.nb;
  if (blockIdx.y > 0) {  // token blockIdx.y of a few-token decode
    a.route_idx += (size_t)blockIdx.y * S;
    a.route_w += (size_t)blockIdx.y * S;
    a.hact += (size_t)blockIdx.y * S * a.hact_stride;
    a.out += (size_t)blockIdx.y * a.rows;
  }
  const int sl = S == 1 ? 0 : 2 * (wave / WPP) + (lane >> 5);  // this lane's slot (S: the ghost)
  const int slc = min(sl, S - 1);  // the slot it loads for: a ghost repeats the last one's
                                   // addresses (the same wave-load, the same lines)
  const int wq = wave % WPP;                      // the wave's place among its pair's waves
  const int p = (lane % LPS) / RW;                // block within a group of BPL
  const int r = lane & (RW - 1);                  // row of the work-group's rows
  // the lane's expert first (loads return in order: waiting for it leaves
  // the activation loads behind it in flight)
  const int ev = PLAIN ? 0 : a.route_idx[slc];
  __builtin_amdgcn_sched_barrier(0);
  // every slot's activation pieces, clamped to the last (no branches, so
  // the waits stay counted)
  constexpr int NT = 64 * NW;
  constexpr int MAXP = S <= 2 ? S * DOWN_TILE_MAX_NB * 3 : S * 128 * 3;  // launcher: nb <= 128 for S > 2
  constexpr int APT = (MAXP + NT - 1) / NT;
  const int npieces = S * nb * 3;
  u32x4 av[APT];
  // PLAIN with x: 8 lanes per block, each its 4 values (the block of lane
  // group q = thread / 8, pass m: q + (NT / 8) m), clamped to the last
  constexpr int XPT = PLAIN ? (DOWN_TILE_MAX_NB * 8 + NT - 1) / NT : 1;
  f32x4 xv[XPT];
  const bool from_x = PLAIN && a.x != nullptr;  // uniform
  if (from_x) {
#pragma unroll
    for (int m = 0; m < XPT; m++) {
      const int b = min((int)(threadIdx.x >> 3) + (NT / 8) * m, nb - 1);
      xv[m] = *(const f32x4*)(a.x + (size_t)b * QK + 4 * (threadIdx.x & 7));
    }
  } else {
#pragma unroll
    for (int m = 0; m < APT; m++) {
      const int i = min((int)threadIdx.x + NT * m, npieces - 1);
      const int s2 = i / (nb * 3), rem = i - s2 * nb * 3;
      av[m] = ((const u32x4*)(a.hact + (size_t)s2 * a.hact_stride))[rem];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // Work-group g runs on XCD g % 8; for RW < 32 the row groups of one tile
  // get ids of one residue class when the grid allows (they share the
  // tile's scale lines).
  constexpr int PER_TILE = 32 / RW;
  const int g = blockIdx.x;
  size_t row0 = (size_t)g * RW;
  if (PER_TILE > 1 && gridDim.x % (8 * PER_TILE) == 0) {
    const int gx = g & 7, gj = g >> 3;
    row0 = (size_t)(gx + 8 * (gj / PER_TILE)) * TILE + (size_t)(gj % PER_TILE) * RW;
  }
  const size_t tile = row0 / TILE;
  const int rt = (int)(row0 % TILE) + r;
  const size_t e = (size_t)ev;
  const uint8_t* cbase = a.codes + e * a.codes_stride + (tile * nb * CH * TILE + rt) * 16;
  const uint16_t* sbase = a.scales + e * a.scales_stride + tile * nb * TILE + rt;
  u32x4 cw[UPW][CH];
  uint16_t sw[UPW];
  // blocks past the end of the row are clamped to the last block (in-bounds
  // loads whose terms are never folded)
  auto block_of = [&](int ch, int s) { return min(ch * CB + (wq * UPW + s) * BPL + p, nb - 1); };
  auto load_block = [&](int ch, int s) {
    const int b = block_of(ch, s);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[s][c] = load_weights<true>((const u32x4*)(cbase + ((size_t)b * CH + c) * TILE * 16));
    sw[s] = sbase[(size_t)b * TILE];
  };
#pragma unroll
  for (int s = 0; s < UPW; s++) {
    load_block(0, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  const float wv = PLAIN ? 0.0f : a.route_w[min(lane, S - 1)];
  if (from_x) {
#pragma unroll
    for (int m = 0; m < XPT; m++) {
      const int b = (int)(threadIdx.x >> 3) + (NT / 8) * m;
      if (b < nb) quant_block8(xv[m], threadIdx.x & 7, s_act + b);  // uniform per 8 lanes
    }
  } else {
#pragma unroll
    for (int m = 0; m < APT; m++) {
      const int i = (int)threadIdx.x + NT * m;
      if (i < npieces) ((u32x4*)s_act)[i] = av[m];
    }
  }
  __syncthreads();  // s_act

  const ActBlock* act = s_act + (size_t)slc * nb;
  const int chain = wave * 64 + lane;  // folding waves: chain RW s + r
  float total = 0.0f;
  const int nchunks = (nb + CB - 1) / CB;
  for (int c = 0; c < nchunks; c++) {
    const int b0 = c * CB;
    const int bend = min(nb, b0 + CB);
    float(*tb)[NCH] = terms[c & 1];
    float tv[UPW];
    const bool more = c + 1 < nchunks;
#pragma unroll
    for (int s0 = 0; s0 < UPW; s0 += GS) {
#pragma unroll
      for (int s = s0; s < s0 + GS; s++) tv[s] = block_term<DT>(cw[s], sw[s], act + block_of(c, s));
#pragma unroll
      for (int s = s0; s < s0 + GS; s++) asm volatile("" : "+v"(tv[s]));  // computed here, not at the store
      __builtin_amdgcn_sched_barrier(0);
      if (more) {
#pragma unroll
        for (int s = s0; s < s0 + GS; s++) load_block(c + 1, s);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int s = 0; s < UPW; s++) tb[(wq * UPW + s) * BPL + p][sl * RW + r] = tv[s];
    __syncthreads();
    if (wave < FW && chain < NCH) {  // the fold chains first when the SIMD has several ready waves
      __builtin_amdgcn_s_setprio(3);
      total = lds_sum_strided<NCH>(&tb[0][chain], bend - b0, total);
      __builtin_amdgcn_s_setprio(0);
    }
  }
  if (wave < FW && chain < NCH) s_tot[chain] = total;
  float wts[S];  // the route weights, lane s's wv
#pragma unroll
  for (int s2 = 0; s2 < S; s2++) wts[s2] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), s2));
  __syncthreads();
  if (PLAIN) {
    if (wave == 0 && lane < RW) {
      const size_t row = row0 + lane;
      if (row < (size_t)a.rows) a.out[row] = total;
    }
    return;
  }
  if (wave == 0 && lane < RW) {
    float o = 0.0f;  // out.fill(0.0), then out = out + w * y in route order
#pragma unroll
    for (int s2 = 0; s2 < S; s2++) o = o + wts[s2] * s_tot[s2 * RW + lane];
    const size_t row = row0 + lane;
    if (row < (size_t)a.rows) a.out[row] = o;
  }
}

// ===========================================================================
// Down projection and combine for 4 to 8 routes, whole chains per wave
// ===========================================================================
//
// MoeLayer::forward's combine (src/model/moe.rs:63-68) over down(h_s) of
// every route s, with a work-group per 8 output rows and one wave per
// route: wave s folds the chains of slot s for the 8 rows (lane 8r + j:
// row r, block 8q + j of group q, as k_matvec_chain), all D groups of a
// short row in flight at once; then the 8 rows' outputs out = out + w_s y_s
// in route order.  Every slot's activation blocks and each wave's scale
// pieces are staged in LDS sized by MAXNB, so several work-groups share a
// CU.  Loads are issued in the order their waits come: the activation
// pieces (they need no route), then, once the slot's expert is known, the
// scale pieces and the code ring; every staging store is unconditional.
template <int DT, int MAXNB, bool NT = true>  // NT as in k_gemv
__global__ __launch_bounds__(512) void k_down_slots(DownArgs a) {
  constexpr int CH = Layout<DT>::CH;
  constexpr int MAXG = (MAXNB + 7) / 8;
  // groups in flight: every group of a row when they fit (no loads past
  // the row's end), else a ring of 16 / CH refilled in batches of four
  constexpr int D = MAXG <= 16 / CH ? MAXG : 16 / CH;
  static_assert(MAXG <= D || D % 4 == 0, "a refilled ring takes batches of four");
  constexpr int SPL = (MAXNB + 63) / 64;                  // scale pieces per lane
  constexpr int APT = (8 * MAXNB * 3 + 511) / 512;        // activation pieces per thread
  __shared__ __attribute__((aligned(16))) u32x4 s_actv[APT * 512];
  __shared__ u32x4 s_scl[8][SPL * 64];
  __shared__ float s_y[8][8];
  __shared__ float s_w[8];

  const int lane = threadIdx.x & 63;
  const int sl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's slot
  const int nt = (int)blockDim.x;                                   // 64 slots
  const int nb = a.nb, slots = a.slots, nbg = (nb + 7) / 8;
  if (blockIdx.y > 0) {  // token blockIdx.y of a few-token decode
    a.route_idx += (size_t)blockIdx.y * slots;
    a.route_w += (size_t)blockIdx.y * slots;
    a.hact += (size_t)blockIdx.y * slots * a.hact_stride;
    a.out += (size_t)blockIdx.y * a.rows;
  }
  // the slot's expert first (loads return in order: waiting for it leaves
  // the activation loads behind it in flight)
  const int ev = a.route_idx[sl];
  __builtin_amdgcn_sched_barrier(0);
  // every slot's activation pieces (slot s's blocks at [s * nb])
  const int npieces = slots * nb * 3;
  u32x4 av[APT];
#pragma unroll
  for (int m = 0; m < APT; m++) {
    const int i = min((int)threadIdx.x + nt * m, npieces - 1);
    const int s2 = i / (nb * 3), rem = i - s2 * nb * 3;
    av[m] = ((const u32x4*)(a.hact + (size_t)s2 * a.hact_stride))[rem];
  }
  __builtin_amdgcn_sched_barrier(0);
  const int e = __builtin_amdgcn_readfirstlane(ev);
  // The four 8-row groups of a 32-row tile share its scale lines; work-group
  // g runs on XCD g % 8, so when the grid is a multiple of 32 the groups of
  // one tile get ids of one residue class (a permutation of the row groups).
  const int g = blockIdx.x;
  size_t row0 = (size_t)g * 8;
  if ((gridDim.x & 31) == 0) {
    const int gx = g & 7, gj = g >> 3;
    row0 = (size_t)(gx + 8 * (gj >> 2)) * TILE + (size_t)(gj & 3) * 8;
  }
  const size_t tile = row0 / TILE;
  const int r = lane >> 3, j = lane & 7;
  const int rt = (int)(row0 % TILE) + r;
  const uint8_t* cbase = a.codes + (size_t)e * a.codes_stride + (tile * nb * CH * TILE + rt) * 16;
  const u32x4* sp = (const u32x4*)(a.scales + (size_t)e * a.scales_stride + tile * nb * TILE + row0 % TILE);
  u32x4 sv[SPL];
#pragma unroll
  for (int m = 0; m < SPL; m++) sv[m] = sp[(size_t)min(lane + 64 * m, nb - 1) * (TILE * 2 / 16)];
  __builtin_amdgcn_sched_barrier(0);
  u32x4 cw[D][CH];
  auto load = [&](int d, int q) {
    const int b = min(min(q, nbg - 1) * 8 + j, nb - 1);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[d][c] = load_weights<NT>((const u32x4*)(cbase + ((size_t)b * CH + c) * TILE * 16));
  };
#pragma unroll
  for (int d = 0; d < D; d++) {
    load(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the route weights, needed only by the combine
  const float wv = a.route_w[min((int)threadIdx.x & 7, slots - 1)];
#pragma unroll
  for (int m = 0; m < SPL; m++) s_scl[sl][lane + 64 * m] = sv[m];
#pragma unroll
  for (int m = 0; m < APT; m++) s_actv[threadIdx.x + nt * m] = av[m];
  __syncthreads();
  const uint16_t* scl16 = (const uint16_t*)s_scl[sl];
  const ActBlock* act = (const ActBlock*)s_actv + (size_t)sl * nb;

  float acc = 0.0f;  // row r's dot product for this slot (valid in lane 8 r)
  auto pass = [&](int q0, auto reload) {
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 4) {
      constexpr int NI_MAX = 4;
      const int ni = D - d0 < NI_MAX ? D - d0 : NI_MAX;  // groups of this batch (compile time)
      const int qb = q0 + d0;
      if (qb < nbg) {
        float t[NI_MAX];
#pragma unroll
        for (int i = 0; i < NI_MAX; i++) {
          if (i < ni) {
            const int b = min((qb + i) * 8 + j, nb - 1);
            t[i] = block_term<DT>(cw[d0 + i], scl16[b * 8 + r], act + b);
          }
        }
        if (qb + ni <= nb / 8) {  // whole groups (wave-uniform): plain adds in block order
#pragma unroll
          for (int i = 0; i < NI_MAX; i++)
            if (i < ni) acc = row_fold(acc + t[i], t[i], std::make_integer_sequence<int, 7>{});
        } else {
#pragma unroll
          for (int i = 0; i < NI_MAX; i++) {
            if (i < ni) {
              const int n = nb - (qb + i) * 8;  // blocks of the group inside the row
              acc = n > 0 ? acc + t[i] : acc;
              acc = row_fold_n(acc, t[i], n, std::make_integer_sequence<int, 7>{});
            }
          }
        }
      }
      if constexpr (decltype(reload)::value) {
#pragma unroll
        for (int i = 0; i < 4; i++) load(d0 + i, qb + i + D);
      }
    }
  };
  if constexpr (MAXG <= D) {
    pass(0, std::false_type{});
  } else {
#pragma unroll 1
    for (int q0 = 0; q0 < nbg; q0 += D) pass(q0, std::true_type{});
  }
  if (j == 0) s_y[sl][r] = acc;
  if (threadIdx.x < 8) s_w[threadIdx.x] = wv;
  __syncthreads();
  if ((int)threadIdx.x < 8) {
    float o = 0.0f;  // out.fill(0.0), then out = out + w * y in route order
    for (int s2 = 0; s2 < slots; s2++) o = o + s_w[s2] * s_y[s2][threadIdx.x];
    const size_t row = row0 + threadIdx.x;
    if (row < (size_t)a.rows) a.out[row] = o;
  }
}

// ===========================================================================
// WeightMatrix::matvec with whole fold chains per wave
// ===========================================================================
//
// out[r] = dot_q8_0 / dot_q4_0 (row r, quantize(x)) (src/tensor/matrix.rs:
// 115-143, src/tensor/quant.rs:77-144), every row's chain in one wave.  A
// wave takes RPW consecutive rows (8 or 4) of one 32-row tile with
// LPR = 64 / RPW lanes per row: lane LPR r + j holds row r and block
// LPR q + j of block group q, so a wave-load reads, per block, the RPW rows'
// 16-byte chunks (128 or 64 contiguous bytes of the tile layout).  D groups
// are in flight per wave; each group's LPR terms join the row's running
// sum in block order by DPP shifts within the row's lanes (one DPP row of
// 16 lanes holds one or two rows).  A work-group is NW waves of one tile.
// With XQ the work-group quantizes x itself (all of it, 8 lanes per block,
// into LDS; the same expressions as k_act_quant), so no quantization launch
// comes first; otherwise the q8 blocks are read from act.  MAXNB bounds the
// blocks per row (the LDS staging and the early loads are sized by it).
// Four rows per wave give twice the waves of eight for the same matrix: the
// launcher takes them when eight leave SIMDs without a wave.
template <int DT, int RPW, int NW, int MAXNB, bool XQ, bool PAIR = false>
__global__ __launch_bounds__(64 * NW) void k_matvec_chain(MatvecArgs a) {
  static_assert(XQ || !PAIR, "the pair form quantizes its input");
  static_assert(!PAIR || NW % 2 == 0, "the pair form splits the waves between the matrices");
  constexpr int CH = Layout<DT>::CH;
  constexpr int LPR = 64 / RPW;                           // lanes (and blocks of a group) per row
  static_assert(RPW == 8 || RPW == 4, "a row's lanes lie in one DPP row");
  static_assert((PAIR ? NW / 2 : NW) * RPW <= TILE, "a work-group's rows lie in one tile");
  constexpr int MAXG = (MAXNB + LPR - 1) / LPR;
  // groups in flight: every group of a row when they fit (no loads past
  // the row's end), else a ring of 16 / CH refilled in batches of four
  constexpr int D = MAXG <= 16 / CH ? MAXG : 16 / CH;
  static_assert(MAXG <= D || D % 4 == 0, "a refilled ring takes batches of four");
  constexpr int SPL = (MAXNB + 63) / 64;                  // scale pieces per lane
  constexpr int NT = 64 * NW;
  constexpr int BPP = NT / 8;                             // x blocks per pass (XQ)
  constexpr int XP = XQ ? (MAXNB + BPP - 1) / BPP : 1;    // passes
  constexpr int APT = XQ ? 1 : (MAXNB * 3 + NT - 1) / NT; // activation pieces per thread
  // a scale piece: the wave's RPW rows' f16 scales of one block
  typedef typename std::conditional<RPW == 8, u32x4, u32x2>::type Piece;
  // (unconditional staging stores: room for every thread's pieces or blocks)
  constexpr int ACT_PIECES = XQ ? XP * BPP * 3 : APT * NT;
  __shared__ __attribute__((aligned(16))) u32x4 s_actv[(ACT_PIECES + 2) / 3 * 3];
  __shared__ Piece s_scl[NW][SPL * 64];
  ActBlock* s_act = (ActBlock*)s_actv;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = a.nb, nbg = (nb + LPR - 1) / LPR;
  // PAIR (Expert::forward's gate and up): waves NW/2 .. NW - 1 take the
  // second matrix's rows of the same row range as waves 0 .. NW/2 - 1 take
  // the first's, and the work-group writes silu(first) * second
  constexpr int RW = PAIR ? NW / 2 : NW;  // row chains per matrix
  const int half = PAIR ? wave / RW : 0;
  const int wv = wave - half * RW;
  if (PAIR && half) {
    a.codes = a.codes2;
    a.scales = a.scales2;
  }
  // The row groups of a 32-row tile share its lines (codes when a wave
  // takes 4 rows, scales always); work-group g runs on XCD g % 8, so when
  // the grid allows, the groups of one tile get ids of one residue class (a
  // permutation of the row groups)
  constexpr int PER_TILE = TILE / (RW * RPW);
  size_t grp = blockIdx.x;
  if (PER_TILE > 1 && gridDim.x % (8 * PER_TILE) == 0) {
    const size_t gx = grp & 7, gj = grp >> 3;
    grp = (gx + 8 * (gj / PER_TILE)) * PER_TILE + gj % PER_TILE;
  }
  const size_t rowg = (grp * RW + wv) * RPW;  // the wave's first row
  const size_t tile = rowg / TILE;
  const int r = lane / LPR, j = lane % LPR;
  const int rt = (int)(rowg % TILE) + r;
  const uint8_t* cbase = a.codes + (tile * nb * CH * TILE + rt) * 16;
  // the RPW rows' scales of block b: one piece at sp + b * TILE * 2 / sizeof(Piece)
  const Piece* sp = (const Piece*)(a.scales + tile * nb * TILE + rowg % TILE);

  // The loads the staging waits for come first, then the ring; scheduling
  // barriers keep that order (loads return in order, so the staging's wait
  // then leaves the ring in flight), and every staging store is
  // unconditional (clamped values past the row's end, never read), so no
  // load is sunk into a branch behind the ring.
  Piece sv[SPL];
#pragma unroll
  for (int m = 0; m < SPL; m++)
    sv[m] = sp[(size_t)min(lane + 64 * m, nb - 1) * (TILE * 2 / sizeof(Piece))];
  f32x4 xv[XP];
  u32x4 av[APT];
  if constexpr (XQ) {
#pragma unroll
    for (int p = 0; p < XP; p++) {
      const int b = min((int)(threadIdx.x >> 3) + BPP * p, nb - 1);
      xv[p] = *(const f32x4*)(a.x + (size_t)b * QK + 4 * (lane & 7));
    }
  } else {
#pragma unroll
    for (int m = 0; m < APT; m++)
      av[m] = ((const u32x4*)a.act)[min((int)threadIdx.x + NT * m, nb * 3 - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 cw[D][CH];
  // group q's codes into ring slot d (groups past the end are clamped to
  // the last: in-bounds loads that are never used)
  auto load = [&](int d, int q) {
    const int b = min(min(q, nbg - 1) * LPR + j, nb - 1);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[d][c] = __builtin_nontemporal_load((const u32x4*)(cbase + ((size_t)b * CH + c) * TILE * 16));
  };
#pragma unroll
  for (int d = 0; d < D; d++) {
    load(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }

  // staging: the wave's scale pieces, and the activation blocks (all waves)
#pragma unroll
  for (int m = 0; m < SPL; m++) s_scl[wave][lane + 64 * m] = sv[m];
  if constexpr (XQ) {
#pragma unroll
    for (int p = 0; p < XP; p++) quant_block8(xv[p], lane & 7, s_act + (threadIdx.x >> 3) + BPP * p);
  } else {
#pragma unroll
    for (int m = 0; m < APT; m++) s_actv[threadIdx.x + NT * m] = av[m];
  }
  __syncthreads();
  const uint16_t* scl16 = (const uint16_t*)s_scl[wave];

  float acc = 0.0f;  // row r's dot product (valid in lane LPR r)
  // Groups q0 .. q0 + D - 1 from the ring; with RELOAD each batch's ring
  // slots then take the groups D further on (clamped past the end).
  auto pass = [&](int q0, auto reload) {
#pragma unroll
    for (int d0 = 0; d0 < D; d0 += 4) {
      const int ni = D - d0 < 4 ? D - d0 : 4;  // groups of this batch (compile time)
      const int qb = q0 + d0;
      if (qb < nbg) {  // wave-uniform; the batch's terms, then their sums in order
        float t[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          if (i < ni) {
            const int b = min((qb + i) * LPR + j, nb - 1);
            t[i] = block_term<DT>(cw[d0 + i], scl16[b * RPW + r], s_act + b);
          }
        }
        if (qb + ni <= nb / LPR) {  // whole groups (wave-uniform): plain adds in block order
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (i < ni) acc = row_fold(acc + t[i], t[i], std::make_integer_sequence<int, LPR - 1>{});
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            if (i < ni) {
              // groups past the row's end have n <= 0 and add nothing
              const int n = nb - (qb + i) * LPR;  // blocks of the group inside the row
              acc = n > 0 ? acc + t[i] : acc;
              acc = row_fold_n(acc, t[i], n, std::make_integer_sequence<int, LPR - 1>{});
            }
          }
        }
      }
      if constexpr (decltype(reload)::value) {
#pragma unroll
        for (int i = 0; i < 4; i++) load(d0 + i, qb + i + D);
      }
    }
  };
  // One pass when every group fits the ring (the usual case: no refills, so
  // each batch waits only for its own groups); else unconditional refills,
  // which keep the wait counts exact across the loop's iterations.
  if constexpr (MAXG <= D) {
    pass(0, std::false_type{});
  } else {
#pragma unroll 1
    for (int q0 = 0; q0 < nbg; q0 += D) pass(q0, std::true_type{});
  }
  const size_t row = rowg + r;
  if constexpr (PAIR) {
    // h = silu(g) * u of the work-group's rows (the gate/up epilogue's
    // expression), by wave 0 with every lane taking part in the exp table
    __shared__ float s_gu[2][RW * RPW];
    if (j == 0) s_gu[half][wv * RPW + r] = acc;
    __syncthreads();
    if (wave == 0) {
      ExpTable tab;
      tab.load();
      const int i = lane % (RW * RPW);
      const float h = wave_silu(s_gu[0][i], tab) * s_gu[1][i];
      const size_t hrow = grp * RW * RPW + lane;
      if (lane < RW * RPW && hrow < (size_t)a.rows) a.out[hrow] = h;
    }
  } else {
    if (j == 0 && row < (size_t)a.rows) a.out[row] = acc;
  }
}

// ===========================================================================
// General shapes
// ===========================================================================
//
// WeightMatrix::matvec for rows of any length, one lane per row: each lane
// folds its row's block terms (d_w * d_x) * isum left to right from +0.0
// (src/tensor/quant.rs:115-144), the 32 rows of a tile reading 512 or
// 1024 contiguous bytes per block.  The activation blocks go through LDS in
// chunks of 64.  The path for shapes the chain kernels do not take.
template <int DT>
__global__ __launch_bounds__(64) void k_matvec_rows(RowsArgs a) {
  constexpr int CH = Layout<DT>::CH;
  __shared__ __attribute__((aligned(16))) u32x4 s_act[64 * 3];
  const int lane = threadIdx.x;
  const int y = blockIdx.y;
  const size_t row = (size_t)blockIdx.x * 64 + lane;  // < padded rows
  const int nb = a.nb;
  const size_t e = a.route ? (size_t)a.route[y] : 0;
  const uint8_t* cbase = a.codes + e * a.codes_stride + ((row / TILE) * nb * CH * TILE + row % TILE) * 16;
  const uint16_t* sbase = a.scales + e * a.scales_stride + (row / TILE) * nb * TILE + row % TILE;
  const u32x4* act = (const u32x4*)(a.act + (size_t)(y / a.act_div) * nb);
  float acc = 0.0f;
  for (int b0 = 0; b0 < nb; b0 += 64) {
    const int n = min(64, nb - b0);
    __syncthreads();  // the previous chunk's reads are done
#pragma unroll
    for (int m = 0; m < 3; m++) {
      const int i = lane + 64 * m;
      if (i < n * 3) s_act[i] = act[(size_t)b0 * 3 + i];
    }
    __syncthreads();
    const ActBlock* sa = (const ActBlock*)s_act;
    int b = 0;
    for (; b + 4 <= n; b += 4) {  // four blocks' loads, then their terms in order
      u32x4 c[4][CH];
      uint16_t sc[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int q = 0; q < CH; q++)
          c[i][q] = *(const u32x4*)(cbase + ((size_t)(b0 + b + i) * CH + q) * TILE * 16);
        sc[i] = sbase[(size_t)(b0 + b + i) * TILE];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) acc = acc + block_term<DT>(c[i], sc[i], sa + b + i);
    }
    for (; b < n; b++) {
      u32x4 c[CH];
#pragma unroll
      for (int q = 0; q < CH; q++) c[q] = *(const u32x4*)(cbase + ((size_t)(b0 + b) * CH + q) * TILE * 16);
      acc = acc + block_term<DT>(c, sbase[(size_t)(b0 + b) * TILE], sa + b);
    }
  }
  if (row < (size_t)a.rows) a.out[(size_t)y * a.out_stride + row] = acc;
}

// h = silu(g) * u (src/expert/mod.rs:99-101, src/ops/activation.rs:5-7),
// quantized as Q8Activations::quantize does, 8 lanes per block.
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ g,
                                                      const float* __restrict__ u, size_t nblocks,
                                                      ActBlock* __restrict__ h) {
  const size_t blk = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) / 8;
  const int j = threadIdx.x & 7;
  if (blk >= nblocks) return;  // uniform across the 8-lane group
  const f32x4 gv = *(const f32x4*)(g + blk * QK + 4 * j);
  const f32x4 uv = *(const f32x4*)(u + blk * QK + 4 * j);
  f32x4 hv;
  hv.x = silu(gv.x) * uv.x;
  hv.y = silu(gv.y) * uv.y;
  hv.z = silu(gv.z) * uv.z;
  hv.w = silu(gv.w) * uv.w;
  quant_block8(hv, j, h + blk);
}

// MoeLayer::route (src/model/moe.rs:36-53) for any number of experts, one
// work-group per token: softmax_in_place (src/ops/activation.rs:11-21: the
// maximum, exp(v - max) with glibc's expf, the sum in index order, each
// value divided by it), top_k (src/ops/topk.rs:27-61: k rounds, each
// taking the largest probability by total order, the lower index on ties)
// and the renormalisation (the chosen scores summed best first from -0.0).
constexpr int RW_THREADS = 256;
__global__ __launch_bounds__(RW_THREADS) void k_route_select_wide(
    const float* __restrict__ logits, int E, int k, int normalize, float* __restrict__ ebuf,
    int* __restrict__ route_idx, float* __restrict__ route_w, unsigned long long* __restrict__ stats) {
  __shared__ float s_red[RW_THREADS];
  __shared__ unsigned s_key[RW_THREADS];
  __shared__ int s_idx[RW_THREADS];
  __shared__ float s_sum;
  const int t = blockIdx.x, tid = threadIdx.x;
  const float* lg = logits + (size_t)t * E;
  float* ev = ebuf + (size_t)t * E;
  // the maximum (order-free)
  float mx = -__builtin_huge_valf();
  for (int i = tid; i < E; i += RW_THREADS) mx = fmaxf(mx, lg[i]);
  s_red[tid] = mx;
  __syncthreads();
  for (int w = RW_THREADS / 2; w > 0; w >>= 1) {
    if (tid < w) s_red[tid] = fmaxf(s_red[tid], s_red[tid + w]);
    __syncthreads();
  }
  mx = s_red[0];
  for (int i = tid; i < E; i += RW_THREADS) ev[i] = hale_expf(lg[i] - mx);
  __syncthreads();  // ebuf is written by this work-group only
  if (tid == 0) {
    float sum = 0.0f;
    for (int i = 0; i < E; i++) sum = sum + ev[i];
    s_sum = sum;
  }
  __syncthreads();
  const float sum = s_sum;
  // probabilities, kept as their total-order keys (0: taken)
  unsigned* key = (unsigned*)ev;
  for (int i = tid; i < E; i += RW_THREADS) key[i] = order_key(ev[i] / sum);
  __syncthreads();
  float norm = normalize ? -0.0f : 1.0f;  // thread 0's
  for (int r = 0; r < k; r++) {
    unsigned bk = 0u;
    int bi = 0x7fffffff;
    for (int i = tid; i < E; i += RW_THREADS) {
      const unsigned ki = key[i];
      if (ki > bk) {  // indices ascend per thread: the first of equal keys stays
        bk = ki;
        bi = i;
      }
    }
    s_key[tid] = bk;
    s_idx[tid] = bi;
    __syncthreads();
    for (int w = RW_THREADS / 2; w > 0; w >>= 1) {
      if (tid < w) {
        const unsigned k2 = s_key[tid + w];
        const int i2 = s_idx[tid + w];
        if (k2 > s_key[tid] || (k2 == s_key[tid] && i2 < s_idx[tid])) {
          s_key[tid] = k2;
          s_idx[tid] = i2;
        }
      }
      __syncthreads();
    }
    // (a key of 0 marks a taken element; a probability with that key, the
    // negative NaN of all-ones bits, cannot come out of the division)
    const int win = s_idx[0] < E ? s_idx[0] : 0;
    const float pw = key_value(s_key[0]);
    __syncthreads();
    if (tid == 0) {
      key[win] = 0u;
      route_idx[(size_t)t * k + r] = win;
      route_w[(size_t)t * k + r] = pw;
      if (normalize) norm = norm + pw;
      if (stats) atomicAdd(&stats[win], 1ull);
    }
    __syncthreads();
  }
  if (tid == 0)
    for (int r = 0; r < k; r++) route_w[(size_t)t * k + r] = route_w[(size_t)t * k + r] / norm;
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

// Plain streaming read, the calibration for what one launch can stream from
// HBM: work-group g reads a contiguous chunk of src with sixteen 16-byte
// loads in flight per thread and writes the XOR of every 32-bit word it
// read to out[g] (0 for a work-group whose chunk is empty).
__global__ __launch_bounds__(256) void k_stream_read(const u32x4* __restrict__ src, size_t n16,
                                                     unsigned* __restrict__ out) {
  constexpr int U = 16;
  const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = min(n16, (size_t)blockIdx.x * chunk), b1 = min(n16, b0 + chunk);
  unsigned acc = 0;
  size_t i = b0 + threadIdx.x;
  for (; i + (size_t)(U - 1) * 256 < b1; i += (size_t)U * 256) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(src + i + u * 256);
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < b1; i += 256) {
    const u32x4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) acc ^= (unsigned)__shfl_xor((int)acc, o);
  __shared__ unsigned s_w[4];
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = s_w[0] ^ s_w[1] ^ s_w[2] ^ s_w[3];
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

hipError_t launch_decode_ref(int dtype, const void* src, size_t n, float* out, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const unsigned grid = (unsigned)((n + 255) / 256);
  const uint8_t* b = (const uint8_t*)src;
  const bool a = (uintptr_t)src % (dtype == F32 ? 4 : 2) == 0;
#define HALE_DECODE_REF(D)                                                            \
  if (dtype == D)                                                                     \
    return a ? launch(k_decode_ref<D, true>, grid, 256, 0, st, b, n, out)            \
             : launch(k_decode_ref<D, false>, grid, 256, 0, st, b, n, out);
  HALE_DECODE_REF(F32)
  HALE_DECODE_REF(F16)
  HALE_DECODE_REF(BF16)
  HALE_DECODE_REF(Q8_0)
  HALE_DECODE_REF(Q4_0)
#undef HALE_DECODE_REF
  return hipErrorInvalidValue;
}

hipError_t launch_decode_tiles(int dtype, const uint8_t* codes, const uint16_t* scales,
                               size_t row0, size_t nrows, size_t cols, float* out,
                               hipStream_t st) {
  const size_t n = nrows * cols;
  if (n == 0) return hipSuccess;
  const unsigned grid = (unsigned)((n + 255) / 256);
  const int nb = (int)(cols / QK);
  if (dtype == Q8_0) return launch(k_decode_tiles<Q8_0>, grid, 256, 0, st, codes, scales, row0, nrows, nb, out);
  if (dtype == Q4_0) return launch(k_decode_tiles<Q4_0>, grid, 256, 0, st, codes, scales, row0, nrows, nb, out);
  return hipErrorInvalidValue;
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

hipError_t launch_route_select_quant(const float* logits, int E, int k, int normalize, int T,
                                    int* route_idx, float* route_w, const float* x,
                                    size_t nblocks, ActBlock* act, hipStream_t st) {
  if (T < 1 || E < 1 || E > ROUTE_MAX_E || k < 1 || k > E || k > 64) return hipErrorInvalidValue;
  if ((uintptr_t)x % 16) {  // the quantization share needs 16-byte loads
    hipError_t e = launch_act_quant(x, nblocks, act, st);
    if (e != hipSuccess) return e;
    return launch_route_select(logits, E, k, normalize, T, route_idx, route_w, nullptr, st);
  }
  const size_t groups = (size_t)T + (nblocks + 7) / 8;
  if (groups > 0x7fffffffu) return hipErrorInvalidValue;
  return launch(k_route_select_quant, (unsigned)groups, 64, 0, st, logits, E, k, normalize, T,
                route_idx, route_w, x, nblocks, act);
}

hipError_t launch_route_logits(const float* router, const float* x, int H, int E, int T,
                               ActBlock* act, float* logits, hipStream_t st) {
  if (H > ROUTE_MAX_H || E > ROUTE_MAX_E || H % QK || E < 1 || T < 1) return hipErrorInvalidValue;
  if (T >= ROUTE_TILED_MIN_T) {
    // many tokens: 16 experts x 8 tokens per work-group, the activation
    // blocks quantized by the same launch
    // 16 experts per work-group, or 8 when 16 would leave CUs without one
    // (Qwen3-30B-A3B layer on the row chains at 48 / 64 / 76 tokens: 103.2-
    // 103.6 / 112.7-113.2 / 120.3-120.6 -> 101.8-101.9 / 112.3-112.7 /
    // 118.9-119.3 us per step; Qwen3-235B-A22B at 48: 315-317 -> 310-313)
    const int tt = (T + RT_T - 1) / RT_T;
    if ((E + 15) / 16 * tt < 256) {
      const dim3 grid8((E + 7) / 8, tt);
      return launch(k_route_logits_tiled<8>, grid8, 512, 0, st, router, x, H, E, T, logits, act);
    }
    const dim3 grid((E + 15) / 16, tt);
    return launch(k_route_logits_tiled<16>, grid, 1024, 0, st, router, x, H, E, T, logits, act);
  }
  dim3 grid(E, T);
  if (H <= 8 * ROUTE_THREADS)
    return launch(k_route_logits<2>, grid, ROUTE_THREADS, 0, st, router, x, H, E, act, logits);
  if (H <= 16 * ROUTE_THREADS)
    return launch(k_route_logits<4>, grid, ROUTE_THREADS, 0, st, router, x, H, E, act, logits);
  return launch(k_route_logits<8>, grid, ROUTE_THREADS, 0, st, router, x, H, E, act, logits);
}

hipError_t launch_route_select(const float* logits, int E, int k, int normalize, int T,
                               int* route_idx, float* route_w, unsigned long long* stats,
                               hipStream_t st) {
  if (E > ROUTE_MAX_E || k > 64 || k > E || k < 1 || T < 1) return hipErrorInvalidValue;
  return launch(k_route_select, T, 64, 0, st, logits, E, k, normalize, route_idx, route_w, stats);
}

// Tokens per decode pass from which the gate/up and down kernels load
// weights through the caches: tokens that share an expert then read its
// bytes from L2 or the last-level cache.  Measured on Qwen3-30B-A3B and
// Qwen3-235B-A22B layers (top-8 of 128), graph replay: ordinary loads
// 1-5% faster from 12 tokens up, non-temporal ones up to 7% faster at 2-7
// tokens (and on Mixtral's top-2 of 8).
constexpr int CACHED_LOAD_TOKENS = 12;

// Work-groups on the busiest XCD of a grid of width gx and height rows whose
// columns x < cols hold the tiles (a column past them, the selector's, ends
// early): work-group x + gx y runs on XCD (x + gx y) % 8.
static long busiest_xcd(long cols, long gx, long rows) {
  long cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < 8; j++) {  // the rows y = j (mod 8)
    const long ny = rows > j ? (rows - j + 7) / 8 : 0;
    const int off = (int)((gx % 8) * j % 8);
    for (int c = 0; c < 8; c++) {  // columns x = c - off (mod 8)
      const long r0 = (c - off + 8) % 8;
      cnt[c] += (cols > r0 ? (cols - r0 + 7) / 8 : 0) * ny;
    }
  }
  long m = 0;
  for (int c = 0; c < 8; c++) m = cnt[c] > m ? cnt[c] : m;
  return m;
}

hipError_t launch_gemv(int dtype, int epi, const GemvArgs& a, int groups, int slots,
                       hipStream_t st) {
  if (groups == 0 || slots == 0) return hipSuccess;
  if (a.nb < 1 || a.nb > GEMV_MAX_NB) return hipErrorInvalidValue;
  if (a.x && (epi != EPI_GATE_UP || a.nb > GEMV_X_MAX_NB || ((uintptr_t)a.x & 15)))
    return hipErrorInvalidValue;
  if (a.logits && (epi != EPI_GATE_UP || a.E > ROUTE_MAX_E || slots > 64 || slots > a.E))
    return hipErrorInvalidValue;
  const int T = a.tokens > 1 ? a.tokens : 1;
  if (T > 1 && (!a.logits || a.x || a.slots != slots || (long)slots * T > 65535))
    return hipErrorInvalidValue;
  const bool many = a.logits && a.E > 256;  // selection state for up to 1024 experts
  // Gate/up: one work-group per (32-row tile, token and slot), or per two tiles when
  // the grid would not be resident at once (at 128 VGPRs and 1024 threads
  // per CU: 256 work-groups of 16 waves, 512 of 8), so that no second round
  // runs on a partly filled GPU.  With routing, one more column of
  // work-groups holds the selector.
  // q4_0 gate/up in sixteen-wave work-groups, for rows of one 64-block
  // chunk and, when it fits, for longer rows with more than 256 tile-slots
  // (eight-wave work-groups of one tile would put two on some CUs and one on
  // the rest, or run in two rounds): each work-group takes the fewest tiles
  // of one slot, 1, 2, 4 or 8, that keep the grid at one work-group per CU
  // (256), runs one selection and folds its tiles' chunks in sequence.  Per
  // step, graph replay: Qwen3-30B-shaped layer at 4 / 7 tokens (four /
  // eight tiles) 31.0-31.5 / 41.9-42.4 -> 28.1 / 38.4 us; Qwen3-235B-shaped
  // at 1 / 2 / 4 tokens (two / four / eight) 27.8 / 45.7 / 73.1 -> 27.4 /
  // 42.4-43.5 / 67.7; Mixtral-shaped at 1 / 2 (four / eight) 43.9 / 75.8 ->
  // 42.4-42.7 / 71.8-72.1.  Longer rows whose tiles do not fit at eight per
  // work-group keep the eight-wave form.
  // "Fits" counts per XCD: work-group x + X y runs on XCD (x + X y) % 8, so
  // an even grid width X puts whole columns on a few XCDs (Qwen3-30B-shaped
  // layer at 9 tokens, eight tiles: X = 3 + the selector, 36 work-groups on
  // each of six XCDs' 32 CUs and the selector column alone on the other
  // two).  Rows of one chunk whose tiles fit at no width take the fewest
  // tiles per work-group by rounds x (tiles + one tile's worth for the
  // work-group's selection and staging): at 9 / 10 tokens of that layer four
  // tiles, 57.3 / 58.5 -> 48 / 50 us per step.
  const long tslots = (long)groups * slots * T;
  const bool sel_col = a.logits != nullptr;
  auto xcd_rounds = [&](int p) {  // rounds of the busiest XCD, 32 CUs each
    const long cols = (groups + p - 1) / p;
    return (busiest_xcd(cols, cols + (sel_col ? 1 : 0), (long)slots * T) + 31) / 32;
  };
  int ipw16 = 0;  // tiles per sixteen-wave work-group
  for (int p = 1; p <= 8 && !ipw16; p *= 2)
    if (xcd_rounds(p) <= 1) ipw16 = p;
  const bool q4gu = dtype == Q4_0 && epi == EPI_GATE_UP && !(a.logits && a.E > 256);
  const bool pair16 = q4gu && a.nb > 64 && tslots > 256 && ipw16 > 0;
  if (q4gu && a.nb <= 64 && !ipw16) {
    long best = 0;
    for (int p = 1; p <= 8; p *= 2) {
      const long cost = xcd_rounds(p) * (p + 1);
      if (!ipw16 || cost < best) ipw16 = p, best = cost;
    }
  }
  auto grid_of = [&](int nw) {
    GemvArgs b = a;
    b.tiles = groups;
    b.ipw = epi == EPI_GATE_UP && (long)groups * slots * T > 256L * (16 / nw) ? 2 : 1;
    if (nw == 16 && q4gu) b.ipw = ipw16;
    return std::make_pair(dim3((groups + b.ipw - 1) / b.ipw + (a.logits ? 1 : 0), slots * T), b);
  };
  const bool cached = T >= CACHED_LOAD_TOKENS;
#define HALE_GEMV_LAUNCH(D, E, W, ME, NT) \
  return launch(k_gemv<D, E, W, ME, NT>, gb.first, 64 * W, 0, st, gb.second)
#define HALE_GEMV_CASE(D, E, W)                                        \
  if (dtype == D && epi == E) {                                        \
    const auto gb = grid_of(W);                                        \
    if (E == EPI_GATE_UP && cached) {                                  \
      if (many) HALE_GEMV_LAUNCH(D, EPI_GATE_UP, W, ROUTE_MAX_E, false); \
      HALE_GEMV_LAUNCH(D, EPI_GATE_UP, W, 256, false);                 \
    }                                                                  \
    if (many) HALE_GEMV_LAUNCH(D, E, W, ROUTE_MAX_E, true);            \
    HALE_GEMV_LAUNCH(D, E, W, 256, true);                              \
  }
  HALE_GEMV_CASE(Q8_0, EPI_PLAIN, 4)
  HALE_GEMV_CASE(Q8_0, EPI_GATE_UP, 8)
  HALE_GEMV_CASE(Q4_0, EPI_PLAIN, 4)
  // sixteen waves leave 128 VGPRs, too few for the selection state of more
  // than 256 experts: those layers take the eight-wave form
  if (dtype == Q4_0 && epi == EPI_GATE_UP && (a.nb <= 64 || pair16) && !many) {
    const auto gb = grid_of(16);
    if (cached) HALE_GEMV_LAUNCH(Q4_0, EPI_GATE_UP, 16, 256, false);
    HALE_GEMV_LAUNCH(Q4_0, EPI_GATE_UP, 16, 256, true);
  }
  HALE_GEMV_CASE(Q4_0, EPI_GATE_UP, 8)
#undef HALE_GEMV_CASE
#undef HALE_GEMV_LAUNCH
  return hipErrorInvalidValue;
}

hipError_t launch_down_combine(int dtype, const DownArgs& a, hipStream_t st) {
  const unsigned T = a.tokens > 1 ? (unsigned)a.tokens : 1u;
  const dim3 groups((unsigned)(padded_rows((size_t)a.rows) / DR), T);
  if (groups.x == 0) return hipSuccess;
  if (a.nb < 1 || a.slots < 1 || a.slots > DOWN_MAX_SLOTS || T > 65535) return hipErrorInvalidValue;
  // Block terms spread over sixteen waves per work-group (k_down_tile):
  // for one and two routes on every shape measured (H 1024-5120, down rows
  // of 8-448 blocks, 1-3 tokens; Mixtral-8x7B-shaped q4_0 layer: 15.2-16.9
  // -> 11.8 us at one token; top-1, H 5120, I 8192: 9.6 -> 7.2 us, H 4096,
  // I 14336: 14.1 -> 8.3 us); for three routes over rows of at most 128
  // blocks (step per layer, H 2048 / I 1024: 14.1 -> 13.1 us at one token,
  // 21.6 -> 17.9 at four; H 4096 / I 2048: 23.1 -> 21.1-21.7, 51.7 ->
  // 40.6-42.0); for four to eight over rows of at most 128 blocks when its
  // 16-row groups give every CU one (Qwen3-235B-shaped layer, 48-block
  // rows: down 8.0 -> 6.4-7.5 us at one token, 23.2 -> 17.3 at four; top-7,
  // H 4096: step 31.4 -> 29.6 us, 69.8 -> 65.1-65.7 at four; H 2048 at one
  // token has 128 such groups, and there the wave-per-route kernel's 8-row
  // groups are as fast or faster); from three routes only for calls below
  // CACHED_LOAD_TOKENS (its weight loads are non-temporal).
  // Work-groups of 16 rows (half a tile) or 32: the size whose busiest CU
  // gets fewer rows, ceil(groups / 256 CUs) x rows per group, 32 on a tie
  // (one token of H 4096: 256 groups of 16 against 128 of 32 that would
  // leave half the CUs idle; two tokens: 256 of 32).
  {
    const size_t prow = padded_rows((size_t)a.rows);
    const bool spread =
        ((a.slots == 1 || a.slots == 2) && a.nb <= DOWN_TILE_MAX_NB) ||
        (a.slots >= 3 && a.slots <= 8 && a.nb <= 128 && (int)T < CACHED_LOAD_TOKENS &&
         (a.slots == 3 || prow / 16 * T >= 256));
    if (spread) {
      const uint32_t lds = (uint32_t)down_tile_lds(a.slots, a.nb);
      auto busiest = [&](size_t rw) { return (prow / rw * T + 255) / 256 * rw; };
      const bool half = busiest(16) < busiest(32);
      const dim3 grid((unsigned)(prow / (half ? 16 : 32)), T);
#define HALE_DOWN_TILE(S_, NW_)                                                                     \
  do {                                                                                              \
    if (half && dtype == Q8_0) return launch(k_down_tile<Q8_0, S_, NW_, 16, 1>, grid, 64 * NW_, lds, st, a); \
    if (half && dtype == Q4_0) return launch(k_down_tile<Q4_0, S_, NW_, 16, 2>, grid, 64 * NW_, lds, st, a); \
    if (dtype == Q8_0) return launch(k_down_tile<Q8_0, S_, NW_, 32, 1>, grid, 64 * NW_, lds, st, a);         \
    if (dtype == Q4_0) return launch(k_down_tile<Q4_0, S_, NW_, 32, 2>, grid, 64 * NW_, lds, st, a);         \
  } while (0)
      // sixteen waves, twelve for three slot pairs (five or six routes)
      switch (a.slots) {
        case 1: HALE_DOWN_TILE(1, 16); break;
        case 2: HALE_DOWN_TILE(2, 16); break;
        case 3: HALE_DOWN_TILE(3, 16); break;
        case 4: HALE_DOWN_TILE(4, 16); break;
        case 5: HALE_DOWN_TILE(5, 12); break;
        case 6: HALE_DOWN_TILE(6, 12); break;
        case 7: HALE_DOWN_TILE(7, 16); break;
        case 8: HALE_DOWN_TILE(8, 16); break;
      }
#undef HALE_DOWN_TILE
      return hipErrorInvalidValue;
    }
  }
  // A wave per (slot, 8 rows) pays off when few routes leave many rows per
  // work-group (three routes that k_down_tile does not take); top-4 and
  // wider use the block-group pipeline.
  if (a.slots <= 3 && a.nb <= DOWN_CHAIN_MAX_NB && a.slots * a.nb <= DOWN_ACT_MAX &&
      down_chain_waves(a.slots, 8) * a.nb <= DOWN_SCL_MAX) {
    const int rg = down_chain_rows(a.slots);
    const dim3 grid((unsigned)(padded_rows((size_t)a.rows) / rg), T);
    // eight rows per wave: four (twice the waves, each row's chunks in
    // 64-byte halves of the tile layout's lines) measured slower on every
    // top-1 and top-2 shape tried, the small ones included
    const int rpw = 8;
    const unsigned threads = 64 * down_chain_waves(a.slots, rpw);
    const uint32_t lds = (uint32_t)down_chain_lds(a.slots, a.nb, rpw);
    const int nbg = (a.nb + 7) / 8;
#define HALE_DOWN_CHAIN(D)                                                                     \
  do {                                                                                         \
    if (dtype == Q8_0) return launch(k_down_chain<Q8_0, 8, D>, grid, threads, lds, st, a);     \
    if (dtype == Q4_0) return launch(k_down_chain<Q4_0, 8, D>, grid, threads, lds, st, a);     \
  } while (0)
    // (k_down_chain sizes its activation staging by these bounds)
    if (nbg <= 4) HALE_DOWN_CHAIN(4);
    if (nbg <= 8 || dtype == Q8_0) HALE_DOWN_CHAIN(8);
    HALE_DOWN_CHAIN(16);
#undef HALE_DOWN_CHAIN
  }
  // 4 to 8 routes over rows of at most 128 blocks: a wave per route
  if (a.slots >= 4 && a.slots <= 8 && a.nb <= 128) {
    const unsigned threads = 64u * (unsigned)a.slots;
    const bool cached = (int)T >= CACHED_LOAD_TOKENS;
#define HALE_DOWN_SLOTS(N)                                                                         \
  do {                                                                                             \
    if (dtype == Q8_0 && cached) return launch(k_down_slots<Q8_0, N, false>, groups, threads, 0, st, a); \
    if (dtype == Q4_0 && cached) return launch(k_down_slots<Q4_0, N, false>, groups, threads, 0, st, a); \
    if (dtype == Q8_0) return launch(k_down_slots<Q8_0, N>, groups, threads, 0, st, a);            \
    if (dtype == Q4_0) return launch(k_down_slots<Q4_0, N>, groups, threads, 0, st, a);            \
  } while (0)
    if (a.nb <= 24) HALE_DOWN_SLOTS(24);
    if (a.nb <= 32) HALE_DOWN_SLOTS(32);
    if (a.nb <= 48) HALE_DOWN_SLOTS(48);
    if (a.nb <= 64) HALE_DOWN_SLOTS(64);
    HALE_DOWN_SLOTS(128);
#undef HALE_DOWN_SLOTS
  }
  if (dtype == Q8_0) return launch(k_down_combine<Q8_0, 8>, groups, 512, 0, st, a);
  if (dtype == Q4_0) return launch(k_down_combine<Q4_0, 8>, groups, 512, 0, st, a);
  return hipErrorInvalidValue;
}

// Four rows per wave when eight would leave fewer waves than the GPU's
// 1024 SIMDs; work-groups of one tile (NW = 32 / RPW waves) when that still
// gives at least 256 work-groups, else half or a quarter of a tile, so
// small matrices spread over more CUs.
static bool matvec_spread(int nb, size_t rows) {
  return nb >= 32 && nb <= DOWN_TILE_MAX_NB && padded_rows(rows) <= 65536;
}

bool matvec_takes_x(int nb, size_t rows) { return nb <= MATVEC_XQ_MAX_NB || matvec_spread(nb, rows); }

hipError_t launch_matvec(int dtype, const MatvecArgs& a, hipStream_t st) {
  if (a.nb < 1 || a.rows < 1) return hipErrorInvalidValue;
  if (dtype != Q8_0 && dtype != Q4_0) return hipErrorInvalidValue;
  const bool xq = a.x != nullptr;
  // Rows of 32 to 512 blocks, at most 65,536 of them: the block terms
  // spread over a work-group's waves (k_down_tile, plain), 512-byte
  // wave-loads where the chain kernel's read 64- or 128-byte pieces (4096
  // x 4096, cold: q8_0 7.40 -> 6.20 us, q4_0 5.72 -> 5.25; 14336 x 4096
  // q4_0 10.7 -> 8.7; 4096 x 14336 13.7 -> 10.3 with x quantized in the
  // kernel (rows of up to 512 blocks), no quantization launch before it;
  // 768 x 2048 q8_0 3.8 -> 3.4).  Rows of 24 blocks (2048 x 768: 3.06 against 3.23-3.48 us) and
  // 151,936 rows (51.9 against 52.5-53.8 us) stay on the chain kernel.
  if (matvec_spread(a.nb, (size_t)a.rows) && (xq ? ((uintptr_t)a.x & 15) == 0 : a.act != nullptr)) {
    DownArgs d{};
    d.codes = a.codes;
    d.scales = a.scales;
    d.nb = a.nb;
    d.rows = a.rows;
    d.hact = a.act;
    d.slots = 1;
    d.out = a.out;
    d.tokens = 1;
    d.x = a.x;
    const size_t prow = padded_rows((size_t)a.rows);
    auto busiest = [&](size_t rw) { return (prow / rw + 255) / 256 * rw; };
    const bool half = busiest(16) < busiest(32);
    const dim3 grid((unsigned)(prow / (half ? 16 : 32)));
    const uint32_t lds = (uint32_t)down_tile_lds(1, a.nb);
    if (half && dtype == Q8_0) return launch(k_down_tile<Q8_0, 1, 16, 16, 1, true>, grid, 1024, lds, st, d);
    if (half) return launch(k_down_tile<Q4_0, 1, 16, 16, 2, true>, grid, 1024, lds, st, d);
    if (dtype == Q8_0) return launch(k_down_tile<Q8_0, 1, 16, 32, 1, true>, grid, 1024, lds, st, d);
    return launch(k_down_tile<Q4_0, 1, 16, 32, 2, true>, grid, 1024, lds, st, d);
  }
  if (xq && (((uintptr_t)a.x & 15) || a.nb > MATVEC_XQ_MAX_NB)) return hipErrorNotSupported;
  if (!xq && (!a.act || a.nb > MATVEC_MAX_NB)) return hipErrorNotSupported;
  const size_t prow = padded_rows((size_t)a.rows);
  const int rpw = prow / 8 >= 1024 ? 8 : 4;
  // waves per work-group: a whole tile, half or a quarter (quantizing x in
  // the kernel takes at least two waves: one leaves too many x loads per lane)
  int nw = TILE / rpw;
  while (nw > 2 && prow / (size_t)(rpw * nw) < 256) nw /= 2;
  const unsigned grid = (unsigned)(prow / (size_t)(rpw * nw));
#define HALE_MV(D, R, NW, MAXNB, XQ) launch(k_matvec_chain<D, R, NW, MAXNB, XQ>, grid, 64 * NW, 0, st, a)
#define HALE_MV_NW(D, MAXNB, XQ)                                                           \
  do {                                                                                     \
    if (rpw == 8) return nw == 4 ? HALE_MV(D, 8, 4, MAXNB, XQ) : HALE_MV(D, 8, 2, MAXNB, XQ); \
    return nw == 8 ? HALE_MV(D, 4, 8, MAXNB, XQ)                                            \
                   : (nw == 4 ? HALE_MV(D, 4, 4, MAXNB, XQ) : HALE_MV(D, 4, 2, MAXNB, XQ)); \
  } while (0)
#define HALE_MV_NB(D, XQ)                                                  \
  do {                                                                     \
    if (a.nb <= 32) HALE_MV_NW(D, 32, XQ);                                 \
    if (a.nb <= 64) HALE_MV_NW(D, 64, XQ);                                 \
    if (a.nb <= MATVEC_XQ_MAX_NB) HALE_MV_NW(D, MATVEC_XQ_MAX_NB, XQ);      \
  } while (0)
#undef HALE_MV
#define HALE_MV(D, R, NW, MAXNB, XQ) launch(k_matvec_chain<D, R, NW, MAXNB, XQ>, grid, 64 * NW, 0, st, a)
  if (dtype == Q8_0) {
    if (xq) HALE_MV_NB(Q8_0, true);
    HALE_MV_NB(Q8_0, false);
    HALE_MV_NW(Q8_0, MATVEC_MAX_NB, false);
  } else {
    if (xq) HALE_MV_NB(Q4_0, true);
    HALE_MV_NB(Q4_0, false);
    HALE_MV_NW(Q4_0, MATVEC_MAX_NB, false);
  }
#undef HALE_MV_NB
#undef HALE_MV_NW
#undef HALE_MV
}

// Both matrices in one launch: a work-group's first half of waves folds the
// first matrix's rows, its second half the same rows of the second, and it
// writes silu(first) * second; rows per wave and waves chosen as for one
// matrix of twice the rows.
hipError_t launch_matvec_pair(int dtype, const MatvecArgs& a, hipStream_t st) {
  if (a.nb < 1 || a.rows < 1 || !a.x || !a.codes2 || !a.scales2) return hipErrorInvalidValue;
  if (dtype != Q8_0 && dtype != Q4_0) return hipErrorInvalidValue;
  if (((uintptr_t)a.x & 15) || a.nb > MATVEC_XQ_MAX_NB) return hipErrorNotSupported;
  const size_t prow = padded_rows((size_t)a.rows);
  const int rpw = 2 * prow / 8 >= 1024 ? 8 : 4;
  int nw = 2 * TILE / rpw;  // waves per work-group, both matrices
  while (nw > 2 && 2 * prow / (size_t)(rpw * nw) < 256) nw /= 2;
  const unsigned grid = (unsigned)(2 * prow / (size_t)(rpw * nw));
#define HALE_MV(D, R, NW, MAXNB) launch(k_matvec_chain<D, R, NW, MAXNB, true, true>, grid, 64 * NW, 0, st, a)
#define HALE_MV_NW(D, MAXNB)                                                                   \
  do {                                                                                         \
    if (rpw == 8)                                                                              \
      return nw == 8 ? HALE_MV(D, 8, 8, MAXNB) : (nw == 4 ? HALE_MV(D, 8, 4, MAXNB) : HALE_MV(D, 8, 2, MAXNB)); \
    return nw == 16 ? HALE_MV(D, 4, 16, MAXNB)                                                 \
                    : (nw == 8 ? HALE_MV(D, 4, 8, MAXNB)                                       \
                               : (nw == 4 ? HALE_MV(D, 4, 4, MAXNB) : HALE_MV(D, 4, 2, MAXNB))); \
  } while (0)
#define HALE_MV_NB(D)                                                  \
  do {                                                                 \
    if (a.nb <= 32) HALE_MV_NW(D, 32);                                 \
    if (a.nb <= 64) HALE_MV_NW(D, 64);                                 \
    HALE_MV_NW(D, MATVEC_XQ_MAX_NB);                                   \
  } while (0)
  if (dtype == Q8_0) HALE_MV_NB(Q8_0);
  else HALE_MV_NB(Q4_0);
#undef HALE_MV_NB
#undef HALE_MV_NW
#undef HALE_MV
}

hipError_t launch_matvec_rows(int dtype, const RowsArgs& a, int ny, hipStream_t st) {
  if (a.nb < 1 || a.rows < 1 || ny < 1 || ny > 65535 || a.act_div < 1) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(padded_rows((size_t)a.rows) / 64), (unsigned)ny);
  if (dtype == Q8_0) return launch(k_matvec_rows<Q8_0>, grid, 64, 0, st, a);
  if (dtype == Q4_0) return launch(k_matvec_rows<Q4_0>, grid, 64, 0, st, a);
  return hipErrorInvalidValue;
}

hipError_t launch_swiglu_quant(const float* g, const float* u, size_t nblocks, ActBlock* h,
                               hipStream_t st) {
  if (nblocks == 0) return hipSuccess;
  if (((uintptr_t)g & 15) || ((uintptr_t)u & 15)) return hipErrorInvalidValue;
  return launch(k_swiglu_quant, blocks_for(nblocks * 8, 256), 256, 0, st, g, u, nblocks, h);
}

hipError_t launch_route_select_wide(const float* logits, int E, int k, int normalize, int T,
                                    float* ebuf, int* route_idx, float* route_w,
                                    unsigned long long* stats, hipStream_t st) {
  if (T < 1 || E < 1 || k < 1 || k > E) return hipErrorInvalidValue;
  return launch(k_route_select_wide, T, RW_THREADS, 0, st, logits, E, k, normalize, ebuf, route_idx,
                route_w, stats);
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

hipError_t launch_stream_read(const void* src, size_t n16, unsigned workgroups, unsigned* out,
                              hipStream_t st) {
  if (workgroups < 1 || workgroups > 65535) return hipErrorInvalidValue;
  return launch(k_stream_read, workgroups, 256, 0, st, (const u32x4*)src, n16, out);
}

hipError_t launch_copy(void* dst, const void* src, size_t n16, hipStream_t st) {
  if (!n16) return hipSuccess;
  const unsigned grid = (unsigned)std::min<size_t>(blocks_for(n16, 256), 256 * 64);
  return launch(k_copy, grid, 256, 0, st, (u32x4*)dst, (const u32x4*)src, n16);
}

}  // namespace hale
