// kernels_prefill.hip -- expert-grouped multi-token MoE layer on gfx950.
//
// The reference feeds a prompt one token at a time (Transformer::prefill,
// src/model/transformer.rs:231-239), so at the MoE layer token t's output is
// MoeLayer::forward(x_t) (src/model/moe.rs:56-70), independent of the other
// tokens.  Here the T*k (token, slot) assignments are grouped by expert and
// each expert's group runs as an int8 MFMA matrix product; every output
// keeps the reference's bits:
//   - one v_mfma_i32_32x32x32_i8 covers exactly one 32-element quantization
//     block, so it yields the block's exact i32 dot sums (dot_q8_0 /
//     dot_q4_0, src/tensor/quant.rs:115-144);
//   - each output element then adds (d_w * d_x) * isum to its f32 sum block
//     after block, the reference's left-to-right order;
//   - SiLU, the q8 requantization of h, the route-order combine and the
//     routing itself are the decode path's exact formulas.
//
// Pipeline: route (per token) -> group (counts, prefix sums, stable scatter,
// tile list) -> grouped gate/up -> grouped down -> combine.  Calls of few
// tokens per expert run the same pipeline with row-chain kernels in place
// of the matrix products (and no gather).
#pragma clang fp contract(off)

#include "hale_device.h"
#include "kernels.h"
#include "prefill.h"

namespace hale {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int TM = 32;          // assignments (rows) per tile
constexpr int TN = 128;         // output columns per work-group (4 waves x 32)
constexpr int GROUP_WAVES = 16;  // waves of the grouping kernel
constexpr int GROUP_MAX_E = 1024;
// Activations of the grouped kernels, tile-major: per (tile, 32-column
// block) the codes as the MFMA's A operand wants them, [K half][32 rows]
// [16 B] (the halves' element order follows the weight operand: see the
// grouped matrix products below), then the 32 rows' f32 scales, so one
// wave's operand of a block is 1 KB contiguous and its scales one line.  The gate/up input is gathered
// into this layout from the token-major blocks; the requantized SiLU output
// is written in it by the gate/up kernel for the down kernel.
constexpr int TACT_CODES = 2 * TM * 16;
constexpr int TACT_BLOCK = TACT_CODES + TM * 4;

struct Tile {
  int expert;
  int row0;  // first sorted position
  int rows;  // 1..tile rows (TM; band_rows for the row-chain kernels)
  int pad;
};

// ---------------------------------------------------------------------------
// grouping: histogram, prefix sums, stable scatter, tile list
// ---------------------------------------------------------------------------
//
// One work-group of 16 waves.  Assignment a = t*k + s is routed to expert
// route_idx[a].  Sorted position of a = (assignments to lower experts) +
// (earlier assignments to the same expert), so each expert's group keeps
// token order.  Wave w owns a contiguous slice of the assignments; lanes
// with equal experts in a 64-wide chunk are found with ballots over the
// expert's bits.  The layer's routing counts (stats, optional) grow by each
// expert's group size here rather than by one atomic per assignment, which
// would serialize on the popular experts' counters.  Each expert's group is
// cut into tiles of at most tm rows.

__device__ __forceinline__ unsigned long long match_mask(int e, int nbits, bool valid) {
  unsigned long long m = __ballot(valid);
  for (int b = 0; b < nbits; b++) {
    const unsigned long long v = __ballot(((e >> b) & 1) != 0);
    m &= ((e >> b) & 1) ? v : ~v;
  }
  return valid ? m : 0ull;
}

__global__ __launch_bounds__(64 * GROUP_WAVES) void k_group(const int* __restrict__ route_idx, int A,
                                                            int E, int* __restrict__ perm,
                                                            int* __restrict__ pos_of,
                                                            Tile* __restrict__ tiles,
                                                            int* __restrict__ ntiles,
                                                            unsigned long long* __restrict__ stats,
                                                            int tm) {
  __shared__ int cnt[GROUP_WAVES][GROUP_MAX_E];
  __shared__ int scan_a[GROUP_MAX_E];
  __shared__ int scan_t[GROUP_MAX_E];
  __shared__ int wsum_a[GROUP_WAVES], wsum_t[GROUP_WAVES];
  static_assert(GROUP_MAX_E == 64 * GROUP_WAVES, "one thread per expert in the scan");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  int nbits = 0;
  while ((1 << nbits) < E) nbits++;
  for (int q = 0; q < GROUP_WAVES; q++)
    if (tid < E) cnt[q][tid] = 0;
  __syncthreads();
  const int slice = (A + GROUP_WAVES * 64 - 1) / (GROUP_WAVES * 64) * 64;
  const int a0 = w * slice, a1 = min(A, a0 + slice);
  const unsigned long long lt = (1ull << lane) - 1ull;

  // The experts of GPRE chunks of 64 assignments are loaded together (one
  // memory round trip per batch rather than per chunk).
  constexpr int GPRE = 16;
  auto load_batch = [&](int cb, int* ev) {
#pragma unroll
    for (int j = 0; j < GPRE; j++) {
      const int a = cb + 64 * j + lane;
      ev[j] = a < a1 ? route_idx[a] : 0;
    }
  };

  // pass 1: per-wave counts.  The first batch stays in registers for pass 2
  // (a wave's whole slice while A <= 16 x 64 x GROUP_WAVES).
  auto count_batch = [&](int cb, const int* ev) {
#pragma unroll
    for (int j = 0; j < GPRE; j++) {
      const int a = cb + 64 * j + lane;
      if (cb + 64 * j >= a1) break;  // wave-uniform
      const bool valid = a < a1;
      const int e = ev[j];
      const unsigned long long m = match_mask(e, nbits, valid);
      if (valid && (m >> lane) == 1ull) cnt[w][e] += __popcll(m);  // highest lane of its group
    }
  };
  int ev0[GPRE];
  load_batch(a0, ev0);
  count_batch(a0, ev0);
  for (int cb = a0 + 64 * GPRE; cb < a1; cb += 64 * GPRE) {
    int ev[GPRE];
    load_batch(cb, ev);
    count_batch(cb, ev);
  }
  __syncthreads();

  // totals, expert offsets and tile offsets: inclusive scans over experts,
  // thread e holding expert e (E <= 1024 = the work-group's threads), a
  // shuffle scan within each wave, then the totals of the lower waves
  {
    int tot = 0;
    if (tid < E)
      for (int q = 0; q < GROUP_WAVES; q++) tot += cnt[q][tid];
    int va = tot, vt = (tot + tm - 1) / tm;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int ua = __shfl_up(va, off), ut = __shfl_up(vt, off);
      if (lane >= off) {
        va += ua;
        vt += ut;
      }
    }
    if (lane == 63) {
      wsum_a[w] = va;
      wsum_t[w] = vt;
    }
    __syncthreads();
    for (int q = 0; q < w; q++) {
      va += wsum_a[q];
      vt += wsum_t[q];
    }
    scan_a[tid] = va;
    scan_t[tid] = vt;
  }
  __syncthreads();
  // per-wave bases: offset(e) + counts of lower waves; tile list
  for (int e = tid; e < E; e += 64 * GROUP_WAVES) {
    const int total = cnt[0][e];
    int base = e ? scan_a[e - 1] : 0;
    const int tot_e = scan_a[e] - base;
    if (stats) stats[e] += (unsigned long long)tot_e;  // routing counts, one add per expert
    int run = base;
    for (int q = 0; q < GROUP_WAVES; q++) {
      const int c = q ? cnt[q][e] : total;
      cnt[q][e] = run;
      run += c;
    }
    const int t0 = e ? scan_t[e - 1] : 0;
    for (int i = 0; i * tm < tot_e; i++) {
      Tile tl;
      tl.expert = e;
      tl.row0 = base + i * tm;
      tl.rows = min(tm, tot_e - i * tm);
      tl.pad = 0;
      tiles[t0 + i] = tl;
    }
  }
  if (tid == 0) *ntiles = scan_t[E - 1];
  __syncthreads();

  // pass 2: stable positions
  auto scatter_batch = [&](int cb, const int* ev) {
#pragma unroll
    for (int j = 0; j < GPRE; j++) {
      const int a = cb + 64 * j + lane;
      if (cb + 64 * j >= a1) break;  // wave-uniform
      const bool valid = a < a1;
      const int e = ev[j];
      const unsigned long long m = match_mask(e, nbits, valid);
      if (valid) {
        const int pos = cnt[w][e] + __popcll(m & lt);
        perm[pos] = a;
        pos_of[a] = pos;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (valid && (m >> lane) == 1ull) cnt[w][e] += __popcll(m);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };
  scatter_batch(a0, ev0);
  for (int cb = a0 + 64 * GPRE; cb < a1; cb += 64 * GPRE) {
    int ev[GPRE];
    load_batch(cb, ev);
    scatter_batch(cb, ev);
  }
}

// ---------------------------------------------------------------------------
// grouped matrix products
// ---------------------------------------------------------------------------
//
// A work-group takes one tile (expert e, 32 sorted rows) and 128 output
// columns; wave w owns columns [n0, n0+32).  Per quantization block b a wave
// issues one 32x32x32 int8 MFMA (two for gate/up): lane l supplies row
// l%32's 16 activation codes of K half h = l/32 and column l%32's 16 weight
// codes of the same half.  q8_0: half h is elements 16h..16h+15, exactly one
// 16-byte chunk of the tile layout.  q4_0: half h is the lane's 8 bytes
// 8h..8h+7 of the column's chunk, both nibbles: elements 8h..8h+7 (low) then
// 16+8h..16+8h+7 (high), and the activation tiles hold the codes in that
// order.  Result element j of lane l is row (j%4) + 4*(l/32) + 8*(j/4),
// column l%32.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// B operand from loaded codes.  q8_0: the signed codes of a 16-byte chunk as
// they are.  q4_0: the unsigned nibbles n (0..15) of the lane's 8 bytes, low
// nibbles then high; the MFMA's accumulator then starts at -8 * sum(x) of
// the row so that it ends at sum((n - 8) * x), the same integer as with
// signed codes.
__device__ __forceinline__ v4i weight_operand(u32x4 v) {
  v4i r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}
__device__ __forceinline__ v4i weight_operand(u32x2 w) {
  const u32x4 v = {w[0] & 0x0f0f0f0fu, w[1] & 0x0f0f0f0fu, (w[0] >> 4) & 0x0f0f0f0fu,
                   (w[1] >> 4) & 0x0f0f0f0fu};
  v4i r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

struct GroupedArgs {
  // weights of the layer, expert e at base + e * stride
  const uint8_t* codes;
  const uint16_t* scales;
  const uint8_t* codes2;  // up (gate/up kernel)
  const uint16_t* scales2;
  size_t codes_stride, scales_stride;
  int nb;        // K blocks
  int ncols;     // N (I for gate/up, H for down)
  const Tile* tiles;
  const int* ntiles;
  const uint8_t* tin;     // input: [tile][nb] TACT_BLOCK
  uint8_t* tout;          // gate/up output: [tile][ncols/32] TACT_BLOCK
  float* y;               // down output: [A][ncols] by sorted position
};

// Work items are (tile, 128-column group) pairs, ordered by blocks of CGB
// column groups, then tile, then column group within the block.  The XCDs
// take work-groups in turn (linear id % 8), so work-group L runs item
// (L % 8) * per + L / 8: each XCD works through a contiguous run of items,
// where neighbouring items share a tile's activation rows (same tile, next
// column group) or an expert's weights (next tile of the same expert, same
// column groups), and both stay in that XCD's L2.
constexpr int CGB = 3;

// At most 128 VGPRs (four waves per SIMD): the kernel is bound by its VALU
// work, and a fourth wave hides more of the matrix-core latency than the
// registers above 128 would save.
// FMA (down projection only): each block term joins its sum in one fused
// multiply-add, (d_w d_x) * isum + sum rounded once, instead of the
// reference's product then sum (two roundings); one VALU operation fewer
// per element and block, at a relative error far below the f32 output's
// tolerance.  The gate/up output is requantized, so it keeps the exact fold.
template <int DT, bool GATE_UP, bool FMA = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_grouped(
    GroupedArgs a) {
  static_assert(!(GATE_UP && FMA), "the gate/up fold is exact");
  constexpr int CH = Layout<DT>::CH;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = *a.ntiles;
  const int ncg = (a.ncols + TN - 1) / TN;
  const int total = nt * ncg;
  const int per = (total + 7) >> 3;
  const int item = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= per || item >= total) return;
  const int ncb = min(CGB, ncg - (item / (nt * CGB)) * CGB);  // column groups in this block
  const int cb = item / (nt * CGB);
  const int rem = item - cb * nt * CGB;
  const int ti = rem / ncb;
  const int colg = cb * CGB + rem % ncb;
  const Tile tl = a.tiles[ti];
  const int n0 = colg * TN + wave * 32;
  if (n0 >= a.ncols) return;
  const int h = lane >> 5;
  const int nb = a.nb;

  // Operands are read through buffer resources over wave-uniform planes
  // (the tile's activations; the expert's 32-column weight tile) with a
  // per-lane offset, so the block loop advances only scalar offsets.
  const int rn = lane & 31;  // column within the tile
  const int tile_n = n0 / TILE;
  const size_t e = (size_t)__builtin_amdgcn_readfirstlane(tl.expert);
  const size_t cplane = (size_t)tile_n * nb * CH * TILE * 16, splane = (size_t)tile_n * nb * TILE;
  const unsigned cbytes = (unsigned)(nb * CH * TILE * 16), sbytes = (unsigned)(nb * TILE * 2);
  const auto ra = buffer_rsrc(a.tin + (size_t)ti * nb * TACT_BLOCK, (unsigned)(nb * TACT_BLOCK));
  const auto rg = buffer_rsrc(a.codes + e * a.codes_stride + cplane, cbytes);
  const auto rsg = buffer_rsrc(a.scales + e * a.scales_stride + splane, sbytes);
  const auto ru = buffer_rsrc(GATE_UP ? a.codes2 + e * a.codes_stride + cplane : a.codes, cbytes);
  const auto rsu = buffer_rsrc(GATE_UP ? a.scales2 + e * a.scales_stride + splane : a.scales, sbytes);
  const int xoff = h * (TM * 16) + rn * 16, dxoff = TACT_CODES + rn * 4;
  const int coff = rn * 16 + (DT == Q8_0 ? h * TILE * 16 : 8 * h);
  const int soff = rn * 2;

  // accumulators start at +0.0 like the reference's `let mut total = 0.0`,
  // so no sum can become -0.0: the sign of a zero scale product never shows
  v16f accg = {}, accu = {};
  // 8-row groups of the tile that hold real rows (the others stay at zero:
  // gate/up then writes h = 0 for them, and down does not store them)
  const int ngr = __builtin_amdgcn_readfirstlane((tl.rows + 7) >> 3);

  // Operands of one block.
  struct Ops {
    using WT = std::conditional_t<DT == Q4_0, u32x2, u32x4>;
    u32x4 xr;
    WT wg, wu;
    float dx;
    uint16_t dg, du;
  };
  // Weights use ordinary (cached) loads: every tile of an expert reads the
  // same column group, and neighbouring items run on one XCD, so the later
  // tiles find the lines in L2.
  auto load = [&](Ops& o, int b) {
    const int ab = b * TACT_BLOCK, cb = b * (CH * TILE * 16), sb = b * (TILE * 2);
    o.xr = __builtin_amdgcn_raw_buffer_load_b128(ra, xoff, ab, 0);
    o.dx = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, dxoff, ab, 0));
    if constexpr (DT == Q4_0) {
      o.wg = __builtin_amdgcn_raw_buffer_load_b64(rg, coff, cb, 0);
    } else {
      o.wg = __builtin_amdgcn_raw_buffer_load_b128(rg, coff, cb, 0);
    }
    o.dg = __builtin_amdgcn_raw_buffer_load_b16(rsg, soff, sb, 0);
    if constexpr (GATE_UP) {
      if constexpr (DT == Q4_0) {
        o.wu = __builtin_amdgcn_raw_buffer_load_b64(ru, coff, cb, 0);
      } else {
        o.wu = __builtin_amdgcn_raw_buffer_load_b128(ru, coff, cb, 0);
      }
      o.du = __builtin_amdgcn_raw_buffer_load_b16(rsu, soff, sb, 0);
    }
  };
  // q4_0 offset term: B = -8 in every byte makes the product -8 * sum(x) of
  // the row, broadcast over the columns
  const v4i minus8 = {(int)0xf8f8f8f8u, (int)0xf8f8f8f8u, (int)0xf8f8f8f8u, (int)0xf8f8f8f8u};
  // `valid` is false for the clamped blocks past the end: their scale
  // products are zero, so they add +0 or -0, which leaves every sum as it is
  // split (q4_0 gate/up only): gate folded before up's product is formed,
  // skipping the tile's padded 8-row groups, for tiles that have them
  auto compute = [&](const Ops& o, bool valid, auto split) {
    v4i xa;
    __builtin_memcpy(&xa, &o.xr, 16);
    v16i c0 = {};
    if constexpr (DT == Q4_0) c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, minus8, c0, 0, 0, 0);
    // Scale products d_w[col] * d_x[row] of the whole 32x32 tile on the
    // matrix core, which rounds each product exactly like a VALU multiply
    // (only the sign of a zero product can differ, and that cannot reach an
    // accumulator that starts at +0).  gate/up: one two-block K=1 outer
    // product, A[row] = d_x in both halves of the wave and B[col] = the gate
    // scale in lanes 0-31 (block 0, results 0-15), the up scale in lanes
    // 32-63 (block 1, results 16-31).  down: a K=2 outer product whose
    // second K column is zero: lanes 0-31 hold A[row][0] = d_x and
    // B[0][col] = d_w.
    v16f pg, pu;
    if constexpr (GATE_UP) {
      const float ax = valid ? o.dx : 0.0f;
      const v32f p2 = __builtin_amdgcn_mfma_f32_32x32x1f32(ax, h2f(lane < 32 ? o.dg : o.du),
                                                            v32f{}, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        pg[j] = p2[j];
        pu[j] = p2[16 + j];
      }
    } else {
      const bool use = lane < 32 && valid;
      pg = __builtin_amdgcn_mfma_f32_32x32x2f32(use ? o.dx : 0.0f, use ? h2f(o.dg) : 0.0f, v16f{},
                                                0, 0, 0);
    }
    // The fold, by 8-row groups: results 4q .. 4q + 3 of a lane are rows
    // 8q .. 8q + 7 of the tile (both halves of the wave), so a group past the
    // tile's real rows is skipped as a whole (wave-uniform); its rows'
    // results are never stored.  Gate's sums are folded before up's product
    // is formed, so one set of 16 block sums is live at a time.
    auto fold = [&](v16f& acc, const v16f& p, const v16i& isum) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        if (q < ngr) {
#pragma unroll
          for (int j = 4 * q; j < 4 * q + 4; j++) {
            if constexpr (FMA) {
              acc[j] = __builtin_fmaf(p[j], (float)isum[j], acc[j]);
            } else {
              acc[j] = acc[j] + p[j] * (float)isum[j];
            }
          }
        }
      }
    };
    if constexpr (GATE_UP && DT == Q4_0 && !decltype(split)::value) {
      // q4_0 gate/up of a full tile folds gate and up together: splitting
      // them costs a second offset product per block, on a kernel that is
      // bound by VALU and MFMA issue
      const v16i ig = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, weight_operand(o.wg), c0, 0, 0, 0);
      const v16i iu = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, weight_operand(o.wu), c0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        accg[j] = accg[j] + pg[j] * (float)ig[j];
        accu[j] = accu[j] + pu[j] * (float)iu[j];
      }
    } else {
      fold(accg, pg, __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, weight_operand(o.wg), c0, 0, 0, 0));
      if constexpr (GATE_UP) {
        __builtin_amdgcn_sched_barrier(0);
        // q4_0: the offset product again rather than kept live over the fold
        v16i c1 = {};
        if constexpr (DT == Q4_0) c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, minus8, c1, 0, 0, 0);
        fold(accu, pu, __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, weight_operand(o.wu), c1, 0, 0, 0));
      }
    }
  };
  // NS operand sets in a ring: block b + NS - 1 loads while block b
  // computes (four sets for the down projection; two for gate/up, whose
  // sets are larger and which is bound by its VALU work, not by latency).
  // The loop body has no branches (so the load counters are tracked across
  // iterations): blocks past the end are loaded clamped to the last block
  // and computed with zero scales.  The scheduling barriers keep each
  // block's loads where they are issued; left free, the scheduler sinks
  // some of them next to their use to save registers, and the wave then
  // waits out a whole L2 round trip.
  constexpr int NS = GATE_UP ? 2 : 4;
  auto run = [&](auto split) {
    Ops S[NS];
#pragma unroll
    for (int j = 0; j < NS - 1; j++) load(S[j], min(j, nb - 1));
    for (int b = 0; b < nb; b += NS) {
#pragma unroll
      for (int j = 0; j < NS; j++) {
        load(S[(j + NS - 1) % NS], min(b + j + NS - 1, nb - 1));
        __builtin_amdgcn_sched_barrier(0);
        compute(S[j], b + j < nb, split);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto epilogue = [&]() {
  if constexpr (GATE_UP) {
    // h = silu(g) * u, quantized per (row, 32-column block): the 32 columns
    // of a row sit in the 32 lanes of one half.  All 32 rows of the tile are
    // written; rows past tl.rows (the last row repeated, with h = 0 in the
    // groups of 8 rows that the fold skipped) only ever feed result rows
    // that the down kernel does not store.
    ExpTable tab;
    tab.load();
    const int nbo = a.ncols / QK;
    uint8_t* tb = a.tout + ((size_t)ti * nbo + n0 / QK) * TACT_BLOCK;
    // element rn of the block: q8_0 half rn / 16, byte rn % 16; q4_0 half
    // (rn / 8) % 2, byte rn % 8 (+ 8 for elements 16..31)
    const int qoff = DT == Q4_0 ? ((rn >> 3) & 1) * (TM * 16) + (rn & 7) + 8 * (rn >> 4)
                                : (rn >> 4) * (TM * 16) + (rn & 15);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int row = (j % 4) + 4 * h + 8 * (j / 4);
      const float hv = wave_silu(accg[j], tab) * accu[j];
      float scale;
      int qsum;
      const int qv = quant_block_lane(hv, &scale, &qsum);
      tb[qoff + row * 16] = (uint8_t)(int8_t)qv;
      if (rn == 0) *(float*)(tb + TACT_CODES + row * 4) = scale;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int row = (j % 4) + 4 * h + 8 * (j / 4);
      if (row < tl.rows) a.y[(size_t)(tl.row0 + row) * a.ncols + n0 + rn] = accg[j];
    }
  }
  };
  // each path with its own epilogue, so no registers merge between them
  if (GATE_UP && DT == Q4_0 && ngr < 4) {  // wave-uniform
    run(std::true_type{});
    epilogue();
  } else {
    run(std::false_type{});
    epilogue();
  }
}

// ---------------------------------------------------------------------------
// row-chain grouped products (few assignments per expert)
// ---------------------------------------------------------------------------
//
// A call of tens of tokens gives most experts one to a few assignments, so
// the 32-row products above are mostly padding and each wave's chain of K
// blocks is bound by its own latency.  Here a band tile holds at most
// NR assignments of one expert, and lane l of a wave owns one weight
// row (gate/up: lanes 0-31 the gate rows, 32-63 the up rows of one 32-row
// I-tile; down: two 32-row H-tiles).  The lane walks its row's K blocks
// with a ring of D blocks in flight and adds each block's term
// (d_w * d_x) * isum to every assignment's sum, block after block: the
// reference's dot_q8_0 / dot_q4_0 and its left-to-right fold
// (src/tensor/quant.rs:115-144).  An assignment's activation block is the
// same for every lane of the wave (staged in LDS by the work-group, read by
// all lanes at once); the gate/up input is read in place (token-major,
// through perm), with no gather.
//
// Assignments per band tile (band_rows): two, or four when a call gives the
// experts two or more assignments each on average and a gate/up row holds
// at least 2 KB (q8_0 from H 2048, q4_0 from H 4096) over rows of at most
// 256 blocks.  Four terms per weight block then outweigh the longer
// per-block chains; with shorter rows or fewer assignments per expert the
// ring's loads wait on those chains and two per tile are faster.  Measured
// per layer, graph replay: Qwen3-235B-A22B q4_0 at 32 / 48 / 60 / 72 tokens
// 283.7 / 317.5 / 352.4 / 388.8 us with two, 261.6 / 306 / 333.9 / 369.2
// with four (at 9 / 16 tokens 129.3 / 188.1 against 149.0 / 197.4);
// Qwen3-30B-A3B q8_0 at 32 / 48 / 64 / 72: 136.7 / 157 / 169.5 / 179.2
// against 122.6 / 150.7 / 159.2 / 159.5; Qwen3-30B-A3B q4_0 (1,152-byte
// rows) slower with four at every size (64 tokens 111.7 against 118.2);
// Mixtral-8x7B (448-block down rows) at 8 / 12 tokens 198.4 / 243.6
// against 234.7 / 254.2.
constexpr int BAND_WAVES = 4;

struct BandArgs {
  const uint8_t* codes;  // gate (gate/up) or down weights, expert e at + e * stride
  const uint16_t* scales;
  const uint8_t* codes2;  // up (gate/up)
  const uint16_t* scales2;
  size_t codes_stride, scales_stride;
  int nb;   // K blocks
  int ntc;  // 32-row output tiles: I / 32 (gate/up), H / 32 (down)
  int rows;  // output rows (down stores rows below it)
  int wpt;   // waves per band tile: ntc (gate/up), ceil(ntc / 2) (down)
  const Tile* tiles;
  const int* ntiles;
  const int* perm;  // gate/up: sorted position p is assignment perm[p], token perm[p] / k
  int k;
  const ActBlock* act;  // gate/up: [T][nb] by token; down: [A][nb] by sorted position
  ActBlock* hout;       // gate/up output: [A][I / 32] by sorted position
  float* y;             // down output: [A][H] by sorted position
};

// LDS of a band work-group: the tile's activation blocks [nr][nb] (48
// bytes each), then per wave the double-buffered scales of its ring cycle,
// [2][2 halves][D blocks][32 rows] f16.
constexpr int BAND_MAX_NB = 512;  // K blocks per row (48 KB of activations at two rows)
static size_t band_lds(int nr, int nb, int d) {
  return (size_t)nr * nb * sizeof(ActBlock) + (size_t)BAND_WAVES * 2 * 2 * d * TILE * 2;
}

// Work-group: BAND_WAVES waves of one band tile (gpt work-groups per tile,
// waves past the tile's wpt only help stage).  The XCDs take work-groups in
// turn (linear id % 8), so work-group L runs item (L % 8) * per + L / 8:
// the work-groups of one tile run on one XCD.  All NR assignments of a
// tile are computed; a shorter tile repeats its last, whose copies are
// never stored.
//
// Each lane's row streams through a ring of D code blocks; per ring cycle
// (D blocks) the wave loads the cycle after next's scales as whole 16-byte
// pieces (8 rows of one block) and parks them in LDS, so a block costs one
// load per lane.  The activation blocks of block b come from LDS: for q4_0
// rows of up to 256 blocks every lane reads the same words (a broadcast:
// Qwen3-30B q4_0 layer 109.4 -> 102.7 us at 48 tokens, Qwen3-235B 326 ->
// 319); for q8_0 and longer rows, where the broadcast measured 1-2 %
// slower, each lane reads one word (word i of assignment j in lane 12 j +
// i) and readlane moves it to a scalar register.  NT: non-temporal weight
// loads, when experts hold about two assignments or fewer (each expert's
// weights read once); with more, ordinary loads let an expert's later tiles
// find its weights in L2.
// MAXNB: the K blocks the activation staging is sized for (256, or 512 for
// longer rows: its loads need registers that cost the others occupancy).
template <int DT, bool GATE_UP, int D, bool NT, int MAXNB, int NR>
__global__ __launch_bounds__(64 * BAND_WAVES) void k_band(BandArgs a) {
  extern __shared__ __attribute__((aligned(16))) u32x4 s_band[];
  constexpr int CH = Layout<DT>::CH;
  static_assert(NR == 2 || (NR == 4 && MAXNB <= 256), "tiles of two, or of four over rows of at most 256 blocks");
  constexpr int SPL = D / 8;   // scale pieces per lane per cycle
  constexpr int APT = (NR * MAXNB * 3 + 64 * BAND_WAVES - 1) / (64 * BAND_WAVES);  // activation pieces per thread
  static_assert(MAXNB <= BAND_MAX_NB, "the staging fits its bound");
  // activation words by broadcast LDS reads (q4_0 rows of up to 256 blocks)
  // or one word per lane moved to scalar registers (q8_0, longer rows)
  constexpr bool BCAST = DT == Q4_0 && MAXNB <= 256;
  static_assert(NR * 12 <= 64, "one word per lane");
  static_assert(D % 8 == 0, "a ring cycle's scales are whole pieces per lane");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nt = *a.ntiles;
  const int gpt = (a.wpt + BAND_WAVES - 1) / BAND_WAVES;
  const int wgs = nt * gpt;
  const int per = (wgs + 7) >> 3;
  const int wg = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= per || wg >= wgs) return;  // the whole work-group
  const int ti = wg / gpt;
  const int wt = min((wg - ti * gpt) * BAND_WAVES + wave, a.wpt - 1);  // spare waves repeat the last
  const Tile tl = a.tiles[ti];
  const int nb = a.nb, n = tl.rows;
  const size_t e = (size_t)tl.expert;

  // the tile's activation blocks: loads first, stored once the ring is in
  // flight.  Threads past the last piece load and store it again (the same
  // bytes to the same place), so the loads need no branches.
  const int np = NR * nb * 3;
  u32x4 av[APT];
  {
    int src[APT];
#pragma unroll
    for (int m = 0; m < APT; m++) {
      const int q = min((int)threadIdx.x + m * 64 * BAND_WAVES, np - 1);
      const int j = q / (nb * 3);
      const int p = tl.row0 + min(j, n - 1);
      src[m] = GATE_UP ? a.perm[p] : p;
    }
#pragma unroll
    for (int m = 0; m < APT; m++) {
      const int q = min((int)threadIdx.x + m * 64 * BAND_WAVES, np - 1);
      const int rem = q - q / (nb * 3) * (nb * 3);
      const size_t row = GATE_UP ? (size_t)(src[m] / a.k) : (size_t)src[m];
      av[m] = ((const u32x4*)(a.act + row * nb))[rem];
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  const int half = lane >> 5, r = lane & 31;
  const size_t tile = GATE_UP ? (size_t)wt : 2 * (size_t)wt + half;
  const uint8_t* crow = (GATE_UP && half ? a.codes2 : a.codes) + e * a.codes_stride +
                        (tile * nb * CH * TILE + r) * 16;
  const uint16_t* splane = (GATE_UP && half ? a.scales2 : a.scales) + e * a.scales_stride +
                           tile * nb * TILE;
  uint16_t* s_scl = (uint16_t*)((char*)s_band + (size_t)NR * nb * sizeof(ActBlock)) +
                    wave * (2 * 2 * D * TILE);
  // scale pieces of ring cycle c: piece m of lane r is block c D + q / 4,
  // rows 8 (q % 4) .. + 7, q = r + 32 m (blocks past the end: the last)
  u32x4 sp[SPL];
  auto scale_load = [&](int c) {
#pragma unroll
    for (int m = 0; m < SPL; m++) {
      const int q = r + 32 * m;
      const int b = min(c * D + q / 4, nb - 1);
      sp[m] = *(const u32x4*)(splane + (size_t)b * TILE + 8 * (q % 4));
    }
  };
  auto scale_store = [&](int c) {
    uint16_t* dst = s_scl + ((c & 1) * 2 + half) * D * TILE;
#pragma unroll
    for (int m = 0; m < SPL; m++) {
      const int q = r + 32 * m;
      *(u32x4*)(dst + (q / 4) * TILE + 8 * (q % 4)) = sp[m];
    }
  };
  u32x4 cw[D][CH];
  // blocks past the row's end load the last block (in bounds; unused)
  auto load = [&](int d, int b) {
    b = min(b, nb - 1);
#pragma unroll
    for (int c = 0; c < CH; c++)
      cw[d][c] = load_weights<NT>((const u32x4*)(crow + ((size_t)b * CH + c) * TILE * 16));
  };
  scale_load(0);
  __builtin_amdgcn_sched_barrier(0);
  // the ring's first loads in slot order, as the refills come: the loop
  // head then waits for slot 0 alone on every pass, the first included
  // (reordered here, it would wait for all of them on every pass)
#pragma unroll
  for (int d = 0; d < D; d++) {
    load(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int m = 0; m < APT; m++) s_band[min((int)threadIdx.x + m * 64 * BAND_WAVES, np - 1)] = av[m];
  scale_store(0);
  __builtin_amdgcn_sched_barrier(0);
  scale_load(1);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the activation blocks

  const ActBlock* s_act = (const ActBlock*)s_band;
  // (readlane form) the lane's word of block b: word i of assignment j in
  // lane 12 j + i
  const unsigned* aword =
      (const unsigned*)(s_act + (size_t)min(lane / 12, NR - 1) * nb) + lane % 12;
  unsigned aw[D];
  // sums start at +0.0 like the reference's `let mut total = 0.0`
  float acc[NR];
#pragma unroll
  for (int j = 0; j < NR; j++) acc[j] = 0.0f;
  uint16_t sw[D];
#pragma unroll 1
  for (int b0 = 0, c = 0; b0 < nb; b0 += D, c++) {
    const uint16_t* scl = s_scl + ((c & 1) * 2 + half) * D * TILE + r;
#pragma unroll
    for (int d = 0; d < D; d++) {
      sw[d] = scl[d * TILE];
      if constexpr (!BCAST) aw[d] = aword[(size_t)min(b0 + d, nb - 1) * (sizeof(ActBlock) / 4)];
    }
#pragma unroll
    for (int d = 0; d < D; d++) {
      // terms of blocks past the row's end become +0.0 (the sums never
      // hold -0.0, so adding it changes nothing)
      const unsigned keep = b0 + d < nb ? ~0u : 0u;
      // weight codes as the dot products take them: q8_0 the signed bytes;
      // q4_0 the low nibbles (elements 0-15) then the high (16-31), raw
      // 0..15, with 8 * sum(x) taken off the sum
      unsigned w[8];
      if constexpr (DT == Q8_0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          w[i] = cw[d][0][i];
          w[4 + i] = cw[d][1][i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          w[i] = cw[d][0][i] & 0x0f0f0f0fu;
          w[4 + i] = (cw[d][0][i] >> 4) & 0x0f0f0f0fu;
        }
      }
      const float dw = h2f(sw[d]);
#pragma unroll
      for (int j = 0; j < NR; j++) {
        // assignment j's block words: codes 0-7, scale 8, code sum 9
        int x[10];
        if constexpr (BCAST) {  // every lane reads the same LDS words
          const ActBlock* xb = s_act + (size_t)j * nb + min(b0 + d, nb - 1);
          const u32x4 xa0 = *(const u32x4*)xb->q, xa1 = *(const u32x4*)(xb->q + 16);
          const u32x2 xs = *(const u32x2*)&xb->scale;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            x[i] = (int)xa0[i];
            x[4 + i] = (int)xa1[i];
          }
          x[8] = (int)xs[0];
          x[9] = (int)xs[1];
        } else {
          // each word into a scalar register, all before the products (one
          // register reused for each would stall every product on its read)
#pragma unroll
          for (int i = 0; i < 10; i++) x[i] = __builtin_amdgcn_readlane((int)aw[d], 12 * j + i);
          asm volatile("" ::"s"(x[0]), "s"(x[1]), "s"(x[2]), "s"(x[3]), "s"(x[4]), "s"(x[5]),
                       "s"(x[6]), "s"(x[7]), "s"(x[8]), "s"(x[9]));
        }
        // two chains of four dot products (integer sums: any order)
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          s0 = __builtin_amdgcn_sdot4((int)w[i], x[i], s0, false);
          s1 = __builtin_amdgcn_sdot4((int)w[4 + i], x[4 + i], s1, false);
        }
        int isum = s0 + s1;
        if constexpr (DT == Q4_0) isum -= 8 * x[9];
        const float t = (dw * __builtin_bit_cast(float, x[8])) * (float)isum;
        acc[j] = acc[j] + __builtin_bit_cast(float, __builtin_bit_cast(unsigned, t) & keep);
      }
      // the ring slot refills right after its block (left free, the
      // scheduler hoists the refills and holds two rings of registers)
      __builtin_amdgcn_sched_barrier(0);
      load(d, b0 + d + D);
      __builtin_amdgcn_sched_barrier(0);
    }
    scale_store(c + 1);
    __builtin_amdgcn_sched_barrier(0);
    scale_load(c + 2);
    __builtin_amdgcn_sched_barrier(0);
  }
  if ((wg - ti * gpt) * BAND_WAVES + wave >= a.wpt) return;  // a spare wave
  if constexpr (GATE_UP) {
    // h = silu(g) * u of each assignment, quantized to its q8 block of 32
    // rows (lanes 0-31) for the down projection
    ExpTable tab;
    tab.load();
#pragma unroll
    for (int j = 0; j < NR; j++) {
      if (j < n) {  // wave-uniform
        const float u = __shfl(acc[j], lane + 32);
        const float h = wave_silu(acc[j], tab) * u;
        float scale;
        int qsum;
        const int q = quant_block_lane(h, &scale, &qsum);
        if (lane < 32) {
          ActBlock* hb = a.hout + (size_t)(tl.row0 + j) * a.ntc + wt;
          hb->q[lane] = (int8_t)q;
          if (lane == 0) {
            hb->scale = scale;
            hb->qsum = qsum;
          }
        }
      }
    }
  } else {
    const int row = (int)tile * TILE + r;
#pragma unroll
    for (int j = 0; j < NR; j++)
      if (j < n && row < a.rows) a.y[(size_t)(tl.row0 + j) * a.rows + row] = acc[j];
  }
}

// Gather of the gate/up input into the tile layout: work-group (tile, 8
// blocks), thread (block, row): row r of tile ti is token perm[row0 + r] / k
// (rows past the tile's end repeat its last row).  Grid: max_tiles x
// ceil(nb / 8); work-groups past the live tile count exit.  Q4: the q4_0
// order of the halves (elements 0-7 and 16-23, then 8-15 and 24-31).
template <bool Q4>
__global__ __launch_bounds__(256) void k_gather_tiles(const ActBlock* __restrict__ act, int nb,
                                                      const Tile* __restrict__ tiles,
                                                      const int* __restrict__ ntiles,
                                                      const int* __restrict__ perm, int k,
                                                      uint8_t* __restrict__ tin) {
  const int ti = blockIdx.x;
  if (ti >= *ntiles) return;
  const int r = threadIdx.x & 31;
  const int b = blockIdx.y * 8 + (threadIdx.x >> 5);
  if (b >= nb) return;
  const Tile tl = tiles[ti];
  const int tok = perm[tl.row0 + min(r, tl.rows - 1)] / k;
  const ActBlock* src = act + (size_t)tok * nb + b;
  u32x4 lo = *(const u32x4*)src->q;
  u32x4 hi = *(const u32x4*)(src->q + 16);
  if constexpr (Q4) {
    const u32x4 h0 = {lo[0], lo[1], hi[0], hi[1]}, h1 = {lo[2], lo[3], hi[2], hi[3]};
    lo = h0;
    hi = h1;
  }
  uint8_t* dst = tin + ((size_t)ti * nb + b) * TACT_BLOCK;
  *(u32x4*)(dst + r * 16) = lo;
  *(u32x4*)(dst + TM * 16 + r * 16) = hi;
  *(float*)(dst + TACT_CODES + r * 4) = src->scale;
}

// out[t] = 0, then out[t] = out[t] + w[t][s] * y[pos(t, s)] for s in route
// order (MoeLayer::forward's combine, src/model/moe.rs:63-68); pos_of null:
// the rows are in (token, slot) order.  Thread i of
// work-group (c, t) owns columns 4i..4i+3 of column chunk c; the rows of 8
// slots are loaded together before they are added in slot order.
constexpr int COMBINE_COLS = 1024;
__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ y,
                                                 const int* __restrict__ pos_of,
                                                 const float* __restrict__ route_w, int k, int H,
                                                 float* __restrict__ out) {
  const int t = blockIdx.y;
  const int i = blockIdx.x * COMBINE_COLS + 4 * (int)threadIdx.x;
  if (i >= H) return;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < k; s0 += 8) {
    f32x4 v[8];
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int s = min(s0 + j, k - 1);
      w[j] = route_w[(size_t)t * k + s];
      const size_t pos = pos_of ? (size_t)pos_of[(size_t)t * k + s] : (size_t)t * k + s;
      v[j] = *(const f32x4*)(y + pos * H + i);
    }
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (s0 + j < k) acc = acc + w[j] * v[j];
  }
  *(f32x4*)(out + (size_t)t * H + i) = acc;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

hipError_t launch_combine_rows(const float* y, const float* route_w, int k, int H, int T,
                               float* out, hipStream_t st) {
  if (T < 1 || k < 1 || H % 4 || T > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((H + COMBINE_COLS - 1) / COMBINE_COLS), (unsigned)T);
  return launch(k_combine, grid, 256, 0, st, y, (const int*)nullptr, route_w, k, H, out);
}

size_t prefill_min_tokens(size_t) { return 8; }

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

struct WsLayout {
  size_t perm, pos_of, tiles, ntiles, tin, tact, y, total;
  size_t max_tiles;
};

// Calls of at most band_max tokens take the row-chain kernels when the
// tiles' activation blocks fit their LDS staging.
static bool band_on(const PrefillLayer& L, size_t T) {
  return T <= L.band_max && std::max(L.H, L.I) / QK <= BAND_MAX_NB;
}

// Assignments per row-chain tile (see k_band): four when the call gives
// the experts two or more each on average and a gate/up row holds at least
// 2 KB over rows of at most 256 blocks, else two.
static int band_rows(const PrefillLayer& L, size_t T) {
  const size_t A = T * (size_t)L.k;
  const size_t row_bytes = (size_t)(L.H / QK) * (L.dtype == Q8_0 ? 34 : 18);
  return A >= 2 * (size_t)L.E && row_bytes >= 2048 && std::max(L.H, L.I) / QK <= 256 ? 4 : 2;
}

// The row-chain kernels' layout has tiles of band_rows rows, no gathered
// input and the SiLU output as [A][I / 32] activation blocks in `tact`.
static WsLayout ws_layout(const PrefillLayer& L, size_t T) {
  WsLayout w{};
  const size_t A = T * (size_t)L.k;
  const bool band = band_on(L, T);
  const size_t tm = band ? (size_t)band_rows(L, T) : TM;
  w.max_tiles = (A + tm - 1) / tm + (size_t)L.E;
  size_t o = 0;
  w.perm = o;
  o += align256(A * 4);
  w.pos_of = o;
  o += align256(A * 4);
  w.tiles = o;
  o += align256(w.max_tiles * sizeof(Tile));
  w.ntiles = o;
  o += 256;
  w.tin = o;
  if (!band) o += align256(w.max_tiles * (size_t)(L.H / QK) * TACT_BLOCK);
  w.tact = o;
  o += band ? align256(A * (size_t)(L.I / QK) * sizeof(ActBlock))
            : align256(w.max_tiles * (size_t)(L.I / QK) * TACT_BLOCK);
  w.y = o;
  o += align256(A * (size_t)L.H * 4);
  w.total = o;
  return w;
}

size_t prefill_workspace_bytes(const PrefillLayer& L, size_t T) { return ws_layout(L, T).total; }

hipError_t prefill_enqueue(const PrefillLayer& L, void* ws, size_t T, const float* x,
                           const float* logits, float* out, hipStream_t st,
                           const LaunchHook& hook) {
  if (L.E > GROUP_MAX_E || L.k < 1 || L.H % QK || L.I % QK || !ws) return hipErrorInvalidValue;
  const WsLayout w = ws_layout(L, T);
  char* b = (char*)ws;
  int* perm = (int*)(b + w.perm);
  int* pos_of = (int*)(b + w.pos_of);
  Tile* tiles = (Tile*)(b + w.tiles);
  int* ntiles = (int*)(b + w.ntiles);
  uint8_t* tin = (uint8_t*)(b + w.tin);
  uint8_t* tact = (uint8_t*)(b + w.tact);
  float* y = (float*)(b + w.y);
  const int nbh = L.H / QK, nbi = L.I / QK;
  const size_t A = T * (size_t)L.k;
  hipError_t e;
#define HALE_STEP(kind, call)       \
  do {                              \
    hook.on_begin(kind);            \
    e = (call);                     \
    hook.on_end();                  \
    if (e != hipSuccess) return e;  \
  } while (0)

  // 1. route every token and quantize its activations (given logits: one
  // launch for both)
  if (logits) {
    HALE_STEP(K_ROUTE, launch_route_select_quant(logits, L.E, L.k, L.normalize, (int)T,
                                                 L.route_idx, L.route_w, x, T * nbh, L.act, st));
  } else {
    HALE_STEP(K_ROUTE, launch_route_logits(L.router, x, L.H, L.E, (int)T, L.act, L.logits, st));
    HALE_STEP(K_ROUTE, launch_route_select(L.logits, L.E, L.k, L.normalize, (int)T, L.route_idx,
                                           L.route_w, nullptr, st));
  }
  // 2. group assignments by expert
  const bool band = band_on(L, T);
  HALE_STEP(K_GROUP, launch(k_group, 1, 64 * GROUP_WAVES, 0, st, L.route_idx, (int)A, L.E, perm,
                            pos_of, tiles, ntiles, L.stats, band ? band_rows(L, T) : TM));
  if (band) {
    // 3-4. row-chain gate/up (input read in place) and down
    BandArgs g{};
    g.codes = L.gate_c;
    g.scales = L.gate_s;
    g.codes2 = L.up_c;
    g.scales2 = L.up_s;
    g.codes_stride = L.gc_bytes;
    g.scales_stride = L.gs_elems;
    g.nb = nbh;
    g.ntc = nbi;
    g.rows = L.I;
    g.wpt = nbi;
    g.tiles = tiles;
    g.ntiles = ntiles;
    g.perm = perm;
    g.k = L.k;
    g.act = L.act;
    g.hout = (ActBlock*)tact;
    auto grid = [&](int wpt) {
      const size_t wgs = w.max_tiles * (size_t)((wpt + BAND_WAVES - 1) / BAND_WAVES);
      return (unsigned)((wgs + 7) / 8 * 8);
    };
    // non-temporal weight loads up to two assignments per expert on average
    // (Qwen3-30B q4_0 layer, per layer: 72.9 against 75.2 us at 16 tokens;
    // cached from there: 121 against 125.7 at 64, 153.8 against 161.8 at 96)
    const bool nt = A <= 2 * (size_t)L.E;
    const int nr = band_rows(L, T);  // four only over rows of at most 256 blocks
#define HALE_BAND_NB(DT_, GU_, D_, NT_, args)                                             \
  do {                                                                                    \
    if (nr == 4)                                                                          \
      HALE_STEP(GU_ ? K_GROUPED_GATE_UP : K_GROUPED_DOWN,                                 \
                (launch(k_band<DT_, GU_, D_, NT_, 256, 4>, grid(args.wpt), 64 * BAND_WAVES, \
                        (uint32_t)band_lds(4, args.nb, D_), st, args)));                    \
    else if (args.nb <= 256)                                                              \
      HALE_STEP(GU_ ? K_GROUPED_GATE_UP : K_GROUPED_DOWN,                                 \
                (launch(k_band<DT_, GU_, D_, NT_, 256, 2>, grid(args.wpt), 64 * BAND_WAVES, \
                        (uint32_t)band_lds(2, args.nb, D_), st, args)));                    \
    else                                                                                  \
      HALE_STEP(GU_ ? K_GROUPED_GATE_UP : K_GROUPED_DOWN,                                 \
                (launch(k_band<DT_, GU_, D_, NT_, BAND_MAX_NB, 2>, grid(args.wpt),          \
                        64 * BAND_WAVES, (uint32_t)band_lds(2, args.nb, D_), st, args)));   \
  } while (0)
#define HALE_BAND(DT_, GU_, D_, args)        \
  do {                                       \
    if (nt)                                  \
      HALE_BAND_NB(DT_, GU_, D_, true, args); \
    else                                     \
      HALE_BAND_NB(DT_, GU_, D_, false, args); \
  } while (0)
    if (L.dtype == Q8_0)
      HALE_BAND(Q8_0, true, 8, g);
    else
      HALE_BAND(Q4_0, true, 8, g);
    BandArgs d{};
    d.codes = L.down_c;
    d.scales = L.down_s;
    d.codes_stride = L.dc_bytes;
    d.scales_stride = L.ds_elems;
    d.nb = nbi;
    d.ntc = nbh;
    d.rows = L.H;
    d.wpt = (nbh + 1) / 2;
    d.tiles = tiles;
    d.ntiles = ntiles;
    d.act = (const ActBlock*)tact;
    d.y = y;
    if (L.dtype == Q8_0)
      HALE_BAND(Q8_0, false, 8, d);
    else if (nbi >= 32)
      HALE_BAND(Q4_0, false, 16, d);
    else
      HALE_BAND(Q4_0, false, 8, d);
#undef HALE_BAND
#undef HALE_BAND_NB
    dim3 gc((unsigned)((L.H + COMBINE_COLS - 1) / COMBINE_COLS), (unsigned)T);
    HALE_STEP(K_COMBINE, launch(k_combine, gc, 256, 0, st, y, pos_of, L.route_w, L.k, L.H, out));
    return hipSuccess;
  }
  // 3. gather the activations into tiles, then the grouped gate/up with SiLU
  // and requantization
  const dim3 ggr((unsigned)w.max_tiles, (unsigned)((nbh + 7) / 8));
  if (L.dtype == Q4_0)
    HALE_STEP(K_GATHER, launch(k_gather_tiles<true>, ggr, 256, 0, st, (const ActBlock*)L.act, nbh,
                               tiles, ntiles, perm, L.k, tin));
  else
    HALE_STEP(K_GATHER, launch(k_gather_tiles<false>, ggr, 256, 0, st, (const ActBlock*)L.act, nbh,
                               tiles, ntiles, perm, L.k, tin));
  GroupedArgs g{};
  g.codes = L.gate_c;
  g.scales = L.gate_s;
  g.codes2 = L.up_c;
  g.scales2 = L.up_s;
  g.codes_stride = L.gc_bytes;
  g.scales_stride = L.gs_elems;
  g.nb = nbh;
  g.ncols = L.I;
  g.tiles = tiles;
  g.ntiles = ntiles;
  g.tin = tin;
  g.tout = tact;
  const unsigned gg = (unsigned)((w.max_tiles * ((L.I + TN - 1) / TN) + 7) / 8 * 8);
  if (L.dtype == Q8_0)
    HALE_STEP(K_GROUPED_GATE_UP, (launch(k_grouped<Q8_0, true>, gg, 256, 0, st, g)));
  else
    HALE_STEP(K_GROUPED_GATE_UP, (launch(k_grouped<Q4_0, true>, gg, 256, 0, st, g)));
  // 4. grouped down
  GroupedArgs d{};
  d.codes = L.down_c;
  d.scales = L.down_s;
  d.codes_stride = L.dc_bytes;
  d.scales_stride = L.ds_elems;
  d.nb = nbi;
  d.ncols = L.H;
  d.tiles = tiles;
  d.ntiles = ntiles;
  d.tin = tact;
  d.y = y;
  const unsigned gd = (unsigned)((w.max_tiles * ((L.H + TN - 1) / TN) + 7) / 8 * 8);
  if (L.dtype == Q8_0 && L.down_fold == DOWN_FOLD_FMA)
    HALE_STEP(K_GROUPED_DOWN, (launch(k_grouped<Q8_0, false, true>, gd, 256, 0, st, d)));
  else if (L.dtype == Q8_0)
    HALE_STEP(K_GROUPED_DOWN, (launch(k_grouped<Q8_0, false>, gd, 256, 0, st, d)));
  else if (L.down_fold == DOWN_FOLD_FMA)
    HALE_STEP(K_GROUPED_DOWN, (launch(k_grouped<Q4_0, false, true>, gd, 256, 0, st, d)));
  else
    HALE_STEP(K_GROUPED_DOWN, (launch(k_grouped<Q4_0, false>, gd, 256, 0, st, d)));
  // 5. route-order combine
  dim3 gc((unsigned)((L.H + COMBINE_COLS - 1) / COMBINE_COLS), (unsigned)T);
  HALE_STEP(K_COMBINE, launch(k_combine, gc, 256, 0, st, y, pos_of, L.route_w, L.k, L.H, out));
#undef HALE_STEP
  return hipSuccess;
}

}  // namespace hale
