// hale_device.h -- device-side helpers shared by the gfx950 kernels.
//
// Arithmetic follows Hale-Token's Rust CPU path bit for bit: every
// translation unit is compiled with -ffp-contract=off (no fused
// multiply-add), f32 division is correctly rounded, denormals are kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define HALE_EXPF_FN static __device__ __forceinline__
#define HALE_EXPF_TABLE static __constant__ const
#include "glibc_expf.h"

namespace hale {

constexpr int QK = 32;         // elements per quantization block
constexpr int TILE = 32;       // rows per tile of the HBM weight layout
constexpr int GROUP = 64;      // rows one wave covers (two tiles)
constexpr int WAVE = 64;

enum DType : int { F32 = 0, F16 = 1, BF16 = 2, Q8_0 = 3, Q4_0 = 4 };

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A weight load: non-temporal when each weight byte is read once (one
// token's routes), ordinary when other tokens of the same pass read it
// again from the caches.
template <bool NT>
__device__ __forceinline__ u32x4 load_weights(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  return *p;
}

// One q8 activation block as the kernels read it: the 32 codes and f32
// scale of Q8Activations (src/tensor/quant.rs:69-93) plus the code sum used
// by the q4 kernels (sum_j (n_j - 8) x_j = sum_j n_j x_j - 8 sum_j x_j).
struct alignas(16) ActBlock {
  int8_t q[QK];
  float scale;
  int32_t qsum;
  int32_t pad[2];
};
static_assert(sizeof(ActBlock) == 48, "ActBlock is 48 bytes");

// ---- buffer resources ------------------------------------------------------
//
// A raw buffer of `bytes` bytes at p (base and size wave-uniform).  Loads
// through it take a per-lane 32-bit offset and a wave-uniform offset, so a
// loop that walks the buffer advances only a scalar; reads past `bytes`
// return zero.  Word 3 0x00020000 is the raw (unswizzled, 32-bit data
// format) setting of the CDNA buffer descriptor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// ---- scalar conversions -------------------------------------------------

__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;  // v_cvt_f32_f16: exact, keeps subnormals
}

__device__ __forceinline__ uint16_t f2h(float f) {
  // The empty asm keeps f a rounded f32 value: without it the compiler may
  // fold a producing multiply into v_fma_mix* with a +0 addend, which rounds
  // the exact product straight to f16 and turns a -0 product into +0.
  asm volatile("" : "+v"(f));
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Rust `v as i8`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
  if (v != v) return 0;
  if (v >= 127.0f) return 127;
  if (v <= -128.0f) return -128;
  return (int)v;
}

// Rust `v as i32`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return 2147483647;
  if (v <= -2147483648.0f) return (int)0x80000000u;
  return (int)v;
}

// exp for a whole wave (all lanes active): the 2^(i/32) table entry comes
// from a register of lane i (ExpTable, loaded once per kernel) through a
// lane shuffle instead of a per-lane memory lookup.
struct ExpTable {
  uint64_t entry;  // hale_exp2_tab[lane % 32]
  __device__ __forceinline__ void load() {
    entry = hale_exp2_tab[__lane_id() & 31];
  }
};

__device__ __forceinline__ float wave_expf(float x, const ExpTable& tab) {
  float res;
  uint64_t ki = 0;
  double r = 0.0;
  const int fin = hale_expf_reduce(x, &res, &ki, &r);
  const uint64_t te = __shfl(tab.entry, (int)(ki & 31));  // every lane takes part
  return fin ? res : hale_expf_finish(ki, r, te);
}

// silu, src/ops/activation.rs:5-7: x / (1 + exp(-x)).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + hale_expf(-x)); }
__device__ __forceinline__ float wave_silu(float x, const ExpTable& tab) {
  return x / (1.0f + wave_expf(-x, tab));
}

// f32::total_cmp as a signed integer key.
__device__ __forceinline__ int total_key(float v) {
  int b = __float_as_int(v);
  return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

// total_cmp order as an unsigned key (larger key = later in total order),
// and back
__device__ __forceinline__ unsigned order_key(float v) { return (unsigned)total_key(v) ^ 0x80000000u; }
__device__ __forceinline__ float key_value(unsigned key) {
  const int bits = (int)(key ^ 0x80000000u);
  return __int_as_float(bits ^ (int)(((unsigned)(bits >> 31)) >> 1));
}

// ---- wave helpers ---------------------------------------------------------

// Reductions over a full wave (all 64 lanes active): DPP within 16-lane rows
// (xor 1, xor 2, half mirror, mirror), then v_permlane16_swap (lane ^ 16)
// and v_permlane32_swap (lane ^ 32), all on the VALU.  Every lane ends with
// the result, returned wave-uniform.
__device__ __forceinline__ unsigned xor16(unsigned x) {
  auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);  // {row 2j, row 2j+1}
  return (threadIdx.x & 16) ? p[0] : p[1];
}
template <typename Op>
__device__ __forceinline__ unsigned wave_reduce_u32(unsigned x, Op op) {
  x = op(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false));   // xor 1
  x = op(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false));   // xor 2
  x = op(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xF, 0xF, false));  // half mirror
  x = op(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xF, 0xF, false));  // mirror
  auto p16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = op(p16[0], p16[1]);
  auto p32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  x = op(p32[0], p32[1]);
  return (unsigned)__builtin_amdgcn_readfirstlane((int)x);
}

struct OpMaxU { __device__ unsigned operator()(unsigned a, unsigned b) const { return a > b ? a : b; } };
struct OpMinU { __device__ unsigned operator()(unsigned a, unsigned b) const { return a < b ? a : b; } };
struct OpOrU { __device__ unsigned operator()(unsigned a, unsigned b) const { return a | b; } };
struct OpAndU { __device__ unsigned operator()(unsigned a, unsigned b) const { return a & b; } };
struct OpMaxF {
  __device__ unsigned operator()(unsigned a, unsigned b) const {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }
};

__device__ __forceinline__ unsigned wave_max_u32(unsigned x) { return wave_reduce_u32(x, OpMaxU()); }

__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(wave_reduce_u32(__float_as_uint(v), OpMaxF()));
}

__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Reductions within each 32-lane half of a wave (the half's lanes active;
// the other half may be inactive): DPP inside 16-lane rows, then
// v_permlane16_swap between the two rows of the half.  Every lane of a half
// gets its half's result.
#define HALE_DPP_F32(x, ctrl) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false))
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, HALE_DPP_F32(v, 0xB1));
  v = fmaxf(v, HALE_DPP_F32(v, 0x4E));
  v = fmaxf(v, HALE_DPP_F32(v, 0x141));
  v = fmaxf(v, HALE_DPP_F32(v, 0x140));
  v = fmaxf(v, __uint_as_float(xor16(__float_as_uint(v))));
  return v;
}

__device__ __forceinline__ int half_wave_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  v += (int)xor16((unsigned)v);
  return v;
}

// acc + p[0] + p[1] + ... + p[n-1], strictly left to right, from LDS with
// p 16-byte aligned: 16 values per batch in two alternating register
// buffers, so the reads of batch c+1 are in flight while batch c is added,
// then the n % 16 tail.  With a wave-uniform n the loop stays under scalar
// control even when p differs between lanes.
__device__ __forceinline__ float lds_sum_in_order_a16(const float* p, int n, float acc) {
  const f32x4* p4 = (const f32x4*)p;
  const int nb = n / 16;
  f32x4 A[4], B[4];
  auto ld = [&](f32x4* d, int c) {
#pragma unroll
    for (int q = 0; q < 4; q++) d[q] = p4[4 * c + q];
  };
  auto add = [&](const f32x4* d) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      acc = acc + d[q].x;
      acc = acc + d[q].y;
      acc = acc + d[q].z;
      acc = acc + d[q].w;
    }
  };
  if (nb > 0) ld(A, 0);
  int c = 0;
  for (; c + 1 < nb; c += 2) {
    ld(B, c + 1);
    add(A);
    if (c + 2 < nb) ld(A, c + 2);
    add(B);
  }
  if (c < nb) add(A);
  for (int i = 16 * nb; i < n; i++) acc = acc + p[i];
  return acc;
}

// The same for any p: the values before the first 16-byte boundary one by
// one, then the aligned sum.  (A p that differs between lanes makes the
// head count, and with it the loop, divergent: use the aligned form there.)
__device__ __forceinline__ float lds_sum_in_order(const float* p, int n, float acc) {
  int head = (int)((16 - ((uintptr_t)p & 15)) & 15) / 4;
  if (head > n) head = n;
  for (int i = 0; i < head; i++) acc = acc + p[i];
  return lds_sum_in_order_a16(p + head, n - head, acc);
}

// acc + p[0] + p[S] + ... + p[(n-1)·S], strictly left to right, from LDS:
// batches of 8 in two alternating register buffers, so the reads of batch
// c+1 are in flight while batch c is added.
template <int S>
__device__ __forceinline__ float lds_sum_strided(const float* p, int n, float acc) {
  const int nb = n / 8;
  float A[8], B[8];
  auto ld = [&](float* d, int c) {
#pragma unroll
    for (int q = 0; q < 8; q++) d[q] = p[(8 * c + q) * S];
  };
  auto add = [&](const float* d) {
#pragma unroll
    for (int q = 0; q < 8; q++) acc = acc + d[q];
  };
  if (nb > 0) ld(A, 0);
  int c = 0;
  for (; c + 1 < nb; c += 2) {
    ld(B, c + 1);
    add(A);
    if (c + 2 < nb) ld(A, c + 2);
    add(B);
  }
  if (c < nb) add(A);
  for (int i = 8 * nb; i < n; i++) acc = acc + p[i * S];
  return acc;
}

// Quantizes one 32-element block held one value per lane of a 32-lane
// group (Q8Activations::quantize, src/tensor/quant.rs:85-91).  The max is
// order independent; the scale stays f32.  Returns the code of this lane.
__device__ __forceinline__ int quant_block_lane(float v, float* scale_out, int* qsum_out) {
  float amax = half_wave_max(fabsf(v));
  float scale = amax / 127.0f;
  float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  int q = sat_i8(roundf(v * inv));
  *scale_out = scale;
  *qsum_out = half_wave_sum(q);
  return q;
}

// ---- weight layout ---------------------------------------------------------
//
// A quantized matrix [rows][cols] lives in HBM as two planes, rows padded to
// a multiple of 64 (zero rows):
//   codes : [rows/32][nb][CH][32 rows][16 B]   CH = 2 (q8_0) or 1 (q4_0)
//   scales: [rows/32][nb][32 rows] f16
// so the 16-byte chunks of one block for 32 consecutive rows are contiguous
// (512 B).  The q4_0 chunk keeps the reference's nibble order: byte j holds
// element j (low) and element j+16 (high).

template <int DT> struct Layout;
template <> struct Layout<Q8_0> { static constexpr int CH = 2; };
template <> struct Layout<Q4_0> { static constexpr int CH = 1; };

__host__ __device__ inline size_t padded_rows(size_t rows) { return (rows + 63) / 64 * 64; }

__host__ __device__ inline size_t code_plane_bytes(int dtype, size_t rows, size_t cols) {
  return padded_rows(rows) * (cols / QK) * (dtype == Q8_0 ? 32 : 16);
}
__host__ __device__ inline size_t scale_plane_bytes(size_t rows, size_t cols) {
  return padded_rows(rows) * (cols / QK) * 2;
}

}  // namespace hale
