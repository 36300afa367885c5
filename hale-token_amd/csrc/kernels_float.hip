// kernels_float.hip -- matvec over float weights (f32, f16, bf16) on gfx950.
//
// The reference's float dot (src/tensor/quant.rs:146-233) keeps eight lane
// accumulators: acc[l] = acc[l] + w[8i+l] * x[8i+l] for i = 0, 1, ...
// (products rounded, then added; no fused multiply-add), then
//   ((acc0 + acc4) + (acc1 + acc5)) + ((acc2 + acc6) + (acc3 + acc7))
// (reduce, :36-40) plus the sum of the last cols % 8 products.  f32 rows
// add that tail as Iterator::sum (from -0.0, dot_f32 :186-194); f16 and
// bf16 rows go through dot_decoded (:166-184), whose tail starts at +0.0.
// Each of a row's 8 chains is one sequential sum, so one lane per chain
// folds it; the products are computed in parallel.
//
// Work-group: 8 rows, 256 threads.  Per chunk of FK columns every thread
// loads 16-byte pieces of the rows (coalesced along each row) and its x,
// converts f16/bf16 to f32, and parks the products in LDS; wave 0 then folds
// them, lane (row r, chain l) reading products 8i + l of row r in order.
// Two LDS buffers: the next chunk's loads are in flight during a fold.
// HBM-bound: every weight byte is read once.
#pragma clang fp contract(off)

#include "hale_device.h"
#include "kernels.h"

namespace hale {

constexpr int FR = 8;        // rows per work-group (FR * 8 fold threads, whole waves)
constexpr int FK = 512;      // columns per chunk
constexpr int FPAD = 8;      // row pitch FK + FPAD = 8 (mod 64) floats: the fold
                             // threads (row r, chain l) of a wave read banks 8r + l

template <int DT>
struct FloatFmt;
template <> struct FloatFmt<F32> { static constexpr int PER16 = 4; };   // values per 16 B
template <> struct FloatFmt<F16> { static constexpr int PER16 = 8; };
template <> struct FloatFmt<BF16> { static constexpr int PER16 = 8; };

template <int DT>
__device__ __forceinline__ void unpack16(const u32x4& v, float* o) {
  if constexpr (DT == F32) {
    o[0] = __uint_as_float(v.x);
    o[1] = __uint_as_float(v.y);
    o[2] = __uint_as_float(v.z);
    o[3] = __uint_as_float(v.w);
  } else {
    const unsigned u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if constexpr (DT == F16) {
        o[2 * i] = h2f((uint16_t)(u[i] & 0xffffu));
        o[2 * i + 1] = h2f((uint16_t)(u[i] >> 16));
      } else {  // bf16 is the upper half of an f32
        o[2 * i] = __uint_as_float(u[i] << 16);
        o[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    }
  }
}

// VEC: every row starts 16-byte aligned, so a piece is one 16-byte load;
// otherwise it is read value by value.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void k_gemv_float(const uint8_t* __restrict__ w,
                                                    const float* __restrict__ x, int rows,
                                                    int cols, float* __restrict__ out) {
  constexpr int PER = FloatFmt<DT>::PER16;
  constexpr int ESZ = DT == F32 ? 4 : 2;
  constexpr int UPR = FK / PER;          // 16-byte pieces per row of a chunk
  constexpr int LPT = FR * UPR / 256;    // pieces per thread per chunk
  constexpr int RPP = 256 / UPR;         // rows one pass of the 256 threads covers
  static_assert(LPT * 256 == FR * UPR && LPT * RPP == FR, "chunk tiling");
  static_assert(FR % 8 == 0 && FR * 8 <= 256, "fold threads fill whole waves");
  __shared__ __attribute__((aligned(16))) float prod[2][FR][FK + FPAD];

  const int tid = threadIdx.x;
  const int row0 = blockIdx.x * FR;
  const int done = cols / 8 * 8;         // columns covered by the lane accumulators
  const int nchunks = (done + FK - 1) / FK;
  const size_t rb = (size_t)cols * ESZ;  // row bytes

  // piece j of this thread: row r_j, columns c .. c + PER - 1 of the chunk
  const int cpiece = (tid % UPR) * PER;
  struct Regs {
    u32x4 w[LPT];
    float x[PER];
  };
  auto load = [&](Regs& R, int ch) {
    // c is a multiple of PER (4 or 8) and `done` one of 8, so a piece below
    // `done` ends at or before it; rows past the end are clamped (loaded,
    // never written)
    const int c = ch * FK + cpiece;
    const bool in = c < done;
#pragma unroll
    for (int j = 0; j < LPT; j++) {
      const int r = min(row0 + j * RPP + tid / UPR, rows - 1);
      const uint8_t* src = w + (size_t)r * rb + (size_t)c * ESZ;
      if (in) {
        if constexpr (VEC) {
          R.w[j] = __builtin_nontemporal_load((const u32x4*)src);
        } else if constexpr (DT == F32) {
          const unsigned* s4 = (const unsigned*)src;
          R.w[j] = u32x4{s4[0], s4[1], s4[2], s4[3]};
        } else {
          const uint16_t* s2 = (const uint16_t*)src;
          R.w[j] = u32x4{s2[0] | ((unsigned)s2[1] << 16), s2[2] | ((unsigned)s2[3] << 16),
                         s2[4] | ((unsigned)s2[5] << 16), s2[6] | ((unsigned)s2[7] << 16)};
        }
      }
    }
    if (in) {
#pragma unroll
      for (int q = 0; q < PER / 4; q++) {
        const f32x4 v = *(const f32x4*)(x + c + 4 * q);
        R.x[4 * q] = v.x;
        R.x[4 * q + 1] = v.y;
        R.x[4 * q + 2] = v.z;
        R.x[4 * q + 3] = v.w;
      }
    }
  };

  // fold thread (row fr, chain fl): the first FR * 8 threads
  constexpr int NF = FR * 8;
  const int fr = tid >> 3, fl = tid & 7;
  float acc = 0.0f;
  auto step = [&](Regs& R, int ch) {
    const int c0 = ch * FK;
    const int ncols = min(FK, done - c0);
    float(*P)[FK + FPAD] = prod[ch & 1];
    if (cpiece < ncols) {
#pragma unroll
      for (int j = 0; j < LPT; j++) {
        float wf[PER];
        unpack16<DT>(R.w[j], wf);
        float* dst = &P[j * RPP + tid / UPR][cpiece];
#pragma unroll
        for (int q = 0; q < PER; q++) dst[q] = wf[q] * R.x[q];  // the rounded product
      }
    }
    __syncthreads();
    if (ch + 1 < nchunks) load(R, ch + 1);
    if (tid < NF) acc = lds_sum_strided<8>(&P[fr][fl], ncols / 8, acc);
  };
  Regs R;
  if (nchunks > 0) load(R, 0);
  for (int ch = 0; ch < nchunks; ch++) step(R, ch);

  if (tid < NF) {
    // reduce (src/tensor/quant.rs:36-40) across the row's 8 chain lanes
    const float a4 = __shfl_down(acc, 4, 8);
    const float s = acc + a4;                    // lanes 0-3: acc_l + acc_{l+4}
    const float s1 = __shfl_down(s, 1, 8);
    const float t = s + s1;                      // lanes 0, 2: pair sums
    const float t2 = __shfl_down(t, 2, 8);
    const float red = t + t2;                    // lane 0: (s0 + s1) + (s2 + s3)
    const int row = row0 + fr;
    if (fl == 0 && row < rows) {
      // the last cols % 8 products, summed in order
      float tail = -0.0f;
      const uint8_t* wr = w + (size_t)row * rb;
      for (int i = done; i < cols; i++) {
        float wi;
        if constexpr (DT == F32) {
          wi = ((const float*)wr)[i];
        } else if constexpr (DT == F16) {
          wi = h2f(((const uint16_t*)wr)[i]);
        } else {
          wi = __uint_as_float((unsigned)((const uint16_t*)wr)[i] << 16);
        }
        tail = tail + wi * x[i];
      }
      if constexpr (DT != F32) tail = 0.0f + tail;  // dot_decoded's `let mut tail = 0.0`
      out[row] = red + tail;
    }
  }
}

// encode_row for the half formats (src/tensor/quant.rs:274-292): half's
// f16::from_f32 / bf16::from_f32, round to nearest even; a NaN keeps its
// sign and top payload bits and becomes quiet.
template <int DT>
__global__ __launch_bounds__(256) void k_encode_half(const float* __restrict__ v, size_t n,
                                                     uint16_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float f = v[i];
  const unsigned x = __float_as_uint(f);
  uint16_t h;
  if constexpr (DT == F16) {
    if ((x & 0x7fffffffu) > 0x7f800000u)
      h = (uint16_t)(((x >> 16) & 0x8000u) | 0x7e00u | ((x & 0x7fffffu) >> 13));
    else
      h = f2h(f);  // v_cvt_f16_f32: round to nearest even, subnormals kept
  } else {
    if ((x & 0x7fffffffu) > 0x7f800000u) {
      h = (uint16_t)((x >> 16) | 0x0040u);
    } else {
      unsigned q = x >> 16;
      const unsigned rem = x & 0xffffu;
      if (rem > 0x8000u || (rem == 0x8000u && (q & 1u))) q++;  // may carry into inf
      h = (uint16_t)q;
    }
  }
  out[i] = h;
}

hipError_t launch_encode_half(int dtype, const float* values, size_t n, void* out, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const unsigned grid = (unsigned)((n + 255) / 256);
  if (dtype == F16) return launch(k_encode_half<F16>, grid, 256, 0, st, values, n, (uint16_t*)out);
  if (dtype == BF16) return launch(k_encode_half<BF16>, grid, 256, 0, st, values, n, (uint16_t*)out);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv_float(int dtype, const void* w, const float* x, size_t rows, size_t cols,
                             float* out, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (rows > (size_t)INT32_MAX - FR || cols > (size_t)INT32_MAX - FK) return hipErrorInvalidValue;
  if ((uintptr_t)x % 16) return hipErrorInvalidValue;  // x is read in 16-byte pieces
  const unsigned grid = (unsigned)((rows + FR - 1) / FR);
  const uint8_t* wb = (const uint8_t*)w;
  const int esz = dtype == F32 ? 4 : 2;
  const bool vec = (cols * esz) % 16 == 0 && (uintptr_t)w % 16 == 0;
#define HALE_FLOAT_CASE(D)                                                                          \
  if (dtype == D)                                                                                 \
    return vec ? launch(k_gemv_float<D, true>, grid, 256, 0, st, wb, x, (int)rows, (int)cols, out) \
               : launch(k_gemv_float<D, false>, grid, 256, 0, st, wb, x, (int)rows, (int)cols, out);
  HALE_FLOAT_CASE(F32)
  HALE_FLOAT_CASE(F16)
  HALE_FLOAT_CASE(BF16)
#undef HALE_FLOAT_CASE
  return hipErrorInvalidValue;
}

}  // namespace hale
