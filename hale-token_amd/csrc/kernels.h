// kernels.h -- launch interface between the host runtime and the kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <tuple>

namespace hale {

// Timing bracket of the per-kernel profiler.  While `stop` is set, launch()
// hands the events to the runtime so that they take the kernels' own start
// and end times: `start` at the first kernel of the bracket, `stop` at the
// end of each kernel (the last one stands).  Per thread; the runtime opens
// and closes brackets around its launchers.
struct ProfEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  bool started = false;
};
ProfEvents& prof_events();

// kernel<<<grid, block, shmem, st>>>(args...), or the same launch with the
// open bracket's events.  Arguments are converted to the kernel's parameter
// types before their addresses are taken.
template <typename... P, typename... A>
hipError_t launch(void (*kernel)(P...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                  A... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  ProfEvents& pe = prof_events();
  if (!pe.stop) {
    kernel<<<grid, block, shmem, st>>>(args...);
    return hipGetLastError();
  }
  std::tuple<P...> typed{static_cast<P>(args)...};
  void* ptrs[sizeof...(P) ? sizeof...(P) : 1];
  std::apply([&](auto&... v) {
    int i = 0;
    ((ptrs[i++] = (void*)&v), ...);
  }, typed);
  hipError_t e = hipExtLaunchKernel((const void*)kernel, grid, block, ptrs, shmem, st,
                                    pe.started ? nullptr : pe.start, pe.stop, 0);
  pe.started = true;
  return e;
}

struct ActBlock;

enum Epilogue : int { EPI_PLAIN = 0, EPI_GATE_UP = 1 };

constexpr int DOWN_ROWS = 8;  // output rows per work-group of k_down_combine

// Arguments of the exact tile GEMV (kernels_decode.hip).  Expert e's planes
// start at codes + e * codes_stride / scales + e * scales_stride; the
// expert of slot s is route_idx[s] (expert 0 when route_idx is null).
struct GemvArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  const uint8_t* codes2;   // up-projection planes (EPI_GATE_UP)
  const uint16_t* scales2;
  size_t codes_stride;     // bytes
  size_t scales_stride;    // f16 elements
  int nb;                  // quantization blocks per row
  int rows;                // real rows (outputs beyond are not written)
  const ActBlock* act;     // [slot][act_stride] activation blocks
  int act_stride;          // 0: one activation shared by all slots
  const int* route_idx;    // [slots]
  float* out;              // [rows]
  ActBlock* hact;          // [slots][hact_stride] (EPI_GATE_UP)
  int hact_stride;
  int slots;
  // EPI_GATE_UP with routing in the prologue: when logits is set, the
  // slot's expert is selected from logits[E] (softmax, top-k, renormalise)
  // and published to route_out_idx / route_out_w (and counted in stats).
  const float* logits;
  int E;
  int normalize;
  int* route_out_idx;
  float* route_out_w;
  unsigned long long* stats;
  // set by launch_gemv (EPI_GATE_UP): the rows' 32-row tiles and the tiles
  // per work-group
  int tiles;
  int ipw;
  // EPI_GATE_UP of one token: the f32 activation (16-byte aligned, nb <=
  // GEMV_X_MAX_NB), quantized by the kernel itself in place of act
  const float* x;
  // EPI_GATE_UP with routing over several tokens (tokens > 1; 0 or 1: one):
  // grid row y is slot y % slots of token y / slots, whose activation is act
  // + token * act_tstride, logits logits + token * E, routes route_out_* +
  // token * slots and h blocks hact + y * hact_stride
  int tokens;
  int act_tstride;
};
constexpr int GEMV_X_MAX_NB = 128;

// Arguments of the down projection + combine (k_down_combine).
struct DownArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  size_t codes_stride;     // bytes per expert
  size_t scales_stride;    // f16 elements per expert
  int nb;                  // blocks per row (inter / 32)
  int rows;                // hidden
  const ActBlock* hact;    // [slots][hact_stride]
  int hact_stride;
  const int* route_idx;    // [slots]
  const float* route_w;    // [slots]
  int slots;
  float* out;              // [rows]
  // tokens > 1: token t's routes at route_idx / route_w + t * slots, its h
  // blocks at hact + t * slots * hact_stride, its output at out + t * rows
  int tokens;
  // WeightMatrix::matvec through the spread-term kernel (one matrix, no
  // routes or combine): x (f32, 16-byte aligned) quantized by the kernel,
  // or hact when null
  const float* x;
};

hipError_t launch_down_combine(int dtype, const DownArgs& a, hipStream_t st);

// WeightMatrix::matvec of one quantized matrix with whole fold chains per
// wave: out[r] for r < rows.  The activation is x (f32, quantized in the
// kernel; 16-byte aligned) or act (q8 blocks already made).  Returns
// hipErrorNotSupported for shapes it does not take (then the caller runs
// act quantization and launch_gemv).
struct MatvecArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  int nb;                // blocks per row
  int rows;
  const float* x;        // or null
  const ActBlock* act;   // used when x is null
  float* out;
  // launch_matvec_pair: a second matrix of the same shape and input
  // (Expert::forward's gate and up); out then receives silu(first row's
  // dot) * (second row's dot) per row, the f32 h of the SwiGLU
  const uint8_t* codes2;
  const uint16_t* scales2;
};
hipError_t launch_matvec(int dtype, const MatvecArgs& a, hipStream_t st);
// Whether launch_matvec takes x (f32, 16-byte aligned) for rows of nb
// blocks, quantizing it in the kernel; otherwise the caller quantizes x
// into act first.
bool matvec_takes_x(int nb, size_t rows);
// both matrices of a in one launch, x quantized in the kernel:
// out[r] = silu(dot(codes row r, x)) * dot(codes2 row r, x)
hipError_t launch_matvec_pair(int dtype, const MatvecArgs& a, hipStream_t st);
constexpr int MATVEC_XQ_MAX_NB = 128;  // blocks per row launch_matvec quantizes x for
constexpr int MATVEC_MAX_NB = 512;     // blocks per row it takes with act given

// Shapes the fast decode and grouped kernels take; a layer beyond any of
// them runs the general path below (any number of experts, top_k, hidden
// and intermediate sizes).
constexpr size_t FAST_MAX_E = 1024, FAST_MAX_H = 8192, FAST_MAX_K = 64, FAST_MAX_NB = 512;

// General-shape matvec: lane per row, every block of the row in order, any
// row length.  Grid row y (of ny) reads the q8 blocks act + (y / act_div) *
// nb, uses expert route[y] (planes at codes + e * codes_stride; expert 0
// without route) and writes out + y * out_stride.
struct RowsArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  size_t codes_stride, scales_stride;
  const int* route;
  int nb, rows;
  const ActBlock* act;
  int act_div;
  float* out;
  size_t out_stride;
};
hipError_t launch_matvec_rows(int dtype, const RowsArgs& a, int ny, hipStream_t st);
// h = silu(g) * u elementwise, quantized to q8 blocks (nblocks blocks of 32)
hipError_t launch_swiglu_quant(const float* g, const float* u, size_t nblocks, ActBlock* h,
                               hipStream_t st);
// MoeLayer::route for any E and k <= E from T tokens' logits: softmax,
// top-k, renormalisation; ebuf holds T * E floats of scratch
hipError_t launch_route_select_wide(const float* logits, int E, int k, int normalize, int T,
                                    float* ebuf, int* route_idx, float* route_w,
                                    unsigned long long* stats, hipStream_t st);
// out[t] = 0, then out[t] = out[t] + w[t][s] * y[t * k + s] for s in route
// order (kernels_prefill.hip's combine with the rows in (token, slot) order)
hipError_t launch_combine_rows(const float* y, const float* route_w, int k, int H, int T,
                               float* out, hipStream_t st);

hipError_t launch_repack(int dtype, const uint8_t* aos, size_t rows, size_t cols, uint8_t* codes,
                         uint16_t* scales, hipStream_t st);
hipError_t launch_unpack(int dtype, const uint8_t* codes, const uint16_t* scales, size_t rows,
                         size_t cols, uint8_t* aos, hipStream_t st);
hipError_t launch_encode(int dtype, const float* values, size_t nblocks, uint8_t* out,
                         hipStream_t st);
// decode_row over n values of reference-layout rows laid end to end (any
// dtype, any base alignment)
hipError_t launch_decode_ref(int dtype, const void* src, size_t n, float* out, hipStream_t st);
// rows row0 .. row0 + nrows - 1 of a tiled q8_0 / q4_0 matrix -> out[nrows][cols]
hipError_t launch_decode_tiles(int dtype, const uint8_t* codes, const uint16_t* scales,
                               size_t row0, size_t nrows, size_t cols, float* out,
                               hipStream_t st);
hipError_t launch_act_quant(const float* x, size_t nblocks, ActBlock* act, hipStream_t st);
hipError_t launch_route_logits(const float* router, const float* x, int H, int E, int T,
                               ActBlock* act, float* logits, hipStream_t st);
hipError_t launch_route_select(const float* logits, int E, int k, int normalize, int T,
                               int* route_idx, float* route_w, unsigned long long* stats,
                               hipStream_t st);
// launch_route_select (no stats) and launch_act_quant in one launch
hipError_t launch_route_select_quant(const float* logits, int E, int k, int normalize, int T,
                                    int* route_idx, float* route_w, const float* x,
                                    size_t nblocks, ActBlock* act, hipStream_t st);
hipError_t launch_gemv(int dtype, int epi, const GemvArgs& a, int groups, int slots,
                       hipStream_t st);
hipError_t launch_block_sums(int dtype, const uint8_t* codes, const ActBlock* act, size_t rows,
                             size_t cols, int32_t* isums, hipStream_t st);
hipError_t launch_fill(float* p, size_t n, float v, hipStream_t st);
hipError_t launch_copy(void* dst, const void* src, size_t n16, hipStream_t st);
// out[g] = XOR of the 32-bit words of work-group g's contiguous chunk of
// src[n16] (workgroups in 1..65535)
hipError_t launch_stream_read(const void* src, size_t n16, unsigned workgroups, unsigned* out,
                              hipStream_t st);
// out[rows] = W x for row-major f32 / f16 / bf16 W [rows][cols] (x 16-byte
// aligned), in the reference's 8-lane dot order.
hipError_t launch_gemv_float(int dtype, const void* w, const float* x, size_t rows, size_t cols,
                             float* out, hipStream_t st);
// out[r] = rms_norm(x[r] (+ delta[r], stored back into x), w) for each of
// `rows` rows of n values (n <= 8192)
hipError_t launch_rms_norm(float* x, const float* delta, const float* w, size_t rows, size_t n,
                           float eps, float* out, hipStream_t st);

// One token of grouped-query attention after the q/k/v projections: QK-norm
// and RoPE of q and k, k/v pushed to the cache at row seq - 1, scores,
// softmax and the context.  keys/values are [ld][nkv*hd] f32, scores
// [nh][ld], ctx [nh*hd].
struct AttnArgs {
  float* q;            // [nh*hd], normalised and rotated in place
  const float* k;      // [nkv*hd] projection output
  const float* v;      // [nkv*hd]
  int nh, nkv, hd;
  const float* q_norm;  // [hd] or null
  const float* k_norm;  // [hd] or null
  float eps;
  const float* cos;     // [hd/2]
  const float* sin;
  float* keys;
  float* values;
  int seq;              // positions after the push (position + 1)
  int ld;               // cache capacity (rows of keys/values, row stride of scores)
  float* scores;
  float* ctx;
};
hipError_t launch_attention_core(const AttnArgs& a, hipStream_t st);

// values[n] -> f16 / bf16 bits (half's from_f32)
hipError_t launch_encode_half(int dtype, const float* values, size_t n, void* out, hipStream_t st);
hipError_t launch_fill_normal(float* p, size_t n, uint64_t seed, float mean, float std,
                              hipStream_t st);

// Kernel kinds for per-kernel timing (hale_profile_*).
enum KernelKind : int {
  K_ROUTE = 0,
  K_GATE_UP,
  K_DOWN,
  K_ACT_QUANT,
  K_GEMV,
  K_ENCODE,
  K_REPACK,
  K_FILL,
  K_GROUP,
  K_GROUPED_GATE_UP,
  K_GROUPED_DOWN,
  K_COMBINE,
  K_COPY,
  K_NORM,
  K_ATTENTION,
  K_GATHER,
  K_DECODE,
  K_STREAM_READ,
  K_KINDS
};

// Lets code outside the runtime bracket its launches for the profiler.
struct LaunchHook {
  void (*begin)(void* self, int kind) = nullptr;
  void (*end)(void* self) = nullptr;
  void* self = nullptr;
  void on_begin(int kind) const {
    if (begin) begin(self, kind);
  }
  void on_end() const {
    if (end) end(self);
  }
};

}  // namespace hale
