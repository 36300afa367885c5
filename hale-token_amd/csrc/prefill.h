// prefill.h -- expert-grouped multi-token path (kernels_prefill.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hale {

struct ActBlock;

// Device workspace of the grouped path (the runtime grows it on demand).
struct PrefillWorkspace {
  void* base = nullptr;
  size_t bytes = 0;
};

// What the grouped path needs to know about one MoE layer.
struct PrefillLayer {
  int dtype;
  int E, H, I, k, normalize;
  const float* router;  // [E][H] or null (logits given)
  const uint8_t *gate_c, *up_c, *down_c;
  const uint16_t *gate_s, *up_s, *down_s;
  size_t gc_bytes, gs_elems, dc_bytes, ds_elems;  // per-expert plane sizes
  ActBlock* act;         // [T][H/32]
  float* logits;         // [T][E]
  int* route_idx;        // [T][k]
  float* route_w;        // [T][k]
  unsigned long long* stats;  // [E]
  int down_fold;         // DOWN_FOLD_EXACT or DOWN_FOLD_FMA (grouped down projection)
  size_t band_max;       // calls of at most this many tokens take the row-chain kernels
};

// Folds of the grouped down projection: the reference's product then sum,
// or one fused multiply-add per term.
constexpr int DOWN_FOLD_EXACT = 0;
constexpr int DOWN_FOLD_FMA = 1;

// Smallest token count routed through the grouped path.
size_t prefill_min_tokens(size_t k);
// Bytes of workspace for T tokens.
size_t prefill_workspace_bytes(const PrefillLayer& L, size_t T);
struct LaunchHook;
// Enqueues the grouped forward of T tokens; ws holds at least
// prefill_workspace_bytes(L, T) bytes of device memory (256-byte aligned).
hipError_t prefill_enqueue(const PrefillLayer& L, void* ws, size_t T, const float* x,
                           const float* logits, float* out, hipStream_t st,
                           const LaunchHook& hook);

}  // namespace hale
