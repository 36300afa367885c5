// kernels_prefill.hip -- expert-grouped multi-token MoE layer (placeholder:
// the grouped path is not enabled yet, every token count runs the decode
// kernels token by token).
#pragma clang fp contract(off)

#include "hale_device.h"
#include "kernels.h"
#include "prefill.h"

namespace hale {

size_t prefill_min_tokens(size_t) { return (size_t)-1; }

size_t prefill_workspace_bytes(const PrefillLayer&, size_t) { return 0; }

hipError_t prefill_enqueue(const PrefillLayer&, PrefillWorkspace&, size_t, const float*,
                           const float*, float*, hipStream_t, const LaunchHook&) {
  return hipErrorNotSupported;
}

void prefill_free(PrefillWorkspace& ws) {
  if (ws.base) (void)hipFree(ws.base);
  ws.base = nullptr;
  ws.bytes = 0;
}

}  // namespace hale
