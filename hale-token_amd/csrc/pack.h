// pack.h -- the Hale expert pack (src/expert/pack.rs), host side: header
// parsing, positioned reads, and the loader that streams a layer's records
// into a MoE layer's HBM planes.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/hale_moe.h"
#include "pack_header.h"

namespace hale {

// Records a failure on a context (hale_last_error) and returns `code`.
int ctx_fail(hale_ctx* c, int code, const char* fmt, ...);

// One load of a layer's experts from a pack: the loader thread and its
// result.  Shared by the pack (its current load) and the layer (its pending
// load); whichever needs the result first joins the thread.
struct PackLoad {
  std::thread th;
  int rc = HALE_OK;  // written by the thread before it ends
  std::string err;
  uint64_t bytes = 0;   // record bytes read, and the wall-clock seconds from
  double seconds = 0;   // the first read to the last repack on the device
  void join() {
    if (th.joinable()) th.join();
  }
};

}  // namespace hale

// One open pack.  The loader thread, its stream and its staging buffers
// belong to the pack, so one load runs per pack at a time.
struct hale_pack {
  hale_ctx* ctx = nullptr;  // bound by the first load into a layer
  int device = 0;
  int fd = -1;
  std::string path;
  hale::PackHeader h;
  hipStream_t stream = nullptr;  // uploads and repacks (default priority)
  // staging: two slots of `slot_bytes`, pinned host and device
  size_t slot_bytes = 0;
  void* pinned[2] = {nullptr, nullptr};
  void* dstage[2] = {nullptr, nullptr};
  hipEvent_t copied[2] = {nullptr, nullptr};  // slot's host->device copy done
  std::shared_ptr<hale::PackLoad> load;  // the running (or last) load
  std::vector<hale_moe*> layers;  // layers whose source this pack is (cleared on close)
};

namespace hale {

// Positioned read of `n` bytes at `off` (retries short reads); false with a
// message on failure or end of file.
bool pack_pread(const hale_pack* p, void* dst, size_t n, uint64_t off, std::string* err);


}  // namespace hale
