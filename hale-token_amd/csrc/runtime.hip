// runtime.hip -- host runtime behind include/hale_moe.h.
//
// Owns device memory (weights repacked into the tile planes, per-layer
// scratch), the context's stream and the error strings, and sequences the
// kernels of kernels_decode.hip / kernels_prefill.hip.  Reference items are
// cited per entry point in the public header.
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/hale_moe.h"
#include "hale_device.h"
#include "kernels.h"
#include "pack.h"
#include "prefill.h"

using namespace hale;

// ---------------------------------------------------------------------------
// handles
// ---------------------------------------------------------------------------

struct ProfRecord {
  int kind;
  hipEvent_t start, stop;
};

struct hale_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::recursive_mutex mu;
  std::string err;
  // scratch of the synchronous single-matrix / single-expert entry points
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // wall timer
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // per-kernel profiler
  bool prof_on = false;
  std::vector<hipEvent_t> ev_pool;
  std::vector<ProfRecord> recs;
  int open_kind = -1;
  bool prof_saved = false;  // prof_on while a capture runs (profiling is off then)
  double prof_ms[K_KINDS] = {};
  uint64_t prof_n[K_KINDS] = {};
  // Graphs keep the device addresses they were captured with.  While any
  // graph of this context exists, scratch that a call outgrows is retired
  // here instead of freed, so that replaying an older graph never touches
  // freed memory; the last hale_graph_destroy frees it.
  int live_graphs = 0;
  std::vector<void*> retired;
  // this device's copy of the fixed scratch array (forward without allocation)
  void* fixed_scratch = nullptr;
  // pinned host staging of the synchronous host-slice entry points: inputs
  // are copied in and outputs out of it by the CPU, the GPU copies from and
  // to it (every such call ends with a stream synchronize, so the next one
  // may reuse it)
  void* pinned = nullptr;
  size_t pinned_bytes = 0;
};

struct hale_graph {
  hale_ctx* ctx = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

struct hale_matrix {
  hale_ctx* ctx = nullptr;
  int dtype = 0;
  size_t rows = 0, cols = 0;
  uint8_t* codes = nullptr;    // quantized: tile planes
  uint16_t* scales = nullptr;
  uint8_t* raw = nullptr;      // f32 / f16 / bf16: the row-major bytes as given
  bool view = false;           // a view of a MoE layer's expert: the layer owns it
};

struct hale_moe {
  hale_ctx* ctx = nullptr;
  uint32_t layer = 0;
  size_t E = 0, H = 0, I = 0, k = 0;
  int dtype = 0;
  int normalize = 0;
  // a shape beyond the fast kernels (FAST_MAX_*): every forward and route
  // runs the general path (moe_wide_enqueue)
  bool wide = false;
  float* router = nullptr;  // [E][H] f32, or null
  // resident experts, [E][plane]
  uint8_t *gate_c = nullptr, *up_c = nullptr, *down_c = nullptr;
  uint16_t *gate_s = nullptr, *up_s = nullptr, *down_s = nullptr;
  size_t gc_bytes = 0, gs_elems = 0, dc_bytes = 0, ds_elems = 0;
  std::vector<char> present;
  unsigned long long* stats = nullptr;  // [E] routing counts
  // per-token scratch (TokScratch, carved from one buffer) for cap_tok tokens,
  // laid out for grouped_min == cap_gmin
  void* tok_base = nullptr;
  size_t cap_tok = 0, cap_gmin = 0;
  // forwards of at least grouped_min tokens take the expert-grouped path,
  // fewer the decode path (one pass over all of them)
  size_t grouped_min = 0;
  // grouped forwards of at most band_max tokens take the row-chain kernels
  size_t band_max = 0;
  // grouped prefill workspace
  PrefillWorkspace pw;
  // load from an expert pack: pending until the layer's next use waits for
  // it (joins the loader thread, then orders the context's stream after
  // `loaded`, recorded on the pack's stream after the last upload)
  std::shared_ptr<hale::PackLoad> load;
  hipEvent_t loaded = nullptr;
  // the provider surface: the pack that fetch misses load from, CacheStats
  // counters, selections recorded by fetch, and per-expert matrix views
  int down_fold = 0;  // grouped down projection: HALE_FOLD_EXACT or HALE_FOLD_FMA
  hale_pack* source = nullptr;
  uint64_t fetch_hits = 0, misses = 0, bytes_loaded = 0;
  double load_seconds = 0;
  std::vector<uint64_t> fetch_counts;  // [E]
  std::vector<hale_matrix*> views;     // [E][gate, up, down], made by the first fetch
};

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------

static thread_local std::string g_create_err;

static int fail(hale_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c)
    c->err = buf;
  else
    g_create_err = buf;
  return code;
}

#define HIPCHK(ctx, call)                                                                  \
  do {                                                                                     \
    hipError_t e_ = (call);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return fail((ctx), HALE_EHIP, "%s failed: %s", #call, hipGetErrorString(e_));        \
  } while (0)

int hale::ctx_fail(hale_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (!c) return fail(nullptr, code, "%s", buf);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  return fail(c, code, "%s", buf);
}

static bool quantized(int dtype) { return dtype == HALE_Q8_0 || dtype == HALE_Q4_0; }
static int moe_wait_load(hale_moe* m);

// ---------------------------------------------------------------------------
// fixed scratch of the forward that allocates nothing
// ---------------------------------------------------------------------------
//
// hale_moe_forward_device_noalloc takes its per-token scratch and grouped
// workspace from this array instead of allocating.  Every device the library
// runs on holds its own copy until the process ends.  In host code the name
// `scratch` only stands for the array; the device address of a device's
// copy comes from hipGetSymbolAddress, looked up once per device when the
// first context on it is created, and only that address is ever handed to
// kernels or copies.

static __device__ __align__(256) unsigned char scratch[HALE_NOALLOC_SCRATCH_BYTES];

static std::mutex g_fixed_mu;
static std::vector<void*> g_fixed_ptr;  // device index -> address of its copy

// The device address of `scratch` on `device`, which must be current.
static hipError_t fixed_scratch_address(int device, void** out) {
  std::lock_guard<std::mutex> g(g_fixed_mu);
  if ((size_t)device >= g_fixed_ptr.size()) g_fixed_ptr.resize((size_t)device + 1, nullptr);
  if (!g_fixed_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_fixed_ptr[device] = p;
  }
  *out = g_fixed_ptr[device];
  return hipSuccess;
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

extern "C" int hale_ctx_create(int device, hale_ctx** out) {
  if (!out) return fail(nullptr, HALE_EINVAL, "hale_ctx_create: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(nullptr, HALE_EHIP, "no HIP device available (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(nullptr, HALE_EINVAL, "device %d of %d", device, n);
  hale_ctx* c = new (std::nothrow) hale_ctx;
  if (!c) return fail(nullptr, HALE_ENOMEM, "out of host memory");
  c->device = device;
  if ((e = hipSetDevice(device)) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess) {
    delete c;
    return fail(nullptr, HALE_EHIP, "stream creation failed: %s", hipGetErrorString(e));
  }
  if ((e = fixed_scratch_address(device, &c->fixed_scratch)) != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return fail(nullptr, HALE_EHIP, "fixed scratch lookup failed: %s", hipGetErrorString(e));
  }
  *out = c;
  return HALE_OK;
}

extern "C" void hale_ctx_destroy(hale_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  if (c->scratch) (void)hipFree(c->scratch);
  if (c->pinned) (void)hipHostFree(c->pinned);
  for (void* p : c->retired) (void)hipFree(p);
  for (auto& r : c->recs) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
  if (c->t0) (void)hipEventDestroy(c->t0);
  if (c->t1) (void)hipEventDestroy(c->t1);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

extern "C" const char* hale_last_error(const hale_ctx* c) {
  return c ? c->err.c_str() : g_create_err.c_str();
}

extern "C" void* hale_ctx_stream(hale_ctx* c) { return c ? (void*)c->stream : nullptr; }

extern "C" int hale_ctx_synchronize(hale_ctx* c) {
  if (!c) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// Device memory a call has outgrown: freed at once, or kept until the last
// graph of the context is destroyed when a graph may still use it.
static void scratch_release(hale_ctx* c, void* p) {
  if (!p) return;
  if (c->live_graphs > 0)
    c->retired.push_back(p);
  else
    (void)hipFree(p);
}

// Scratch may only grow outside graph capture: growing synchronizes the
// stream and allocates, which a capture cannot record.
static int growth_allowed(hale_ctx* c, const char* what, size_t bytes) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  HIPCHK(c, hipStreamIsCapturing(c->stream, &st));
  if (st != hipStreamCaptureStatusNone)
    return fail(c, HALE_EINVAL,
                "%s must grow to %zu bytes while the stream is being captured; make the same "
                "call once before the capture",
                what, bytes);
  return HALE_OK;
}

// Grows the context scratch to at least `bytes` (synchronous).
static int ctx_scratch(hale_ctx* c, size_t bytes, void** p) {
  if (c->scratch_bytes < bytes) {
    int rc = growth_allowed(c, "context scratch", bytes);
    if (rc) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    scratch_release(c, c->scratch);
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    if (hipMalloc(&c->scratch, bytes) != hipSuccess)
      return fail(c, HALE_ENOMEM, "device scratch of %zu bytes", bytes);
    c->scratch_bytes = bytes;
  }
  *p = c->scratch;
  return HALE_OK;
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// The context's pinned staging of at least `bytes` (grown; not while the
// stream is captured, where host-slice calls cannot run anyway).
static int ctx_pinned(hale_ctx* c, size_t bytes, char** out) {
  if (c->pinned_bytes < bytes) {
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (c->pinned) (void)hipHostFree(c->pinned);
    c->pinned = nullptr;
    c->pinned_bytes = 0;
    const size_t want = std::max<size_t>(bytes, 1 << 20);
    if (hipHostMalloc(&c->pinned, want, hipHostMallocDefault) != hipSuccess) {
      c->pinned = nullptr;
      return fail(c, HALE_ENOMEM, "pinned staging of %zu bytes", want);
    }
    c->pinned_bytes = want;
  }
  *out = (char*)c->pinned;
  return HALE_OK;
}

// Host-slice staging of one synchronous call: inputs are copied into the
// pinned buffer and sent to the device; outputs come back into it and are
// copied out after the call's synchronize (finish).
struct HostStage {
  hale_ctx* c;
  char* base = nullptr;
  size_t used = 0;
  struct Out {
    void* host;
    size_t off, n;
  };
  Out outs[4];
  int nouts = 0;
  explicit HostStage(hale_ctx* ctx) : c(ctx) {}
  // room for every input and output of the call (before any in/out)
  int reserve(size_t bytes) { return ctx_pinned(c, bytes, &base); }
  int in(void* dev, const void* host, size_t n) {
    std::memcpy(base + used, host, n);
    const hipError_t e = hipMemcpyAsync(dev, base + used, n, hipMemcpyHostToDevice, c->stream);
    used += align_up(n, 256);
    return e == hipSuccess ? HALE_OK : fail(c, HALE_EHIP, "copy to device: %s", hipGetErrorString(e));
  }
  int out(void* host, const void* dev, size_t n) {
    const hipError_t e = hipMemcpyAsync(base + used, dev, n, hipMemcpyDeviceToHost, c->stream);
    if (e != hipSuccess) return fail(c, HALE_EHIP, "copy to host: %s", hipGetErrorString(e));
    outs[nouts++] = {host, used, n};
    used += align_up(n, 256);
    return HALE_OK;
  }
  int finish() {
    const hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return fail(c, HALE_EHIP, "synchronize: %s", hipGetErrorString(e));
    for (int i = 0; i < nouts; i++) std::memcpy(outs[i].host, base + outs[i].off, outs[i].n);
    return HALE_OK;
  }
};

// ---------------------------------------------------------------------------
// per-kernel profiler (events on the context's stream around each launch)
// ---------------------------------------------------------------------------

static hipEvent_t prof_event(hale_ctx* c) {
  if (!c->ev_pool.empty()) {
    hipEvent_t e = c->ev_pool.back();
    c->ev_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

ProfEvents& hale::prof_events() {
  static thread_local ProfEvents pe;
  return pe;
}

// Opens a bracket: the kernels launched until prof_end record its events.
static void prof_begin(hale_ctx* c, int kind) {
  if (!c->prof_on) return;
  hipEvent_t a = prof_event(c), b = prof_event(c);
  if (!a || !b) {
    if (a) c->ev_pool.push_back(a);
    if (b) c->ev_pool.push_back(b);
    return;
  }
  ProfEvents& pe = prof_events();
  pe.start = a;
  pe.stop = b;
  pe.started = false;
  c->open_kind = kind;
}

static void prof_end(hale_ctx* c) {
  ProfEvents& pe = prof_events();
  if (!pe.stop) return;
  if (pe.started) {
    c->recs.push_back({c->open_kind, pe.start, pe.stop});
  } else {  // no kernel ran
    c->ev_pool.push_back(pe.start);
    c->ev_pool.push_back(pe.stop);
  }
  pe = ProfEvents{};
}

static void hook_begin(void* self, int kind) { prof_begin((hale_ctx*)self, kind); }
static void hook_end(void* self) { prof_end((hale_ctx*)self); }

static LaunchHook ctx_hook(hale_ctx* c) {
  LaunchHook h;
  h.begin = hook_begin;
  h.end = hook_end;
  h.self = c;
  return h;
}

// Launches `call` (returning hipError_t) bracketed for the profiler.
#define LAUNCH(ctx, kind, call)   \
  do {                            \
    prof_begin((ctx), (kind));    \
    hipError_t le_ = (call);      \
    prof_end((ctx));              \
    HIPCHK((ctx), le_);           \
  } while (0)

// ---------------------------------------------------------------------------
// geometry
// ---------------------------------------------------------------------------

extern "C" size_t hale_block_bytes(int dtype) {
  switch (dtype) {
    case HALE_F32: return 4;
    case HALE_F16:
    case HALE_BF16: return 2;
    case HALE_Q8_0: return 34;
    case HALE_Q4_0: return 18;
    default: return 0;
  }
}

extern "C" long long hale_row_bytes(int dtype, size_t cols) {
  size_t bb = hale_block_bytes(dtype);
  if (bb == 0) return -1;
  size_t bl = quantized(dtype) ? HALE_QK : 1;
  if (cols % bl) return -1;
  return (long long)(cols / bl * bb);
}

// ---------------------------------------------------------------------------
// matrices
// ---------------------------------------------------------------------------

static int matrix_create(hale_ctx* c, int dtype, size_t rows, size_t cols, const void* bytes,
                         size_t nbytes, bool on_device, hale_matrix** out) {
  if (!c || !out) return fail(c, HALE_EINVAL, "matrix upload: NULL argument");
  *out = nullptr;
  if (dtype < HALE_F32 || dtype > HALE_Q4_0)
    return fail(c, HALE_EINVAL, "matrix upload: unknown dtype %d", dtype);
  long long rb = hale_row_bytes(dtype, cols);
  if (rb < 0) return fail(c, HALE_EINVAL, "dtype %d needs row length divisible by 32, got %zu", dtype, cols);
  if (nbytes != rows * (size_t)rb)
    return fail(c, HALE_EINVAL, "matrix %zux%zu needs %zu bytes, got %zu", rows, cols,
                rows * (size_t)rb, nbytes);
  if (rows == 0 || cols == 0) return fail(c, HALE_EINVAL, "empty matrix %zux%zu", rows, cols);
  if (!bytes) return fail(c, HALE_EINVAL, "matrix upload: bytes is NULL");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  hale_matrix* m = new (std::nothrow) hale_matrix;
  if (!m) return fail(c, HALE_ENOMEM, "out of host memory");
  m->ctx = c;
  m->dtype = dtype;
  m->rows = rows;
  m->cols = cols;
  hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  if (!quantized(dtype)) {
    if (hipMalloc(&m->raw, nbytes) != hipSuccess) {
      delete m;
      return fail(c, HALE_ENOMEM, "device allocation of %zu bytes", nbytes);
    }
    hipError_t e = hipMemcpyAsync(m->raw, bytes, nbytes, kind, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
      (void)hipFree(m->raw);
      delete m;
      return fail(c, HALE_EHIP, "upload: %s", hipGetErrorString(e));
    }
    *out = m;
    return HALE_OK;
  }
  size_t cb = code_plane_bytes(dtype, rows, cols), sb = scale_plane_bytes(rows, cols);
  uint8_t* staging = nullptr;
  hipError_t e = hipMalloc(&m->codes, cb);
  if (e == hipSuccess) e = hipMalloc(&m->scales, sb);
  if (e == hipSuccess && !on_device) e = hipMalloc(&staging, nbytes);
  if (e != hipSuccess) {
    (void)hipFree(m->codes);
    (void)hipFree(m->scales);
    (void)hipFree(staging);
    delete m;
    return fail(c, HALE_ENOMEM, "device allocation for a %zux%zu matrix", rows, cols);
  }
  const uint8_t* src = (const uint8_t*)bytes;
  if (!on_device) {
    e = hipMemcpyAsync(staging, bytes, nbytes, hipMemcpyHostToDevice, c->stream);
    src = staging;
  }
  if (e == hipSuccess) e = launch_repack(dtype, src, rows, cols, m->codes, m->scales, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  (void)hipFree(staging);
  if (e != hipSuccess) {
    (void)hipFree(m->codes);
    (void)hipFree(m->scales);
    delete m;
    return fail(c, HALE_EHIP, "upload/repack: %s", hipGetErrorString(e));
  }
  *out = m;
  return HALE_OK;
}

extern "C" int hale_matrix_upload(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                  const void* bytes, size_t nbytes, hale_matrix** out) {
  return matrix_create(c, dtype, rows, cols, bytes, nbytes, false, out);
}

extern "C" int hale_matrix_upload_device(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                         const void* d_bytes, size_t nbytes, hale_matrix** out) {
  return matrix_create(c, dtype, rows, cols, d_bytes, nbytes, true, out);
}

extern "C" void hale_matrix_destroy(hale_matrix* m) {
  if (!m || m->view) return;
  std::lock_guard<std::recursive_mutex> g(m->ctx->mu);
  (void)hipSetDevice(m->ctx->device);
  (void)hipStreamSynchronize(m->ctx->stream);
  (void)hipFree(m->codes);
  (void)hipFree(m->scales);
  (void)hipFree(m->raw);
  delete m;
}

extern "C" int hale_matrix_shape(const hale_matrix* m, int* dtype, size_t* rows, size_t* cols) {
  if (!m) return HALE_EINVAL;
  if (dtype) *dtype = m->dtype;
  if (rows) *rows = m->rows;
  if (cols) *cols = m->cols;
  return HALE_OK;
}

extern "C" int hale_matrix_download(hale_ctx* c, const hale_matrix* m, void* bytes, size_t nbytes) {
  if (!c || !m || !bytes) return fail(c, HALE_EINVAL, "matrix download: NULL argument");
  size_t need = m->rows * (size_t)hale_row_bytes(m->dtype, m->cols);
  if (nbytes != need) return fail(c, HALE_EINVAL, "matrix download needs %zu bytes, got %zu", need, nbytes);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  if (!quantized(m->dtype)) {
    HIPCHK(c, hipMemcpyAsync(bytes, m->raw, nbytes, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return HALE_OK;
  }
  void* tmp;
  int rc = ctx_scratch(c, nbytes, &tmp);
  if (rc) return rc;
  LAUNCH(c, K_REPACK, launch_unpack(m->dtype, m->codes, m->scales, m->rows, m->cols, (uint8_t*)tmp, c->stream));
  HIPCHK(c, hipMemcpyAsync(bytes, tmp, nbytes, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// quantization
// ---------------------------------------------------------------------------

extern "C" int hale_quantize_q8_act(hale_ctx* c, const float* x, size_t n, float* scales,
                                    int8_t* quants) {
  if (!c || !x || !scales || !quants) return fail(c, HALE_EINVAL, "quantize: NULL argument");
  if (n % HALE_QK) return fail(c, HALE_EINVAL, "activation length must be a multiple of 32, got %zu", n);
  if (n == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  size_t nb = n / HALE_QK;
  size_t xoff = 0, aoff = align_up(n * 4, 256);
  void* s;
  int rc = ctx_scratch(c, aoff + nb * sizeof(ActBlock), &s);
  if (rc) return rc;
  float* dx = (float*)((char*)s + xoff);
  ActBlock* act = (ActBlock*)((char*)s + aoff);
  HIPCHK(c, hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->stream));
  LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, nb, act, c->stream));
  std::vector<ActBlock> h(nb);
  HIPCHK(c, hipMemcpyAsync(h.data(), act, nb * sizeof(ActBlock), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  for (size_t b = 0; b < nb; b++) {
    scales[b] = h[b].scale;
    memcpy(quants + b * HALE_QK, h[b].q, HALE_QK);
  }
  return HALE_OK;
}

static int encode_check(hale_ctx* c, int dtype, size_t rows, size_t cols) {
  if (dtype < HALE_F32 || dtype > HALE_Q4_0) return fail(c, HALE_EINVAL, "encode: unknown dtype %d", dtype);
  if (quantized(dtype) && cols % HALE_QK)
    return fail(c, HALE_EINVAL, "encode: row length %zu not a multiple of 32", cols);
  (void)rows;
  return HALE_OK;
}

// Enqueues encode_row over rows x cols device values into d_bytes.
static int encode_enqueue(hale_ctx* c, int dtype, size_t rows, size_t cols, const float* dv,
                          void* db) {
  if (dtype == HALE_F32) {
    if (rows * cols) HIPCHK(c, hipMemcpyAsync(db, dv, rows * cols * 4, hipMemcpyDeviceToDevice, c->stream));
  } else if (!quantized(dtype)) {
    LAUNCH(c, K_ENCODE, launch_encode_half(dtype, dv, rows * cols, db, c->stream));
  } else {
    LAUNCH(c, K_ENCODE, launch_encode(dtype, dv, rows * (cols / HALE_QK), (uint8_t*)db, c->stream));
  }
  return HALE_OK;
}

extern "C" int hale_encode_rows_device(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                       const float* d_values, void* d_bytes) {
  if (!c || !d_values || !d_bytes) return fail(c, HALE_EINVAL, "encode: NULL argument");
  int rc = encode_check(c, dtype, rows, cols);
  if (rc) return rc;
  if (quantized(dtype) && (uintptr_t)d_values % 16)  // the block encoder loads float4
    return fail(c, HALE_EINVAL, "encode: values must be 16-byte aligned for q8_0 / q4_0");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  return encode_enqueue(c, dtype, rows, cols, d_values, d_bytes);
}

extern "C" int hale_encode_rows(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                const float* values, void* bytes) {
  if (!c || !values || !bytes) return fail(c, HALE_EINVAL, "encode: NULL argument");
  int rc = encode_check(c, dtype, rows, cols);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  size_t nin = rows * cols * 4, nout = rows * (size_t)hale_row_bytes(dtype, cols);
  void* s;
  rc = ctx_scratch(c, align_up(nin, 256) + nout, &s);
  if (rc) return rc;
  float* dv = (float*)s;
  uint8_t* db = (uint8_t*)s + align_up(nin, 256);
  HIPCHK(c, hipMemcpyAsync(dv, values, nin, hipMemcpyHostToDevice, c->stream));
  rc = encode_enqueue(c, dtype, rows, cols, dv, db);
  if (rc) return rc;
  HIPCHK(c, hipMemcpyAsync(bytes, db, nout, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// decoding and conversion
// ---------------------------------------------------------------------------

static int decode_check(hale_ctx* c, int dtype, size_t cols) {
  if (dtype < HALE_F32 || dtype > HALE_Q4_0) return fail(c, HALE_EINVAL, "decode: unknown dtype %d", dtype);
  if (hale_row_bytes(dtype, cols) < 0)
    return fail(c, HALE_EINVAL, "%s needs row length divisible by 32, got %zu", dtype == HALE_Q8_0 ? "Q8_0" : "Q4_0", cols);
  return HALE_OK;
}

extern "C" int hale_decode_rows_device(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                       const void* d_bytes, float* d_values) {
  if (!c || !d_bytes || !d_values) return fail(c, HALE_EINVAL, "decode: NULL argument");
  int rc = decode_check(c, dtype, cols);
  if (rc) return rc;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  LAUNCH(c, K_DECODE, launch_decode_ref(dtype, d_bytes, rows * cols, d_values, c->stream));
  return HALE_OK;
}

extern "C" int hale_decode_rows(hale_ctx* c, int dtype, size_t rows, size_t cols,
                                const void* bytes, float* values) {
  if (!c || !bytes || !values) return fail(c, HALE_EINVAL, "decode: NULL argument");
  int rc = decode_check(c, dtype, cols);
  if (rc) return rc;
  if (rows == 0 || cols == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  const size_t nin = rows * (size_t)hale_row_bytes(dtype, cols), nout = rows * cols * 4;
  void* s;
  rc = ctx_scratch(c, align_up(nin, 256) + nout, &s);
  if (rc) return rc;
  uint8_t* db = (uint8_t*)s;
  float* dv = (float*)((char*)s + align_up(nin, 256));
  HIPCHK(c, hipMemcpyAsync(db, bytes, nin, hipMemcpyHostToDevice, c->stream));
  LAUNCH(c, K_DECODE, launch_decode_ref(dtype, db, rows * cols, dv, c->stream));
  HIPCHK(c, hipMemcpyAsync(values, dv, nout, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// Enqueues rows first .. first + count - 1 of m, decoded, into dv[count][cols].
static int matrix_rows_enqueue(hale_ctx* c, const hale_matrix* m, size_t first, size_t count,
                               float* dv) {
  if (quantized(m->dtype)) {
    LAUNCH(c, K_DECODE, launch_decode_tiles(m->dtype, m->codes, m->scales, first, count, m->cols, dv, c->stream));
  } else {
    const size_t rb = (size_t)hale_row_bytes(m->dtype, m->cols);
    LAUNCH(c, K_DECODE, launch_decode_ref(m->dtype, (const uint8_t*)m->raw + first * rb, count * m->cols, dv, c->stream));
  }
  return HALE_OK;
}

extern "C" int hale_matrix_rows_to_f32_device(hale_ctx* c, const hale_matrix* m, size_t first,
                                              size_t count, float* d_values) {
  if (!c || !m || !d_values) return fail(c, HALE_EINVAL, "row_to_f32: NULL argument");
  if (first > m->rows || count > m->rows - first)
    return fail(c, HALE_EINVAL, "rows %zu..%zu of a %zu-row matrix", first, first + count, m->rows);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  return matrix_rows_enqueue(c, m, first, count, d_values);
}

extern "C" int hale_matrix_rows_to_f32(hale_ctx* c, const hale_matrix* m, size_t first,
                                       size_t count, float* values) {
  if (!c || !m || !values) return fail(c, HALE_EINVAL, "row_to_f32: NULL argument");
  if (first > m->rows || count > m->rows - first)
    return fail(c, HALE_EINVAL, "rows %zu..%zu of a %zu-row matrix", first, first + count, m->rows);
  if (count == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  const size_t n = count * m->cols;
  void* s;
  int rc = ctx_scratch(c, n * 4, &s);
  if (rc) return rc;
  rc = matrix_rows_enqueue(c, m, first, count, (float*)s);
  if (rc) return rc;
  HIPCHK(c, hipMemcpyAsync(values, s, n * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

extern "C" int hale_matrix_to_f32(hale_ctx* c, const hale_matrix* m, float* values, size_t n) {
  if (!c || !m || !values) return fail(c, HALE_EINVAL, "to_f32: NULL argument");
  if (n != m->rows * m->cols)
    return fail(c, HALE_EINVAL, "to_f32 of a %zux%zu matrix needs %zu values, got %zu", m->rows, m->cols,
                m->rows * m->cols, n);
  return hale_matrix_rows_to_f32(c, m, 0, m->rows, values);
}

// Rows per pass of hale_matrix_convert: the f32 rows of one pass stay
// within 64 MiB of scratch.
static size_t convert_rows_per_pass(size_t cols) { return std::max<size_t>(1, (64u << 20) / (cols * 4)); }

extern "C" int hale_matrix_convert(hale_ctx* c, const hale_matrix* m, int dtype, hale_matrix** out) {
  if (!c || !m || !out) return fail(c, HALE_EINVAL, "convert: NULL argument");
  *out = nullptr;
  int rc = encode_check(c, dtype, m->rows, m->cols);
  if (rc) return rc;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  const size_t rb = (size_t)hale_row_bytes(dtype, m->cols), nbytes = m->rows * rb;
  void* bytes = nullptr;  // the converted matrix in the reference layout
  if (hipMalloc(&bytes, nbytes) != hipSuccess)
    return fail(c, HALE_ENOMEM, "device allocation of %zu bytes", nbytes);
  if (dtype == m->dtype && !quantized(dtype)) {
    rc = hipMemcpyAsync(bytes, m->raw, nbytes, hipMemcpyDeviceToDevice, c->stream) == hipSuccess
             ? HALE_OK
             : fail(c, HALE_EHIP, "convert: copy failed");
  } else if (dtype == m->dtype) {
    rc = launch_unpack(dtype, m->codes, m->scales, m->rows, m->cols, (uint8_t*)bytes, c->stream) == hipSuccess
             ? HALE_OK
             : fail(c, HALE_EHIP, "convert: unpack failed");
  } else {  // to_f32, then from_f32 into the new dtype, a pass of rows at a time
    const size_t per = convert_rows_per_pass(m->cols);
    void* s = nullptr;
    rc = ctx_scratch(c, std::min(per, m->rows) * m->cols * 4, &s);
    for (size_t r = 0; rc == HALE_OK && r < m->rows; r += per) {
      const size_t n = std::min(per, m->rows - r);
      rc = matrix_rows_enqueue(c, m, r, n, (float*)s);
      if (rc == HALE_OK) rc = encode_enqueue(c, dtype, n, m->cols, (const float*)s, (uint8_t*)bytes + r * rb);
    }
  }
  if (rc == HALE_OK) rc = matrix_create(c, dtype, m->rows, m->cols, bytes, nbytes, true, out);
  (void)hipStreamSynchronize(c->stream);
  (void)hipFree(bytes);
  return rc;
}

// ---------------------------------------------------------------------------
// matvec
// ---------------------------------------------------------------------------

static GemvArgs plain_args(const hale_matrix* m, const ActBlock* act, float* out) {
  GemvArgs a{};
  a.codes = m->codes;
  a.scales = m->scales;
  a.nb = (int)(m->cols / HALE_QK);
  a.rows = (int)m->rows;
  a.act = act;
  a.out = out;
  a.slots = 1;
  return a;
}

// Enqueues out = m x for device x/out: float matrices through the 8-lane
// float GEMV, quantized ones through activation quantization and the tile
// GEMV.
static int matvec_enqueue(hale_ctx* c, const hale_matrix* m, const float* dx, float* dout,
                          ActBlock* act) {
  if (!quantized(m->dtype)) {
    if ((uintptr_t)dx % 16) return fail(c, HALE_EINVAL, "matvec: x must be 16-byte aligned");
    LAUNCH(c, K_GEMV, launch_gemv_float(m->dtype, m->raw, dx, m->rows, m->cols, dout, c->stream));
    return HALE_OK;
  }
  size_t nb = m->cols / HALE_QK;
  MatvecArgs mv{m->codes, m->scales, (int)nb, (int)m->rows, nullptr, nullptr, dout};
  if (((uintptr_t)dx & 15) == 0 && matvec_takes_x((int)nb, m->rows)) {  // one launch
    mv.x = dx;
    LAUNCH(c, K_GEMV, launch_matvec(m->dtype, mv, c->stream));
    return HALE_OK;
  }
  LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, nb, act, c->stream));
  if (nb <= (size_t)MATVEC_MAX_NB) {
    mv.act = act;
    LAUNCH(c, K_GEMV, launch_matvec(m->dtype, mv, c->stream));
    return HALE_OK;
  }
  // longer rows: lane-per-row chains over every block
  RowsArgs r{};
  r.codes = m->codes;
  r.scales = m->scales;
  r.nb = (int)nb;
  r.rows = (int)m->rows;
  r.act = act;
  r.act_div = 1;
  r.out = dout;
  LAUNCH(c, K_GEMV, launch_matvec_rows(m->dtype, r, 1, c->stream));
  return HALE_OK;
}

extern "C" int hale_matvec(hale_ctx* c, const hale_matrix* m, const float* x, size_t xlen,
                           float* out, size_t outlen) {
  if (!c || !m || !x || !out) return fail(c, HALE_EINVAL, "matvec: NULL argument");
  if (xlen != m->cols) return fail(c, HALE_EINVAL, "matvec input length %zu != cols %zu", xlen, m->cols);
  if (outlen != m->rows) return fail(c, HALE_EINVAL, "matvec output length %zu != rows %zu", outlen, m->rows);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  size_t nb = m->cols / HALE_QK;
  size_t o1 = align_up(xlen * 4, 256), o2 = o1 + align_up(outlen * 4, 256);
  void* s;
  int rc = ctx_scratch(c, o2 + nb * sizeof(ActBlock), &s);
  if (rc) return rc;
  float* dx = (float*)s;
  float* dout = (float*)((char*)s + o1);
  ActBlock* act = (ActBlock*)((char*)s + o2);
  HostStage st(c);
  if ((rc = st.reserve(o2)) || (rc = st.in(dx, x, xlen * 4))) return rc;
  rc = matvec_enqueue(c, m, dx, dout, act);
  if (rc || (rc = st.out(out, dout, outlen * 4))) return rc;
  return st.finish();
}

extern "C" int hale_matvec_device(hale_ctx* c, const hale_matrix* m, const float* d_x, float* d_out) {
  if (!c || !m || !d_x || !d_out) return fail(c, HALE_EINVAL, "matvec: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  void* s;
  int rc = ctx_scratch(c, (m->cols / HALE_QK) * sizeof(ActBlock), &s);
  if (rc) return rc;
  return matvec_enqueue(c, m, d_x, d_out, (ActBlock*)s);
}

extern "C" int hale_matvec_block_sums(hale_ctx* c, const hale_matrix* m, const float* x,
                                      size_t xlen, int32_t* isums) {
  if (!c || !m || !x || !isums) return fail(c, HALE_EINVAL, "block_sums: NULL argument");
  if (!quantized(m->dtype)) return fail(c, HALE_EINVAL, "block sums need a quantized matrix");
  if (xlen != m->cols) return fail(c, HALE_EINVAL, "input length %zu != cols %zu", xlen, m->cols);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  size_t nb = m->cols / HALE_QK;
  size_t n = m->rows * nb;
  size_t o1 = align_up(xlen * 4, 256), o2 = o1 + align_up(nb * sizeof(ActBlock), 256);
  void* s;
  int rc = ctx_scratch(c, o2 + n * 4, &s);
  if (rc) return rc;
  float* dx = (float*)s;
  ActBlock* act = (ActBlock*)((char*)s + o1);
  int32_t* dsum = (int32_t*)((char*)s + o2);
  HIPCHK(c, hipMemcpyAsync(dx, x, xlen * 4, hipMemcpyHostToDevice, c->stream));
  LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, nb, act, c->stream));
  LAUNCH(c, K_GEMV, launch_block_sums(m->dtype, m->codes, act, m->rows, m->cols, dsum, c->stream));
  HIPCHK(c, hipMemcpyAsync(isums, dsum, n * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// expert
// ---------------------------------------------------------------------------

static int expert_check(hale_ctx* c, const hale_matrix* gate, const hale_matrix* up,
                        const hale_matrix* down) {
  if (!quantized(gate->dtype) || gate->dtype != up->dtype || gate->dtype != down->dtype)
    return fail(c, HALE_EINVAL, "expert matrices must share one quantized dtype");
  size_t I = gate->rows, H = gate->cols;
  if (up->rows != I || up->cols != H || down->rows != H || down->cols != I)
    return fail(c, HALE_EINVAL, "expert shapes: gate %zux%zu up %zux%zu down %zux%zu", gate->rows,
                gate->cols, up->rows, up->cols, down->rows, down->cols);
  return HALE_OK;
}

// Bytes of scratch expert_enqueue needs after `lead` bytes of the caller's:
// x's q8 blocks, h's q8 blocks, then the f32 h (or g) and u.
static size_t expert_scratch_bytes(const hale_matrix* gate, size_t lead) {
  const size_t nbh = gate->cols / HALE_QK, nbi = gate->rows / HALE_QK;
  return lead + align_up(nbh * sizeof(ActBlock), 256) + align_up(nbi * sizeof(ActBlock), 256) +
         2 * align_up(gate->rows * 4, 256);
}

// Enqueues Expert::forward for device x/out: q8 activation blocks of x, the
// gate/up GEMV with SiLU and requantization, the down GEMV.  The activation
// blocks live in the context scratch from byte `lead` on (the caller's own
// staging sits before it).
static int expert_enqueue(hale_ctx* c, const hale_matrix* gate, const hale_matrix* up,
                          const hale_matrix* down, const float* dx, float* dout, size_t lead) {
  const size_t I = gate->rows, H = gate->cols, nbh = H / HALE_QK, nbi = I / HALE_QK;
  void* s;
  int rc = ctx_scratch(c, expert_scratch_bytes(gate, lead), &s);
  if (rc) return rc;
  ActBlock* act = (ActBlock*)((char*)s + lead);
  ActBlock* hact = (ActBlock*)((char*)s + lead + align_up(nbh * sizeof(ActBlock), 256));
  float* gv = (float*)((char*)hact + align_up(nbi * sizeof(ActBlock), 256));  // f32 h
  // An aligned x of up to 128 blocks, with h of up to 128: gate and up rows
  // in one launch of row chains (x quantized in the kernel), a work-group's
  // gate and up chains of the same rows writing their f32 h = silu(g) * u;
  // then down, which quantizes h while staging its input (the same
  // expressions as requantizing h in the gate/up epilogue, so the same
  // bits), each launch spread over rows rather than over h's 32-row blocks.
  if (((uintptr_t)dx & 15) == 0 && nbh <= (size_t)MATVEC_XQ_MAX_NB && nbi <= (size_t)MATVEC_XQ_MAX_NB) {
    MatvecArgs p{};
    p.codes = gate->codes;
    p.scales = gate->scales;
    p.codes2 = up->codes;
    p.scales2 = up->scales;
    p.nb = (int)nbh;
    p.rows = (int)I;
    p.x = dx;
    p.out = gv;
    LAUNCH(c, K_GATE_UP, launch_matvec_pair(gate->dtype, p, c->stream));
    MatvecArgs d{};
    d.codes = down->codes;
    d.scales = down->scales;
    d.nb = (int)nbi;
    d.rows = (int)H;
    d.x = gv;
    d.out = dout;
    LAUNCH(c, K_DOWN, launch_matvec(down->dtype, d, c->stream));
    return HALE_OK;
  }
  if (nbh > FAST_MAX_NB || nbi > (size_t)MATVEC_MAX_NB) {
    // rows longer than the tile kernels take: lane-per-row chains for gate
    // and up, h = silu(g) * u requantized, lane-per-row chains for down
    float* uv = gv + align_up(I * 4, 256) / 4;
    LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, nbh, act, c->stream));
    RowsArgs r{};
    r.nb = (int)nbh;
    r.rows = (int)I;
    r.act = act;
    r.act_div = 1;
    r.codes = gate->codes;
    r.scales = gate->scales;
    r.out = gv;
    LAUNCH(c, K_GATE_UP, launch_matvec_rows(gate->dtype, r, 1, c->stream));
    r.codes = up->codes;
    r.scales = up->scales;
    r.out = uv;
    LAUNCH(c, K_GATE_UP, launch_matvec_rows(up->dtype, r, 1, c->stream));
    LAUNCH(c, K_GATE_UP, launch_swiglu_quant(gv, uv, nbi, hact, c->stream));
    RowsArgs d{};
    d.codes = down->codes;
    d.scales = down->scales;
    d.nb = (int)nbi;
    d.rows = (int)H;
    d.act = hact;
    d.act_div = 1;
    d.out = dout;
    LAUNCH(c, K_DOWN, launch_matvec_rows(down->dtype, d, 1, c->stream));
    return HALE_OK;
  }
  // the gate/up kernel quantizes an aligned x of up to 128 blocks itself
  const bool fuse = ((uintptr_t)dx & 15) == 0 && nbh <= (size_t)GEMV_X_MAX_NB;
  if (!fuse) LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, nbh, act, c->stream));
  GemvArgs a{};
  a.codes = gate->codes;
  a.scales = gate->scales;
  a.codes2 = up->codes;
  a.scales2 = up->scales;
  a.nb = (int)nbh;
  a.rows = (int)I;
  a.act = fuse ? nullptr : act;
  a.x = fuse ? dx : nullptr;
  a.hact = hact;
  a.hact_stride = (int)nbi;
  a.slots = 1;
  LAUNCH(c, K_GATE_UP, launch_gemv(gate->dtype, EPI_GATE_UP, a, (int)nbi, 1, c->stream));
  if (nbi <= (size_t)MATVEC_MAX_NB) {
    MatvecArgs mv{down->codes, down->scales, (int)nbi, (int)H, nullptr, hact, dout};
    LAUNCH(c, K_DOWN, launch_matvec(down->dtype, mv, c->stream));
  } else {
    GemvArgs d = plain_args(down, hact, dout);
    LAUNCH(c, K_DOWN, launch_gemv(down->dtype, EPI_PLAIN, d, (int)(padded_rows(H) / 64), 1, c->stream));
  }
  return HALE_OK;
}

extern "C" int hale_expert_forward(hale_ctx* c, const hale_matrix* gate, const hale_matrix* up,
                                   const hale_matrix* down, const float* x, float* out) {
  if (!c || !gate || !up || !down || !x || !out) return fail(c, HALE_EINVAL, "expert_forward: NULL argument");
  int rc = expert_check(c, gate, up, down);
  if (rc) return rc;
  const size_t H = gate->cols, io = align_up(H * 4, 256);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  void* s;
  rc = ctx_scratch(c, expert_scratch_bytes(gate, 2 * io), &s);  // x, out, then the blocks
  if (rc) return rc;
  float* dx = (float*)s;
  float* dout = (float*)((char*)s + io);
  HostStage st(c);
  if ((rc = st.reserve(2 * io)) || (rc = st.in(dx, x, H * 4))) return rc;
  rc = expert_enqueue(c, gate, up, down, dx, dout, 2 * io);
  if (rc || (rc = st.out(out, dout, H * 4))) return rc;
  return st.finish();
}

extern "C" int hale_expert_forward_device(hale_ctx* c, const hale_matrix* gate,
                                          const hale_matrix* up, const hale_matrix* down,
                                          const float* d_x, float* d_out) {
  if (!c || !gate || !up || !down || !d_x || !d_out)
    return fail(c, HALE_EINVAL, "expert_forward: NULL argument");
  int rc = expert_check(c, gate, up, down);
  if (rc) return rc;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  return expert_enqueue(c, gate, up, down, d_x, d_out, 0);
}

// ---------------------------------------------------------------------------
// MoE layer
// ---------------------------------------------------------------------------

// Per-token scratch of one forward over ntok tokens, carved from one
// buffer: q8 activation blocks, router logits, the chosen experts and their
// weights.  Nothing in it has to start at zero.
struct TokScratch {
  ActBlock* act;   // [ntok][H/32]
  float* logits;   // [ntok][E]
  int* route_idx;  // [ntok][k]
  float* route_w;  // [ntok][k]
  ActBlock* hact;  // [decode tokens][k][I/32], the decode path's requantized h
};

// h blocks are kept for the tokens a decode pass can take: min(ntok,
// grouped_min - 1), so scratch laid out for more tokens holds at least as many
static size_t hact_tokens(const hale_moe* m, size_t ntok) {
  return m->wide ? 0 : std::min(ntok, m->grouped_min - 1);
}

static size_t tok_scratch_bytes(const hale_moe* m, size_t ntok) {
  const size_t k = std::max<size_t>(m->k, 1);
  return align_up(ntok * (m->H / HALE_QK) * sizeof(ActBlock), 256) + align_up(ntok * m->E * 4, 256) +
         2 * align_up(ntok * k * 4, 256) +
         align_up(hact_tokens(m, ntok) * k * (m->I / HALE_QK) * sizeof(ActBlock), 256);
}

static TokScratch tok_scratch_carve(const hale_moe* m, void* base, size_t ntok) {
  const size_t k = std::max<size_t>(m->k, 1);
  char* p = (char*)base;
  TokScratch s;
  s.act = (ActBlock*)p;
  p += align_up(ntok * (m->H / HALE_QK) * sizeof(ActBlock), 256);
  s.logits = (float*)p;
  p += align_up(ntok * m->E * 4, 256);
  s.route_idx = (int*)p;
  p += align_up(ntok * k * 4, 256);
  s.route_w = (float*)p;
  p += align_up(ntok * k * 4, 256);
  s.hact = (ActBlock*)p;
  return s;
}

// The layer's per-token scratch for at least ntok tokens (laid out anew
// after the grouped threshold changed).
static int moe_reserve(hale_moe* m, size_t ntok, TokScratch* out) {
  hale_ctx* c = m->ctx;
  if (m->cap_tok < ntok || m->cap_gmin != m->grouped_min) {
    const size_t bytes = tok_scratch_bytes(m, ntok);
    int rc = growth_allowed(c, "MoE layer scratch", bytes);
    if (rc) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    scratch_release(c, m->tok_base);
    m->tok_base = nullptr;
    m->cap_tok = 0;
    hipError_t e = hipMalloc(&m->tok_base, bytes);
    if (e != hipSuccess) {
      m->tok_base = nullptr;
      return fail(c, HALE_ENOMEM, "MoE scratch for %zu tokens: %s", ntok, hipGetErrorString(e));
    }
    m->cap_tok = std::max(ntok, m->cap_tok);
    m->cap_gmin = m->grouped_min;
  }
  *out = tok_scratch_carve(m, m->tok_base, m->cap_tok);
  return HALE_OK;
}

// The layer's workspace (the grouped path's, or the general path's) of at
// least `need` bytes.
static int moe_ws(hale_moe* m, size_t need, void** out) {
  hale_ctx* c = m->ctx;
  if (m->pw.bytes < need) {
    int rc = growth_allowed(c, "MoE layer workspace", need);
    if (rc) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    scratch_release(c, m->pw.base);
    m->pw.base = nullptr;
    m->pw.bytes = 0;
    if (hipMalloc(&m->pw.base, need) != hipSuccess)
      return fail(c, HALE_ENOMEM, "MoE layer workspace of %zu bytes", need);
    m->pw.bytes = need;
  }
  *out = m->pw.base;
  return HALE_OK;
}

// Fewest tokens per forward that take the expert-grouped path.  The
// grouped path has a fixed cost (routing, grouping, combine launches) and
// then reads each touched expert once; the decode path adds each token's k
// experts' bytes.  Measured crossovers against the row-chain grouped
// kernels (graph replay over layers visited in turn, one MI355X):
// Qwen3-30B q4_0 (top-8 of 128) between 10 and 11 tokens (49.3 against
// 55.0 us at 10, 58.9 against 58.2 at 11), Qwen3-235B q4_0 at 8 (125.8
// both; 153 against 136 at 10), Qwen3-30B q8_0 between 10 and 12 (73.4
// against 75.7 at 10, 85.1 against 83.1 at 12), a Qwen3-235B-shaped q8_0
// layer between 7 and 8 (175.6 against 177.4 us at 7, 196.3 against 188.8
// at 8); Mixtral (top-2 of 8)
// between 6 and 7 (173.1 against 180.5 us at 6, 208.8 against 186.9 at 7,
// with the spread-term down projection and four-tile gate/up work-groups).
static size_t default_grouped_min(int dtype, size_t E, size_t H, size_t I, size_t k) {
  (void)E;
  (void)I;
  if (k < 4) return 7;
  if (dtype == HALE_Q4_0) return H <= 2048 ? 11 : 9;
  return H <= 2048 ? 12 : 8;
}

// Most tokens per grouped forward that take the row-chain kernels rather
// than the matrix products.  The row-chain kernels read an expert's weights
// once per tile of two or four assignments (from L2 for an expert's later
// tiles, with ordinary loads above two assignments per expert), so they
// lose once experts hold several.  The crossovers (same measurement):
// Qwen3-30B q4_0 at about 4.75 E / k tokens (72 tokens: 118.4 against 121.7
// us, 80: 124.4 against 122.1), Qwen3-235B q4_0 with tiles of four at 4.25
// E / k (68 tokens 355.1 against 356.9 us, 72: 367.6 against 357.6),
// Qwen3-30B q8_0 with tiles of four at 5 E / k (80 tokens 160.9 against
// 164.9 us, 88: 171.9 against 165.1), a Qwen3-235B-shaped q8_0 layer with
// tiles of four at 3.75 E / k (60 tokens 498.8 against 511.9 us, 64: 517.5
// against 515.1) and Mixtral (448-block down rows) at 3.25 E / k (12
// tokens 244.5 against 252 us, 14: 261 against 252).
static size_t default_band_max(int dtype, size_t E, size_t H, size_t I, size_t k) {
  size_t c4;  // quarter-assignments per expert
  if (I / HALE_QK > 256) c4 = 13;
  else if (dtype == HALE_Q4_0) c4 = H <= 2048 ? 19 : 17;
  else c4 = H <= 2048 ? 20 : 15;
  return c4 * E / (4 * std::max<size_t>(k, 1));
}

extern "C" int hale_moe_create(hale_ctx* c, uint32_t layer, size_t E, size_t H, size_t I, int dtype,
                               size_t top_k, int normalize, const hale_matrix* router,
                               hale_moe** out) {
  if (!c || !out) return fail(c, HALE_EINVAL, "moe_create: NULL argument");
  *out = nullptr;
  if (!quantized(dtype)) return fail(c, HALE_EINVAL, "expert dtype %d is not q8_0/q4_0", dtype);
  if (E == 0 || E > (size_t)INT32_MAX) return fail(c, HALE_EINVAL, "num_experts %zu outside 1..2^31-1", E);
  if (H == 0 || I == 0 || H % HALE_QK || I % HALE_QK)
    return fail(c, HALE_EINVAL, "hidden %zu / inter %zu must be non-zero multiples of 32", H, I);
  if (H > (size_t)INT32_MAX / 4 || I > (size_t)INT32_MAX / 4)
    return fail(c, HALE_EINVAL, "hidden %zu / inter %zu too large", H, I);
  if (router && (router->dtype != HALE_F32 || router->rows != E || router->cols != H))
    return fail(c, HALE_EINVAL, "router must be f32 [%zu x %zu]", E, H);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  hale_moe* m = new (std::nothrow) hale_moe;
  if (!m) return fail(c, HALE_ENOMEM, "out of host memory");
  m->ctx = c;
  m->layer = layer;
  m->E = E;
  m->H = H;
  m->I = I;
  m->k = std::min(top_k, E);  // top_k clamps k to the number of scores
  m->wide = E > FAST_MAX_E || H > FAST_MAX_H || m->k > FAST_MAX_K || I / HALE_QK > FAST_MAX_NB;
  // (a wide layer never takes the grouped path)
  m->grouped_min = m->wide ? SIZE_MAX : default_grouped_min(dtype, E, H, I, m->k);
  m->band_max = default_band_max(dtype, E, H, I, m->k);
  m->dtype = dtype;
  m->normalize = normalize;
  m->gc_bytes = code_plane_bytes(dtype, I, H);
  m->gs_elems = scale_plane_bytes(I, H) / 2;
  m->dc_bytes = code_plane_bytes(dtype, H, I);
  m->ds_elems = scale_plane_bytes(H, I) / 2;
  m->present.assign(E, 0);
  m->fetch_counts.assign(E, 0);
  m->views.assign(3 * E, nullptr);
  hipError_t e = hipSuccess;
#define ALLOC(p, n) \
  if (e == hipSuccess) e = hipMalloc(&(p), (n))
  ALLOC(m->gate_c, E * m->gc_bytes);
  ALLOC(m->up_c, E * m->gc_bytes);
  ALLOC(m->down_c, E * m->dc_bytes);
  ALLOC(m->gate_s, E * m->gs_elems * 2);
  ALLOC(m->up_s, E * m->gs_elems * 2);
  ALLOC(m->down_s, E * m->ds_elems * 2);
  ALLOC(m->stats, E * 8);
  if (router) ALLOC(m->router, E * H * 4);
#undef ALLOC
  if (e == hipSuccess) e = launch_fill((float*)m->stats, 2 * E, 0.0f, c->stream);  // zero counts
  if (e == hipSuccess && router)
    e = hipMemcpyAsync(m->router, router->raw, E * H * 4, hipMemcpyDeviceToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    hale_moe_destroy(m);
    return fail(c, HALE_ENOMEM, "MoE layer allocation (%zu experts): %s", E, hipGetErrorString(e));
  }
  *out = m;
  return HALE_OK;
}

extern "C" void hale_moe_destroy(hale_moe* m) {
  if (!m) return;
  hale_ctx* c = m->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)moe_wait_load(m);
  (void)hipStreamSynchronize(c->stream);
  if (m->loaded) (void)hipEventDestroy(m->loaded);
  (void)hipFree(m->tok_base);
  (void)hipFree(m->pw.base);
  (void)hipFree(m->gate_c);
  (void)hipFree(m->up_c);
  (void)hipFree(m->down_c);
  (void)hipFree(m->gate_s);
  (void)hipFree(m->up_s);
  (void)hipFree(m->down_s);
  (void)hipFree(m->stats);
  (void)hipFree(m->router);
  for (hale_matrix* v : m->views) delete v;
  if (m->source) {
    auto& ls = m->source->layers;
    ls.erase(std::remove(ls.begin(), ls.end(), m), ls.end());
  }
  delete m;
}

static int set_expert(hale_moe* m, uint32_t e, const void* gate, const void* up, const void* down,
                      size_t ng, size_t nd, bool on_device) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !gate || !up || !down) return fail(c, HALE_EINVAL, "set_expert: NULL argument");
  if (e >= m->E) return fail(c, HALE_EINVAL, "expert %u of %zu", e, m->E);
  size_t need_g = m->I * (size_t)hale_row_bytes(m->dtype, m->H);
  size_t need_d = m->H * (size_t)hale_row_bytes(m->dtype, m->I);
  if (ng != need_g || nd != need_d)
    return fail(c, HALE_EINVAL, "expert bytes gate/up %zu (need %zu), down %zu (need %zu)", ng,
                need_g, nd, need_d);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc0 = moe_wait_load(m);
  if (rc0) return rc0;
  const uint8_t *sg = (const uint8_t*)gate, *su = (const uint8_t*)up, *sd = (const uint8_t*)down;
  if (!on_device) {
    void* s;
    int rc = ctx_scratch(c, 2 * align_up(need_g, 256) + need_d, &s);
    if (rc) return rc;
    uint8_t* b = (uint8_t*)s;
    HIPCHK(c, hipMemcpyAsync(b, gate, need_g, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(b + align_up(need_g, 256), up, need_g, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(b + 2 * align_up(need_g, 256), down, need_d, hipMemcpyHostToDevice, c->stream));
    sg = b;
    su = b + align_up(need_g, 256);
    sd = b + 2 * align_up(need_g, 256);
  }
  LAUNCH(c, K_REPACK, launch_repack(m->dtype, sg, m->I, m->H, m->gate_c + e * m->gc_bytes, m->gate_s + e * m->gs_elems, c->stream));
  LAUNCH(c, K_REPACK, launch_repack(m->dtype, su, m->I, m->H, m->up_c + e * m->gc_bytes, m->up_s + e * m->gs_elems, c->stream));
  LAUNCH(c, K_REPACK, launch_repack(m->dtype, sd, m->H, m->I, m->down_c + e * m->dc_bytes, m->down_s + e * m->ds_elems, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  m->present[e] = 1;
  return HALE_OK;
}

extern "C" int hale_moe_set_expert(hale_moe* m, uint32_t e, const void* gate, const void* up,
                                   const void* down, size_t ng, size_t nd) {
  return set_expert(m, e, gate, up, down, ng, nd, false);
}

extern "C" int hale_moe_set_expert_device(hale_moe* m, uint32_t e, const void* gate, const void* up,
                                          const void* down, size_t ng, size_t nd) {
  return set_expert(m, e, gate, up, down, ng, nd, true);
}

extern "C" int hale_moe_set_expert_matrices(hale_moe* m, uint32_t e, const hale_matrix* gate,
                                            const hale_matrix* up, const hale_matrix* down) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !gate || !up || !down) return fail(c, HALE_EINVAL, "set_expert: NULL argument");
  if (e >= m->E) return fail(c, HALE_EINVAL, "expert %u of %zu", e, m->E);
  for (const hale_matrix* x : {gate, up, down})
    if (x->dtype != m->dtype) return fail(c, HALE_EINVAL, "expert dtype %d != layer dtype %d", x->dtype, m->dtype);
  if (gate->rows != m->I || gate->cols != m->H || up->rows != m->I || up->cols != m->H ||
      down->rows != m->H || down->cols != m->I)
    return fail(c, HALE_EINVAL, "expert shapes do not match the layer");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_wait_load(m);
  if (rc) return rc;
  // identical padded geometry, so the planes copy as they are
  HIPCHK(c, hipMemcpyAsync(m->gate_c + e * m->gc_bytes, gate->codes, m->gc_bytes, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(m->up_c + e * m->gc_bytes, up->codes, m->gc_bytes, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(m->down_c + e * m->dc_bytes, down->codes, m->dc_bytes, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(m->gate_s + e * m->gs_elems, gate->scales, m->gs_elems * 2, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(m->up_s + e * m->gs_elems, up->scales, m->gs_elems * 2, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(m->down_s + e * m->ds_elems, down->scales, m->ds_elems * 2, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  m->present[e] = 1;
  return HALE_OK;
}

// Waits for this layer's pending pack load: joins the loader thread, then
// orders the context's stream after the uploads.
static int moe_wait_load(hale_moe* m) {
  if (!m->load) return HALE_OK;
  hale_ctx* c = m->ctx;
  std::shared_ptr<hale::PackLoad> L = std::move(m->load);
  L->join();
  if (L->rc != HALE_OK) return fail(c, L->rc, "%s", L->err.c_str());
  HIPCHK(c, hipStreamWaitEvent(c->stream, m->loaded, 0));
  std::fill(m->present.begin(), m->present.end(), (char)1);
  m->bytes_loaded += L->bytes;
  m->load_seconds += L->seconds;
  return HALE_OK;
}

static int check_all_present(hale_moe* m) {
  for (size_t e = 0; e < m->E; e++)
    if (!m->present[e])
      return fail(m->ctx, HALE_ENOTFOUND, "expert L%uE%zu is not registered", m->layer, e);
  return HALE_OK;
}

// Enqueues the decode path for ntok tokens (token t's route in slot range
// [t*k, t*k+k)).  x/logits/out are device pointers.
static int moe_decode_enqueue(hale_moe* m, size_t ntok, const float* dx, const float* dlogits,
                              float* dout, const TokScratch& s) {
  hale_ctx* c = m->ctx;
  const int k = (int)m->k;
  const size_t nbh = m->H / HALE_QK, nbi = m->I / HALE_QK;
  if (dlogits)
    LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, ntok * nbh, s.act, c->stream));
  else
    LAUNCH(c, K_ROUTE, launch_route_logits(m->router, dx, (int)m->H, (int)m->E, (int)ntok, s.act,
                                           s.logits, c->stream));
  // every token's gate/up in one launch (grid row = token x k + slot), then
  // every token's down projection and combine in one
  const float* lg = dlogits ? dlogits : s.logits;
  {
    GemvArgs a{};
    a.codes = m->gate_c;
    a.scales = m->gate_s;
    a.codes2 = m->up_c;
    a.scales2 = m->up_s;
    a.codes_stride = m->gc_bytes;
    a.scales_stride = m->gs_elems;
    a.nb = (int)nbh;
    a.rows = (int)m->I;
    a.act = s.act;
    a.act_stride = 0;
    a.act_tstride = (int)nbh;
    a.tokens = (int)ntok;
    a.route_idx = nullptr;  // the prologue selects the experts from the logits
    a.logits = lg;
    a.E = (int)m->E;
    a.normalize = m->normalize;
    a.route_out_idx = s.route_idx;
    a.route_out_w = s.route_w;
    a.stats = m->stats;
    a.hact = s.hact;
    a.hact_stride = (int)nbi;
    a.slots = k;
    LAUNCH(c, K_GATE_UP, launch_gemv(m->dtype, EPI_GATE_UP, a, (int)nbi, k, c->stream));
    DownArgs d{};
    d.codes = m->down_c;
    d.scales = m->down_s;
    d.codes_stride = m->dc_bytes;
    d.scales_stride = m->ds_elems;
    d.nb = (int)nbi;
    d.rows = (int)m->H;
    d.hact = s.hact;
    d.hact_stride = (int)nbi;
    d.route_idx = s.route_idx;
    d.route_w = s.route_w;
    d.slots = k;
    d.out = dout;
    d.tokens = (int)ntok;
    LAUNCH(c, K_DOWN, launch_down_combine(m->dtype, d, c->stream));
  }
  return HALE_OK;
}

static PrefillLayer prefill_layer(hale_moe* m, const TokScratch& s) {
  PrefillLayer L{};
  L.dtype = m->dtype;
  L.E = (int)m->E;
  L.H = (int)m->H;
  L.I = (int)m->I;
  L.k = (int)m->k;
  L.normalize = m->normalize;
  L.router = m->router;
  L.gate_c = m->gate_c;
  L.up_c = m->up_c;
  L.down_c = m->down_c;
  L.gate_s = m->gate_s;
  L.up_s = m->up_s;
  L.down_s = m->down_s;
  L.gc_bytes = m->gc_bytes;
  L.gs_elems = m->gs_elems;
  L.dc_bytes = m->dc_bytes;
  L.ds_elems = m->ds_elems;
  L.act = s.act;
  L.logits = s.logits;
  L.route_idx = s.route_idx;
  L.route_w = s.route_w;
  L.stats = m->stats;
  L.down_fold = m->down_fold == HALE_FOLD_FMA ? DOWN_FOLD_FMA : DOWN_FOLD_EXACT;
  L.band_max = m->band_max;
  return L;
}

// ---------------------------------------------------------------------------
// the general path: layers beyond the fast kernels' shapes
// ---------------------------------------------------------------------------

// The general path's workspace over T tokens: the routing kernel's exp
// values [T][E], then per (token, slot) the gate and up outputs [T k][I],
// h's q8 blocks [T k][I/32] and the down outputs [T k][H].  base null: the
// layout only.
struct WideWs {
  float* ebuf;
  float* g;
  float* u;
  ActBlock* hact;
  float* y;
  size_t total;
};

static WideWs wide_layout(const hale_moe* m, size_t T, char* base) {
  WideWs w{};
  const size_t A = T * m->k;
  size_t o = 0;
  auto take = [&](size_t bytes) -> char* {
    const size_t at = o;
    o += align_up(bytes, 256);
    return base ? base + at : nullptr;
  };
  w.ebuf = (float*)take(T * m->E * 4);
  w.g = (float*)take(A * m->I * 4);
  w.u = (float*)take(A * m->I * 4);
  w.hact = (ActBlock*)take(A * (m->I / HALE_QK) * sizeof(ActBlock));
  w.y = (float*)take(A * m->H * 4);
  w.total = o;
  return w;
}

// MoeLayer::forward over ntok tokens for any E, top_k, H and I: the router
// logits by the f32 GEMV (dot_f32's lane order), the routes by the general
// routing kernel, then per (token, slot) the gate and up matvecs, h =
// silu(g) * u requantized, the down matvec (lane-per-row chains, the
// expert read from the route on the device) and the route-order combine.
// Every step has the reference's arithmetic, so the outputs are its bits.
static int moe_wide_enqueue(hale_moe* m, size_t ntok, const float* dx, const float* dlogits,
                            float* dout, const TokScratch& s, void* ws) {
  hale_ctx* c = m->ctx;
  const size_t E = m->E, H = m->H, I = m->I, k = m->k, nbh = H / HALE_QK, nbi = I / HALE_QK;
  const WideWs w = wide_layout(m, ntok, (char*)ws);
  const float* lg = dlogits;
  if (!lg) {
    for (size_t t = 0; t < ntok; t++)
      LAUNCH(c, K_ROUTE, launch_gemv_float(HALE_F32, m->router, dx + t * H, E, H, s.logits + t * E, c->stream));
    lg = s.logits;
  }
  LAUNCH(c, K_ROUTE, launch_route_select_wide(lg, (int)E, (int)k, m->normalize, (int)ntok, w.ebuf,
                                              s.route_idx, s.route_w, m->stats, c->stream));
  LAUNCH(c, K_ACT_QUANT, launch_act_quant(dx, ntok * nbh, s.act, c->stream));
  const size_t tc = std::max<size_t>(1, 65535 / k);  // tokens per pass: grid rows (token, slot)
  for (size_t t0 = 0; t0 < ntok; t0 += tc) {
    const size_t nt = std::min(tc, ntok - t0), A0 = t0 * k, ny = nt * k;
    RowsArgs r{};
    r.route = s.route_idx + A0;
    r.nb = (int)nbh;
    r.rows = (int)I;
    r.act = s.act + t0 * nbh;
    r.act_div = (int)k;
    r.out_stride = I;
    r.codes_stride = m->gc_bytes;
    r.scales_stride = m->gs_elems;
    r.codes = m->gate_c;
    r.scales = m->gate_s;
    r.out = w.g + A0 * I;
    LAUNCH(c, K_GATE_UP, launch_matvec_rows(m->dtype, r, (int)ny, c->stream));
    r.codes = m->up_c;
    r.scales = m->up_s;
    r.out = w.u + A0 * I;
    LAUNCH(c, K_GATE_UP, launch_matvec_rows(m->dtype, r, (int)ny, c->stream));
    LAUNCH(c, K_GATE_UP, launch_swiglu_quant(w.g + A0 * I, w.u + A0 * I, ny * nbi, w.hact + A0 * nbi, c->stream));
    RowsArgs d{};
    d.codes = m->down_c;
    d.scales = m->down_s;
    d.codes_stride = m->dc_bytes;
    d.scales_stride = m->ds_elems;
    d.route = s.route_idx + A0;
    d.nb = (int)nbi;
    d.rows = (int)H;
    d.act = w.hact + A0 * nbi;
    d.act_div = 1;
    d.out = w.y + A0 * H;
    d.out_stride = H;
    LAUNCH(c, K_DOWN, launch_matvec_rows(m->dtype, d, (int)ny, c->stream));
    LAUNCH(c, K_COMBINE, launch_combine_rows(w.y + A0 * H, s.route_w + A0, (int)k, (int)H, (int)nt,
                                             dout + t0 * H, c->stream));
  }
  return HALE_OK;
}

// Checks that apply to every forward: device x 16-byte aligned (the router
// reads it as float4) and device logits float-aligned (host buffers are
// staged, dx NULL), a pending pack load, every expert present, a router or
// logits.
static int moe_forward_check(hale_moe* m, const float* dx, const float* logits) {
  if (dx && (uintptr_t)dx % 16) return fail(m->ctx, HALE_EINVAL, "moe_forward: x must be 16-byte aligned");
  if (dx && (uintptr_t)logits % 4)
    return fail(m->ctx, HALE_EINVAL, "moe_forward: logits must be 4-byte aligned");
  int rc = moe_wait_load(m);
  if (rc) return rc;
  rc = check_all_present(m);
  if (rc) return rc;
  if (!m->router && !logits) return fail(m->ctx, HALE_EINVAL, "layer has no router: logits are required");
  return HALE_OK;
}

// Enqueues MoeLayer::forward over ntok tokens with the given per-token
// scratch and (ntok >= grouped_min) grouped workspace.  top_k = 0
// routes nowhere: the reference's forward leaves out at zero.
static int moe_forward_enqueue(hale_moe* m, size_t ntok, const float* dx, const float* dlogits,
                               float* dout, const TokScratch& s, void* pws) {
  hale_ctx* c = m->ctx;
  if (m->k == 0) {
    LAUNCH(c, K_FILL, launch_fill(dout, ntok * m->H, 0.0f, c->stream));
    return HALE_OK;
  }
  if (m->wide) return moe_wide_enqueue(m, ntok, dx, dlogits, dout, s, pws);
  if (ntok >= m->grouped_min) {
    PrefillLayer L = prefill_layer(m, s);
    hipError_t e = prefill_enqueue(L, pws, ntok, dx, dlogits, dout, c->stream, ctx_hook(c));
    if (e != hipSuccess) return fail(c, HALE_EHIP, "grouped prefill: %s", hipGetErrorString(e));
    return HALE_OK;
  }
  return moe_decode_enqueue(m, ntok, dx, dlogits, dout, s);
}

// Scratch and workspace of a forward from the layer's own (growing) buffers.
static int moe_forward_scratch(hale_moe* m, size_t ntok, TokScratch* s, void** pws) {
  int rc = moe_reserve(m, ntok, s);
  if (rc) return rc;
  *pws = nullptr;
  if (m->k > 0 && m->wide) return moe_ws(m, wide_layout(m, ntok, nullptr).total, pws);
  if (m->k > 0 && ntok >= m->grouped_min) {
    PrefillLayer L = prefill_layer(m, *s);
    rc = moe_ws(m, prefill_workspace_bytes(L, ntok), pws);
  }
  return rc;
}

extern "C" int hale_moe_forward_device(hale_moe* m, size_t ntok, const float* d_x,
                                       const float* d_logits, float* d_out, uint32_t* d_index,
                                       float* d_weight) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !d_x || !d_out) return fail(c, HALE_EINVAL, "moe_forward: NULL argument");
  if (ntok == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_forward_check(m, d_x, d_logits);
  if (rc) return rc;
  TokScratch s;
  void* pws;
  rc = moe_forward_scratch(m, ntok, &s, &pws);
  if (rc) return rc;
  rc = moe_forward_enqueue(m, ntok, d_x, d_logits, d_out, s, pws);
  if (rc) return rc;
  if (d_index && m->k)
    HIPCHK(c, hipMemcpyAsync(d_index, s.route_idx, ntok * m->k * 4, hipMemcpyDeviceToDevice, c->stream));
  if (d_weight && m->k)
    HIPCHK(c, hipMemcpyAsync(d_weight, s.route_w, ntok * m->k * 4, hipMemcpyDeviceToDevice, c->stream));
  return HALE_OK;
}

// Keeps the per-kernel profiler off for the duration of a call (its event
// brackets create HIP events).
struct ProfPause {
  hale_ctx* c;
  bool was;
  explicit ProfPause(hale_ctx* ctx) : c(ctx), was(ctx->prof_on) { c->prof_on = false; }
  ~ProfPause() { c->prof_on = was; }
};

// Bytes of the fixed scratch a no-allocation forward over n tokens uses:
// the per-token scratch, then (grouped path) the grouped workspace.
static size_t noalloc_bytes(hale_moe* m, size_t n) {
  const size_t tb = align_up(tok_scratch_bytes(m, n), 256);
  if (m->k > 0 && m->wide) return tb + wide_layout(m, n, nullptr).total;
  if (m->k == 0 || n < m->grouped_min) return tb;
  return tb + prefill_workspace_bytes(prefill_layer(m, TokScratch{}), n);
}

// Tokens per chunk of a no-allocation forward over ntok tokens: all of them
// when they fit the fixed scratch; else the most that fit on the grouped
// path, if its threshold fits; else decode passes below the threshold.
// Each size's bytes grow with the token count, so a bisection finds the
// largest.  0: not even one token fits.
static size_t noalloc_chunk(hale_moe* m, size_t ntok) {
  const size_t cap = HALE_NOALLOC_SCRATCH_BYTES;
  if (noalloc_bytes(m, ntok) <= cap) return ntok;
  size_t lo, hi;  // noalloc_bytes(lo) fits (or lo == 0), noalloc_bytes(hi) does not
  const size_t gmin = std::max<size_t>(m->grouped_min, 1);
  if (m->k > 0 && ntok >= gmin && noalloc_bytes(m, gmin) <= cap) {
    lo = gmin;
    hi = ntok;
  } else {
    lo = 0;
    hi = std::min(ntok, gmin);  // decode passes of fewer than gmin tokens
    if (hi < ntok && noalloc_bytes(m, hi) <= cap) return hi;
  }
  while (hi - lo > 1) {
    const size_t mid = lo + (hi - lo) / 2;
    if (noalloc_bytes(m, mid) <= cap) lo = mid;
    else hi = mid;
  }
  return lo;
}

extern "C" int hale_moe_forward_device_noalloc(hale_moe* m, size_t ntok, const float* d_x,
                                               const float* d_logits, float* d_out,
                                               uint32_t* d_index, float* d_weight) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !d_x || !d_out) return fail(c, HALE_EINVAL, "moe_forward_noalloc: NULL argument");
  if (ntok == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  if (!c->fixed_scratch) return fail(c, HALE_EHIP, "no fixed scratch on device %d", c->device);
  int rc = moe_forward_check(m, d_x, d_logits);
  if (rc) return rc;
  const size_t chunk = noalloc_chunk(m, ntok);
  if (chunk == 0)
    return fail(c, HALE_EINVAL,
                "moe_forward_noalloc: one token needs %zu bytes of scratch, the fixed scratch "
                "holds %zu",
                noalloc_bytes(m, 1), (size_t)HALE_NOALLOC_SCRATCH_BYTES);
  char* base = (char*)c->fixed_scratch;
  const size_t k = m->k;
  ProfPause pause(c);
  // Chunks run one after another on the stream, each reusing the array from
  // its start.  Tokens are independent, so a chunk boundary changes no bits;
  // a last chunk below the grouped threshold takes the decode path, which
  // gives the same bits as the grouped one.
  for (size_t t0 = 0; t0 < ntok; t0 += chunk) {
    const size_t n = std::min(chunk, ntok - t0);
    const size_t tb = align_up(tok_scratch_bytes(m, n), 256);
    const TokScratch s = tok_scratch_carve(m, base, n);
    const bool ws = k > 0 && (m->wide || n >= m->grouped_min);
    rc = moe_forward_enqueue(m, n, d_x + t0 * m->H, d_logits ? d_logits + t0 * m->E : nullptr,
                             d_out + t0 * m->H, s, ws ? base + tb : nullptr);
    if (rc) return rc;
    if (d_index && k)
      HIPCHK(c, hipMemcpyAsync(d_index + t0 * k, s.route_idx, n * k * 4, hipMemcpyDeviceToDevice,
                               c->stream));
    if (d_weight && k)
      HIPCHK(c, hipMemcpyAsync(d_weight + t0 * k, s.route_w, n * k * 4, hipMemcpyDeviceToDevice,
                               c->stream));
  }
  return HALE_OK;
}

extern "C" int hale_moe_forward(hale_moe* m, size_t ntok, const float* x, const float* logits,
                                float* out, uint32_t* index, float* weight) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !x || !out) return fail(c, HALE_EINVAL, "moe_forward: NULL argument");
  if (ntok == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_forward_check(m, nullptr, logits);
  if (rc) return rc;
  size_t xb = ntok * m->H * 4, lb = logits ? ntok * m->E * 4 : 0;
  size_t o1 = align_up(xb, 256), o2 = o1 + align_up(xb, 256);
  void* sp;
  rc = ctx_scratch(c, o2 + lb, &sp);
  if (rc) return rc;
  float* dx = (float*)sp;
  float* dout = (float*)((char*)sp + o1);
  float* dl = logits ? (float*)((char*)sp + o2) : nullptr;
  TokScratch s;
  void* pws;
  rc = moe_forward_scratch(m, ntok, &s, &pws);
  if (rc) return rc;
  HostStage st(c);
  const size_t rb = align_up(ntok * m->k * 4, 256);
  if ((rc = st.reserve(2 * align_up(xb, 256) + align_up(lb, 256) + 2 * rb))) return rc;
  if ((rc = st.in(dx, x, xb))) return rc;
  if (logits && (rc = st.in(dl, logits, lb))) return rc;
  rc = moe_forward_enqueue(m, ntok, dx, dl, dout, s, pws);
  if (rc || (rc = st.out(out, dout, xb))) return rc;
  if (index && m->k && (rc = st.out(index, s.route_idx, ntok * m->k * 4))) return rc;
  if (weight && m->k && (rc = st.out(weight, s.route_w, ntok * m->k * 4))) return rc;
  return st.finish();
}

extern "C" int hale_moe_route(hale_moe* m, const float* x, uint32_t* index, float* weight) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !x || !index || !weight) return fail(c, HALE_EINVAL, "moe_route: NULL argument");
  if (!m->router) return fail(c, HALE_EINVAL, "layer has no router matrix");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  if (m->k == 0) return HALE_OK;  // top_k of nothing: no routes
  TokScratch s;
  int rc = moe_reserve(m, 1, &s);
  if (rc) return rc;
  void* sp;
  rc = ctx_scratch(c, align_up(m->H * 4, 256) + (m->wide ? m->E * 4 : 0), &sp);
  if (rc) return rc;
  HostStage st(c);
  if ((rc = st.reserve(align_up(m->H * 4, 256) + 2 * align_up(m->k * 4, 256))) ||
      (rc = st.in(sp, x, m->H * 4)))
    return rc;
  if (m->wide) {  // the general path's routing, its exp values after x
    float* ebuf = (float*)((char*)sp + align_up(m->H * 4, 256));
    LAUNCH(c, K_ROUTE, launch_gemv_float(HALE_F32, m->router, (const float*)sp, m->E, m->H, s.logits, c->stream));
    LAUNCH(c, K_ROUTE, launch_route_select_wide(s.logits, (int)m->E, (int)m->k, m->normalize, 1, ebuf,
                                                s.route_idx, s.route_w, nullptr, c->stream));
  } else {
    LAUNCH(c, K_ROUTE, launch_route_logits(m->router, (const float*)sp, (int)m->H, (int)m->E, 1,
                                           s.act, s.logits, c->stream));
    LAUNCH(c, K_ROUTE, launch_route_select(s.logits, (int)m->E, (int)m->k, m->normalize, 1,
                                           s.route_idx, s.route_w, nullptr, c->stream));
  }
  if ((rc = st.out(index, s.route_idx, m->k * 4)) || (rc = st.out(weight, s.route_w, m->k * 4))) return rc;
  return st.finish();
}

extern "C" int hale_moe_reserve(hale_moe* m, size_t max_tokens) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m) return fail(c, HALE_EINVAL, "moe_reserve: NULL layer");
  if (max_tokens == 0) return HALE_OK;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  TokScratch s;
  void* pws;
  return moe_forward_scratch(m, max_tokens, &s, &pws);  // the largest call's scratch
}

extern "C" int hale_moe_set_grouped_min_tokens(hale_moe* m, size_t n) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m) return fail(c, HALE_EINVAL, "set_grouped_min_tokens: NULL layer");
  if (n < 2 || n > HALE_DECODE_MAX_TOKENS + 1)
    return fail(c, HALE_EINVAL, "set_grouped_min_tokens: %zu is outside 2..%d", n,
                HALE_DECODE_MAX_TOKENS + 1);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  if (m->wide) return HALE_OK;  // the general path has no grouped form
  m->grouped_min = n;  // the next forward lays the scratch out for it
  return HALE_OK;
}

extern "C" int hale_moe_grouped_min_tokens(const hale_moe* m, size_t* n) {
  if (!m || !n) return fail(m ? m->ctx : nullptr, HALE_EINVAL, "grouped_min_tokens: NULL argument");
  *n = m->grouped_min;
  return HALE_OK;
}

extern "C" int hale_moe_set_band_max_tokens(hale_moe* m, size_t n) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m) return fail(c, HALE_EINVAL, "set_band_max_tokens: NULL layer");
  if (n > (size_t)INT32_MAX / 64)
    return fail(c, HALE_EINVAL, "set_band_max_tokens: %zu is above %d", n, INT32_MAX / 64);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  m->band_max = n;  // the next grouped forward sizes its workspace for it
  return HALE_OK;
}

extern "C" int hale_moe_band_max_tokens(const hale_moe* m, size_t* n) {
  if (!m || !n) return fail(m ? m->ctx : nullptr, HALE_EINVAL, "band_max_tokens: NULL argument");
  *n = m->band_max;
  return HALE_OK;
}

extern "C" int hale_moe_set_down_fold(hale_moe* m, int fold) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m) return fail(c, HALE_EINVAL, "set_down_fold: NULL layer");
  if (fold != HALE_FOLD_EXACT && fold != HALE_FOLD_FMA)
    return fail(c, HALE_EINVAL, "set_down_fold: unknown fold %d", fold);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  m->down_fold = fold;
  return HALE_OK;
}

extern "C" int hale_moe_routing_counts(hale_moe* m, uint64_t* counts) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !counts) return fail(c, HALE_EINVAL, "routing_counts: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(counts, m->stats, m->E * 8, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  for (size_t e = 0; e < m->E; e++) counts[e] += m->fetch_counts[e];
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// the provider surface: ExpertProvider::{fetch, stats, routing_stats}
// ---------------------------------------------------------------------------

extern "C" int hale_moe_expert_present(hale_moe* m, uint32_t expert, int* present) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !present) return fail(c, HALE_EINVAL, "expert_present: NULL argument");
  if (expert >= m->E) return fail(c, HALE_EINVAL, "expert %u of %zu", expert, m->E);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_wait_load(m);
  if (rc) return rc;
  *present = m->present[expert] ? 1 : 0;
  return HALE_OK;
}

// The layer's view of expert e's three matrices (made on first use).
static hale_matrix* expert_view(hale_moe* m, uint32_t e, int which) {
  hale_matrix*& v = m->views[3 * (size_t)e + which];
  if (v) return v;
  v = new (std::nothrow) hale_matrix;
  if (!v) return nullptr;
  v->ctx = m->ctx;
  v->dtype = m->dtype;
  v->view = true;
  if (which < 2) {
    v->rows = m->I;
    v->cols = m->H;
    v->codes = (which == 0 ? m->gate_c : m->up_c) + e * m->gc_bytes;
    v->scales = (which == 0 ? m->gate_s : m->up_s) + e * m->gs_elems;
  } else {
    v->rows = m->H;
    v->cols = m->I;
    v->codes = m->down_c + e * m->dc_bytes;
    v->scales = m->down_s + e * m->ds_elems;
  }
  return v;
}

// ExpertSource::load for a pack (one positioned read of the record), then
// the upload into the layer's planes.
static int load_from_source(hale_moe* m, uint32_t e) {
  hale_pack* p = m->source;
  const hale::PackHeader& h = p->h;
  uint64_t off = 0;
  std::string err;
  if (!hale::pack_offset_of(h, m->layer, e, &off, &err)) return fail(m->ctx, HALE_EPACK, "%s", err.c_str());
  std::vector<uint8_t> rec(h.record_bytes);
  if (!hale::pack_pread(p, rec.data(), rec.size(), off, &err)) return fail(m->ctx, HALE_EIO, "%s", err.c_str());
  const size_t ng = m->I * (size_t)hale_row_bytes(m->dtype, m->H);
  const size_t nd = m->H * (size_t)hale_row_bytes(m->dtype, m->I);
  return set_expert(m, e, rec.data(), rec.data() + ng, rec.data() + 2 * ng, ng, nd, false);
}

extern "C" int hale_moe_fetch(hale_moe* m, const uint32_t* experts, size_t n,
                              const hale_matrix** gate, const hale_matrix** up,
                              const hale_matrix** down) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || (n && !experts)) return fail(c, HALE_EINVAL, "fetch: NULL argument");
  for (size_t i = 0; i < n; i++)
    if (experts[i] >= m->E) return fail(c, HALE_EINVAL, "fetch: expert %u of %zu", experts[i], m->E);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_wait_load(m);
  if (rc) return rc;
  for (size_t i = 0; i < n; i++) m->fetch_counts[experts[i]]++;  // routing.record, before any load
  // pass 1: hits; pass 2: misses from the source, timed as one load
  uint64_t hits = 0;
  std::vector<uint32_t> missing;
  for (size_t i = 0; i < n; i++) {
    const uint32_t e = experts[i];
    if (m->present[e])
      hits++;
    else if (std::find(missing.begin(), missing.end(), e) == missing.end())
      missing.push_back(e);
  }
  if (!missing.empty() && !m->source)
    return fail(c, HALE_ENOTFOUND, "expert L%uE%u is not resident and the layer has no source",
                m->layer, missing[0]);
  // a key missing twice in one request is loaded once and counted as two
  // misses, as the reference counts every request its first pass missed
  const auto t0 = std::chrono::steady_clock::now();
  for (uint32_t e : missing) {
    rc = load_from_source(m, e);
    if (rc) return rc;
  }
  const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  const uint64_t nmiss = n - hits;
  m->fetch_hits += hits;
  m->misses += nmiss;
  if (nmiss) {
    m->bytes_loaded += nmiss * (uint64_t)m->source->h.record_bytes;
    m->load_seconds += dt;
  }
  for (size_t i = 0; i < n; i++) {
    const hale_matrix* v[3];
    for (int w = 0; w < 3; w++)
      if (!(v[w] = expert_view(m, experts[i], w))) return fail(c, HALE_ENOMEM, "out of host memory");
    if (gate) gate[i] = v[0];
    if (up) up[i] = v[1];
    if (down) down[i] = v[2];
  }
  return HALE_OK;
}

extern "C" int hale_moe_cache_stats(hale_moe* m, hale_cache_stats* out) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !out) return fail(c, HALE_EINVAL, "cache_stats: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_wait_load(m);
  if (rc) return rc;
  std::vector<uint64_t> sel(m->E);
  HIPCHK(c, hipMemcpyAsync(sel.data(), m->stats, m->E * 8, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  uint64_t forward_sel = 0;
  for (uint64_t v : sel) forward_sel += v;
  size_t resident = 0;
  for (char p : m->present) resident += p ? 1 : 0;
  const size_t eb = 2 * m->I * (size_t)hale_row_bytes(m->dtype, m->H) +
                    m->H * (size_t)hale_row_bytes(m->dtype, m->I);
  *out = hale_cache_stats{};
  out->pinned_hits = m->fetch_hits + forward_sel;
  out->misses = m->misses;
  out->bytes_loaded = m->bytes_loaded;
  out->load_seconds = m->load_seconds;
  out->pinned_experts = resident;
  out->pinned_bytes = resident * eb;
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// bulk expert registration
// ---------------------------------------------------------------------------

extern "C" int hale_moe_set_experts_device(hale_moe* m, uint32_t first, uint32_t count,
                                           const void* d_gate, const void* d_up,
                                           const void* d_down) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !d_gate || !d_up || !d_down) return fail(c, HALE_EINVAL, "set_experts: NULL argument");
  if ((size_t)first + count > m->E) return fail(c, HALE_EINVAL, "experts %u..%u of %zu", first, first + count, m->E);
  size_t ng = m->I * (size_t)hale_row_bytes(m->dtype, m->H);
  size_t nd = m->H * (size_t)hale_row_bytes(m->dtype, m->I);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = moe_wait_load(m);
  if (rc) return rc;
  for (uint32_t i = 0; i < count; i++) {
    size_t e = first + i;
    LAUNCH(c, K_REPACK, launch_repack(m->dtype, (const uint8_t*)d_gate + i * ng, m->I, m->H,
                                      m->gate_c + e * m->gc_bytes, m->gate_s + e * m->gs_elems, c->stream));
    LAUNCH(c, K_REPACK, launch_repack(m->dtype, (const uint8_t*)d_up + i * ng, m->I, m->H,
                                      m->up_c + e * m->gc_bytes, m->up_s + e * m->gs_elems, c->stream));
    LAUNCH(c, K_REPACK, launch_repack(m->dtype, (const uint8_t*)d_down + i * nd, m->H, m->I,
                                      m->down_c + e * m->dc_bytes, m->down_s + e * m->ds_elems, c->stream));
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  for (uint32_t i = 0; i < count; i++) m->present[first + i] = 1;
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// expert pack -> HBM (the file tier under the resident tier)
// ---------------------------------------------------------------------------

// Loader thread of one layer: the layer's records are contiguous in the
// file, so each batch is one positioned read into a pinned slot, one copy to
// the matching device slot and a repack per matrix, on the pack's stream.
// A slot is refilled only after its previous copy has finished.
static void pack_loader(hale_pack* p, hale_moe* m, hale::PackLoad* L, uint64_t off0, size_t batch) {
  const size_t stride = p->h.record_stride, rbytes = p->h.record_bytes;
  const size_t proj = m->I * (size_t)hale_row_bytes(m->dtype, m->H);
  auto hip = [&](hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    L->rc = HALE_EHIP;
    L->err = std::string("pack load: ") + what + ": " + hipGetErrorString(e);
    return false;
  };
  if (!hip(hipSetDevice(p->device), "hipSetDevice")) return;
  const auto t0 = std::chrono::steady_clock::now();
  for (size_t e0 = 0, it = 0; e0 < m->E; e0 += batch, it++) {
    const int s = (int)(it & 1);
    const size_t n = std::min(batch, m->E - e0);
    const size_t bytes = (n - 1) * stride + rbytes;
    if (!hip(hipEventSynchronize(p->copied[s]), "hipEventSynchronize")) return;
    std::string err;
    if (!hale::pack_pread(p, p->pinned[s], bytes, off0 + e0 * stride, &err)) {
      L->rc = HALE_EIO;
      L->err = err;
      return;
    }
    if (!hip(hipMemcpyAsync(p->dstage[s], p->pinned[s], bytes, hipMemcpyHostToDevice, p->stream),
             "upload"))
      return;
    if (!hip(hipEventRecord(p->copied[s], p->stream), "hipEventRecord")) return;
    for (size_t i = 0; i < n; i++) {
      const size_t e = e0 + i;
      const uint8_t* rec = (const uint8_t*)p->dstage[s] + i * stride;
      hipError_t r = launch_repack(m->dtype, rec, m->I, m->H, m->gate_c + e * m->gc_bytes,
                                   m->gate_s + e * m->gs_elems, p->stream);
      if (r == hipSuccess)
        r = launch_repack(m->dtype, rec + proj, m->I, m->H, m->up_c + e * m->gc_bytes,
                          m->up_s + e * m->gs_elems, p->stream);
      if (r == hipSuccess)
        r = launch_repack(m->dtype, rec + 2 * proj, m->H, m->I, m->down_c + e * m->dc_bytes,
                          m->down_s + e * m->ds_elems, p->stream);
      if (!hip(r, "repack")) return;
    }
  }
  if (!hip(hipEventRecord(m->loaded, p->stream), "hipEventRecord")) return;
  // the load's wall-clock time ends with its last repack on the device
  if (!hip(hipEventSynchronize(m->loaded), "hipEventSynchronize")) return;
  L->bytes = (uint64_t)m->E * rbytes;
  L->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

static void pack_free_staging(hale_pack* p) {
  for (int s = 0; s < 2; s++) {
    if (p->pinned[s]) (void)hipHostFree(p->pinned[s]);
    if (p->dstage[s]) (void)hipFree(p->dstage[s]);
    p->pinned[s] = p->dstage[s] = nullptr;
  }
  p->slot_bytes = 0;
}

// Checks that pack p can serve layer m (same dtype, shapes and record size,
// the layer present in the pack) and gives the layer's first record offset.
static int pack_check_layer(hale_moe* m, hale_pack* p, uint64_t* off0) {
  hale_ctx* c = m->ctx;
  if (p->ctx && p->ctx != c)
    return fail(c, HALE_EINVAL, "the pack already loads into another context's layers");
  const hale::PackHeader& h = p->h;
  if (h.dtype != m->dtype || h.hidden != m->H || h.inter != m->I || h.num_experts != m->E)
    return fail(c, HALE_EINVAL,
                "pack (dtype %d, hidden %zu, inter %zu, %zu experts) does not match the layer "
                "(dtype %d, hidden %zu, inter %zu, %zu experts)",
                h.dtype, h.hidden, h.inter, h.num_experts, m->dtype, m->H, m->I, m->E);
  const size_t need = 2 * m->I * (size_t)hale_row_bytes(m->dtype, m->H) +
                      m->H * (size_t)hale_row_bytes(m->dtype, m->I);
  if (h.record_bytes != need)
    return fail(c, HALE_EPACK, "record is %zu bytes, expected %zu", h.record_bytes, need);
  std::string err;
  if (!hale::pack_offset_of(h, m->layer, 0, off0, &err)) return fail(c, HALE_EPACK, "%s", err.c_str());
  return HALE_OK;
}

// Binds pack p to context c's device (its stream and events) on first use,
// and makes it layer m's source.  Caller holds c->mu.
static int pack_bind(hale_moe* m, hale_pack* p) {
  hale_ctx* c = m->ctx;
  if (!p->ctx) {
    HIPCHK(c, hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking));
    for (int s = 0; s < 2; s++) HIPCHK(c, hipEventCreateWithFlags(&p->copied[s], hipEventDisableTiming));
    p->ctx = c;
    p->device = c->device;
  }
  if (m->source != p) {
    if (m->source) {
      auto& ls = m->source->layers;
      ls.erase(std::remove(ls.begin(), ls.end(), m), ls.end());
    }
    p->layers.push_back(m);
    m->source = p;
  }
  return HALE_OK;
}

extern "C" int hale_moe_set_source(hale_moe* m, hale_pack* p) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m) return fail(c, HALE_EINVAL, "set_source: NULL layer");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  if (!p) {
    if (m->source) {
      auto& ls = m->source->layers;
      ls.erase(std::remove(ls.begin(), ls.end(), m), ls.end());
      m->source = nullptr;
    }
    return HALE_OK;
  }
  uint64_t off0 = 0;
  int rc = pack_check_layer(m, p, &off0);
  if (rc) return rc;
  return pack_bind(m, p);
}

extern "C" int hale_moe_prefetch_pack(hale_moe* m, hale_pack* p) {
  hale_ctx* c = m ? m->ctx : nullptr;
  if (!m || !p) return fail(c, HALE_EINVAL, "prefetch_pack: NULL argument");
  uint64_t off0 = 0;
  int rc = pack_check_layer(m, p, &off0);
  if (rc) return rc;
  const hale::PackHeader& h = p->h;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  rc = pack_bind(m, p);
  if (rc) return rc;
  rc = moe_wait_load(m);  // this layer's previous load
  if (rc) return rc;
  if (p->load) p->load->join();  // the pack's previous load (its layer keeps the result)
  // batches of about 64 MiB of records
  const size_t batch = std::max<size_t>(1, std::min<size_t>(m->E, (size_t(64) << 20) / h.record_stride));
  const size_t slot = batch * h.record_stride;
  if (p->slot_bytes < slot) {
    HIPCHK(c, hipStreamSynchronize(p->stream));
    pack_free_staging(p);
    for (int s = 0; s < 2; s++)
      if (hipHostMalloc(&p->pinned[s], slot, hipHostMallocDefault) != hipSuccess ||
          hipMalloc(&p->dstage[s], slot) != hipSuccess) {
        pack_free_staging(p);
        return fail(c, HALE_ENOMEM, "pack staging: 2 x %zu bytes", slot);
      }
    p->slot_bytes = slot;
  }
  if (!m->loaded) HIPCHK(c, hipEventCreateWithFlags(&m->loaded, hipEventDisableTiming));
  auto L = std::make_shared<hale::PackLoad>();
  try {
    L->th = std::thread(pack_loader, p, m, L.get(), off0, batch);
  } catch (...) {
    return fail(c, HALE_ENOMEM, "cannot start the pack loader thread");
  }
  p->load = L;
  m->load = L;
  return HALE_OK;
}

extern "C" int hale_moe_load_pack(hale_moe* m, hale_pack* p) {
  int rc = hale_moe_prefetch_pack(m, p);
  if (rc) return rc;
  hale_ctx* c = m->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  rc = moe_wait_load(m);
  if (rc) return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

extern "C" void hale_pack_close(hale_pack* p) {
  if (!p) return;
  if (hale_ctx* c = p->ctx) {
    std::lock_guard<std::recursive_mutex> g(c->mu);
    for (hale_moe* m : p->layers) m->source = nullptr;
    if (p->load) p->load->join();
    p->load.reset();
    (void)hipSetDevice(p->device);
    (void)hipStreamSynchronize(p->stream);
    pack_free_staging(p);
    for (int s = 0; s < 2; s++)
      if (p->copied[s]) (void)hipEventDestroy(p->copied[s]);
    (void)hipStreamDestroy(p->stream);
  }
  if (p->fd >= 0) ::close(p->fd);
  delete p;
}

// ---------------------------------------------------------------------------
// RMSNorm and attention (the steps on either side of the MoE block)
// ---------------------------------------------------------------------------

extern "C" int hale_rms_norm_device(hale_ctx* c, float* d_x, const float* d_delta,
                                    const float* d_weight, size_t rows, size_t n, float eps,
                                    float* d_out) {
  if (!c || !d_x || !d_weight || !d_out) return fail(c, HALE_EINVAL, "rms_norm: NULL argument");
  if (n == 0 || n > 8192) return fail(c, HALE_EINVAL, "rms_norm: length %zu outside 1..8192", n);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  LAUNCH(c, K_NORM, launch_rms_norm(d_x, d_delta, d_weight, rows, n, eps, d_out, c->stream));
  return HALE_OK;
}

extern "C" int hale_rms_norm(hale_ctx* c, const float* x, const float* weight, size_t n, float eps,
                             float* out) {
  if (!c || !x || !weight || !out) return fail(c, HALE_EINVAL, "rms_norm: NULL argument");
  if (n == 0 || n > 8192) return fail(c, HALE_EINVAL, "rms_norm: length %zu outside 1..8192", n);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  const size_t b = align_up(n * 4, 256);
  void* s;
  int rc = ctx_scratch(c, 3 * b, &s);
  if (rc) return rc;
  float* dx = (float*)s;
  float* dw = (float*)((char*)s + b);
  float* dout = (float*)((char*)s + 2 * b);
  HIPCHK(c, hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(dw, weight, n * 4, hipMemcpyHostToDevice, c->stream));
  LAUNCH(c, K_NORM, launch_rms_norm(dx, nullptr, dw, 1, n, eps, dout, c->stream));
  HIPCHK(c, hipMemcpyAsync(out, dout, n * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

struct hale_attention {
  hale_ctx* ctx = nullptr;
  const hale_matrix *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
  size_t H = 0, nh = 0, nkv = 0, hd = 0, max_len = 0, len = 0;
  float eps = 0.0f;
  float *q_norm = nullptr, *k_norm = nullptr;  // [hd] device copies, or null
  float *keys = nullptr, *values = nullptr;    // the layer cache, [max_len][nkv*hd]
  // per-call buffers: q, k, v, context, scores [nh][max_len], x/cos/sin/out
  // staging of the host entry point, q8 activation blocks
  float *dq = nullptr, *dk = nullptr, *dv = nullptr, *dctx = nullptr, *scores = nullptr;
  float *hx = nullptr, *hcos = nullptr, *hsin = nullptr, *hout = nullptr;
  ActBlock* act = nullptr;
};

extern "C" void hale_attention_destroy(hale_attention* a) {
  if (!a) return;
  hale_ctx* c = a->ctx;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (void* p : {(void*)a->q_norm, (void*)a->k_norm, (void*)a->keys, (void*)a->values, (void*)a->dq,
                  (void*)a->dk, (void*)a->dv, (void*)a->dctx, (void*)a->scores, (void*)a->hx,
                  (void*)a->hcos, (void*)a->hsin, (void*)a->hout, (void*)a->act})
    (void)hipFree(p);
  delete a;
}

extern "C" int hale_attention_create(hale_ctx* c, const hale_matrix* q, const hale_matrix* k,
                                     const hale_matrix* v, const hale_matrix* o,
                                     const float* q_norm, const float* k_norm, size_t num_heads,
                                     size_t num_kv_heads, size_t head_dim, float norm_eps,
                                     size_t max_len, hale_attention** out) {
  if (!c || !q || !k || !v || !o || !out) return fail(c, HALE_EINVAL, "attention_create: NULL argument");
  *out = nullptr;
  const size_t nh = num_heads, nkv = num_kv_heads, hd = head_dim, H = q->cols;
  if (nh == 0 || nkv == 0 || nh % nkv)
    return fail(c, HALE_EINVAL, "num_heads %zu must be a positive multiple of num_kv_heads %zu", nh, nkv);
  if (hd < 16 || hd > 1024 || hd % 16)
    return fail(c, HALE_EINVAL, "head_dim %zu must be a multiple of 16 in 16..1024", hd);
  if (nh / nkv > 16) return fail(c, HALE_EINVAL, "GQA group %zu above 16", nh / nkv);
  if (max_len == 0 || max_len > (1u << 24)) return fail(c, HALE_EINVAL, "max_len %zu outside 1..2^24", max_len);
  if (q->rows != nh * hd || k->rows != nkv * hd || v->rows != nkv * hd || k->cols != H ||
      v->cols != H || o->rows != H || o->cols != nh * hd)
    return fail(c, HALE_EINVAL, "projection shapes do not match %zu heads x %zu, %zu kv heads, hidden %zu",
                nh, hd, nkv, H);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  hale_attention* a = new (std::nothrow) hale_attention;
  if (!a) return fail(c, HALE_ENOMEM, "out of host memory");
  a->ctx = c;
  a->q = q;
  a->k = k;
  a->v = v;
  a->o = o;
  a->H = H;
  a->nh = nh;
  a->nkv = nkv;
  a->hd = hd;
  a->eps = norm_eps;
  a->max_len = max_len;
  const size_t kv_dim = nkv * hd, wide = std::max(H, nh * hd);
  hipError_t e = hipSuccess;
#define ALLOC(p, n) \
  if (e == hipSuccess) e = hipMalloc(&(p), (n))
  if (q_norm) ALLOC(a->q_norm, hd * 4);
  if (k_norm) ALLOC(a->k_norm, hd * 4);
  ALLOC(a->keys, max_len * kv_dim * 4);
  ALLOC(a->values, max_len * kv_dim * 4);
  ALLOC(a->dq, nh * hd * 4);
  ALLOC(a->dk, kv_dim * 4);
  ALLOC(a->dv, kv_dim * 4);
  ALLOC(a->dctx, nh * hd * 4);
  ALLOC(a->scores, nh * ((max_len + 3) / 4 * 4) * 4);
  ALLOC(a->hx, H * 4);
  ALLOC(a->hcos, hd * 2);
  ALLOC(a->hsin, hd * 2);
  ALLOC(a->hout, H * 4);
  ALLOC(a->act, (wide / HALE_QK + 1) * sizeof(ActBlock));
#undef ALLOC
  if (e == hipSuccess && q_norm) e = hipMemcpyAsync(a->q_norm, q_norm, hd * 4, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess && k_norm) e = hipMemcpyAsync(a->k_norm, k_norm, hd * 4, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    hale_attention_destroy(a);
    return fail(c, HALE_ENOMEM, "attention allocation (%zu positions): %s", max_len, hipGetErrorString(e));
  }
  *out = a;
  return HALE_OK;
}

extern "C" int hale_attention_reset(hale_attention* a) {
  if (!a) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(a->ctx->mu);
  a->len = 0;
  return HALE_OK;
}

extern "C" int hale_attention_len(const hale_attention* a, size_t* len) {
  if (!a || !len) return HALE_EINVAL;
  *len = a->len;
  return HALE_OK;
}

extern "C" int hale_attention_forward_device(hale_attention* a, const float* d_x, size_t position,
                                             const float* d_cos, const float* d_sin, float* d_out) {
  hale_ctx* c = a ? a->ctx : nullptr;
  if (!a || !d_x || !d_cos || !d_sin || !d_out) return fail(c, HALE_EINVAL, "attention: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  if (position != a->len)
    return fail(c, HALE_EINVAL, "attention at position %zu, but the cache holds %zu positions", position, a->len);
  if (position >= a->max_len)
    return fail(c, HALE_EINVAL, "context overflow: %zu positions needed, the cache holds %zu",
                position + 1, a->max_len);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = matvec_enqueue(c, a->q, d_x, a->dq, a->act);
  if (!rc) rc = matvec_enqueue(c, a->k, d_x, a->dk, a->act);
  if (!rc) rc = matvec_enqueue(c, a->v, d_x, a->dv, a->act);
  if (rc) return rc;
  AttnArgs t{};
  t.q = a->dq;
  t.k = a->dk;
  t.v = a->dv;
  t.nh = (int)a->nh;
  t.nkv = (int)a->nkv;
  t.hd = (int)a->hd;
  t.q_norm = a->q_norm;
  t.k_norm = a->k_norm;
  t.eps = a->eps;
  t.cos = d_cos;
  t.sin = d_sin;
  t.keys = a->keys;
  t.values = a->values;
  t.seq = (int)position + 1;
  t.ld = (int)((a->max_len + 3) / 4 * 4);  // score rows 16-byte aligned
  t.scores = a->scores;
  t.ctx = a->dctx;
  LAUNCH(c, K_ATTENTION, launch_attention_core(t, c->stream));
  rc = matvec_enqueue(c, a->o, a->dctx, d_out, a->act);
  if (rc) return rc;
  a->len = position + 1;  // LayerCache::push
  return HALE_OK;
}

extern "C" int hale_attention_forward(hale_attention* a, const float* x, size_t position,
                                      const float* cos, const float* sin, float* out) {
  hale_ctx* c = a ? a->ctx : nullptr;
  if (!a || !x || !cos || !sin || !out) return fail(c, HALE_EINVAL, "attention: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  const size_t half = a->hd / 2;
  HIPCHK(c, hipMemcpyAsync(a->hx, x, a->H * 4, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(a->hcos, cos, half * 4, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipMemcpyAsync(a->hsin, sin, half * 4, hipMemcpyHostToDevice, c->stream));
  int rc = hale_attention_forward_device(a, a->hx, position, a->hcos, a->hsin, a->hout);
  if (rc) return rc;
  HIPCHK(c, hipMemcpyAsync(out, a->hout, a->H * 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

// ---------------------------------------------------------------------------
// support entry points
// ---------------------------------------------------------------------------

extern "C" int hale_device_malloc(hale_ctx* c, size_t bytes, void** out) {
  if (!c || !out) return fail(c, HALE_EINVAL, "device_malloc: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  *out = nullptr;
  if (hipMalloc(out, bytes ? bytes : 1) != hipSuccess) return fail(c, HALE_ENOMEM, "device allocation of %zu bytes", bytes);
  return HALE_OK;
}

extern "C" int hale_device_free(hale_ctx* c, void* p) {
  if (!c) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipFree(p));
  return HALE_OK;
}

extern "C" int hale_memcpy_htod(hale_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (n && (!dst || !src))) return fail(c, HALE_EINVAL, "memcpy: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

extern "C" int hale_memcpy_dtoh(hale_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (n && (!dst || !src))) return fail(c, HALE_EINVAL, "memcpy: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return HALE_OK;
}

extern "C" int hale_fill_normal_device(hale_ctx* c, uint64_t seed, float mean, float std,
                                       float* d_out, size_t n) {
  if (!c || (n && !d_out)) return fail(c, HALE_EINVAL, "fill_normal: NULL argument");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  LAUNCH(c, K_FILL, launch_fill_normal(d_out, n, seed, mean, std, c->stream));
  return HALE_OK;
}

extern "C" int hale_copy_device(hale_ctx* c, void* d_dst, const void* d_src, size_t n) {
  if (!c || (n && (!d_dst || !d_src))) return fail(c, HALE_EINVAL, "copy_device: NULL argument");
  if (n % 16 || (uintptr_t)d_dst % 16 || (uintptr_t)d_src % 16)
    return fail(c, HALE_EINVAL, "copy_device: size and addresses must be multiples of 16");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  LAUNCH(c, K_COPY, launch_copy(d_dst, d_src, n / 16, c->stream));
  return HALE_OK;
}

extern "C" int hale_stream_read_device(hale_ctx* c, const void* d_src, size_t n, unsigned workgroups,
                                       uint32_t* d_out) {
  if (!c || !d_out || (n && !d_src)) return fail(c, HALE_EINVAL, "stream_read_device: NULL argument");
  if (n % 16 || (uintptr_t)d_src % 16)
    return fail(c, HALE_EINVAL, "stream_read_device: size and address must be multiples of 16");
  if (workgroups < 1 || workgroups > 65535)
    return fail(c, HALE_EINVAL, "stream_read_device: %u work-groups outside 1..65535", workgroups);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  LAUNCH(c, K_STREAM_READ, launch_stream_read(d_src, n / 16, workgroups, d_out, c->stream));
  return HALE_OK;
}

extern "C" int hale_timer_start(hale_ctx* c) {
  if (!c) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  if (!c->t0) HIPCHK(c, hipEventCreate(&c->t0));
  if (!c->t1) HIPCHK(c, hipEventCreate(&c->t1));
  HIPCHK(c, hipEventRecord(c->t0, c->stream));
  return HALE_OK;
}

extern "C" int hale_timer_stop(hale_ctx* c, double* ms) {
  if (!c || !ms || !c->t0) return fail(c, HALE_EINVAL, "timer_stop without timer_start");
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipEventRecord(c->t1, c->stream));
  HIPCHK(c, hipEventSynchronize(c->t1));
  float f = 0.0f;
  HIPCHK(c, hipEventElapsedTime(&f, c->t0, c->t1));
  *ms = f;
  return HALE_OK;
}

extern "C" int hale_profile_enable(hale_ctx* c, int on) {
  if (!c) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  c->prof_on = on != 0;
  return HALE_OK;
}

static int prof_collect(hale_ctx* c) {
  if (c->recs.empty()) return HALE_OK;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  for (auto& r : c->recs) {
    float f = 0.0f;
    HIPCHK(c, hipEventElapsedTime(&f, r.start, r.stop));
    if (r.kind >= 0 && r.kind < K_KINDS) {
      c->prof_ms[r.kind] += f;
      c->prof_n[r.kind] += 1;
    }
    c->ev_pool.push_back(r.start);
    c->ev_pool.push_back(r.stop);
  }
  c->recs.clear();
  return HALE_OK;
}

extern "C" int hale_profile_read(hale_ctx* c, int kind, double* total_ms, uint64_t* launches) {
  if (!c || kind < 0 || kind >= K_KINDS) return fail(c, HALE_EINVAL, "profile_read: bad kind %d", kind);
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = prof_collect(c);
  if (rc) return rc;
  if (total_ms) *total_ms = c->prof_ms[kind];
  if (launches) *launches = c->prof_n[kind];
  return HALE_OK;
}

extern "C" int hale_profile_reset(hale_ctx* c) {
  if (!c) return HALE_EINVAL;
  std::lock_guard<std::recursive_mutex> g(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  int rc = prof_collect(c);
  if (rc) return rc;
  for (int k = 0; k < K_KINDS; k++) {
    c->prof_ms[k] = 0.0;
    c->prof_n[k] = 0;
  }
  return HALE_OK;
}

extern "C" int hale_kernel_kinds(void) { return K_KINDS; }

extern "C" const char* hale_kernel_name(int kind) {
  static const char* names[K_KINDS] = {"route", "gate_up", "down", "act_quant", "gemv", "encode",
                                       "repack", "fill", "group", "grouped_gate_up",
                                       "grouped_down", "combine", "copy", "rms_norm",
                                       "attention", "gather", "decode", "stream_read"};
  return kind >= 0 && kind < K_KINDS ? names[kind] : "";
}

extern "C" int hale_graph_begin(hale_ctx* c) {
  if (!c) return HALE_EINVAL;
  c->mu.lock();  // held until hale_graph_end: nothing else may enqueue meanwhile
  hipError_t e = hipSetDevice(c->device);
  if (e == hipSuccess) e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    c->mu.unlock();
    return fail(c, HALE_EHIP, "begin capture: %s", hipGetErrorString(e));
  }
  c->prof_saved = c->prof_on;  // profiler events are not captured into graphs
  c->prof_on = false;
  return HALE_OK;
}

extern "C" int hale_graph_end(hale_ctx* c, hale_graph** out) {
  if (!c || !out) return HALE_EINVAL;
  *out = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &graph);
  c->prof_on = c->prof_saved;
  c->mu.unlock();
  if (e != hipSuccess) return fail(c, HALE_EHIP, "end capture: %s", hipGetErrorString(e));
  hale_graph* g = new (std::nothrow) hale_graph;
  if (!g) {
    (void)hipGraphDestroy(graph);
    return fail(c, HALE_ENOMEM, "out of host memory");
  }
  g->ctx = c;
  g->graph = graph;
  e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(graph);
    delete g;
    return fail(c, HALE_EHIP, "instantiate: %s", hipGetErrorString(e));
  }
  std::lock_guard<std::recursive_mutex> lk(c->mu);
  // the exec's device-side resources are set up now, on the context's
  // stream, so its first launch costs what every other does
  e = hipSetDevice(c->device);
  if (e == hipSuccess) e = hipGraphUpload(g->exec, c->stream);
  if (e != hipSuccess) {
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(graph);
    delete g;
    return fail(c, HALE_EHIP, "graph upload: %s", hipGetErrorString(e));
  }
  c->live_graphs++;
  *out = g;
  return HALE_OK;
}

extern "C" int hale_graph_launch(hale_graph* g) {
  if (!g) return HALE_EINVAL;
  hale_ctx* c = g->ctx;
  std::lock_guard<std::recursive_mutex> lk(c->mu);
  HIPCHK(c, hipSetDevice(c->device));
  HIPCHK(c, hipGraphLaunch(g->exec, c->stream));
  return HALE_OK;
}

extern "C" void hale_graph_destroy(hale_graph* g) {
  if (!g) return;
  hale_ctx* c = g->ctx;
  std::lock_guard<std::recursive_mutex> lk(c->mu);
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  delete g;
  if (--c->live_graphs == 0) {  // no graph can use the retired scratch any more
    for (void* p : c->retired) (void)hipFree(p);
    c->retired.clear();
  }
}
