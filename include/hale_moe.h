/*
 * hale_moe.h -- C ABI of the MI355X (gfx950) quantized MoE expert path.
 *
 * This is the drop-in seam behind Hale-Token's Rust surface for the path:
 * WeightMatrix::matvec, Q8Activations::quantize, encode_row,
 * Expert::forward, MoeLayer::{route, forward} and the ExpertProvider trait.
 * Every declaration names the reference item it replaces (Hale-Token
 * file:line).  The ABI uses plain pointers, sizes and opaque handles only.
 *
 * Conventions
 *   - Every fallible call returns an int status (hale_status).  Nothing
 *     unwinds across the ABI.  The message of the last failure on a context
 *     is available from hale_last_error().  A Rust wrapper maps
 *     HALE_EINVAL to the reference's panics/asserts (length checks,
 *     `len % 32`, float dtype in dot_quantized) and everything else to
 *     HaleError.
 *   - Entry points without a `_device` suffix take HOST buffers and are
 *     synchronous, matching the Rust semantics (the result is in `out` when
 *     the call returns).  `_device` entry points take device pointers, are
 *     enqueued on the context's stream (hale_ctx_stream) and return at once.
 *   - Weight bytes are accepted in the reference's block layout
 *     (src/tensor/quant.rs:20-26: q8_0 = [f16 scale][32 x i8], 34 B;
 *     q4_0 = [f16 scale][16 B nibbles], 18 B, byte j = element j low nibble,
 *     element j+16 high nibble).  They are copied to HBM once and repacked
 *     into an aligned tile layout; the bytes read per matvec are unchanged.
 *   - A context serialises its own calls; distinct contexts may run
 *     concurrently.  All calls on one context share its stream.
 */
#ifndef HALE_MOE_H
#define HALE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Ref: HaleError (src/error.rs:11-60) and the panics listed
 * above. */
typedef enum {
  HALE_OK = 0,
  HALE_EINVAL = 1,   /* bad shape, dtype, length or argument            */
  HALE_EHIP = 2,     /* HIP runtime error (message in hale_last_error)  */
  HALE_ENOMEM = 3,   /* device or host allocation failed                */
  HALE_ENOTFOUND = 4, /* expert not registered (ExpertProvider::fetch)  */
  HALE_EIO = 5,       /* file I/O failed (HaleError::Io)                 */
  HALE_EPACK = 6      /* not a valid expert pack, or a key outside it
                         (HaleError::InvalidArgument / Json from
                         src/expert/pack.rs)                              */
} hale_status;

/* Element formats.  Ref: DType (src/tensor/dtype.rs:15-25), same order. */
typedef enum {
  HALE_F32 = 0,
  HALE_F16 = 1,
  HALE_BF16 = 2,
  HALE_Q8_0 = 3,
  HALE_Q4_0 = 4
} hale_dtype;

#define HALE_QK 32 /* Ref: QK (src/tensor/dtype.rs:28) */

typedef struct hale_ctx hale_ctx;       /* device + stream + scratch      */
typedef struct hale_matrix hale_matrix; /* Ref: WeightMatrix              */
typedef struct hale_moe hale_moe;       /* Ref: MoeLayer + its provider   */
typedef struct hale_pack hale_pack;     /* Ref: PackExpertSource          */

/* ---- context --------------------------------------------------------- */

/* Creates a context on HIP device `device` (one stream, default priority). */
int hale_ctx_create(int device, hale_ctx **out);
/* Destroys the context; matrices, layers, graphs and buffers created on it
 * must be destroyed first. */
void hale_ctx_destroy(hale_ctx *ctx);
/* Message of the last failed call on ctx ("" if none).  NULL ctx gives the
 * message of the last failed hale_ctx_create or hale_pack_* call in this
 * thread. */
const char *hale_last_error(const hale_ctx *ctx);
/* The hipStream_t the context enqueues on (for the _device entry points). */
void *hale_ctx_stream(hale_ctx *ctx);
int hale_ctx_synchronize(hale_ctx *ctx);

/* ---- geometry -------------------------------------------------------- */

/* Ref: DType::row_bytes (src/tensor/dtype.rs:53-61); -1 when cols is not a
 * multiple of the block length or dtype is unknown. */
long long hale_row_bytes(int dtype, size_t cols);
/* Ref: DType::block_bytes (src/tensor/dtype.rs:40-47); 0 if unknown. */
size_t hale_block_bytes(int dtype);

/* ---- weight matrices ------------------------------------------------- */

/* Ref: WeightMatrix::new (src/tensor/matrix.rs:19-47).  `bytes` holds
 * rows x row_bytes(cols) bytes in the reference layout (host memory), in
 * any dtype: Q8_0 / Q4_0 are repacked into the tile layout, F32 / F16 /
 * BF16 stay row-major as given (dense weights such as attention
 * projections, the lm_head, the router). */
int hale_matrix_upload(hale_ctx *ctx, int dtype, size_t rows, size_t cols,
                       const void *bytes, size_t nbytes, hale_matrix **out);
/* Same, with the reference-layout bytes already in device memory (for
 * example written by hale_encode_rows_device). */
int hale_matrix_upload_device(hale_ctx *ctx, int dtype, size_t rows,
                              size_t cols, const void *d_bytes, size_t nbytes,
                              hale_matrix **out);
void hale_matrix_destroy(hale_matrix *m);
/* Ref: WeightMatrix::{rows, cols, dtype} (src/tensor/matrix.rs:65-77). */
int hale_matrix_shape(const hale_matrix *m, int *dtype, size_t *rows,
                      size_t *cols);
/* Ref: WeightMatrix::bytes (src/tensor/matrix.rs:78-81): the matrix back in
 * the reference layout (undoes the HBM repack). */
int hale_matrix_download(hale_ctx *ctx, const hale_matrix *m, void *bytes,
                         size_t nbytes);

/* ---- quantization ---------------------------------------------------- */

/* Ref: Q8Activations::quantize (src/tensor/quant.rs:77-93).  n % 32 == 0;
 * scales[n/32] (f32, not rounded to f16), quants[n]. */
int hale_quantize_q8_act(hale_ctx *ctx, const float *x, size_t n,
                         float *scales, int8_t *quants);
/* Ref: encode_row (src/tensor/quant.rs:274-321), applied to each row of a
 * row-major rows x cols f32 matrix (WeightMatrix::from_f32,
 * src/tensor/matrix.rs:48-61): Q8_0 / Q4_0 blocks, F16 / BF16 rounded to
 * nearest even (half's from_f32), F32 copied.  Host buffers; bytes gets
 * rows*row_bytes. */
int hale_encode_rows(hale_ctx *ctx, int dtype, size_t rows, size_t cols,
                     const float *values, void *bytes);
/* Same on device buffers, enqueued on the context's stream (d_values
 * 16-byte aligned for Q8_0 / Q4_0). */
int hale_encode_rows_device(hale_ctx *ctx, int dtype, size_t rows,
                            size_t cols, const float *d_values,
                            void *d_bytes);

/* Ref: decode_row (src/tensor/quant.rs:236-269), applied to each of `rows`
 * reference-layout rows laid end to end (rows*row_bytes bytes, any
 * alignment, as the reference's unaligned fallback allows): F32 copied,
 * F16 through half's to_f32 (exact; a NaN gets the quiet bit), BF16 shifted
 * into the upper half, Q8_0 scale*q, Q4_0 scale*(nibble-8) with the low
 * nibbles first.  values gets rows*cols f32.  Host buffers. */
int hale_decode_rows(hale_ctx *ctx, int dtype, size_t rows, size_t cols,
                     const void *bytes, float *values);
int hale_decode_rows_device(hale_ctx *ctx, int dtype, size_t rows,
                            size_t cols, const void *d_bytes,
                            float *d_values);
/* Ref: WeightMatrix::row_to_f32 (src/tensor/matrix.rs:88-92) for rows
 * first .. first+count-1 (count 1: the embedding lookup of
 * src/model/transformer.rs:185), decoded straight from the HBM layout into
 * d_values[count][cols], enqueued on the context's stream.  HALE_EINVAL
 * for rows past the end. */
int hale_matrix_rows_to_f32_device(hale_ctx *ctx, const hale_matrix *m,
                                   size_t first, size_t count,
                                   float *d_values);
/* Same into host memory (values[count][cols]), returning with the rows in
 * place. */
int hale_matrix_rows_to_f32(hale_ctx *ctx, const hale_matrix *m, size_t first,
                            size_t count, float *values);
/* Ref: WeightMatrix::to_f32 (src/tensor/matrix.rs:95-102): every row into
 * values[rows*cols] (host memory); n must be rows*cols. */
int hale_matrix_to_f32(hale_ctx *ctx, const hale_matrix *m, float *values,
                       size_t n);
/* Ref: WeightMatrix::convert (src/tensor/matrix.rs:104-109): the matrix
 * re-encoded in `dtype` as a new resident matrix (to_f32, then from_f32's
 * encode_row per row), both on the GPU; the same dtype gives a copy.
 * HALE_EINVAL when `dtype` needs a row length divisible by 32 and cols is
 * not. */
int hale_matrix_convert(hale_ctx *ctx, const hale_matrix *m, int dtype,
                        hale_matrix **out);

/* ---- matvec ---------------------------------------------------------- */

/* Ref: WeightMatrix::matvec (src/tensor/matrix.rs:115-126) and
 * matvec_serial (:130-143), which return identical bits.  xlen must equal
 * cols and outlen rows (the reference asserts both).  Quantized matrices:
 * x is quantized once, then dot_q8_0 / dot_q4_0 per row (quant.rs:
 * 115-144).  Float matrices: dot_f32 / dot_decoded per row (quant.rs:
 * 146-233: eight lane accumulators, the fixed reduce, then the tail).
 * Any row length (a multiple of 32 for q8_0 / q4_0). */
int hale_matvec(hale_ctx *ctx, const hale_matrix *m, const float *x,
                size_t xlen, float *out, size_t outlen);
/* Same on device buffers (d_x 16-byte aligned for float matrices),
 * enqueued on the context's stream. */
int hale_matvec_device(hale_ctx *ctx, const hale_matrix *m, const float *d_x,
                       float *d_out);
/* The per-block i32 sums of dot_q8_0 / dot_q4_0 (src/tensor/quant.rs:
 * 115-144, `isum`) for every row: isums[rows][cols/32].  For parity tests. */
int hale_matvec_block_sums(hale_ctx *ctx, const hale_matrix *m,
                           const float *x, size_t xlen, int32_t *isums);

/* ---- expert ---------------------------------------------------------- */

/* Ref: Expert::forward (src/expert/mod.rs:91-103): gate.matvec(x) and
 * up.matvec(x), h = silu(g)*u, down.matvec(h).  gate/up are [I][H], down is
 * [H][I], all of one quantized dtype.  x[H] -> out[H]. */
int hale_expert_forward(hale_ctx *ctx, const hale_matrix *gate,
                        const hale_matrix *up, const hale_matrix *down,
                        const float *x, float *out);
/* Same on device buffers (d_x 16-byte aligned), enqueued on the context's
 * stream. */
int hale_expert_forward_device(hale_ctx *ctx, const hale_matrix *gate,
                               const hale_matrix *up, const hale_matrix *down,
                               const float *d_x, float *d_out);

/* ---- MoE layer and its HBM-resident expert provider ------------------ */

/* Ref: MoeLayer (src/model/moe.rs:25-32) with an ExpertProvider
 * (src/expert/mod.rs:128-137) that keeps all E experts of the layer
 * resident in HBM.  `router` is the f32 [E][H] router matrix, or NULL for a
 * layer whose router logits are supplied to hale_moe_forward.
 * normalize_topk: ModelConfig::normalize_topk (src/config.rs:205-208).
 * top_k is clamped to num_experts (top_k, src/ops/topk.rs:45); top_k = 0
 * routes every token nowhere, so forward leaves out at zero.  Any
 * num_experts, top_k, hidden and inter (multiples of 32) are taken, as in
 * the reference.  Layers within 1024 experts, top-64, hidden 8192 and down
 * rows of 512 blocks run the decode and expert-grouped kernels; larger ones
 * run a general path (router logits by the f32 GEMV, a routing kernel for
 * any expert count, row-chain matvecs per route, the route-order combine)
 * with the same bits, and never take the grouped path. */
int hale_moe_create(hale_ctx *ctx, uint32_t layer, size_t num_experts,
                    size_t hidden, size_t inter, int dtype, size_t top_k,
                    int normalize_topk, const hale_matrix *router,
                    hale_moe **out);
void hale_moe_destroy(hale_moe *moe);

/* Registers expert `expert` from reference-layout bytes (host memory):
 * gate/up [I][H], down [H][I].  Ref: ExpertSource::load + the pinned tier
 * of ExpertCache (src/expert/cache.rs:82-115), which here is all of HBM. */
int hale_moe_set_expert(hale_moe *moe, uint32_t expert, const void *gate,
                        const void *up, const void *down, size_t nbytes_gate,
                        size_t nbytes_down);
/* Same with the reference-layout bytes already in device memory. */
int hale_moe_set_expert_device(hale_moe *moe, uint32_t expert,
                               const void *d_gate, const void *d_up,
                               const void *d_down, size_t nbytes_gate,
                               size_t nbytes_down);
/* Registers an expert from uploaded matrices (copied into the layer). */
int hale_moe_set_expert_matrices(hale_moe *moe, uint32_t expert,
                                 const hale_matrix *gate,
                                 const hale_matrix *up,
                                 const hale_matrix *down);

/* Ref: MoeLayer::route (src/model/moe.rs:36-53): router matvec (8-lane f32
 * order), softmax_in_place, top_k (ties to the lower index), renormalise.
 * index[top_k], weight[top_k], best first. */
int hale_moe_route(hale_moe *moe, const float *x, uint32_t *index,
                   float *weight);

/* Ref: MoeLayer::forward (src/model/moe.rs:56-70) for ntok tokens.  ntok
 * == 1 is decode; ntok > 1 is the reference's token-at-a-time prefill
 * (src/model/transformer.rs:231-239), computed as one decode pass over all
 * tokens below the grouped threshold (hale_moe_set_grouped_min_tokens) and
 * as one expert-grouped batch from it: token t's output equals
 * MoeLayer::forward(x_t) either way.  x and out are
 * [ntok][H].  logits: NULL to run the router matvec, else [ntok][E] router
 * outputs used as given.  index/weight: NULL or [ntok][top_k].  The
 * _device form takes device buffers, enqueued on the context's stream:
 * d_x 16-byte aligned and d_logits 4-byte aligned, else HALE_EINVAL. */
int hale_moe_forward(hale_moe *moe, size_t ntok, const float *x,
                     const float *logits, float *out, uint32_t *index,
                     float *weight);
int hale_moe_forward_device(hale_moe *moe, size_t ntok, const float *d_x,
                            const float *d_logits, float *d_out,
                            uint32_t *d_index, float *d_weight);

/* Sizes the layer's per-token scratch and, from the grouped threshold on,
 * its grouped workspace for calls of up to max_tokens tokens, as the first
 * such call would.  No counterpart in the reference; for callers that
 * capture graphs (growth is refused during a capture) or want no
 * allocation inside a serving loop.  Refused (HALE_EINVAL) while the
 * context's stream is being captured only when the scratch or workspace
 * would have to grow; a reserve that fits what is held succeeds. */
int hale_moe_reserve(hale_moe *moe, size_t max_tokens);

/* Fewest tokens per hale_moe_forward* call that take the expert-grouped
 * path (default for top_k >= 4: 11 for q4_0 with hidden <= 2048, 9 for
 * wider q4_0, 12 for q8_0 with hidden <= 2048, 8 for wider q8_0; 7 for
 * top_k < 4); fewer tokens run the decode
 * kernels in one pass over all of them.  Both give the reference's bits; the choice is speed only.
 * n in 2..HALE_DECODE_MAX_TOKENS + 1.  A new threshold re-lays the layer's
 * per-token scratch on its next call, which must then come outside a graph
 * capture (or call hale_moe_reserve first).  No counterpart in the
 * reference (its prefill runs token by token); for callers tuning small
 * batches.  A layer on the general path (see hale_moe_create) has no
 * grouped form: the setting is accepted and ignored, and the threshold
 * reads SIZE_MAX. */
#define HALE_DECODE_MAX_TOKENS 256
int hale_moe_set_grouped_min_tokens(hale_moe *moe, size_t n);
int hale_moe_grouped_min_tokens(const hale_moe *moe, size_t *n);

/* Most tokens per expert-grouped call that run the row-chain kernels
 * (each lane one weight row, each expert's assignments two or four at a
 * time as scalar operands) in place of the int8 matrix products; larger
 * grouped calls take the matrix products.  Default c * num_experts / top_k
 * with c = 4.75 for q4_0 layers with hidden <= 2048, 4.25 for larger q4_0
 * ones, 5 for q8_0 ones with hidden <= 2048, 3.75 for larger q8_0 ones
 * and 3.25 for layers whose intermediate size exceeds 8192 (76, 68, 80 and
 * 60 tokens at 128 experts, top-8; 13 at 8 experts, top-2); layers whose intermediate
 * size exceeds 16384 never take them.  Both give the reference's bits; the choice is
 * speed only.  0 never takes them.  No counterpart in the reference; for
 * callers tuning batched decode and small prefill chunks. */
int hale_moe_set_band_max_tokens(hale_moe *moe, size_t n);
int hale_moe_band_max_tokens(const hale_moe *moe, size_t *n);

/* Folds of the expert-grouped down projection (hale_moe_forward with
 * ntok >= the grouped threshold).  HALE_FOLD_EXACT, the default, adds each
 * block term (d_w*d_x)*isum to its row sum as the reference does, product
 * then sum, and returns the reference's bits.  HALE_FOLD_FMA adds it with
 * one fused multiply-add, one rounding instead of two: the down output
 * then agrees with the reference to a relative L2 error far below 1e-5,
 * not bit for bit.  No counterpart in the reference; for callers that
 * accept that tolerance in exchange for a faster prefill.  The gate/up
 * projection and the decode path (below the grouped threshold) stay exact
 * in both. */
#define HALE_FOLD_EXACT 0
#define HALE_FOLD_FMA 1
int hale_moe_set_down_fold(hale_moe *moe, int fold);

/* Bytes of the fixed device scratch of hale_moe_forward_device_noalloc. */
#define HALE_NOALLOC_SCRATCH_BYTES (64u << 20)

/* No counterpart in the reference: hale_moe_forward_device for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same arguments, results
 * and errors, but the per-token scratch and the grouped workspace come from
 * a fixed array of HALE_NOALLOC_SCRATCH_BYTES per device, held until the
 * process ends; the call makes no device or host allocation.  A forward
 * whose scratch would exceed it runs as consecutive chunks of tokens that
 * fit, with the same bits (every token's output, routes and routing count
 * are independent of the others).  A grouped chunk of T tokens needs about
 * (T*top_k/32 + E) * (H + I)/32 * 1152 bytes of operand tiles plus
 * T*top_k*H*4 bytes of down outputs and about T*(H/32*48 + E*4) bytes of
 * per-token scratch: at 64 MiB, chunks of up to about 570 tokens for
 * E 128, H 2048, I 768, top-8 and about 215 for E 128, H 4096, I 1536.
 * When not even a chunk of the grouped threshold fits, the tokens run as
 * decode passes of fewer tokens.  Only a layer whose single token does not
 * fit is refused (HALE_EINVAL, before anything is enqueued).  Every
 * context on one device shares that device's
 * array, which keeps the last call's contents (nothing in it must start at
 * zero): calls that overlap in time on one device, from different contexts
 * or streams, race. */
int hale_moe_forward_device_noalloc(hale_moe *moe, size_t ntok,
                                    const float *d_x, const float *d_logits,
                                    float *d_out, uint32_t *d_index,
                                    float *d_weight);

/* Registers experts first .. first+count-1 from device buffers holding
 * their reference-layout bytes back to back: d_gate/d_up [count][I][H],
 * d_down [count][H][I] (bulk form of hale_moe_set_expert_device). */
int hale_moe_set_experts_device(hale_moe *moe, uint32_t first, uint32_t count,
                                const void *d_gate, const void *d_up,
                                const void *d_down);

/* Ref: ExpertProvider::routing_stats (src/expert/mod.rs:136) /
 * RoutingStats::count (src/expert/stats.rs:53-55): selections per expert
 * of this layer since creation.  counts[num_experts]. */
int hale_moe_routing_counts(hale_moe *moe, uint64_t *counts);

/* Ref: CacheStats (src/expert/cache.rs:15-33), field for field.  The HBM
 * layer is one tier, reported as the pinned tier: pinned_experts /
 * pinned_bytes are the resident experts; pinned_hits counts the selections
 * its forwards served (every selection, since a forward needs every expert
 * resident) plus the fetch requests that found their expert resident; the
 * LRU fields stay 0 (nothing is evicted); passthrough is 0.  misses are
 * fetch requests that loaded from the layer's source.  bytes_loaded and
 * load_seconds sum every read from a pack into the layer: fetch misses
 * (expert bytes per miss, as the reference counts them) and whole-layer
 * loads (hale_moe_load_pack / prefetch_pack, timed from the first read to
 * the last repack on the device). */
typedef struct hale_cache_stats {
  uint64_t pinned_hits;
  uint64_t lru_hits;
  uint64_t misses;
  uint64_t bytes_loaded;
  double load_seconds;
  size_t pinned_experts;
  size_t pinned_bytes;
  size_t lru_experts;
  size_t lru_bytes;
  size_t lru_capacity_bytes;
  int passthrough;
} hale_cache_stats;

/* Ref: ExpertProvider::stats (src/expert/mod.rs:133). */
int hale_moe_cache_stats(hale_moe *moe, hale_cache_stats *out);

/* Ref: ExpertProvider::fetch (src/expert/mod.rs:130) as ExpertCache
 * implements it (src/expert/cache.rs:124-194), for keys (layer, experts[i])
 * of this layer: records one selection per key (routing_stats), serves the
 * resident experts, and loads each missing one from the layer's source
 * into HBM (hale_moe_set_source; without a source a missing expert is
 * HALE_ENOTFOUND).  gate/up/down (each NULL or [n]) receive, in request
 * order, the experts' matrices as views into the layer: usable wherever a
 * hale_matrix is (hale_matvec, hale_expert_forward[_device], download,
 * convert), owned by the layer and valid until hale_moe_destroy
 * (hale_matrix_destroy ignores them).  An expert index >= num_experts is
 * HALE_EINVAL. */
int hale_moe_fetch(hale_moe *moe, const uint32_t *experts, size_t n,
                   const hale_matrix **gate, const hale_matrix **up,
                   const hale_matrix **down);
/* Whether expert `expert` is resident (after any pending pack load). */
int hale_moe_expert_present(hale_moe *moe, uint32_t expert, int *present);

/* ---- expert pack: the file tier under the HBM tier ------------------ */

/* Opens a Hale expert pack ("HALEPACK" magic, u64 LE header length, JSON
 * PackHeader, records gate|up|down at a fixed stride from data_offset).
 * Rejects, with HALE_EPACK, what PackExpertSource::open rejects: a wrong
 * magic, a header longer than 64 x 16 KiB, unparsable JSON, a version other
 * than 1, a file shorter than data_offset + layers x experts x stride.
 * Ref: PackExpertSource::open (src/expert/pack.rs:207-249), PackHeader
 * (:55-73).  The hale_pack_* calls take no context: their failures are
 * reported by hale_last_error(NULL) in the calling thread.  The first load
 * into a layer binds the pack to that layer's context, on whose device it
 * then uploads through its own HIP stream. */
int hale_pack_open(const char *path, hale_pack **out);
/* Waits for a load in progress, then closes the file. */
void hale_pack_close(hale_pack *pack);
/* PackHeader fields (any output may be NULL). */
int hale_pack_info(const hale_pack *pack, int *dtype, size_t *hidden,
                   size_t *inter, size_t *num_experts, size_t *num_moe_layers,
                   size_t *record_bytes, size_t *record_stride,
                   size_t *data_offset);
/* Model layer index of the pack's `ordinal`-th MoE layer (file order). */
int hale_pack_moe_layer(const hale_pack *pack, size_t ordinal,
                        uint32_t *layer);
/* Byte offset of (layer, expert)'s record; HALE_EPACK for a layer without
 * experts in the pack or an expert out of range.  Ref: PackHeader::offset_of
 * (src/expert/pack.rs:104-123). */
int hale_pack_offset_of(const hale_pack *pack, uint32_t layer,
                        uint32_t expert, uint64_t *offset);
/* Reads one record (record_bytes: gate | up | down in the pack dtype) into
 * host memory with a positioned read.  Ref: ExpertSource::load for
 * PackExpertSource (src/expert/pack.rs:252-260). */
int hale_pack_read_expert(hale_pack *pack, uint32_t layer, uint32_t expert,
                          void *buf, size_t nbytes);

/* HBM tier from the pack: makes every expert of moe's layer resident.  The
 * pack's dtype and shapes must match the layer (HALE_EINVAL otherwise; a
 * layer missing from the pack is HALE_EPACK).  hale_moe_prefetch_pack
 * returns at once: a loader thread reads the layer's records (one large
 * sequential read per batch into pinned host buffers) and uploads and
 * repacks them on the pack's stream, so the layer's experts arrive while
 * other layers compute.  The layer's next use (forward, set_expert, load
 * or destroy) waits for the load and reports its error.  One load per
 * pack at a time: a second prefetch on the same pack waits for the first
 * load's reads.  hale_moe_load_pack is the synchronous form.  Ref: the
 * ExpertCache miss path (src/expert/cache.rs:124-194) over
 * PackExpertSource, and roadmap item 2 (prefetch the next layer's
 * experts, docs/roadmap.md:13-16). */
int hale_moe_load_pack(hale_moe *moe, hale_pack *pack);
int hale_moe_prefetch_pack(hale_moe *moe, hale_pack *pack);
/* Makes `pack` the layer's source, the ExpertSource behind its HBM tier
 * (src/expert/mod.rs:110-124), without loading anything: hale_moe_fetch
 * loads missing experts from it.  Checked like hale_moe_prefetch_pack,
 * which binds its pack the same way.  NULL unbinds; hale_pack_close
 * unbinds the pack from every layer. */
int hale_moe_set_source(hale_moe *moe, hale_pack *pack);

/* ---- the steps on either side of the MoE block ------------------------ */

typedef struct hale_attention hale_attention; /* Ref: Attention + LayerCache */

/* Ref: rms_norm (src/ops/norm.rs:7-14): out = x * scale * w with
 * scale = 1 / sqrt(sum(x^2) / n + eps), the squares summed in order.
 * n <= 8192. */
int hale_rms_norm(hale_ctx *ctx, const float *x, const float *weight, size_t n,
                  float eps, float *out);
/* Device form over `rows` rows of n values.  With d_delta non-NULL, each row
 * first becomes x = x + delta, stored back into d_x (add_in_place,
 * src/model/transformer.rs:203-205,242-246, the residual before the next norm).
 * d_out may equal d_x. */
int hale_rms_norm_device(hale_ctx *ctx, float *d_x, const float *d_delta,
                         const float *d_weight, size_t rows, size_t n,
                         float eps, float *d_out);

/* Ref: Attention (src/model/attention.rs:11-24) with its layer's KV cache
 * (src/model/kv_cache.rs:9-32), room for max_len positions.  q [heads*hd][H],
 * k / v [kv_heads*hd][H], o [H][heads*hd] are uploaded matrices of any
 * dtype, borrowed (they must outlive the attention).  q_norm / k_norm:
 * QK-norm weights [head_dim] (host memory, copied) or NULL (Mixtral).
 * head_dim a multiple of 16 up to 1024; heads a multiple of kv_heads, at
 * most 16 query heads per key/value head. */
int hale_attention_create(hale_ctx *ctx, const hale_matrix *q_proj,
                          const hale_matrix *k_proj, const hale_matrix *v_proj,
                          const hale_matrix *o_proj, const float *q_norm,
                          const float *k_norm, size_t num_heads,
                          size_t num_kv_heads, size_t head_dim, float norm_eps,
                          size_t max_len, hale_attention **out);
void hale_attention_destroy(hale_attention *attn);
/* Empties the cache (a new sequence). */
int hale_attention_reset(hale_attention *attn);
/* Positions in the cache (the position of the next token). */
int hale_attention_len(const hale_attention *attn, size_t *len);
/* Ref: Attention::forward (src/model/attention.rs:31-86) for the token at
 * `position`, which must equal the cache length: q/k/v projections,
 * QK-norm and RoPE (rotate-half, cos/sin [head_dim/2] from Rope::angles),
 * the cache push, scores in order, softmax_in_place, the context in
 * position order, o projection.  x, out [H].  HALE_EINVAL on a position
 * other than the cache length or past max_len (ContextOverflow). */
int hale_attention_forward(hale_attention *attn, const float *x, size_t position,
                           const float *cos, const float *sin, float *out);
/* Same on device buffers (d_x 16-byte aligned), enqueued on the stream. */
int hale_attention_forward_device(hale_attention *attn, const float *d_x,
                                  size_t position, const float *d_cos,
                                  const float *d_sin, float *d_out);

/* ---- support entry points -------------------------------------------
 * No counterpart in the reference: device memory, timing and graph capture
 * for benchmarks and tests, so that a caller needs no second HIP runtime. */

int hale_device_malloc(hale_ctx *ctx, size_t bytes, void **out);
int hale_device_free(hale_ctx *ctx, void *p);
/* Synchronous copies between host and device memory. */
int hale_memcpy_htod(hale_ctx *ctx, void *dst, const void *src, size_t n);
int hale_memcpy_dtoh(hale_ctx *ctx, void *dst, const void *src, size_t n);
/* Fills d_out[n] with seeded N(mean, std^2) values (counter-based
 * generator, enqueued on the context's stream). */
int hale_fill_normal_device(hale_ctx *ctx, uint64_t seed, float mean,
                            float std, float *d_out, size_t n);
/* d_dst[0, n) = d_src[0, n) by a plain streaming kernel (n and both
 * addresses multiples of 16), enqueued on the context's stream: one read and
 * one write per byte, the calibration for HBM traffic counters. */
int hale_copy_device(hale_ctx *ctx, void *d_dst, const void *d_src, size_t n);
/* Reads d_src[0, n) once by a plain streaming kernel of `workgroups`
 * work-groups (1..65535), each over a contiguous chunk, and writes the XOR
 * of the 32-bit words of chunk g to d_out[g] (n and d_src multiples of 16).
 * No counterpart in the reference: the yardstick for what one launch of n
 * bytes can stream from HBM, timed beside the decode kernels. */
int hale_stream_read_device(hale_ctx *ctx, const void *d_src, size_t n, unsigned workgroups,
                            uint32_t *d_out);

/* Wall time of the work enqueued between start and stop, from HIP events
 * recorded on the context's stream; stop waits for that work. */
int hale_timer_start(hale_ctx *ctx);
int hale_timer_stop(hale_ctx *ctx, double *ms);

/* Per-kernel timing: while enabled, every kernel the context launches is
 * bracketed by HIP events on its stream.  hale_profile_read waits for the
 * stream and returns the summed duration and launch count of one kernel
 * kind since the last reset; hale_kernel_name names the kinds
 * (0 .. hale_kernel_kinds()-1). */
int hale_profile_enable(hale_ctx *ctx, int on);
int hale_profile_read(hale_ctx *ctx, int kind, double *total_ms,
                      uint64_t *launches);
int hale_profile_reset(hale_ctx *ctx);
int hale_kernel_kinds(void);
const char *hale_kernel_name(int kind);

/* Graph capture of the context's stream: the _device entry points called
 * between begin and end are recorded (not run) and replayed by launch.
 * Rules:
 *   - Scratch (the context's, a layer's per-token scratch and grouped
 *     workspace) only grows outside a capture.  A call that would have to
 *     grow it while the stream is being captured fails with HALE_EINVAL and
 *     records nothing; make the same call once before the capture, or size
 *     a layer with hale_moe_reserve.
 *   - A graph keeps the addresses it was captured with.  Scratch that a
 *     later call outgrows while any graph of the context exists is kept,
 *     not freed, until the last of those graphs is destroyed, so an older
 *     graph replays correctly after a larger call.
 *   - Matrices, layers and attention blocks a graph uses must outlive it. */
typedef struct hale_graph hale_graph;
int hale_graph_begin(hale_ctx *ctx);
int hale_graph_end(hale_ctx *ctx, hale_graph **out);
int hale_graph_launch(hale_graph *g);
void hale_graph_destroy(hale_graph *g);

#ifdef __cplusplus
}
#endif
#endif /* HALE_MOE_H */
