/* relx.h - C ABI of librelx, the MI355X-native executor for Sym relocation
 * plans (wire v0 layout plans and wire v1 typed plans).
 *
 * Every entry point is extern "C", takes plain pointers and sizes, and never
 * throws. Failures return a nonzero status and fill `relx_err` with a stable
 * code (the reference's codes where one exists) and a message. Calls block
 * until their device work completes unless a function says otherwise.
 *
 * Each declaration names the reference interface it replaces (file:line under
 * the reference tree JueonPark/sym).
 */
#ifndef RELX_H
#define RELX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RELX_OK 0
#define RELX_ERROR 1

/* Completion of a failed call (reference QueueCompletion,
 * libreloc/include/reloc/Backend.h:63-69; TransferError::completion). */
#define RELX_NOT_LAUNCHED 0
#define RELX_COMPLETE 1
#define RELX_UNKNOWN 2

typedef struct relx_err {
  char code[48];     /* e.g. "decode_error", "bind_error", "invalid_view" */
  char message[464]; /* human-readable detail (byte offset for decode errors) */
  int64_t offset;    /* decode errors: byte offset; else -1 */
  int completion;    /* RELX_NOT_LAUNCHED / RELX_COMPLETE / RELX_UNKNOWN */
} relx_err;

typedef struct relx_plan relx_plan;   /* decoded, immutable plan */
typedef struct relx_bound relx_bound; /* bound plan + prepared device program */
typedef struct relx_ctx relx_ctx;     /* per-device retained execution context */

/* ---------------------------------------------------------------- plans */

/* Library identification string. Replaces reloc::versionString
 * (libreloc/src/Version.cpp:5-8). */
const char *relx_version(void);

/* Wire version in bytes 4..8 of an "RPLN" blob, or -1 when the header is not
 * a plan. Replaces reloc::peekWireVersion (libreloc/src/Decode.cpp:868-874). */
int relx_wire_version(const uint8_t *blob, size_t n);

/* Decode a wire v0 (layout), v1 (typed) or v2 (indexed) plan; the header
 * picks the decoder. Replaces reloc::decodePlan / reloc::decodeTypedPlan /
 * reloc::decodeIndexedPlan (libreloc/src/Decode.cpp:876-948,993-1012) and
 * pyreloc.load_plan / load_typed_plan / load_indexed_plan
 * (libreloc/python/PyReloc.cpp:596,864,921). Errors: code "decode_error"
 * with the byte offset of the violated item. */
int relx_plan_load(const uint8_t *blob, size_t n, relx_plan **out, relx_err *err);

/* 1 for a typed (v1) plan, 0 otherwise. */
int relx_plan_is_typed(const relx_plan *plan);

/* The decoded plan's wire version (0, 1 or 2). */
int relx_plan_version(const relx_plan *plan);

/* Number of plan symbols and the i-th symbol name (owned by the plan). */
int relx_plan_symbol_count(const relx_plan *plan);
const char *relx_plan_symbol(const relx_plan *plan, int i);

void relx_plan_free(relx_plan *plan);

/* Decoded value stages of a typed (v1) plan (reference TypedPlanHandle
 * .stages / .fills / .parameters, libreloc/python/PyReloc.cpp:241-288,
 * 803-840). Types are (kind 0 float, 1 bfloat, 2 integer; bits);
 * signedness 0 signless, 1 signed, 2 unsigned; parameter kinds 0 none,
 * 1 inline, 2 binding. */
typedef struct relx_plan_stage_info {
  int transform; /* 0 cast, 1 quantize, 2 dequantize */
  int policy;    /* 0 ieee_rne, 1 exact, 2 symmetric_rne, 3 affine */
  int in_kind, in_bits, in_signedness;
  int out_kind, out_bits, out_signedness;
  int rank;
  int64_t axis; /* -1 for a per-tensor stage */
  int has_channel;
  int scale_kind, zero_point_kind;
} relx_plan_stage_info;
int relx_plan_stage_count(const relx_plan *plan);
int relx_plan_stage(const relx_plan *plan, int i, relx_plan_stage_info *out);
int relx_plan_fill_count(const relx_plan *plan);
/* Runtime parameter declarations in first-declaration order, one per name:
 * name (owned by the plan), type, rank, first stage and role (0 scale,
 * 1 zero point). Returns the count, or fills entry i when 0 <= i < count. */
int relx_plan_parameter(const relx_plan *plan, int i, const char **name, int *kind, int *bits,
                        int *rank, int *stage, int *role);

/* A runtime parameter value by declared name (reference ParameterValue,
 * libreloc/include/reloc/Bind.h:125-133): element type (kind 0 float,
 * 1 bfloat, 2 integer; bitwidth), rank 0 or 1 with its length, and the
 * little-endian element bytes. Bytes are copied during the call. */
typedef struct relx_param {
  const char *name;
  int kind;
  int bits;
  int rank;
  int64_t length;
  const void *data;
  size_t nbytes;
} relx_param;

/* Bind symbols (and, for typed plans, parameters), then prepare the device
 * program. Replaces reloc::bind / reloc::bindTyped
 * (libreloc/src/Bind.cpp:176-384, 494-699) + typed::prepareProgram
 * (libreloc/src/TypedExecute.cpp:292-403), pyreloc.bind / bind_typed
 * (libreloc/python/PyReloc.cpp:674,987). Errors: "bind_error",
 * "unsupported_stage", "invalid_parameter". */
int relx_bind(const relx_plan *plan, const char *const *sym_names, const int64_t *sym_values,
              int nsym, const relx_param *params, int nparam, relx_bound **out,
              relx_err *err);

/* Bind an indexed (v2) plan: symbols plus the index operand, given as its
 * element type (kind 2 integer; bits 32 or 64), extents and little-endian
 * bytes, which are copied and range-checked during the call. The bound plan
 * describes the selected rows: an identity relocation of
 * [count, row elements] plus the plan's cast. Replaces reloc::bindIndexed
 * (libreloc/src/Bind.cpp:701-819) and pyreloc.bind_indexed /
 * bind_indexed_from_pointer (libreloc/python/PyReloc.cpp:876-919). Errors:
 * "bind_error" with the reference's messages, including
 * "index_out_of_range: index_select row is outside the source". */
int relx_bind_indexed(const relx_plan *plan, const char *const *sym_names,
                      const int64_t *sym_values, int nsym, int index_kind, int index_bits,
                      const int64_t *index_extents, int index_rank, const void *index_data,
                      size_t index_bytes, relx_bound **out, relx_err *err);

void relx_bound_free(relx_bound *bound);

/* Bound-plan facts (reference BoundPlan / TypedBoundPlan fields,
 * libreloc/include/reloc/Bind.h:82-102,164-190). Stage boundaries are
 * 0..stages; bytes_at[k] is the dense footprint at boundary k. */
#define RELX_MAX_RANK 8
#define RELX_MAX_STAGES 8
typedef struct relx_bound_info {
  int typed;
  int rank; /* coalesced axes */
  int64_t extents[RELX_MAX_RANK];
  int64_t src_strides[RELX_MAX_RANK];
  int64_t dst_strides[RELX_MAX_RANK];
  int64_t pad_lo[RELX_MAX_RANK];
  int64_t pad_hi[RELX_MAX_RANK];
  int element_size; /* result element bytes */
  int64_t total_bytes; /* destination footprint */
  int64_t source_bytes;
  int64_t destination_bytes;
  int64_t parameter_bytes;
  int stages;
  int64_t bytes_at[RELX_MAX_STAGES + 1];
  int source_width;
  int result_width;
  int source_rank;
  int64_t source_extents[RELX_MAX_RANK];
  int result_rank;
  int64_t result_extents[RELX_MAX_RANK];
  char kernel[32]; /* device kernel family the program runs */
  int host_stages_max;  /* leading per-tensor stages a host may apply */
  int host_stages_auto; /* of those, the narrowing ones the host applies by default */
  int64_t wire_bytes_at[RELX_MAX_STAGES + 1]; /* H2D wire (source layout) at boundary k */
  /* indexed (v2) plans (reference IndexedBoundPlan, libreloc/include/reloc/Bind.h):
   * the physical source is table_rows rows of row_elements elements;
   * source_bytes above counts the selected rows only */
  int indexed;
  int64_t table_rows;
  int64_t row_elements;
  int64_t table_bytes;
  int64_t index_count;
  /* permute programs: 1 when every launch of the whole box (the launches of
   * relx_relayout_device) runs the direct body, whose divisions are shifts
   * and whose vectors take stage parameters from their own channel
   * coordinate; 0 otherwise */
  int permute_direct;
  /* transpose programs: the q width (source-contiguous axis) of the tile
   * kernel's tiles, 128 for one-byte sources whose q extent is a multiple of
   * 128, else 64; and their c width (destination-contiguous axis), 128 for
   * two- and four-byte results when q and c both are multiples of 128 (tiles
   * kept in LDS as bytes), else 64; 0 for the other kernel families */
  int transpose_tile_q;
  int transpose_tile_c;
  /* transpose programs: 1 when every launch of the whole box indexes the
   * parameters of its dequantize -> f16 chain by destination row (one
   * channel per row, proven per launch), else 0 */
  int transpose_row_params;
} relx_bound_info;

int relx_bound_query(const relx_bound *bound, relx_bound_info *out);

/* ------------------------------------------------------------- contexts */

/* A retained per-device context: two copy streams and a compute stream, a
 * pinned host staging ring, device wire scratch and events. Replaces
 * CudaBackend (libreloc/cuda/CudaBackend.cu:55-282) and the retained
 * ScratchBackend of dispatch::Resources
 * (libreloc/src/DispatchResources.cpp:44,552-686). `max_retained_bytes`
 * bounds the scratch kept between calls, pinned ring plus device wire arena,
 * as the reference's maxRetainedBytes does
 * (libreloc/include/reloc/DispatchResources.h:57-61): once a blocking call,
 * or relx_ctx_synchronize, finds every call on the context completed, the
 * ring and the arena are released, the larger first, until what is kept
 * fits; the next call that needs them allocates them again. 0 keeps none;
 * a negative value sets no bound. Submitted and no_wait calls keep their
 * scratch until such a point. The parameter tables of the plans run on the
 * context are kept apart from this bound, by content (at most 4096 tables
 * or 16 MiB; a fresh binding of the same plan and parameters uploads
 * nothing), until the context is closed. */
int relx_ctx_create(int device, int64_t max_retained_bytes, relx_ctx **out, relx_err *err);

/* Drain and free. A context whose completion is unknown is quarantined (its
 * memory is kept for the process lifetime), as the reference does
 * (libreloc/src/Transfer.cpp:336-343). */
int relx_ctx_close(relx_ctx *ctx, relx_err *err);

/* Retained-resource gauges. */
typedef struct relx_ctx_stats {
  int64_t pinned_bytes;
  int64_t device_bytes;
  int64_t calls;
  int64_t failures;
  int quarantined;
} relx_ctx_stats;
int relx_ctx_stats_get(const relx_ctx *ctx, relx_ctx_stats *out);

/* ------------------------------------------------------------ execution */

/* Per-call options (reference TransferOptions,
 * libreloc/include/reloc/Transfer.h:121-155). Zeroed = defaults. */
typedef struct relx_options {
  int n_buffers;        /* pinned ring slots: 0 = 3; with chunk_bytes 0 (the
                         * library's chunks) at least 3, else exactly this many */
  int64_t chunk_bytes;  /* wire bytes per chunk (0 = schedule picks) */
  int host_stages;      /* leading per-tensor cast stages the host applies
                           while staging (-1 = auto: the leading narrowing
                           ones, whatever the source's memory; 0 = none) */
  int gather_threads;   /* host staging threads (0 = default: 8, and 12 for
                           the host row gathers of indexed plans) */
  int source_pinned;    /* 1: source is page-locked; DMA it directly.
                           -1: probe; 0: pageable (stage through the ring) */
  uint64_t caller_stream; /* hipStream_t the call's kernels and direct
                             copies are ordered after, and that a no_wait
                             call's end is ordered before, when
                             has_caller_stream is set; 0 is HIP's legacy
                             null stream */
  int no_wait;          /* 1: return after enqueue; the caller's stream (or
                           relx_ctx_synchronize) orders later work */
  int has_caller_stream; /* 1: order after caller_stream (reference
                            TransferOptions::hasCallerStream,
                            libreloc/include/reloc/Transfer.h:126-128);
                            0: no producer stream to order after */
  int n_streams;        /* copy streams the call's chunks alternate over
                           (reference execute_dispatch n_streams,
                           libreloc/python/PyDispatch.cpp:159-235): 1 puts
                           every copy and kernel on one stream; 0 (default)
                           and 2 or more use the context's two copy streams */
} relx_options;

/* Scalar report of one call (reference dispatch::Report,
 * libreloc/include/reloc/Dispatch.h:104-124). */
typedef struct relx_report {
  char implementation[40]; /* "hip_relayout", "hip_relayout@k", "hip_table_gather" */
  int64_t source_bytes;
  int64_t wire_bytes;
  int64_t destination_bytes;
  int64_t parameter_bytes;
  int64_t payload_bytes_transferred;
  int64_t chunks;
  int64_t kernel_launches;
  int wire_boundary;
  int direct_dma; /* 1 when the source was DMA'd without staging */
  /* The host side of the call (reference Report::hostChunkBytes /
   * hostBuffers and the staging rows, libreloc/include/reloc/Dispatch.h:
   * 104-124, Transfer.h:112-119): */
  int64_t host_chunk_bytes; /* bytes of the largest chunk moved (staged or DMA'd) */
  int64_t host_buffers;     /* ring slots the staged chunks cycled through (0: none staged) */
  int64_t staging_bytes;    /* page-locked bytes of the staging ring the call used (0: none) */
  int64_t staging_slots;    /* that ring's slot count */
  int staging_reused;       /* 1: the ring was kept from an earlier call (nothing allocated) */
  int copy_streams;         /* copy streams the call's chunks used */
} relx_report;

/* Run one bound plan: host source (dense, source layout, source dtype) ->
 * device destination (dense result layout). The source bytes move through
 * the chunked pinned H2D pipeline on the copy stream; relayout and value
 * stages run as HIP kernels behind each chunk's copy on its copy stream, while
 * the next chunk's copy runs on the other copy stream. With
 * `has_caller_stream` the call's kernels and its direct copies of a
 * page-locked source run after the work enqueued on `caller_stream` so far
 * (copies out of the library's staging ring touch no caller memory and
 * start at once); a call that returns early (no_wait) makes `caller_stream`
 * wait for its end, and a blocking call has completed when it returns.
 * Replaces dispatch::executeDispatch (libreloc/src/Dispatch.cpp:1983-2046)
 * for the H2D direction, executeTransfer (libreloc/src/Transfer.cpp:493-544)
 * for layout plans, and pyreloc.execute_dispatch / execute_transfer
 * (libreloc/python/PyDispatch.cpp:159-235, PyTransfer.cpp:180-219).
 * An indexed (v2) bound plan takes the whole host table as `src`: worker
 * threads gather the selected rows (through the leading per-tensor stages
 * the staging applies) into the pinned ring, as the reference's CPU path
 * does (libreloc/src/Dispatch.cpp:1238-1247), and the device runs the rest.
 * Errors: "insufficient_capacity", "invalid_options", "backend_failure",
 * "channel_out_of_range", "invalid_view". */
int relx_execute_h2d(relx_ctx *ctx, const relx_bound *bound, const void *src, size_t src_bytes,
                     void *dst, size_t dst_bytes, const relx_options *opt, relx_report *report,
                     relx_err *err);

/* The upload of relx_execute_h2d with no allocation: the call allocates no
 * device or pinned host memory (no hipMalloc, hipFree, hipHostMalloc or
 * allocating library routine). No counterpart in the reference; it is for
 * callers that cannot allocate: tight serving loops, harnesses that forbid
 * allocation. It is not for HIP graph capture: a blocking call waits on the
 * host, and each call copies its parameter tables from host memory when it
 * is made. The wire is staged in the library's static device scratch, a
 * file-scope array of 64 MiB that each GPU the library runs on holds until
 * the process ends (63 MiB of wire, and parameter tables of up to 512 KiB
 * of floats and 512 KiB of ints), and the source must be page-locked: it
 * crosses by direct DMA, with no host stages. Errors:
 * "insufficient_capacity" for a wire or parameter tables beyond those
 * limits, "invalid_options" for a pageable source or host stages,
 * "plan_mismatch" for an indexed plan, else as relx_execute_h2d. Every
 * static call on a GPU uses that GPU's one scratch and leaves its contents
 * behind; calls from several contexts or threads take it in turn (a lock
 * per GPU, and each call's copies into the scratch wait on the device for
 * the previous static call's end, also after a no_wait call). */
int relx_execute_h2d_static(relx_ctx *ctx, const relx_bound *bound, const void *src,
                            size_t src_bytes, void *dst, size_t dst_bytes, const relx_options *opt,
                            relx_report *report, relx_err *err);

/* ------------------------------------------------- layout transfers */

/* A framework buffer as the caller declares it (reference BufferView,
 * libreloc/include/reloc/Transfer.h:47-56): the allocation (base, capacity
 * in bytes from base), the byte offset of logical element 0, extents,
 * element strides, element size, memory kind and device ordinal (-1 for
 * host memory). */
#define RELX_MAX_VIEW_RANK 16
#define RELX_KIND_HOST 0
#define RELX_KIND_DEVICE 1
#define RELX_H2D 0
#define RELX_D2H 1
typedef struct relx_view {
  uint64_t base;
  uint64_t capacity_bytes;
  uint64_t offset_bytes;
  int rank;
  int64_t extents[RELX_MAX_VIEW_RANK];
  int64_t strides[RELX_MAX_VIEW_RANK];
  uint32_t element_size;
  int kind;
  int device;
} relx_view;

/* Bytes from element 0 the view can address, after rejecting empty,
 * negative-stride, broadcast and overlapping views, every step
 * overflow-checked; `role` names the view in messages. Replaces
 * reloc::viewSpanBytes (libreloc/src/Transfer.cpp:65-113) and
 * pyreloc.BufferView.span_bytes (libreloc/python/PyTransfer.cpp:327-330).
 * Errors: "invalid_view", "unsupported_layout", "integer_overflow",
 * "insufficient_capacity". */
int relx_view_span_bytes(const relx_view *view, const char *role, uint64_t *span, relx_err *err);

/* Preflight: the layout plan's source reads fit `source` and the view is
 * admissible for `direction` (RELX_H2D / RELX_D2H); `*span` receives the
 * source span. Allocates and launches nothing. Replaces
 * reloc::validateTransferSource (libreloc/src/Transfer.cpp:233-244) and
 * pyreloc.validate_transfer_source (libreloc/python/PyTransfer.cpp:91-99).
 * Errors: the view's, "direction_mismatch", "typed_unsupported",
 * "plan_mismatch", "integer_overflow". */
int relx_validate_transfer_source(const relx_bound *bound, const relx_view *source,
                                  int direction, uint64_t *span, relx_err *err);

/* Full validation with the destination: dense, exactly the plan's
 * footprint, every padded write inside. Replaces reloc::validateTransfer
 * (libreloc/src/Transfer.cpp:246-268) and pyreloc.make_transfer
 * (libreloc/python/PyTransfer.cpp:109-118). */
int relx_validate_transfer(const relx_bound *bound, const relx_view *source,
                           const relx_view *destination, int direction, uint64_t *source_span,
                           uint64_t *destination_bytes, relx_err *err);

/* Validate, then run the layout plan's forward transfer on the context's
 * device: host -> device through the upload pipeline (the source view's
 * span is uploaded from its element 0), device -> host through the download
 * pipeline. Blocks like relx_execute_h2d / relx_execute_d2h. Replaces
 * reloc::executeTransfer (libreloc/src/Transfer.cpp:493-544) and
 * pyreloc.execute_transfer (libreloc/python/PyTransfer.cpp:120-219).
 * Errors: the validators', "device_mismatch" (the device view is not on the
 * context's device), "backend_mismatch" (both views in host memory), and
 * those of the pipelines. */
int relx_execute_transfer(relx_ctx *ctx, const relx_bound *bound, const relx_view *source,
                          const relx_view *destination, int direction, const relx_options *opt,
                          relx_report *report, relx_err *err);

/* The device ordinal owning a device pointer (hipPointerGetAttributes).
 * Replaces reloc::cudaPointerDevice and pyreloc.cuda_pointer_device
 * (libreloc/python/PyTransfer.cpp:291-306). Errors: "invalid_view" for
 * host or unknown memory. */
int relx_pointer_device(const void *pointer, int *device, relx_err *err);

/* A group of bound plans as one schedule: all members' wire bytes through
 * one ring and one event barrier (reference group_detail::executeGroup,
 * libreloc/src/Dispatch.cpp:1833-1981; pyreloc.execute_dispatch_group).
 * `reports` has n entries; `total` (optional) sums them. */
int relx_execute_group_h2d(relx_ctx *ctx, int n, const relx_bound *const *bounds,
                           const void *const *srcs, const size_t *src_bytes, void *const *dsts,
                           const size_t *dst_bytes, const relx_options *opt,
                           relx_report *reports, relx_report *total, relx_err *err);

/* ------------------------------------------------------- asynchronous */

typedef struct relx_completion relx_completion;

/* Enqueue a group like relx_execute_group_h2d and return without waiting:
 * `*out` is the group's completion (Resources::submit,
 * libreloc/src/DispatchResources.cpp:688-747; pyreloc.submit_dispatch_group,
 * libreloc/python/PyDispatch.cpp:696-707). Staging of pageable sources runs
 * during this call (the pinned ring is host-driven); pinned sources move by
 * DMA entirely after it returns. Sources and destinations must stay alive
 * until the completion has been waited for or freed. */
int relx_submit_group_h2d(relx_ctx *ctx, int n, const relx_bound *const *bounds,
                          const void *const *srcs, const size_t *src_bytes, void *const *dsts,
                          const size_t *dst_bytes, const relx_options *opt, relx_report *reports,
                          relx_report *total, relx_completion **out, relx_err *err);

/* Completion::query: *done = 1 once every kernel of the call finished.
 * When the device reports a failure for the group, the context is drained:
 * "backend_failure" with a complete completion, or, when completion cannot
 * be proven, "completion_unknown" with RELX_UNKNOWN and the context
 * quarantined (reference Completion, libreloc/src/DispatchResources.cpp:
 * 325-361). The outcome is kept: later queries and waits report it. */
int relx_completion_query(relx_completion *c, int *done, relx_err *err);

/* Completion::wait: block until done; reports a channel outside the
 * parameters (`channel_out_of_range`) like the blocking call would, and a
 * device failure as relx_completion_query does. */
int relx_completion_wait(relx_completion *c, relx_err *err);

/* Completion::waitStream: order `stream` after the call without blocking
 * the host (H2D: the destination is ready for kernels on `stream`). */
int relx_completion_wait_stream(relx_completion *c, uint64_t stream, relx_err *err);

/* Free a completion; an unfinished call is waited for first (abandoning a
 * handle drains, as the reference's ~Completion does). */
void relx_completion_free(relx_completion *c);

/* Device-resident source -> host destination: the D2H direction of
 * dispatch::executeDispatch / executeTransfer (libreloc/src/Transfer.cpp:469-488,
 * libreloc/src/Dispatch.cpp:1072-1099,1513-1530; the reference's
 * cuda_stages_then_cpu rows). The device runs the relayout and every stage
 * into the context's device result buffer, one chunk of destination rows at
 * a time, and each chunk is copied to the host while the next chunk's kernel
 * runs. For this call `opt->source_pinned` describes the HOST buffer (the
 * destination): 1 pinned (direct DMA), 0 pageable (pinned ring, worker
 * threads copy each slot out), -1 probe; `host_stages` must be 0 or -1. The
 * source is ordered after `opt->caller_stream` when `has_caller_stream` is
 * set (0 being the legacy null stream). Blocks until the
 * destination holds the result. */
int relx_execute_d2h(relx_ctx *ctx, const relx_bound *bound, const void *src, size_t src_bytes,
                     void *dst, size_t dst_bytes, const relx_options *opt, relx_report *report,
                     relx_err *err);

/* Device-resident relayout: `wire` is already in device memory (dense source
 * layout at boundary `wire_boundary`); run the relayout + stages
 * [wire_boundary, stages) into `dst` on `stream`, a hipStream_t where 0 is
 * HIP's legacy null stream, as the reference's wrappers take a null stream
 * (void *stream = nullptr). Asynchronous: returns after the launch. This is
 * the device half of relx_execute_h2d and the unit the kernel roofline is
 * measured on; it replaces the reference's kernel launch wrappers
 * reloc::cuda::* (libreloc/include/reloc/CudaKernels.h:28-122).
 * A program on the element-wise kernel reports a stage channel outside its
 * parameters through a status flag of its own; the next
 * relx_ctx_synchronize waits for such launches and fails with
 * "channel_out_of_range" once for all of them. */
int relx_relayout_device(relx_ctx *ctx, const relx_bound *bound, int wire_boundary,
                         const void *wire, void *dst, uint64_t stream, relx_err *err);

/* Indexed plans with a device-resident table: gather the bound's selected
 * rows of `table` (table_rows x row_elements source elements, dense) into
 * `dst` (dense selected rows of the result type), the plan's cast fused into
 * the gather, on `stream` (0 = HIP's legacy null stream). Asynchronous:
 * returns after the launch. The reference executes indexed plans only from
 * host memory, gathering on the CPU (libreloc/src/Dispatch.cpp:1269-1283,
 * 1397-1404); this is the device form of its index_select. Errors:
 * "plan_mismatch" (not an indexed plan), "insufficient_capacity",
 * "invalid_view" (null or misaligned buffers). */
int relx_index_select_device(relx_ctx *ctx, const relx_bound *bound, const void *table,
                             size_t table_bytes, void *dst, size_t dst_bytes, uint64_t stream,
                             relx_err *err);

/* Apply a bound plan's leading `host_stages` stages to a dense source on the
 * host (the staging-side transform of relx_execute_h2d), writing the wire
 * at that boundary. Used by callers that pre-stage. */
int relx_host_stage(const relx_bound *bound, int host_stages, const void *src, void *wire,
                    int threads, relx_err *err);

/* Host-side check of every kernel launch relx_execute_h2d would make for
 * this bound plan with the wire at `wire_boundary` and chunks of
 * `chunk_bytes` (0 = the default), and of relx_relayout_device's launch:
 * every access inside the wire and the result, 16-byte vectors aligned,
 * every parameter index inside its table. Runs on the CPU with no device.
 * `launches` (optional) receives the number checked. The same check runs
 * before every launch when the environment variable RELX_VERIFY_LAUNCHES is
 * set. No counterpart in the reference: it backs this library's tests. */
int relx_verify_launches(const relx_bound *bound, int wire_boundary, int64_t chunk_bytes,
                         int64_t *launches, relx_err *err);

/* Block until every call on the context has completed: its own streams, and
 * the device-resident launches that report a status (see
 * relx_relayout_device). Fails with "channel_out_of_range" when one of those
 * launches selected a channel outside its parameters. Then releases scratch
 * beyond the context's max_retained_bytes. */
int relx_ctx_synchronize(relx_ctx *ctx, relx_err *err);

/* Kernel timing of a context's blocking uploads (relx_execute_h2d and
 * relx_execute_group_h2d without no_wait): when enabled, each chunk's
 * relayout launches are bracketed by timing events on the copy stream they
 * run on (the first completes when the chunk's copy has landed), and the
 * elapsed times are summed when the call completes. Enabling resets the
 * sums. The device-side counterpart of the reference's trace ranges
 * (libreloc/src/Trace.h:15-39); no other counterpart. */
typedef struct relx_kernel_times {
  int64_t calls;    /* timed calls */
  int64_t chunks;   /* timed chunks (one event pair each) */
  int64_t launches; /* kernel launches inside them */
  double ms;        /* summed elapsed milliseconds */
} relx_kernel_times;
int relx_ctx_time_kernels(relx_ctx *ctx, int enable, relx_err *err);
int relx_ctx_kernel_times(relx_ctx *ctx, relx_kernel_times *out, relx_err *err);

/* Pinned host memory helpers (hipHostMalloc / hipHostFree). */
int relx_host_alloc(size_t bytes, void **out, relx_err *err);
int relx_host_free(void *p);

/* Measured pinned H2D ceiling (GB/s): `bytes` per copy, `iters` copies after
 * a warmup, best of `rounds` (restates bench/rtrack/multigpu_h2d.cu:46-91). */
double relx_measure_h2d(int device, size_t bytes, int iters, int rounds);

/* The same measurement device -> host into pinned memory: the ceiling the
 * D2H direction of relx_execute_d2h is reported against. */
double relx_measure_d2h(int device, size_t bytes, int iters, int rounds);

/* Measured HBM copy ceiling (GB/s of bytes read + written): a 16-byte vector
 * copy kernel of `bytes` (wave-contiguous vectors streamed past the caches,
 * one and then two per lane, the faster form counting) over buffer pairs
 * spanning at least 2 GiB (eight times the Infinity Cache), `iters` copies
 * but at least one per pair, best of `rounds`. The
 * device-side counterpart of relx_measure_h2d; the reference measures its
 * copy kernel the same way (copyF32Vec4Kernel, libreloc/cuda/CudaKernels.cu:30-36).
 * Returns -1 on failure. */
double relx_measure_copy(int device, size_t bytes, int iters, int rounds);

#ifdef __cplusplus
}
#endif

#endif /* RELX_H */
