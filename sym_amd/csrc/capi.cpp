// capi.cpp - extern "C" entry points of librelx (declared in include/relx.h).
// No exception crosses this boundary: every failure becomes a status code and
// a filled relx_err.
#include "../../include/relx.h"

#include <cstdio>
#include <cstring>

#include "runtime.h"

namespace relx {
void execute_members(Context &ctx, int n, BoundHandle *const *bounds, const void *const *srcs,
                     const size_t *src_bytes, void *const *dsts, const size_t *dst_bytes,
                     const relx_options &opt, relx_report *reports, relx_report *total,
                     Completion *comp);
std::unique_ptr<Context> make_context(int device, int64_t max_retained);
bool drain(Context &ctx);
void destroy_context(Context &ctx);
void relayout_device(Context &ctx, BoundHandle &h, uint32_t k, const void *wire, void *dst,
                     hipStream_t stream);
void resolve_checks(Context &ctx);
void execute_static(Context &ctx, BoundHandle &h, const void *src, size_t src_bytes, void *dst,
                    size_t dst_bytes, const relx_options &opt, relx_report *report);
uint64_t view_span_bytes(const relx_view &v, const std::string &role);
uint64_t validate_transfer_source(const BoundHandle &h, const relx_view &src, int direction);
void validate_transfer(const BoundHandle &h, const relx_view &src, const relx_view &dst,
                       int direction, uint64_t &src_span, uint64_t &dst_bytes);
void execute_transfer(Context &ctx, BoundHandle &h, const relx_view &src, const relx_view &dst,
                      int direction, const relx_options &opt, relx_report *report);
int pointer_device(const void *p);
double measure_h2d(int device, size_t bytes, int iters, int rounds);
double measure_copy(int device, size_t bytes, int iters, int rounds, bool d2h);
} // namespace relx

struct relx_plan {
  std::unique_ptr<relx::Plan> plan;
};
struct relx_bound {
  relx::BoundHandle h;
};
struct relx_ctx {
  std::shared_ptr<relx::Context> ctx;
};

struct relx_completion {
  relx::Completion c;
  // The outcome of a group the device failed, kept for later queries and
  // waits (reference Completion's stored TransferOutcome).
  bool failed = false;
  std::string code, message;
  int completion = 0;
};

namespace {

void set_err(relx_err *err, const std::string &code, const std::string &msg, int64_t offset = -1,
             int completion = RELX_NOT_LAUNCHED) {
  if (!err)
    return;
  std::memset(err, 0, sizeof(*err));
  std::snprintf(err->code, sizeof(err->code), "%s", code.c_str());
  std::snprintf(err->message, sizeof(err->message), "%s", msg.c_str());
  err->offset = offset;
  err->completion = completion;
}

void clear_err(relx_err *err) {
  if (err) {
    std::memset(err, 0, sizeof(*err));
    err->offset = -1;
  }
}

template <class F> int guarded(relx_err *err, F &&fn) {
  try {
    clear_err(err);
    fn();
    return RELX_OK;
  } catch (const relx::Error &e) {
    set_err(err, e.code, e.message, e.offset);
  } catch (const std::bad_alloc &) {
    set_err(err, "out_of_memory", "host allocation failed");
  } catch (const std::exception &e) {
    set_err(err, "internal_error", e.what());
  }
  return RELX_ERROR;
}

// Errors raised before a call enqueues any work.
bool before_launch(const char *code) {
  static const char *const codes[] = {"invalid_argument", "invalid_options", "insufficient_capacity",
                                      "invalid_view",     "plan_mismatch",   "resources_closed",
                                      "unsupported_layout", "device_mismatch", "backend_mismatch",
                                      "invalid_boundary"};
  for (const char *c : codes)
    if (std::strcmp(code, c) == 0)
      return true;
  return false;
}

// After a failed call: drain what was enqueued. When completion cannot be
// proven the context is quarantined and the error becomes
// "completion_unknown" with an unknown completion (reference
// libreloc/src/DispatchResources.cpp:652-666); otherwise the call's own
// error stands, with a known completion (complete, or not launched for
// errors raised before any work was enqueued).
void after_failure(relx::Context &c, relx_err *err) {
  ++c.failures;
  if (!relx::drain(c)) {
    c.quarantined = true;
    if (err) {
      const std::string cause = std::string(err->code) + ": " + err->message;
      set_err(err, "completion_unknown",
              "the call failed (" + cause + ") and its context could not be drained; quarantined",
              -1, RELX_UNKNOWN);
    }
    return;
  }
  if (err)
    err->completion = before_launch(err->code) ? RELX_NOT_LAUNCHED : RELX_COMPLETE;
}

} // namespace

extern "C" {

const char *relx_version(void) {
  return "librelx 0.1 (gfx950; wire format v0 layout, v1 typed)";
}

int relx_wire_version(const uint8_t *blob, size_t n) {
  return blob ? relx::peek_wire_version(blob, n) : -1;
}

int relx_plan_load(const uint8_t *blob, size_t n, relx_plan **out, relx_err *err) {
  return guarded(err, [&] {
    if (!blob || !out)
      throw relx::Error("invalid_argument", "null blob or output");
    auto p = relx::decode(blob, n);
    *out = new relx_plan{std::move(p)};
  });
}

int relx_plan_is_typed(const relx_plan *plan) { return plan && plan->plan->version == 1; }

int relx_plan_version(const relx_plan *plan) {
  return plan ? static_cast<int>(plan->plan->version) : -1;
}

int relx_plan_symbol_count(const relx_plan *plan) {
  return plan ? static_cast<int>(plan->plan->symbols.size()) : 0;
}

const char *relx_plan_symbol(const relx_plan *plan, int i) {
  if (!plan || i < 0 || i >= static_cast<int>(plan->plan->symbols.size()))
    return nullptr;
  return plan->plan->symbols[static_cast<size_t>(i)].c_str();
}

void relx_plan_free(relx_plan *plan) { delete plan; }

int relx_plan_stage_count(const relx_plan *plan) {
  return plan ? static_cast<int>(plan->plan->stages.size()) : 0;
}

int relx_plan_stage(const relx_plan *plan, int i, relx_plan_stage_info *out) {
  if (!plan || !out || i < 0 || i >= static_cast<int>(plan->plan->stages.size()))
    return RELX_ERROR;
  const relx::PlanStage &s = plan->plan->stages[static_cast<size_t>(i)];
  out->transform = s.transform;
  out->policy = s.policy;
  out->in_kind = s.in.kind;
  out->in_bits = static_cast<int>(s.in.bits);
  out->in_signedness = s.in_sign;
  out->out_kind = s.out.kind;
  out->out_bits = static_cast<int>(s.out.bits);
  out->out_signedness = s.out_sign;
  out->rank = static_cast<int>(s.shape.size());
  out->axis = s.axis;
  out->has_channel = s.has_channel ? 1 : 0;
  out->scale_kind = s.scale.kind;
  out->zero_point_kind = s.zero_point.kind;
  return RELX_OK;
}

int relx_plan_fill_count(const relx_plan *plan) {
  return plan ? static_cast<int>(plan->plan->fills.size()) : 0;
}

int relx_plan_parameter(const relx_plan *plan, int i, const char **name, int *kind, int *bits,
                        int *rank, int *stage, int *role) {
  if (!plan)
    return 0;
  int n = 0;
  std::vector<const std::string *> seen;
  const auto &stages = plan->plan->stages;
  for (size_t k = 0; k < stages.size(); ++k) {
    const relx::StageParam *params[2] = {&stages[k].scale, &stages[k].zero_point};
    for (int r = 0; r < 2; ++r) {
      const relx::StageParam &p = *params[r];
      if (p.kind != relx::kParamBinding)
        continue;
      bool dup = false;
      for (const std::string *s : seen)
        dup = dup || *s == p.name;
      if (dup)
        continue;
      seen.push_back(&p.name);
      if (n == i) {
        if (name)
          *name = p.name.c_str();
        if (kind)
          *kind = p.type.kind;
        if (bits)
          *bits = static_cast<int>(p.type.bits);
        if (rank)
          *rank = p.rank;
        if (stage)
          *stage = static_cast<int>(k);
        if (role)
          *role = r;
      }
      ++n;
    }
  }
  return n;
}

int relx_bind(const relx_plan *plan, const char *const *sym_names, const int64_t *sym_values,
              int nsym, const relx_param *params, int nparam, relx_bound **out,
              relx_err *err) {
  return guarded(err, [&] {
    if (!plan || !out)
      throw relx::Error("invalid_argument", "null plan or output");
    std::map<std::string, int64_t> syms;
    for (int i = 0; i < nsym; ++i)
      syms[sym_names[i]] = sym_values[i];
    std::map<std::string, relx::ParamValue> pv;
    for (int i = 0; i < nparam; ++i) {
      const relx_param &p = params[i];
      relx::ParamValue v;
      v.type.kind = static_cast<uint8_t>(p.kind);
      v.type.bits = static_cast<uint32_t>(p.bits);
      if (p.rank == 1)
        v.extents.push_back(p.length);
      else if (p.rank != 0)
        throw relx::Error("bind_error", "parameter rank must be 0 or 1");
      const auto *d = static_cast<const uint8_t *>(p.data);
      if (p.nbytes && !d)
        throw relx::Error("bind_error", "parameter data is null");
      v.bytes.assign(d, d + p.nbytes);
      pv[p.name] = std::move(v);
    }
    auto b = new relx_bound;
    try {
      b->h.bound = relx::bind(*plan->plan, syms, pv);
      if (b->h.bound->typed)
        relx::prepare_stages(*b->h.bound, b->h.prep);
      // Build the default device program now so unsupported plans fail here.
      (void)b->h.program(0);
    } catch (...) {
      delete b;
      throw;
    }
    *out = b;
  });
}

int relx_bind_indexed(const relx_plan *plan, const char *const *sym_names,
                      const int64_t *sym_values, int nsym, int index_kind, int index_bits,
                      const int64_t *index_extents, int index_rank, const void *index_data,
                      size_t index_bytes, relx_bound **out, relx_err *err) {
  return guarded(err, [&] {
    if (!plan || !out)
      throw relx::Error("invalid_argument", "null plan or output");
    if (index_rank < 0 || (index_rank > 0 && !index_extents))
      throw relx::Error("bind_error", "index operand extents are missing");
    std::map<std::string, int64_t> syms;
    for (int i = 0; i < nsym; ++i)
      syms[sym_names[i]] = sym_values[i];
    relx::DType t;
    t.kind = static_cast<uint8_t>(index_kind);
    t.bits = static_cast<uint32_t>(index_bits);
    const std::vector<int64_t> ext(index_extents, index_extents + index_rank);
    auto b = new relx_bound;
    try {
      b->h.bound = relx::bind_indexed(*plan->plan, syms, t, ext, index_data, index_bytes);
      relx::prepare_stages(*b->h.bound, b->h.prep);
      (void)b->h.program(0);
    } catch (...) {
      delete b;
      throw;
    }
    *out = b;
  });
}

void relx_bound_free(relx_bound *bound) { delete bound; }

int relx_bound_query(const relx_bound *bound, relx_bound_info *out) {
  if (!bound || !out)
    return RELX_ERROR;
  std::memset(out, 0, sizeof(*out));
  const relx::Bound &b = *bound->h.bound;
  const relx::BoundLayout &L = b.layout;
  out->typed = b.typed;
  out->rank = static_cast<int>(L.extents.size());
  for (int i = 0; i < out->rank && i < RELX_MAX_RANK; ++i) {
    out->extents[i] = L.extents[static_cast<size_t>(i)];
    out->src_strides[i] = L.src_strides[static_cast<size_t>(i)];
    out->dst_strides[i] = L.dst_strides[static_cast<size_t>(i)];
  }
  for (const relx::BoundPad &p : L.pads)
    if (p.axis < RELX_MAX_RANK) {
      out->pad_lo[p.axis] = p.lo;
      out->pad_hi[p.axis] = p.hi;
    }
  out->element_size = static_cast<int>(L.element_size);
  out->total_bytes = L.total_bytes;
  out->source_bytes = b.source_bytes;
  out->destination_bytes = b.typed ? b.destination_bytes : L.total_bytes;
  out->parameter_bytes = b.parameter_bytes;
  out->stages = static_cast<int>(b.stages.size());
  for (size_t i = 0; i < b.bytes_at.size() && i <= RELX_MAX_STAGES; ++i)
    out->bytes_at[i] = b.bytes_at[i];
  out->source_width = static_cast<int>(b.typed ? b.source_type.width() : L.element_size);
  out->result_width = static_cast<int>(L.element_size);
  out->source_rank = static_cast<int>(b.source_extents.size());
  for (int i = 0; i < out->source_rank && i < RELX_MAX_RANK; ++i)
    out->source_extents[i] = b.source_extents[static_cast<size_t>(i)];
  out->result_rank = static_cast<int>(b.result_extents.size());
  for (int i = 0; i < out->result_rank && i < RELX_MAX_RANK; ++i)
    out->result_extents[i] = b.result_extents[static_cast<size_t>(i)];
  out->host_stages_max = 0;
  for (const relx::HostStage &st : bound->h.prep.stages) {
    if (st.mode != relx::kChanNone)
      break;
    ++out->host_stages_max;
  }
  out->host_stages_auto = static_cast<int>(relx::auto_host_stages(bound->h));
  out->indexed = b.indexed ? 1 : 0;
  out->table_rows = b.table_rows;
  out->row_elements = b.row_elements;
  out->table_bytes = b.table_bytes;
  out->index_count = static_cast<int64_t>(b.indices.size());
  {
    int64_t elems = 1;
    for (int64_t e : b.source_extents)
      elems *= e;
    const auto &st = bound->h.prep.stages;
    for (size_t k = 0; k <= st.size() && k <= RELX_MAX_STAGES; ++k)
      out->wire_bytes_at[k] =
          elems * (k == 0 ? static_cast<int64_t>(out->source_width) : st[k - 1].out_width);
  }
  try {
    const relx::DeviceProgram &dp = const_cast<relx::BoundHandle &>(bound->h).program(0);
    std::snprintf(out->kernel, sizeof(out->kernel), "%s", dp.kernel);
    if (dp.family == relx::kFamTranspose) {
      out->transpose_tile_q = static_cast<int>(dp.base.t_wq);
      out->transpose_tile_c = static_cast<int>(dp.base.t_wc);
      const std::vector<relx::KArgs> ls = relx::axis_launches(dp, -1, 0, 0);
      int tiles = 0, rows = 0;
      for (const relx::KArgs &a : ls)
        if (!a.edge_box) {
          ++tiles;
          rows += (a.t_flags & relx::kTileRowChannel) ? 1 : 0;
        }
      out->transpose_row_params = tiles > 0 && rows == tiles ? 1 : 0;
    }
    if (dp.family == relx::kFamPermute) {
      const std::vector<relx::KArgs> ls = relx::axis_launches(dp, -1, 0, 0);
      out->permute_direct = ls.empty() ? 0 : 1;
      for (const relx::KArgs &a : ls)
        if (!a.p_direct)
          out->permute_direct = 0;
    }
    if (!b.typed)
      out->source_bytes = dp.wire_elems * L.element_size;
  } catch (...) {
    std::snprintf(out->kernel, sizeof(out->kernel), "unavailable");
  }
  return RELX_OK;
}

int relx_ctx_create(int device, int64_t max_retained_bytes, relx_ctx **out, relx_err *err) {
  return guarded(err, [&] {
    if (!out)
      throw relx::Error("invalid_argument", "null output");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
      throw relx::Error("backend_failure", "no HIP device is visible");
    if (device < 0 || device >= n)
      throw relx::Error("device_mismatch", "device " + std::to_string(device) + " out of range");
    *out = new relx_ctx{relx::make_context(device, max_retained_bytes)};
  });
}

int relx_ctx_close(relx_ctx *ctx, relx_err *err) {
  return guarded(err, [&] {
    if (!ctx)
      return;
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    if (!relx::drain(*ctx->ctx)) {
      // Completion unknown: keep every resource for the process lifetime.
      ctx->ctx->quarantined = true;
      ctx->ctx->closed = true;
      throw relx::Error("completion_unknown", "context could not be drained; quarantined");
    }
    relx::destroy_context(*ctx->ctx);
    ctx->ctx->closed = true;
  }) == RELX_OK
             ? (delete ctx, RELX_OK)
             : RELX_ERROR;
}

int relx_ctx_stats_get(const relx_ctx *ctx, relx_ctx_stats *out) {
  if (!ctx || !out)
    return RELX_ERROR;
  relx::Context &c = *ctx->ctx;
  std::lock_guard<std::mutex> g(c.mu);
  out->pinned_bytes = static_cast<int64_t>(c.slots.size() * c.slot_bytes);
  out->device_bytes = static_cast<int64_t>(c.wire_cap);
  out->calls = c.calls;
  out->failures = c.failures;
  out->quarantined = c.quarantined ? 1 : 0;
  return RELX_OK;
}

static int run_group(relx_ctx *ctx, int n, const relx_bound *const *bounds,
                     const void *const *srcs, const size_t *src_bytes, void *const *dsts,
                     const size_t *dst_bytes, const relx_options *opt, relx_report *reports,
                     relx_report *total, relx_err *err, relx_completion *comp = nullptr) {
  if (!ctx) {
    set_err(err, "invalid_argument", "null context");
    return RELX_ERROR;
  }
  relx::Context &c = *ctx->ctx;
  std::lock_guard<std::mutex> g(c.mu);
  if (c.closed || c.quarantined) {
    set_err(err, "resources_closed", "context is closed or quarantined");
    return RELX_ERROR;
  }
  relx_options o{};
  o.host_stages = -1;
  o.source_pinned = -1;
  if (opt)
    o = *opt;
  ++c.calls;
  const int rc = guarded(err, [&] {
    if (n < 1 || n > 256)
      throw relx::Error("invalid_options", "a group holds 1..256 members");
    std::vector<relx::BoundHandle *> hs;
    for (int i = 0; i < n; ++i) {
      if (!bounds[i])
        throw relx::Error("invalid_argument", "null bound plan");
      hs.push_back(const_cast<relx::BoundHandle *>(&bounds[i]->h));
    }
    relx::execute_members(c, n, hs.data(), srcs, src_bytes, dsts, dst_bytes, o, reports, total,
                          comp ? &comp->c : nullptr);
  });
  if (rc != RELX_OK)
    after_failure(c, err);
  return rc;
}

int relx_execute_h2d(relx_ctx *ctx, const relx_bound *bound, const void *src, size_t src_bytes,
                     void *dst, size_t dst_bytes, const relx_options *opt, relx_report *report,
                     relx_err *err) {
  return run_group(ctx, 1, &bound, &src, &src_bytes, &dst, &dst_bytes, opt, report, nullptr,
                   err);
}

int relx_execute_group_h2d(relx_ctx *ctx, int n, const relx_bound *const *bounds,
                           const void *const *srcs, const size_t *src_bytes, void *const *dsts,
                           const size_t *dst_bytes, const relx_options *opt,
                           relx_report *reports, relx_report *total, relx_err *err) {
  return run_group(ctx, n, bounds, srcs, src_bytes, dsts, dst_bytes, opt, reports, total, err);
}

int relx_submit_group_h2d(relx_ctx *ctx, int n, const relx_bound *const *bounds,
                          const void *const *srcs, const size_t *src_bytes, void *const *dsts,
                          const size_t *dst_bytes, const relx_options *opt, relx_report *reports,
                          relx_report *total, relx_completion **out, relx_err *err) {
  if (!ctx || !out) {
    set_err(err, "invalid_argument", "null context or output");
    return RELX_ERROR;
  }
  auto *comp = new relx_completion{};
  comp->c.ctx = ctx->ctx;
  {
    relx::DeviceScope scope(ctx->ctx->device);
    if (hipEventCreateWithFlags(&comp->c.ev, hipEventDisableTiming) != hipSuccess) {
      delete comp;
      set_err(err, "backend_failure", "hipEventCreateWithFlags failed");
      return RELX_ERROR;
    }
  }
  const int rc =
      run_group(ctx, n, bounds, srcs, src_bytes, dsts, dst_bytes, opt, reports, total, err, comp);
  if (rc != RELX_OK) {
    relx_completion_free(comp);
    return rc;
  }
  *out = comp;
  return RELX_OK;
}

namespace {

// A submitted group the device failed: drain the context; when completion
// cannot be proven the context is quarantined and the outcome is
// "completion_unknown", else the device's error with a known completion
// (reference Completion, libreloc/src/DispatchResources.cpp:325-361). The
// outcome is kept for every later query and wait.
int fail_completion(relx_completion *c, const char *what, hipError_t e, relx_err *err) {
  if (!c->failed) {
    relx::Context &ctx = *c->c.ctx;
    std::lock_guard<std::mutex> g(ctx.mu);
    ++ctx.failures;
    c->failed = true;
    if (relx::drain(ctx)) {
      c->code = "backend_failure";
      c->message = std::string(what) + ": " + hipGetErrorString(e);
      c->completion = RELX_COMPLETE;
    } else {
      ctx.quarantined = true;
      c->code = "completion_unknown";
      c->message = std::string("asynchronous group failed (") + what + ": " + hipGetErrorString(e) +
                   ") and the context could not be drained; quarantined";
      c->completion = RELX_UNKNOWN;
    }
  }
  set_err(err, c->code, c->message, -1, c->completion);
  return RELX_ERROR;
}

} // namespace

int relx_completion_query(relx_completion *c, int *done, relx_err *err) {
  if (c && c->failed)
    return fail_completion(c, "", hipSuccess, err);
  hipError_t failed = hipSuccess;
  const int rc = guarded(err, [&] {
    if (!c || !done)
      throw relx::Error("invalid_argument", "null argument");
    relx::DeviceScope scope(c->c.ctx->device);
    const hipError_t e = hipEventQuery(c->c.ev);
    if (e != hipSuccess && e != hipErrorNotReady) {
      failed = e;
      return;
    }
    *done = e == hipSuccess ? 1 : 0;
    if (*done)
      relx::completion_check(c->c); // reports a channel error once complete
  });
  return failed != hipSuccess ? fail_completion(c, "hipEventQuery", failed, err) : rc;
}

int relx_completion_wait(relx_completion *c, relx_err *err) {
  if (c && c->failed)
    return fail_completion(c, "", hipSuccess, err);
  hipError_t failed = hipSuccess;
  const int rc = guarded(err, [&] {
    if (!c)
      throw relx::Error("invalid_argument", "null completion");
    relx::DeviceScope scope(c->c.ctx->device);
    const hipError_t e = hipEventSynchronize(c->c.ev);
    if (e != hipSuccess) {
      failed = e;
      return;
    }
    relx::completion_check(c->c);
  });
  return failed != hipSuccess ? fail_completion(c, "hipEventSynchronize", failed, err) : rc;
}

int relx_completion_wait_stream(relx_completion *c, uint64_t stream, relx_err *err) {
  if (c && c->failed)
    return fail_completion(c, "", hipSuccess, err);
  return guarded(err, [&] {
    if (!c)
      throw relx::Error("invalid_argument", "null completion");
    relx::DeviceScope scope(c->c.ctx->device);
    const hipError_t e = hipStreamWaitEvent(reinterpret_cast<hipStream_t>(stream), c->c.ev, 0);
    if (e != hipSuccess)
      throw relx::Error("backend_failure", std::string("hipStreamWaitEvent: ") + hipGetErrorString(e));
  });
}

void relx_completion_free(relx_completion *c) {
  if (!c)
    return;
  {
    relx::DeviceScope scope(c->c.ctx->device);
    if (c->c.ev) {
      (void)hipEventSynchronize(c->c.ev); // abandoning a handle drains its work
      (void)hipEventDestroy(c->c.ev);
    }
  }
  delete c;
}

int relx_execute_d2h(relx_ctx *ctx, const relx_bound *bound, const void *src, size_t src_bytes,
                     void *dst, size_t dst_bytes, const relx_options *opt, relx_report *report,
                     relx_err *err) {
  if (!ctx) {
    set_err(err, "invalid_argument", "null context");
    return RELX_ERROR;
  }
  relx::Context &c = *ctx->ctx;
  std::lock_guard<std::mutex> g(c.mu);
  if (c.closed || c.quarantined) {
    set_err(err, "resources_closed", "context is closed or quarantined");
    return RELX_ERROR;
  }
  relx_options o{};
  o.host_stages = -1;
  o.source_pinned = -1;
  if (opt)
    o = *opt;
  ++c.calls;
  const int rc = guarded(err, [&] {
    if (!bound)
      throw relx::Error("invalid_argument", "null bound plan");
    if (o.host_stages > 0)
      throw relx::Error("invalid_options", "device-to-host runs every stage on the device");
    relx::execute_d2h(c, const_cast<relx::BoundHandle &>(bound->h), src, src_bytes, dst,
                      dst_bytes, o, report);
  });
  if (rc != RELX_OK)
    after_failure(c, err);
  return rc;
}

int relx_execute_h2d_static(relx_ctx *ctx, const relx_bound *bound, const void *src,
                            size_t src_bytes, void *dst, size_t dst_bytes, const relx_options *opt,
                            relx_report *report, relx_err *err) {
  if (!ctx) {
    set_err(err, "invalid_argument", "null context");
    return RELX_ERROR;
  }
  relx::Context &c = *ctx->ctx;
  std::lock_guard<std::mutex> g(c.mu);
  if (c.closed || c.quarantined) {
    set_err(err, "resources_closed", "context is closed or quarantined");
    return RELX_ERROR;
  }
  relx_options o{};
  o.host_stages = -1;
  o.source_pinned = -1;
  if (opt)
    o = *opt;
  ++c.calls;
  const int rc = guarded(err, [&] {
    if (!bound)
      throw relx::Error("invalid_argument", "null bound plan");
    relx::execute_static(c, const_cast<relx::BoundHandle &>(bound->h), src, src_bytes, dst,
                         dst_bytes, o, report);
  });
  if (rc != RELX_OK)
    after_failure(c, err);
  return rc;
}

int relx_view_span_bytes(const relx_view *view, const char *role, uint64_t *span, relx_err *err) {
  return guarded(err, [&] {
    if (!view || !span)
      throw relx::Error("invalid_argument", "null view or output");
    *span = relx::view_span_bytes(*view, role ? role : "view");
  });
}

int relx_validate_transfer_source(const relx_bound *bound, const relx_view *source,
                                  int direction, uint64_t *span, relx_err *err) {
  return guarded(err, [&] {
    if (!bound || !source)
      throw relx::Error("invalid_argument", "null bound plan or view");
    if (direction != RELX_H2D && direction != RELX_D2H)
      throw relx::Error("invalid_options", "direction must be host-to-device or device-to-host");
    const uint64_t s = relx::validate_transfer_source(bound->h, *source, direction);
    if (span)
      *span = s;
  });
}

int relx_validate_transfer(const relx_bound *bound, const relx_view *source,
                           const relx_view *destination, int direction, uint64_t *source_span,
                           uint64_t *destination_bytes, relx_err *err) {
  return guarded(err, [&] {
    if (!bound || !source || !destination)
      throw relx::Error("invalid_argument", "null bound plan or view");
    uint64_t s = 0, d = 0;
    relx::validate_transfer(bound->h, *source, *destination, direction, s, d);
    if (source_span)
      *source_span = s;
    if (destination_bytes)
      *destination_bytes = d;
  });
}

int relx_execute_transfer(relx_ctx *ctx, const relx_bound *bound, const relx_view *source,
                          const relx_view *destination, int direction, const relx_options *opt,
                          relx_report *report, relx_err *err) {
  if (!ctx) {
    set_err(err, "invalid_argument", "null context");
    return RELX_ERROR;
  }
  relx::Context &c = *ctx->ctx;
  std::lock_guard<std::mutex> g(c.mu);
  if (c.closed || c.quarantined) {
    set_err(err, "resources_closed", "context is closed or quarantined");
    return RELX_ERROR;
  }
  relx_options o{};
  o.host_stages = -1;
  o.source_pinned = -1;
  if (opt)
    o = *opt;
  ++c.calls;
  const int rc = guarded(err, [&] {
    if (!bound || !source || !destination)
      throw relx::Error("invalid_argument", "null bound plan or view");
    relx::execute_transfer(c, const_cast<relx::BoundHandle &>(bound->h), *source, *destination,
                           direction, o, report);
  });
  if (rc != RELX_OK)
    after_failure(c, err);
  return rc;
}

int relx_pointer_device(const void *pointer, int *device, relx_err *err) {
  return guarded(err, [&] {
    if (!device)
      throw relx::Error("invalid_argument", "null output");
    if (!pointer)
      throw relx::Error("invalid_view", "pointer is null");
    *device = relx::pointer_device(pointer);
  });
}

int relx_relayout_device(relx_ctx *ctx, const relx_bound *bound, int wire_boundary,
                         const void *wire, void *dst, uint64_t stream, relx_err *err) {
  return guarded(err, [&] {
    if (!ctx || !bound || !wire || !dst)
      throw relx::Error("invalid_argument", "null argument");
    if (wire_boundary < 0)
      throw relx::Error("invalid_boundary", "negative wire boundary");
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    if (ctx->ctx->closed || ctx->ctx->quarantined)
      throw relx::Error("resources_closed", "context is closed or quarantined");
    relx::relayout_device(*ctx->ctx, const_cast<relx::BoundHandle &>(bound->h),
                          static_cast<uint32_t>(wire_boundary), wire, dst,
                          reinterpret_cast<hipStream_t>(stream));
  });
}

int relx_index_select_device(relx_ctx *ctx, const relx_bound *bound, const void *table,
                             size_t table_bytes, void *dst, size_t dst_bytes, uint64_t stream,
                             relx_err *err) {
  return guarded(err, [&] {
    if (!ctx || !bound)
      throw relx::Error("invalid_argument", "null argument");
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    if (ctx->ctx->closed || ctx->ctx->quarantined)
      throw relx::Error("resources_closed", "context is closed or quarantined");
    relx::index_select_device(*ctx->ctx, const_cast<relx::BoundHandle &>(bound->h), table,
                              table_bytes, dst, dst_bytes, reinterpret_cast<hipStream_t>(stream));
  });
}

int relx_verify_launches(const relx_bound *bound, int wire_boundary, int64_t chunk_bytes,
                         int64_t *launches, relx_err *err) {
  return guarded(err, [&] {
    if (!bound)
      throw relx::Error("invalid_argument", "null argument");
    if (wire_boundary < 0)
      throw relx::Error("invalid_boundary", "negative wire boundary");
    const int64_t n = relx::verify_launches(const_cast<relx::BoundHandle &>(bound->h),
                                            static_cast<uint32_t>(wire_boundary), chunk_bytes);
    if (launches)
      *launches = n;
  });
}

int relx_host_stage(const relx_bound *bound, int host_stages, const void *src, void *wire,
                    int threads, relx_err *err) {
  return guarded(err, [&] {
    if (!bound || !src || !wire)
      throw relx::Error("invalid_argument", "null argument");
    const relx::BoundHandle &h = bound->h;
    if (!h.bound->typed && host_stages != 0)
      throw relx::Error("invalid_boundary", "layout plans have no stages");
    if (host_stages < 0 || host_stages > static_cast<int>(h.prep.stages.size()))
      throw relx::Error("invalid_boundary", "host stages outside the program");
    for (int j = 0; j < host_stages; ++j)
      if (h.prep.stages[static_cast<size_t>(j)].mode != relx::kChanNone)
        throw relx::Error("invalid_options", "host stages must be per-tensor stages");
    const uint32_t sw = h.bound->typed ? h.bound->source_type.width() : h.bound->layout.element_size;
    int64_t n = 1;
    if (h.bound->typed)
      for (int64_t e : h.bound->source_extents)
        n *= e;
    else
      n = const_cast<relx::BoundHandle &>(h).program(0).wire_elems;
    relx::Workers w(static_cast<unsigned>(threads > 0 ? threads : 1));
    if (h.bound->indexed) {
      const int64_t wout =
          host_stages ? h.prep.stages[static_cast<size_t>(host_stages - 1)].out_width : sw;
      w.parallel_for(n, int64_t{1} << 16, [&](int64_t a, int64_t b) {
        relx::host_gather(*h.bound, h.prep, static_cast<uint32_t>(host_stages), src,
                          static_cast<uint8_t *>(wire) + a * wout, a, b);
      });
      return;
    }
    w.parallel_for(n, int64_t{1} << 16, [&](int64_t a, int64_t b) {
      relx::host_transform(h.prep, static_cast<uint32_t>(host_stages), sw, src, wire, a, b);
    });
  });
}

int relx_ctx_synchronize(relx_ctx *ctx, relx_err *err) {
  return guarded(err, [&] {
    if (!ctx)
      throw relx::Error("invalid_argument", "null context");
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    if (!relx::drain(*ctx->ctx))
      throw relx::Error("backend_failure", "stream synchronize failed");
    relx::resolve_checks(*ctx->ctx);
    ctx->ctx->unsynced = false; // every call on the context has completed
    relx::trim_retained(*ctx->ctx);
  });
}

int relx_ctx_time_kernels(relx_ctx *ctx, int enable, relx_err *err) {
  return guarded(err, [&] {
    if (!ctx)
      throw relx::Error("invalid_argument", "null context");
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    ctx->ctx->time_kernels = enable != 0;
    ctx->ctx->kt = relx::KernelTimes{};
  });
}

int relx_ctx_kernel_times(relx_ctx *ctx, relx_kernel_times *out, relx_err *err) {
  return guarded(err, [&] {
    if (!ctx || !out)
      throw relx::Error("invalid_argument", "null argument");
    std::lock_guard<std::mutex> g(ctx->ctx->mu);
    const relx::KernelTimes &k = ctx->ctx->kt;
    out->calls = k.calls;
    out->chunks = k.chunks;
    out->launches = k.launches;
    out->ms = k.ms;
  });
}

int relx_host_alloc(size_t bytes, void **out, relx_err *err) {
  return guarded(err, [&] {
    if (!out)
      throw relx::Error("invalid_argument", "null output");
    if (hipHostMalloc(out, bytes, hipHostMallocDefault) != hipSuccess)
      throw relx::Error("out_of_memory", "hipHostMalloc failed");
  });
}

int relx_host_free(void *p) { return hipHostFree(p) == hipSuccess ? RELX_OK : RELX_ERROR; }

double relx_measure_h2d(int device, size_t bytes, int iters, int rounds) {
  try {
    return relx::measure_h2d(device, bytes, iters, rounds);
  } catch (...) {
    return -1.0;
  }
}

double relx_measure_copy(int device, size_t bytes, int iters, int rounds) {
  try {
    return relx::measure_device_copy(device, bytes, iters, rounds);
  } catch (...) {
    return -1.0;
  }
}

double relx_measure_d2h(int device, size_t bytes, int iters, int rounds) {
  try {
    return relx::measure_copy(device, bytes, iters, rounds, true);
  } catch (...) {
    return -1.0;
  }
}

} // extern "C"
