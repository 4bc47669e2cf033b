// transfer.cpp - validated layout transfers: the buffer views a framework
// hands the library, the proofs that a bound plan's accesses fit them, and
// the forward transfer over the upload and download pipelines.
//
// Role of the reference's Transfer.cpp (libreloc/src/Transfer.cpp:65-279,
// 493-544) and its Python surface (libreloc/python/PyTransfer.cpp:82-461).
// The admitted views, the checks and their reason codes are the reference's
// observable contract; the code is this library's.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "runtime.h"

namespace relx {

void execute_members(Context &ctx, int n, BoundHandle *const *bounds, const void *const *srcs,
                     const size_t *src_bytes, void *const *dsts, const size_t *dst_bytes,
                     const relx_options &opt, relx_report *reports, relx_report *total,
                     Completion *comp);

namespace {

bool mul_ok(int64_t a, int64_t b, int64_t &out) { return !__builtin_mul_overflow(a, b, &out); }
bool add_ok(int64_t a, int64_t b, int64_t &out) { return !__builtin_add_overflow(a, b, &out); }
bool mul_ok(uint64_t a, uint64_t b, uint64_t &out) { return !__builtin_mul_overflow(a, b, &out); }
bool add_ok(uint64_t a, uint64_t b, uint64_t &out) { return !__builtin_add_overflow(a, b, &out); }

[[noreturn]] void fail_view(const char *code, const std::string &role, const char *what) {
  throw Error(code, role + " " + what);
}

// Row-major dense: every axis of extent above one has the stride of the
// axes inside it.
bool dense(const relx_view &v) {
  int64_t expect = 1;
  for (int k = v.rank - 1; k >= 0; --k) {
    if (v.extents[k] != 1 && v.strides[k] != expect)
      return false;
    if (!mul_ok(expect, v.extents[k], expect))
      return false;
  }
  return true;
}

int64_t element_count(const int64_t *ext, int rank) {
  int64_t n = 1;
  for (int i = 0; i < rank; ++i)
    if (ext[i] < 1 || !mul_ok(n, ext[i], n))
      return -1;
  return n;
}

} // namespace

// Bytes from element 0 a view can address (libreloc/src/Transfer.cpp:65-113):
// nonempty extents, no negative, broadcast or overlapping strides, every
// step overflow-checked, and offset + span within the declared capacity.
uint64_t view_span_bytes(const relx_view &v, const std::string &role) {
  if (v.base == 0)
    fail_view("invalid_view", role, "base pointer is null");
  if (v.element_size == 0)
    fail_view("invalid_view", role, "element size is zero");
  if (v.rank < 1)
    fail_view("invalid_view", role, "has rank zero");
  if (v.rank > RELX_MAX_VIEW_RANK)
    fail_view("invalid_view", role, "has more axes than a view can describe");
  if (v.kind == RELX_KIND_DEVICE && v.device < 0)
    fail_view("invalid_view", role, "CUDA view lacks a device ordinal");
  if (v.kind == RELX_KIND_HOST && v.device >= 0)
    fail_view("invalid_view", role, "host view declares a CUDA device");
  if (v.kind != RELX_KIND_HOST && v.kind != RELX_KIND_DEVICE)
    fail_view("invalid_view", role, "has an unknown memory kind");
  std::vector<std::pair<int64_t, int64_t>> axes; // (stride, extent) of axes above one
  for (int k = 0; k < v.rank; ++k) {
    if (v.extents[k] < 1)
      fail_view("invalid_view", role, "has an extent below one");
    if (v.strides[k] < 0)
      fail_view("unsupported_layout", role, "has a negative stride");
    if (v.extents[k] == 1)
      continue;
    if (v.strides[k] == 0)
      fail_view("unsupported_layout", role, "broadcasts a stride of zero");
    axes.emplace_back(v.strides[k], v.extents[k]);
  }
  // Injective addressing: in stride order each stride must pass the farthest
  // element the smaller strides reach.
  std::sort(axes.begin(), axes.end());
  int64_t reach = 0;
  for (const auto &ax : axes) {
    if (ax.first <= reach)
      fail_view("unsupported_layout", role, "has overlapping strides");
    int64_t step = 0;
    if (!mul_ok(ax.second - 1, ax.first, step) || !add_ok(reach, step, reach))
      fail_view("integer_overflow", role, "span overflows");
  }
  uint64_t bytes = 0, last = 0;
  if (!mul_ok(static_cast<uint64_t>(reach) + 1, static_cast<uint64_t>(v.element_size), bytes) ||
      !add_ok(v.offset_bytes, bytes, last))
    fail_view("integer_overflow", role, "byte span overflows");
  if (last > v.capacity_bytes)
    throw Error("insufficient_capacity", role + " needs " + std::to_string(last) +
                                             " bytes from its allocation base but only " +
                                             std::to_string(v.capacity_bytes) + " are declared");
  return bytes;
}

// The bound plan's reads against the source view
// (libreloc/src/Transfer.cpp:138-184): a layout plan of the view's element
// size and element count whose farthest read lies inside the view's span.
uint64_t validate_transfer_source(const BoundHandle &h, const relx_view &src, int direction) {
  if (direction == RELX_H2D && src.kind == RELX_KIND_DEVICE)
    throw Error("direction_mismatch", "host-to-device source must be host memory");
  const uint64_t span = view_span_bytes(src, "source");
  const Bound &b = *h.bound;
  const BoundLayout &L = b.layout;
  if (L.extents.empty() || L.extents.size() != L.src_strides.size() ||
      L.extents.size() != L.dst_strides.size())
    throw Error("plan_mismatch", "bound plan has inconsistent axes");
  if (b.typed)
    throw Error("typed_unsupported", "bound plan is the layout of a typed plan; the layout-only "
                                     "transfer path cannot execute it");
  if (L.element_size == 0 || L.element_size != src.element_size)
    throw Error("plan_mismatch", "plan element size differs from the source view");
  const int64_t plan_elements = element_count(L.extents.data(), static_cast<int>(L.extents.size()));
  if (plan_elements < 0)
    throw Error("integer_overflow", "plan element count overflows");
  const int64_t view_elements = element_count(src.extents, src.rank);
  if (view_elements < 0)
    throw Error("integer_overflow", "source element count overflows");
  if (plan_elements != view_elements)
    throw Error("plan_mismatch", "plan relocates " + std::to_string(plan_elements) +
                                     " elements but the source view holds " +
                                     std::to_string(view_elements));
  int64_t far = 0;
  for (size_t k = 0; k < L.extents.size(); ++k) {
    if (L.src_strides[k] < 0)
      throw Error("plan_mismatch", "plan has a negative source stride");
    int64_t step = 0;
    if (!mul_ok(L.extents[k] - 1, L.src_strides[k], step) || !add_ok(far, step, far))
      throw Error("integer_overflow", "plan source reach overflows");
  }
  uint64_t need = 0;
  if (!mul_ok(static_cast<uint64_t>(far) + 1, static_cast<uint64_t>(L.element_size), need))
    throw Error("integer_overflow", "plan source footprint overflows");
  if (need > span)
    throw Error("plan_mismatch", "plan reads " + std::to_string(need) +
                                     " bytes beyond a source view spanning " +
                                     std::to_string(span));
  return span;
}

// Full validation with the destination (libreloc/src/Transfer.cpp:186-279):
// a CUDA view sits on the device end of its direction; the destination is
// dense, spans exactly the plan's footprint, and holds every padded write.
void validate_transfer(const BoundHandle &h, const relx_view &src, const relx_view &dst,
                       int direction, uint64_t &src_span, uint64_t &dst_bytes) {
  if (direction != RELX_H2D && direction != RELX_D2H)
    throw Error("invalid_options", "direction must be host-to-device or device-to-host");
  if (direction == RELX_H2D && src.kind == RELX_KIND_DEVICE)
    throw Error("direction_mismatch", "host-to-device source must be host memory");
  if (direction == RELX_D2H && dst.kind == RELX_KIND_DEVICE)
    throw Error("direction_mismatch", "device-to-host destination must be host memory");
  src_span = validate_transfer_source(h, src, direction);
  const uint64_t span = view_span_bytes(dst, "destination");
  const BoundLayout &L = h.bound->layout;
  if (L.element_size != dst.element_size)
    throw Error("plan_mismatch", "plan element size differs from the destination view");
  if (!dense(dst))
    throw Error("unsupported_layout", "destination view must be dense row-major");
  if (L.total_bytes <= 0)
    throw Error("plan_mismatch", "bound plan has no destination footprint");
  if (span != static_cast<uint64_t>(L.total_bytes))
    throw Error("plan_mismatch", "destination view spans " + std::to_string(span) +
                                     " bytes but the plan writes " +
                                     std::to_string(L.total_bytes));
  std::vector<int64_t> padded = L.extents;
  for (const BoundPad &p : L.pads) {
    if (p.axis < 0 || static_cast<size_t>(p.axis) >= padded.size() || p.lo < 0 || p.hi < 0)
      throw Error("plan_mismatch", "bound plan has an invalid pad region");
    if (!add_ok(padded[p.axis], p.lo, padded[p.axis]) ||
        !add_ok(padded[p.axis], p.hi, padded[p.axis]))
      throw Error("integer_overflow", "padded extent overflows");
  }
  int64_t far = 0;
  for (size_t k = 0; k < padded.size(); ++k) {
    if (L.dst_strides[k] < 0)
      throw Error("plan_mismatch", "plan has a negative destination stride");
    int64_t step = 0;
    if (!mul_ok(padded[k] - 1, L.dst_strides[k], step) || !add_ok(far, step, far))
      throw Error("integer_overflow", "plan destination reach overflows");
  }
  uint64_t need = 0;
  if (!mul_ok(static_cast<uint64_t>(far) + 1, static_cast<uint64_t>(L.element_size), need))
    throw Error("integer_overflow", "plan destination footprint overflows");
  if (need > static_cast<uint64_t>(L.total_bytes))
    throw Error("plan_mismatch", "plan writes beyond its declared destination footprint");
  dst_bytes = static_cast<uint64_t>(L.total_bytes);
}

// The forward transfer of a validated pair of views on `ctx`: host ->
// device through the upload pipeline, device -> host through the download
// pipeline. The plan reads its source from the view's element 0 and writes
// its dense result at the destination's element 0.
void execute_transfer(Context &ctx, BoundHandle &h, const relx_view &src, const relx_view &dst,
                      int direction, const relx_options &opt, relx_report *report) {
  uint64_t src_span = 0, dst_bytes = 0;
  validate_transfer(h, src, dst, direction, src_span, dst_bytes);
  if (src.kind == RELX_KIND_HOST && dst.kind == RELX_KIND_HOST)
    throw Error("backend_mismatch", "a host-to-host transfer runs on a host backend; this "
                                    "library moves data between host and device memory");
  const relx_view &dev = direction == RELX_H2D ? dst : src;
  if (dev.device != ctx.device)
    throw Error("device_mismatch", std::string(direction == RELX_H2D ? "destination" : "source") +
                                       " view is on device " + std::to_string(dev.device) +
                                       " but the context runs on device " +
                                       std::to_string(ctx.device));
  const void *s = reinterpret_cast<const void *>(src.base + src.offset_bytes);
  void *d = reinterpret_cast<void *>(dst.base + dst.offset_bytes);
  if (direction == RELX_H2D) {
    BoundHandle *hp = &h;
    const size_t sb = static_cast<size_t>(src_span), db = static_cast<size_t>(dst_bytes);
    execute_members(ctx, 1, &hp, &s, &sb, &d, &db, opt, report, nullptr, nullptr);
  } else {
    relx_options o = opt;
    o.host_stages = 0;
    execute_d2h(ctx, h, s, static_cast<size_t>(src_span), d, static_cast<size_t>(dst_bytes), o,
                report);
  }
}

// The device owning a pointer (libreloc/python/PyTransfer.cpp:291-306).
int pointer_device(const void *p) {
  hipPointerAttribute_t attr;
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    throw Error("invalid_view", std::string("pointer is not known to the HIP runtime: ") +
                                    hipGetErrorString(e));
  }
  if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged)
    throw Error("invalid_view", "pointer is not device memory");
  return attr.device;
}

} // namespace relx
