// indexed.cpp - execution of indexed (wire v2) plans: index_select along
// axis 0 with at most one cast (reference bindIndexed,
// libreloc/src/Bind.cpp:701-819; dispatch prepareIndexSelect,
// libreloc/src/Dispatch.cpp:1269-1283).
//
// Three paths:
//   upload  the host gathers the selected rows of a host table (through the
//           leading stages the staging applies) into the pinned ring, and the
//           device runs the rest of the plan on the dense selected rows
//           (runtime.cpp). The reference does the same gather on the host
//           and runs no part of such a plan on the GPU
//           (libreloc/src/Dispatch.cpp:1397-1404).
//   table   a long selection from a table no larger than the gathered rows
//           (table_upload_pays): the table itself crosses PCIe into the wire
//           arena and the device gathers from it (runtime.cpp).
//   device  a device-resident table: one gather kernel per launch box, with
//           the cast fused (k_gather.hip).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "index.h"
#include "runtime.h"

namespace relx {

namespace {

void hipcheck(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw Error("backend_failure", std::string(what) + ": " + hipGetErrorString(e));
}

bool verify_env() {
  static const bool on = [] {
    const char *v = std::getenv("RELX_VERIFY_LAUNCHES");
    return v && *v && std::strcmp(v, "0") != 0;
  }();
  return on;
}

} // namespace

const void *BoundHandle::device_indices(int device) {
  std::lock_guard<std::mutex> g(mu);
  auto it = dev_indices.find(device);
  if (it != dev_indices.end())
    return it->second;
  const Bound &b = *bound;
  const size_t n = b.indices.size();
  const bool narrow = b.table_rows <= INT32_MAX;
  std::vector<int32_t> i32;
  const void *host = b.indices.data();
  size_t bytes = n * sizeof(int64_t);
  if (narrow) {
    i32.assign(b.indices.begin(), b.indices.end());
    host = i32.data();
    bytes = n * sizeof(int32_t);
  }
  void *d = nullptr;
  hipcheck(hipMalloc(&d, std::max<size_t>(bytes, 4)), "hipMalloc(indices)");
  const hipError_t e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    hipcheck(e, "hipMemcpy(indices)");
  }
  dev_indices.emplace(device, d);
  return d;
}

GatherPlan gather_plan(const Bound &b, const void *table, const void *dst) {
  if (!b.indexed)
    throw Error("plan_mismatch", "not an indexed plan");
  const uint32_t sw = b.source_type.width(), rw = b.result_type.width();
  const uintptr_t t = reinterpret_cast<uintptr_t>(table), d = reinterpret_cast<uintptr_t>(dst);
  if (t % sw || d % rw)
    throw Error("invalid_view", "table and destination must be aligned to their element width");
  GatherPlan g;
  g.iw = b.table_rows <= INT32_MAX ? 4 : 8;
  if (sw == rw) {
    // A bit copy: the widest power-of-two byte vector (up to 16) that divides
    // the row and keeps both sides aligned.
    const int64_t row_bytes = b.row_elements * sw;
    int nb = 16;
    while (nb > 1 && (row_bytes % nb || t % nb || d % nb))
      nb /= 2;
    g.op = kGatherCopy;
    g.nbi = g.nbo = nb;
  } else {
    int v = 4;
    while (v > 1 && (b.row_elements % v || t % (v * sw) || d % (v * rw)))
      v /= 2;
    g.op = sw == 4 ? kGatherF32F16 : kGatherF16F32;
    g.nbi = v * static_cast<int>(sw);
    g.nbo = v * static_cast<int>(rw);
  }
  g.row_items = b.row_elements * sw / g.nbi;
  g.nt = g.nbi >= 8 && b.row_elements * sw >= 256;
  if (g.row_items >= kMaxLaunchWork)
    throw Error("unsupported_layout", "an indexed row spans 2^31 or more vector items");
  return g;
}

std::vector<GatherArgs> gather_launches(const Bound &b, const GatherPlan &g, const void *table,
                                        void *dst, const void *idx) {
  std::vector<GatherArgs> out;
  const int64_t count = static_cast<int64_t>(b.indices.size());
  const int64_t per = std::max<int64_t>(1, (kMaxLaunchWork - 1) / g.row_items);
  const int64_t row_out = g.row_items * g.nbo;
  for (int64_t r0 = 0; r0 < count; r0 += per) {
    const int64_t r1 = std::min(count, r0 + per);
    GatherArgs a{};
    a.table = static_cast<const uint8_t *>(table);
    a.dst = static_cast<uint8_t *>(dst) + r0 * row_out;
    a.idx = static_cast<const uint8_t *>(idx) + r0 * g.iw;
    a.work = static_cast<uint32_t>((r1 - r0) * g.row_items);
    a.row_items = static_cast<uint32_t>(g.row_items);
    a.per_row = make_div(g.row_items);
    out.push_back(a);
  }
  return out;
}

void verify_gather(const Bound &b, const GatherPlan &g, const std::vector<GatherArgs> &launches,
                   const void *table, size_t table_bytes, const void *dst, size_t dst_bytes,
                   const void *idx) {
  auto bad = [](const std::string &m) { throw Error("launch_check", "gather: " + m); };
  const uint32_t sw = b.source_type.width();
  const int64_t row_in = g.row_items * g.nbi;
  if (row_in != b.row_elements * static_cast<int64_t>(sw))
    bad("row length disagrees with the vector shape");
  if (b.table_rows * row_in > static_cast<int64_t>(table_bytes))
    bad("table rows exceed the table buffer");
  for (int64_t v : b.indices)
    if (v < 0 || v >= b.table_rows)
      bad("index outside the table");
  const uintptr_t t = reinterpret_cast<uintptr_t>(table);
  if (t % g.nbi)
    bad("table misaligned for the item size");
  const uint8_t *d0 = static_cast<const uint8_t *>(dst);
  const uint8_t *i0 = static_cast<const uint8_t *>(idx);
  int64_t rows = 0;
  for (const GatherArgs &a : launches) {
    if (a.table != table || a.row_items != g.row_items || a.per_row.d != a.row_items)
      bad("launch fields disagree with the plan");
    if (a.work % a.row_items)
      bad("launch covers a partial row");
    const int64_t n = a.work / a.row_items;
    if (a.dst != d0 + rows * g.row_items * g.nbo || a.idx != i0 + rows * g.iw)
      bad("launch does not continue the previous one");
    if (reinterpret_cast<uintptr_t>(a.dst) % g.nbo)
      bad("destination misaligned for the item size");
    if (a.work >= kMaxLaunchWork)
      bad("launch work of 2^31 or more");
    rows += n;
    if (rows * g.row_items * g.nbo > static_cast<int64_t>(dst_bytes))
      bad("destination overrun");
    // The kernel's row of item i: check the division on the last item.
    if (a.work && fdiv(a.work - 1, a.per_row) != static_cast<uint32_t>(n - 1))
      bad("row division");
  }
  if (rows != static_cast<int64_t>(b.indices.size()))
    bad("launches do not cover every selected row");
}

void host_gather(const Bound &b, const Prepared &p, uint32_t k, const void *table, void *dst,
                 int64_t g0, int64_t g1) {
  // No software prefetch: measured on the host, the hardware prefetchers
  // cover rows of 256 bytes and more, and explicit prefetches of the next
  // rows only slowed the copy down.
  const uint32_t sw = b.source_type.width();
  const uint32_t wout = k ? p.stages[k - 1].out_width : sw;
  const uint8_t *t = static_cast<const uint8_t *>(table);
  uint8_t *out = static_cast<uint8_t *>(dst);
  const int64_t row = b.row_elements, row_in = row * sw;
  const int64_t *idx = b.indices.data();
  int64_t r = g0 / row, c = g0 - (g0 / row) * row, g = g0;
  if (k == 0) { // bit copy: whole rows in a tight loop, partial rows at the ends
    if (c) {
      const int64_t n = std::min(row - c, g1 - g);
      std::memcpy(out, t + idx[r] * row_in + c * sw, static_cast<size_t>(n * sw));
      out += n * sw;
      g += n;
      ++r;
    }
    const int64_t full = (g1 - g) / row;
    for (int64_t j = 0; j < full; ++j, ++r, out += row_in)
      std::memcpy(out, t + idx[r] * row_in, static_cast<size_t>(row_in));
    g += full * row;
    if (g < g1)
      std::memcpy(out, t + idx[r] * row_in, static_cast<size_t>((g1 - g) * sw));
    return;
  }
  if (row >= 256) { // long rows: the stage's vector loop runs on each row
    for (; g < g1; ++r, c = 0) {
      const int64_t n = std::min(row - c, g1 - g);
      host_transform(p, k, sw, t + (idx[r] * row + c) * sw, out + (g - g0) * wout, 0, n);
      g += n;
    }
    return;
  }
  // Short rows with a stage: gather source values into a small buffer and
  // convert them in batches (the vector conversions need long runs).
  alignas(64) uint8_t tmp[16384];
  const int64_t cap = static_cast<int64_t>(sizeof(tmp)) / sw;
  while (g < g1) {
    const int64_t base = g;
    int64_t filled = 0;
    while (g < g1 && filled < cap) {
      const int64_t n = std::min(std::min(row - c, g1 - g), cap - filled);
      std::memcpy(tmp + filled * sw, t + (idx[r] * row + c) * sw, static_cast<size_t>(n * sw));
      filled += n;
      g += n;
      c += n;
      if (c == row) {
        c = 0;
        ++r;
      }
    }
    host_transform(p, k, sw, tmp, out + (base - g0) * wout, 0, filled);
  }
}

bool table_upload_pays(const Bound &b, int64_t gathered_wire) {
  return b.indexed && static_cast<int64_t>(b.indices.size()) >= kTableUploadRows &&
         b.table_bytes <= gathered_wire;
}

int64_t index_select_device(Context &ctx, BoundHandle &h, const void *table, size_t table_bytes,
                            void *dst, size_t dst_bytes, hipStream_t stream) {
  const Bound &b = *h.bound;
  if (!b.indexed)
    throw Error("plan_mismatch", "index_select needs an indexed plan");
  if (!table || !dst)
    throw Error("invalid_view", "null table or destination");
  if (static_cast<int64_t>(table_bytes) < b.table_bytes)
    throw Error("insufficient_capacity", "table holds " + std::to_string(table_bytes) +
                                             " bytes, the plan reads " +
                                             std::to_string(b.table_bytes));
  if (static_cast<int64_t>(dst_bytes) < b.destination_bytes)
    throw Error("insufficient_capacity", "destination holds " + std::to_string(dst_bytes) +
                                             " bytes, the plan writes " +
                                             std::to_string(b.destination_bytes));
  DeviceScope scope(ctx.device);
  const GatherPlan g = gather_plan(b, table, dst);
  const void *idx = h.device_indices(ctx.device);
  const std::vector<GatherArgs> launches = gather_launches(b, g, table, dst, idx);
  if (verify_env())
    verify_gather(b, g, launches, table, table_bytes, dst, dst_bytes, idx);
  // `stream` as given: 0 is the legacy null stream
  for (const GatherArgs &a : launches)
    hipcheck(gather_launch(a, g.op, g.nbi, g.iw, g.nt, stream), "gather launch");
  return static_cast<int64_t>(launches.size());
}

} // namespace relx
