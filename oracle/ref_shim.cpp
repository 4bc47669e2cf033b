// C driver over the reference's own CPU libreloc (TEST INFRASTRUCTURE ONLY).
//
// Built by oracle/Makefile together with the reference's libreloc sources
// (read in place under /root/reference, never copied) into
// oracle/_ref/libreloc_ref.so. Tests use it to cross-check the numpy oracle
// on config-sized inputs; bench.py times it as the CPU baseline. It calls:
//   decodePlan / decodeTypedPlan   libreloc/src/Decode.cpp:876-948
//   bind / bindTyped               libreloc/src/Bind.cpp:176-699
//   typed::prepareProgram          libreloc/src/TypedExecute.cpp:292-403
//   typed::executeHost             libreloc/src/TypedExecute.cpp:926-931
//   executeH2DThreaded             libreloc/src/Execute.cpp:145-216
//   decodeIndexedPlan / bindIndexed libreloc/src/Decode.cpp:993-1012,
//                                  libreloc/src/Bind.cpp:701-819; the program
//                                  fields prepareIndexSelect sets
//                                  (libreloc/src/Dispatch.cpp:1269-1283)
#include "reloc/Bind.h"
#include "reloc/Decode.h"
#include "reloc/Execute.h"
#include "reloc/GatherPool.h"
#include "reloc/Transfer.h"
#include "reloc/TypedExecute.h"

#include <cstring>
#include <memory>
#include <string>

namespace {
void setErr(char *err, size_t cap, const std::string &msg) {
  if (err && cap) {
    std::strncpy(err, msg.c_str(), cap - 1);
    err[cap - 1] = 0;
  }
}
reloc::ElementType typeOf(int kind, int bits) {
  return reloc::ElementType{static_cast<reloc::ElementTypeKind>(kind),
                            static_cast<uint32_t>(bits)};
}
} // namespace

struct RefTyped {
  reloc::typed::Program program;
  std::unique_ptr<reloc::GatherPool> pool;
};

struct RefLayout {
  reloc::BoundPlan bound;
  unsigned threads = 1;
};

extern "C" {

// Decode + bindTyped + prepareProgram. Parameters: names, dtype (kind, bits),
// rank-1 length (-1 for rank 0) and little-endian bytes.
void *ref_typed_prepare(const uint8_t *blob, size_t n, const char **symNames,
                        const int64_t *symVals, int nsym,
                        const char **paramNames, const int *paramKind,
                        const int *paramBits, const int64_t *paramLen,
                        const void **paramData, const size_t *paramBytes,
                        int nparam, unsigned threads, char *err, size_t cap) {
  auto decoded = reloc::decodeTypedPlan(blob, n);
  if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
    setErr(err, cap, "decode: " + e->message);
    return nullptr;
  }
  reloc::SymbolMap symbols;
  for (int i = 0; i < nsym; ++i)
    symbols[symNames[i]] = symVals[i];
  reloc::ParameterMap params;
  for (int i = 0; i < nparam; ++i) {
    reloc::ParameterValue v;
    v.elementType = typeOf(paramKind[i], paramBits[i]);
    if (paramLen[i] >= 0)
      v.extents.push_back(paramLen[i]);
    const auto *p = static_cast<const uint8_t *>(paramData[i]);
    v.bytes.assign(p, p + paramBytes[i]);
    params[paramNames[i]] = std::move(v);
  }
  auto bound = reloc::bindTyped(std::get<reloc::TypedRelocationPlan>(decoded),
                                symbols, params);
  if (auto *e = std::get_if<reloc::BindError>(&bound)) {
    setErr(err, cap, "bind: " + e->message);
    return nullptr;
  }
  auto program =
      reloc::typed::prepareProgram(std::get<reloc::TypedBoundPlan>(bound));
  if (auto *e = std::get_if<reloc::typed::ExecutionError>(&program)) {
    setErr(err, cap, e->code + ": " + e->message);
    return nullptr;
  }
  auto *h = new RefTyped{std::move(std::get<reloc::typed::Program>(program)),
                         nullptr};
  if (threads > 1)
    h->pool = std::make_unique<reloc::GatherPool>(threads);
  return h;
}

int64_t ref_typed_result_bytes(void *h) {
  auto *t = static_cast<RefTyped *>(h);
  return t->program.plan.destinationBytes;
}

// executeHost over all stages [0, n): dense source -> dense result.
int ref_typed_execute(void *h, const void *src, void *dst, char *err,
                      size_t cap) {
  auto *t = static_cast<RefTyped *>(h);
  const uint32_t to = static_cast<uint32_t>(t->program.stages.size());
  auto e = reloc::typed::executeHost(t->program, 0, to, src, dst,
                                     t->pool.get(), 1);
  if (e) {
    setErr(err, cap, e->code + ": " + e->message);
    return 1;
  }
  return 0;
}

void ref_typed_free(void *h) { delete static_cast<RefTyped *>(h); }

void *ref_layout_prepare(const uint8_t *blob, size_t n, const char **symNames,
                         const int64_t *symVals, int nsym, unsigned threads,
                         char *err, size_t cap) {
  auto decoded = reloc::decodePlan(blob, n);
  if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
    setErr(err, cap, "decode: " + e->message);
    return nullptr;
  }
  reloc::SymbolMap symbols;
  for (int i = 0; i < nsym; ++i)
    symbols[symNames[i]] = symVals[i];
  auto bound = reloc::bind(std::get<reloc::RelocationPlan>(decoded), symbols);
  if (auto *e = std::get_if<reloc::BindError>(&bound)) {
    setErr(err, cap, "bind: " + e->message);
    return nullptr;
  }
  return new RefLayout{std::get<reloc::BoundPlan>(bound), threads};
}

int64_t ref_layout_total_bytes(void *h) {
  return static_cast<RefLayout *>(h)->bound.totalBytes;
}

int ref_layout_execute(void *h, const void *src, void *dst) {
  auto *l = static_cast<RefLayout *>(h);
  reloc::executeH2DThreaded(l->bound, src, dst, l->threads);
  return 0;
}

void ref_layout_free(void *h) { delete static_cast<RefLayout *>(h); }

// Decode a wire v2 blob: 0 when valid, else 1 with the message and offset.
int ref_indexed_decode(const uint8_t *blob, size_t n, int64_t *offset, char *err, size_t cap) {
  auto decoded = reloc::decodeIndexedPlan(blob, n);
  if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
    setErr(err, cap, e->message);
    if (offset)
      *offset = static_cast<int64_t>(e->offset);
    return 1;
  }
  return 0;
}

// Decode + bindIndexed + prepareProgram, then the indexed program fields
// (rows, row elements, row indices) as prepareIndexSelect sets them; errors
// are "decode: ...", "bind: ..." or "<code>: ...".
void *ref_indexed_prepare(const uint8_t *blob, size_t n, const char **symNames,
                          const int64_t *symVals, int nsym, int idxKind, int idxBits,
                          const int64_t *idxExtents, int idxRank, const void *idxData,
                          size_t idxBytes, unsigned threads, char *err, size_t cap) {
  auto decoded = reloc::decodeIndexedPlan(blob, n);
  if (auto *e = std::get_if<reloc::DecodeError>(&decoded)) {
    setErr(err, cap, "decode: " + e->message);
    return nullptr;
  }
  reloc::SymbolMap symbols;
  for (int i = 0; i < nsym; ++i)
    symbols[symNames[i]] = symVals[i];
  std::vector<int64_t> extents(idxExtents, idxExtents + idxRank);
  auto bound = reloc::bindIndexed(std::get<reloc::IndexedRelocationPlan>(decoded), symbols,
                                  typeOf(idxKind, idxBits), extents, idxData, idxBytes);
  if (auto *e = std::get_if<reloc::BindError>(&bound)) {
    setErr(err, cap, "bind: " + e->message);
    return nullptr;
  }
  auto &b = std::get<reloc::IndexedBoundPlan>(bound);
  auto program = reloc::typed::prepareProgram(b.selected);
  if (auto *e = std::get_if<reloc::typed::ExecutionError>(&program)) {
    setErr(err, cap, e->code + ": " + e->message);
    return nullptr;
  }
  auto *h = new RefTyped{std::move(std::get<reloc::typed::Program>(program)), nullptr};
  h->program.indexedSourceRows = b.sourceExtents.front();
  h->program.indexedRowElements = b.rowElements;
  h->program.rowIndices = b.indices;
  if (threads > 1)
    h->pool = std::make_unique<reloc::GatherPool>(threads);
  return h;
}

// validateTransferSource (sourceOnly) or validateTransfer on a decoded and
// bound layout plan (libreloc/src/Transfer.cpp:233-268). A view is given as
// (base, capacity, offset) words, rank, extents, strides, element size,
// kind (0 host, 1 cuda) and device. Returns 0 with the source span, 1 with
// "<code>: <message>", 2 when the plan does not decode or bind.
int ref_validate_transfer(const uint8_t *blob, size_t n, const char **symNames,
                          const int64_t *symVals, int nsym, const uint64_t *sw, int srank,
                          const int64_t *sext, const int64_t *sstr, uint32_t ses, int skind,
                          int sdev, const uint64_t *dw, int drank, const int64_t *dext,
                          const int64_t *dstr, uint32_t des, int dkind, int ddev, int direction,
                          int sourceOnly, uint64_t *span, char *err, size_t cap) {
  auto decoded = reloc::decodePlan(blob, n);
  if (std::holds_alternative<reloc::DecodeError>(decoded))
    return 2;
  reloc::SymbolMap symbols;
  for (int i = 0; i < nsym; ++i)
    symbols[symNames[i]] = symVals[i];
  auto bound = reloc::bind(std::get<reloc::RelocationPlan>(decoded), symbols);
  if (std::holds_alternative<reloc::BindError>(bound))
    return 2;
  auto view = [](const uint64_t *w, int rank, const int64_t *ext, const int64_t *str, uint32_t es,
                 int kind, int dev) {
    reloc::BufferView v;
    v.base = static_cast<uintptr_t>(w[0]);
    v.capacityBytes = static_cast<size_t>(w[1]);
    v.offsetBytes = static_cast<size_t>(w[2]);
    v.extents.assign(ext, ext + rank);
    v.strides.assign(str, str + rank);
    v.elementSize = es;
    v.kind = kind ? reloc::MemoryKind::Cuda : reloc::MemoryKind::Host;
    v.device = dev;
    return v;
  };
  const auto dir = direction ? reloc::TransferDirection::DeviceToHost
                             : reloc::TransferDirection::HostToDevice;
  const reloc::BufferView src = view(sw, srank, sext, sstr, ses, skind, sdev);
  const auto &b = std::get<reloc::BoundPlan>(bound);
  if (sourceOnly) {
    auto r = reloc::validateTransferSource(b, src, dir);
    if (auto *e = std::get_if<reloc::TransferError>(&r)) {
      setErr(err, cap, e->code + ": " + e->message);
      return 1;
    }
    *span = std::get<size_t>(r);
    return 0;
  }
  auto r = reloc::validateTransfer(b, src, view(dw, drank, dext, dstr, des, dkind, ddev), dir);
  if (auto *e = std::get_if<reloc::TransferError>(&r)) {
    setErr(err, cap, e->code + ": " + e->message);
    return 1;
  }
  *span = std::get<reloc::TransferRequest>(r).sourceSpanBytes;
  return 0;
}

} // extern "C"
