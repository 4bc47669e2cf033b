// plan.h - relocation plan model, wire decoder and binder (host C++).
//
// Semantics follow the reference runtime so results are interchangeable:
//   wire format v0/v1   docs/reloc-plan-format.md; libreloc/src/Decode.cpp
//   wire format v2      docs/reloc-plan-format.md:287-345; Decode.cpp:950-1012
//   evaluation/binding  libreloc/src/Bind.cpp:84-699
//   indexed binding     libreloc/src/Bind.cpp:701-819
// The representation is this library's own: plans are decoded into flat
// structs with expression streams kept as postfix token vectors, and every
// failure is a relx::Error carrying a stable code.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace relx {

// ------------------------------------------------------------------ errors

struct Error : std::exception {
  std::string code;
  std::string message;
  int64_t offset = -1;
  Error(std::string c, std::string m, int64_t off = -1)
      : code(std::move(c)), message(std::move(m)), offset(off) {}
  const char *what() const noexcept override { return message.c_str(); }
};

[[noreturn]] inline void fail(const std::string &code, const std::string &msg) {
  throw Error(code, msg);
}

// ------------------------------------------------------------- plan model

enum : uint8_t { kPushSym = 0, kPushConst, kAdd, kSub, kMul, kFloorDiv, kMod, kPushDim };
struct Token {
  uint8_t op;
  int64_t value;
  bool operator==(const Token &o) const { return op == o.op && value == o.value; }
};
using Expr = std::vector<Token>;

enum : uint8_t { kFloat = 0, kBFloat = 1, kInteger = 2, kIndex = 3 };
struct DType {
  uint8_t kind = 0;
  uint32_t bits = 0;
  bool operator==(const DType &o) const { return kind == o.kind && bits == o.bits; }
  bool operator!=(const DType &o) const { return !(*this == o); }
  // bytes per element; 0 when the width is not a whole number of bytes
  uint32_t width() const { return (bits && bits % 8 == 0) ? bits / 8 : 0; }
  bool f32() const { return kind == kFloat && bits == 32; }
  bool f16() const { return kind == kFloat && bits == 16; }
  bool bf16() const { return kind == kBFloat && bits == 16; }
  bool i8() const { return kind == kInteger && bits == 8; }
};

struct TensorDesc {
  std::vector<Expr> extents;
  std::vector<Expr> strides; // empty = canonical row-major
  Expr offset;
  DType type;
};

struct PlanAxis {
  std::string name;
  Expr extent, src_stride, dst_stride;
};

struct PlanPad {
  uint32_t axis = 0;
  Expr lo, hi;
  DType type;
  uint64_t bits = 0;
};

struct LayoutPlan {
  TensorDesc src, dst;
  std::vector<uint32_t> perm;
  std::vector<PlanAxis> axes;
  std::vector<PlanPad> pads;
  std::vector<std::pair<Expr, int64_t>> divisibility;
  std::vector<std::pair<uint32_t, int64_t>> alignment;
  std::vector<uint8_t> contiguity;
  bool no_copy = false;
  bool runtime_pad_check = false;
  std::vector<Expr> inverse;
};

enum : uint8_t { kCast = 0, kQuantize = 1, kDequantize = 2 };
enum : uint8_t { kIeeeRne = 0, kExact = 1, kSymmetricRne = 2, kAffine = 3 };
enum : uint8_t { kParamNone = 0, kParamInline = 1, kParamBinding = 2 };

struct StageParam {
  uint8_t kind = kParamNone;
  uint8_t rank = 0;
  DType type;
  std::vector<uint64_t> inline_bits;
  std::string name;
  std::vector<Expr> extents;
};

struct PlanStage {
  uint8_t transform = kCast, policy = kIeeeRne;
  DType in, out;
  uint8_t in_sign = 0, out_sign = 0; // 0 signless, 1 signed, 2 unsigned
  std::vector<Expr> shape;
  StageParam scale, zero_point;
  int64_t axis = -1;
  bool has_channel = false;
  Expr channel; // PushDim = logical result coordinate
};

struct PlanFill {
  uint32_t axis = 0, stage = 0;
  DType type;
  uint64_t bits = 0;
};

struct Plan {
  uint32_t version = 0; // 0 layout, 1 typed, 2 indexed
  std::vector<std::string> symbols;
  LayoutPlan layout;
  // typed (v1) and indexed (v2)
  TensorDesc source, result;
  std::vector<PlanStage> stages;
  std::vector<PlanFill> fills;
  // indexed (v2) only: rows `indices` of `source` along `axis` (always 0),
  // cast to the result type under `policy`
  TensorDesc indices;
  uint32_t axis = 0;
  uint8_t policy = kExact;
};

// Wire version of an "RPLN" blob, -1 otherwise.
int peek_wire_version(const uint8_t *data, size_t n);
// Decode v0, v1 or v2 (by header). Throws Error{"decode_error", msg, offset}.
std::unique_ptr<Plan> decode(const uint8_t *data, size_t n);
// The indexed-plan invariants (reference validateIndexedPlan,
// libreloc/src/Decode.cpp:950-991); empty when the plan is valid.
std::string validate_indexed(const Plan &p);

// Scalar stage arithmetic on bit patterns (docs/reloc-typed-semantics.md).
uint16_t f32_to_f16_bits(uint32_t f);
uint32_t f16_to_f32_bits(uint16_t h);
uint16_t f32_to_bf16_bits(uint32_t f);
uint32_t bf16_to_f32_bits(uint16_t b);
int8_t quantize_one(float x, float inv);
// Fold a fill value through one stage with inline per-tensor parameters;
// false when the stage needs per-channel or runtime parameters.
bool fold_fill(uint64_t &bits, DType &type, const PlanStage &stage);

// ------------------------------------------------------------ evaluation

// Postfix evaluation with checked int64 arithmetic (FLOORDIV/MOD are floor
// semantics). `dims` is null in the plan context. Throws Error{"bind_error"}.
int64_t eval(const Expr &e, const std::vector<int64_t> &symbols,
             const std::vector<int64_t> *dims = nullptr);

// ---------------------------------------------------------------- binding

struct BoundPad {
  int axis;
  int64_t lo, hi;
  uint64_t bits;
};

struct BoundLayout {
  std::vector<int64_t> extents; // valid extents, coalesced destination order
  std::vector<int64_t> src_strides, dst_strides;
  std::vector<BoundPad> pads;
  std::vector<uint32_t> perm;
  uint32_t element_size = 0;
  int64_t total_bytes = 0;
  int64_t inner_run = 1;
  bool no_copy = false;
  std::vector<std::pair<uint32_t, int64_t>> alignment; // coalesced axis index
};

struct BoundParam {
  bool present = false;
  DType type;
  int64_t length = 0;
  std::vector<uint8_t> bytes;
  std::string name;
};

struct BoundStage {
  uint8_t transform = kCast, policy = kIeeeRne;
  DType in, out;
  std::vector<int64_t> shape;
  int64_t axis = -1;
  bool has_channel = false;
  Expr channel;
  BoundParam scale, zero_point;
};

struct ParamValue {
  DType type;
  std::vector<int64_t> extents;
  std::vector<uint8_t> bytes;
};

struct Bound {
  bool typed = false;
  BoundLayout layout;
  std::vector<int64_t> symbols;
  // typed
  std::vector<int64_t> source_extents, result_extents;
  DType source_type, result_type;
  std::vector<BoundStage> stages;
  std::vector<PlanFill> fills;
  std::vector<int64_t> bytes_at; // dense footprint per stage boundary
  int64_t source_bytes = 0, destination_bytes = 0, parameter_bytes = 0;
  // indexed (v2): the typed fields above describe the selected rows (an
  // identity layout over [count, row_elements] plus at most one cast); the
  // physical source is `table_rows` rows of `row_elements` elements.
  bool indexed = false;
  std::vector<int64_t> table_extents;
  std::vector<int64_t> indices; // one per selected row, each in [0, table_rows)
  int64_t table_rows = 0, row_elements = 0, table_bytes = 0;
  DType index_type;
};

// bind (v0) / bindTyped (v1). Throws Error{"bind_error", ...}.
std::unique_ptr<Bound> bind(const Plan &plan, const std::map<std::string, int64_t> &symbols,
                            const std::map<std::string, ParamValue> &params);

// bindIndexed (v2): symbols plus the index operand (element type, extents,
// little-endian bytes), whose values are copied and range-checked.
std::unique_ptr<Bound> bind_indexed(const Plan &plan,
                                    const std::map<std::string, int64_t> &symbols,
                                    DType index_type, const std::vector<int64_t> &index_extents,
                                    const void *index_data, size_t index_bytes);

} // namespace relx
