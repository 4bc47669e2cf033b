// plan.cpp - wire decoder, expression evaluator and binder.
//
// Wire layout: docs/reloc-plan-format.md (v0 sections 0-12, v1 sections
// 0-7). Validation rules follow the reference decoder
// (libreloc/src/Decode.cpp:115-948) and binder (libreloc/src/Bind.cpp:
// 84-699) so that a blob either runtime rejects is rejected here too, with
// the byte offset of the violated item.
#include "plan.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <set>

namespace relx {
namespace {

// ------------------------------------------------------------ wire reader

class Cursor {
public:
  Cursor(const uint8_t *p, size_t n) : p_(p), n_(n) {}
  size_t pos() const { return at_; }
  size_t left() const { return n_ - at_; }

  [[noreturn]] void reject(size_t at, const std::string &msg) const {
    throw Error("decode_error", msg, static_cast<int64_t>(at));
  }
  void need(size_t k, const char *what) const {
    if (left() < k)
      reject(at_, std::string("truncated: expected ") + what);
  }
  uint8_t u8() {
    need(1, "u8");
    return p_[at_++];
  }
  uint32_t u32() {
    need(4, "u32");
    uint32_t v;
    std::memcpy(&v, p_ + at_, 4);
    at_ += 4;
    return v;
  }
  uint64_t u64() {
    need(8, "u64");
    uint64_t v;
    std::memcpy(&v, p_ + at_, 8);
    at_ += 8;
    return v;
  }
  int64_t i64() { return static_cast<int64_t>(u64()); }
  // A count that sizes an allocation may not exceed the bytes left: every
  // counted item occupies at least one byte.
  uint32_t count(const char *what) {
    size_t at = at_;
    uint32_t v = u32();
    if (v > left())
      reject(at, std::string("count exceeds remaining bytes: ") + what);
    return v;
  }
  std::string str() {
    uint32_t k = count("string length");
    std::string s(reinterpret_cast<const char *>(p_ + at_), k);
    at_ += k;
    return s;
  }

private:
  const uint8_t *p_;
  size_t n_;
  size_t at_ = 0;
};

enum class Ctx { Plan, Inverse, Channel };

Expr read_expr(Cursor &c, Ctx ctx, size_t nsym, size_t ndim) {
  const size_t start = c.pos();
  const uint32_t ops = c.count("expression op_count");
  if (ops == 0)
    c.reject(start, "empty expression stream");
  Expr e;
  e.reserve(ops);
  int64_t depth = 0;
  for (uint32_t i = 0; i < ops; ++i) {
    const size_t at = c.pos();
    Token t{c.u8(), 0};
    switch (t.op) {
    case kPushSym:
      if (ctx == Ctx::Inverse)
        c.reject(at, "PUSH_SYM is not allowed in inverse expressions");
      t.value = c.u32();
      if (static_cast<size_t>(t.value) >= nsym)
        c.reject(at, "PUSH_SYM symbol index out of range");
      ++depth;
      break;
    case kPushConst:
      t.value = c.i64();
      ++depth;
      break;
    case kPushDim:
      if (ctx == Ctx::Plan)
        c.reject(at, "PUSH_DIM is only allowed in inverse and channel expressions");
      t.value = c.u32();
      if (static_cast<size_t>(t.value) >= ndim)
        c.reject(at, "PUSH_DIM dim index out of range");
      ++depth;
      break;
    case kAdd:
    case kSub:
    case kMul:
    case kFloorDiv:
    case kMod:
      if (depth < 2)
        c.reject(at, "expression stack underflow");
      --depth;
      break;
    default:
      c.reject(at, "unknown expression opcode");
    }
    e.push_back(t);
  }
  if (depth != 1)
    c.reject(start, "expression stream must leave exactly one value");
  return e;
}

DType read_type(Cursor &c) {
  const size_t at = c.pos();
  DType t;
  t.kind = c.u8();
  t.bits = c.u32();
  bool ok = false;
  switch (t.kind) {
  case kFloat:
    ok = t.bits == 16 || t.bits == 32 || t.bits == 64;
    break;
  case kBFloat:
    ok = t.bits == 16;
    break;
  case kInteger:
    ok = t.bits >= 1 && t.bits <= 64;
    break;
  case kIndex:
    ok = t.bits == 64;
    break;
  }
  if (!ok)
    c.reject(at, "invalid element type kind/bitwidth");
  return t;
}

TensorDesc read_desc(Cursor &c, size_t nsym) {
  TensorDesc d;
  const uint32_t rank = c.count("tensor_desc rank");
  for (uint32_t i = 0; i < rank; ++i)
    d.extents.push_back(read_expr(c, Ctx::Plan, nsym, 0));
  const size_t at = c.pos();
  const uint32_t ns = c.count("tensor_desc stride_count");
  if (ns != 0 && ns != rank)
    c.reject(at, "tensor_desc stride_count must be 0 or the rank");
  for (uint32_t i = 0; i < ns; ++i)
    d.strides.push_back(read_expr(c, Ctx::Plan, nsym, 0));
  d.offset = read_expr(c, Ctx::Plan, nsym, 0);
  d.type = read_type(c);
  return d;
}

uint8_t read_flag(Cursor &c, const char *msg) {
  const size_t at = c.pos();
  uint8_t v = c.u8();
  if (v > 1)
    c.reject(at, msg);
  return v;
}

void read_layout(Cursor &c, size_t nsym, LayoutPlan &L) {
  L.src = read_desc(c, nsym);
  const size_t dst_at = c.pos();
  L.dst = read_desc(c, nsym);
  const size_t perm_at = c.pos();
  const uint32_t np = c.count("perm count");
  for (uint32_t i = 0; i < np; ++i)
    L.perm.push_back(c.u32());
  const size_t axes_at = c.pos();
  const uint32_t na = c.count("axes count");
  if (na < 1)
    c.reject(axes_at, "axis count must be >= 1");
  for (uint32_t i = 0; i < na; ++i) {
    PlanAxis a;
    a.name = c.str();
    a.extent = read_expr(c, Ctx::Plan, nsym, 0);
    a.src_stride = read_expr(c, Ctx::Plan, nsym, 0);
    a.dst_stride = read_expr(c, Ctx::Plan, nsym, 0);
    L.axes.push_back(std::move(a));
  }
  if (L.perm.size() != L.axes.size())
    c.reject(perm_at, "perm size must equal the axis count");
  std::vector<char> seen(L.axes.size(), 0);
  for (uint32_t v : L.perm) {
    if (v >= L.axes.size() || seen[v])
      c.reject(perm_at, "perm is not a permutation of [0, axis count)");
    seen[v] = 1;
  }
  if (L.dst.extents.size() != L.axes.size())
    c.reject(dst_at, "dst rank must equal the axis count");
  const uint32_t npad = c.count("pad_fill count");
  for (uint32_t i = 0; i < npad; ++i) {
    PlanPad p;
    const size_t at = c.pos();
    p.axis = c.u32();
    if (p.axis >= L.axes.size())
      c.reject(at, "pad_fill dst_axis out of range");
    p.lo = read_expr(c, Ctx::Plan, nsym, 0);
    p.hi = read_expr(c, Ctx::Plan, nsym, 0);
    p.type = read_type(c);
    p.bits = c.u64();
    L.pads.push_back(std::move(p));
  }
  const uint32_t nd = c.count("divisibility count");
  for (uint32_t i = 0; i < nd; ++i) {
    Expr e = read_expr(c, Ctx::Plan, nsym, 0);
    L.divisibility.emplace_back(std::move(e), c.i64());
  }
  const uint32_t nal = c.count("alignment count");
  for (uint32_t i = 0; i < nal; ++i) {
    const size_t at = c.pos();
    uint32_t ax = c.u32();
    if (ax >= L.axes.size())
      c.reject(at, "alignment axis out of range");
    L.alignment.emplace_back(ax, c.i64());
  }
  const size_t ct_at = c.pos();
  const uint32_t nc = c.count("contiguity count");
  if (nc != 0 && nc != L.axes.size())
    c.reject(ct_at, "contiguity count must be 0 or the axis count");
  for (uint32_t i = 0; i < nc; ++i)
    L.contiguity.push_back(read_flag(c, "contiguity flag must be 0 or 1"));
  L.no_copy = read_flag(c, "no_copy flag must be 0 or 1") != 0;
  L.runtime_pad_check = read_flag(c, "runtime_pad_check flag must be 0 or 1") != 0;
  const size_t dims_at = c.pos();
  const uint32_t ndims = c.u32();
  const size_t res_at = c.pos();
  const uint32_t nres = c.u32();
  if (ndims != L.axes.size())
    c.reject(dims_at, "inverse num_dims must equal the axis count");
  if (nres != L.axes.size())
    c.reject(res_at, "inverse num_results must equal the axis count");
  for (uint32_t i = 0; i < nres; ++i)
    L.inverse.push_back(read_expr(c, Ctx::Inverse, nsym, ndims));
}

std::vector<std::string> read_header(Cursor &c, const uint8_t *data, uint32_t &version) {
  if (c.left() < 4)
    c.reject(0, "truncated: expected magic");
  if (std::memcmp(data, "RPLN", 4) != 0)
    c.reject(0, "bad magic (expected RPLN)");
  c.u32();
  const size_t at = c.pos();
  version = c.u32();
  if (version > 2)
    c.reject(at, "unsupported wire format version");
  std::vector<std::string> syms;
  const uint32_t ns = c.count("symbol table count");
  for (uint32_t i = 0; i < ns; ++i)
    syms.push_back(c.str());
  return syms;
}

StageParam read_param(Cursor &c, size_t nsym) {
  StageParam p;
  const size_t at = c.pos();
  p.kind = c.u8();
  if (p.kind > 2)
    c.reject(at, "invalid parameter kind");
  if (p.kind == kParamNone)
    return p;
  if (p.kind == kParamInline) {
    const size_t rat = c.pos();
    p.rank = c.u8();
    if (p.rank > 1)
      c.reject(rat, "parameter rank must be 0 or 1");
    p.type = read_type(c);
    const size_t cat = c.pos();
    const uint32_t n = c.count("inline parameter count");
    if (n == 0)
      c.reject(cat, "inline parameter must hold a value");
    if (p.rank == 0 && n != 1)
      c.reject(cat, "rank-0 inline parameter must hold exactly one value");
    if (n > c.left() / 8)
      c.reject(cat, "count exceeds remaining bytes: inline parameter");
    for (uint32_t i = 0; i < n; ++i)
      p.inline_bits.push_back(c.u64());
    return p;
  }
  const size_t nat = c.pos();
  p.name = c.str();
  if (p.name.empty())
    c.reject(nat, "binding name must not be empty");
  const size_t rat = c.pos();
  p.rank = c.u8();
  if (p.rank > 1)
    c.reject(rat, "parameter rank must be 0 or 1");
  for (uint8_t i = 0; i < p.rank; ++i)
    p.extents.push_back(read_expr(c, Ctx::Plan, nsym, 0));
  p.type = read_type(c);
  return p;
}

PlanStage read_stage(Cursor &c, size_t nsym, size_t result_rank) {
  PlanStage s;
  const size_t at = c.pos();
  s.transform = c.u8();
  if (s.transform > 2)
    c.reject(at, "unknown stage transform");
  const size_t pat = c.pos();
  s.policy = c.u8();
  if (s.policy > 3)
    c.reject(pat, "unknown numerical policy");
  auto sign = [&](uint8_t &out) {
    const size_t sat = c.pos();
    out = c.u8();
    if (out > 2)
      c.reject(sat, "invalid stage type signedness");
  };
  s.in = read_type(c);
  sign(s.in_sign);
  s.out = read_type(c);
  sign(s.out_sign);
  const size_t rat = c.pos();
  const uint32_t rank = c.count("stage shape rank");
  if (rank == 0)
    c.reject(rat, "stage shape must have rank >= 1");
  for (uint32_t i = 0; i < rank; ++i)
    s.shape.push_back(read_expr(c, Ctx::Plan, nsym, 0));
  s.scale = read_param(c, nsym);
  s.zero_point = read_param(c, nsym);
  s.axis = c.i64();
  s.has_channel = read_flag(c, "has_channel flag must be 0 or 1") != 0;
  if (s.has_channel) {
    const size_t dat = c.pos();
    const uint32_t nd = c.u32();
    if (nd != result_rank)
      c.reject(dat, "channel map num_dims must equal the result rank");
    s.channel = read_expr(c, Ctx::Channel, nsym, nd);
  }
  return s;
}

int64_t sign_extend(uint64_t bits, uint32_t width) {
  if (width >= 64)
    return static_cast<int64_t>(bits);
  const uint64_t mask = (uint64_t{1} << width) - 1;
  uint64_t v = bits & mask;
  if (v >> (width - 1))
    v |= ~mask;
  return static_cast<int64_t>(v);
}

bool nan_bits(uint64_t bits, DType t) {
  if (t.bf16())
    return ((bits >> 7) & 0xff) == 0xff && (bits & 0x7f);
  if (t.f32())
    return ((bits >> 23) & 0xff) == 0xff && (bits & 0x7fffff);
  if (t.f16())
    return ((bits >> 10) & 0x1f) == 0x1f && (bits & 0x3ff);
  return false;
}

float as_float(uint64_t bits) {
  uint32_t b = static_cast<uint32_t>(bits);
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
uint32_t as_bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return b;
}

// The typed-plan invariants of docs/reloc-plan-format.md ("Decoder-enforced
// invariants"); order and messages follow libreloc/src/Decode.cpp:628-866.
void validate_typed(const Cursor &c, const Plan &p, size_t layout_at, size_t stages_at,
                    const std::vector<size_t> &stage_at, size_t fills_at,
                    const std::vector<size_t> &fill_at) {
  const DType st = p.source.type, rt = p.result.type;
  if (p.layout.src.type != st)
    c.reject(layout_at, "layout src element type must equal the source type");
  if (p.layout.dst.type != rt)
    c.reject(layout_at, "layout dst element type must equal the result type");
  if (p.layout.src.extents.size() != p.source.extents.size())
    c.reject(layout_at, "layout src rank must equal the source rank");
  if (p.stages.empty())
    c.reject(stages_at, "typed plan needs at least one stage");
  if (p.stages.front().in != st)
    c.reject(stage_at[0], "stage 0 input type must equal the source type");
  for (size_t k = 1; k < p.stages.size(); ++k)
    if (p.stages[k].in != p.stages[k - 1].out)
      c.reject(stage_at[k], "stage input type must equal the previous stage's output type");
  if (p.stages.back().out != rt)
    c.reject(stage_at.back(), "last stage output type must equal the result type");

  std::vector<const StageParam *> bindings;
  for (size_t k = 0; k < p.stages.size(); ++k) {
    const PlanStage &s = p.stages[k];
    const size_t at = stage_at[k];
    const bool signless = s.in_sign == 0 && s.out_sign == 0;
    if (s.transform == kCast) {
      const bool narrow = s.in.f32() && (s.out.f16() || s.out.bf16()) && s.policy == kIeeeRne;
      const bool widen = (s.in.f16() || s.in.bf16()) && s.out.f32() && s.policy == kExact;
      if (!(narrow || widen) || !signless)
        c.reject(at, "invalid cast signature (f32 -> f16/bf16 ieee_rne or f16/bf16 -> f32 "
                     "exact, signless)");
      if (s.scale.kind != kParamNone || s.zero_point.kind != kParamNone || s.axis != -1 ||
          s.has_channel)
        c.reject(at, "cast stages carry no parameters");
      continue;
    }
    if (s.transform == kQuantize) {
      if (!(s.in.f32() && s.in_sign == 0 && s.out.i8() && s.out_sign == 1 &&
            s.policy == kSymmetricRne))
        c.reject(at, "invalid quantize signature (f32 -> signed int 8, symmetric_rne)");
    } else if (!(s.in.i8() && s.in_sign == 1 && s.out.f32() && s.out_sign == 0 &&
                 s.policy == kAffine)) {
      c.reject(at, "invalid dequantize signature (signed int 8 -> f32, affine)");
    }
    if (s.scale.kind == kParamNone)
      c.reject(at, "quantize/dequantize stages require a scale");
    if (!s.scale.type.f32())
      c.reject(at, "scale element type must be f32");
    if (s.zero_point.kind != kParamNone) {
      if (s.zero_point.type.kind != kInteger)
        c.reject(at, "zero_point element type must be an integer");
      if (s.zero_point.kind == kParamBinding && s.zero_point.type.bits != 32)
        c.reject(at, "zero_point bindings must declare int 32");
    }
    if (s.axis == -1) {
      if (s.scale.rank != 0 || (s.zero_point.kind != kParamNone && s.zero_point.rank != 0) ||
          s.has_channel)
        c.reject(at, "per-tensor stage requires rank-0 parameters and no channel map");
    } else {
      if (s.axis < 0 || static_cast<uint64_t>(s.axis) >= s.shape.size())
        c.reject(at, "axis out of range for the stage shape");
      if (s.scale.rank != 1)
        c.reject(at, "per-channel stage requires a rank-1 scale");
      if (!s.has_channel)
        c.reject(at, "per-channel stage requires a channel map");
      const Expr &ext = s.shape[static_cast<size_t>(s.axis)];
      if (ext.size() == 1 && ext[0].op == kPushConst)
        for (const StageParam *prm : {&s.scale, &s.zero_point})
          if (prm->kind == kParamInline && prm->rank == 1 &&
              static_cast<int64_t>(prm->inline_bits.size()) != ext[0].value)
            c.reject(at, "inline parameter length must equal the channel extent");
    }
    if (s.scale.kind == kParamInline)
      for (uint64_t b : s.scale.inline_bits) {
        const float v = as_float(b);
        if (!std::isfinite(v) || !(v > 0.0f))
          c.reject(at, "inline scale must be finite and strictly positive");
      }
    if (s.zero_point.kind == kParamInline)
      for (uint64_t b : s.zero_point.inline_bits) {
        const int64_t v = sign_extend(b, s.zero_point.type.bits);
        if (v < -128 || v > 127)
          c.reject(at, "inline zero point out of [-128, 127]");
        if (s.policy == kSymmetricRne && v != 0)
          c.reject(at, "symmetric_rne admits only the constant zero point 0");
      }
    if (s.policy == kSymmetricRne && s.zero_point.kind == kParamBinding)
      c.reject(at, "symmetric_rne rejects a zero-point binding");
    if (s.scale.kind == kParamBinding && s.zero_point.kind == kParamBinding &&
        s.scale.name == s.zero_point.name)
      c.reject(at, "runtime parameters must use distinct binding names");
    for (const StageParam *prm : {&s.scale, &s.zero_point}) {
      if (prm->kind != kParamBinding)
        continue;
      for (const StageParam *seen : bindings)
        if (seen->name == prm->name &&
            !(seen->rank == prm->rank && seen->type == prm->type && seen->extents == prm->extents))
          c.reject(at, "conflicting parameter declaration for binding '" + prm->name + "'");
      bindings.push_back(prm);
    }
  }

  std::vector<char> covered(p.layout.pads.size(), 0);
  for (size_t i = 0; i < p.fills.size(); ++i) {
    const PlanFill &f = p.fills[i];
    const size_t at = fill_at[i];
    const PlanPad *pad = nullptr;
    for (size_t j = 0; j < p.layout.pads.size(); ++j)
      if (p.layout.pads[j].axis == f.axis) {
        if (covered[j])
          c.reject(at, "duplicate fill for a layout pad");
        covered[j] = 1;
        pad = &p.layout.pads[j];
      }
    if (!pad)
      c.reject(at, "fill dst_axis has no layout pad");
    if (f.stage > p.stages.size())
      c.reject(at, "fill stage out of range");
    const DType entry = f.stage == 0 ? st : p.stages[f.stage - 1].out;
    if (f.type != entry)
      c.reject(at, "fill type must equal the type entering its stage");
    if (pad->type != rt)
      c.reject(at, "layout pad fill type must equal the result type");
    uint64_t bits = f.bits;
    DType t = f.type;
    for (size_t k = f.stage; k < p.stages.size(); ++k)
      if (!fold_fill(bits, t, p.stages[k]))
        c.reject(at, "fill cannot fold through a per-channel or runtime-parameter stage");
    if (bits != pad->bits && !(nan_bits(bits, rt) && nan_bits(pad->bits, rt)))
      c.reject(at, "fill fold mismatch with the layout's fused fill");
  }
  for (char k : covered)
    if (!k)
      c.reject(fills_at, "layout pad without a typed fill");
}

// ----------------------------------------------------------- checked math

bool mul_ok(int64_t a, int64_t b, int64_t &out) { return !__builtin_mul_overflow(a, b, &out); }

int64_t floor_div(int64_t a, int64_t b) {
  if (b == 0)
    fail("bind_error", "division by zero");
  if (a == std::numeric_limits<int64_t>::min() && b == -1)
    fail("bind_error", "integer overflow in floordiv");
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0)))
    --q;
  return q;
}

} // namespace

// ------------------------------------------------------- stage arithmetic

namespace {
// Shift `v` right by `s` bits rounding to nearest, ties to even.
uint32_t shr_rne(uint32_t v, unsigned s) {
  if (s == 0)
    return v;
  if (s > 31)
    return 0;
  const uint32_t q = v >> s, r = v & ((1u << s) - 1u), half = 1u << (s - 1);
  return q + ((r > half || (r == half && (q & 1u))) ? 1u : 0u);
}
} // namespace

// IEEE binary32 -> binary16, round to nearest even, overflow to infinity,
// exact subnormals. NaN keeps the top payload bits with the quiet bit set
// (what x86 F16C and the reference CPU executor produce).
uint16_t f32_to_f16_bits(uint32_t f) {
  const uint16_t sign = static_cast<uint16_t>((f >> 16) & 0x8000u);
  const uint32_t mag = f & 0x7fffffffu;
  const uint32_t exp = mag >> 23;
  if (exp == 0xff)
    return mag & 0x7fffffu ? static_cast<uint16_t>(sign | 0x7e00u | ((mag >> 13) & 0x3ffu))
                           : static_cast<uint16_t>(sign | 0x7c00u);
  if (exp >= 113) { // |x| >= 2^-14: normal binary16 range (or overflow)
    // Rebias the exponent (127 -> 15) and round the 13 dropped mantissa bits;
    // a carry out of the mantissa increments the exponent, and anything at
    // or past the top rounds onto the infinity encoding.
    const uint32_t rebased = ((exp - 112) << 23) | (mag & 0x7fffffu);
    const uint32_t h = shr_rne(rebased, 13);
    return static_cast<uint16_t>(sign | (h >= 0x7c00u ? 0x7c00u : h));
  }
  if (exp == 0)
    return sign; // binary32 zero or subnormal: far below 2^-25
  // binary16 subnormal: value = m * 2^(exp-150), result unit 2^-24.
  const uint32_t m = (mag & 0x7fffffu) | 0x800000u;
  return static_cast<uint16_t>(sign | shr_rne(m, 126 - exp));
}

uint32_t f16_to_f32_bits(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f)
    return sign | 0x7f800000u | (m << 13);
  if (e != 0)
    return sign | ((e + 112) << 23) | (m << 13);
  if (m == 0)
    return sign;
  // subnormal: m * 2^-24; normalise so the leading one lands on bit 10
  const int lead = 31 - __builtin_clz(m); // 0..9
  const uint32_t frac = (m << (10 - lead)) & 0x3ffu;
  return sign | (static_cast<uint32_t>(lead + 103) << 23) | (frac << 13);
}

uint16_t f32_to_bf16_bits(uint32_t f) {
  if ((f & 0x7fffffffu) > 0x7f800000u)
    return static_cast<uint16_t>((f >> 16) | 0x40u);
  const uint64_t wide = static_cast<uint64_t>(f);
  const uint64_t lsb = (wide >> 16) & 1u;
  return static_cast<uint16_t>((wide + 0x7fffu + lsb) >> 16);
}

uint32_t bf16_to_f32_bits(uint16_t b) { return static_cast<uint32_t>(b) << 16; }

int8_t quantize_one(float x, float inv) {
  // docs/reloc-typed-semantics.md section 3.3: product, maxNum then minNum
  // (so NaN -> -128), round half to even.
  float y = x * inv;
  y = std::fmax(y, -128.0f);
  y = std::fmin(y, 127.0f);
  return static_cast<int8_t>(std::nearbyint(y));
}

bool fold_fill(uint64_t &bits, DType &type, const PlanStage &s) {
  if (type != s.in)
    return false;
  if (s.transform == kCast) {
    if (type.f32() && s.out.f16())
      bits = f32_to_f16_bits(static_cast<uint32_t>(bits));
    else if (type.f16() && s.out.f32())
      bits = f16_to_f32_bits(static_cast<uint16_t>(bits));
    else if (type.f32() && s.out.bf16())
      bits = f32_to_bf16_bits(static_cast<uint32_t>(bits));
    else if (type.bf16() && s.out.f32())
      bits = bf16_to_f32_bits(static_cast<uint16_t>(bits));
    else
      return false;
    type = s.out;
    return true;
  }
  if (s.axis >= 0 || s.scale.kind != kParamInline || s.scale.rank != 0 ||
      s.scale.inline_bits.empty())
    return false;
  const float scale = as_float(s.scale.inline_bits[0]);
  if (s.transform == kQuantize) {
    if (!type.f32() || !s.out.i8())
      return false;
    const float inv = 1.0f / scale;
    bits = static_cast<uint8_t>(quantize_one(as_float(bits), inv));
    type = s.out;
    return true;
  }
  if (!type.i8() || !s.out.f32())
    return false;
  int64_t zp = 0;
  if (s.zero_point.kind == kParamInline) {
    if (s.zero_point.rank != 0 || s.zero_point.inline_bits.empty())
      return false;
    zp = sign_extend(s.zero_point.inline_bits[0], s.zero_point.type.bits);
  } else if (s.zero_point.kind != kParamNone) {
    return false;
  }
  const float d = static_cast<float>(sign_extend(bits, 8) - zp);
  bits = as_bits(d * scale);
  type = s.out;
  return true;
}

// ----------------------------------------------------------------- decode

int peek_wire_version(const uint8_t *data, size_t n) {
  if (n < 8 || std::memcmp(data, "RPLN", 4) != 0)
    return -1;
  uint32_t v;
  std::memcpy(&v, data + 4, 4);
  return static_cast<int>(v > 0x7fffffffu ? 0x7fffffff : v);
}

std::unique_ptr<Plan> decode(const uint8_t *data, size_t n) {
  Cursor c(data, n);
  auto p = std::make_unique<Plan>();
  p->symbols = read_header(c, data, p->version);
  const size_t nsym = p->symbols.size();
  if (p->version == 0) {
    read_layout(c, nsym, p->layout);
    if (c.left())
      c.reject(c.pos(), "trailing bytes after inverse section");
    return p;
  }
  if (p->version == 2) {
    // docs/reloc-plan-format.md:287-345: source, indices and result
    // descriptors, u32 axis, u8 numeric policy; nothing after.
    p->source = read_desc(c, nsym);
    p->indices = read_desc(c, nsym);
    p->result = read_desc(c, nsym);
    p->axis = c.u32();
    p->policy = c.u8();
    if (c.left())
      c.reject(c.pos(), "trailing bytes after indexed plan");
    const std::string why = validate_indexed(*p);
    if (!why.empty())
      c.reject(c.pos(), why);
    return p;
  }
  p->source = read_desc(c, nsym);
  p->result = read_desc(c, nsym);
  const size_t layout_at = c.pos();
  read_layout(c, nsym, p->layout);
  const size_t stages_at = c.pos();
  const uint32_t ns = c.count("stage count");
  std::vector<size_t> stage_at;
  for (uint32_t i = 0; i < ns; ++i) {
    stage_at.push_back(c.pos());
    p->stages.push_back(read_stage(c, nsym, p->result.extents.size()));
  }
  const size_t fills_at = c.pos();
  const uint32_t nf = c.count("fill count");
  std::vector<size_t> fill_at;
  for (uint32_t i = 0; i < nf; ++i) {
    fill_at.push_back(c.pos());
    PlanFill f;
    f.axis = c.u32();
    f.stage = c.u32();
    f.type = read_type(c);
    f.bits = c.u64();
    p->fills.push_back(f);
  }
  if (c.left())
    c.reject(c.pos(), "trailing bytes after fills section");
  validate_typed(c, *p, layout_at, stages_at, stage_at, fills_at, fill_at);
  return p;
}

std::string validate_indexed(const Plan &p) {
  auto is_const = [](const Expr &e) { return e.size() == 1 && e[0].op == kPushConst; };
  for (const TensorDesc *d : {&p.source, &p.indices, &p.result}) {
    if (d->extents.empty() || !d->strides.empty() || !is_const(d->offset) ||
        d->offset[0].value != 0)
      return "indexed plan requires dense zero-offset positive-rank descriptors";
    for (const Expr &e : d->extents)
      if (is_const(e) && e[0].value <= 0)
        return "indexed plan extents must be positive";
  }
  if (p.axis != 0 || p.indices.extents.size() != 1 || p.indices.type.kind != kInteger ||
      (p.indices.type.bits != 32 && p.indices.type.bits != 64))
    return "indexed plan requires axis 0 and rank-one i32/i64 indices";
  if (p.source.extents.size() != p.result.extents.size())
    return "indexed plan source/result rank mismatch";
  // Constant extents must already agree: result[0] with the index count,
  // result[i] with source[i] for i > 0.
  for (size_t i = 0; i < p.result.extents.size(); ++i) {
    const Expr &a = p.result.extents[i];
    const Expr &b = i == 0 ? p.indices.extents[0] : p.source.extents[i];
    if (is_const(a) && is_const(b) && a[0].value != b[0].value)
      return "indexed plan result extent mismatch";
  }
  const DType a = p.source.type, b = p.result.type;
  const bool supported = a.f32() || a.f16() || a.i8();
  if ((a == b && supported && p.policy == kExact) ||
      (a.f32() && b.f16() && p.policy == kIeeeRne) || (a.f16() && b.f32() && p.policy == kExact))
    return std::string();
  return "indexed plan has an unsupported type/policy pair";
}

// ------------------------------------------------------------- evaluation

int64_t eval(const Expr &e, const std::vector<int64_t> &symbols,
             const std::vector<int64_t> *dims) {
  int64_t stack[64];
  std::vector<int64_t> spill;
  int64_t *st = stack;
  if (e.size() > 64) {
    spill.resize(e.size());
    st = spill.data();
  }
  size_t sp = 0;
  for (const Token &t : e) {
    switch (t.op) {
    case kPushSym:
      if (t.value < 0 || static_cast<size_t>(t.value) >= symbols.size())
        fail("bind_error", "symbol index out of range");
      st[sp++] = symbols[static_cast<size_t>(t.value)];
      break;
    case kPushConst:
      st[sp++] = t.value;
      break;
    case kPushDim:
      if (!dims)
        fail("bind_error", "PUSH_DIM is not valid in a plan expression");
      if (t.value < 0 || static_cast<size_t>(t.value) >= dims->size())
        fail("bind_error", "dimension index out of range");
      st[sp++] = (*dims)[static_cast<size_t>(t.value)];
      break;
    default: {
      if (sp < 2)
        fail("bind_error", "expression stack underflow");
      const int64_t b = st[--sp], a = st[--sp];
      int64_t r = 0;
      switch (t.op) {
      case kAdd:
        if (__builtin_add_overflow(a, b, &r))
          fail("bind_error", "integer overflow in add");
        break;
      case kSub:
        if (__builtin_sub_overflow(a, b, &r))
          fail("bind_error", "integer overflow in sub");
        break;
      case kMul:
        if (__builtin_mul_overflow(a, b, &r))
          fail("bind_error", "integer overflow in mul");
        break;
      case kFloorDiv:
        r = floor_div(a, b);
        break;
      case kMod: {
        const int64_t q = floor_div(a, b);
        int64_t prod;
        if (__builtin_mul_overflow(q, b, &prod) || __builtin_sub_overflow(a, prod, &r))
          fail("bind_error", "integer overflow in mod");
        break;
      }
      default:
        fail("bind_error", "unknown expression opcode");
      }
      st[sp++] = r;
    }
    }
  }
  if (sp != 1)
    fail("bind_error", "expression did not evaluate to a single value");
  return st[0];
}

// ---------------------------------------------------------------- binding

namespace {

std::vector<int64_t> resolve(const std::vector<std::string> &names,
                             const std::map<std::string, int64_t> &given) {
  for (const auto &kv : given)
    if (std::find(names.begin(), names.end(), kv.first) == names.end())
      fail("bind_error", "unknown symbol in binding: " + kv.first);
  std::vector<int64_t> out;
  for (const std::string &n : names) {
    auto it = given.find(n);
    if (it == given.end())
      fail("bind_error", "unbound symbol: " + n);
    out.push_back(it->second);
  }
  return out;
}

int64_t field(const Expr &e, const std::vector<int64_t> &syms, const std::string &what) {
  try {
    return eval(e, syms);
  } catch (const Error &err) {
    fail("bind_error", what + ": " + err.message);
  }
}

struct Ax {
  int64_t extent, src, dst;
  bool padded = false;
  int64_t lo = 0, hi = 0;
  uint64_t bits = 0;
};

BoundLayout bind_layout(const LayoutPlan &L, const std::vector<int64_t> &syms) {
  for (const auto &d : L.divisibility) {
    if (d.second <= 0)
      fail("bind_error", "divisibility divisor must be positive");
    const int64_t v = field(d.first, syms, "divisibility expr");
    if (v % d.second != 0)
      fail("bind_error", "divisibility violated: value " + std::to_string(v) +
                             " not divisible by " + std::to_string(d.second));
  }
  if (L.axes.empty())
    fail("bind_error", "plan must have >= 1 axis (v0)");
  std::vector<Ax> ax;
  for (const PlanAxis &a : L.axes) {
    Ax x{field(a.extent, syms, "axis extent"), field(a.src_stride, syms, "axis src_stride"),
         field(a.dst_stride, syms, "axis dst_stride")};
    if (x.extent < 1)
      fail("bind_error", "axis extent must be >= 1 (v0 rejects zero/negative)");
    if (x.src < 0 || x.dst < 0)
      fail("bind_error", "strides must be non-negative in v0");
    ax.push_back(x);
  }
  for (const PlanPad &p : L.pads) {
    const int64_t lo = field(p.lo, syms, "pad lo"), hi = field(p.hi, syms, "pad hi");
    if (p.axis >= ax.size())
      fail("bind_error", "pad dst_axis out of range");
    Ax &a = ax[p.axis];
    a.padded = true;
    a.lo = lo;
    a.hi = hi;
    a.bits = p.bits;
    if (lo < 0 || hi < 0)
      fail("bind_error", "pad width negative");
    if (L.runtime_pad_check) {
      if (p.axis >= L.dst.extents.size())
        fail("bind_error", "pad dst_axis out of range for dst extents");
      const int64_t want = field(L.dst.extents[p.axis], syms, "dst extent");
      int64_t sum;
      if (__builtin_add_overflow(a.extent, lo, &sum) || __builtin_add_overflow(sum, hi, &sum))
        fail("bind_error", "overflow in pad-range check");
      if (sum != want)
        fail("bind_error", "pad range inconsistent: extent + lo + hi (" + std::to_string(sum) +
                               ") != dst extent (" + std::to_string(want) + ")");
    }
  }
  // Merge neighbours that are contiguous on both sides (never padded ones),
  // to a fixpoint; `span[c]` counts the plan axes folded into axis c.
  std::vector<size_t> span(ax.size(), 1);
  for (bool merged = true; merged;) {
    merged = false;
    for (size_t k = 0; k + 1 < ax.size(); ++k) {
      const Ax &o = ax[k], &i = ax[k + 1];
      if (o.padded || i.padded)
        continue;
      int64_t sp, dp, ep;
      if (!mul_ok(i.src, i.extent, sp) || !mul_ok(i.dst, i.extent, dp) ||
          !mul_ok(o.extent, i.extent, ep))
        continue;
      if (o.src != sp || o.dst != dp)
        continue;
      ax[k] = Ax{ep, i.src, i.dst};
      ax.erase(ax.begin() + static_cast<long>(k) + 1);
      span[k] += span[k + 1];
      span.erase(span.begin() + static_cast<long>(k) + 1);
      merged = true;
      break;
    }
  }
  std::vector<uint32_t> to_coalesced;
  for (size_t c = 0; c < span.size(); ++c)
    for (size_t j = 0; j < span[c]; ++j)
      to_coalesced.push_back(static_cast<uint32_t>(c));

  BoundLayout b;
  b.perm = L.perm;
  const uint32_t bits = L.dst.type.bits;
  if (bits == 0 || bits % 8)
    fail("bind_error", "element type bitwidth must be a positive multiple of 8 in v0");
  b.element_size = bits / 8;
  b.no_copy = L.no_copy;
  for (const auto &a : L.alignment) {
    if (a.first >= L.axes.size())
      fail("bind_error", "alignment axis out of range");
    b.alignment.emplace_back(to_coalesced[a.first], a.second);
  }
  int64_t elements = 1;
  for (size_t k = 0; k < ax.size(); ++k) {
    b.extents.push_back(ax[k].extent);
    b.src_strides.push_back(ax[k].src);
    b.dst_strides.push_back(ax[k].dst);
    int64_t padded = ax[k].extent;
    if (ax[k].padded) {
      b.pads.push_back(BoundPad{static_cast<int>(k), ax[k].lo, ax[k].hi, ax[k].bits});
      if (__builtin_add_overflow(padded, ax[k].lo, &padded) ||
          __builtin_add_overflow(padded, ax[k].hi, &padded))
        fail("bind_error", "overflow computing padded extent");
    }
    if (!mul_ok(elements, padded, elements))
      fail("bind_error", "overflow computing total element count");
  }
  if (!mul_ok(elements, static_cast<int64_t>(b.element_size), b.total_bytes))
    fail("bind_error", "overflow computing total bytes");
  const Ax &inner = ax.back();
  b.inner_run = (inner.src == 1 && inner.dst == 1) ? inner.extent : 1;
  return b;
}

std::vector<int64_t> dense_extents(const TensorDesc &d, const std::vector<int64_t> &syms,
                                   const std::string &what) {
  std::vector<int64_t> ext;
  for (const Expr &e : d.extents)
    ext.push_back(field(e, syms, what));
  if (ext.empty())
    fail("bind_error", what + ": rank must be >= 1");
  for (int64_t e : ext)
    if (e < 1)
      fail("bind_error", what + ": extents must be >= 1");
  if (field(d.offset, syms, what) != 0)
    fail("bind_error", what + ": only zero offsets are supported");
  if (!d.strides.empty()) {
    int64_t running = 1;
    for (size_t k = ext.size(); k-- > 0;) {
      if (field(d.strides[k], syms, what) != running)
        fail("bind_error", what + ": only dense row-major strides are supported");
      if (!mul_ok(running, ext[k], running))
        fail("bind_error", what + ": stride product overflows");
    }
  }
  return ext;
}

void check_values(const BoundParam &p, bool is_scale, uint8_t policy) {
  const uint32_t w = p.type.width();
  for (int64_t i = 0; i < p.length; ++i) {
    const uint8_t *el = p.bytes.data() + static_cast<size_t>(i) * w;
    if (is_scale) {
      float v;
      std::memcpy(&v, el, 4);
      if (!std::isfinite(v) || !(v > 0.0f))
        fail("bind_error", "scale: scale must be finite and strictly positive");
      continue;
    }
    uint64_t bits = 0;
    std::memcpy(&bits, el, w);
    const int64_t zp = sign_extend(bits, p.type.bits);
    if (zp < -128 || zp > 127)
      fail("bind_error", "zero_point: zero point must lie in [-128, 127]");
    if (policy == kSymmetricRne && zp != 0)
      fail("bind_error", "zero_point: symmetric_rne admits only the zero point 0");
  }
}

} // namespace

std::unique_ptr<Bound> bind(const Plan &plan, const std::map<std::string, int64_t> &symbols,
                            const std::map<std::string, ParamValue> &params) {
  if (plan.version == 2)
    fail("bind_error", "indexed (wire v2) plans bind with their index operand");
  auto out = std::make_unique<Bound>();
  out->symbols = resolve(plan.symbols, symbols);
  if (plan.version == 0) {
    if (!params.empty())
      fail("bind_error", "layout plans take no parameters");
    out->layout = bind_layout(plan.layout, out->symbols);
    return out;
  }
  out->typed = true;
  try {
    out->layout = bind_layout(plan.layout, out->symbols);
  } catch (const Error &e) {
    fail("bind_error", "layout: " + e.message);
  }
  const auto &syms = out->symbols;
  out->source_extents = dense_extents(plan.source, syms, "source");
  out->result_extents = dense_extents(plan.result, syms, "result");
  out->source_type = plan.source.type;
  out->result_type = plan.result.type;
  if (!out->source_type.width() || !out->result_type.width())
    fail("bind_error", "element type bitwidth must be a positive multiple of 8");
  out->fills = plan.fills;

  std::set<std::string> used;
  for (const PlanStage &s : plan.stages) {
    BoundStage b;
    b.transform = s.transform;
    b.policy = s.policy;
    b.in = s.in;
    b.out = s.out;
    b.axis = s.axis;
    b.has_channel = s.has_channel;
    b.channel = s.channel;
    for (const Expr &e : s.shape)
      b.shape.push_back(field(e, syms, "stage shape"));
    for (int64_t e : b.shape)
      if (e < 1)
        fail("bind_error", "stage shape extents must be >= 1");
    if (s.axis >= 0 && static_cast<uint64_t>(s.axis) >= b.shape.size())
      fail("bind_error", "stage channel axis out of range");
    for (int role = 0; role < 2; ++role) {
      const StageParam &decl = role == 0 ? s.scale : s.zero_point;
      BoundParam &tgt = role == 0 ? b.scale : b.zero_point;
      if (decl.kind == kParamNone)
        continue;
      const int64_t expected = decl.rank == 0 ? 1 : b.shape[static_cast<size_t>(s.axis)];
      const uint32_t w = decl.type.width();
      if (!w)
        fail("bind_error", "parameter element type bitwidth must be a positive multiple of 8");
      if (decl.kind == kParamInline) {
        tgt.present = true;
        tgt.type = decl.type;
        tgt.length = static_cast<int64_t>(decl.inline_bits.size());
        for (uint64_t v : decl.inline_bits)
          for (uint32_t i = 0; i < w; ++i)
            tgt.bytes.push_back(static_cast<uint8_t>(v >> (8 * i)));
        if (tgt.length != expected)
          fail("bind_error", "inline parameter holds " + std::to_string(tgt.length) +
                                 " values but the channel extent is " + std::to_string(expected));
      } else {
        auto it = params.find(decl.name);
        if (it == params.end())
          fail("bind_error", "unbound parameter: " + decl.name);
        used.insert(decl.name);
        const ParamValue &v = it->second;
        const std::string q = "parameter '" + decl.name + "'";
        if (v.type != decl.type)
          fail("bind_error", q + " element type differs from its declaration");
        if (v.extents.size() != decl.rank)
          fail("bind_error", q + " rank differs from its declaration");
        const int64_t declared =
            decl.rank == 1 ? field(decl.extents[0], syms, "parameter extent") : 1;
        if (declared != expected)
          fail("bind_error", q + " declares length " + std::to_string(declared) +
                                 " but the channel extent is " + std::to_string(expected));
        const int64_t have = decl.rank == 0 ? 1 : v.extents[0];
        if (have != expected)
          fail("bind_error", q + " has length " + std::to_string(have) +
                                 " but the channel extent is " + std::to_string(expected));
        int64_t need;
        if (!mul_ok(expected, static_cast<int64_t>(w), need))
          fail("bind_error", "parameter byte count overflows");
        if (v.bytes.size() != static_cast<size_t>(need))
          fail("bind_error", q + " has " + std::to_string(v.bytes.size()) + " bytes, expected " +
                                 std::to_string(need));
        tgt.present = true;
        tgt.type = decl.type;
        tgt.length = expected;
        tgt.bytes = v.bytes;
        tgt.name = decl.name;
      }
      check_values(tgt, role == 0, s.policy);
      out->parameter_bytes += static_cast<int64_t>(tgt.bytes.size());
    }
    out->stages.push_back(std::move(b));
  }
  for (const auto &kv : params)
    if (!used.count(kv.first))
      fail("bind_error", "unknown parameter in binding: " + kv.first);

  // Footprints per boundary: pads count from the stage they enter at.
  int64_t src_elems = 1;
  for (int64_t e : out->source_extents)
    if (!mul_ok(src_elems, e, src_elems))
      fail("bind_error", "source element count overflows");
  if (!mul_ok(src_elems, static_cast<int64_t>(out->source_type.width()), out->source_bytes))
    fail("bind_error", "source byte count overflows");
  std::vector<int64_t> ax_ext;
  for (const PlanAxis &a : plan.layout.axes)
    ax_ext.push_back(field(a.extent, syms, "layout axis extent"));
  std::vector<int64_t> pad_w(ax_ext.size(), 0);
  std::vector<uint32_t> pad_stage(ax_ext.size(), 0);
  for (const PlanPad &p : plan.layout.pads) {
    const int64_t lo = field(p.lo, syms, "pad lo"), hi = field(p.hi, syms, "pad hi");
    int64_t w;
    if (lo < 0 || hi < 0 || __builtin_add_overflow(lo, hi, &w))
      fail("bind_error", "pad widths must be non-negative");
    pad_w[p.axis] = w;
    for (const PlanFill &f : plan.fills)
      if (f.axis == p.axis)
        pad_stage[p.axis] = f.stage;
  }
  for (uint32_t k = 0; k <= plan.stages.size(); ++k) {
    const DType t = k == 0 ? out->source_type : plan.stages[k - 1].out;
    int64_t n = 1;
    for (size_t a = 0; a < ax_ext.size(); ++a) {
      int64_t e = ax_ext[a];
      if (pad_w[a] && pad_stage[a] <= k && __builtin_add_overflow(e, pad_w[a], &e))
        fail("bind_error", "padded extent overflows");
      if (!mul_ok(n, e, n))
        fail("bind_error", "stage element count overflows");
    }
    if (!t.width())
      fail("bind_error", "stage element type bitwidth must be a positive multiple of 8");
    int64_t bytes;
    if (!mul_ok(n, static_cast<int64_t>(t.width()), bytes))
      fail("bind_error", "stage byte count overflows");
    out->bytes_at.push_back(bytes);
    if (k == plan.stages.size()) {
      int64_t res = 1;
      for (int64_t e : out->result_extents)
        if (!mul_ok(res, e, res))
          fail("bind_error", "result element count overflows");
      out->destination_bytes = bytes;
      if (bytes != out->layout.total_bytes)
        fail("bind_error", "layout footprint (" + std::to_string(out->layout.total_bytes) +
                               " bytes) disagrees with the result descriptor (" +
                               std::to_string(bytes) + " bytes)");
      if (res != n)
        fail("bind_error", "result descriptor element count disagrees with the layout");
    }
  }
  return out;
}

std::unique_ptr<Bound> bind_indexed(const Plan &plan,
                                    const std::map<std::string, int64_t> &symbols,
                                    DType index_type, const std::vector<int64_t> &index_extents,
                                    const void *index_data, size_t index_bytes) {
  if (plan.version != 2)
    fail("bind_error", "bind_indexed needs an indexed (wire v2) plan");
  {
    const std::string why = validate_indexed(plan);
    if (!why.empty())
      fail("bind_error", why);
  }
  auto out = std::make_unique<Bound>();
  out->symbols = resolve(plan.symbols, symbols);
  const auto &syms = out->symbols;
  out->table_extents = dense_extents(plan.source, syms, "source");
  const std::vector<int64_t> ind = dense_extents(plan.indices, syms, "indices");
  out->result_extents = dense_extents(plan.result, syms, "result");
  if (index_extents != ind || index_type != plan.indices.type)
    fail("bind_error", "index operand dtype/extents do not match the plan");
  std::vector<int64_t> selected = out->table_extents;
  selected[0] = ind[0];
  if (selected != out->result_extents)
    fail("bind_error", "indexed result shape does not match source and indices");
  const int64_t count = ind[0];
  const uint32_t iw = index_type.width();
  int64_t ibytes;
  if (!mul_ok(count, static_cast<int64_t>(iw), ibytes) ||
      static_cast<uint64_t>(ibytes) != index_bytes)
    fail("bind_error", "index operand byte size mismatch or overflow");
  int64_t row = 1;
  for (size_t i = 1; i < out->table_extents.size(); ++i)
    if (!mul_ok(row, out->table_extents[i], row))
      fail("bind_error", "indexed row size overflow");
  out->source_type = plan.source.type;
  out->result_type = plan.result.type;
  const int64_t sw = out->source_type.width(), rw = out->result_type.width();
  const int64_t rows = out->table_extents[0];
  int64_t table_elems, elems;
  if (!mul_ok(rows, row, table_elems) || !mul_ok(table_elems, sw, out->table_bytes) ||
      !mul_ok(count, row, elems) || !mul_ok(elems, sw, out->source_bytes) ||
      !mul_ok(elems, rw, out->destination_bytes))
    fail("bind_error", "indexed tensor size overflow");
  // Snapshot the index values (little-endian, sign-extended) and check them.
  const uint8_t *raw = static_cast<const uint8_t *>(index_data);
  if (count && !raw)
    fail("bind_error", "index operand bytes are missing");
  out->indices.resize(static_cast<size_t>(count));
  bool in_range = true;
  for (int64_t i = 0; i < count; ++i) {
    uint64_t bits = 0;
    std::memcpy(&bits, raw + i * iw, iw);
    const int64_t v = sign_extend(bits, index_type.bits);
    out->indices[static_cast<size_t>(i)] = v;
    in_range &= v >= 0 && v < rows;
  }
  if (!in_range)
    fail("bind_error", "index_out_of_range: index_select row is outside the source");
  out->indexed = true;
  out->typed = true;
  out->index_type = index_type;
  out->table_rows = rows;
  out->row_elements = row;
  out->parameter_bytes = ibytes;
  out->source_extents = selected;
  // The selected rows relocate by identity: one coalesced axis of every
  // selected element, dense on both sides.
  BoundLayout &L = out->layout;
  L.extents = {elems};
  L.src_strides = {1};
  L.dst_strides = {1};
  L.perm = {0};
  L.element_size = static_cast<uint32_t>(rw);
  L.total_bytes = out->destination_bytes;
  L.inner_run = elems;
  out->bytes_at.push_back(out->source_bytes);
  if (out->source_type != out->result_type) {
    BoundStage st;
    st.transform = kCast;
    st.policy = plan.policy;
    st.in = out->source_type;
    st.out = out->result_type;
    st.shape = selected;
    out->stages.push_back(std::move(st));
    out->bytes_at.push_back(out->destination_bytes);
  }
  return out;
}

} // namespace relx
