// program.cpp - turn a bound plan into device launch programs.
//
// prepareProgram's checks (libreloc/src/TypedExecute.cpp:292-403) are
// restated here: every stage must be one of the implemented policy tables,
// quantize reciprocals are formed once in binary32 from the declared scale,
// and channel maps that are a single result coordinate (possibly `dN mod K`
// with K >= the extent) are recognised so the fast kernels can index
// parameters without evaluating expressions. The fill written into pads is
// the original fill folded to the result type (fillAt,
// libreloc/src/TypedExecute.cpp:422-464).
#include "runtime.h"

#include <algorithm>
#include <cstring>

namespace relx {

namespace {

FastDiv make_div(int64_t d64) {
  FastDiv f{};
  const uint32_t d = static_cast<uint32_t>(d64 < 1 ? 1 : d64);
  f.d = d;
  uint32_t s = 0;
  while (s < 32 && (uint64_t{1} << s) < d)
    ++s;
  f.s = s;
  // m = floor(2^32 * (2^s - d) / d) + 1
  const unsigned __int128 num = (static_cast<unsigned __int128>(1) << 32) *
                                ((static_cast<unsigned __int128>(1) << s) - d);
  f.m = static_cast<uint32_t>(num / d + 1);
  return f;
}

uint8_t op_of(const BoundStage &s) {
  if (s.transform == kCast) {
    if (s.in.f32() && s.out.f16() && s.policy == kIeeeRne)
      return kOpF32toF16;
    if (s.in.f16() && s.out.f32() && s.policy == kExact)
      return kOpF16toF32;
    if (s.in.f32() && s.out.bf16() && s.policy == kIeeeRne)
      return kOpF32toBF16;
    if (s.in.bf16() && s.out.f32() && s.policy == kExact)
      return kOpBF16toF32;
    fail("unsupported_stage",
         "only cast f32->f16/bf16 ieee_rne and f16/bf16->f32 exact are implemented");
  }
  if (s.transform == kQuantize) {
    if (!(s.in.f32() && s.out.i8() && s.policy == kSymmetricRne))
      fail("unsupported_stage", "only quantize f32->s8 symmetric_rne is implemented");
    return kOpQuantize;
  }
  if (!(s.in.i8() && s.out.f32() && s.policy == kAffine))
    fail("unsupported_stage", "only dequantize s8->f32 affine is implemented");
  return kOpDequantize;
}

int64_t sext(uint64_t bits, uint32_t width) {
  if (width >= 64)
    return static_cast<int64_t>(bits);
  const uint64_t mask = (uint64_t{1} << width) - 1;
  uint64_t v = bits & mask;
  if (v >> (width - 1))
    v |= ~mask;
  return static_cast<int64_t>(v);
}

} // namespace

// --------------------------------------------------------------- stages

void prepare_stages(const Bound &b, Prepared &p) {
  const size_t rank = b.result_extents.size();
  p.res_strides.assign(rank, 1);
  for (size_t j = rank; j-- > 1;)
    p.res_strides[j - 1] = p.res_strides[j] * b.result_extents[j];
  for (size_t k = 0; k < b.stages.size(); ++k) {
    const BoundStage &s = b.stages[k];
    HostStage h;
    h.op = op_of(s);
    h.in_width = s.in.width();
    h.out_width = s.out.width();
    const std::string where = "stage " + std::to_string(k) + ": ";
    if (h.op == kOpQuantize || h.op == kOpDequantize) {
      if (!s.scale.present || !s.scale.type.f32() ||
          s.scale.bytes.size() != static_cast<size_t>(s.scale.length) * 4)
        fail("invalid_parameter", where + "scale is absent or malformed");
      h.scale.resize(static_cast<size_t>(s.scale.length));
      std::memcpy(h.scale.data(), s.scale.bytes.data(), s.scale.bytes.size());
      for (float v : h.scale)
        if (!(v > 0.0f) || v == __builtin_inff())
          fail("invalid_parameter", where + "scale is not finite and strictly positive");
      h.zero_point.assign(1, 0);
      if (s.zero_point.present) {
        const uint32_t w = s.zero_point.type.width();
        if (s.zero_point.type.kind != kInteger || !w || w > 8 ||
            s.zero_point.bytes.size() != static_cast<size_t>(s.zero_point.length) * w)
          fail("invalid_parameter", where + "zero point is malformed");
        h.zero_point.resize(static_cast<size_t>(s.zero_point.length));
        for (int64_t i = 0; i < s.zero_point.length; ++i) {
          uint64_t raw = 0;
          std::memcpy(&raw, s.zero_point.bytes.data() + i * w, w);
          const int64_t v = sext(raw, s.zero_point.type.bits);
          if (v < -128 || v > 127)
            fail("invalid_parameter", where + "zero point outside [-128, 127]");
          h.zero_point[static_cast<size_t>(i)] = static_cast<int32_t>(v);
        }
      }
      if (h.op == kOpQuantize) {
        for (int32_t zp : h.zero_point)
          if (zp != 0)
            fail("invalid_parameter", where + "symmetric_rne admits only zero point 0");
        h.inv.resize(h.scale.size());
        for (size_t i = 0; i < h.scale.size(); ++i)
          h.inv[i] = 1.0f / h.scale[i]; // fl32(1/scale), formed once
      }
    }
    if (s.has_channel) {
      if (h.scale.empty())
        fail("invalid_parameter", where + "per-channel stage without scales");
      h.len = static_cast<int64_t>(h.scale.size());
      if (h.zero_point.size() > 1 && h.zero_point.size() != h.scale.size())
        fail("invalid_parameter", where + "zero point length disagrees with the scale");
      h.mode = kChanExpr;
      const Expr &c = s.channel;
      if (!c.empty() && c[0].op == kPushDim && c[0].value >= 0 &&
          static_cast<size_t>(c[0].value) < rank) {
        const int dim = static_cast<int>(c[0].value);
        bool is_dim = c.size() == 1;
        if (c.size() == 3 && c[2].op == kMod && (c[1].op == kPushConst || c[1].op == kPushSym)) {
          const int64_t mod = c[1].op == kPushConst ? c[1].value
                                                    : b.symbols[static_cast<size_t>(c[1].value)];
          if (mod > 0 && b.result_extents[static_cast<size_t>(dim)] <= mod)
            is_dim = true;
        }
        if (is_dim) {
          h.mode = kChanDim;
          h.dim = dim;
        }
      }
      if (h.mode == kChanExpr) {
        for (const Token &t : c) {
          ChanToken ct{t.op, 0, t.value};
          if (t.op == kPushSym) {
            ct.op = kPushConst;
            ct.value = b.symbols[static_cast<size_t>(t.value)];
          }
          h.tokens.push_back(ct);
        }
      }
    } else {
      h.mode = kChanNone;
      h.len = 1;
      if (h.scale.size() > 1 || h.zero_point.size() > 1)
        fail("invalid_parameter", where + "per-tensor stage with more than one parameter");
    }
    p.stages.push_back(std::move(h));
  }
}

// Fill bits at boundary `to` (every pad settled), folded through the stages
// after each pad's entry stage; nullopt-like `has` = false without pads.
bool fill_at(const Bound &b, const Prepared &p, uint32_t to, uint64_t &bits) {
  if (b.fills.empty()) {
    if (!b.typed && !b.layout.pads.empty()) {
      bits = b.layout.pads.front().bits;
      return true;
    }
    return false;
  }
  bool have = false;
  for (const PlanFill &f : b.fills) {
    if (f.stage > to)
      fail("pads_not_settled", "a pad enters after boundary " + std::to_string(to));
    uint64_t v = f.bits;
    for (uint32_t k = f.stage; k < to; ++k) {
      const HostStage &s = p.stages[k];
      if (s.mode != kChanNone)
        fail("fill_crosses_channel_stage",
             "a pad fill would cross per-channel stage " + std::to_string(k));
      v = host_apply(s, v, 0);
    }
    if (have && v != bits)
      fail("mixed_fills_unsupported",
           "pads carry different values at boundary " + std::to_string(to));
    bits = v;
    have = true;
  }
  if (to == p.stages.size() && !b.layout.pads.empty() && b.layout.pads.front().bits != bits)
    fail("fill_mismatch", "folded fill disagrees with the layout's fused fill");
  return have;
}

uint64_t host_apply(const HostStage &s, uint64_t x, int64_t c) {
  switch (s.op) {
  case kOpF32toF16:
    return f32_to_f16_bits(static_cast<uint32_t>(x));
  case kOpF16toF32:
    return f16_to_f32_bits(static_cast<uint16_t>(x));
  case kOpF32toBF16:
    return f32_to_bf16_bits(static_cast<uint32_t>(x));
  case kOpBF16toF32:
    return bf16_to_f32_bits(static_cast<uint16_t>(x));
  case kOpQuantize: {
    float f;
    const uint32_t b = static_cast<uint32_t>(x);
    std::memcpy(&f, &b, 4);
    return static_cast<uint8_t>(quantize_one(f, s.inv[static_cast<size_t>(c)]));
  }
  default: {
    const int32_t q = static_cast<int8_t>(static_cast<uint8_t>(x));
    const int32_t zp = s.zero_point.size() == 1 ? s.zero_point[0]
                                                : s.zero_point[static_cast<size_t>(c)];
    const float y = static_cast<float>(q - zp) * s.scale[static_cast<size_t>(c)];
    uint32_t r;
    std::memcpy(&r, &y, 4);
    return r;
  }
  }
}

// ------------------------------------------------------------ programs

namespace {

bool dense_dst(const BoundLayout &L, const std::vector<int64_t> &pext) {
  int64_t running = 1;
  for (size_t k = pext.size(); k-- > 0;) {
    if (L.dst_strides[k] != running)
      return false;
    running *= pext[k];
  }
  return true;
}

// Per-vector channel behaviour for V consecutive destination elements whose
// dense offset is a multiple of V: 0 constant, 1 +1 per element, -1 neither.
int vec_mode(const HostStage &s, const Prepared &p, const Bound &b, int64_t V) {
  if (s.mode == kChanNone)
    return 0;
  if (s.mode != kChanDim)
    return -1;
  const int64_t rs = p.res_strides[static_cast<size_t>(s.dim)];
  const int64_t re = b.result_extents[static_cast<size_t>(s.dim)];
  if (re > s.len)
    return -1; // a coordinate could leave the table: keep the checked kernel
  if (rs % V == 0)
    return 0;
  if (rs == 1 && re % V == 0)
    return 1;
  return -1;
}

} // namespace

std::unique_ptr<DeviceProgram> build_program(const Bound &b, const Prepared &p, uint32_t k) {
  const BoundLayout &L = b.layout;
  const int r = static_cast<int>(L.extents.size());
  if (r > kMaxRank)
    fail("unsupported_layout", "more than " + std::to_string(kMaxRank) + " coalesced axes");
  const uint32_t nst = static_cast<uint32_t>(p.stages.size());
  if (k > nst)
    fail("invalid_boundary", "wire boundary beyond the last stage");
  if (nst - k > static_cast<uint32_t>(kMaxStages))
    fail("unsupported_stage", "too many device stages");
  auto dp = std::make_unique<DeviceProgram>();
  dp->boundary = k;
  KArgs &a = dp->base;
  std::memset(&a, 0, sizeof(a));
  a.rank = r;
  const int win = b.typed ? static_cast<int>(k == 0 ? b.source_type.width()
                                                    : p.stages[k - 1].out_width)
                          : static_cast<int>(L.element_size);
  const int wout = static_cast<int>(L.element_size);
  a.win = win;
  a.wout = wout;
  std::vector<int64_t> pext(static_cast<size_t>(r)), lo(static_cast<size_t>(r), 0);
  bool any_pad = false, inner_pad = false;
  for (int i = 0; i < r; ++i) {
    pext[static_cast<size_t>(i)] = L.extents[static_cast<size_t>(i)];
    a.vext[i] = L.extents[static_cast<size_t>(i)];
    a.ss[i] = L.src_strides[static_cast<size_t>(i)];
    a.ds[i] = L.dst_strides[static_cast<size_t>(i)];
  }
  for (const BoundPad &pd : L.pads) {
    pext[static_cast<size_t>(pd.axis)] += pd.lo + pd.hi;
    lo[static_cast<size_t>(pd.axis)] = pd.lo;
    any_pad = true;
    if (pd.axis == r - 1)
      inner_pad = true;
  }
  for (int i = 0; i < r; ++i) {
    a.pext[i] = pext[static_cast<size_t>(i)];
    a.lo[i] = lo[static_cast<size_t>(i)];
  }
  uint64_t fill = 0;
  a.has_fill = fill_at(b, p, nst, fill) ? 1 : 0;
  a.fill = fill;

  // result coordinates (channels); layout plans have none
  a.res_rank = static_cast<int32_t>(b.result_extents.size());
  for (int j = 0; j < a.res_rank && j < kMaxRank; ++j) {
    a.rs[j] = p.res_strides[static_cast<size_t>(j)];
    a.re[j] = b.result_extents[static_cast<size_t>(j)];
  }
  if (a.res_rank > kMaxRank)
    fail("unsupported_layout", "result rank above the device limit");

  // stages [k, n): parameters packed into one float and one int table
  Chain &ch = a.chain;
  ch.n = static_cast<int32_t>(nst - k);
  bool needs_expr = false;
  for (uint32_t i = k; i < nst; ++i) {
    const HostStage &h = p.stages[i];
    DevStage &d = ch.st[i - k];
    d.op = h.op;
    d.mode = h.mode;
    if (h.mode == kChanDim) {
      d.ch_rs = p.res_strides[static_cast<size_t>(h.dim)];
      d.ch_re = b.result_extents[static_cast<size_t>(h.dim)];
      d.ch_rs_div = make_div(d.ch_rs);
      d.ch_re_div = make_div(d.ch_re);
    }
    d.len = static_cast<uint32_t>(h.len);
    d.scale_off = static_cast<uint32_t>(dp->pf.size());
    const std::vector<float> &f = h.op == kOpQuantize ? h.inv : h.scale;
    dp->pf.insert(dp->pf.end(), f.begin(), f.end());
    d.zp_off = static_cast<uint32_t>(dp->pi.size());
    dp->pi.insert(dp->pi.end(), h.zero_point.begin(), h.zero_point.end());
    d.zp_per_ch = h.zero_point.size() > 1 ? 1 : 0;
    if (h.mode == kChanExpr) {
      needs_expr = true;
      if (ch.ntok + static_cast<int>(h.tokens.size()) > kMaxChanTokens)
        fail("unsupported_stage", "channel expression too long for the device");
      d.tok_begin = ch.ntok;
      d.tok_count = static_cast<int32_t>(h.tokens.size());
      for (const ChanToken &t : h.tokens)
        ch.tok[ch.ntok++] = t;
    }
  }
  if (dp->pf.empty())
    dp->pf.push_back(0.0f);
  if (dp->pi.empty())
    dp->pi.push_back(0);

  int64_t wire_elems = 1;
  if (b.typed) {
    for (int64_t e : b.source_extents)
      wire_elems *= e;
  } else {
    int64_t span = 0; // layout plans: the source span the strides reach
    for (int i = 0; i < r; ++i)
      span += (a.vext[i] - 1) * a.ss[i];
    wire_elems = span + 1;
  }
  dp->wire_elems = wire_elems;
  dp->wire_bytes = wire_elems * win;
  // Bounds proofs the kernels rely on: every source offset the valid box
  // reaches lies inside the wire, every destination offset inside the result.
  int64_t src_span = 0, dst_span = 0, total = 1;
  for (int i = 0; i < r; ++i) {
    if (a.ss[i] < 0 || a.ds[i] < 0)
      fail("unsupported_layout", "negative stride");
    int64_t t;
    if (__builtin_mul_overflow(a.vext[i] - 1, a.ss[i], &t) ||
        __builtin_add_overflow(src_span, t, &src_span) ||
        __builtin_mul_overflow(a.pext[i] - 1, a.ds[i], &t) ||
        __builtin_add_overflow(dst_span, t, &dst_span) ||
        __builtin_mul_overflow(total, a.pext[i], &total))
      fail("integer_overflow", "layout offsets overflow");
  }
  if (src_span >= wire_elems)
    fail("unsupported_layout", "the plan reads beyond its source (span " +
                                   std::to_string(src_span + 1) + " > " +
                                   std::to_string(wire_elems) + " elements)");
  dp->dst_elems = std::max(total, dst_span + 1);

  // ------------------------------------------------------ family choice
  const bool widths_ok = (win == 1 || win == 2 || win == 4) && (wout == 1 || wout == 2 || wout == 4);
  const bool dense = dense_dst(L, pext);
  int family = kFamGeneric;
  const int V = widths_ok ? 16 / std::min(win, wout) : 0;
  auto channels_ok = [&](int64_t vlen) {
    for (uint32_t i = k; i < nst; ++i) {
      const int m = vec_mode(p.stages[i], p, b, vlen);
      if (m < 0)
        return false;
      ch.st[i - k].vec = static_cast<uint8_t>(m);
    }
    return true;
  };
  if (widths_ok && dense && !needs_expr) {
    // stream: innermost axis contiguous on both sides, unpadded
    if (a.ss[r - 1] == 1 && a.ds[r - 1] == 1 && !inner_pad && a.vext[r - 1] % V == 0) {
      bool ok = true;
      for (int i = 0; i < r - 1; ++i)
        ok = ok && a.ss[i] % V == 0;
      if (ok && channels_ok(V)) {
        family = kFamStream;
        a.vec = V;
      }
    }
    // transpose: dst-inner axis has a source stride, another axis is
    // source-contiguous; tile-aligned extents, no pads
    if (family == kFamGeneric && !any_pad && r >= 2 && a.ss[r - 1] != 1) {
      int qa = -1;
      for (int i = 0; i < r - 1; ++i)
        if (a.ss[i] == 1 && a.vext[i] > 1)
          qa = i;
      const int VI = 16 / win, VO = 16 / wout;
      if (qa >= 0 && a.vext[qa] % 64 == 0 && a.vext[r - 1] % 64 == 0 && a.ss[r - 1] % VI == 0 &&
          a.ds[qa] % VO == 0) {
        bool ok = true;
        for (int i = 0; i < r - 1; ++i)
          if (i != qa)
            ok = ok && a.ss[i] % VI == 0 && a.ds[i] % VO == 0;
        int64_t tiles = (a.vext[qa] / 64) * (a.vext[r - 1] / 64);
        for (int i = 0; i < r - 1; ++i)
          if (i != qa)
            tiles *= a.vext[i];
        ok = ok && tiles < (int64_t{1} << 22); // one block per tile
        if (ok && channels_ok(VO)) {
          family = kFamTranspose;
          dp->qa = qa;
          dp->ca = r - 1;
        }
      }
    }
    // interleave: [batch..., P, C(pad)] planar source
    if (family == kFamGeneric && r >= 2 && a.ss[r - 1] != 1 && a.ss[r - 2] == 1 &&
        a.ds[r - 2] == pext[static_cast<size_t>(r - 1)]) {
      const int64_t cp = pext[static_cast<size_t>(r - 1)];
      const int G = 16 / win;
      bool pa_pad = lo[static_cast<size_t>(r - 2)] != 0 || pext[static_cast<size_t>(r - 2)] != a.vext[r - 2];
      bool ok = (cp == 2 || cp == 4 || cp == 8) && !pa_pad && a.vext[r - 2] % G == 0 &&
                a.ss[r - 1] % G == 0 && (G * cp * wout) % 16 == 0;
      for (int i = 0; i < r - 2; ++i)
        ok = ok && a.ss[i] % G == 0;
      for (uint32_t i = k; i < nst; ++i)
        ok = ok && p.stages[i].mode == kChanNone;
      if (ok) {
        family = kFamInterleave;
        a.vec = G;
        a.cpad = static_cast<int32_t>(cp);
      }
    }
  }
  if (family == kFamGeneric)
    for (uint32_t i = k; i < nst; ++i)
      ch.st[i - k].vec = 0;
  dp->family = family;
  {
    // stage sequences with a compile-time kernel body
    std::vector<uint8_t> ops;
    for (uint32_t i = k; i < nst; ++i)
      ops.push_back(p.stages[i].op);
    using V8 = std::vector<uint8_t>;
    int code = kChainGeneric;
    if (ops.empty())
      code = kChainNone;
    else if (ops == V8{kOpF32toF16})
      code = kChainF32F16;
    else if (ops == V8{kOpF16toF32})
      code = kChainF16F32;
    else if (ops == V8{kOpDequantize, kOpF32toF16})
      code = kChainDeqF16;
    else if (ops == V8{kOpDequantize})
      code = kChainDeq;
    else if (ops == V8{kOpF16toF32, kOpQuantize})
      code = kChainF16Quant;
    else if (ops == V8{kOpQuantize})
      code = kChainQuant;
    a.chain_code = code;
  }
  static const char *names[] = {"generic", "stream", "transpose", "interleave"};
  dp->kernel = names[family];

  // ------------------------------------------------------- chunk axis
  dp->chunk_axis = -1;
  dp->chunk_align = 1;
  {
    int ax = -1;
    for (int i = 0; i < r; ++i)
      if (a.vext[i] > 1 && (ax < 0 || a.ss[i] > a.ss[ax]))
        ax = i;
    if (ax >= 0) {
      int64_t rest = 0;
      for (int i = 0; i < r; ++i)
        if (i != ax)
          rest += (a.vext[i] - 1) * a.ss[i];
      if (a.ss[ax] * a.vext[ax] == wire_elems && rest < a.ss[ax]) {
        dp->chunk_axis = ax;
        dp->chunk_stride = a.ss[ax];
        if (family == kFamStream && ax == r - 1)
          dp->chunk_align = V;
        else if (family == kFamTranspose && (ax == dp->qa || ax == dp->ca))
          dp->chunk_align = 64;
        else if (family == kFamInterleave && ax == r - 2)
          dp->chunk_align = a.vec;
      }
    }
  }
  return dp;
}

// Launch arguments for valid coordinates [v0, v1) of the chunk axis (the
// whole box when the axis is -1). The first/last chunk also cover the axis'
// leading/trailing pad.
KArgs box_args(const DeviceProgram &dp, int64_t v0, int64_t v1, bool first, bool last) {
  KArgs a = dp.base;
  const int r = a.rank;
  for (int i = 0; i < r; ++i) {
    a.box_lo[i] = 0;
    a.box_ext[i] = a.pext[i];
  }
  if (dp.chunk_axis >= 0) {
    const int ax = dp.chunk_axis;
    const int64_t plo = first ? 0 : v0 + a.lo[ax];
    const int64_t phi = last ? a.pext[ax] : v1 + a.lo[ax];
    a.box_lo[ax] = plo;
    a.box_ext[ax] = phi - plo;
  }
  int64_t box_total = 1;
  for (int i = 0; i < r; ++i)
    box_total *= a.box_ext[i];
  // the axes outside a 2-D block, outer first (transpose / interleave)
  auto batch = [&](int skip0, int skip1) {
    int n = 0;
    for (int i = 0; i < r; ++i) {
      if (i == skip0 || i == skip1)
        continue;
      a.b_ext[n] = a.box_ext[i];
      a.b_lo[n] = a.box_lo[i];
      a.b_pad[n] = a.lo[i];
      a.b_vext[n] = a.vext[i];
      a.b_ss[n] = a.ss[i];
      a.b_ds[n] = a.ds[i];
      a.b_div[n] = make_div(a.box_ext[i]);
      ++n;
    }
    a.nbatch = n;
  };
  switch (dp.family) {
  case kFamStream: {
    for (int i = 0; i < r; ++i)
      a.box_div[i] = make_div(i == r - 1 ? a.box_ext[i] / a.vec : a.box_ext[i]);
    a.work = box_total / a.vec;
    break;
  }
  case kFamTranspose: {
    const int qa = dp.qa, ca = dp.ca;
    batch(qa, ca);
    a.t_nq = a.box_ext[qa] / 64;
    a.t_nc = a.box_ext[ca] / 64;
    a.t_q0 = a.box_lo[qa];
    a.t_c0 = a.box_lo[ca];
    a.t_ssc = a.ss[ca];
    a.t_dsq = a.ds[qa];
    int64_t n = a.t_nq * a.t_nc;
    for (int i = 0; i < a.nbatch; ++i)
      n *= a.b_ext[i];
    a.work = n;
    break;
  }
  case kFamInterleave: {
    const int pa = r - 2, ca = r - 1;
    batch(pa, ca);
    a.i_ngroups = a.box_ext[pa] / a.vec;
    a.i_ngroups_div = make_div(a.i_ngroups);
    a.i_p0 = a.box_lo[pa];
    a.i_ssc = a.ss[ca];
    a.i_loc = a.lo[ca];
    a.i_vc = a.vext[ca];
    int64_t n = a.i_ngroups;
    for (int i = 0; i < a.nbatch; ++i)
      n *= a.b_ext[i];
    a.work = n;
    break;
  }
  default:
    for (int i = 0; i < r; ++i)
      a.box_div[i] = make_div(a.box_ext[i]);
    a.work = box_total;
  }
  a.idx32 = (box_total < (int64_t{1} << 32) && dp.dst_elems < (int64_t{1} << 32)) ? 1 : 0;
  return a;
}

} // namespace relx
