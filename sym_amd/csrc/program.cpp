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
#include <cstdlib>
#include <cstring>

#include "index.h"

// Rows of m per permute block: at most this many source bytes over all C.
#ifndef RELX_PERMUTE_SOURCE_BYTES
#define RELX_PERMUTE_SOURCE_BYTES 8192
#endif
// A permute block reads G of the C channels of each source row, at most this
// many bytes of the row (G halves from C while it is more), and the blocks run
// group by group: the resident blocks then write the result planes of one
// group, not all C. Measured on the MI355X over buffers spanning 2.4 GB, C5's
// [8,4096,32,128] f16 -> int8 launch: 74.1 us with all 32 heads per block
// (2 rows), 68.2 us with 16 (2 rows of 4 KiB), 66.3 us with 16 and one row
// per block (RELX_PERMUTE_SOURCE_BYTES), against 65.2 us for a 16-byte copy
// of the same bytes; [64,4096,..] 572 -> 498 us.
#ifndef RELX_PERMUTE_GROUP_BYTES
#define RELX_PERMUTE_GROUP_BYTES 4096
#endif


namespace relx {

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

namespace {

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
  a.fill64 = fill;
  a.fill = static_cast<uint32_t>(fill);

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
    d.ch_rs_div = make_div(1); // per tensor: entry 0
    d.ch_re_div = make_div(1);
    if (h.mode == kChanDim) {
      d.ch_rs = p.res_strides[static_cast<size_t>(h.dim)];
      d.ch_re = b.result_extents[static_cast<size_t>(h.dim)];
      if (d.ch_rs < (int64_t{1} << 32) && d.ch_re < (int64_t{1} << 32)) {
        d.ch_rs_div = make_div(d.ch_rs);
        d.ch_re_div = make_div(d.ch_re);
      }
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
  // stream items: 16 bytes on the wider side
  const int V = widths_ok ? 16 / std::max(win, wout) : 0;
  // per-channel stages in the fast kernels index with a 32-bit result offset
  const bool off32 = dp->dst_elems < (int64_t{1} << 32);
  auto channels_ok = [&](int64_t vlen) {
    for (uint32_t i = k; i < nst; ++i) {
      const int m = vec_mode(p.stages[i], p, b, vlen);
      if (m < 0 || (p.stages[i].mode == kChanDim && !off32))
        return false;
      ch.st[i - k].vec = static_cast<uint8_t>(m);
    }
    return true;
  };
  // stage sequences with a compile-time kernel body
  int chain_code = kChainGeneric;
  {
    std::vector<uint8_t> ops;
    for (uint32_t i = k; i < nst; ++i)
      ops.push_back(p.stages[i].op);
    using V8 = std::vector<uint8_t>;
    if (ops.empty())
      chain_code = kChainNone;
    else if (ops == V8{kOpF32toF16})
      chain_code = kChainF32F16;
    else if (ops == V8{kOpF16toF32})
      chain_code = kChainF16F32;
    else if (ops == V8{kOpDequantize, kOpF32toF16})
      chain_code = kChainDeqF16;
    else if (ops == V8{kOpDequantize})
      chain_code = kChainDeq;
    else if (ops == V8{kOpF16toF32, kOpQuantize})
      chain_code = kChainF16Quant;
    else if (ops == V8{kOpQuantize})
      chain_code = kChainQuant;
  }
  if (widths_ok && dense && !needs_expr && !any_pad && r >= 3 && r - 3 <= kBatchLevels) {
    // permute: destination [batch..., c, m, e] from a source holding
    // (m, c, e) contiguously -- two axes swapped above a contiguous inner
    // block (an activation's [B,S,H,D] -> [B,H,S,D])
    const int c = r - 3, m = r - 2, e = r - 1;
    const int64_t E = a.vext[e], C = a.vext[c], M = a.vext[m];
    const int VI = 16 / win;
    bool ok = a.ss[e] == 1 && a.ds[e] == 1 && a.ss[c] == E && a.ss[m] == C * E &&
              a.ds[m] == E && a.ds[c] == M * E && E % VI == 0 && (E * wout) % 16 == 0 &&
              C > 1 && M > 1;
    for (int i = 0; i < c; ++i)
      ok = ok && a.ss[i] % VI == 0;
    // G channels per block (RELX_PERMUTE_GROUP_BYTES)
    int64_t G = C;
    while (G % 2 == 0 && G * E * win > RELX_PERMUTE_GROUP_BYTES)
      G /= 2;
    // T rows of m per block: at most RELX_PERMUTE_SOURCE_BYTES of source over
    // all C (at least one row), an LDS tile of at most 32 KiB, T dividing M
    int64_t T = 0;
    if (ok) {
      T = 1;
      while (T * 2 <= M && M % (T * 2) == 0 && T * 2 * C * E * win <= RELX_PERMUTE_SOURCE_BYTES &&
             T * 2 * G * E * wout <= 32768)
        T *= 2;
      ok = T * G * E * wout <= 32768;
    }
    if (ok && channels_ok(VI)) {
      family = kFamPermute;
      a.vec = VI;
      a.p_t = static_cast<uint32_t>(T);
      a.p_g = static_cast<uint32_t>(G);
      a.p_lds = static_cast<uint32_t>(T * G * E * wout);
    }
  }
  if (family == kFamGeneric && widths_ok && dense && !needs_expr) {
    // stream: innermost axis contiguous on both sides, unpadded
    // a single contiguous axis need not be a multiple of the vector: its
    // tail (fewer than V elements) runs element-wise (prefix_launches)
    if (a.ss[r - 1] == 1 && a.ds[r - 1] == 1 && !inner_pad &&
        (a.vext[r - 1] % V == 0 || (r == 1 && a.vext[0] >= V))) {
      bool ok = true;
      for (int i = 0; i < r - 1; ++i)
        ok = ok && a.ss[i] % V == 0;
      if (ok && channels_ok(V)) {
        family = kFamStream;
        a.vec = V;
        a.nlev = r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : 8;
      }
    }
    // transpose: dst-inner axis has a source stride, another axis is
    // source-contiguous; tile-aligned extents, no pads
    if (family == kFamGeneric && !any_pad && r >= 2 && r - 2 <= kBatchLevels && a.ss[r - 1] != 1) {
      int qa = -1;
      for (int i = 0; i < r - 1; ++i)
        if (a.ss[i] == 1 && a.vext[i] > 1)
          qa = i;
      const int VI = 16 / win, VO = 16 / wout;
      // extents need not be multiples of 64: the launches split off the
      // partial tiles at the q and c edges and run them element-wise
      if (qa >= 0 && a.vext[qa] >= 64 && a.vext[r - 1] >= 64 && a.ss[r - 1] % VI == 0 &&
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
          // one-byte sources take tiles 128 q wide when q allows it (each
          // tile row then reads a whole 128-byte line); with two- and
          // four-byte results, 128 c wide too, kept in LDS as bytes, when c
          // allows it
          a.t_wq = win == 1 && a.vext[qa] % 128 == 0 ? 128 : 64;
          a.t_wc = a.t_wq == 128 && wout >= 2 && a.vext[r - 1] % 128 == 0 ? 128 : 64;
        }
      }
    }
    // interleave: [batch..., P, C(pad)] planar source
    if (family == kFamGeneric && r >= 2 && r - 2 <= kBatchLevels && a.ss[r - 1] != 1 &&
        a.ss[r - 2] == 1 && a.ds[r - 2] == pext[static_cast<size_t>(r - 1)]) {
      const int64_t cp = pext[static_cast<size_t>(r - 1)];
      const int G = interleave_pixels(win, wout, static_cast<int>(cp));
      const int64_t bo = G * cp * wout;
      bool pa_pad = lo[static_cast<size_t>(r - 2)] != 0 || pext[static_cast<size_t>(r - 2)] != a.vext[r - 2];
      bool ok = (cp == 2 || cp == 4 || cp == 8) && !pa_pad && a.vext[r - 2] % G == 0 &&
                a.ss[r - 1] % G == 0 && (bo == 4 || bo == 8 || bo % 16 == 0);
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
  a.chain_code = chain_code;
  static const char *names[] = {"generic", "stream", "transpose", "interleave", "permute"};
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
          dp->chunk_align = ax == dp->qa ? a.t_wq : a.t_wc;
        else if (family == kFamInterleave && ax == r - 2)
          dp->chunk_align = a.vec;
        // an interleave launch writes every channel of its pixels, so its
        // boxes never split the channel axis
        if (family == kFamInterleave && ax == r - 1)
          dp->chunk_axis = -1;
        // a permute block takes T rows of m and all of c and e
        if (family == kFamPermute) {
          if (ax == r - 2)
            dp->chunk_align = a.p_t;
          else if (ax >= r - 3)
            dp->chunk_axis = -1;
        }
      }
    }
  }
  return dp;
}

namespace {

struct Box {
  int64_t lo[kMaxRank], ext[kMaxRank];
};

// Work items of a box for the program's family.
int64_t box_work(const DeviceProgram &dp, const Box &b) {
  const KArgs &a = dp.base;
  const int r = a.rank;
  int64_t n = 1;
  for (int i = 0; i < r; ++i) {
    int64_t e = b.ext[i];
    if (dp.family == kFamStream && i == r - 1)
      e /= a.vec;
    else if (dp.family == kFamTranspose && (i == dp.qa || i == dp.ca))
      e /= i == dp.qa ? a.t_wq : a.t_wc;
    else if (dp.family == kFamInterleave && i == r - 2)
      e /= a.vec;
    else if (dp.family == kFamInterleave && i == r - 1)
      e = 1;
    else if (dp.family == kFamPermute && i == r - 2)
      e /= a.p_t;
    else if (dp.family == kFamPermute && i == r - 3)
      e /= a.p_g;
    else if (dp.family == kFamPermute && i > r - 3)
      e = 1;
    n *= e;
  }
  return n;
}

// Coordinates a split of axis i must keep together (0: never split).
int64_t split_align(const DeviceProgram &dp, int i) {
  const int r = dp.base.rank;
  if (dp.family == kFamStream && i == r - 1)
    return dp.base.vec;
  if (dp.family == kFamTranspose && (i == dp.qa || i == dp.ca))
    return i == dp.qa ? dp.base.t_wq : dp.base.t_wc;
  if (dp.family == kFamInterleave && i == r - 2)
    return dp.base.vec;
  if (dp.family == kFamInterleave && i == r - 1)
    return 0;
  if (dp.family == kFamPermute && i == r - 2)
    return dp.base.p_t;
  if (dp.family == kFamPermute && i > r - 4)
    return 0;
  return 1;
}

// Axes whose coordinates the decomposition levels carry (the others are the
// 2-D block of the transpose/interleave kernels).
bool level_axis(const DeviceProgram &dp, int i) {
  const int r = dp.base.rank;
  if (dp.family == kFamTranspose)
    return i != dp.qa && i != dp.ca;
  if (dp.family == kFamInterleave)
    return i < r - 2;
  if (dp.family == kFamPermute)
    return i < r - 3;
  return true;
}

// Largest element offset the levels of box b reach from its base, on the
// source and the destination side; contrib[i] the larger of axis i's two.
int64_t level_span(const DeviceProgram &dp, const Box &b, int64_t *contrib) {
  int64_t ss = 0, ds = 0;
  for (int i = 0; i < dp.base.rank; ++i) {
    contrib[i] = 0;
    if (!level_axis(dp, i) || b.ext[i] <= 1)
      continue;
    const int64_t s = (b.ext[i] - 1) * dp.base.ss[i], d = (b.ext[i] - 1) * dp.base.ds[i];
    ss += s;
    ds += d;
    contrib[i] = std::max(s, d);
  }
  return std::max(ss, ds);
}

// Split a fast-family box until it has fewer than 2^31 work items and level
// spans below 2^31 elements: halve (keeping alignment) the splittable axis
// with the largest span contribution, or the outermost one for work alone.
void split_box(const DeviceProgram &dp, const Box &b, std::vector<Box> &out) {
  if (dp.family == kFamGeneric) {
    out.push_back(b);
    return;
  }
  int64_t contrib[kMaxRank];
  const bool wide = level_span(dp, b, contrib) >= kMaxLaunchWork;
  if (!wide && box_work(dp, b) < kMaxLaunchWork) {
    out.push_back(b);
    return;
  }
  int axis = -1;
  for (int i = 0; i < dp.base.rank; ++i) {
    const int64_t al = split_align(dp, i);
    if (al == 0 || b.ext[i] <= al)
      continue;
    if (axis < 0 || (wide && contrib[i] > contrib[axis]))
      axis = i;
  }
  if (axis < 0)
    fail("unsupported_layout", "a launch box cannot be split below 2^31 elements");
  const int64_t al = split_align(dp, axis);
  const int64_t half = (b.ext[axis] / al + 1) / 2 * al; // extents are multiples of al
  Box c = b;
  c.ext[axis] = half;
  split_box(dp, c, out);
  c.lo[axis] = b.lo[axis] + half;
  c.ext[axis] = b.ext[axis] - half;
  split_box(dp, c, out);
}

Level trivial_level() {
  Level l{};
  l.div = make_div(1);
  l.vlo = 0;
  l.vcnt = 1;
  return l;
}

// Level of axis i counting units of `unit` coordinates (unit > 1 only on
// unpadded axes whose box start is a multiple of unit). The valid units of
// the box are [vlo, vlo + vcnt).
Level axis_level(const KArgs &a, const Box &b, int i, int64_t unit) {
  Level l{};
  const int64_t n = b.ext[i] / unit;
  l.div = make_div(n);
  const int64_t vmin = (a.lo[i] - b.lo[i]) / unit, vmax = vmin + a.vext[i] / unit;
  const int64_t lo = std::min(std::max<int64_t>(vmin, 0), n), hi = std::min(std::max<int64_t>(vmax, 0), n);
  l.vlo = static_cast<uint32_t>(lo);
  l.vcnt = static_cast<uint32_t>(hi - lo);
  if (n > 1) { // a single coordinate never moves the offset
    const int64_t ss = a.ss[i] * unit, ds = a.ds[i] * unit;
    if (ss >= kMaxLaunchWork || ds >= kMaxLaunchWork || n >= kMaxLaunchWork)
      fail("internal_launch_check", "a level stride exceeds 32 bits");
    l.ss = static_cast<uint32_t>(ss);
    l.ds = static_cast<uint32_t>(ds);
  }
  return l;
}

int64_t box_elements(const Box &b, int rank) {
  int64_t n = 1;
  for (int i = 0; i < rank; ++i)
    n *= b.ext[i];
  return n;
}

// Arguments of an edge box: the element-wise kernel over the box.
KArgs edge_args(const DeviceProgram &dp, const Box &b) {
  KArgs a = dp.base;
  for (int i = 0; i < a.rank; ++i) {
    a.box_lo[i] = b.lo[i];
    a.box_ext[i] = b.ext[i];
  }
  a.work64 = box_elements(b, a.rank);
  a.work = 0;
  a.edge_box = 1;
  return a;
}

bool pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

// A byte-tile transpose launch indexes the parameters of its dequantize ->
// f16 chain by destination row (kTileRowChannel) when the stage has one
// channel per
// destination row of the box. For a result offset o = D + q * dsq + c of
// box row q < Q and column c < C (the box is one plane: no batch levels),
// chan_of(o) = (o / rs) mod re = D / dsq + q exactly when rs = dsq,
// (D mod dsq) + C <= dsq (the box's columns stay inside one row) and
// D / dsq + Q <= re (no wrap). t_choff = D / dsq.
bool row_channel(KArgs &a, const Box &b, int qa, int ca) {
  if (a.chain_code != kChainDeqF16 || a.wout != 2)
    return false;
  const DevStage &s = a.chain.st[0];
  const int64_t dsq = a.ds[qa];
  if (s.mode != kChanDim || s.vec != 0 || s.ch_rs != dsq || a.ds[ca] != 1 || dsq <= 0)
    return false;
  for (int j = 0; j < kBatchLevels; ++j)
    if (a.lv[j].div.d != 1)
      return false;
  if (a.dbase % dsq + b.ext[ca] > dsq || a.dbase / dsq + b.ext[qa] > s.ch_re)
    return false;
  a.t_choff = static_cast<uint32_t>(a.dbase / dsq);
  return true;
}

// The zero points of channels [c0, c0 + n) of a dequantize stage are all 0.
bool zero_points_zero(const DeviceProgram &dp, const DevStage &s, int64_t c0, int64_t n) {
  const int64_t lo = s.zp_off + (s.zp_per_ch ? c0 : 0), hi = lo + (s.zp_per_ch ? n : 1);
  if (lo < 0 || hi > static_cast<int64_t>(dp.pi.size()))
    return false;
  for (int64_t i = lo; i < hi; ++i)
    if (dp.pi[static_cast<size_t>(i)] != 0)
      return false;
  return true;
}

// A permute launch runs the direct body when its divisions are shifts (G*E,
// E and the 16-byte vectors of a run are powers of two, so make_div gives
// m = 1 and s = log2 d), its batch entries lie along one level (the outer
// levels are unit levels) and the parameter stage, if any, takes a vector's
// entry from the block's own c coordinate. For a stage per channel along c
// (rs = M*E, re = C) at result offset o = D + c*M*E + m*E + e, with m < M,
// e < E and D the offset of the block's batch entry, (o / (M*E)) mod C = c
// exactly when D is a multiple of C*M*E: every batch level's destination
// stride is, and the launch origin is one plus an offset inside a plane
// (below M*E; a launch may start at any m). A per-tensor stage takes entry 0.
bool permute_direct(KArgs &a, int64_t C, int64_t M, int64_t E) {
  a.p_cmask = 0;
  if (a.chain_code == kChainGeneric || !pow2(a.p_ge.d) || !pow2(a.p_e.d) || !pow2(a.p_run.d))
    return false;
  // the direct kernel takes a batch entry's offsets from the innermost level
  for (int j = 0; j + 1 < kBatchLevels; ++j)
    if (a.lv[j].div.d != 1 || a.lv[j].vcnt != 1)
      return false;
  const int k = chain_param_stage(a.chain_code);
  if (k < 0)
    return true;
  const DevStage &s = a.chain.st[k];
  if (s.vec != 0)
    return false;
  if (s.mode == kChanNone)
    return true;
  const int64_t plane = C * M * E;
  if (s.mode != kChanDim || s.ch_rs != M * E || s.ch_re != C || a.dbase % plane >= M * E)
    return false;
  for (int j = 0; j < kBatchLevels; ++j)
    if (a.lv[j].div.d > 1 && a.lv[j].ds % plane != 0)
      return false;
  a.p_cmask = ~0u;
  return true;
}

KArgs launch_args(const DeviceProgram &dp, const Box &b) {
  KArgs a = dp.base;
  const int r = a.rank;
  for (int i = 0; i < r; ++i) {
    a.box_lo[i] = b.lo[i];
    a.box_ext[i] = b.ext[i];
  }
  // box origin: destination offset of its first padded coordinate, source
  // offset of the valid coordinate it corresponds to (interleave channels are
  // addressed by the kernel itself)
  a.sbase = 0;
  a.dbase = 0;
  for (int i = 0; i < r; ++i) {
    if (dp.family == kFamInterleave && i == r - 1)
      continue;
    a.sbase += (b.lo[i] - a.lo[i]) * a.ss[i];
    a.dbase += b.lo[i] * a.ds[i];
  }
  for (int i = 0; i < kMaxRank; ++i)
    a.lv[i] = trivial_level();
  const int64_t work = box_work(dp, b);
  a.work = static_cast<uint32_t>(work);
  a.work64 = work;
  // batch levels of the 2-D families: every axis but skip0/skip1, outer first
  auto batch = [&](int skip0, int skip1) {
    int idx[kMaxRank], n = 0;
    for (int i = 0; i < r; ++i)
      if (i != skip0 && i != skip1)
        idx[n++] = i;
    for (int j = 0; j < n; ++j)
      a.lv[kBatchLevels - n + j] = axis_level(a, b, idx[j], 1);
  };
  switch (dp.family) {
  case kFamStream:
    for (int i = 0; i < r; ++i)
      a.lv[a.nlev - r + i] = axis_level(a, b, i, i == r - 1 ? a.vec : 1);
    break;
  case kFamTranspose:
    batch(dp.qa, dp.ca);
    {
      // orders (measured on C3's int8 -> f16 transpose, 8 KiB result rows):
      // 128-wide tiles q fastest with each q-tile's c-tiles rotated, so the
      // blocks in flight write their rows at different column offsets
      // (30.0 -> 27.1 us); 64-wide one-byte tiles q fastest, grouped by XCD
      // so that the two halves of each source line meet in one L2; wider
      // elements in groups of kTileGroup q-tiles
      const int64_t nq = b.ext[dp.qa] / a.t_wq, nc = b.ext[dp.ca] / a.t_wc;
      const bool bytes = a.win == 1, wide = a.t_wq == 128;
      const int64_t g = bytes ? nq : std::min<int64_t>(kTileGroup, nq);
      const int64_t full = nq / g * g;
      a.t_plane = make_div(nq * nc);
      a.t_group = make_div(g * nc);
      a.t_g = make_div(g);
      a.t_tail = make_div(nq - full > 0 ? nq - full : 1);
      a.t_nc = make_div(nc);
      a.t_full = static_cast<uint32_t>(full);
      a.t_flags = (bytes && !wide ? kTileXcd : 0u) | (wide ? kTileSkew : 0u);
      a.t_choff = 0;
      if (a.t_wc == 128 && row_channel(a, b, dp.qa, dp.ca)) {
        a.t_flags |= kTileRowChannel;
        if (zero_points_zero(dp, a.chain.st[0], a.t_choff, b.ext[dp.qa]))
          a.t_flags |= kTileZeroPoint0;
      }
    }
    a.t_ssc = a.ss[dp.ca];
    a.t_dsq = a.ds[dp.qa];
    break;
  case kFamPermute: {
    int idx[kMaxRank], n = 0;
    for (int i = 0; i < r - 3; ++i)
      idx[n++] = i;
    for (int j = 0; j < n; ++j)
      a.lv[kBatchLevels - n + j] = axis_level(a, b, idx[j], 1);
    const int64_t E = a.vext[r - 1], C = a.vext[r - 3], M = a.vext[r - 2], T = a.p_t;
    a.p_tiles = make_div(b.ext[r - 2] / T);
    a.p_cgt = make_div(work / (C / a.p_g));
    a.p_ce = make_div(C * E);
    a.p_ge = make_div(int64_t{a.p_g} * E);
    a.p_e = make_div(E);
    a.p_run = make_div(T * E * a.wout / 16);
    a.p_dsc = M * E;
    a.p_direct = permute_direct(a, C, M, E) ? 1 : 0;
    break;
  }
  case kFamInterleave:
    batch(r - 2, r - 1);
    a.i_ng = make_div(b.ext[r - 2] / a.vec);
    a.i_ssc = a.ss[r - 1];
    a.i_loc = static_cast<int32_t>(a.lo[r - 1]);
    a.i_vc = static_cast<int32_t>(a.vext[r - 1]);
    break;
  default: {
    int64_t n = 1;
    for (int i = 0; i < r; ++i)
      n *= b.ext[i];
    a.work64 = n;
  }
  }
  return a;
}

} // namespace

// Launch arguments for valid coordinates [v0, v1) of the chunk axis (the
// whole box when the axis is -1). The first/last chunk also cover the axis'
// leading/trailing pad. One entry per launch.
std::vector<KArgs> box_launches(const DeviceProgram &dp, int64_t v0, int64_t v1, bool first,
                                bool last) {
  const KArgs &a = dp.base;
  if (dp.chunk_axis < 0)
    return axis_launches(dp, -1, 0, 0);
  const int ax = dp.chunk_axis;
  const int64_t plo = first ? 0 : v0 + a.lo[ax];
  const int64_t phi = last ? a.pext[ax] : v1 + a.lo[ax];
  return axis_launches(dp, ax, plo, phi);
}

int64_t axis_align(const DeviceProgram &dp, int i) { return split_align(dp, i); }

std::vector<KArgs> axis_launches(const DeviceProgram &dp, int axis, int64_t plo, int64_t phi) {
  return prefix_launches(dp, nullptr, axis, plo, phi);
}

std::vector<KArgs> prefix_launches(const DeviceProgram &dp, const int64_t *fixed, int axis,
                                   int64_t plo, int64_t phi) {
  const KArgs &a = dp.base;
  Box b{};
  for (int i = 0; i < a.rank; ++i) {
    b.lo[i] = 0;
    b.ext[i] = a.pext[i];
  }
  if (axis >= 0) {
    for (int i = 0; fixed && i < axis; ++i) {
      b.lo[i] = fixed[i];
      b.ext[i] = 1;
    }
    b.lo[axis] = plo;
    b.ext[axis] = phi - plo;
  }
  std::vector<KArgs> out;
  // A transpose box whose q or c extent is not a multiple of the tile: the
  // whole tiles go to the tile kernel, the strips past them (the q strip
  // over the whole c range, the c strip beside the whole q tiles) to the
  // element-wise kernel. Box starts on those axes are multiples of the tile
  // (t_wq along q, t_wc along c: chunks and splits keep the tile alignment).
  std::vector<Box> edges;
  if (dp.family == kFamStream && a.rank == 1 && b.ext[0] % a.vec != 0) {
    // the tail of a single contiguous axis (box starts are multiples of V)
    const int64_t m = b.ext[0] / a.vec * a.vec;
    Box e = b;
    e.lo[0] = b.lo[0] + m;
    e.ext[0] = b.ext[0] - m;
    edges.push_back(e);
    b.ext[0] = m;
  }
  if (dp.family == kFamTranspose) {
    const int q = dp.qa, c = dp.ca;
    const int64_t wq = a.t_wq, wc = a.t_wc;
    const int64_t mq = b.ext[q] / wq * wq, mc = b.ext[c] / wc * wc;
    if (mq < b.ext[q]) {
      Box e = b;
      e.lo[q] = b.lo[q] + mq;
      e.ext[q] = b.ext[q] - mq;
      edges.push_back(e);
    }
    if (mc < b.ext[c] && mq > 0) {
      Box e = b;
      e.ext[q] = mq;
      e.lo[c] = b.lo[c] + mc;
      e.ext[c] = b.ext[c] - mc;
      edges.push_back(e);
    }
    b.ext[q] = mq;
    b.ext[c] = mc;
  }
  std::vector<Box> boxes;
  if (box_elements(b, a.rank) > 0)
    split_box(dp, b, boxes);
  out.reserve(boxes.size() + edges.size());
  for (const Box &x : boxes)
    if (box_work(dp, x) > 0)
      out.push_back(launch_args(dp, x));
  for (const Box &x : edges)
    if (box_elements(x, a.rank) > 0)
      out.push_back(edge_args(dp, x));
  return out;
}

namespace {

[[noreturn]] void bad_launch(const DeviceProgram &dp, const std::string &what) {
  fail("internal_launch_check", std::string(dp.kernel) + " launch: " + what);
}

template <int L>
bool decompose_n(const Level *lv, uint32_t i, int64_t &sof, int64_t &dof) {
  return decompose<L>(lv, i, sof, dof);
}

bool decompose_rt(int n, const Level *lv, uint32_t i, int64_t &sof, int64_t &dof) {
  switch (n) {
  case 1:
    return decompose_n<1>(lv, i, sof, dof);
  case 2:
    return decompose_n<2>(lv, i, sof, dof);
  case 3:
    return decompose_n<3>(lv, i, sof, dof);
  case 4:
    return decompose_n<4>(lv, i, sof, dof);
  default:
    return decompose_n<8>(lv, i, sof, dof);
  }
}

struct Checker {
  const DeviceProgram &dp;
  const KArgs &a;
  int64_t wire, dst; // elements
  size_t npf, npi;
  int64_t wire_lo; // first wire element the launch may read

  // n elements from `off`, accessed as one vector of n * width bytes when
  // `vec` (which must then be aligned to its size)
  void src_run(int64_t off, int64_t n, bool vec) const {
    if (off < wire_lo || off + n > wire)
      bad_launch(dp, "source run [" + std::to_string(off) + ", " + std::to_string(off + n) +
                         ") outside wire elements [" + std::to_string(wire_lo) + ", " +
                         std::to_string(wire) + ")");
    if (vec && (off * a.win) % (n * a.win) != 0)
      bad_launch(dp, "unaligned " + std::to_string(n * a.win) + "-byte source access at element " +
                         std::to_string(off));
  }
  void dst_run(int64_t off, int64_t n, bool vec) const {
    if (off < 0 || off + n > dst)
      bad_launch(dp, "destination run [" + std::to_string(off) + ", " + std::to_string(off + n) +
                         ") outside " + std::to_string(dst) + " result elements");
    if (vec && (off * a.wout) % (n * a.wout) != 0)
      bad_launch(dp, "unaligned " + std::to_string(n * a.wout) +
                         "-byte destination access at element " + std::to_string(off));
  }
  // channels of V consecutive result elements from dense offset o, as the
  // fast kernels index them (constant, or +1 per element)
  void channels(int64_t o, int V) const {
    for (int k = 0; k < a.chain.n; ++k) {
      const DevStage &s = a.chain.st[k];
      const uint32_t c = chan_of(s, o);
      const uint32_t last = chan_of(s, o + V - 1);
      const uint32_t want = s.vec ? c + static_cast<uint32_t>(V - 1) : c;
      if (last != want)
        bad_launch(dp, "channel pattern of stage " + std::to_string(k) + " breaks inside a vector");
      const bool reads_params = s.op == kOpQuantize || s.op == kOpDequantize;
      if (want >= s.len ||
          (reads_params && (s.scale_off + want >= npf ||
                            s.zp_off + (s.zp_per_ch ? want : 0u) >= npi)))
        bad_launch(dp, "parameter index outside its table at stage " + std::to_string(k));
    }
  }
};

} // namespace

void verify_launch(const DeviceProgram &dp_in, const KArgs &a, int64_t wire_lo, int64_t wire_hi) {
  DeviceProgram edge;
  if (a.edge_box && dp_in.family != kFamGeneric) { // run by the element-wise kernel
    edge = dp_in;
    edge.family = kFamGeneric;
  }
  const DeviceProgram &dp = a.edge_box && dp_in.family != kFamGeneric ? edge : dp_in;
  const Checker ck{dp,          a,           wire_hi < 0 ? dp.wire_elems : wire_hi,
                   dp.dst_elems, dp.pf.size(), dp.pi.size(),
                   wire_lo};
  if (dp.family != kFamGeneric) { // the levels' 32-bit offsets cannot wrap
    int64_t ss = 0, ds = 0;
    for (const Level &l : a.lv) {
      ss += (int64_t{l.div.d} - 1) * l.ss;
      ds += (int64_t{l.div.d} - 1) * l.ds;
      if (int64_t{l.vlo} + l.vcnt > l.div.d)
        bad_launch(dp, "a level's valid range leaves its extent");
    }
    if (ss >= kMaxLaunchWork || ds >= kMaxLaunchWork)
      bad_launch(dp, "level offsets exceed 31 bits");
  }
  const int win = a.win, wout = a.wout;
  switch (dp.family) {
  case kFamStream: {
    if (a.work64 >= kMaxLaunchWork || a.work != a.work64)
      bad_launch(dp, "work above 2^31");
    const int V = a.vec;
    for (uint32_t i = 0; i < a.work; ++i) {
      int64_t sof = a.sbase, dof = a.dbase;
      const bool pad = decompose_rt(a.nlev, a.lv, i, sof, dof);
      ck.dst_run(dof, V, true);
      if (!pad) {
        ck.src_run(sof, V, true);
        ck.channels(dof, V);
      }
    }
    break;
  }
  case kFamTranspose: {
    if (a.work64 > (int64_t{1} << 22) || a.work != a.work64)
      bad_launch(dp, "more tiles than one launch takes");
    const int VO = 16 / wout;
    const int64_t TQ = a.t_wq, TC = a.t_wc;
    if (!(TQ == 64 || (TQ == 128 && win == 1)) || !(TC == 64 || (TC == 128 && TQ == 128)) ||
        a.t_nc.d != a.t_group.d / a.t_g.d || (a.t_flags & ~(kTileXcd | kTileSkew | kTileRowChannel | kTileZeroPoint0)) ||
        ((a.t_flags & kTileSkew) && (a.t_flags & kTileXcd)) || (TC == 128 && (a.t_flags & kTileXcd)) ||
        ((a.t_flags & kTileRowChannel) && TC != 128))
      bad_launch(dp, "tile geometry disagrees with the kernel");
    std::vector<bool> seen(a.work, false); // the order must be a bijection
    for (uint32_t blk = 0; blk < a.work; ++blk) { // grid = one block per tile
      const uint32_t t = (a.t_flags & kTileXcd) ? xcd_tile(blk, a.work) : blk;
      if (t >= a.work)
        bad_launch(dp, "a block maps past the last tile");
      uint32_t tq, tc, r2;
      tile_of(a, t, tq, tc, r2);
      const uint32_t nc = a.t_group.d / a.t_g.d, nq = a.t_plane.d / nc;
      if (tq >= nq || tc >= nc)
        bad_launch(dp, "tile coordinates outside the plane");
      const size_t id = (static_cast<size_t>(r2) * nq + tq) * nc + tc;
      if (id >= seen.size() || seen[id])
        bad_launch(dp, "the tile order visits a tile twice");
      seen[id] = true;
      int64_t sbase = a.sbase, dbase = a.dbase;
      if (decompose_rt(kBatchLevels, a.lv, r2, sbase, dbase))
        bad_launch(dp, "a transpose tile reaches a pad");
      const int64_t q0 = int64_t{tq} * TQ, c0 = int64_t{tc} * TC;
      // a tile row moves as 16-byte vectors: TC source rows of TQ elements,
      // TQ destination rows of TC
      for (int64_t row = 0; row < TC; row += TC - 1) {
        const int64_t so = sbase + (c0 + row) * a.t_ssc + q0;
        ck.src_run(so, TQ, false);
        if ((so * win) % 16 != 0)
          bad_launch(dp, "a tile row is not 16-byte aligned");
      }
      for (int64_t row = 0; row < TQ; row += TQ - 1) {
        const int64_t d = dbase + (q0 + row) * a.t_dsq + c0;
        ck.dst_run(d, TC, false);
        if ((d * wout) % 16 != 0)
          bad_launch(dp, "a tile row is not 16-byte aligned");
      }
      if ((a.t_ssc * win) % 16 != 0 || (a.t_dsq * wout) % 16 != 0)
        bad_launch(dp, "row strides break 16-byte alignment");
      const bool rowch = (a.t_flags & kTileRowChannel) != 0;
      if (rowch && (r2 != 0 || a.chain_code != kChainDeqF16 || a.chain.st[0].vec != 0))
        bad_launch(dp, "row-indexed parameters with a chain or batch they do not fit");
      if ((a.t_flags & kTileZeroPoint0) &&
          (!rowch || !zero_points_zero(dp, a.chain.st[0], a.t_choff, int64_t{a.t_plane.d} /
                                                                       a.t_nc.d * TQ)))
        bad_launch(dp, "a launch that leaves zero points out reads one that is not 0");
      for (int64_t row = 0; row < TQ; ++row)
        for (int64_t cv = 0; cv < TC; cv += VO) {
          const int64_t o = dbase + (q0 + row) * a.t_dsq + c0 + cv;
          ck.channels(o, VO);
          if (rowch && chan_of(a.chain.st[0], o) != a.t_choff + static_cast<uint32_t>(q0 + row))
            bad_launch(dp, "a row-indexed launch reads another parameter entry");
        }
    }
    break;
  }
  case kFamInterleave: {
    if (a.work64 >= kMaxLaunchWork || a.work != a.work64)
      bad_launch(dp, "work above 2^31");
    const int G = a.vec, CP = a.cpad;
    for (int k = 0; k < a.chain.n; ++k)
      if (a.chain.st[k].mode != kChanNone)
        bad_launch(dp, "per-channel stage in an interleave program");
    if ((a.i_ssc * win) % (G * win) != 0)
      bad_launch(dp, "plane stride breaks the alignment of plane loads");
    if (G != interleave_pixels(win, wout, CP))
      bad_launch(dp, "pixels per item disagree with the kernel");
    for (uint32_t i = 0; i < a.work; ++i) {
      const uint32_t rest = fdiv(i, a.i_ng);
      const uint32_t g = i - rest * a.i_ng.d;
      int64_t sbase = a.sbase, dbase = a.dbase;
      const bool pad = decompose_rt(kBatchLevels, a.lv, rest, sbase, dbase);
      const int64_t p0 = int64_t{g} * G;
      ck.dst_run(dbase + p0 * CP, int64_t{G} * CP, true);
      for (int c = 0; c < CP; ++c) {
        const int32_t vc = c - a.i_loc;
        if (!pad && static_cast<uint32_t>(vc) < static_cast<uint32_t>(a.i_vc))
          ck.src_run(sbase + vc * a.i_ssc + p0, G, true);
      }
    }
    break;
  }
  case kFamPermute: {
    if (a.work64 > (int64_t{1} << 22) || a.work != a.work64)
      bad_launch(dp, "more blocks than one launch takes");
    const int64_t CE = a.p_ce.d, E = a.p_e.d, T = a.p_t, C = CE / E, G = a.p_g, GE = a.p_ge.d;
    const int VI = 16 / win;
    if (G < 1 || C % G != 0 || GE != G * E || a.p_lds != T * GE * wout || a.p_lds > 32768 ||
        int64_t{a.p_run.d} * 16 != T * E * wout || a.vec != VI || GE % VI != 0 ||
        (E * wout) % 16 != 0 || int64_t{a.p_cgt.d} * (C / G) != a.work64)
      bad_launch(dp, "block geometry disagrees with the kernel");
    // a direct launch replaces each division by a shift and mask, and each
    // vector's parameter entry by c & p_cmask
    const int pk = chain_param_stage(a.chain_code);
    if (a.p_direct) {
      for (const FastDiv *f : {&a.p_ge, &a.p_e, &a.p_run})
        if (!pow2(f->d) || f->m != 1 || (uint64_t{1} << f->s) != f->d)
          bad_launch(dp, "a direct permute divides by a number that is not a power of two");
      if (a.chain_code == kChainGeneric || (pk >= 0 && a.chain.st[pk].vec != 0) ||
          (a.p_cmask != 0 && a.p_cmask != ~0u))
        bad_launch(dp, "a direct permute with a chain it cannot run");
      for (int j = 0; j + 1 < kBatchLevels; ++j)
        if (a.lv[j].div.d != 1 || a.lv[j].vcnt != 1 || a.lv[j].ss != 0 || a.lv[j].ds != 0)
          bad_launch(dp, "a direct permute over more than one batch level");
      if (a.lv[kBatchLevels - 1].div.d > 1 &&
          (int64_t{a.lv[kBatchLevels - 1].ss} * (a.lv[kBatchLevels - 1].div.d - 1) >= kMaxLaunchWork ||
           int64_t{a.lv[kBatchLevels - 1].ds} * (a.lv[kBatchLevels - 1].div.d - 1) >= kMaxLaunchWork))
        bad_launch(dp, "a direct permute's batch offsets leave 32 bits");
    }
    for (uint32_t t = 0; t < a.work; ++t) {
      // the kernel's own decomposition: group, then batch entry and m-tile
      const uint32_t cg = fdiv(t, a.p_cgt);
      const uint32_t t2 = t - cg * a.p_cgt.d;
      const uint32_t batch = fdiv(t2, a.p_tiles);
      const int64_t m0 = int64_t{t2 - batch * a.p_tiles.d} * T;
      int64_t sbase = a.sbase, dbase = a.dbase;
      if (decompose_rt(kBatchLevels, a.lv, batch, sbase, dbase))
        bad_launch(dp, "a permute block reaches a pad");
      for (int64_t tt = 0; tt < T; ++tt) {
        const int64_t so = sbase + (m0 + tt) * CE + int64_t{cg} * GE;
        ck.src_run(so, GE, false);
        if ((so * win) % 16 != 0)
          bad_launch(dp, "unaligned source rows");
      }
      for (int64_t cl = 0; cl < G; ++cl) {
        const int64_t c = int64_t{cg} * G + cl;
        ck.dst_run(dbase + c * a.p_dsc + m0 * E, T * E, false);
        if (((dbase + c * a.p_dsc + m0 * E) * wout) % 16 != 0)
          bad_launch(dp, "unaligned destination runs");
        for (int64_t tt = 0; tt < T; ++tt)
          for (int64_t e = 0; e < E; e += VI) {
            const int64_t o = dbase + c * a.p_dsc + (m0 + tt) * E + e;
            ck.channels(o, VI);
            if (a.p_direct && pk >= 0 &&
                chan_of(a.chain.st[pk], o) != (static_cast<uint32_t>(c) & a.p_cmask))
              bad_launch(dp, "a direct permute reads another parameter entry");
          }
      }
    }
    break;
  }
  default: {
    for (int64_t i = 0; i < a.work64; ++i) {
      int64_t rem = i, dof = 0, sof = 0;
      bool pad = false;
      for (int k = a.rank - 1; k >= 0; --k) {
        const int64_t p = rem % a.box_ext[k] + a.box_lo[k];
        rem /= a.box_ext[k];
        dof += p * a.ds[k];
        const int64_t v = p - a.lo[k];
        if (v < 0 || v >= a.vext[k])
          pad = true;
        else
          sof += v * a.ss[k];
      }
      ck.dst_run(dof, 1, false);
      if (!pad)
        ck.src_run(sof, 1, false);
    }
  }
  }
}

namespace {

bool verify_enabled() {
  static const bool on = [] {
    const char *v = std::getenv("RELX_VERIFY_LAUNCHES");
    return v && *v && std::strcmp(v, "0") != 0;
  }();
  return on;
}

} // namespace

int64_t launch_program(const DeviceProgram &dp, int64_t v0, int64_t v1, bool first, bool last,
                       const void *src, void *dst, const float *pf, const int32_t *pi,
                       int32_t *status, hipStream_t s) {
  const bool part = dp.chunk_axis >= 0 && v1 > v0; // else the whole box
  return launch_all(dp, box_launches(dp, v0, v1, first, last), src, dst, pf, pi, status, s,
                    part ? v0 * dp.chunk_stride : 0, part ? v1 * dp.chunk_stride : -1);
}

int64_t launch_all(const DeviceProgram &dp, std::vector<KArgs> launches, const void *src,
                   void *dst, const float *pf, const int32_t *pi, int32_t *status, hipStream_t s,
                   int64_t wire_lo, int64_t wire_hi) {
  // the fast kernels move 16-byte vectors: buffers that are not 16-byte
  // aligned take the element-wise kernel
  const bool aligned = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  int64_t n = 0;
  for (KArgs &a : launches) {
    int family = a.edge_box ? kFamGeneric : dp.family;
    if (!aligned && family != kFamGeneric) {
      family = kFamGeneric;
      int64_t e = 1;
      for (int i = 0; i < a.rank; ++i)
        e *= a.box_ext[i];
      a.work64 = e;
    }
    if (verify_enabled()) {
      DeviceProgram view = dp;
      view.family = family;
      verify_launch(view, a, wire_lo, wire_hi);
    }
    a.src = static_cast<const uint8_t *>(src);
    a.dst = static_cast<uint8_t *>(dst);
    a.pf = pf;
    a.pi = pi;
    const hipError_t e = launch_box(family, a, status, s);
    if (e != hipSuccess)
      fail("backend_failure", std::string("kernel launch: ") + hipGetErrorString(e));
    ++n;
  }
  return n;
}

} // namespace relx
