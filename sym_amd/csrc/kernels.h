// kernels.h - gfx950 relayout + value-stage kernel templates (device code).
//
// Every kernel maps dense SOURCE-layout wire values at some stage boundary to
// the dense RESULT layout after the last stage, over an iteration box of
// padded destination coordinates (so a chunked pipeline can launch one box
// per arrived chunk). Pads are written with the folded fill; every value
// stage keeps its own rounding (docs/reloc-typed-semantics.md), including the
// reference's NaN encodings, so results are bit-identical to the reference
// CPU executor (libreloc/src/TypedExecute.cpp:472-499).
//
// Families (chosen on the host, program.cpp):
//   generic    one element per thread, any rank/stride/pad/channel map
//   stream     innermost axis contiguous on both sides: one vector of
//              16/min(width) elements per thread (16-byte loads/stores)
//   transpose  batched 2-D transpose through a 64x64 LDS tile (32-bit
//              words, row pitch 65: conflict-free for every element width
//              pairing), tiles visited in groups of destination rows (XCD-grouped
//              for one-byte sources)
//   interleave planar -> interleaved with a small padded inner axis
//              (NCHW -> NHWC + pad): per-plane 16-byte loads, packed pixels
// The common stage sequences get a compile-time body (ChainCode); the rest
// dispatch per stage. Fast kernels index in 32 bits relative to their launch
// box (the host splits boxes of 2^31 or more work items) and form 64-bit
// element offsets from the per-level strides.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "index.h"
#include "program.h"

namespace relx {
namespace {

constexpr int kBlock = 256;

// Native 16-byte vector.
typedef uint32_t vec4 __attribute__((ext_vector_type(4)));


// ------------------------------------------------------------ value ops

__device__ __forceinline__ uint32_t op_f32_f16(uint32_t b) {
  float f = __uint_as_float(b);
  // The binary32 value must exist before it is narrowed: without this
  // barrier the backend folds a producing multiply and the narrowing into
  // v_fma_mixlo_f16 (one rounding), breaking dequantize -> cast, whose
  // contract keeps both roundings. v_cvt_f16_f32 itself rounds to nearest
  // even and encodes NaN as sign | 0x7e00 | payload >> 13 -- the reference's
  // encoding (checked on gfx950 for every binary32 NaN).
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(f));
}

// Exact binary16 -> binary32. The hardware quiets signalling NaNs; the
// reference keeps the payload as is, so NaNs are rebuilt.
__device__ __forceinline__ uint32_t op_f16_f32(uint32_t h) {
  const _Float16 x = __builtin_bit_cast(_Float16, static_cast<unsigned short>(h));
  uint32_t r = __float_as_uint(static_cast<float>(x));
  if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)) // NaN: payload shifted, not quieted
    r = ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13);
  return r;
}

// Widening whose NaN payload is never observed (a following quantize maps
// every NaN to -128).
__device__ __forceinline__ float op_f16_f32_value(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

__device__ __forceinline__ uint32_t op_f32_bf16(uint32_t b) {
  if ((b & 0x7fffffffu) > 0x7f800000u)
    return ((b >> 16) | 0x40u) & 0xffffu;
  const uint64_t w = b;
  return static_cast<uint32_t>((w + 0x7fffu + ((w >> 16) & 1u)) >> 16);
}

// symmetric_rne: t = fl32(x * inv); maxNum(t, -128) then minNum(t, 127)
// (NaN -> -128); round half to even. Adding 1.5 * 2^23 rounds the clamped
// value to the nearest even integer in the low mantissa bits, whose low byte
// is the two's-complement code (equal to rint + convert on all 2^32 inputs).
__device__ __forceinline__ uint32_t quant_value(float x, float inv) {
  float y = x * inv;
  y = __builtin_fmaxf(y, -128.0f);
  y = __builtin_fminf(y, 127.0f);
  return __float_as_uint(y + 12582912.0f) & 0xffu;
}

__device__ __forceinline__ uint32_t op_quant(uint32_t b, float inv) {
  return quant_value(__uint_as_float(b), inv);
}

__device__ __forceinline__ uint32_t op_dequant(uint32_t b, float scale, int32_t zp) {
  const int32_t q = static_cast<int8_t>(static_cast<uint8_t>(b));
  return __float_as_uint(static_cast<float>(q - zp) * scale);
}

__device__ __forceinline__ uint32_t apply(const DevStage &s, uint32_t x, uint32_t c,
                                          const float *pf, const int32_t *pi) {
  switch (s.op) {
  case kOpF32toF16:
    return op_f32_f16(x);
  case kOpF16toF32:
    return op_f16_f32(x);
  case kOpF32toBF16:
    return op_f32_bf16(x);
  case kOpBF16toF32:
    return x << 16;
  case kOpQuantize:
    return op_quant(x, pf[s.scale_off + c]);
  default:
    return op_dequant(x, pf[s.scale_off + c], pi[s.zp_off + (s.zp_per_ch ? c : 0u)]);
  }
}

// ------------------------------------------------------- argument loads

// Kernel arguments arrive through scalar loads from the kernarg segment. The
// compiler issues each one lazily, behind the first branch that needs it, so
// a prologue with a few branches makes several dependent round trips to
// memory before its first global load (five in the transpose). Naming every
// argument a kernel reads in empty asm statements at its entry puts all of
// those loads in one batch (C2's interleave: 8.0 -> 7.6 us).
__device__ __forceinline__ void hot(const FastDiv &f) { asm volatile("" ::"s"(f.d), "s"(f.m), "s"(f.s)); }
__device__ __forceinline__ void hot(const Level &l) {
  hot(l.div);
  asm volatile("" ::"s"(l.ss), "s"(l.ds), "s"(l.vlo), "s"(l.vcnt));
}
template <int L> __device__ __forceinline__ void hot_levels(const KArgs &a) {
#pragma unroll
  for (int k = 0; k < L; ++k)
    hot(a.lv[k]);
}
__device__ __forceinline__ void hot_stage(const DevStage &s) {
  asm volatile("" ::"s"(uint32_t{s.vec}), "s"(uint32_t{s.zp_per_ch}), "s"(s.scale_off), "s"(s.zp_off));
  hot(s.ch_rs_div);
  hot(s.ch_re_div);
}
// The stage fields a compile-time chain body reads (generic chains read
// theirs stage by stage).
template <int CH> __device__ __forceinline__ void hot_chain(const KArgs &a) {
  if constexpr (CH == kChainDeqF16 || CH == kChainDeq || CH == kChainQuant) {
    hot_stage(a.chain.st[0]);
    asm volatile("" ::"s"(a.pf), "s"(a.pi));
  } else if constexpr (CH == kChainF16Quant) {
    hot_stage(a.chain.st[1]);
    asm volatile("" ::"s"(a.pf));
  }
}

// Cache policy of the fast kernels' global accesses: nontemporal (streamed
// past the caches) or plain, per family, element widths and `run` (16-byte
// vectors one thread moves back to back), as measured on gfx950 over the
// configurations and a width sweep. Every byte is touched once, so streaming
// pays where each access instruction of a wave covers one contiguous run (the
// stream kernel, the interleave's plane loads) -- except the narrow loads of
// a widening stream (8 or 4 bytes per lane), which run 11-12% faster
// through the cache (C4's int8 -> f16: 29.4 -> 25.8 us). The interleave's
// stores go through the cache (C2: 7.6 -> 7.25 us with one 16-byte vector
// per item; faster too where a thread writes two or more consecutive
// vectors). Transposes read 64 elements per tile row: with one-byte elements
// that is half a 128-byte line whose other half a neighbouring tile reads, so
// those loads stay cached; narrowing transposes store through the cache.
constexpr bool nt_load_policy(int fam, int win, int wout, int run) {
  return fam == kFamTranspose ? win >= 2 : fam == kFamStream ? win >= wout : run == 1;
}
constexpr bool nt_store_policy(int fam, int win, int wout, int run) {
  return fam == kFamTranspose ? wout >= win : fam == kFamInterleave ? false : run == 1;
}
#ifndef RELX_NT_LOAD
#define RELX_NT_LOAD(FAM, WIN, WOUT, RUN) nt_load_policy(FAM, WIN, WOUT, RUN)
#endif
#ifndef RELX_NT_STORE
#define RELX_NT_STORE(FAM, WIN, WOUT, RUN) nt_store_policy(FAM, WIN, WOUT, RUN)
#endif

template <bool NT> __device__ __forceinline__ vec4 ld16(const vec4 *p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

template <bool NT> __device__ __forceinline__ void st16(vec4 *p, const vec4 &v) {
  if constexpr (NT)
    __builtin_nontemporal_store(v, p);
  else
    *p = v;
}

typedef uint32_t vec2 __attribute__((ext_vector_type(2)));

// NB-byte (4, 8 or 16) access into the low words of a 16-byte vector.
// 16 readable bytes for loads whose value is not used (a lane past the end
// of its launch, or a pad plane): pointing such a load here instead of
// branching around it keeps every load of a trip unconditional, so they
// issue back to back. A load under a per-lane branch makes the compiler wait
// for it before the branch ends, which serialises the loads.
__device__ __align__(16) uint8_t g_unused_src[16];

template <int NB, bool NT> __device__ __forceinline__ vec4 ld_n(const uint8_t *p) {
  vec4 r = {0u, 0u, 0u, 0u};
  if constexpr (NB == 16) {
    r = ld16<NT>(reinterpret_cast<const vec4 *>(p));
  } else if constexpr (NB == 8) {
    const vec2 *q = reinterpret_cast<const vec2 *>(p);
    const vec2 t = NT ? __builtin_nontemporal_load(q) : *q;
    r.x = t.x;
    r.y = t.y;
  } else {
    static_assert(NB == 4, "4, 8 or 16 bytes");
    const uint32_t *q = reinterpret_cast<const uint32_t *>(p);
    r.x = NT ? __builtin_nontemporal_load(q) : *q;
  }
  return r;
}

template <int NB, bool NT> __device__ __forceinline__ void st_n(uint8_t *p, const vec4 &v) {
  if constexpr (NB == 16) {
    st16<NT>(reinterpret_cast<vec4 *>(p), v);
  } else if constexpr (NB == 8) {
    vec2 *q = reinterpret_cast<vec2 *>(p);
    const vec2 t = {v.x, v.y};
    if constexpr (NT)
      __builtin_nontemporal_store(t, q);
    else
      *q = t;
  } else {
    static_assert(NB == 4, "4, 8 or 16 bytes");
    uint32_t *q = reinterpret_cast<uint32_t *>(p);
    if constexpr (NT)
      __builtin_nontemporal_store(v.x, q);
    else
      *q = v.x;
  }
}

// --------------------------------------------------------- element access

__device__ __forceinline__ uint64_t load_el(const uint8_t *p, int w) {
  switch (w) {
  case 1:
    return *p;
  case 2:
    return *reinterpret_cast<const uint16_t *>(p);
  case 4:
    return *reinterpret_cast<const uint32_t *>(p);
  default:
    return *reinterpret_cast<const uint64_t *>(p);
  }
}

__device__ __forceinline__ void store_el(uint8_t *p, uint64_t v, int w) {
  switch (w) {
  case 1:
    *p = static_cast<uint8_t>(v);
    break;
  case 2:
    *reinterpret_cast<uint16_t *>(p) = static_cast<uint16_t>(v);
    break;
  case 4:
    *reinterpret_cast<uint32_t *>(p) = static_cast<uint32_t>(v);
    break;
  default:
    *reinterpret_cast<uint64_t *>(p) = v;
  }
}

__device__ int64_t eval_channel(const KArgs &a, const DevStage &s, int64_t o) {
  int64_t st[kMaxChanTokens];
  int sp = 0;
  for (int t = s.tok_begin; t < s.tok_begin + s.tok_count; ++t) {
    const ChanToken &k = a.chain.tok[t];
    switch (k.op) {
    case 1: // PUSH_CONST (symbols were resolved on the host)
      st[sp++] = k.value;
      break;
    case 7: // PUSH_DIM
      st[sp++] = (o / a.rs[k.value]) % a.re[k.value];
      break;
    default: {
      const int64_t r = st[--sp], l = st[--sp];
      int64_t v = 0;
      if (k.op == 2)
        v = l + r;
      else if (k.op == 3)
        v = l - r;
      else if (k.op == 4)
        v = l * r;
      else {
        if (r == 0)
          return -1;
        int64_t q = l / r;
        if ((l % r != 0) && ((l < 0) != (r < 0)))
          --q;
        v = k.op == 5 ? q : l - q * r;
      }
      st[sp++] = v;
    }
    }
  }
  return st[0];
}

// -------------------------------------------------------------- generic

// One element per thread; runtime indices are fine here (correctness path).
__global__ __launch_bounds__(kBlock) __attribute__((unused)) void k_generic(KArgs a, int32_t *status) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < a.work64;
       i += stride) {
    int64_t rem = i, dof = 0, sof = 0;
    bool pad = false;
    for (int k = a.rank - 1; k >= 0; --k) {
      const int64_t e = a.box_ext[k];
      const int64_t p = rem % e + a.box_lo[k];
      rem /= e;
      dof += p * a.ds[k];
      const int64_t v = p - a.lo[k];
      if (v < 0 || v >= a.vext[k])
        pad = true;
      else
        sof += v * a.ss[k];
    }
    uint64_t x;
    if (pad) {
      x = a.fill64;
    } else {
      x = load_el(a.src + sof * a.win, a.win);
      for (int k = 0; k < a.chain.n; ++k) {
        const DevStage &s = a.chain.st[k];
        int64_t c = 0;
        if (s.mode == kChanDim)
          c = (dof / s.ch_rs) % s.ch_re;
        else if (s.mode == kChanExpr)
          c = eval_channel(a, s, dof);
        if (c < 0 || c >= s.len) {
          // channel_out_of_range, reported by the host: a plain store (the
          // flag is in pinned host memory, where atomics would need PCIe
          // atomics; every writer stores the same 1)
          *static_cast<volatile int32_t *>(status) = 1;
          c = 0;
        }
        x = apply(s, static_cast<uint32_t>(x), static_cast<uint32_t>(c), a.pf, a.pi);
      }
    }
    store_el(a.dst + dof * a.wout, x, a.wout);
  }
}

// --------------------------------------------------------- vector helpers

// 32-bit word `i` of an array of 16-byte vectors.
__device__ __forceinline__ uint32_t word(const vec4 *p, int i) { return p[i >> 2][i & 3]; }
__device__ __forceinline__ void set_word(vec4 *p, int i, uint32_t x) { p[i >> 2][i & 3] = x; }

template <int W, int V>
__device__ __forceinline__ void unpack(const vec4 *in, uint32_t (&v)[V]) {
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if constexpr (W == 4)
      v[e] = word(in, e);
    else if constexpr (W == 2)
      v[e] = (word(in, e >> 1) >> ((e & 1) * 16)) & 0xffffu;
    else
      v[e] = (word(in, e >> 2) >> ((e & 3) * 8)) & 0xffu;
  }
}

template <int W, int V>
__device__ __forceinline__ void pack(const uint32_t (&v)[V], vec4 *out) {
  if constexpr (W == 4) {
#pragma unroll
    for (int e = 0; e < V; ++e)
      set_word(out, e, v[e]);
  } else if constexpr (W == 2) {
#pragma unroll
    for (int e = 0; e < V / 2; ++e)
      set_word(out, e, (v[2 * e] & 0xffffu) | (v[2 * e + 1] << 16));
  } else {
#pragma unroll
    for (int e = 0; e < V / 4; ++e)
      set_word(out, e,
               (v[4 * e] & 0xffu) | ((v[4 * e + 1] & 0xffu) << 8) |
                   ((v[4 * e + 2] & 0xffu) << 16) | (v[4 * e + 3] << 24));
  }
}

// One stage over V consecutive destination elements starting at dense result
// offset `o` (channel constant or +1 per element, proven on the host).
template <int V>
__device__ __forceinline__ void stage_vec(const KArgs &a, const DevStage &s, uint32_t (&v)[V],
                                          int64_t o) {
  const uint32_t c = chan_of(s, o);
  switch (s.op) {
  case kOpF32toF16:
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = op_f32_f16(v[e]);
    break;
  case kOpF16toF32:
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = op_f16_f32(v[e]);
    break;
  case kOpF32toBF16:
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = op_f32_bf16(v[e]);
    break;
  case kOpBF16toF32:
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] <<= 16;
    break;
  case kOpQuantize:
    if (s.vec == 0) {
      const float inv = a.pf[s.scale_off + c];
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_quant(v[e], inv);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_quant(v[e], a.pf[s.scale_off + c + e]);
    }
    break;
  default:
    if (s.vec == 0) {
      const float sc = a.pf[s.scale_off + c];
      const int32_t zp = a.pi[s.zp_off + (s.zp_per_ch ? c : 0u)];
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_dequant(v[e], sc, zp);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_dequant(v[e], a.pf[s.scale_off + c + e],
                          a.pi[s.zp_off + (s.zp_per_ch ? c + e : 0u)]);
    }
  }
}

// The stage chain over one vector: compile-time bodies for the common
// sequences, per-stage dispatch (stage index still compile-time) otherwise.
template <int CH, int V>
__device__ __forceinline__ void chain_vec(const KArgs &a, uint32_t (&v)[V], int64_t o) {
  if constexpr (CH == kChainNone) {
  } else if constexpr (CH == kChainF32F16) {
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = op_f32_f16(v[e]);
  } else if constexpr (CH == kChainF16F32) {
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = op_f16_f32(v[e]);
  } else if constexpr (CH == kChainDeqF16) {
    const DevStage &s = a.chain.st[0];
    const uint32_t c = chan_of(s, o);
    if (s.vec == 0) {
      const float sc = a.pf[s.scale_off + c];
      const int32_t zp = a.pi[s.zp_off + (s.zp_per_ch ? c : 0u)];
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_f32_f16(op_dequant(v[e], sc, zp));
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_f32_f16(op_dequant(v[e], a.pf[s.scale_off + c + e],
                                     a.pi[s.zp_off + (s.zp_per_ch ? c + e : 0u)]));
    }
  } else if constexpr (CH == kChainDeq) {
    stage_vec<V>(a, a.chain.st[0], v, o);
  } else if constexpr (CH == kChainF16Quant) {
    const DevStage &s = a.chain.st[1];
    const uint32_t c = chan_of(s, o);
    if (s.vec == 0) {
      const float inv = a.pf[s.scale_off + c];
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = quant_value(op_f16_f32_value(v[e]), inv);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = quant_value(op_f16_f32_value(v[e]), a.pf[s.scale_off + c + e]);
    }
  } else if constexpr (CH == kChainQuant) {
    stage_vec<V>(a, a.chain.st[0], v, o);
  } else {
#pragma unroll
    for (int k = 0; k < kMaxStages; ++k) {
      if (k >= a.chain.n)
        break;
      stage_vec<V>(a, a.chain.st[k], v, o);
    }
  }
}

// Per-vector stage parameters of the compile-time bodies with a per-channel
// stage, for vectors whose channel is constant (DevStage::vec == 0): fetched
// right after a kernel issues its data loads, so that every vector's
// parameter load is in flight with them instead of waited for one by one
// while the vectors are converted. The loads are unconditional (a vector
// with one channel per element reads its first element's entry, in range)
// so that no branch forces an early wait.
struct VecParams {
  float sc;
  int32_t zp;
};

template <int CH> __device__ __forceinline__ VecParams fetch_params(const KArgs &a, int64_t o) {
  VecParams p{0.0f, 0};
  if constexpr (CH == kChainDeqF16) {
    const DevStage &s = a.chain.st[0];
    const uint32_t c = chan_of(s, o);
    p.sc = a.pf[s.scale_off + c];
    p.zp = a.pi[s.zp_off + (s.zp_per_ch ? c : 0u)];
  } else if constexpr (CH == kChainF16Quant) {
    const DevStage &s = a.chain.st[1];
    p.sc = a.pf[s.scale_off + chan_of(s, o)];
  }
  return p;
}

// chain_vec with the parameters of a channel-constant vector given.
template <int CH, int V>
__device__ __forceinline__ void chain_vec_p(const KArgs &a, uint32_t (&v)[V], int64_t o,
                                            const VecParams &p) {
  if constexpr (CH == kChainDeqF16) {
    if (a.chain.st[0].vec == 0) {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = op_f32_f16(op_dequant(v[e], p.sc, p.zp));
      return;
    }
  } else if constexpr (CH == kChainF16Quant) {
    if (a.chain.st[1].vec == 0) {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = quant_value(op_f16_f32_value(v[e]), p.sc);
      return;
    }
  }
  chain_vec<CH, V>(a, v, o);
}

// ---------------------------------------------------------------- stream

// Stream work items hold V = 16/max(win, wout) elements: the wider side
// moves 16 bytes per item, the narrower 8 or 4. Each lane takes U items 64
// apart, so every load and store instruction of a wave covers one contiguous
// run (a lane-contiguous run of two 16-byte vectors per lane measured ~15%
// slower for widening stages). The innermost level counts items.
#ifndef RELX_STREAM_ITEMS
#define RELX_STREAM_ITEMS(WIN, WOUT) 2
#endif

template <int WIN, int WOUT> constexpr int stream_items() {
  return RELX_STREAM_ITEMS(WIN, WOUT);
}

template <int WIN, int WOUT, int L, int CH>
__global__ __launch_bounds__(kBlock) void k_stream(KArgs a) {
  constexpr int V = 16 / (WIN > WOUT ? WIN : WOUT);
  constexpr int BI = V * WIN, BO = V * WOUT;
  constexpr int U = stream_items<WIN, WOUT>();
  static_assert(U == 1 || U == 2, "the 32-bit index covers at most two items per lane");
  constexpr bool NTL = RELX_NT_LOAD(kFamStream, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamStream, WIN, WOUT, 1);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const uint32_t stride = gridDim.x * (kBlock / 64) * (64 * U);
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.work), "s"(a.fill), "s"(a.sbase), "s"(a.dbase),
               "s"(stride));
  hot_levels<L>(a);
  hot_chain<CH>(a);
  for (uint32_t base = wave * (64 * U) + lane; base < a.work; base += stride) {
    int64_t sof[U], dof[U];
    bool pad[U], live[U];
    vec4 in[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = base + 64u * u;
      live[u] = u == 0 || i < a.work;
      sof[u] = a.sbase;
      dof[u] = a.dbase;
      pad[u] = decompose<L>(a.lv, live[u] ? i : base, sof[u], dof[u]);
      if (live[u] && !pad[u])
        in[u] = ld_n<BI, NTL>(a.src + sof[u] * WIN);
    }
    VecParams par[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      par[u] = fetch_params<CH>(a, dof[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!live[u])
        break;
      uint32_t v[V];
      if (pad[u]) {
#pragma unroll
        for (int e = 0; e < V; ++e)
          v[e] = a.fill;
      } else {
        unpack<WIN, V>(&in[u], v);
        chain_vec_p<CH, V>(a, v, dof[u], par[u]);
      }
      vec4 out = {0u, 0u, 0u, 0u};
      pack<WOUT, V>(v, &out);
      st_n<BO, NTS>(a.dst + dof[u] * WOUT, out);
    }
  }
}

// ------------------------------------------------------------- transpose

constexpr int kTile = 64;

// One tile of 64 c by TQ q per block (TQ = 64, or 128 for one-byte sources,
// KArgs::t_wq): [c][q] source rows (q contiguous) into LDS, out as [q][c]
// destination rows (c contiguous). Stages run on the way out.
template <int WIN, int WOUT, int CH, int TQ>
__global__ __launch_bounds__(kBlock) void k_transpose(KArgs a) {
  constexpr int kPitch = TQ + 1;
  __shared__ uint32_t tile[kTile * kPitch]; // [c][q]
  constexpr int VI = 16 / WIN, VO = 16 / WOUT;
  constexpr int VPRI = TQ / VI, VPRO = kTile / VO;
  constexpr int NI = kTile * VPRI / kBlock, NO = TQ * VPRO / kBlock;
  static_assert(NI * kBlock == kTile * VPRI && NO * kBlock == TQ * VPRO, "whole tiles per block");
  constexpr bool NTL = RELX_NT_LOAD(kFamTranspose, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamTranspose, WIN, WOUT, 1);
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.work), "s"(a.sbase), "s"(a.dbase), "s"(a.t_full),
               "s"(a.t_flags), "s"(a.t_choff), "s"(a.t_ssc), "s"(a.t_dsq), "s"(gridDim.x));
  hot(a.t_plane);
  hot(a.t_group);
  hot(a.t_g);
  hot(a.t_tail);
  hot(a.t_nc);
  hot_levels<kBatchLevels>(a);
  hot_chain<CH>(a);
  const uint32_t t = (a.t_flags & kTileXcd) ? xcd_tile(blockIdx.x, gridDim.x) : blockIdx.x;
  if (t >= a.work)
    return;
  uint32_t tq, tc, r2;
  tile_of(a, t, tq, tc, r2);
  int64_t sbase = a.sbase, dbase = a.dbase;
  decompose<kBatchLevels>(a.lv, r2, sbase, dbase); // transposes carry no pads
  const int64_t q0 = static_cast<int64_t>(tq) * TQ, c0 = static_cast<int64_t>(tc) * kTile;
  // load: source rows c (stride t_ssc), contiguous q; all loads in flight
  // before the first LDS write
  vec4 in[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRI, cv = vid % VPRI;
    in[j] = ld16<NTL>(reinterpret_cast<const vec4 *>(
        a.src + (sbase + (c0 + row) * a.t_ssc + q0 + cv * VI) * WIN));
  }
  // the store phase's stage parameters, in flight with the tile loads
  VecParams par[NO];
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRO, cv = vid % VPRO;
    par[j] = fetch_params<CH>(a, dbase + (q0 + row) * a.t_dsq + c0 + cv * VO);
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRI, cv = vid % VPRI;
    uint32_t v[VI];
    unpack<WIN, VI>(&in[j], v);
#pragma unroll
    for (int e = 0; e < VI; ++e)
      tile[row * kPitch + cv * VI + e] = v[e];
  }
  __syncthreads();
  // store: destination rows q (stride t_dsq), contiguous c
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRO, cv = vid % VPRO;
    uint32_t v[VO];
#pragma unroll
    for (int e = 0; e < VO; ++e)
      v[e] = tile[(cv * VO + e) * kPitch + row];
    const int64_t dof = dbase + (q0 + row) * a.t_dsq + c0 + cv * VO;
    chain_vec_p<CH, VO>(a, v, dof, par[j]);
    vec4 out;
    pack<WOUT, VO>(v, &out);
    st16<NTS>(reinterpret_cast<vec4 *>(a.dst + dof * WOUT), out);
  }
}

// One-byte sources with four-byte results whose q and c extents are
// multiples of 128 (KArgs::t_wc 128): a tile of 128 c by 128 q per block,
// kept in LDS as bytes already transposed ([q][c], a 16-byte source segment
// of row c written to column c of 16 rows), and stored in units of one
// 64-element chunk of one result row: a wave's store instruction covers
// 64 / L rows of one chunk (L = lanes per chunk), the block's four waves
// alternate the row's two chunks, so each block writes 512-byte runs of its
// 128 result rows. int8 [4096, 11008] dequantized to f32 and transposed:
// 49.7 -> 41.3 us against the 64 c x 128 q word tile; the same tile for
// f16 results ran 27.8 against 27.9 us and for int8 results 24.2 against
// 23.4 us, so those keep the word tile. The body is written for any result
// width.
template <int WIN, int WOUT, int CH, bool ROWCH, bool ZP0 = false>
__device__ __forceinline__ void transpose_b_body(const KArgs &a) {
  static_assert(WIN == 1, "byte tiles hold one-byte source elements");
  static_assert(!ROWCH || CH == kChainDeqF16, "row channels index the f16 dequantize's parameters");
  constexpr int TC = 128, TQ = 128;
  constexpr int PAD = WOUT == 1 ? 16 : 8, P = TC + PAD; // LDS reads of VO bytes stay aligned
  __shared__ __align__(16) uint8_t tile[TQ * P];        // [q][c]
  constexpr int VPRI = TQ / 16, NI = TC * VPRI / kBlock;
  constexpr int VO = 16 / WOUT;          // result elements (source bytes) per 16-byte store
  constexpr int L = kTile / VO;          // lanes per 64-element chunk of a row
  constexpr int RPI = 64 / L;            // rows per store instruction
  constexpr int NCH = TC / kTile;        // chunks per tile row
  constexpr int NW = kBlock / 64;
  constexpr int NO = TQ * NCH / (RPI * NW);
  static_assert(NI * kBlock == TC * VPRI && NO * RPI * NW == TQ * NCH, "whole tiles per block");
  // the tile reads whole source lines: streaming loads (41.3 against 41.8
  // us cached)
  constexpr bool NTL = true;
  constexpr bool NTS = RELX_NT_STORE(kFamTranspose, 1, WOUT, 1);
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.work), "s"(a.sbase), "s"(a.dbase), "s"(a.t_full),
               "s"(a.t_flags), "s"(a.t_choff), "s"(a.t_ssc), "s"(a.t_dsq), "s"(gridDim.x));
  hot(a.t_plane);
  hot(a.t_group);
  hot(a.t_g);
  hot(a.t_tail);
  hot(a.t_nc);
  hot_levels<kBatchLevels>(a);
  hot_chain<CH>(a);
  const uint32_t t = blockIdx.x;
  if (t >= a.work)
    return;
  uint32_t tq, tc, r2;
  tile_of(a, t, tq, tc, r2);
  int64_t sbase = a.sbase, dbase = a.dbase;
  decompose<kBatchLevels>(a.lv, r2, sbase, dbase); // transposes carry no pads
  const int64_t q0 = static_cast<int64_t>(tq) * TQ, c0 = static_cast<int64_t>(tc) * TC;
  vec4 in[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRI, cv = vid % VPRI;
    in[j] = ld16<NTL>(reinterpret_cast<const vec4 *>(a.src + sbase + (c0 + row) * a.t_ssc + q0 + cv * 16));
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, k = lane / L, v = lane % L;
  // store j of this lane: tile row and chunk, result offset (recomputed after
  // the barrier rather than held across it, which would cost the kernel half
  // its waves)
  auto unit = [&](int j, int &row, int &ch) {
    const int ins = j * NW + wv;
    ch = ins % NCH;
    row = (ins / NCH) * RPI + k;
  };
  const int64_t drow = dbase + q0 * a.t_dsq + c0 + v * VO;
  VecParams par[NO];
  if constexpr (ROWCH) {
    // kTileRowChannel: the channel of row q of the box is t_choff + q; a
    // per-tensor zero point is read once
    const DevStage &s = a.chain.st[0];
    const uint32_t c0r = a.t_choff + static_cast<uint32_t>(q0);
    if (ZP0) { // kTileZeroPoint0 (2% on C3 against a zero read from the table)
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        int row, ch;
        unit(j, row, ch);
        par[j].sc = a.pf[s.scale_off + c0r + row];
        par[j].zp = 0;
      }
    } else if (s.zp_per_ch) {
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        int row, ch;
        unit(j, row, ch);
        par[j].sc = a.pf[s.scale_off + c0r + row];
        par[j].zp = a.pi[s.zp_off + c0r + row];
      }
    } else {
      const int32_t zp = a.pi[s.zp_off];
#pragma unroll
      for (int j = 0; j < NO; ++j) {
        int row, ch;
        unit(j, row, ch);
        par[j].sc = a.pf[s.scale_off + c0r + row];
        par[j].zp = zp;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NO; ++j) {
      int row, ch;
      unit(j, row, ch);
      par[j] = fetch_params<CH>(a, drow + row * a.t_dsq + ch * kTile);
    }
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRI, cv = vid % VPRI;
#pragma unroll
    for (int e = 0; e < 16; ++e)
      tile[(cv * 16 + e) * P + row] = static_cast<uint8_t>(in[j][e >> 2] >> ((e & 3) * 8));
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    int row, ch;
    unit(j, row, ch);
    const uint8_t *tp = tile + row * P + ch * kTile + v * VO;
    const int64_t dof = drow + row * a.t_dsq + ch * kTile;
    vec4 w = {0u, 0u, 0u, 0u};
    if constexpr (VO == 16) {
      w = *reinterpret_cast<const vec4 *>(tp);
    } else if constexpr (VO == 8) {
      const uint2 b = *reinterpret_cast<const uint2 *>(tp);
      w.x = b.x;
      w.y = b.y;
    } else {
      w.x = *reinterpret_cast<const uint32_t *>(tp);
    }
    uint32_t val[VO];
    unpack<1, VO>(&w, val);
    chain_vec_p<CH, VO>(a, val, dof, par[j]);
    vec4 out;
    pack<WOUT, VO>(val, &out);
    st16<NTS>(reinterpret_cast<vec4 *>(a.dst + dof * WOUT), out);
  }
}

template <int WIN, int WOUT, int CH>
__global__ __launch_bounds__(kBlock) void k_transpose_b(KArgs a) {
  transpose_b_body<WIN, WOUT, CH, false>(a);
}

// The compile-time chains at eight waves per SIMD (at most 64 VGPRs, no
// spill; unbounded, int8 -> f16 dequantization takes 70 and seven waves,
// and int8 -> f32 measured 42.3 against 41.8 us). The generic per-stage
// chain would spill under the bound and keeps the kernel above.
template <int WIN, int WOUT, int CH, bool ROWCH, bool ZP0>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_transpose_b8(
    KArgs a) {
  transpose_b_body<WIN, WOUT, CH, ROWCH, ZP0>(a);
}

// ------------------------------------------------------------ interleave

// Axes: [batch..., P, C] with C (padded to CP) innermost in the destination
// and a plane stride in the source; P contiguous in the source. A work item
// is G consecutive pixels (interleave_pixels): one 4-16 byte load per valid
// plane, one packed run of G*CP output elements (16 bytes when a pixel allows).
// Each lane takes U items 64 apart, so every plane load and every store
// instruction of a wave covers one contiguous run. Stages are per tensor.
// The batch index is decomposed over the innermost NL batch levels; the
// launches use all kBatchLevels (an NCHW batch with a per-tensor chain takes
// k_interleave1p below instead).
template <int WIN, int WOUT, int CP, int CH, int NL>
__global__ __launch_bounds__(kBlock) void k_interleave(KArgs a) {
  constexpr int G = interleave_pixels(WIN, WOUT, CP);
  constexpr int BI = G * WIN, BO = G * CP * WOUT;
  static_assert(BO == 4 || BO == 8 || BO % 16 == 0, "packed pixels must fill a store");
  constexpr int NO = BO >= 16 ? BO / 16 : 1;
  constexpr int U = 2;
  constexpr bool NTL = RELX_NT_LOAD(kFamInterleave, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamInterleave, WIN, WOUT, NO);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const uint32_t stride = gridDim.x * (kBlock / 64) * (64 * U);
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.work), "s"(a.fill), "s"(a.sbase), "s"(a.dbase),
               "s"(a.i_ssc), "s"(a.i_loc), "s"(a.i_vc), "s"(stride));
  hot(a.i_ng);
  hot_levels<kBatchLevels>(a);
  hot_chain<CH>(a);
  for (uint32_t base = wave * (64 * U) + lane; base < a.work; base += stride) {
    vec4 in[U][CP];
    bool valid[U][CP], live[U];
    int64_t dbase[U], p0[U];
    // every plane load of both items is issued before any is used
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i0 = base + 64u * u;
      live[u] = u == 0 || i0 < a.work;
      const uint32_t i = live[u] ? i0 : base;
      const uint32_t rest = fdiv(i, a.i_ng);
      const uint32_t g = i - rest * a.i_ng.d;
      int64_t sbase = a.sbase;
      dbase[u] = a.dbase;
      const bool pad = decompose<NL>(a.lv + (kBatchLevels - NL), rest, sbase, dbase[u]);
      p0[u] = static_cast<int64_t>(g) * G; // the pixel axis is unpadded
#pragma unroll
      for (int ch = 0; ch < CP; ++ch) {
        const int32_t vc = ch - a.i_loc;
        valid[u][ch] = live[u] && !pad && static_cast<uint32_t>(vc) < static_cast<uint32_t>(a.i_vc);
        in[u][ch] = ld_n<BI, NTL>(valid[u][ch] ? a.src + (sbase + vc * a.i_ssc + p0[u]) * WIN
                                               : g_unused_src);
      }
    }
    // one body per item with a compile-time index (a runtime-indexed loop
    // the unroller gives up on would move `in` to scratch memory)
    auto emit = [&](auto uc) {
      constexpr int u = decltype(uc)::value;
      uint32_t flat[G * CP];
#pragma unroll
      for (int ch = 0; ch < CP; ++ch) {
        uint32_t v[G];
        if (!valid[u][ch]) {
#pragma unroll
          for (int e = 0; e < G; ++e)
            v[e] = a.fill;
        } else {
          unpack<WIN, G>(&in[u][ch], v);
          chain_vec<CH, G>(a, v, 0);
        }
#pragma unroll
        for (int e = 0; e < G; ++e)
          flat[e * CP + ch] = v[e];
      }
      vec4 out[NO];
      out[0] = vec4{0u, 0u, 0u, 0u};
      pack<WOUT, G * CP>(flat, out);
      uint8_t *dst = a.dst + (dbase[u] + p0[u] * CP) * WOUT;
      if constexpr (BO >= 16) {
#pragma unroll
        for (int j = 0; j < NO; ++j)
          st16<NTS>(reinterpret_cast<vec4 *>(dst) + j, out[j]);
      } else {
        st_n<BO, NTS>(dst, out[0]);
      }
    };
    static_assert(U == 2, "two items per lane");
    emit(std::integral_constant<int, 0>{});
    if (live[1])
      emit(std::integral_constant<int, 1>{});
  }
}

// The one-batch-level interleave (an NCHW batch: the two outer batch levels
// are unit levels) with the arguments its first loads need passed as 14
// leading dwords, which the dispatch preloads into scalar registers
// (k_interleave.hip is built with -amdgpu-kernarg-preload-count=16; 14 is
// what gfx950 takes): the first loads issue without waiting for argument
// loads. The rest comes from the argument block when the stores need it.
// C2: 7.0 -> 6.65-6.8 us.
template <int WIN, int WOUT, int CP, int CH>
__global__ __launch_bounds__(kBlock) void k_interleave1p(const uint8_t *src, int64_t sbase,
                                                         int64_t ssc, uint32_t work,
                                                         uint32_t loc_vc, uint32_t ng_m,
                                                         uint32_t ng_s, uint32_t ng_d,
                                                         uint32_t l_ss, uint32_t l_vlo,
                                                         uint32_t l_vcnt, uint32_t stride, KArgs a) {
  const int32_t loc = static_cast<int16_t>(loc_vc & 0xffffu);
  const int32_t vc_n = static_cast<int32_t>(loc_vc >> 16);
  constexpr int G = interleave_pixels(WIN, WOUT, CP);
  constexpr int BI = G * WIN, BO = G * CP * WOUT;
  constexpr int NO = BO >= 16 ? BO / 16 : 1;
  constexpr int U = 2;
  constexpr bool NTL = RELX_NT_LOAD(kFamInterleave, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamInterleave, WIN, WOUT, NO);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const FastDiv ng{ng_d, ng_m, ng_s, 0u};
  for (uint32_t base = wave * (64 * U) + lane; base < work; base += stride) {
    vec4 in[U][CP];
    bool valid[U][CP], live[U];
    int64_t dbase[U], p0[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i0 = base + 64u * u;
      live[u] = u == 0 || i0 < work;
      const uint32_t i = live[u] ? i0 : base;
      const uint32_t rest = fdiv(i, ng);
      const uint32_t g = i - rest * ng_d;
      const bool pad = rest - l_vlo >= l_vcnt;
      const int64_t sb = sbase + static_cast<int64_t>(rest * l_ss);
      dbase[u] = a.dbase + static_cast<int64_t>(rest * a.lv[2].ds);
      p0[u] = static_cast<int64_t>(g) * G;
#pragma unroll
      for (int ch = 0; ch < CP; ++ch) {
        const int32_t vc = ch - loc;
        valid[u][ch] = live[u] && !pad && static_cast<uint32_t>(vc) < static_cast<uint32_t>(vc_n);
        in[u][ch] = ld_n<BI, NTL>(valid[u][ch] ? src + (sb + vc * ssc + p0[u]) * WIN : g_unused_src);
      }
    }
    auto emit = [&](auto uc) {
      constexpr int u = decltype(uc)::value;
      uint32_t flat[G * CP];
#pragma unroll
      for (int ch = 0; ch < CP; ++ch) {
        uint32_t v[G];
        if (!valid[u][ch]) {
#pragma unroll
          for (int e = 0; e < G; ++e)
            v[e] = a.fill;
        } else {
          unpack<WIN, G>(&in[u][ch], v);
          chain_vec<CH, G>(a, v, 0);
        }
#pragma unroll
        for (int e = 0; e < G; ++e)
          flat[e * CP + ch] = v[e];
      }
      vec4 out[NO];
      out[0] = vec4{0u, 0u, 0u, 0u};
      pack<WOUT, G * CP>(flat, out);
      uint8_t *dst = a.dst + (dbase[u] + p0[u] * CP) * WOUT;
      if constexpr (BO >= 16) {
#pragma unroll
        for (int j = 0; j < NO; ++j)
          st16<NTS>(reinterpret_cast<vec4 *>(dst) + j, out[j]);
      } else {
        st_n<BO, NTS>(dst, out[0]);
      }
    };
    emit(std::integral_constant<int, 0>{});
    if (live[1])
      emit(std::integral_constant<int, 1>{});
  }
}

// ------------------------------------------------------------- permute

// Destination axes [batch..., c, m, e] from a source holding (m, c, e)
// contiguously. A block takes T consecutive m of a group of G consecutive c
// (T source runs of G*E elements, C*E apart), applies the stages on the way
// into LDS, which it fills in destination order [c][t][e], then writes G
// contiguous runs of T*E elements. The blocks of one group come before the
// next group's, so the blocks resident at once write G planes of the result.
template <int WIN, int WOUT, int CH>
__device__ __forceinline__ void permute_body(const KArgs &a) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int VI = 16 / WIN, BO = VI * WOUT;
  constexpr int U = 4; // source vectors in flight per thread
  constexpr bool NTL = RELX_NT_LOAD(kFamPermute, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamPermute, WIN, WOUT, 1);
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.work), "s"(a.sbase), "s"(a.dbase), "s"(a.p_t),
               "s"(a.p_lds), "s"(a.p_dsc));
  hot(a.p_tiles);
  hot(a.p_cgt);
  hot(a.p_ce);
  hot(a.p_ge);
  hot(a.p_e);
  hot(a.p_run);
  asm volatile("" ::"s"(a.p_g));
  hot_levels<kBatchLevels>(a);
  hot_chain<CH>(a);
  const uint32_t t = blockIdx.x;
  if (t >= a.work)
    return;
  // group of G channels (slowest), then batch entry and m-tile
  const uint32_t cg = fdiv(t, a.p_cgt);
  const uint32_t t2 = t - cg * a.p_cgt.d;
  const uint32_t batch = fdiv(t2, a.p_tiles);
  const uint32_t m0 = (t2 - batch * a.p_tiles.d) * a.p_t;
  int64_t sbase = a.sbase, dbase = a.dbase;
  decompose<kBatchLevels>(a.lv, batch, sbase, dbase); // permutes carry no pads
  const uint32_t CE = a.p_ce.d, GE = a.p_ge.d, E = a.p_e.d, c0 = cg * a.p_g;
  // the block's T row parts of GE elements, CE apart
  const vec4 *src = reinterpret_cast<const vec4 *>(
      a.src + (sbase + static_cast<int64_t>(m0) * CE + static_cast<int64_t>(c0) * E) * WIN);
  const uint32_t gap = (CE - GE) / VI; // vectors between two row parts
  const uint32_t nvec = a.p_t * GE / VI;
  for (uint32_t v0 = threadIdx.x; v0 < nvec; v0 += kBlock * U) {
    vec4 in[U];
    // each vector's place: (t, c, e) in the block and its dense result offset
    uint32_t tt[U], rem[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = v0 + u * kBlock < nvec ? v0 + u * kBlock : v0;
      tt[u] = fdiv(v * VI, a.p_ge); // v * VI: element offset in the row parts
      rem[u] = v * VI - tt[u] * GE;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = v0 + u * kBlock;
      if (v < nvec)
        in[u] = ld16<NTL>(src + v + tt[u] * gap);
    }
    uint32_t lds_off[U];
    int64_t ro[U];
    VecParams par[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t cl = fdiv(rem[u], a.p_e);
      const uint32_t e = rem[u] - cl * E;
      lds_off[u] = ((cl * a.p_t + tt[u]) * E + e) * WOUT;
      ro[u] = dbase + (c0 + cl) * a.p_dsc + static_cast<int64_t>(m0 + tt[u]) * E + e;
      par[u] = fetch_params<CH>(a, ro[u]);
    }
    // one body per vector with a compile-time index, so `in` stays in
    // registers whatever the chain's size
    auto emit = [&](auto uc) {
      constexpr int u = decltype(uc)::value;
      const uint32_t v = v0 + u * kBlock;
      if (v >= nvec)
        return;
      uint32_t x[VI];
      unpack<WIN, VI>(&in[u], x);
      chain_vec_p<CH, VI>(a, x, ro[u], par[u]);
      vec4 o[(BO + 15) / 16];
      o[0] = vec4{0u, 0u, 0u, 0u};
      pack<WOUT, VI>(x, o);
      uint8_t *dstl = lds + lds_off[u];
      if constexpr (BO >= 16) {
#pragma unroll
        for (int j = 0; j < BO / 16; ++j)
          reinterpret_cast<vec4 *>(dstl)[j] = o[j];
      } else if constexpr (BO == 8) {
        *reinterpret_cast<vec2 *>(dstl) = vec2{o[0].x, o[0].y};
      } else {
        *reinterpret_cast<uint32_t *>(dstl) = o[0].x;
      }
    };
    static_assert(U == 4, "four vectors in flight");
    emit(std::integral_constant<int, 0>{});
    emit(std::integral_constant<int, 1>{});
    emit(std::integral_constant<int, 2>{});
    emit(std::integral_constant<int, 3>{});
  }
  __syncthreads();
  const uint32_t nout = a.p_lds / 16, run = a.p_run.d;
  uint8_t *dst = a.dst + (dbase + static_cast<int64_t>(c0) * a.p_dsc + static_cast<int64_t>(m0) * E) * WOUT;
  for (uint32_t w = threadIdx.x; w < nout; w += kBlock) {
    const uint32_t cl = fdiv(w, a.p_run);
    const uint32_t j = w - cl * run;
    const vec4 val = reinterpret_cast<const vec4 *>(lds)[w];
    st16<NTS>(reinterpret_cast<vec4 *>(dst + cl * a.p_dsc * WOUT) + j, val);
  }
}

// Stage parameters of a direct launch's vector: entry `ch` of the chain's
// parameter stage.
template <int CH>
__device__ __forceinline__ VecParams direct_params(const PermArgs &a, uint32_t ch) {
  VecParams p{0.0f, 0};
  if constexpr (chain_param_stage(CH) >= 0) {
    p.sc = a.pf[a.scale_off + ch];
    if constexpr (CH == kChainDeqF16 || CH == kChainDeq)
      p.zp = a.pi[a.zp_off + (a.zp_per_ch ? ch : 0u)];
  }
  return p;
}

// The chain over one vector whose parameters are constant across it.
template <int CH, int V>
__device__ __forceinline__ void chain_vec_direct(uint32_t (&v)[V], const VecParams &p) {
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if constexpr (CH == kChainF32F16)
      v[e] = op_f32_f16(v[e]);
    else if constexpr (CH == kChainF16F32)
      v[e] = op_f16_f32(v[e]);
    else if constexpr (CH == kChainDeqF16)
      v[e] = op_f32_f16(op_dequant(v[e], p.sc, p.zp));
    else if constexpr (CH == kChainDeq)
      v[e] = op_dequant(v[e], p.sc, p.zp);
    else if constexpr (CH == kChainF16Quant)
      v[e] = quant_value(op_f16_f32_value(v[e]), p.sc);
    else if constexpr (CH == kChainQuant)
      v[e] = op_quant(v[e], p.sc);
  }
}

// The permute of a direct launch: the same blocks, tile and store order from
// PermArgs, with shifts and masks for the divisions inside a block, the batch
// entry's offset as one multiply, and a vector's parameters by its channel.
template <int WIN, int WOUT, int CH>
__device__ __forceinline__ void permute_direct_body(const PermArgs &a) {
  static_assert(CH != kChainGeneric, "direct launches run compile-time chains");
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int VI = 16 / WIN, BO = VI * WOUT;
  constexpr int U = 2; // source vectors in flight per thread
  constexpr bool NTL = RELX_NT_LOAD(kFamPermute, WIN, WOUT, 1);
  constexpr bool NTS = RELX_NT_STORE(kFamPermute, WIN, WOUT, 1);
  // every argument named at entry: their scalar loads issue in one round
  asm volatile("" ::"s"(a.src), "s"(a.dst), "s"(a.pf), "s"(a.sbase), "s"(a.dbase), "s"(a.dsc),
               "s"(a.work), "s"(a.cgt_d), "s"(a.cgt_m), "s"(a.cgt_s), "s"(a.tiles_d),
               "s"(a.tiles_m), "s"(a.tiles_s));
  asm volatile("" ::"s"(a.t), "s"(a.g), "s"(a.ge_s), "s"(a.e_s), "s"(a.run_s), "s"(a.ce),
               "s"(a.bss), "s"(a.bds), "s"(a.nout), "s"(a.cmask), "s"(a.scale_off));
  if constexpr (CH == kChainDeqF16 || CH == kChainDeq)
    asm volatile("" ::"s"(a.pi), "s"(a.zp_off), "s"(a.zp_per_ch));
  const uint32_t t = blockIdx.x;
  if (t >= a.work)
    return;
  const uint32_t cg = fdiv(t, FastDiv{a.cgt_d, a.cgt_m, a.cgt_s, 0});
  const uint32_t t2 = t - cg * a.cgt_d;
  const uint32_t b = fdiv(t2, FastDiv{a.tiles_d, a.tiles_m, a.tiles_s, 0});
  const uint32_t m0 = (t2 - b * a.tiles_d) * a.t, c0 = cg * a.g;
  const uint32_t GE = 1u << a.ge_s, E = 1u << a.e_s;
  const vec4 *src = reinterpret_cast<const vec4 *>(
      a.src + (a.sbase + static_cast<int64_t>(b) * a.bss + static_cast<int64_t>(m0) * a.ce +
               static_cast<int64_t>(c0) * E) * WIN);
  const uint32_t gap = (a.ce - GE) / VI; // vectors between two row parts
  const uint32_t nvec = (a.t << a.ge_s) / VI;
  for (uint32_t v0 = threadIdx.x; v0 < nvec; v0 += kBlock * U) {
    uint32_t tt[U], rem[U];
    vec4 in[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = v0 + u * kBlock < nvec ? v0 + u * kBlock : v0;
      tt[u] = (v * VI) >> a.ge_s;
      rem[u] = (v * VI) & (GE - 1);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t v = v0 + u * kBlock;
      if (v < nvec)
        in[u] = ld16<NTL>(src + v + tt[u] * gap);
    }
    uint32_t lds_off[U];
    VecParams par[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t cl = rem[u] >> a.e_s, e = rem[u] & (E - 1);
      lds_off[u] = ((cl * a.t + tt[u]) * E + e) * WOUT;
      par[u] = direct_params<CH>(a, (c0 + cl) & a.cmask);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (v0 + u * kBlock >= nvec)
        break;
      uint32_t x[VI];
      unpack<WIN, VI>(&in[u], x);
      chain_vec_direct<CH, VI>(x, par[u]);
      vec4 o[(BO + 15) / 16];
      o[0] = vec4{0u, 0u, 0u, 0u};
      pack<WOUT, VI>(x, o);
      uint8_t *dstl = lds + lds_off[u];
      if constexpr (BO >= 16) {
#pragma unroll
        for (int j = 0; j < BO / 16; ++j)
          reinterpret_cast<vec4 *>(dstl)[j] = o[j];
      } else if constexpr (BO == 8) {
        *reinterpret_cast<vec2 *>(dstl) = vec2{o[0].x, o[0].y};
      } else {
        *reinterpret_cast<uint32_t *>(dstl) = o[0].x;
      }
    }
  }
  __syncthreads();
  uint8_t *dst = a.dst + (a.dbase + static_cast<int64_t>(b) * a.bds + static_cast<int64_t>(c0) * a.dsc +
                          static_cast<int64_t>(m0) * E) * WOUT;
  const uint32_t rmask = (1u << a.run_s) - 1;
  for (uint32_t w = threadIdx.x; w < a.nout; w += kBlock) {
    const vec4 val = reinterpret_cast<const vec4 *>(lds)[w];
    st16<NTS>(reinterpret_cast<vec4 *>(dst + static_cast<int64_t>(w >> a.run_s) * a.dsc * WOUT) +
                  (w & rmask),
              val);
  }
}

template <int WIN, int WOUT, int CH>
__global__ __launch_bounds__(kBlock) void k_permute(KArgs a) {
  permute_body<WIN, WOUT, CH>(a);
}

// The same kernel at eight waves per SIMD (at most 64 VGPRs): 256 CUs then
// hold 2048 blocks of four waves at once, and the power-of-two block counts
// of activation shapes run as whole rounds, instead of ending on a round of
// 256 blocks, one per CU, too few to keep HBM busy. The f16 -> int8 chain
// needs 69 VGPRs without the bound, which leaves seven waves.
template <int WIN, int WOUT, int CH>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_permute8(
    KArgs a) {
  permute_body<WIN, WOUT, CH>(a);
}

template <int WIN, int WOUT, int CH>
__global__ __launch_bounds__(kBlock) void k_permute_direct(PermArgs a) {
  permute_direct_body<WIN, WOUT, CH>(a);
}

template <int WIN, int WOUT, int CH>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_permute_direct8(
    PermArgs a) {
  permute_direct_body<WIN, WOUT, CH>(a);
}

// ------------------------------------------------------------ launch

// One work item per thread up to 2^22 blocks (2^30 work-items per launch,
// inside HIP's 2^32 limit); larger launches grid-stride. Fast-kernel work
// stays below 2^31, so a 32-bit index plus the grid stride cannot wrap.
__attribute__((unused)) unsigned grid_for(int64_t work) {
  const int64_t blocks = (work + kBlock - 1) / kBlock;
  return static_cast<unsigned>(blocks < (1 << 22) ? (blocks > 0 ? blocks : 1) : (1 << 22));
}

template <int WIN, int WOUT, int CH>
hipError_t stream_launch(const KArgs &a, hipStream_t s) {
  constexpr int U = stream_items<WIN, WOUT>();
  const dim3 grid(grid_for((a.work + U - 1) / U)), block(kBlock);
  switch (a.nlev) {
  case 1:
    hipLaunchKernelGGL((k_stream<WIN, WOUT, 1, CH>), grid, block, 0, s, a);
    break;
  case 2:
    hipLaunchKernelGGL((k_stream<WIN, WOUT, 2, CH>), grid, block, 0, s, a);
    break;
  case 4:
    hipLaunchKernelGGL((k_stream<WIN, WOUT, 4, CH>), grid, block, 0, s, a);
    break;
  case 8:
    hipLaunchKernelGGL((k_stream<WIN, WOUT, 8, CH>), grid, block, 0, s, a);
    break;
  default:
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int WIN, int WOUT, int CH>
hipError_t transpose_launch(const KArgs &a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.work)), block(kBlock);
  if (a.t_wc == 128) {
    if constexpr (WIN == 1 && WOUT == 2 && CH == kChainDeqF16) {
      // parameters by row at eight waves; the channel computed from each
      // vector's offset needs 65 registers, so that form runs unbounded
      if ((a.t_flags & kTileRowChannel) && (a.t_flags & kTileZeroPoint0))
        hipLaunchKernelGGL((k_transpose_b8<WIN, WOUT, CH, true, true>), grid, block, 0, s, a);
      else if (a.t_flags & kTileRowChannel)
        hipLaunchKernelGGL((k_transpose_b8<WIN, WOUT, CH, true, false>), grid, block, 0, s, a);
      else
        hipLaunchKernelGGL((k_transpose_b<WIN, WOUT, CH>), grid, block, 0, s, a);
    } else if constexpr (WIN == 1 && WOUT == 4 && CH != kChainGeneric) {
      if (a.t_flags & kTileRowChannel)
        return hipErrorInvalidValue;
      hipLaunchKernelGGL((k_transpose_b8<WIN, WOUT, CH, false, false>), grid, block, 0, s, a);
    } else if constexpr (WIN == 1 && WOUT >= 2) {
      if (a.t_flags & kTileRowChannel)
        return hipErrorInvalidValue;
      hipLaunchKernelGGL((k_transpose_b<WIN, WOUT, CH>), grid, block, 0, s, a);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (a.t_wq == 128) {
    if constexpr (WIN == 1)
      hipLaunchKernelGGL((k_transpose<WIN, WOUT, CH, 128>), grid, block, 0, s, a);
    else
      return hipErrorInvalidValue;
  } else {
    hipLaunchKernelGGL((k_transpose<WIN, WOUT, CH, kTile>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

// The two outer batch levels are unit levels: one valid coordinate each,
// which moves no offset, so decomposing over the innermost level alone gives
// the same offsets and pad flag.
inline bool outer_batch_levels_unit(const KArgs &a) {
  static_assert(kBatchLevels == 3, "two outer batch levels");
  return a.lv[0].div.d == 1 && a.lv[0].vcnt == 1 && a.lv[1].div.d == 1 && a.lv[1].vcnt == 1;
}

template <int WIN, int WOUT, int CH, int CP>
hipError_t interleave_cp(const KArgs &a, hipStream_t s) {
  constexpr int BO = interleave_pixels(WIN, WOUT, CP) * CP * WOUT;
  if constexpr (BO == 4 || BO == 8 || BO % 16 == 0) {
    const dim3 grid(grid_for((a.work + 1) / 2)), block(kBlock);
    // per-tensor chains also come in a one-level variant with preloaded
    // arguments (fewer divisions and no argument-load wait ahead of the
    // first load)
    if (CH != kChainGeneric && outer_batch_levels_unit(a))
      hipLaunchKernelGGL((k_interleave1p<WIN, WOUT, CP, CH>), grid, block, 0, s, a.src, a.sbase,
                         a.i_ssc, a.work,
                         (static_cast<uint32_t>(a.i_loc) & 0xffffu) |
                             (static_cast<uint32_t>(a.i_vc) << 16),
                         a.i_ng.m, a.i_ng.s, a.i_ng.d, a.lv[2].ss, a.lv[2].vlo, a.lv[2].vcnt,
                         grid.x * (kBlock / 64) * (64 * 2), a);
    else
      hipLaunchKernelGGL((k_interleave<WIN, WOUT, CP, CH, kBatchLevels>), grid, block, 0, s, a);
    return hipGetLastError();
  } else {
    return hipErrorInvalidValue;
  }
}

// A direct launch's PermArgs (KArgs::p_direct; the host has proven the shifts,
// the channel entries and a single batch level).
inline PermArgs permute_direct_args(const KArgs &a) {
  PermArgs p{};
  p.src = a.src;
  p.dst = a.dst;
  p.pf = a.pf;
  p.pi = a.pi;
  p.sbase = a.sbase;
  p.dbase = a.dbase;
  p.dsc = a.p_dsc;
  p.work = a.work;
  p.cgt_d = a.p_cgt.d;
  p.cgt_m = a.p_cgt.m;
  p.cgt_s = a.p_cgt.s;
  p.tiles_d = a.p_tiles.d;
  p.tiles_m = a.p_tiles.m;
  p.tiles_s = a.p_tiles.s;
  p.t = a.p_t;
  p.g = a.p_g;
  p.ge_s = a.p_ge.s;
  p.e_s = a.p_e.s;
  p.run_s = a.p_run.s;
  p.ce = a.p_ce.d;
  p.bss = a.lv[kBatchLevels - 1].ss;
  p.bds = a.lv[kBatchLevels - 1].ds;
  p.nout = a.p_lds / 16;
  p.cmask = a.p_cmask;
  const int k = chain_param_stage(a.chain_code);
  if (k >= 0) {
    p.scale_off = a.chain.st[k].scale_off;
    p.zp_off = a.chain.st[k].zp_off;
    p.zp_per_ch = a.chain.st[k].zp_per_ch;
  }
  return p;
}

template <int WIN, int WOUT, int CH>
hipError_t permute_launch(const KArgs &a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.work)), block(kBlock);
  if constexpr (CH != kChainGeneric) {
    if (a.p_direct) {
      const PermArgs p = permute_direct_args(a);
      if constexpr (permute_eight_waves(WIN, CH))
        hipLaunchKernelGGL((k_permute_direct8<WIN, WOUT, CH>), grid, block, a.p_lds, s, p);
      else
        hipLaunchKernelGGL((k_permute_direct<WIN, WOUT, CH>), grid, block, a.p_lds, s, p);
      return hipGetLastError();
    }
  }
  if constexpr (permute_eight_waves(WIN, CH))
    hipLaunchKernelGGL((k_permute8<WIN, WOUT, CH>), grid, block, a.p_lds, s, a);
  else
    hipLaunchKernelGGL((k_permute<WIN, WOUT, CH>), grid, block, a.p_lds, s, a);
  return hipGetLastError();
}

template <int WIN, int WOUT, int CH>
hipError_t interleave_launch(const KArgs &a, hipStream_t s) {
  switch (a.cpad) {
  case 2:
    return interleave_cp<WIN, WOUT, CH, 2>(a, s);
  case 4:
    return interleave_cp<WIN, WOUT, CH, 4>(a, s);
  case 8:
    return interleave_cp<WIN, WOUT, CH, 8>(a, s);
  default:
    return hipErrorInvalidValue;
  }
}

// Instantiations are split over several translation units (one per family
// and chain class) so the build compiles them in parallel.
#define RELX_DISPATCH_FAST(NAME, FN)                                                       \
  hipError_t NAME(const KArgs &a, hipStream_t s, bool &handled) {                          \
    const int w = a.win * 8 + a.wout;                                                      \
    handled = true;                                                                        \
    switch (a.chain_code) {                                                                \
    case kChainNone:                                                                       \
      if (w == 9)                                                                          \
        return FN<1, 1, kChainNone>(a, s);                                                 \
      if (w == 18)                                                                         \
        return FN<2, 2, kChainNone>(a, s);                                                 \
      if (w == 36)                                                                         \
        return FN<4, 4, kChainNone>(a, s);                                                 \
      break;                                                                               \
    case kChainF32F16:                                                                     \
      if (w == 34)                                                                         \
        return FN<4, 2, kChainF32F16>(a, s);                                               \
      break;                                                                               \
    case kChainF16F32:                                                                     \
      if (w == 20)                                                                         \
        return FN<2, 4, kChainF16F32>(a, s);                                               \
      break;                                                                               \
    case kChainDeqF16:                                                                     \
      if (w == 10)                                                                         \
        return FN<1, 2, kChainDeqF16>(a, s);                                               \
      break;                                                                               \
    case kChainDeq:                                                                        \
      if (w == 12)                                                                         \
        return FN<1, 4, kChainDeq>(a, s);                                                  \
      break;                                                                               \
    case kChainF16Quant:                                                                   \
      if (w == 17)                                                                         \
        return FN<2, 1, kChainF16Quant>(a, s);                                             \
      break;                                                                               \
    case kChainQuant:                                                                      \
      if (w == 33)                                                                         \
        return FN<4, 1, kChainQuant>(a, s);                                                \
      break;                                                                               \
    default:                                                                               \
      break;                                                                               \
    }                                                                                      \
    handled = false;                                                                       \
    return hipSuccess;                                                                     \
  }

#define RELX_DISPATCH_GENERIC(NAME, FN)                                                    \
  hipError_t NAME(const KArgs &a, hipStream_t s) {                                         \
    switch (a.win * 8 + a.wout) {                                                          \
    case 9:                                                                                \
      return FN<1, 1, kChainGeneric>(a, s);                                                \
    case 10:                                                                               \
      return FN<1, 2, kChainGeneric>(a, s);                                                \
    case 12:                                                                               \
      return FN<1, 4, kChainGeneric>(a, s);                                                \
    case 17:                                                                               \
      return FN<2, 1, kChainGeneric>(a, s);                                                \
    case 18:                                                                               \
      return FN<2, 2, kChainGeneric>(a, s);                                                \
    case 20:                                                                               \
      return FN<2, 4, kChainGeneric>(a, s);                                                \
    case 33:                                                                               \
      return FN<4, 1, kChainGeneric>(a, s);                                                \
    case 34:                                                                               \
      return FN<4, 2, kChainGeneric>(a, s);                                                \
    case 36:                                                                               \
      return FN<4, 4, kChainGeneric>(a, s);                                                \
    default:                                                                               \
      return hipErrorInvalidValue;                                                         \
    }                                                                                      \
  }

} // namespace

// Entry points of the per-family translation units.
hipError_t stream_fast(const KArgs &a, hipStream_t s, bool &handled);
hipError_t stream_generic(const KArgs &a, hipStream_t s);
hipError_t transpose_fast(const KArgs &a, hipStream_t s, bool &handled);
hipError_t transpose_generic(const KArgs &a, hipStream_t s);
hipError_t interleave_fast(const KArgs &a, hipStream_t s, bool &handled);
hipError_t interleave_generic(const KArgs &a, hipStream_t s);
hipError_t permute_fast(const KArgs &a, hipStream_t s, bool &handled);
hipError_t permute_generic(const KArgs &a, hipStream_t s);

} // namespace relx
