// kernels.hip - gfx950 relayout + value-stage kernels.
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
//   stream     innermost axis contiguous on both sides: 16-byte vector
//              loads/stores, one vector per thread
//   transpose  batched 2-D transpose through a 64x64 LDS tile (32-bit
//              words, row pitch 65: conflict-free for every element width
//              pairing used), XCD-grouped tile order
//   interleave planar -> interleaved with a small padded inner axis
//              (NCHW -> NHWC + pad): per-plane 16-byte loads, packed pixels
#include <hip/hip_runtime.h>

#include "program.h"

namespace relx {
namespace {

constexpr int kBlock = 256;

// Native 16-byte vector (the nontemporal builtins need a builtin vector type).
typedef uint32_t vec4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  const uint32_t hi = __umulhi(n, f.m);
  return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> f.s);
}

// ------------------------------------------------------------ value ops

__device__ __forceinline__ uint32_t op_f32_f16(uint32_t b) {
  const _Float16 h = static_cast<_Float16>(__uint_as_float(b));
  uint32_t r = __builtin_bit_cast(unsigned short, h);
  if ((b & 0x7fffffffu) > 0x7f800000u) // NaN: quiet, top payload bits kept
    r = ((b >> 16) & 0x8000u) | 0x7e00u | ((b >> 13) & 0x3ffu);
  return r;
}

__device__ __forceinline__ uint32_t op_f16_f32(uint32_t h) {
  const _Float16 x = __builtin_bit_cast(_Float16, static_cast<unsigned short>(h));
  uint32_t r = __float_as_uint(static_cast<float>(x));
  if ((h & 0x7c00u) == 0x7c00u && (h & 0x3ffu)) // NaN: payload shifted, not quieted
    r = ((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13);
  return r;
}

__device__ __forceinline__ uint32_t op_f32_bf16(uint32_t b) {
  if ((b & 0x7fffffffu) > 0x7f800000u)
    return ((b >> 16) | 0x40u) & 0xffffu;
  const uint64_t w = b;
  return static_cast<uint32_t>((w + 0x7fffu + ((w >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t op_quant(uint32_t b, float inv) {
  float y = __uint_as_float(b) * inv;
  y = __builtin_fmaxf(y, -128.0f); // maxNum: NaN -> -128
  y = __builtin_fminf(y, 127.0f);
  return static_cast<uint32_t>(static_cast<int32_t>(__builtin_rintf(y))) & 0xffu;
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

__global__ __launch_bounds__(kBlock) void k_generic(KArgs a, int32_t *status) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < a.work;
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
      x = a.fill;
    } else {
      x = load_el(a.src + sof * a.win, a.win);
      for (int k = 0; k < a.chain.n; ++k) {
        const DevStage &s = a.chain.st[k];
        int64_t c = 0;
        if (s.mode == kChanDim)
          c = (dof / a.rs[s.dim]) % a.re[s.dim];
        else if (s.mode == kChanExpr)
          c = eval_channel(a, s, dof);
        if (c < 0 || c >= s.len) {
          atomicExch(status, 1); // channel_out_of_range, reported by the host
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

// Apply the chain to V consecutive destination elements starting at dense
// result offset `o` (channels constant or +1 per element, per the host's
// eligibility proof).
template <int V>
__device__ __forceinline__ void chain_vec(const KArgs &a, uint32_t (&v)[V], int64_t o) {
  for (int k = 0; k < a.chain.n; ++k) {
    const DevStage &s = a.chain.st[k];
    uint32_t c = 0;
    if (s.mode == kChanDim) {
      if (a.idx32) {
        const uint32_t q = fdiv(static_cast<uint32_t>(o), a.rs_div[s.dim]);
        c = q - fdiv(q, a.re_div[s.dim]) * a.re_div[s.dim].d;
      } else {
        c = static_cast<uint32_t>((o / a.rs[s.dim]) % a.re[s.dim]);
      }
    }
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
}

// ---------------------------------------------------------------- stream

// Box decomposition of work item `i` into padded coordinates; `inner_mul`
// scales the innermost box coordinate (vector index -> element index).
// Returns true when any coordinate lies in a pad.
__device__ __forceinline__ bool locate(const KArgs &a, int64_t i, int inner_mul, int64_t &sof,
                                       int64_t &dof) {
  bool pad = false;
  sof = 0;
  dof = 0;
  if (a.idx32) {
    uint32_t rem = static_cast<uint32_t>(i);
#pragma unroll
    for (int k = kMaxRank - 1; k >= 0; --k) {
      if (k >= a.rank)
        continue;
      const uint32_t q = fdiv(rem, a.box_div[k]);
      uint32_t ck = rem - q * a.box_div[k].d;
      rem = q;
      if (k == a.rank - 1)
        ck *= inner_mul;
      const int64_t p = static_cast<int64_t>(ck) + a.box_lo[k];
      dof += p * a.ds[k];
      const int64_t v = p - a.lo[k];
      if (v < 0 || v >= a.vext[k])
        pad = true;
      else
        sof += v * a.ss[k];
    }
  } else {
    int64_t rem = i;
    for (int k = a.rank - 1; k >= 0; --k) {
      const int64_t e = k == a.rank - 1 ? a.box_ext[k] / inner_mul : a.box_ext[k];
      int64_t ck = rem % e;
      rem /= e;
      if (k == a.rank - 1)
        ck *= inner_mul;
      const int64_t p = ck + a.box_lo[k];
      dof += p * a.ds[k];
      const int64_t v = p - a.lo[k];
      if (v < 0 || v >= a.vext[k])
        pad = true;
      else
        sof += v * a.ss[k];
    }
  }
  return pad;
}

template <int WIN, int WOUT>
__global__ __launch_bounds__(kBlock) void k_stream(KArgs a) {
  constexpr int V = 16 / (WIN < WOUT ? WIN : WOUT);
  constexpr int NI = V * WIN / 16, NO = V * WOUT / 16;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < a.work;
       i += stride) {
    int64_t sof, dof;
    const bool pad = locate(a, i, V, sof, dof);
    uint32_t v[V];
    if (pad) {
#pragma unroll
      for (int e = 0; e < V; ++e)
        v[e] = static_cast<uint32_t>(a.fill);
    } else {
      vec4 in[NI];
      const vec4 *src = reinterpret_cast<const vec4 *>(a.src + sof * WIN);
#pragma unroll
      for (int j = 0; j < NI; ++j)
        in[j] = __builtin_nontemporal_load(src + j);
      unpack<WIN, V>(in, v);
      chain_vec<V>(a, v, dof);
    }
    vec4 out[NO];
    pack<WOUT, V>(v, out);
    vec4 *dst = reinterpret_cast<vec4 *>(a.dst + dof * WOUT);
#pragma unroll
    for (int j = 0; j < NO; ++j)
      __builtin_nontemporal_store(out[j], dst + j);
  }
}

// ------------------------------------------------------------- transpose

constexpr int kTile = 64;
constexpr int kPitch = kTile + 1;

// Map a linear block id so that the blocks one XCD runs (ids congruent mod 8)
// take a contiguous run of tiles: neighbouring tiles share source cache lines.
__device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t n) {
  constexpr uint32_t kXcd = 8;
  if (n < kXcd)
    return b;
  const uint32_t per = n / kXcd, extra = n % kXcd, x = b % kXcd, j = b / kXcd;
  // XCD x owns tiles [x*per + min(x, extra), ...) of length per + (x < extra)
  return x * per + (x < extra ? x : extra) + j;
}

template <int WIN, int WOUT>
__global__ __launch_bounds__(kBlock) void k_transpose(KArgs a) {
  __shared__ uint32_t tile[kTile * kPitch]; // [c][q]
  constexpr int VI = 16 / WIN, VO = 16 / WOUT;
  constexpr int VPRI = kTile / VI, VPRO = kTile / VO;
  constexpr int NI = kTile * VPRI / kBlock, NO = kTile * VPRO / kBlock;
  const int qa = a.qa, ca = a.ca;
  const int64_t nq = a.box_ext[qa] / kTile, nc = a.box_ext[ca] / kTile;
  const uint32_t t = xcd_tile(blockIdx.x, gridDim.x);
  if (t >= a.work)
    return;
  int64_t rest = t;
  const int64_t tq = rest % nq;
  rest /= nq;
  const int64_t tc = rest % nc;
  rest /= nc;
  // batch axes: every axis other than qa/ca, row-major over the box
  int64_t sbase = 0, dbase = 0;
  for (int k = a.rank - 1; k >= 0; --k) {
    if (k == qa || k == ca)
      continue;
    const int64_t e = a.box_ext[k];
    const int64_t p = rest % e + a.box_lo[k];
    rest /= e;
    sbase += p * a.ss[k];
    dbase += p * a.ds[k];
  }
  const int64_t q0 = a.box_lo[qa] + tq * kTile, c0 = a.box_lo[ca] + tc * kTile;
  // load: source rows c (stride ss[ca]), contiguous q
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int row = vid / VPRI, cv = vid % VPRI;
    const vec4 *p = reinterpret_cast<const vec4 *>(
        a.src + (sbase + (c0 + row) * a.ss[ca] + q0 + cv * VI) * WIN);
    vec4 in = __builtin_nontemporal_load(p);
    uint32_t v[VI];
    unpack<WIN, VI>(&in, v);
#pragma unroll
    for (int e = 0; e < VI; ++e)
      tile[row * kPitch + cv * VI + e] = v[e];
  }
  __syncthreads();
  // store: destination rows q (stride ds[qa]), contiguous c
#pragma unroll
  for (int j = 0; j < NO; ++j) {
    const int vid = threadIdx.x + j * kBlock;
    const int q = vid / VPRO, cv = vid % VPRO;
    uint32_t v[VO];
#pragma unroll
    for (int e = 0; e < VO; ++e)
      v[e] = tile[(cv * VO + e) * kPitch + q];
    const int64_t o = dbase + (q0 + q) * a.ds[qa] + c0 + cv * VO;
    chain_vec<VO>(a, v, o);
    vec4 out;
    pack<WOUT, VO>(v, &out);
    __builtin_nontemporal_store(out, reinterpret_cast<vec4 *>(a.dst + o * WOUT));
  }
}

// ------------------------------------------------------------ interleave

// Axes: [batch..., P, C] with C (padded to CP) innermost in the destination
// and a plane stride in the source; P contiguous in the source. Each thread
// takes G = 16/WIN consecutive pixels: one 16-byte load per valid plane, one
// packed run of G*CP output elements.
template <int WIN, int WOUT, int CP>
__global__ __launch_bounds__(kBlock) void k_interleave(KArgs a) {
  constexpr int G = 16 / WIN;
  constexpr int NO = G * CP * WOUT / 16;
  static_assert(G * CP * WOUT % 16 == 0, "packed pixels must fill whole vectors");
  const int r = a.rank;
  const int pa = r - 2, ca = r - 1;
  const int64_t ngroups = a.box_ext[pa] / G;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < a.work;
       i += stride) {
    int64_t rest = i;
    const int64_t g = rest % ngroups;
    rest /= ngroups;
    int64_t sbase = 0, dbase = 0;
    bool pad = false;
    for (int k = pa - 1; k >= 0; --k) {
      const int64_t e = a.box_ext[k];
      const int64_t p = rest % e + a.box_lo[k];
      rest /= e;
      dbase += p * a.ds[k];
      const int64_t v = p - a.lo[k];
      if (v < 0 || v >= a.vext[k])
        pad = true;
      else
        sbase += v * a.ss[k];
    }
    const int64_t p0 = a.box_lo[pa] + g * G; // pixel axis is unpadded
    uint32_t px[CP][G];
#pragma unroll
    for (int ch = 0; ch < CP; ++ch) {
      const int64_t vc = ch - a.lo[ca];
      if (pad || vc < 0 || vc >= a.vext[ca]) {
#pragma unroll
        for (int e = 0; e < G; ++e)
          px[ch][e] = static_cast<uint32_t>(a.fill);
      } else {
        vec4 in = __builtin_nontemporal_load(
            reinterpret_cast<const vec4 *>(a.src + (sbase + vc * a.ss[ca] + p0) * WIN));
        uint32_t v[G];
        unpack<WIN, G>(&in, v);
        for (int k = 0; k < a.chain.n; ++k) { // per-tensor stages only
          const DevStage &s = a.chain.st[k];
#pragma unroll
          for (int e = 0; e < G; ++e)
            v[e] = apply(s, v[e], 0u, a.pf, a.pi);
        }
#pragma unroll
        for (int e = 0; e < G; ++e)
          px[ch][e] = v[e];
      }
    }
    uint32_t flat[G * CP];
#pragma unroll
    for (int e = 0; e < G; ++e)
#pragma unroll
      for (int ch = 0; ch < CP; ++ch)
        flat[e * CP + ch] = px[ch][e];
    vec4 out[NO];
    pack<WOUT, G * CP>(flat, out);
    vec4 *dst = reinterpret_cast<vec4 *>(a.dst + (dbase + p0 * CP) * WOUT);
#pragma unroll
    for (int j = 0; j < NO; ++j)
      __builtin_nontemporal_store(out[j], dst + j);
  }
}

// ------------------------------------------------------------ dispatch

unsigned grid_for(int64_t work) {
  const int64_t blocks = (work + kBlock - 1) / kBlock;
  return static_cast<unsigned>(blocks < (1 << 20) ? (blocks > 0 ? blocks : 1) : (1 << 20));
}

template <int WIN, int WOUT>
hipError_t stream_launch(const KArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((k_stream<WIN, WOUT>), dim3(grid_for(a.work)), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

template <int WIN, int WOUT>
hipError_t transpose_launch(const KArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((k_transpose<WIN, WOUT>), dim3(static_cast<unsigned>(a.work)), dim3(kBlock),
                     0, s, a);
  return hipGetLastError();
}

template <int WIN, int WOUT, int CP>
hipError_t interleave_launch(const KArgs &a, hipStream_t s) {
  if constexpr ((16 / WIN) * CP * WOUT % 16 == 0) {
    hipLaunchKernelGGL((k_interleave<WIN, WOUT, CP>), dim3(grid_for(a.work)), dim3(kBlock), 0,
                       s, a);
    return hipGetLastError();
  } else {
    return hipErrorInvalidValue;
  }
}

#define RELX_W2(F, ...)                                                                    \
  switch (a.win * 8 + a.wout) {                                                            \
  case 1 * 8 + 1: return F<1, 1 __VA_ARGS__>(a, s);                                        \
  case 1 * 8 + 2: return F<1, 2 __VA_ARGS__>(a, s);                                        \
  case 1 * 8 + 4: return F<1, 4 __VA_ARGS__>(a, s);                                        \
  case 2 * 8 + 1: return F<2, 1 __VA_ARGS__>(a, s);                                        \
  case 2 * 8 + 2: return F<2, 2 __VA_ARGS__>(a, s);                                        \
  case 2 * 8 + 4: return F<2, 4 __VA_ARGS__>(a, s);                                        \
  case 4 * 8 + 1: return F<4, 1 __VA_ARGS__>(a, s);                                        \
  case 4 * 8 + 2: return F<4, 2 __VA_ARGS__>(a, s);                                        \
  case 4 * 8 + 4: return F<4, 4 __VA_ARGS__>(a, s);                                        \
  default: return hipErrorInvalidValue;                                                    \
  }

hipError_t interleave_dispatch(const KArgs &a, hipStream_t s) {
  switch (a.cpad) {
  case 2:
    RELX_W2(interleave_launch, , 2)
  case 4:
    RELX_W2(interleave_launch, , 4)
  case 8:
    RELX_W2(interleave_launch, , 8)
  default:
    return hipErrorInvalidValue;
  }
}

} // namespace

// Launch one box of a program. `status` is a device int the generic kernel
// sets when a channel index falls outside its parameter table.
hipError_t launch_box(int family, const KArgs &a, int32_t *status, hipStream_t s) {
  if (a.work <= 0)
    return hipSuccess;
  switch (family) {
  case kFamStream:
    RELX_W2(stream_launch, )
  case kFamTranspose:
    RELX_W2(transpose_launch, )
  case kFamInterleave:
    return interleave_dispatch(a, s);
  default:
    hipLaunchKernelGGL(k_generic, dim3(grid_for(a.work)), dim3(kBlock), 0, s, a, status);
    return hipGetLastError();
  }
}

} // namespace relx
