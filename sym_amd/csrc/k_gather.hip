// k_gather.hip - row gather kernels for indexed plans (index_select along
// axis 0 of a device-resident table, with the plan's optional cast fused).
//
// Each lane moves one vector item (up to 16 bytes of a row) at a time, two
// or four items 64 apart per trip (gather_items), like the stream kernel: a wave covers 64
// consecutive items of the output, which are consecutive items of one or a
// few source rows, so loads and stores stay contiguous per row. The row index
// of an item comes from one division by the row length in items; lanes of the
// same row read the same index word. Output is written once and streamed past
// the caches. Table loads of long rows (256 bytes or more, 8- or 16-byte
// items) stream too (3-4% faster); short rows load through the cache, where
// neighbouring rows share lines (20-byte rows: 94 us cached, 128 us
// streamed).
#include "kernels.h"

#ifndef RELX_GATHER_NT_STORE
#define RELX_GATHER_NT_STORE true
#endif

namespace relx {
namespace {

template <int NB, bool NT> __device__ __forceinline__ vec4 gload(const uint8_t *p) {
  if constexpr (NB >= 4) {
    return ld_n<NB, NT>(p);
  } else {
    vec4 r = {0u, 0u, 0u, 0u};
    if constexpr (NB == 2)
      r.x = *reinterpret_cast<const uint16_t *>(p);
    else
      r.x = *p;
    return r;
  }
}

template <int NB, bool NT> __device__ __forceinline__ void gstore(uint8_t *p, const vec4 &v) {
  if constexpr (NB >= 4) {
    st_n<NB, NT>(p, v);
  } else if constexpr (NB == 2) {
    *reinterpret_cast<uint16_t *>(p) = static_cast<uint16_t>(v.x);
  } else {
    *p = static_cast<uint8_t>(v.x);
  }
}

constexpr int gather_out_bytes(int op, int nbi) {
  return op == kGatherCopy ? nbi : op == kGatherF32F16 ? nbi / 2 : nbi * 2;
}

// Items per lane: a widening gather loads half its store bytes per item and
// takes four items 64 apart (f16 -> f32 rows of 2 KiB: 75.7 -> 72.5 us); the
// others take two (four slowed them by 3-4%).
constexpr int gather_items(int op) { return op == kGatherF16F32 ? 4 : 2; }

// One item's value conversion: NBI source bytes -> the item's output bytes.
template <int OP, int NBI> __device__ __forceinline__ vec4 convert(const vec4 &in) {
  if constexpr (OP == kGatherCopy) {
    return in;
  } else if constexpr (OP == kGatherF32F16) {
    constexpr int V = NBI / 4;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < V; ++e)
      w[e >> 1] |= op_f32_f16(in[e]) << ((e & 1) * 16);
    return vec4{w[0], w[1], 0u, 0u};
  } else {
    constexpr int V = NBI / 2;
    vec4 out = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < V; ++e)
      out[e] = op_f16_f32((in[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
    return out;
  }
}

template <int OP, int NBI, int IW, bool NTL>
__global__ __launch_bounds__(kBlock) void k_gather(GatherArgs a) {
  constexpr int NBO = gather_out_bytes(OP, NBI);
  constexpr int U = gather_items(OP);
  constexpr bool NTS = RELX_GATHER_NT_STORE;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  const uint32_t stride = gridDim.x * (kBlock / 64) * (64 * U);
  // every argument in one batch of scalar loads (see hot() in kernels.h)
  asm volatile("" ::"s"(a.table), "s"(a.dst), "s"(a.idx), "s"(a.work), "s"(a.row_items),
               "s"(stride));
  hot(a.per_row);
  for (uint32_t base = wave * (64 * U) + lane; base < a.work; base += stride) {
    vec4 in[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i0 = base + 64u * u;
      live[u] = u == 0 || i0 < a.work;
      // a lane past the end re-reads its first item: every load of the trip
      // is unconditional, so the index and table loads of all items issue
      // back to back (a load under a per-lane branch is waited for before
      // the branch ends)
      const uint32_t i = live[u] ? i0 : base;
      const uint32_t r = fdiv(i, a.per_row);
      const uint32_t c = i - r * a.row_items;
      int64_t row;
      if constexpr (IW == 4)
        row = reinterpret_cast<const int32_t *>(a.idx)[r];
      else
        row = reinterpret_cast<const int64_t *>(a.idx)[r];
      const uint64_t item = static_cast<uint64_t>(row) * a.row_items + c;
      in[u] = gload<NBI, NTL>(a.table + item * NBI);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!live[u])
        break;
      const uint32_t i = base + 64u * u;
      gstore<NBO, NTS>(a.dst + static_cast<uint64_t>(i) * NBO, convert<OP, NBI>(in[u]));
    }
  }
}

template <int OP, int NBI>
hipError_t gather_iw(const GatherArgs &a, int iw, bool nt, hipStream_t s) {
  constexpr int U = gather_items(OP);
  const dim3 grid(grid_for((static_cast<int64_t>(a.work) + U - 1) / U)), block(kBlock);
  if constexpr (NBI >= 8) {
    if (nt) {
      if (iw == 4)
        hipLaunchKernelGGL((k_gather<OP, NBI, 4, true>), grid, block, 0, s, a);
      else if (iw == 8)
        hipLaunchKernelGGL((k_gather<OP, NBI, 8, true>), grid, block, 0, s, a);
      else
        return hipErrorInvalidValue;
      return hipGetLastError();
    }
  } else if (nt) {
    return hipErrorInvalidValue;
  }
  if (iw == 4)
    hipLaunchKernelGGL((k_gather<OP, NBI, 4, false>), grid, block, 0, s, a);
  else if (iw == 8)
    hipLaunchKernelGGL((k_gather<OP, NBI, 8, false>), grid, block, 0, s, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

} // namespace

// Launch one gather: `op` a GatherOp, `nbi` source bytes per item (copy 1, 2,
// 4, 8 or 16; f32 -> f16 4, 8 or 16; f16 -> f32 2, 4 or 8), `iw` index bytes,
// `nt` streaming table loads (items of 8 bytes or more only).
hipError_t gather_launch(const GatherArgs &a, int op, int nbi, int iw, bool nt, hipStream_t s) {
  if (a.work == 0)
    return hipSuccess;
  switch (op) {
  case kGatherCopy:
    switch (nbi) {
    case 1:
      return gather_iw<kGatherCopy, 1>(a, iw, nt, s);
    case 2:
      return gather_iw<kGatherCopy, 2>(a, iw, nt, s);
    case 4:
      return gather_iw<kGatherCopy, 4>(a, iw, nt, s);
    case 8:
      return gather_iw<kGatherCopy, 8>(a, iw, nt, s);
    case 16:
      return gather_iw<kGatherCopy, 16>(a, iw, nt, s);
    }
    break;
  case kGatherF32F16:
    switch (nbi) {
    case 4:
      return gather_iw<kGatherF32F16, 4>(a, iw, nt, s);
    case 8:
      return gather_iw<kGatherF32F16, 8>(a, iw, nt, s);
    case 16:
      return gather_iw<kGatherF32F16, 16>(a, iw, nt, s);
    }
    break;
  case kGatherF16F32:
    switch (nbi) {
    case 2:
      return gather_iw<kGatherF16F32, 2>(a, iw, nt, s);
    case 4:
      return gather_iw<kGatherF16F32, 4>(a, iw, nt, s);
    case 8:
      return gather_iw<kGatherF16F32, 8>(a, iw, nt, s);
    }
    break;
  }
  return hipErrorInvalidValue;
}

} // namespace relx
