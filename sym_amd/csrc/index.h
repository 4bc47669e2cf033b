// index.h - index arithmetic shared by the fast kernels and the host-side
// launch verifier (program.cpp), so both derive exactly the same offsets.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "program.h"

namespace relx {

// n / d for n < 2^32: q = (umulhi(n, m) + n) >> s.
__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> 32);
  return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> f.s);
}

// Parameter entry of a stage for dense result offset `o` (fast kernels:
// the result has fewer than 2^32 elements whenever a stage is per-channel;
// per-tensor stages carry rs = re = 1, which yields entry 0 for any o).
__host__ __device__ __forceinline__ uint32_t chan_of(const DevStage &s, int64_t o) {
  const uint32_t q = fdiv(static_cast<uint32_t>(o), s.ch_rs_div);
  return q - fdiv(q, s.ch_re_div) * s.ch_re_div.d;
}

// Decompose box-relative work index `i` over levels lv[0..L) (lv[0]
// outermost, needing no division) into source/destination offsets added to
// sof/dof (32-bit arithmetic: the relative spans are below 2^31). Returns true
// when any coordinate lies in a pad.
template <int L>
__host__ __device__ __forceinline__ bool decompose(const Level *lv, uint32_t i, int64_t &sof,
                                                   int64_t &dof) {
  bool pad = false;
  uint32_t rem = i, s = 0, d = 0;
#pragma unroll
  for (int k = L - 1; k >= 0; --k) {
    uint32_t u = rem;
    if (k > 0) {
      const uint32_t q = fdiv(rem, lv[k].div);
      u = rem - q * lv[k].div.d;
      rem = q;
    }
    pad |= u - lv[k].vlo >= lv[k].vcnt;
    s += u * lv[k].ss;
    d += u * lv[k].ds;
  }
  sof += s;
  dof += d;
  return pad;
}

// Map a linear block id so that the blocks one XCD runs (ids congruent mod 8)
// take a contiguous run of the tile order.
__host__ __device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t n) {
  constexpr uint32_t kXcd = 8;
  if (n < kXcd)
    return b;
  const uint32_t per = n / kXcd, extra = n % kXcd, x = b % kXcd, j = b / kXcd;
  // XCD x owns tiles [x*per + min(x, extra), ...) of length per + (x < extra)
  return x * per + (x < extra ? x : extra) + j;
}

// Tile t of a transpose launch -> (q-tile, c-tile, batch index). Within a
// batch element's plane of nq x nc tiles, whole groups of g q-tiles come
// first (q fastest, then c), then the partial group of the remaining q-tiles.
// With kTileSkew, q-tile tq takes c-tile (c + tq) mod nc at step c, so the
// blocks in flight, which share c while q runs fastest, write their
// destination rows at different column offsets.
__host__ __device__ __forceinline__ void tile_of(const KArgs &a, uint32_t t, uint32_t &tq,
                                                 uint32_t &tc, uint32_t &batch) {
  batch = fdiv(t, a.t_plane);
  const uint32_t tp = t - batch * a.t_plane.d;
  const uint32_t nc = a.t_nc.d;
  if (tp < a.t_full * nc) {
    const uint32_t grp = fdiv(tp, a.t_group);
    const uint32_t r = tp - grp * a.t_group.d;
    const uint32_t c = fdiv(r, a.t_g);
    tq = grp * a.t_g.d + (r - c * a.t_g.d);
    tc = c;
  } else {
    const uint32_t r = tp - a.t_full * nc;
    const uint32_t c = fdiv(r, a.t_tail);
    tq = a.t_full + (r - c * a.t_tail.d);
    tc = c;
  }
  if (a.t_flags & kTileSkew) {
    const uint32_t x = tc + (tq - fdiv(tq, a.t_nc) * nc); // < 2 nc
    tc = x >= nc ? x - nc : x;
  }
}

} // namespace relx
