// program.h - the device form of a bound plan: POD launch arguments shared
// by the host planner (program.cpp) and the HIP kernels (kernels.hip).
//
// A DeviceProgram describes, for one wire boundary k, how to turn the dense
// SOURCE-layout wire values at boundary k into the dense RESULT-layout values
// after the last stage: an iteration box over the coalesced destination axes
// (padded coordinates), the source strides of the valid region, the pad fill,
// and the remaining value stages with their per-channel parameters.
//
// Every field a fast kernel reads is addressed with a compile-time index
// (arrays only inside fully unrolled loops of fixed trip count, per-stage and
// per-family scalars precomputed here) and read before any branch: a runtime
// index into the by-value argument block turns a read into a vector-memory
// load, and a read under a branch serialises its scalar load behind the
// branch -- both on the kernel's critical path.
#pragma once

#include <cstdint>

namespace relx {

constexpr int kMaxRank = 8;
constexpr int kMaxStages = 6;
constexpr int kMaxChanTokens = 24;

// Value-stage operations the device runs (docs/reloc-typed-semantics.md).
enum DevOp : uint8_t {
  kOpF32toF16 = 0, // cast ieee_rne
  kOpF16toF32 = 1, // cast exact
  kOpF32toBF16 = 2,
  kOpBF16toF32 = 3,
  kOpQuantize = 4,   // symmetric_rne with inv = fl32(1/scale) formed on the host
  kOpDequantize = 5, // affine: (q - zp) * scale, one rounding
};

// How a stage picks its parameter entry.
enum ChanMode : uint8_t {
  kChanNone = 0, // per tensor: entry 0
  kChanDim = 1,  // the logical result coordinate along one dimension
  kChanExpr = 2, // a channel expression over result coordinates (generic kernel)
};

// Stage sequences with a compile-time kernel body; anything else runs the
// generic per-stage dispatch.
enum ChainCode : int32_t {
  kChainGeneric = 0,
  kChainNone = 1,     // layout only
  kChainF32F16 = 2,   // cast f32 -> f16
  kChainF16F32 = 3,   // cast f16 -> f32
  kChainDeqF16 = 4,   // dequantize -> cast f16 (fused, both roundings kept)
  kChainDeq = 5,      // dequantize
  kChainF16Quant = 6, // cast f16 -> f32 -> quantize
  kChainQuant = 7,    // quantize
};

// Chains whose permute kernel fits eight waves per SIMD (64 VGPRs) without
// spilling registers: the generic per-stage chain and the dequantizing
// chains over one-byte sources do not (they spill hundreds of VGPRs under
// the bound) and run at the occupancy their registers allow.
constexpr bool permute_eight_waves(int win, int ch) {
  return ch != kChainGeneric && !(win == 1 && (ch == kChainDeqF16 || ch == kChainDeq));
}

// The one stage of a compile-time chain that reads parameters (-1: none).
constexpr int chain_param_stage(int ch) {
  return ch == kChainDeqF16 || ch == kChainDeq || ch == kChainQuant ? 0
         : ch == kChainF16Quant                                     ? 1
                                                                    : -1;
}

// Division by a runtime constant for n < 2^32: q = (umulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s, pad_;
};

struct ChanToken {
  int32_t op; // plan opcode; PUSH_SYM is resolved to PUSH_CONST at prepare time
  int32_t pad_;
  int64_t value;
};

struct DevStage {
  uint8_t op;
  uint8_t mode;
  uint8_t zp_per_ch; // zero point has one entry per channel
  uint8_t vec;       // vector kernels: 0 channel constant across a vector, 1 +1 per element
  uint32_t scale_off; // float param index (dequant scale / quant reciprocal)
  uint32_t zp_off;    // int param index
  uint32_t len;       // parameter entries
  // Fast kernels: channel = (o / rs) mod re for a dense result offset o < 2^32;
  // per-tensor stages carry rs = re = 1 (channel 0).
  FastDiv ch_rs_div, ch_re_div;
  // Generic kernel: the same map in 64 bits, or a token range (kChanExpr).
  int64_t ch_rs, ch_re;
  int32_t tok_begin, tok_count;
};

struct Chain {
  int32_t n;
  int32_t ntok;
  DevStage st[kMaxStages];
  ChanToken tok[kMaxChanTokens];
};

enum Family : int32_t {
  kFamGeneric = 0,
  kFamStream = 1,     // innermost axis contiguous on both sides
  kFamTranspose = 2,  // batched 2-D transpose, LDS tiled
  kFamInterleave = 3, // planar -> interleaved with a small padded inner axis
  kFamPermute = 4,    // swap of two axes above a contiguous inner block, through LDS
};

// Pixels per interleave work item: the packed output of an item fills one
// 16-byte vector when a pixel is at most 16 bytes, and each plane is read in
// one access of 4 to 16 bytes.
constexpr int interleave_pixels(int win, int wout, int cp) {
  int g = 16 / (cp * wout);
  if (g < 1)
    g = 1;
  if (g * win < 4)
    g = 4 / win;
  if (g * win > 16)
    g = 16 / win;
  return g;
}

// Transpose tiles are visited in groups of this many q-tiles (destination
// rows), c-tiles within a group: the blocks in flight write long runs of
// few destination rows and read runs of kTileGroup tile rows. One-byte
// sources take tiles 128 q wide (a whole 128-byte line per tile row) when q
// is a multiple of 128, walked q fastest with each q-tile's c-tiles rotated
// by its index; otherwise 64-wide tiles (a tile row is half a line, the
// other half belongs to the next q-tile) walk q fastest with each XCD on a
// contiguous run, so both halves of a line meet in one L2.
#ifndef RELX_TILE_GROUP
#define RELX_TILE_GROUP 16
#endif
constexpr uint32_t kTileGroup = RELX_TILE_GROUP;

// Transpose tile orders and parameter indexing (KArgs::t_flags).
constexpr uint32_t kTileXcd = 1;  // each XCD takes a contiguous run of the order
constexpr uint32_t kTileSkew = 2; // q-tile tq visits its c-tiles rotated by tq (mod nc)
// The parameter stage's channel of every vector is t_choff plus its
// box-relative destination row: the kernel indexes the parameters by row
// (the host proves it for the launch, the verifier for every vector).
constexpr uint32_t kTileRowChannel = 4;
// With kTileRowChannel: every zero point the launch reads is 0 (symmetric
// dequantization), so the kernel leaves the subtraction out.
constexpr uint32_t kTileZeroPoint0 = 8;

// Decomposition levels of the batch axes of the 2-D families.
constexpr int kBatchLevels = 3;
// Work items per launch of a fast kernel, and the source and destination
// element spans its decomposition levels reach, stay below this (32-bit
// indexing); the host splits larger boxes.
constexpr int64_t kMaxLaunchWork = int64_t{1} << 31;

// One level of a fast kernel's index decomposition. A box-relative
// coordinate u in [0, div.d) adds u * ss to the source and u * ds to the
// destination offset (elements, relative to the launch's base offsets: the
// host keeps every launch's relative spans below 2^31); it lies in the valid
// (unpadded) region iff (u - vlo) < vcnt as unsigned 32-bit numbers. Unused
// outer levels have d = 1 and zero strides.
struct Level {
  FastDiv div;
  uint32_t ss, ds;
  uint32_t vlo, vcnt;
};

// Launch arguments (by value). The fast families read only the first block,
// unconditionally at entry, so its scalar loads issue together.
struct KArgs {
  // ---- fast families
  const uint8_t *src; // wire (device) at the program's boundary
  uint8_t *dst;       // result (device)
  const float *pf;    // float parameters
  const int32_t *pi;  // int parameters
  uint32_t work;      // work items of this launch (< 2^31)
  uint32_t fill;      // pad fill bits (fast families move elements of at most 4 bytes)
  int64_t sbase, dbase; // element offsets of the box origin (source: of its valid origin)
  Level lv[kMaxRank];   // stream: box axes (innermost in vectors); 2-D families: batch axes
  // transpose: tiles of t_wq q by t_wc c along the source-inner axis q
  // (destination rows) and the destination-inner axis c, visited in groups
  // of g q-tiles (see tile_of): plane = nq * nc tiles, group = g * nc tiles,
  // g, tail = the q-tiles of the last, partial group, nc = c-tiles
  FastDiv t_plane, t_group, t_g, t_tail, t_nc;
  uint32_t t_full;  // q-tiles in whole groups
  uint32_t t_flags; // kTileXcd | kTileSkew | kTileRowChannel
  // q-tile width (64, or 128 for one-byte sources) and c-tile width (64, or
  // 128 for one-byte sources with wider results: byte tiles), read on
  // the host only; 16 bits each keep the fields the kernels read where they
  // were
  uint16_t t_wq, t_wc;
  uint32_t t_choff; // kTileRowChannel: the parameter channel of tile row 0 of the box
  int64_t t_ssc, t_dsq; // source stride of c, destination stride of q
  // interleave: pixel groups along the source-contiguous axis p; channel axis c
  FastDiv i_ng;
  int64_t i_ssc;        // plane stride (source stride of c)
  int32_t i_loc, i_vc;  // leading pad and valid extent of c
  // permute: destination axes [batch..., c, m, e]; the source holds (m, c, e)
  // contiguously (rows of C*E per m). A block takes T consecutive m of one
  // group of G consecutive c; blocks run group by group (the group is the
  // slowest index: cg = t / p_cgt).
  FastDiv p_tiles;      // m-tiles in the box
  FastDiv p_cgt;        // blocks per group: the box's batch entries x m-tiles
  FastDiv p_ce, p_e;    // C*E and E (source row and inner extents)
  FastDiv p_ge;         // G*E (a block's part of a source row)
  FastDiv p_run;        // 16-byte output vectors per (c, tile) run: T*E*wout/16
  uint32_t p_t, p_lds;  // T, LDS bytes per block (T*G*E*wout)
  uint32_t p_g, p_pad2_; // G
  // direct launches (p_direct): a vector's parameter entry is c & p_cmask
  // (~0: the stage is per channel along c; 0: per tensor)
  uint32_t p_cmask, p_pad_;
  int64_t p_dsc;        // destination stride of c (M*E)
  Chain chain;
  // ---- generic kernel and host bookkeeping (coalesced destination axes)
  int32_t rank;
  int32_t win, wout; // element bytes of the wire and of the result
  int32_t has_fill;
  int32_t chain_code;
  int32_t nlev;      // stream: decomposition levels (1, 2, 4 or 8)
  int32_t cpad;      // interleave: padded inner extent
  int32_t vec;       // stream: elements per vector; interleave: pixels per thread
  int32_t res_rank;
  int32_t edge_box;  // 1: a box of a fast-family program at its unaligned edge,
                     // run by the generic kernel
  int32_t p_direct;  // permute: G*E, E and the run are powers of two, one
                     // batch level, and the parameter stage's channel is c
                     // or 0 (permute_direct)
  int64_t work64;    // generic: elements of the box
  uint64_t fill64;
  int64_t pext[kMaxRank]; // padded extents
  int64_t lo[kMaxRank];   // leading pad per axis
  int64_t vext[kMaxRank]; // valid extents
  int64_t ss[kMaxRank];   // source strides (valid coordinates)
  int64_t ds[kMaxRank];   // destination strides (padded coordinates)
  int64_t box_lo[kMaxRank];
  int64_t box_ext[kMaxRank];
  int64_t rs[kMaxRank]; // result strides and extents (channel expressions)
  int64_t re[kMaxRank];
};

// Arguments of a direct permute launch (KArgs::p_direct): only the fields its
// blocks read, 34 dwords that a block fetches in one round of scalar loads.
// (Built from KArgs, 2,024 bytes, whose fields the general kernel reads from
// its first 656 in three dependent rounds, spilling scalar registers, before
// its first data load; with blocks of 4-8 KiB of source that start costs C5
// [8,4096,32,128] 20%.) The
// launch's batch entries lie along one level: entry b starts b * bss source
// and b * bds result elements past the launch origin.
struct PermArgs {
  const uint8_t *src;
  uint8_t *dst;
  const float *pf;
  const int32_t *pi;
  int64_t sbase, dbase;               // element offsets of the launch origin
  int64_t dsc;                        // result stride of c (M*E)
  uint32_t work;                      // blocks
  uint32_t cgt_d, cgt_m, cgt_s;       // blocks per channel group (FastDiv)
  uint32_t tiles_d, tiles_m, tiles_s; // m-tiles per batch entry (FastDiv)
  uint32_t t, g;                      // rows and channels per block
  uint32_t ge_s, e_s, run_s;          // log2 of G*E, E and a run's 16-byte vectors
  uint32_t ce;                        // C*E, a source row
  uint32_t bss, bds;                  // element strides of a batch entry
  uint32_t nout;                      // 16-byte vectors a block stores
  uint32_t cmask;                     // a vector's parameter entry: c & cmask
  uint32_t scale_off, zp_off, zp_per_ch;
};

// Row gather of an indexed plan (index_select along axis 0, at most one cast):
// a launch covers `work` vector items of consecutive selected rows, each row
// `row_items` items; item i belongs to selected row r = i / row_items and
// reads item i - r * row_items of table row idx[r]. The host splits launches
// so that `work` < 2^31 and offsets `dst` and `idx` to the launch's first row.
enum GatherOp : int32_t {
  kGatherCopy = 0,   // same element type (bit copy)
  kGatherF32F16 = 1, // cast f32 -> f16, ieee_rne
  kGatherF16F32 = 2, // cast f16 -> f32, exact
};

struct GatherArgs {
  const uint8_t *table;
  uint8_t *dst;
  const void *idx; // int32 or int64 row indices
  uint32_t work;
  uint32_t row_items;
  FastDiv per_row; // division by row_items
};

} // namespace relx
