// Wavefront-walk SBDA kernels (shared declarations): the fast path for the
// SBDA schedule.  Kernels live in sbda_walk_fwd.hip (forward),
// sbda_walk_bwd.hip (backward: independent, chained and transposed-chain
// walks), sbda_walk_pro.hip (fused norm + RoPE prologue); sbda_walk.hip picks
// the configuration and dispatches.
//
// Layout.  One 64-lane wavefront holds all G = 64/LPR heads of one position
// ("head group"): lane = g * LPR + li, so one 16-byte-per-lane load moves one
// position's rows of the group (1 KiB for 8 heads x 64 dims x bf16).  Each
// wave owns a tile of P consecutive positions and walks it in order.
//
// Sources.  Offsets split into "near" ones (0, 1, 2: a compile-time mask NM)
// and at most one "far" offset F >= 3.  Near sources are the rows the walk
// just loaded, kept in a register rotation (no reload).  Tiles are ordered so
// that the tile holding positions t - F (and t + F) is walked next to this
// one -- linear order for F < P, column order (tile a, a + F, a + 2F, ...)
// otherwise -- and the workgroup id is remapped so consecutive tiles share
// an XCD (and its L2).
//
// Forward: per position, scores against the near rows and the far row
// (loaded directly), softmax, O and one log-normaliser per row.
//
// Backward (gather form, every row written once, no atomics).  Walking
// queries u = a-2 .. end+1, the wave computes each query's weights p_s and
// score gradients dS_s once from its lse; dQ_u is complete at once.  Key
// j = u-2 is then finalised from queries j, j+1, j+2 (near slots, kept in the
// rotation) and its far query i = j + F.  In column order a workgroup of
// waves walks consecutive rows of the column in lockstep and passes rows and
// the far slot's weights through LDS (bwd_chain); otherwise the far query's
// weights are recomputed from q_i, dO_i, lse_i and i's own sources (bwd_pipe).
// Keys are written as soon as they complete.
//
// Addressing.  Row addresses are formed from a wave-uniform row offset and a
// constant per-lane offset (Stream), so the loops carry no per-lane 64-bit
// arithmetic.
//
// Reference semantics: BiAttn/left_v2.py:313-405 (forward maths) and the
// key-centric backward specified by BiAttn/sbda_triton.py:507-671.

#pragma once

#include <type_traits>

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {
namespace walk {

// Pipelined walks (all but the chained backwards): 8-wave workgroups walking consecutive
// tiles in lockstep (one barrier per unrolled iteration), launched with
// 112 KiB of (otherwise unused) LDS so one workgroup runs per CU.  Linear
// tiles are 32 positions, so a workgroup covers 256 consecutive positions
// and the rows in flight across the chip stay within a compact window (~64
// MiB per tensor at T = 2^20 instead of ~512 MiB).  Measured at T = 2^20,
// D = 64, bf16: far-free backward 1.55 -> 1.42 ms, forward 0.86 -> 0.79 ms,
// against 4-wave independent workgroups with 128-position tiles; without
// the barrier or without the LDS cap most of the gain is lost.
constexpr int kPipeWaves = 8;
// Row stride (bytes between positions t and t + F) from which lockstep groups
// hold at most 4 rows of a column.
constexpr int64_t kBigStride = (int64_t)32 << 20;
constexpr int kPipeBlock = kPipeWaves * 64;
constexpr unsigned kPipeLds = 114688;

struct WalkCfg {
  int waves;     // waves per workgroup
  int P;         // positions per tile
  int HG;        // head groups (waves per position)
  int tiles_t;   // tiles per (batch, head group) along T
  int column;    // 1: column order (far offset F is a multiple of P)
  int rows;      // column order: ceil(T / F)
  int rg;        // column order: rows per lockstep group (0: consecutive tiles are rows)
  int bands;     // column order: F / P
  int F;         // far offset (0 if none)
  int nwg;       // workgroups in the grid
  int xs;        // XCD stagger in workgroups (0: none; xcd_stagger)
  int64_t total; // tiles in the grid
};

// Row chains (column order, F a multiple of P): a workgroup of W waves walks
// W consecutive rows of F positions (t = r * F + c) over one column band in
// lockstep, so each wave's far rows are its neighbours' own rows.
struct ChainCfg {
  int P, F, rows, W, bands;
  int L;        // rows per chain; a workgroup holds W / L chains on adjacent bands
  int blocks;   // row blocks (ceil(rows / L)) per band
  int bgroups;  // band groups (ceil(bands / (W / L)))
  int HG, nwg;
  int xs;         // XCD stagger in workgroups (0: none; xcd_stagger)
  int band_fast;  // workgroup order: 1 band groups fastest, 0 row blocks fastest
};

// XCD stagger of a column-order launch (column walks, chains), in workgroups,
// by the far row stride (bytes between positions t and t + F).  Without it
// the eight XCDs walk their ranges in step, each at the same offset of its
// own range.  Measured at T = 2^20 (1 KiB rows, so F = stride / 1 KiB):
//  * rows >= 16 MiB apart (F >= 16384): one eighth of an XCD's range, forwards
//    2-6% and backwards 2-12% faster (-0.6 ms per step, two boxes);
//  * 16 KiB - 1 MiB (F = 16 .. 512) forward and 16 KiB - 4 MiB (F = 16 ..
//    2048) backward: one sixteenth (-0.11 to -0.14 ms per step in A/B runs
//    against the build without it, mostly F = 128 .. 1024; at F = 2048, with
//    the row pairs' band-first order, -14 us);
//  * not at 1-16 MiB forward or 4-16 MiB backward, where every stagger tried
//    (1/32 .. 1/2 of the range) cost up to 6% or did not hold in an A/B run.
constexpr int64_t kStaggerStride = (int64_t)16 << 20;
inline int xcd_stagger(int nwg, int64_t far_stride_bytes, bool fwd) {
  if (nwg <= 0 || nwg % 8 != 0) return 0;
  const int per = nwg / 8;
  const int64_t fs = far_stride_bytes, KiB = 1024, MiB = KiB * KiB;
  if (fs >= kStaggerStride) return per / 8;
  if (fs < 16 * KiB) return 0;
  if (fwd) return fs < MiB ? per / 16 : 0;
  return fs < 4 * MiB ? per / 16 : 0;
}

// Row pairs (the plain backward): a workgroup of 8 waves holds chains of 2
// rows on 4 adjacent bands, row blocks fastest, so a workgroup's waves sit on
// 2 rows of 4 consecutive tiles and the rows beyond the pair (the first
// row's far-left sources, the second row's far queries) are the own rows of
// the workgroups beside it, fetched at about the same time on the same XCD.
// Measured at T = 2^20 against 8-row chains on 128-position tiles: layers
// 9-11 and 15-20 1.49-1.58 -> 1.34-1.47 ms, layer 14 (8 MiB between rows)
// 1.64 -> 1.48 ms.  Not at a row stride of 4 MiB, where pairs of rows collide
// in the DRAM channel mapping (layer 13: 1.54 -> 1.72 ms on one box, no
// better on another); that keeps the 8-row chains.
inline bool chain_pairs_apply(const WalkCfg& wc, int64_t row_stride_bytes) {
  const int64_t fs = (int64_t)wc.F * row_stride_bytes;
  return wc.F >= 128 && wc.rows >= 2 && !(fs >= ((int64_t)4 << 20) && fs < ((int64_t)8 << 20));
}

// Otherwise W = 8 rows (fewer when the sequence has fewer rows), at most 4
// when rows are 32 MiB or more apart: eight lockstep waves on addresses that
// far apart collide in the DRAM channel mapping.  One chain per workgroup
// (L = W).
inline ChainCfg make_chain_cfg(int64_t B, int64_t row_stride_bytes, const WalkCfg& wc,
                               bool pairs = false) {
  ChainCfg c{};
  c.P = wc.P;
  c.F = wc.F;
  c.rows = wc.rows;
  c.W = c.rows >= 8 ? 8 : c.rows >= 4 ? 4 : c.rows >= 2 ? 2 : 1;
  if ((int64_t)wc.F * row_stride_bytes >= kBigStride && c.W > 4) c.W = 4;
  c.L = c.W;
  if (pairs) {
    c.W = kPipeWaves;
    c.L = 2;
  }
  c.bands = wc.F / wc.P;
  c.blocks = (c.rows + c.L - 1) / c.L;
  c.bgroups = (c.bands + c.W / c.L - 1) / (c.W / c.L);
  c.HG = wc.HG;
  const int64_t nwg = B * c.HG * c.bgroups * c.blocks;
  c.nwg = (nwg <= 0 || nwg > 0x7fffffff) ? 0 : (int)nwg;
  return c;
}

// Chained prologue backward (far F >= 16): the keys of a chain's last row
// whose far query lies in the next chain are finished by a second kernel
// from a workspace of deferred slots, one per (batch, head group, row block
// but the last, column): the key's near-slot dK' and dV rows (fp32, 64 / LPR
// heads x D each) and the far query's weight pair per head.  The last row
// block has no next chain, so nothing of it is deferred.
constexpr int kFixCols = 8;   // deferred columns per finishing wave

__host__ __device__ inline int64_t chain_pro_deferring_blocks(const ChainCfg& c) {
  return c.blocks > 1 ? c.blocks - 1 : 0;
}
__host__ __device__ inline int64_t chain_pro_slots(int64_t B, const ChainCfg& c) {
  return B * c.HG * chain_pro_deferring_blocks(c) * c.F;
}
// Slot of (batch, head group, row block rb < blocks - 1, column).
__host__ __device__ inline int64_t chain_pro_slot(const ChainCfg& c, int b, int hg, int rb, int col) {
  return (((int64_t)b * c.HG + hg) * chain_pro_deferring_blocks(c) + rb) * c.F + col;
}
__host__ __device__ inline int64_t chain_pro_slot_floats(int lpr, int D) {
  return 2 * (64 / lpr) * (int64_t)D;
}
__host__ __device__ inline int64_t chain_pro_fix_waves(int64_t B, const ChainCfg& c) {
  return B * c.HG * chain_pro_deferring_blocks(c) * ((c.F + kFixCols - 1) / kFixCols);
}

// Workgroups are dealt to the 8 XCDs round-robin; give each XCD a contiguous
// range of tiles instead.  With a stagger xs > 0 (and a grid that divides
// evenly), XCD x starts its range x * xs workgroups in and wraps around, so
// the eight XCDs' streams are not at the same offset of their ranges at the
// same time (see xcd_stagger).
__device__ inline int64_t xcd_remap(int wg, int nwg, int xs = 0) {
  const int xcd = wg & 7, idx = wg >> 3, per = nwg >> 3, rem = nwg & 7;
  if (xs > 0 && rem == 0) return (int64_t)xcd * per + ((int64_t)idx + (int64_t)xcd * xs) % per;
  return (int64_t)xcd * per + min(xcd, rem) + idx;
}

__device__ inline bool decode_tile(const Params& p, const WalkCfg& c, int64_t n, int& b, int& hg,
                                   int& a) {
  if (n >= c.total) return false;
  hg = (int)(n % c.HG);
  const int64_t rest = n / c.HG;
  const int k = (int)(rest % c.tiles_t);
  b = (int)(rest / c.tiles_t);
  if (c.column && c.rg) {
    // Groups of `waves` tiles: rg rows x (waves / rg) bands.
    const int bg_size = c.waves / c.rg;
    const int rowgroups = (c.rows + c.rg - 1) / c.rg;
    const int g = k / c.waves, w = k % c.waves;
    const int r = (g % rowgroups) * c.rg + w % c.rg;
    const int cb = (g / rowgroups) * bg_size + w / c.rg;
    if (r >= c.rows || cb >= c.bands) return false;
    a = r * c.F + cb * c.P;
  } else if (c.column) {
    const int r = k % c.rows, cb = k / c.rows;
    a = r * c.F + cb * c.P;
  } else {
    a = k * c.P;
  }
  return a < p.T;
}

template <int NM>
struct NearSet {
  static constexpr bool has0 = NM & 1, has1 = NM & 2, has2 = NM & 4;
  static constexpr int count = (int)has0 + (int)has1 + (int)has2;
  // n-th near offset present (0 <= idx < count).
  static constexpr int off(int idx) {
    int seen = 0;
    for (int o = 0; o < 3; ++o)
      if (NM & (1 << o)) {
        if (seen == idx) return o;
        ++seen;
      }
    return -1;
  }
};

// Sums a per-lane weight-gradient partial over the wave's heads and writes
// it as row `wave` of `part` (fixed butterfly order: deterministic).
template <typename T, int LPR, bool SPLIT>
__device__ inline void write_wave_partial(float (&x)[VecOf<T>::value], float* part, int64_t wave,
                                          int D) {
  constexpr int VEC = VecOf<T>::value;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
#pragma unroll
    for (int m = LPR; m < 64; m <<= 1) x[e] += __shfl_xor(x[e], m, 64);
  }
  if (lane < LPR) {
    float* row = part + wave * D;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int d = elem_index<T, SPLIT>(lane, e, D);
      if (SPLIT ? (lane * (VEC / 2) < (D >> 1)) : (lane * VEC < D)) row[d] = x[e];
    }
  }
}

// Walk rows cover the head dimension exactly (LPR lanes x VEC elements = D),
// so the per-wave rows below are complete.  Sums NV per-lane partials (x[0],
// then x[1]) over the wave's heads, then over the workgroup's waves in wave
// order through LDS `red` (NV * waves * D floats, free for reuse), and writes
// row `row` of part[v] -- one row per workgroup instead of one per wave.
// Deterministic; every thread of the workgroup must call it (one barrier,
// plus one before `red` is written when it held other data).
template <typename T, int LPR, int NV>
__device__ inline void write_group_partials(float (&x)[NV][VecOf<T>::value], float* red, int waves,
                                            float* const (&part)[NV], int64_t row, int D) {
  constexpr int VEC = VecOf<T>::value;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
#pragma unroll
      for (int m = LPR; m < 64; m <<= 1) x[v][e] += __shfl_xor(x[v][e], m, 64);
    }
  }
  __syncthreads();
  if (lane < LPR) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) red[(v * waves + w) * D + elem_index<T, true>(lane, e, D)] = x[v][e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NV * D; i += 64 * waves) {
    const int v = i / D, d = i % D;
    float s = 0.f;
    for (int k = 0; k < waves; ++k) s += red[(v * waves + k) * D + d];
    part[v][row * D + d] = s;
  }
}

// ========================================================= pipelined walks
//
// Software-pipelined walks (no prologue): while step u is computed, every
// row step u+1 needs is already in flight.  Loads are
// unconditional (positions clamped into [0, T), validity applied as masks)
// so the compiler can keep them outstanding across steps.  Rows stay in
// their 16-byte raw form; dot products use v_dot2_f32_{bf16,f16} on the raw
// pairs and rows are widened to fp32 only where they are accumulated.
// Rotation depth 4 (positions u+1 .. u-2) with the loop unrolled by 4.

struct Raw {
  uint32_t w[4];
};

// Cache policy.  Results are written with non-temporal stores (nothing
// re-reads them in the kernel).  A row a wave loads for its own position is
// re-read by no other wave when the pattern has no far offset, so those loads
// are non-temporal too; with a far offset the neighbouring wave (column t + F)
// reads the same k/v rows, and they must stay in L2 / the Infinity Cache.
// The forward's q rows are read by their own position only: non-temporal in
// every pattern (far forwards at T = 2^20: 0.42 ms less per 20-layer step).
// The chained backwards load from global memory only the rows no chain
// neighbour holds: a chain's middle waves' rows, and its last wave's q / dO,
// are read by no other wave and are non-temporal (so is every own row of the
// transposed chain), keeping L2 for the rows two chains share (backward at
// T = 2^20, layers 3-20: 25.90 -> 25.52 ms per step, two boxes).  Loads of
// another wave's rows (far-left, far-right) stay cached: non-temporal there
// cost 1.3 ms per step.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ inline void widen(const Raw& r, float (&x)[VecOf<T>::value]) {
  unpack_words<T, 4>(r.w, x);
}

template <typename T>
__device__ inline float dot_raw(const Raw& a, const Raw& b) {
  float s = 0.f;
  if constexpr (std::is_same<T, __bf16>::value) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf2;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w[i]),
                                          __builtin_bit_cast(bf2, b.w[i]), s, false);
  } else if constexpr (std::is_same<T, _Float16>::value) {
    typedef __attribute__((ext_vector_type(2))) _Float16 h2;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.w[i]), __builtin_bit_cast(h2, b.w[i]),
                                 s, false);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_fmaf(__uint_as_float(a.w[i]), __uint_as_float(b.w[i]), s);
  }
  return s;
}

__device__ inline int clampi(int x, int hi) { return x < 0 ? 0 : (x > hi ? hi : x); }

// One tensor as a walking wave sees it: a wave-uniform base (batch and head
// group applied) and row stride in bytes, plus this lane's byte offset inside
// a position (its head within the group and its 16-byte chunk).  A load adds
// the row's 32-bit byte offset (one scalar multiply per row) to the lane
// offset (one full-rate vector add) and uses the scalar-base + 32-bit
// vector-offset addressing form, so no per-lane 64-bit arithmetic is left in
// the loop.  The host only picks these kernels when every offset of a head
// group's span fits in 32 bits (walk_applies).
struct Stream {
  const char* base;
  uint32_t st;
  uint32_t lane;

  __device__ inline uint32_t at(int t) const { return lane + (uint32_t)t * st; }
};

template <typename Vw>
__device__ inline Stream make_stream(const Vw& vw, int esz, int b, int h0, int hl, int li) {
  Stream s;
  s.base = (const char*)vw.p + ((int64_t)b * vw.sb + (int64_t)h0 * vw.sh) * esz;
  s.st = (uint32_t)(vw.st * esz);
  s.lane = (uint32_t)((int64_t)hl * vw.sh * esz) + (uint32_t)li * 16u;
  return s;
}

template <bool NT = false>
__device__ inline Raw load_at(const Stream& s, int t) {
  const u32x4* p = reinterpret_cast<const u32x4*>(s.base + (uint64_t)s.at(t));
  u32x4 x;
  if constexpr (NT) x = __builtin_nontemporal_load(p);
  else x = *p;
  return Raw{{x.x, x.y, x.z, x.w}};
}

template <typename T>
__device__ inline void store_at(const Stream& s, int t, const float (&x)[VecOf<T>::value]) {
  uint32_t w[4];
  pack_words<T, 4>(x, w);
  u32x4 v = {w[0], w[1], w[2], w[3]};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(const_cast<char*>(s.base) + (uint64_t)s.at(t)));
}

// A row load that may be skipped, without a branch: a buffer load whose
// offset lies past the resource's range returns zeros and touches no memory.
// The load stays in the wave's in-order count of outstanding loads, so the
// wait before the next use stays exact (a branch around a load made the
// compiler wait for every load in flight, the next step's prefetch included).
// Every walk span is below kSkipOffset (walk_applies).
constexpr uint32_t kSkipOffset = 0xFFFFFF00u;

template <bool NT = false>
__device__ inline Raw load_at_if(const Stream& s, int t, bool ok) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(s.base), (short)0, kSkipOffset, 0x00020000);
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, ok ? s.at(t) : kSkipOffset, 0, NT ? 2 : 0);
  return Raw{{x.x, x.y, x.z, x.w}};
}

__device__ inline float load_f32_if(const Stream& s, int t, bool ok) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(s.base), (short)0, kSkipOffset, 0x00020000);
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ok ? s.at(t) : kSkipOffset, 0, 0));
}

__device__ inline float load_f32(const Stream& s, int t) {
  return *reinterpret_cast<const float*>(s.base + (uint64_t)s.at(t));
}

__device__ inline void store_f32(const Stream& s, int t, float x) {
  *reinterpret_cast<float*>(const_cast<char*>(s.base) + (uint64_t)s.at(t)) = x;
}

// lse rows: fp32 [B, T, H]; the group's heads are contiguous.
__device__ inline Stream lse_stream(const Params& p, int b, int h0, int hl) {
  Stream s;
  s.base = (const char*)(p.lse + ((int64_t)b * p.T * p.H + h0));
  s.st = (uint32_t)p.H * 4u;
  s.lane = (uint32_t)hl * 4u;
  return s;
}

// Wave-uniform tile decode shared by the pipelined walks.
struct WaveTile {
  int b, hg, a;
  int hl, li;   // this lane's head within the group, 16-byte chunk within the row
};

// Every wave of a lockstep workgroup must run the same number of steps, so a
// wave without a tile (past the last tile or past the end of the sequence)
// walks from a = T: clamped loads, nothing stored.
template <int LPR>
__device__ inline void wave_tile(const Params& p, const WalkCfg& c, WaveTile& w) {
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t n = xcd_remap(blockIdx.x, gridDim.x, c.xs) * c.waves + wv;
  if (!decode_tile(p, c, n, w.b, w.hg, w.a)) {
    w.b = 0;
    w.hg = 0;
    w.a = p.T;
  }
  const int lane = threadIdx.x & 63;
  w.hl = lane / LPR;
  w.li = lane % LPR;
}

struct Pattern {
  int nm;     // near mask over offsets {0, 1, 2}
  int far;    // far offset (0 if none)
};

template <typename T>
struct TypeTag {
  using type = T;
};

// Calls f(TypeTag<T>{}, std::integral_constant<int, LPR>{}) for the row
// element type of `dtype` and `lpr` lanes per row.
template <typename Fn>
hipError_t by_type_lpr(int dtype, int lpr, Fn&& f) {
  auto by_lpr = [&](auto tag) -> hipError_t {
    switch (lpr) {
      case 4: return f(tag, std::integral_constant<int, 4>{});
      case 8: return f(tag, std::integral_constant<int, 8>{});
      case 16: return f(tag, std::integral_constant<int, 16>{});
      default: return hipErrorInvalidValue;
    }
  };
  switch (dtype) {
    case kBF16: return by_lpr(TypeTag<__bf16>{});
    case kFP16: return by_lpr(TypeTag<_Float16>{});
    case kFP32: return by_lpr(TypeTag<float>{});
    default: return hipErrorInvalidValue;
  }
}

// One launcher per translation unit.
hipError_t launch_fwd(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype, int lpr,
                      hipStream_t st);
hipError_t launch_bwd(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype, int lpr,
                      hipStream_t st);
hipError_t launch_fwd_pro(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype,
                          int lpr, hipStream_t st);
hipError_t launch_bwd_pro(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype,
                          int lpr, hipStream_t st);

}  // namespace walk
}  // namespace sbda
