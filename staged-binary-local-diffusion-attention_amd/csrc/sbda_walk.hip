// Walk-kernel dispatch: which patterns the walks take, the tile / workgroup
// configuration of each launch, and the entry points the C ABI calls.

#include "sbda_walk.h"

namespace sbda {
namespace walk {
namespace {


// Classifies offsets: each distinct, at most one offset >= 3.
bool classify(const Params& p, Pattern* out) {
  int nm = 0, far = 0, nfar = 0;
  for (int s = 0; s < p.S; ++s) {
    const int o = p.off[s];
    for (int r = 0; r < s; ++r)
      if (p.off[r] == o) return false;
    if (o <= 2) {
      nm |= 1 << o;
    } else {
      far = o;
      ++nfar;
    }
  }
  if (nfar > 1) return false;
  // Supported patterns: (0,1), (0,2), (0,1,2,F), (0,F).
  const bool ok = (nfar == 0 && (nm == 3 || nm == 5)) || (nfar == 1 && (nm == 7 || nm == 1));
  if (!ok) return false;
  out->nm = nm;
  out->far = far;
  return true;
}

int walk_lpr(const Params& p, int dtype) {
  const int esz = dtype == kFP32 ? 4 : 2;
  if ((p.D * esz) % 16) return 0;
  const int lpr = p.D * esz / 16;
  if (lpr != 4 && lpr != 8 && lpr != 16) return 0;
  return lpr;
}

// Tile order shared by both configurations: column order when the far offset
// is a multiple of the tile, linear otherwise.
void order_tiles(const Params& p, const Pattern& pat, int64_t lanes_rows, WalkCfg& c) {
  c.F = pat.far;
  if (pat.far >= c.P && pat.far % c.P == 0) {
    c.column = 1;
    c.rows = (p.T + pat.far - 1) / pat.far;
    c.bands = pat.far / c.P;
    if (c.rg) {
      const int bg_size = c.waves / c.rg;
      c.tiles_t = ((c.rows + c.rg - 1) / c.rg) * c.rg *
                  ((c.bands + bg_size - 1) / bg_size) * bg_size;
    } else {
      c.tiles_t = c.rows * c.bands;
    }
  } else {
    c.column = 0;
    c.rows = 0;
    c.tiles_t = (p.T + c.P - 1) / c.P;
  }
  c.total = lanes_rows * c.tiles_t;
  c.nwg = (int)((c.total + c.waves - 1) / c.waves);
}

// Pipelined walks and the chained backward: lin_tile-position tiles in
// linear order, or min(max_col_tile, F) for a power-of-two far offset F >= 16
// (column order, far rows one column row away); halved (not below min_tile)
// while the grid has fewer than 256 full workgroups.
WalkCfg make_pipe_cfg(const Params& p, int lpr, const Pattern& pat, int max_col_tile,
                      int lin_tile = 32, int min_tile = 16) {
  WalkCfg c{};
  c.waves = kPipeWaves;
  c.HG = p.H / (64 / lpr);
  const int64_t lanes_rows = (int64_t)p.B * c.HG;
  const bool pow2far = pat.far >= 16 && (pat.far & (pat.far - 1)) == 0;
  int P = pow2far ? min(max_col_tile, pat.far) : lin_tile;
  while (P > min_tile && lanes_rows * ((p.T + P - 1) / P) < 256 * kPipeWaves) P >>= 1;
  c.P = P;
  order_tiles(p, pat, lanes_rows, c);
  return c;
}

int64_t far_stride_bytes(const Params& p, const Pattern& pat, int dtype) {
  return (int64_t)pat.far * p.q.st * (dtype == kFP32 ? 4 : 2);
}

// The configuration a walk launch uses (also sizes the prologue backward's
// norm-weight partials).  Lockstep waves on rows F positions apart: at a row
// stride of 32 MiB and more, eight of them at once collide in the DRAM channel
// mapping (the forward at T = 2^20 lost up to 30% at F = 2^16, 2^17), so a
// workgroup then takes 4 rows x 2 bands.  The chained backward has its own
// limit (launch_chain).
WalkCfg launch_cfg(const Params& p, int dtype, const Pattern& pat, int lpr, bool fwd, bool pro) {
  if (fwd && !pro && pat.far >= 128) {
    // The forward needs no row chain: 64-position tiles in groups of 2 rows
    // x 4 bands keep each workgroup's rows within two 256 KiB windows.
    // Measured at T = 2^20 over layers 8-20: 16.8 ms of forwards against
    // 17.3 ms with 8 rows x 128 positions per workgroup.
    // (Fewer than 4 bands: more rows per group, so no wave is left idle.)
    // Rows 4 MiB apart are the exception: pairs of 64-position rows that far
    // apart collide in the DRAM channel mapping, 8 rows x 1 band do not
    // (layer 13 at T = 2^20: 1.01 -> 0.89 ms, two boxes).  At 8 and 16 MiB, with
    // at least 4 rows, pairs of 32-position tiles (2 rows x 4 bands of 32)
    // measured faster than 64 (layers 14-15: 0.75-0.78 against 0.77-0.79 ms);
    // from 32 MiB up, with the XCD stagger, 64 is faster again (layers 16-19:
    // 0.73-0.75 against 0.75-0.76 ms, two repetitions).  With 2 rows (layer
    // 20) 64 was faster already (0.74 against 0.80 ms).
    // At F = 128, 64-position tiles leave 2 bands (a group of 4 rows x 2
    // bands); 32-position tiles keep the 2-row groups (layer 8: 0.787 against
    // 0.801 ms in the sweep below).
    const int64_t fs = far_stride_bytes(p, pat, dtype);
    const int64_t rows = (p.T + pat.far - 1) / pat.far;
    const bool narrow =
        (fs >= ((int64_t)8 << 20) && fs < kBigStride && rows >= 4) || pat.far < 4 * 64;
    WalkCfg c = make_pipe_cfg(p, lpr, pat, narrow ? 32 : 64);
    if (c.column && c.rows >= 2) {
      int rg = (fs >= ((int64_t)4 << 20) && fs < ((int64_t)8 << 20)) ? 8 : 2;
      while (rg < kPipeWaves && rg * c.bands < kPipeWaves) rg <<= 1;
      c.rg = rg;
      order_tiles(p, pat, (int64_t)p.B * c.HG, c);
    }
    if (c.column) c.xs = xcd_stagger(c.nwg, fs, true);
    return c;
  }
  // The far-free forward takes 64-position tiles: its tiles load the 2 rows
  // before them once more (the neighbouring tile's last rows, long gone from
  // L2 when they are needed), and halving that share measured 0.73-0.75 ms
  // against 0.77-0.80 ms per layer at T = 2^20 (outputs bitwise identical).
  // Not the backward (4 halo rows; 64-position tiles measured 2-7% slower)
  // nor the forward with far offsets 4 and 8 (6-7% slower).
  const int lin = (fwd && !pro && pat.far == 0) ? 64 : 32;
  // The plain backward's row-pair chains take 64-position tiles (32 at F =
  // 128, so a workgroup still finds 4 bands); 32- and 128-position tiles
  // measured slower at F >= 256.
  int col_tile = 128;
  if (!fwd && !pro && pat.far >= 128) {
    WalkCfg probe = make_pipe_cfg(p, lpr, pat, 64, lin);
    if (probe.column && walk::chain_pairs_apply(probe, far_stride_bytes(p, pat, dtype) / pat.far))
      col_tile = pat.far >= 256 ? 64 : 32;
  }
  // The rotation backward at F = 4 keeps 32-position tiles (its trip layout).
  const int min_tile = (!fwd && !pro && pat.far == 4) ? 32 : 16;
  WalkCfg c = make_pipe_cfg(p, lpr, pat, col_tile, lin, min_tile);
  if ((fwd || pro) && c.column && c.rows > 4 && far_stride_bytes(p, pat, dtype) >= kBigStride) {
    c.rg = 4;
    order_tiles(p, pat, (int64_t)p.B * c.HG, c);
  }
  // The prologue walks keep the plain XCD order (the stagger was measured on
  // the plain walks only), and so do the linear layouts.
  if (!pro && c.column) c.xs = xcd_stagger(c.nwg, far_stride_bytes(p, pat, dtype), fwd);
  return c;
}

template <bool FWD>
hipError_t walk_launch(const Params& p, int dtype, bool pro, hipStream_t st) {
  Pattern pat;
  if (!classify(p, &pat)) return hipErrorInvalidValue;
  const int lpr = walk_lpr(p, dtype);
  const WalkCfg c = launch_cfg(p, dtype, pat, lpr, FWD, pro);
  if (FWD) return pro ? launch_fwd_pro(p, c, pat, dtype, lpr, st) : launch_fwd(p, c, pat, dtype, lpr, st);
  return pro ? launch_bwd_pro(p, c, pat, dtype, lpr, st) : launch_bwd(p, c, pat, dtype, lpr, st);
}

}  // namespace
}  // namespace walk

using walk::Pattern;
using walk::WalkCfg;
using walk::classify;
using walk::walk_lpr;
using walk::launch_cfg;
using walk::walk_launch;

// Every byte offset a wave forms from its head group's base (row offset plus
// lane offset) must fit the 32-bit vector offset of the load/store form.
template <typename Vw>
bool span_fits_32(const Vw& vw, const Params& p, int esz, int lpr) {
  if (vw.p == nullptr) return true;
  if (vw.st < 0 || vw.sh < 0) return false;
  const int64_t span =
      ((int64_t)(p.T - 1) * vw.st + (int64_t)(64 / lpr - 1) * vw.sh) * esz + 16 * lpr;
  return span <= (int64_t)walk::kSkipOffset;
}

bool walk_applies(const Params& p, int dtype) {
  Pattern pat;
  if (p.group != 1 || p.seg != nullptr || !classify(p, &pat)) return false;
  const int lpr = walk_lpr(p, dtype);
  if (lpr == 0) return false;
  if (p.H % (64 / lpr) != 0) return false;
  const int esz = dtype == kFP32 ? 4 : 2;
  if ((int64_t)p.T * p.H * 4 > (int64_t)0xffffffffLL) return false;
  return span_fits_32(p.q, p, esz, lpr) && span_fits_32(p.k, p, esz, lpr) &&
         span_fits_32(p.v, p, esz, lpr) && span_fits_32(p.dout, p, esz, lpr) &&
         span_fits_32(p.o, p, esz, lpr) && span_fits_32(p.dq, p, esz, lpr) &&
         span_fits_32(p.dk, p, esz, lpr) && span_fits_32(p.dv, p, esz, lpr);
}

hipError_t walk_forward(const Params& p, int dtype, bool pro, hipStream_t st) {
  return walk_launch<true>(p, dtype, pro, st);
}

hipError_t walk_backward(const Params& p, int dtype, bool pro, hipStream_t st) {
  return walk_launch<false>(p, dtype, pro, st);
}

void walk_partials(const Params& p, int dtype, int64_t* pq, int64_t* pk, int64_t* tab_floats) {
  Pattern pat;
  classify(p, &pat);
  const WalkCfg c = launch_cfg(p, dtype, pat, walk_lpr(p, dtype), false, true);
  if (pat.far == 0) {   // fused single-pass backward: no weight table
    *pq = *pk = (int64_t)c.nwg * c.waves;
    *tab_floats = 0;
    return;
  }
  if (c.column) {   // chained backward + finishing kernel (sbda_walk_pro.hip)
    // The chain height depends on the row stride, which the size query does
    // not see: with strides (a launch) the sizes of that chain height, without
    // (a query, p.q.st == 0) the larger of the two heights' sizes.
    const int lpr = walk_lpr(p, dtype);
    const int esz = dtype == kFP32 ? 4 : 2;
    *pq = *pk = *tab_floats = 0;
    for (int k = 0; k < 2; ++k) {
      const int64_t stride = p.q.st > 0 ? p.q.st * (int64_t)esz : (k ? walk::kBigStride : 0);
      const walk::ChainCfg cc = walk::make_chain_cfg(p.B, stride, c);
      // One partial row per workgroup of either kernel.
      const int64_t q_ = cc.nwg;
      const int64_t k_ = q_ + (walk::chain_pro_fix_waves(p.B, cc) + 3) / 4;
      const int64_t t_ = walk::chain_pro_slots(p.B, cc) *
                         (walk::chain_pro_slot_floats(lpr, p.D) + 2 * (64 / lpr));
      *pq = std::max(*pq, q_);
      *pk = std::max(*pk, k_);
      *tab_floats = std::max(*tab_floats, t_);
      if (p.q.st > 0) break;
    }
    return;
  }
  *pq = (int64_t)c.nwg * c.waves;
  *pk = *pq;
  *tab_floats = (int64_t)p.B * p.T * p.H * 2 * p.S;
}

}  // namespace sbda
