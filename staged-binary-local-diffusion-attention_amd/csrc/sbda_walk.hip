// Wavefront-walk SBDA kernels: the fast path for the SBDA schedule.
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

#include <type_traits>

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {

namespace {

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
  int64_t total; // tiles in the grid
};

// Workgroups are dealt to the 8 XCDs round-robin; give each XCD a contiguous
// range of tiles instead.
__device__ inline int64_t xcd_remap(int wg, int nwg) {
  const int xcd = wg & 7, idx = wg >> 3, per = nwg >> 3, rem = nwg & 7;
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
// reads the same rows, and they must stay in L2 / the Infinity Cache.
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
  const int64_t n = xcd_remap(blockIdx.x, gridDim.x) * c.waves + wv;
  if (!decode_tile(p, c, n, w.b, w.hg, w.a)) {
    w.b = 0;
    w.hg = 0;
    w.a = p.T;
  }
  const int lane = threadIdx.x & 63;
  w.hl = lane / LPR;
  w.li = lane % LPR;
}

// FR > 0: the far offset is the compile-time constant FR (4 or 8) and the far
// row is taken from the rotation (depth FR + 2) instead of being loaded: a
// row loaded FR steps earlier is long gone from L2 at the streaming rate.
template <typename T, int LPR, int NM, bool FAR, int FR>
struct FwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);
  static constexpr int RD = FR > 0 ? FR + 2 : 4;   // rotation depth (even)
  static_assert(FR == 0 || FAR, "a rotation far source needs a far slot");

  Stream q, k, v, o, lse;
  float scale;
  int F, Tm1, li;
  Raw kr[RD];           // k at t (slot R), t-1, ...; slot R+1 is being fetched
  Raw vraw[2], qn[2];   // this step's v and q (stage R & 1)
  Raw kl[2], vl[2];     // far source t - F (FR == 0)
  float vr[RD][VEC];    // widened v rotation

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, Tm1);
    kr[R] = load_at<!FAR>(k, tc);
    vraw[R & 1] = load_at<!FAR>(v, tc);
    qn[R & 1] = load_at<!FAR>(q, tc);
    if constexpr (FAR && FR == 0) {
      const int tf = clampi(t - F, Tm1);
      kl[R & 1] = load_at(k, tf);
      vl[R & 1] = load_at(v, tf);
    }
  }

  template <int R>
  __device__ inline void compute(int t, bool store) {
    widen<T>(vraw[R & 1], vr[R]);
    float sc[NS];
    bool ok[NS];
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        ok[idx] = t - n >= 0;
        sc[idx] = row_sum<LPR>(dot_raw<T>(qn[R & 1], kr[(R + RD - n) % RD])) * scale;
        ++idx;
      }
    }
    float vf[VEC];
    if constexpr (FAR) {
      ok[NS - 1] = t - F >= 0;
      if constexpr (FR > 0) {
        constexpr int sf = (R + RD - FR) % RD;
        sc[NS - 1] = row_sum<LPR>(dot_raw<T>(qn[R & 1], kr[sf])) * scale;
#pragma unroll
        for (int e = 0; e < VEC; ++e) vf[e] = vr[sf][e];
      } else {
        sc[NS - 1] = row_sum<LPR>(dot_raw<T>(qn[R & 1], kl[R & 1])) * scale;
        widen<T>(vl[R & 1], vf);
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; ++s) m = ok[s] ? fmaxf(m, sc[s]) : m;
    float w[NS], l = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      w[s] = ok[s] ? fast_exp(sc[s] - m) : 0.f;
      l += w[s];
    }
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        const int slot = (R + RD - n) % RD;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[idx], vr[slot][e], acc[e]);
        ++idx;
      }
    }
    if constexpr (FAR) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[NS - 1], vf[e], acc[e]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= inv;
    if (store) {
      store_at<T>(o, t, acc);
      if (li == 0) store_f32(lse, t, l > 0.f ? m + fast_log(l) : INFINITY);
    }
  }

  // Steps R .. RD-1 of one trip around the rotation (position of slot 0 is t).
  template <int R>
  __device__ inline void steps(int t, int a, int end) {
    if constexpr (R < RD) {
      prefetch<(R + 1) % RD>(t + R + 1);
      compute<R>(t + R, t + R >= a && t + R < end);
      steps<R + 1>(t, a, end);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR, int FR>
__global__ __launch_bounds__(kPipeBlock) void fwd_pipe(Params p, WalkCfg c) {
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int G = 64 / LPR, esz = (int)sizeof(T);
  const int h0 = wt.hg * G;
  using W = FwdPipe<T, LPR, NM, FAR, FR>;
  W w;
  w.q = make_stream(p.q, esz, wt.b, h0, wt.hl, wt.li);
  w.k = make_stream(p.k, esz, wt.b, h0, wt.hl, wt.li);
  w.v = make_stream(p.v, esz, wt.b, h0, wt.hl, wt.li);
  w.o = make_stream(p.o, esz, wt.b, h0, wt.hl, wt.li);
  w.lse = lse_stream(p, wt.b, h0, wt.hl);
  w.scale = p.scale;
  w.F = c.F;
  w.Tm1 = p.T - 1;
  w.li = wt.li;
  const int a = wt.a, end = min(a + c.P, p.T);
  // The walk starts early enough to fill the rotation (2 positions, or FR
  // for a rotation far source); those steps store nothing.  Slot of
  // position t is (t - t0) % RD.
  // The trip count depends only on P (same for every wave of the workgroup).
  const int t0 = a - (FR > 2 ? FR : 2);
  w.template prefetch<0>(t0);
  for (int t = t0; t < a + c.P; t += W::RD) {
    __syncthreads();
    w.template steps<0>(t, a, end);
  }
}

template <typename T, int LPR, int NM, bool FAR>
struct BwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  Stream q, k, v, go, dq, dk, dv, lse;
  float scale;
  int F, T_, Tm1, a, end;
  Raw kr[4], vr[4];     // own k/v rotation: slot of u is R
  Raw qr[4], gr[4];     // own q/dO rotation (key finalisation reads u-2 .. u)
  float lr[4];
  Raw fk[4], fv[4];     // far-right k/v rotation over i = u - 2 + F
  Raw kl[2], vl[2];     // far-left sources of query u
  Raw qi[2], gi[2];     // far query i of key u - 2
  float li_[2];
  float sp[4][3], sd[4][3];  // query u's near-slot p_n and scale * dS_n

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, Tm1);
    kr[R] = load_at<!FAR>(k, uc);
    vr[R] = load_at<!FAR>(v, uc);
    qr[R] = load_at<!FAR>(q, uc);
    gr[R] = load_at<!FAR>(go, uc);
    lr[R] = load_f32(lse, uc);
    if constexpr (FAR) {
      const int ul = clampi(u - F, Tm1);
      kl[R & 1] = load_at(k, ul);
      vl[R & 1] = load_at(v, ul);
      const int i = clampi(u - 2 + F, Tm1);
      fk[R] = load_at(k, i);
      fv[R] = load_at(v, i);
      qi[R & 1] = load_at(q, i);
      gi[R & 1] = load_at(go, i);
      li_[R & 1] = load_f32(lse, i);
    }
  }

  // p and dS of one query from its raw operands and sources.
  __device__ inline void grads(const Raw& qq, const Raw& gg, float l, const Raw* const (&ks)[NS],
                               const Raw* const (&vs)[NS], const bool (&ok)[NS], float (&pp)[NS],
                               float (&ds)[NS]) const {
    float dp[NS];
    float delta = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float sc = row_sum<LPR>(dot_raw<T>(qq, *ks[s])) * scale;
      dp[s] = row_sum<LPR>(dot_raw<T>(gg, *vs[s]));
      pp[s] = ok[s] ? fast_exp(sc - l) : 0.f;
      delta = __builtin_fmaf(pp[s], dp[s], delta);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) ds[s] = pp[s] * (dp[s] - delta);
  }

  template <int R>
  __device__ inline void compute(int u) {
    // Own query u (its operands are clamped rows outside [0, T); the results
    // are only used for queries inside the tile's range).
    {
      const Raw* ks[NS];
      const Raw* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          ks[idx] = &kr[(R + 4 - n) & 3];
          vs[idx] = &vr[(R + 4 - n) & 3];
          ok[idx] = u - n >= 0;
          ++idx;
        }
      }
      if constexpr (FAR) {
        ks[NS - 1] = &kl[R & 1];
        vs[NS - 1] = &vl[R & 1];
        ok[NS - 1] = u - F >= 0;
      }
      float pp[NS], ds[NS];
      grads(qr[R], gr[R], lr[R], ks, vs, ok, pp, ds);
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        sp[R][n] = pp[n];
        sd[R][n] = ds[n] * scale;
      }
      if (u >= a && u < end) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          float kx[VEC];
          widen<T>(*ks[s], kx);
          const float c = ds[s] * scale;
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(c, kx[e], g[e]);
        }
        store_at<T>(dq, u, g);
      }
    }
    // Key j = u - 2: near contributions from queries j + n, far from j + F.
    const int j = u - 2;
    if (j >= a && j < end) {
      float ak[VEC], av[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) { ak[e] = 0.f; av[e] = 0.f; }
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + 2 + n) & 3;   // slot of query j + n
          const bool there = j + n < T_;
          const float cs = there ? sd[slot][idx] : 0.f;
          const float cp = there ? sp[slot][idx] : 0.f;
          float qx[VEC], gx[VEC];
          widen<T>(qr[slot], qx);
          widen<T>(gr[slot], gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
            av[e] = __builtin_fmaf(cp, gx[e], av[e]);
          }
          ++idx;
        }
      }
      if constexpr (FAR) {
        const Raw* ks[NS];
        const Raw* vs[NS];
        bool ok[NS];
        int n2 = 0;
#pragma unroll
        for (int n = 0; n < 3; ++n) {
          if (NM & (1 << n)) {
            ks[n2] = &fk[(R + 4 - n) & 3];
            vs[n2] = &fv[(R + 4 - n) & 3];
            ok[n2] = true;   // i - n >= F - 2 > 0
            ++n2;
          }
        }
        ks[NS - 1] = &kr[(R + 2) & 3];   // key j itself
        vs[NS - 1] = &vr[(R + 2) & 3];
        ok[NS - 1] = true;
        float pp[NS], ds[NS];
        grads(qi[R & 1], gi[R & 1], li_[R & 1], ks, vs, ok, pp, ds);
        const bool there = j + F < T_;
        const float cs = there ? ds[NS - 1] * scale : 0.f;
        const float cp = there ? pp[NS - 1] : 0.f;
        float qx[VEC], gx[VEC];
        widen<T>(qi[R & 1], qx);
        widen<T>(gi[R & 1], gx);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
          av[e] = __builtin_fmaf(cp, gx[e], av[e]);
        }
      }
      store_at<T>(dk, j, ak);
      store_at<T>(dv, j, av);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kPipeBlock) void bwd_pipe(Params p, WalkCfg c) {
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int G = 64 / LPR, esz = (int)sizeof(T);
  const int h0 = wt.hg * G;
  BwdPipe<T, LPR, NM, FAR> w;
  w.q = make_stream(p.q, esz, wt.b, h0, wt.hl, wt.li);
  w.k = make_stream(p.k, esz, wt.b, h0, wt.hl, wt.li);
  w.v = make_stream(p.v, esz, wt.b, h0, wt.hl, wt.li);
  w.go = make_stream(p.dout, esz, wt.b, h0, wt.hl, wt.li);
  w.dq = make_stream(p.dq, esz, wt.b, h0, wt.hl, wt.li);
  w.dk = make_stream(p.dk, esz, wt.b, h0, wt.hl, wt.li);
  w.dv = make_stream(p.dv, esz, wt.b, h0, wt.hl, wt.li);
  w.lse = lse_stream(p, wt.b, h0, wt.hl);
  w.scale = p.scale;
  w.F = c.F;
  w.T_ = p.T;
  w.Tm1 = p.T - 1;
  w.a = wt.a;
  w.end = min(wt.a + c.P, p.T);
  // Walk u = a-2 .. a+P+1 (slot of u is (u - a + 2) & 3); the trip count
  // depends only on P, the same for every wave of the workgroup.
  const int u0 = wt.a - 2, last = wt.a + c.P + 1;
  w.template prefetch<0>(u0);
  for (int u = u0; u <= last; u += 4) {
    __syncthreads();
    w.template prefetch<1>(u + 1);
    w.template compute<0>(u);
    w.template prefetch<2>(u + 2);
    w.template compute<1>(u + 1);
    w.template prefetch<3>(u + 3);
    w.template compute<2>(u + 2);
    w.template prefetch<0>(u + 4);
    w.template compute<3>(u + 3);
  }
}

// ============================================== chained backward (far >= tile)
//
// With the far offset F a multiple of the tile P, the tiles of one band form
// a column t, t + F, t + 2F, ...: the far-left sources of row r + 1 are row
// r's own k/v rows, and the far query of row r's key j is row r + 1's query
// j + F.  Independent waves re-read those rows from L2 a few steps after
// their owner loaded them, and at the streaming rate of a whole XCD most of
// them have been evicted by then.  Here a workgroup of W waves walks W
// consecutive rows of one band in lockstep (one barrier per step) and passes
// the rows through LDS instead: wave w publishes its k/v (for wave w + 1's
// far-left slot) and its q/dO plus the far slot's (p, scale dS) (for wave
// w - 1's far key contribution).  Only the first wave loads far-left rows
// and only the last wave recomputes its far queries from global memory.
//
// Every wave of the workgroup runs the same number of steps (tiles past the
// end of the sequence walk clamped rows and store nothing), so all barriers
// are reached by all waves.

constexpr int kChainRing = 4;   // q/dO/weight ring: written at step u, read at u + 2

struct ChainSlot {
  u32x4 kv[2][2][64];             // [u & 1][k, v][lane]
  u32x4 qd[kChainRing][2][64];    // [u & 3][q, dO][lane]
  float2 pd[kChainRing][64];      // [u & 3][lane]: (p_far, scale * dS_far) of query u
};

struct ChainCfg {
  int P, F, rows, W, bands;
  int L;        // rows per chain; a workgroup holds W / L chains on adjacent bands
  int blocks;   // row blocks (ceil(rows / L)) per band
  int bgroups;  // band groups (ceil(bands / (W / L)))
  int HG, nwg;
};

template <typename T, int LPR, int NM, bool LEFT_LDS, bool RIGHT_LDS>
struct BwdChain {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + 1;

  Stream q, k, v, go, dq, dk, dv, lse;
  float scale;
  int F, T_, Tm1, a, end, lane;
  ChainSlot* mine;
  const ChainSlot* up;     // wave w - 1 (far-left provider)
  const ChainSlot* down;   // wave w + 1 (far-right provider)
  Raw kr[4], vr[4], qr[4], gr[4];
  float lr[4];
  Raw fk[4], fv[4];        // far-right k/v rotation over i = u - 2 + F (last wave)
  Raw kl[2], vl[2];        // far-left sources of query u (first wave)
  Raw qi[2], gi[2];
  float li_[2];
  float sp[4][3], sd[4][3];

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, Tm1);
    kr[R] = load_at(k, uc);
    vr[R] = load_at(v, uc);
    qr[R] = load_at(q, uc);
    gr[R] = load_at(go, uc);
    lr[R] = load_f32(lse, uc);
    if constexpr (!LEFT_LDS) {
      const int ul = clampi(u - F, Tm1);
      kl[R & 1] = load_at(k, ul);
      vl[R & 1] = load_at(v, ul);
    }
    if constexpr (!RIGHT_LDS) {
      const int i = clampi(u - 2 + F, Tm1);
      fk[R] = load_at(k, i);
      fv[R] = load_at(v, i);
      qi[R & 1] = load_at(q, i);
      gi[R & 1] = load_at(go, i);
      li_[R & 1] = load_f32(lse, i);
    }
  }

  __device__ static inline u32x4 pack(const Raw& r) { return u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}; }
  __device__ static inline Raw unpack(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

  __device__ inline void grads(const Raw& qq, const Raw& gg, float l, const Raw* const (&ks)[NS],
                               const Raw* const (&vs)[NS], const bool (&ok)[NS], float (&pp)[NS],
                               float (&ds)[NS]) const {
    float dp[NS];
    float delta = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float sc = row_sum<LPR>(dot_raw<T>(qq, *ks[s])) * scale;
      dp[s] = row_sum<LPR>(dot_raw<T>(gg, *vs[s]));
      pp[s] = ok[s] ? fast_exp(sc - l) : 0.f;
      delta = __builtin_fmaf(pp[s], dp[s], delta);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) ds[s] = pp[s] * (dp[s] - delta);
  }

  template <int R>
  __device__ inline void compute(int u) {
    // Publish this step's rows, then wait for the neighbours' rows.
    mine->kv[R & 1][0][lane] = pack(kr[R]);
    mine->kv[R & 1][1][lane] = pack(vr[R]);
    mine->qd[R][0][lane] = pack(qr[R]);
    mine->qd[R][1][lane] = pack(gr[R]);
    __syncthreads();
    Raw kf, vf;
    if constexpr (LEFT_LDS) {
      kf = unpack(up->kv[R & 1][0][lane]);
      vf = unpack(up->kv[R & 1][1][lane]);
    } else {
      kf = kl[R & 1];
      vf = vl[R & 1];
    }
    {
      const Raw* ks[NS];
      const Raw* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          ks[idx] = &kr[(R + 4 - n) & 3];
          vs[idx] = &vr[(R + 4 - n) & 3];
          ok[idx] = u - n >= 0;
          ++idx;
        }
      }
      ks[NS - 1] = &kf;
      vs[NS - 1] = &vf;
      ok[NS - 1] = u - F >= 0;
      float pp[NS], ds[NS];
      grads(qr[R], gr[R], lr[R], ks, vs, ok, pp, ds);
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        sp[R][n] = pp[n];
        sd[R][n] = ds[n] * scale;
      }
      mine->pd[R][lane] = make_float2(pp[NS - 1], ds[NS - 1] * scale);
      if (u >= a && u < end) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          float kx[VEC];
          widen<T>(*ks[s], kx);
          const float c = ds[s] * scale;
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(c, kx[e], g[e]);
        }
        store_at<T>(dq, u, g);
      }
    }
    // Key j = u - 2: near contributions from queries j + n, far from j + F.
    const int j = u - 2;
    if (j >= a && j < end) {
      float ak[VEC], av[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) { ak[e] = 0.f; av[e] = 0.f; }
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + 2 + n) & 3;
          const bool there = j + n < T_;
          const float cs = there ? sd[slot][idx] : 0.f;
          const float cp = there ? sp[slot][idx] : 0.f;
          float qx[VEC], gx[VEC];
          widen<T>(qr[slot], qx);
          widen<T>(gr[slot], gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
            av[e] = __builtin_fmaf(cp, gx[e], av[e]);
          }
          ++idx;
        }
      }
      const bool there = j + F < T_;
      float cs, cp;
      Raw qf, gf;
      if constexpr (RIGHT_LDS) {
        // Query j + F is wave w + 1's query of step u - 2.
        const float2 w2 = down->pd[(R + 2) & 3][lane];
        qf = unpack(down->qd[(R + 2) & 3][0][lane]);
        gf = unpack(down->qd[(R + 2) & 3][1][lane]);
        cs = there ? w2.y : 0.f;
        cp = there ? w2.x : 0.f;
      } else {
        const Raw* ks[NS];
        const Raw* vs[NS];
        bool ok[NS];
        int n2 = 0;
#pragma unroll
        for (int n = 0; n < 3; ++n) {
          if (NM & (1 << n)) {
            ks[n2] = &fk[(R + 4 - n) & 3];
            vs[n2] = &fv[(R + 4 - n) & 3];
            ok[n2] = true;   // i - n >= F - 2 > 0
            ++n2;
          }
        }
        ks[NS - 1] = &kr[(R + 2) & 3];
        vs[NS - 1] = &vr[(R + 2) & 3];
        ok[NS - 1] = true;
        float pp[NS], ds[NS];
        grads(qi[R & 1], gi[R & 1], li_[R & 1], ks, vs, ok, pp, ds);
        qf = qi[R & 1];
        gf = gi[R & 1];
        cs = there ? ds[NS - 1] * scale : 0.f;
        cp = there ? pp[NS - 1] : 0.f;
      }
      float qx[VEC], gx[VEC];
      widen<T>(qf, qx);
      widen<T>(gf, gx);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
        av[e] = __builtin_fmaf(cp, gx[e], av[e]);
      }
      store_at<T>(dk, j, ak);
      store_at<T>(dv, j, av);
    }
  }

  __device__ inline void walk(int steps_from) {
    // u = a-2 .. a+P+1 for every wave of the workgroup (same trip count).
    const int u0 = steps_from;
    prefetch<0>(u0);
    for (int u = u0; u <= u0 + (end_u - u0); u += 4) {
      prefetch<1>(u + 1);
      compute<0>(u);
      prefetch<2>(u + 2);
      compute<1>(u + 1);
      prefetch<3>(u + 3);
      compute<2>(u + 2);
      prefetch<0>(u + 4);
      compute<3>(u + 3);
    }
  }
  int end_u;
};

template <typename T, int LPR, int NM, bool LEFT_LDS, bool RIGHT_LDS>
__device__ inline void chain_wave(const Params& p, const ChainCfg& c, ChainSlot* lds, int w, int b,
                                  int h0, int a, int hl, int li) {
  constexpr int esz = (int)sizeof(T);
  BwdChain<T, LPR, NM, LEFT_LDS, RIGHT_LDS> x;
  x.q = make_stream(p.q, esz, b, h0, hl, li);
  x.k = make_stream(p.k, esz, b, h0, hl, li);
  x.v = make_stream(p.v, esz, b, h0, hl, li);
  x.go = make_stream(p.dout, esz, b, h0, hl, li);
  x.dq = make_stream(p.dq, esz, b, h0, hl, li);
  x.dk = make_stream(p.dk, esz, b, h0, hl, li);
  x.dv = make_stream(p.dv, esz, b, h0, hl, li);
  x.lse = lse_stream(p, b, h0, hl);
  x.scale = p.scale;
  x.F = c.F;
  x.T_ = p.T;
  x.Tm1 = p.T - 1;
  x.a = a;
  x.end = min(a + c.P, p.T);   // < a for a row past the end: nothing is stored
  x.lane = threadIdx.x & 63;
  x.mine = lds + w;
  x.up = lds + (LEFT_LDS ? w - 1 : w);
  x.down = lds + (RIGHT_LDS ? w + 1 : w);
  // The trip count depends only on P: u = a-2 .. a+P+1 in steps of 4.
  x.end_u = a + c.P + 1;
  x.walk(a - 2);
}

template <typename T, int LPR, int NM, int W>
__global__ __launch_bounds__(64 * W) void bwd_chain(Params p, ChainCfg c) {
  __shared__ ChainSlot lds[W];
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Workgroup -> (batch, head group, band group, row block), XCD-contiguous;
  // wave w -> row w % L of the block, band w / L of the group.
  int64_t g = xcd_remap(blockIdx.x, gridDim.x);
  const int rb = (int)(g % c.blocks);
  g /= c.blocks;
  const int bgi = (int)(g % c.bgroups);
  g /= c.bgroups;
  const int hg = (int)(g % c.HG);
  const int b = (int)(g / c.HG);
  const int lr = w % c.L;
  const int r = rb * c.L + lr;
  const int cb = bgi * (W / c.L) + w / c.L;
  // Rows past the end (row blocks are padded to L rows, band groups to W / L
  // bands) start at T: their loads are clamped and they store nothing.
  const int64_t a64 = (int64_t)r * c.F + (int64_t)cb * c.P;
  const int a = (r < c.rows && cb < c.bands && a64 < p.T) ? (int)a64 : p.T;
  const int lane = threadIdx.x & 63;
  const int hl = lane / LPR, li = lane % LPR;
  const int h0 = hg * (64 / LPR);
  if (c.L == 1) {
    chain_wave<T, LPR, NM, false, false>(p, c, lds, w, b, h0, a, hl, li);
  } else if (lr == 0) {
    chain_wave<T, LPR, NM, false, true>(p, c, lds, w, b, h0, a, hl, li);
  } else if (lr == c.L - 1) {
    chain_wave<T, LPR, NM, true, false>(p, c, lds, w, b, h0, a, hl, li);
  } else {
    chain_wave<T, LPR, NM, true, true>(p, c, lds, w, b, h0, a, hl, li);
  }
}

// ============================================= transposed chain (far = 4, 8)
//
// For a small far offset F the far rows are F steps back in a wave's own walk
// -- evicted from L2 by then.  Here the sequence is seen as rows of F
// positions (t = r * F + c) and a workgroup of F waves walks R consecutive
// rows in lockstep, wave c owning column c: the far source of (r, c) is
// (r - 1, c), the wave's own previous step, kept in registers; the near
// sources t - 1, t - 2 are the neighbouring waves' rows of the same step (or
// the previous step across the row boundary), passed through LDS.  Keys are
// finalised two rows behind their query row, from the own queries (r - 2, c)
// (self slot) and (r - 1, c) (far slot) in registers and the near queries'
// q/dO rows and slot weights from LDS.  One barrier per step; every wave of
// the workgroup runs the same number of steps.

struct TcSlot {
  u32x4 kv[4][2][64];     // [row & 3][k, v][lane]
  u32x4 qd[4][2][64];     // [row & 3][q, dO][lane]
  float4 w[4][16];        // [row & 3][head]: (p_1, scale dS_1, p_2, scale dS_2)
};

struct TcCfg {
  int R;        // rows per workgroup
  int blocks;   // row blocks per (batch, head group)
  int HG, nwg;
};

template <typename T, int LPR, int NM, int F>
struct BwdTc {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + 1;
  static constexpr int G = 64 / LPR;

  Stream q, k, v, go, dq, dk, dv, lse;
  float scale;
  int T_, Tm1, r0, R, c, lane, hl, li;
  TcSlot* lds;
  Raw kr[4], vr[4], qr[4], gr[4];   // own rows by row & 3
  float lr[4];
  float p0[4], d0[4];               // own query's self-slot (p, scale dS) by row & 3
  float pf[4], df[4];               // own query's far-slot (p, scale dS) by row & 3

  template <int K>
  __device__ inline void prefetch(int r) {
    const int t = clampi(r * F + c, Tm1);
    kr[K] = load_at(k, t);
    vr[K] = load_at(v, t);
    qr[K] = load_at(q, t);
    gr[K] = load_at(go, t);
    lr[K] = load_f32(lse, t);
  }

  __device__ static inline u32x4 pack(const Raw& x) { return u32x4{x.w[0], x.w[1], x.w[2], x.w[3]}; }
  __device__ static inline Raw unpack(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

  // Step of row r (K = r & 3, static).
  template <int K>
  __device__ inline void step(int r) {
    constexpr int K1 = (K + 3) & 3, K2 = (K + 2) & 3;   // rows r - 1, r - 2
    TcSlot& me = lds[c];
    me.kv[K][0][lane] = pack(kr[K]);
    me.kv[K][1][lane] = pack(vr[K]);
    me.qd[K][0][lane] = pack(qr[K]);
    me.qd[K][1][lane] = pack(gr[K]);
    __syncthreads();
    const int t = r * F + c;
    // ---- query (r, c): rows r0 .. r0 + R (row r0 + R feeds the last keys)
    if (r >= r0 && r <= r0 + R) {
      Raw kn[3], vn[3];
      const Raw* ks[NS];
      const Raw* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          if (n == 0) {
            ks[idx] = &kr[K];
            vs[idx] = &vr[K];
          } else {
            // Source t - n: wave c - n of this row, or wave c - n + F of row r - 1.
            const bool wrap = c < n;
            const int src = wrap ? c - n + F : c - n;
            const TcSlot& o = lds[src];
            kn[n] = unpack(wrap ? o.kv[K1][0][lane] : o.kv[K][0][lane]);
            vn[n] = unpack(wrap ? o.kv[K1][1][lane] : o.kv[K][1][lane]);
            ks[idx] = &kn[n];
            vs[idx] = &vn[n];
          }
          ok[idx] = t - n >= 0;
          ++idx;
        }
      }
      ks[NS - 1] = &kr[K1];   // far source (r - 1, c)
      vs[NS - 1] = &vr[K1];
      ok[NS - 1] = t - F >= 0;
      float pp[NS], ds[NS];
      {
        float dp[NS];
        float delta = 0.f;
#pragma unroll
        for (int s_ = 0; s_ < NS; ++s_) {
          const float sc = row_sum<LPR>(dot_raw<T>(qr[K], *ks[s_])) * scale;
          dp[s_] = row_sum<LPR>(dot_raw<T>(gr[K], *vs[s_]));
          pp[s_] = ok[s_] ? fast_exp(sc - lr[K]) : 0.f;
          delta = __builtin_fmaf(pp[s_], dp[s_], delta);
        }
#pragma unroll
        for (int s_ = 0; s_ < NS; ++s_) ds[s_] = pp[s_] * (dp[s_] - delta);
      }
      // Slot weights for the keys this query feeds: self (kept), far (kept),
      // t - 1 and t - 2 (published for the owning waves).
      p0[K] = pp[0];
      d0[K] = ds[0] * scale;
      pf[K] = pp[NS - 1];
      df[K] = ds[NS - 1] * scale;
      float4 wn = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr (NM & 2) {
        wn.x = pp[1];
        wn.y = ds[1] * scale;
      }
      if constexpr (NM & 4) {
        constexpr int i2 = NearSet<NM>::count - 1;
        wn.z = pp[i2];
        wn.w = ds[i2] * scale;
      }
      if (li == 0) me.w[K][hl] = wn;
      if (r < r0 + R && t < T_) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
        for (int s_ = 0; s_ < NS; ++s_) {
          float kx[VEC];
          widen<T>(*ks[s_], kx);
          const float cc = ds[s_] * scale;
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(cc, kx[e], g[e]);
        }
        store_at<T>(dq, t, g);
      }
    }
    // ---- key (r - 2, c)
    const int rj = r - 2;
    const int j = rj * F + c;
    if (rj >= r0 && rj < r0 + R && j < T_) {
      float ak[VEC], av[VEC];
      float qx[VEC], gx[VEC];
      // self slot: own query (r - 2, c)
      {
        const float cs = d0[K2];
        const float cp = p0[K2];
        widen<T>(qr[K2], qx);
        widen<T>(gr[K2], gx);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          ak[e] = cs * qx[e];
          av[e] = cp * gx[e];
        }
      }
      // near slots n = 1, 2: query j + n = wave c + n of row r - 2, or wave
      // c + n - F of row r - 1.
#pragma unroll
      for (int n = 1; n < 3; ++n) {
        if (NM & (1 << n)) {
          const bool wrap = c + n >= F;
          const int src = wrap ? c + n - F : c + n;
          const TcSlot& o = lds[src];
          const float4 wq = wrap ? o.w[K1][hl] : o.w[K2][hl];
          const bool there = j + n < T_;
          const float cs = there ? (n == 1 ? wq.y : wq.w) : 0.f;
          const float cp = there ? (n == 1 ? wq.x : wq.z) : 0.f;
          const Raw qq = unpack(wrap ? o.qd[K1][0][lane] : o.qd[K2][0][lane]);
          const Raw gg = unpack(wrap ? o.qd[K1][1][lane] : o.qd[K2][1][lane]);
          widen<T>(qq, qx);
          widen<T>(gg, gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
            av[e] = __builtin_fmaf(cp, gx[e], av[e]);
          }
        }
      }
      // far slot: own query (r - 1, c) = j + F
      {
        const bool there = j + F < T_;
        const float cs = there ? df[K1] : 0.f;
        const float cp = there ? pf[K1] : 0.f;
        widen<T>(qr[K1], qx);
        widen<T>(gr[K1], gx);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
          av[e] = __builtin_fmaf(cp, gx[e], av[e]);
        }
      }
      store_at<T>(dk, j, ak);
      store_at<T>(dv, j, av);
    }
  }
};

template <typename T, int LPR, int NM, int F>
__global__ __launch_bounds__(64 * F) void bwd_tc(Params p, TcCfg cfg) {
  __shared__ TcSlot lds[F];
  const int c = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  int64_t g = xcd_remap(blockIdx.x, gridDim.x);
  const int rb = (int)(g % cfg.blocks);
  g /= cfg.blocks;
  const int hg = (int)(g % cfg.HG);
  const int b = (int)(g / cfg.HG);
  constexpr int esz = (int)sizeof(T);
  const int lane = threadIdx.x & 63;
  const int hl = lane / LPR, li = lane % LPR;
  const int h0 = hg * (64 / LPR);
  BwdTc<T, LPR, NM, F> x;
  x.q = make_stream(p.q, esz, b, h0, hl, li);
  x.k = make_stream(p.k, esz, b, h0, hl, li);
  x.v = make_stream(p.v, esz, b, h0, hl, li);
  x.go = make_stream(p.dout, esz, b, h0, hl, li);
  x.dq = make_stream(p.dq, esz, b, h0, hl, li);
  x.dk = make_stream(p.dk, esz, b, h0, hl, li);
  x.dv = make_stream(p.dv, esz, b, h0, hl, li);
  x.lse = lse_stream(p, b, h0, hl);
  x.scale = p.scale;
  x.T_ = p.T;
  x.Tm1 = p.T - 1;
  x.R = cfg.R;
  x.r0 = rb * cfg.R;
  x.c = c;
  x.lane = lane;
  x.hl = hl;
  x.li = li;
  x.lds = lds;
  // Rows r0-1 .. r0+R+1 (R + 3 steps, rounded up to a multiple of 4; the
  // extra steps compute nothing).  Row & 3 is the static slot K.
  const int s0 = x.r0 - 1;
  const int steps = (cfg.R + 3 + 3) & ~3;
  // s0 & 3 is not known statically: walk from the multiple of 4 below s0
  // (steps before s0 compute nothing; they only fill the rotation).
  const int sa = s0 & ~3;
  const int sb = s0 + steps;
  x.template prefetch<0>(sa);
  for (int r = sa; r < sb; r += 4) {
    x.template prefetch<1>(r + 1);
    x.template step<0>(r);
    x.template prefetch<2>(r + 2);
    x.template step<1>(r + 1);
    x.template prefetch<3>(r + 3);
    x.template step<2>(r + 2);
    x.template prefetch<0>(r + 4);
    x.template step<3>(r + 3);
  }
}

// ============================================== pipelined walks, fused prologue
//
// The prologue (head-RMSNorm + RoPE of q and k) is applied to each raw row
// once, when it arrives; roped rows are kept in fp32.  Rows are in the split
// layout (a lane holds the same positions of both halves, so RoPE partners
// share a lane); v and dO stay raw and their dot products use v_dot2.
//
// The backward runs as two walks so that each fits in registers:
//   A (query side): per query u, p_s and dS_s, dQ (through the transposed
//     prologue) and, per (row, slot), the pair (p_s, scale * dS_s) into a
//     workspace table [B, T, H, 2 * NS] (fp32);
//   B (key side): per key j, dK/dV from queries j + n (near slots) and j + F
//     (far slot) using that table -- no weight recomputation -- then dK
//     through the transposed prologue.

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Split-layout rows: a lane holds HV elements of each half (byte offsets
// lo and hi inside a position), so RoPE partners share a lane.
struct SplitStream {
  const char* base;
  uint32_t st;
  uint32_t lo, hi;

  __device__ inline uint32_t at(int t) const { return (uint32_t)t * st; }
};

template <typename Vw>
__device__ inline SplitStream make_split(const Vw& vw, int esz, int b, int h0, int hl, int li,
                                         int D, int hv) {
  SplitStream s;
  s.base = (const char*)vw.p + ((int64_t)b * vw.sb + (int64_t)h0 * vw.sh) * esz;
  s.st = (uint32_t)(vw.st * esz);
  const uint32_t head = (uint32_t)((int64_t)hl * vw.sh * esz);
  s.lo = head + (uint32_t)(li * hv * esz);
  s.hi = head + (uint32_t)(((D >> 1) + li * hv) * esz);
  return s;
}

template <bool NT = false>
__device__ inline Raw load_split(const SplitStream& s, int t) {
  const uint32_t r = s.at(t);
  const u32x2* px = reinterpret_cast<const u32x2*>(s.base + (uint64_t)(r + s.lo));
  const u32x2* py = reinterpret_cast<const u32x2*>(s.base + (uint64_t)(r + s.hi));
  u32x2 x, y;
  if constexpr (NT) {
    x = __builtin_nontemporal_load(px);
    y = __builtin_nontemporal_load(py);
  } else {
    x = *px;
    y = *py;
  }
  return Raw{{x.x, x.y, y.x, y.y}};
}

template <typename T>
__device__ inline void store_split(const SplitStream& s, int t, const float (&x)[VecOf<T>::value]) {
  constexpr int HV = VecOf<T>::value / 2;
  uint32_t wa[2], wb[2];
  pack_words<T, 2>(x, wa);
  pack_words<T, 2>(x + HV, wb);
  const uint32_t r = s.at(t);
  char* base = const_cast<char*>(s.base);
  __builtin_nontemporal_store(u32x2{wa[0], wa[1]}, reinterpret_cast<u32x2*>(base + (uint64_t)(r + s.lo)));
  __builtin_nontemporal_store(u32x2{wb[0], wb[1]}, reinterpret_cast<u32x2*>(base + (uint64_t)(r + s.hi)));
}

template <typename T, int LPR>
struct ProBase {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int HV = VEC / 2;
  using PL = Prologue<T, LPR>;
  Stream rc, rs;   // fp32 [T, D/2] RoPE tables: this lane's HV entries of a position
  float eps;
  int li, D, Tm1;
  float wq[VEC], wk[VEC];

  __device__ inline void init(const Params& p, int lane_in_row) {
    li = lane_in_row;
    D = p.D;
    Tm1 = p.T - 1;
    eps = p.eps;
    const int half = D >> 1;
    rc.base = (const char*)p.rope_cos;
    rs.base = (const char*)p.rope_sin;
    rc.st = rs.st = (uint32_t)half * 4u;
    rc.lane = rs.lane = (uint32_t)(li * HV) * 4u;
    PL::load_w(p.wq, li, D, wq);
    PL::load_w(p.wk, li, D, wk);
  }
  // cos/sin of position t (every lane of a walk row is inside the row).
  __device__ inline void cs(int t, float (&c)[HV], float (&s)[HV]) const {
    const uint32_t oc = rc.at(t), os = rs.at(t);
    if constexpr (HV == 4) {
      const float4 a = *reinterpret_cast<const float4*>(rc.base + (uint64_t)oc);
      const float4 b = *reinterpret_cast<const float4*>(rs.base + (uint64_t)os);
      c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
      s[0] = b.x; s[1] = b.y; s[2] = b.z; s[3] = b.w;
    } else {
      static_assert(HV == 2, "16-bit rows hold 4, fp32 rows 2 elements per half");
      const float2 a = *reinterpret_cast<const float2*>(rc.base + (uint64_t)oc);
      const float2 b = *reinterpret_cast<const float2*>(rs.base + (uint64_t)os);
      c[0] = a.x; c[1] = a.y;
      s[0] = b.x; s[1] = b.y;
    }
  }
  // Widens a raw q/k row and applies the prologue; returns the rms factor.
  __device__ inline float rope(const Raw& r, const float (&w)[VEC], const float (&c)[HV],
                               const float (&s)[HV], float (&x)[VEC]) const {
    widen<T>(r, x);
    return PL::forward_w(x, w, c, s, D, eps);
  }
};

template <typename T, int LPR, int NM, bool FAR>
struct FwdPipePro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  SplitStream q, k, v, o;
  Stream lse;
  int F;
  float scale;
  Raw kraw[2], qraw[2], vraw[2], klr[2], vlr[2];
  float cc[2][HV], ss[2][HV], clc[2][HV], cls[2][HV];
  float kq[4][VEC], vr[4][VEC];

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, this->Tm1);
    kraw[R & 1] = load_split<!FAR>(k, tc);
    qraw[R & 1] = load_split<!FAR>(q, tc);
    vraw[R & 1] = load_split<!FAR>(v, tc);
    this->cs(tc, cc[R & 1], ss[R & 1]);
    if constexpr (FAR) {
      const int tf = clampi(t - F, this->Tm1);
      klr[R & 1] = load_split(k, tf);
      vlr[R & 1] = load_split(v, tf);
      this->cs(tf, clc[R & 1], cls[R & 1]);
    }
  }

  template <int R>
  __device__ inline void compute(int t, bool store) {
    this->rope(kraw[R & 1], this->wk, cc[R & 1], ss[R & 1], kq[R]);
    widen<T>(vraw[R & 1], vr[R]);
    float qr[VEC];
    this->rope(qraw[R & 1], this->wq, cc[R & 1], ss[R & 1], qr);
    float sc[NS];
    bool ok[NS];
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        ok[idx] = t - n >= 0;
        sc[idx] = row_sum<LPR>(dot_partial<VEC>(qr, kq[(R + 4 - n) & 3])) * scale;
        ++idx;
      }
    }
    float vf[VEC];
    if constexpr (FAR) {
      float kf[VEC];
      this->rope(klr[R & 1], this->wk, clc[R & 1], cls[R & 1], kf);
      widen<T>(vlr[R & 1], vf);
      ok[NS - 1] = t - F >= 0;
      sc[NS - 1] = row_sum<LPR>(dot_partial<VEC>(qr, kf)) * scale;
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; ++s) m = ok[s] ? fmaxf(m, sc[s]) : m;
    float w[NS], l = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      w[s] = ok[s] ? fast_exp(sc[s] - m) : 0.f;
      l += w[s];
    }
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        const int slot = (R + 4 - n) & 3;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[idx], vr[slot][e], acc[e]);
        ++idx;
      }
    }
    if constexpr (FAR) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[NS - 1], vf[e], acc[e]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= inv;
    if (store) {
      store_split<T>(o, t, acc);
      if (this->li == 0) store_f32(lse, t, l > 0.f ? m + fast_log(l) : INFINITY);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kPipeBlock) void fwd_pipe_pro(Params p, WalkCfg c) {
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int esz = (int)sizeof(T);
  const int h0 = wt.hg * (64 / LPR);
  FwdPipePro<T, LPR, NM, FAR> w;
  w.init(p, wt.li);
  w.q = make_split(p.q, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.k = make_split(p.k, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.v = make_split(p.v, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.o = make_split(p.o, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.lse = lse_stream(p, wt.b, h0, wt.hl);
  w.scale = p.scale;
  w.F = c.F;
  const int a = wt.a, end = min(a + c.P, p.T);
  // Slot of t is (t - a + 2) & 3; the trip count depends only on P.
  const int t0 = a - 2;
  w.template prefetch<0>(t0);
  for (int t = t0; t < a + c.P; t += 4) {
    __syncthreads();
    w.template prefetch<1>(t + 1);
    w.template compute<0>(t, t >= a && t < end);
    w.template prefetch<2>(t + 2);
    w.template compute<1>(t + 1, t + 1 >= a && t + 1 < end);
    w.template prefetch<3>(t + 3);
    w.template compute<2>(t + 2, t + 2 >= a && t + 2 < end);
    w.template prefetch<0>(t + 4);
    w.template compute<3>(t + 3, t + 3 >= a && t + 3 < end);
  }
}

// ---- backward A: query side

template <typename T, int LPR, int NM, bool FAR>
struct BwdQPro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using PL = typename B_::PL;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  SplitStream q, k, v, go, dq;
  Stream lse;
  float* __restrict__ tab;   // (p, scale * dS) per (row, slot)
  int64_t tst;
  int F, a, end;
  float scale;
  Raw kraw[2], qraw[2], graw[2], klr[2], vlr[2];
  float lv[2];
  float cc[2][HV], ss[2][HV], clc[2][HV], cls[2][HV];
  float kq[4][VEC];
  Raw vr[4];
  float dw[VEC];

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, this->Tm1);
    kraw[R & 1] = load_split<!FAR>(k, uc);
    vr[R] = load_split<!FAR>(v, uc);
    qraw[R & 1] = load_split<!FAR>(q, uc);
    graw[R & 1] = load_split<!FAR>(go, uc);
    lv[R & 1] = load_f32(lse, uc);
    this->cs(uc, cc[R & 1], ss[R & 1]);
    if constexpr (FAR) {
      const int ul = clampi(u - F, this->Tm1);
      klr[R & 1] = load_split(k, ul);
      vlr[R & 1] = load_split(v, ul);
      this->cs(ul, clc[R & 1], cls[R & 1]);
    }
  }

  template <int R>
  __device__ inline void compute(int u) {
    this->rope(kraw[R & 1], this->wk, cc[R & 1], ss[R & 1], kq[R]);
    float qx[VEC], qr[VEC];
    widen<T>(qraw[R & 1], qx);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qr[e] = qx[e];
    const float rq = PL::forward_w(qr, this->wq, cc[R & 1], ss[R & 1], this->D, this->eps);
    float kf[VEC];
    if constexpr (FAR) this->rope(klr[R & 1], this->wk, clc[R & 1], cls[R & 1], kf);
    const float* ks[NS];
    const Raw* vs[NS];
    bool ok[NS];
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        ks[idx] = kq[(R + 4 - n) & 3];
        vs[idx] = &vr[(R + 4 - n) & 3];
        ok[idx] = u - n >= 0;
        ++idx;
      }
    }
    if constexpr (FAR) {
      ks[NS - 1] = kf;
      vs[NS - 1] = &vlr[R & 1];
      ok[NS - 1] = u - F >= 0;
    }
    float pp[NS], dp[NS], delta = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float a_ = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) a_ = __builtin_fmaf(qr[e], ks[s][e], a_);
      const float sc = row_sum<LPR>(a_) * scale;
      dp[s] = row_sum<LPR>(dot_raw<T>(graw[R & 1], *vs[s]));
      pp[s] = ok[s] ? fast_exp(sc - lv[R & 1]) : 0.f;
      delta = __builtin_fmaf(pp[s], dp[s], delta);
    }
    if (u >= a && u < end) {
      float g[VEC], ds[NS];
#pragma unroll
      for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        ds[s] = pp[s] * (dp[s] - delta) * scale;
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(ds[s], ks[s][e], g[e]);
      }
      PL::backward_w(g, qx, rq, this->wq, cc[R & 1], ss[R & 1], this->D, dw);
      store_split<T>(dq, u, g);
      float* trow = tab + (int64_t)u * tst;
#pragma unroll
      for (int vix = 0; vix < 2 * NS; ++vix) {
        const int s = vix >> 1;
        if (vix % LPR == this->li) trow[vix] = (vix & 1) ? ds[s] : pp[s];
      }
    }
  }
};

// ---- backward B: key side

template <typename T, int LPR, int NM, bool FAR>
struct BwdKPro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using PL = typename B_::PL;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  SplitStream q, k, go, dk, dv;
  const float* __restrict__ tab;
  int64_t tst;
  int F, a, end, T_;
  Raw qraw[2], kraw[2], qir[2], gir[2];
  Raw gr[4];
  float cc[2][HV], ss[2][HV], cic[2][HV], cis[2][HV], ckc[2][HV], cks[2][HV];
  float tp[2][NS], td[2][NS];   // (p, scale dS) feeding key u - 2, per slot
  float qq[4][VEC];
  float dw[VEC];

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, this->Tm1);
    qraw[R & 1] = load_split<!FAR>(q, uc);
    gr[R] = load_split<!FAR>(go, uc);
    this->cs(uc, cc[R & 1], ss[R & 1]);
    const int j = u - 2;
    const int jc = clampi(j, this->Tm1);
    kraw[R & 1] = load_split<!FAR>(k, jc);
    this->cs(jc, ckc[R & 1], cks[R & 1]);
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        const float* trow = tab + (int64_t)clampi(j + n, this->Tm1) * tst;
        tp[R & 1][idx] = trow[2 * idx];
        td[R & 1][idx] = trow[2 * idx + 1];
        ++idx;
      }
    }
    if constexpr (FAR) {
      const int ic = clampi(j + F, this->Tm1);
      const float* trow = tab + (int64_t)ic * tst;
      tp[R & 1][NS - 1] = trow[2 * (NS - 1)];
      td[R & 1][NS - 1] = trow[2 * (NS - 1) + 1];
      qir[R & 1] = load_split(q, ic);
      gir[R & 1] = load_split(go, ic);
      this->cs(ic, cic[R & 1], cis[R & 1]);
    }
  }

  template <int R>
  __device__ inline void compute(int u) {
    this->rope(qraw[R & 1], this->wq, cc[R & 1], ss[R & 1], qq[R]);
    const int j = u - 2;
    if (j >= a && j < end) {
      float ak[VEC], av[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) { ak[e] = 0.f; av[e] = 0.f; }
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + 2 + n) & 3;   // query j + n
          const bool there = j + n < T_;
          const float cs_ = there ? td[R & 1][idx] : 0.f;
          const float cp_ = there ? tp[R & 1][idx] : 0.f;
          float gx[VEC];
          widen<T>(gr[slot], gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs_, qq[slot][e], ak[e]);
            av[e] = __builtin_fmaf(cp_, gx[e], av[e]);
          }
          ++idx;
        }
      }
      if constexpr (FAR) {
        const bool there = j + F < T_;
        const float cs_ = there ? td[R & 1][NS - 1] : 0.f;
        const float cp_ = there ? tp[R & 1][NS - 1] : 0.f;
        float qf[VEC], gx[VEC];
        this->rope(qir[R & 1], this->wq, cic[R & 1], cis[R & 1], qf);
        widen<T>(gir[R & 1], gx);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          ak[e] = __builtin_fmaf(cs_, qf[e], ak[e]);
          av[e] = __builtin_fmaf(cp_, gx[e], av[e]);
        }
      }
      float kx[VEC];
      widen<T>(kraw[R & 1], kx);
      const float rk = PL::rms_factor(kx, this->D, this->eps);
      PL::backward_w(ak, kx, rk, this->wk, ckc[R & 1], cks[R & 1], this->D, dw);
      store_split<T>(dk, j, ak);
      store_split<T>(dv, j, av);
    }
  }
};

// Four steps per trip with one barrier (the workgroup walks in lockstep).
template <typename W>
__device__ inline void walk4(W& w, int first, int last) {
  w.template prefetch<0>(first);
  for (int u = first; u <= last; u += 4) {
    __syncthreads();
    w.template prefetch<1>(u + 1);
    w.template compute<0>(u);
    w.template prefetch<2>(u + 2);
    w.template compute<1>(u + 1);
    w.template prefetch<3>(u + 3);
    w.template compute<2>(u + 2);
    w.template prefetch<0>(u + 4);
    w.template compute<3>(u + 3);
  }
}

__device__ inline int64_t pipe_wave_id(const WalkCfg& c) {
  return xcd_remap(blockIdx.x, gridDim.x) * c.waves +
         __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kPipeBlock) void bwd_q_pro(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value, esz = (int)sizeof(T);
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  const int h0 = wt.hg * (64 / LPR);
  BwdQPro<T, LPR, NM, FAR> w;
#pragma unroll
  for (int e = 0; e < VEC; ++e) w.dw[e] = 0.f;
  w.init(p, wt.li);
  w.q = make_split(p.q, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.k = make_split(p.k, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.v = make_split(p.v, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.go = make_split(p.dout, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.dq = make_split(p.dq, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.lse = lse_stream(p, wt.b, h0, wt.hl);
  w.tab = p.tab + ((int64_t)wt.b * p.T * p.H + h0 + wt.hl) * (2 * w.NS);
  w.tst = (int64_t)p.H * 2 * w.NS;
  w.scale = p.scale;
  w.F = c.F;
  w.a = wt.a;
  w.end = min(wt.a + c.P, p.T);
  // Queries a-2, a-1 only fill the near-source rotation (slot of u is
  // (u - a + 2) & 3); the trip count depends only on P.
  walk4(w, wt.a - 2, wt.a + c.P - 1);
  write_wave_partial<T, LPR, true>(w.dw, p.dwq_part, pipe_wave_id(c), p.D);
}

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kPipeBlock) void bwd_k_pro(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value, esz = (int)sizeof(T);
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  const int h0 = wt.hg * (64 / LPR);
  BwdKPro<T, LPR, NM, FAR> w;
#pragma unroll
  for (int e = 0; e < VEC; ++e) w.dw[e] = 0.f;
  w.init(p, wt.li);
  w.q = make_split(p.q, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.k = make_split(p.k, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.go = make_split(p.dout, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.dk = make_split(p.dk, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.dv = make_split(p.dv, esz, wt.b, h0, wt.hl, wt.li, p.D, w.HV);
  w.tab = p.tab + ((int64_t)wt.b * p.T * p.H + h0 + wt.hl) * (2 * w.NS);
  w.tst = (int64_t)p.H * 2 * w.NS;
  w.F = c.F;
  w.a = wt.a;
  w.end = min(wt.a + c.P, p.T);
  w.T_ = p.T;
  // Walk u = a .. a+P+1 (slot of u is (u - a) & 3); key u - 2 is finished at step u.
  walk4(w, wt.a, wt.a + c.P + 1);
  write_wave_partial<T, LPR, true>(w.dw, p.dwk_part, pipe_wave_id(c), p.D);
}

// ================================================================= dispatch

struct Pattern {
  int nm;     // near mask over offsets {0, 1, 2}
  int far;    // far offset (0 if none)
};

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

// Pipelined walks and the chained backward: 32-position tiles, or
// min(max_col_tile, F) for a power-of-two far offset F >= 16 (column order,
// far rows one column row away); halved (not below 16) while the grid has
// fewer than 256 full workgroups.
WalkCfg make_pipe_cfg(const Params& p, int lpr, const Pattern& pat, int max_col_tile) {
  WalkCfg c{};
  c.waves = kPipeWaves;
  c.HG = p.H / (64 / lpr);
  const int64_t lanes_rows = (int64_t)p.B * c.HG;
  const bool pow2far = pat.far >= 16 && (pat.far & (pat.far - 1)) == 0;
  int P = pow2far ? min(max_col_tile, pat.far) : 32;
  while (P > 16 && lanes_rows * ((p.T + P - 1) / P) < 256 * kPipeWaves) P >>= 1;
  c.P = P;
  order_tiles(p, pat, lanes_rows, c);
  return c;
}

template <typename T, int LPR, int NM>
hipError_t launch_chain(const Params& p, const WalkCfg& wc, hipStream_t st) {
  ChainCfg c{};
  c.P = wc.P;
  c.F = wc.F;
  c.rows = wc.rows;
  c.W = c.rows >= 8 ? 8 : c.rows >= 4 ? 4 : c.rows >= 2 ? 2 : 1;
  // Same DRAM-channel limit as the forward's row groups (walk_launch).
  if ((int64_t)wc.F * p.q.st * (int64_t)sizeof(T) >= kBigStride && c.W > 4) c.W = 4;
  // One chain per workgroup (L = W): shorter chains on more bands measured
  // slower (backward 30.7 -> 32.0 ms per step at L = 4).
  c.L = c.W;
  c.bands = wc.F / wc.P;
  c.blocks = (c.rows + c.L - 1) / c.L;
  c.bgroups = (c.bands + c.W / c.L - 1) / (c.W / c.L);
  c.HG = wc.HG;
  const int64_t nwg = (int64_t)p.B * c.HG * c.bgroups * c.blocks;
  if (nwg <= 0 || nwg > 0x7fffffff) return hipErrorInvalidValue;
  c.nwg = (int)nwg;
  const dim3 grid((unsigned)c.nwg), block(64 * c.W);
  switch (c.W) {
    case 8: hipLaunchKernelGGL((bwd_chain<T, LPR, NM, 8>), grid, block, 0, st, p, c); break;
    case 4: hipLaunchKernelGGL((bwd_chain<T, LPR, NM, 4>), grid, block, 0, st, p, c); break;
    case 2: hipLaunchKernelGGL((bwd_chain<T, LPR, NM, 2>), grid, block, 0, st, p, c); break;
    default: hipLaunchKernelGGL((bwd_chain<T, LPR, NM, 1>), grid, block, 0, st, p, c); break;
  }
  return hipGetLastError();
}

template <typename T, int LPR, int NM, int F>
hipError_t launch_tc(const Params& p, const WalkCfg& wc, hipStream_t st) {
  TcCfg c{};
  const int64_t rows = (p.T + F - 1) / F;
  const int64_t lanes_rows = (int64_t)p.B * wc.HG;
  int R = 256;
  while (R > 16 && lanes_rows * ((rows + R - 1) / R) < 1024) R >>= 1;
  c.R = R;
  c.blocks = (int)((rows + R - 1) / R);
  c.HG = wc.HG;
  const int64_t nwg = lanes_rows * c.blocks;
  if (nwg <= 0 || nwg > 0x7fffffff) return hipErrorInvalidValue;
  c.nwg = (int)nwg;
  hipLaunchKernelGGL((bwd_tc<T, LPR, NM, F>), dim3((unsigned)c.nwg), dim3(64 * F), 0, st, p, c);
  return hipGetLastError();
}

template <typename T, int LPR, bool PRO, bool FWD>
hipError_t launch_pattern(const Params& p, const WalkCfg& c, const Pattern& pat, hipStream_t st) {
  if (!FWD && !PRO && pat.far != 0 && c.column) {
    return pat.nm == 7 ? launch_chain<T, LPR, 7>(p, c, st) : launch_chain<T, LPR, 1>(p, c, st);
  }
  if (!FWD && !PRO && (pat.far == 4 || pat.far == 8) && !c.column) {
    if (pat.far == 4)
      return pat.nm == 7 ? launch_tc<T, LPR, 7, 4>(p, c, st) : launch_tc<T, LPR, 1, 4>(p, c, st);
    return pat.nm == 7 ? launch_tc<T, LPR, 7, 8>(p, c, st) : launch_tc<T, LPR, 1, 8>(p, c, st);
  }
  const dim3 grid((unsigned)c.nwg);
  const dim3 pblock(kPipeBlock);
#define SBDA_WALK_CASE(NMV, FARV)                                                            \
  if (pat.nm == NMV && (pat.far != 0) == FARV) {                                             \
    if (FWD && PRO) {                                                                        \
      hipLaunchKernelGGL((fwd_pipe_pro<T, LPR, NMV, FARV>), grid, pblock, kPipeLds, st, p, c); \
    } else if (FWD) {                                                                        \
      if (FARV && pat.far == 4 && !c.column)                                                 \
        hipLaunchKernelGGL((fwd_pipe<T, LPR, NMV, FARV, FARV ? 4 : 0>), grid, pblock,       \
                           kPipeLds, st, p, c);                                              \
      else if (FARV && pat.far == 8 && !c.column)                                            \
        hipLaunchKernelGGL((fwd_pipe<T, LPR, NMV, FARV, FARV ? 8 : 0>), grid, pblock,       \
                           kPipeLds, st, p, c);                                              \
      else                                                                                   \
        hipLaunchKernelGGL((fwd_pipe<T, LPR, NMV, FARV, 0>), grid, dim3(64 * c.waves),       \
                           kPipeLds / (kPipeWaves / c.waves), st, p, c);                     \
    } else if (PRO) {                                                                        \
      hipLaunchKernelGGL((bwd_q_pro<T, LPR, NMV, FARV>), grid, pblock, kPipeLds, st, p, c); \
      hipError_t e_ = hipGetLastError();                                                     \
      if (e_ != hipSuccess) return e_;                                                       \
      hipLaunchKernelGGL((bwd_k_pro<T, LPR, NMV, FARV>), grid, pblock, kPipeLds, st, p, c); \
    } else {                                                                                 \
      hipLaunchKernelGGL((bwd_pipe<T, LPR, NMV, FARV>), grid, pblock, kPipeLds, st, p, c);  \
    }                                                                                        \
    return hipGetLastError();                                                                \
  }
  SBDA_WALK_CASE(3, false)
  SBDA_WALK_CASE(5, false)
  SBDA_WALK_CASE(7, true)
  SBDA_WALK_CASE(1, true)
#undef SBDA_WALK_CASE
  return hipErrorInvalidValue;
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
    WalkCfg c = make_pipe_cfg(p, lpr, pat, 64);
    if (c.column && c.rows >= 2) {
      int rg = 2;
      while (rg < kPipeWaves && rg * c.bands < kPipeWaves) rg <<= 1;
      c.rg = rg;
      order_tiles(p, pat, (int64_t)p.B * c.HG, c);
    }
    return c;
  }
  WalkCfg c = make_pipe_cfg(p, lpr, pat, 128);
  if ((fwd || pro) && c.column && c.rows > 4 && far_stride_bytes(p, pat, dtype) >= kBigStride) {
    c.rg = 4;
    order_tiles(p, pat, (int64_t)p.B * c.HG, c);
  }
  return c;
}

template <typename T>
struct TypeTag {
  using type = T;
};

template <bool FWD>
hipError_t walk_launch(const Params& p, int dtype, bool pro, hipStream_t st) {
  Pattern pat;
  if (!classify(p, &pat)) return hipErrorInvalidValue;
  const int lpr = walk_lpr(p, dtype);
  const WalkCfg c = launch_cfg(p, dtype, pat, lpr, FWD, pro);
  auto go = [&](auto tag, auto lprc) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int L = decltype(lprc)::value;
    return pro ? launch_pattern<T, L, true, FWD>(p, c, pat, st)
               : launch_pattern<T, L, false, FWD>(p, c, pat, st);
  };
  auto by_lpr = [&](auto tag) -> hipError_t {
    switch (lpr) {
      case 4: return go(tag, std::integral_constant<int, 4>{});
      case 8: return go(tag, std::integral_constant<int, 8>{});
      case 16: return go(tag, std::integral_constant<int, 16>{});
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

}  // namespace

// Every byte offset a wave forms from its head group's base (row offset plus
// lane offset) must fit the 32-bit vector offset of the load/store form.
template <typename Vw>
bool span_fits_32(const Vw& vw, const Params& p, int esz, int lpr) {
  if (vw.p == nullptr) return true;
  if (vw.st < 0 || vw.sh < 0) return false;
  const int64_t span =
      ((int64_t)(p.T - 1) * vw.st + (int64_t)(64 / lpr - 1) * vw.sh) * esz + 16 * lpr;
  return span <= (int64_t)0xffffffffLL;
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
  *pq = (int64_t)c.nwg * c.waves;
  *pk = *pq;
  *tab_floats = (int64_t)p.B * p.T * p.H * 2 * p.S;
}

}  // namespace sbda
