// Backward walks (gather form, every gradient row written once, no atomics):
// independent lockstep walks (bwd_pipe; bwd_fr4 for far offset 4), chained
// column walks (bwd_chain) and transposed chains for far offset 8 (bwd_tc).
// Reference semantics: the key-centric backward specified by
// BiAttn/sbda_triton.py:507-671.

#include "sbda_walk.h"

namespace sbda {
namespace walk {

namespace {

// Far-free walks: the rows of a tile's first four steps (a - 2 .. a + 1) are
// the last four steps' rows of the tile before it.  A wave whose left
// neighbour in the workgroup walks that tile leaves them in LDS, and the
// neighbour takes its last four steps' rows from there instead of loading
// them again (they are long gone from L2 by then).
struct PipeStash {
  u32x4 row[4][4][64];   // [step][k, v, q, dO][lane]
  float lse[4][64];      // [step][lane]
};

template <typename T, int LPR, int NM, bool FAR>
struct BwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  Stream q, k, v, go, dq, dk, dv, lse;
  float scale;
  int F, T_, Tm1, a, end, last;   // the walk's steps are u = a - 2 .. last
  bool has_prev;                  // the wave before walks the tile before (stash it)
  PipeStash* mine;                // this wave's stash (far-free)
  const PipeStash* next;          // the next wave's stash
  Raw kr[4], vr[4];     // own k/v rotation: slot of u is R
  Raw qr[4], gr[4];     // own q/dO rotation (key finalisation reads u-2 .. u)
  float lr[4];
  Raw fk[4], fv[4];     // far-right k/v rotation over i = u - 2 + F
  Raw kl[2], vl[2];     // far-left sources of query u
  Raw qi[2], gi[2];     // far query i of key u - 2
  float li_[2];
  float sp[4][3], sd[4][3];  // query u's near-slot p_n and scale * dS_n

  // Rows of step u.  The two warm-up steps before the tile (u < a) only
  // provide k and v (near sources of the first queries): their queries and
  // far rows feed nothing that is stored, so those loads are skipped
  // (load_at_if: zeros, no traffic), and so is the prefetch past the walk's
  // last step.
  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, Tm1);
    const bool walk = u <= last;
    const bool live = (u >= a || (!FAR && has_prev)) && walk;
    kr[R] = load_at_if<!FAR>(k, uc, walk);
    vr[R] = load_at_if<!FAR>(v, uc, walk);
    qr[R] = load_at_if<!FAR>(q, uc, live);
    gr[R] = load_at_if<!FAR>(go, uc, live);
    lr[R] = load_f32_if(lse, uc, live);
    if constexpr (FAR) {
      const int ul = clampi(u - F, Tm1);
      kl[R & 1] = load_at_if(k, ul, live);
      vl[R & 1] = load_at_if(v, ul, live);
      const int i = clampi(u - 2 + F, Tm1);
      fk[R] = load_at_if(k, i, live);
      fv[R] = load_at_if(v, i, live);
      qi[R & 1] = load_at_if(q, i, live);
      gi[R & 1] = load_at_if(go, i, live);
      li_[R & 1] = load_f32_if(lse, i, live);
    }
  }

  // Step u's rows from the next wave's stash (slot i = u - (a + P - 2)).
  template <int R>
  __device__ inline void prefetch_lds(int i, int lane) {
    kr[R] = unpack(next->row[i][0][lane]);
    vr[R] = unpack(next->row[i][1][lane]);
    qr[R] = unpack(next->row[i][2][lane]);
    gr[R] = unpack(next->row[i][3][lane]);
    lr[R] = next->lse[i][lane];
  }
  template <int R>
  __device__ inline void stash(int lane) {
    mine->row[R][0][lane] = pack(kr[R]);
    mine->row[R][1][lane] = pack(vr[R]);
    mine->row[R][2][lane] = pack(qr[R]);
    mine->row[R][3][lane] = pack(gr[R]);
    mine->lse[R][lane] = lr[R];
  }
  __device__ static inline u32x4 pack(const Raw& r) { return u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}; }
  __device__ static inline Raw unpack(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

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
  __shared__ PipeStash stash_lds[FAR ? 1 : kPipeWaves];
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int G = 64 / LPR, esz = (int)sizeof(T);
  const int h0 = wt.hg * G;
  const int lane = threadIdx.x & 63;
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
  w.last = last;
  bool next_adj = false;
  w.has_prev = false;
  if constexpr (!FAR) {
    // Neighbours in the workgroup on the tiles just before / after this one.
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t n = xcd_remap(blockIdx.x, gridDim.x, c.xs) * c.waves + wv;
    int b2, hg2, a2;
    if (wt.a < p.T && wv + 1 < c.waves && decode_tile(p, c, n + 1, b2, hg2, a2))
      next_adj = b2 == wt.b && hg2 == wt.hg && a2 == wt.a + c.P;
    if (wt.a < p.T && wv > 0 && decode_tile(p, c, n - 1, b2, hg2, a2))
      w.has_prev = b2 == wt.b && hg2 == wt.hg && a2 + c.P == wt.a;
    w.mine = &stash_lds[wv];
    w.next = &stash_lds[wv + 1 < kPipeWaves ? wv + 1 : wv];
  }
  w.template prefetch<0>(u0);
  // First trip: its rows (a - 2 .. a + 1) also go to the stash when the wave
  // before walks the tile before.
  __syncthreads();
  w.template prefetch<1>(u0 + 1);
  w.template compute<0>(u0);
  if (!FAR && w.has_prev) w.template stash<0>(lane);
  w.template prefetch<2>(u0 + 2);
  w.template compute<1>(u0 + 1);
  if (!FAR && w.has_prev) w.template stash<1>(lane);
  w.template prefetch<3>(u0 + 3);
  w.template compute<2>(u0 + 2);
  if (!FAR && w.has_prev) w.template stash<2>(lane);
  w.template prefetch<0>(u0 + 4);
  w.template compute<3>(u0 + 3);
  if (!FAR && w.has_prev) w.template stash<3>(lane);
  // Middle trips.
  const int ls = wt.a + c.P - 2;   // first of the last four steps
  for (int u = u0 + 4; u < ls - 4; u += 4) {
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
  // Last two trips (steps ls - 4 .. ls + 3): the last four steps' rows come
  // from the next wave's stash when it walks the next tile.
  const int u = ls - 4;
  if (!FAR && next_adj) {
    __syncthreads();
    w.template prefetch<1>(u + 1);
    w.template compute<0>(u);
    w.template prefetch<2>(u + 2);
    w.template compute<1>(u + 1);
    w.template prefetch<3>(u + 3);
    w.template compute<2>(u + 2);
    w.template prefetch_lds<0>(0, lane);
    w.template compute<3>(u + 3);
    __syncthreads();
    w.template prefetch_lds<1>(1, lane);
    w.template compute<0>(ls);
    w.template prefetch_lds<2>(2, lane);
    w.template compute<1>(ls + 1);
    w.template prefetch_lds<3>(3, lane);
    w.template compute<2>(ls + 2);
    w.template compute<3>(ls + 3);
  } else {
    __syncthreads();
    w.template prefetch<1>(u + 1);
    w.template compute<0>(u);
    w.template prefetch<2>(u + 2);
    w.template compute<1>(u + 1);
    w.template prefetch<3>(u + 3);
    w.template compute<2>(u + 2);
    w.template prefetch<0>(ls);
    w.template compute<3>(u + 3);
    __syncthreads();
    w.template prefetch<1>(ls + 1);
    w.template compute<0>(ls);
    w.template prefetch<2>(ls + 2);
    w.template compute<1>(ls + 1);
    w.template prefetch<3>(ls + 3);
    w.template compute<2>(ls + 2);
    w.template compute<3>(ls + 3);
  }
}

// ====================================== rotation backward (far offset 4)
//
// For F = 4 the far source of query u is the wave's own row u - 4 and the far
// query of key j is its own query j + 4: with rotations 6 deep (k/v for the
// query's sources, q/dO for the key's queries) a wave walks its tile alone,
// as the far-free walk does (8-wave lockstep groups over consecutive tiles);
// key j is finished at step j + 4.  Steps u = a - 4 .. a + P + 3 (the first
// four load only k/v), in trips of 6.  Same sums in the same order as the
// transposed chain (outputs bitwise identical); at T = 2^20, layer 3: 1.52 ->
// 1.39 ms.  (F = 8 would need rotations 10 deep: more registers than a lane
// has; it keeps the transposed chain.)

template <typename T, int LPR, int NM>
struct BwdFr4 {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + 1;
  static constexpr int FR = 4, RD = 6;

  Stream q, k, v, go, dq, dk, dv, lse;
  float scale;
  int T_, Tm1, a, end, last;
  PipeStash* mine;          // this wave's first four rows, for the wave before
  const PipeStash* next;    // the next wave's first four rows
  int stash_from;           // first row to stash (past the loop's steps: none)
  Raw kr[RD], vr[RD], qr[RD], gr[RD];
  float lr[RD];
  float sp[RD][3], sd[RD][3];

  template <int S>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, Tm1);
    const bool walk = u <= last;
    const bool live = u >= a && walk;
    kr[S] = load_at_if<true>(k, uc, walk);
    vr[S] = load_at_if<true>(v, uc, walk);
    qr[S] = load_at_if<true>(q, uc, live);
    gr[S] = load_at_if<true>(go, uc, live);
    lr[S] = load_f32_if(lse, uc, live);
  }
  // Row a + P + i (the next tile's row i) from the next wave's stash.
  template <int S>
  __device__ inline void prefetch_lds(int i, int lane) {
    kr[S] = unpack(next->row[i][0][lane]);
    vr[S] = unpack(next->row[i][1][lane]);
    qr[S] = unpack(next->row[i][2][lane]);
    gr[S] = unpack(next->row[i][3][lane]);
    lr[S] = next->lse[i][lane];
  }
  // Row a + i (slot R) into this wave's stash.
  template <int R>
  __device__ inline void stash(int i, int lane) {
    mine->row[i][0][lane] = pack(kr[R]);
    mine->row[i][1][lane] = pack(vr[R]);
    mine->row[i][2][lane] = pack(qr[R]);
    mine->row[i][3][lane] = pack(gr[R]);
    mine->lse[i][lane] = lr[R];
  }
  __device__ static inline u32x4 pack(const Raw& r) { return u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}; }
  __device__ static inline Raw unpack(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

  template <int R>
  __device__ inline void compute(int u) {
    const Raw* ks[NS];
    const Raw* vs[NS];
    bool ok[NS];
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        ks[idx] = &kr[(R + RD - n) % RD];
        vs[idx] = &vr[(R + RD - n) % RD];
        ok[idx] = u - n >= 0;
        ++idx;
      }
    }
    constexpr int sf = (R + RD - FR) % RD;
    ks[NS - 1] = &kr[sf];
    vs[NS - 1] = &vr[sf];
    ok[NS - 1] = u - FR >= 0;
    float pp[NS], ds[NS];
    {
      float dp[NS];
      float delta = 0.f;
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) {
        const float sc = row_sum<LPR>(dot_raw<T>(qr[R], *ks[s_])) * scale;
        dp[s_] = row_sum<LPR>(dot_raw<T>(gr[R], *vs[s_]));
        pp[s_] = ok[s_] ? fast_exp(sc - lr[R]) : 0.f;
        delta = __builtin_fmaf(pp[s_], dp[s_], delta);
      }
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) ds[s_] = pp[s_] * (dp[s_] - delta);
    }
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
      for (int s_ = 0; s_ < NS; ++s_) {
        float kx[VEC];
        widen<T>(*ks[s_], kx);
        const float c = ds[s_] * scale;
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(c, kx[e], g[e]);
      }
      store_at<T>(dq, u, g);
    }
    // Key j = u - 4: near queries j + n, far query u.
    const int j = u - FR;
    if (j >= a && j < end) {
      float ak[VEC], av[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) { ak[e] = 0.f; av[e] = 0.f; }
      int i2 = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + RD - FR + n) % RD;   // slot of query j + n
          const bool there = j + n < T_;
          const float cs = there ? sd[slot][i2] : 0.f;
          const float cp = there ? sp[slot][i2] : 0.f;
          float qx[VEC], gx[VEC];
          widen<T>(qr[slot], qx);
          widen<T>(gr[slot], gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
            av[e] = __builtin_fmaf(cp, gx[e], av[e]);
          }
          ++i2;
        }
      }
      const bool there = u < T_;
      const float cs = there ? ds[NS - 1] * scale : 0.f;
      const float cp = there ? pp[NS - 1] : 0.f;
      float qx[VEC], gx[VEC];
      widen<T>(qr[R], qx);
      widen<T>(gr[R], gx);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        ak[e] = __builtin_fmaf(cs, qx[e], ak[e]);
        av[e] = __builtin_fmaf(cp, gx[e], av[e]);
      }
      store_at<T>(dk, j, ak);
      store_at<T>(dv, j, av);
    }
  }

  // Steps R .. RD - 1 of the trip from u (slot of u + R is R); the steps of
  // rows stash_from .. stash_from + 3 also leave them in the stash.
  template <int R>
  __device__ inline void steps_stash(int u, int lane) {
    if constexpr (R < RD) {
      prefetch<(R + 1) % RD>(u + R + 1);
      compute<R>(u + R);
      const int i = u + R - stash_from;
      if (i >= 0 && i < 4) stash<R>(i, lane);
      steps_stash<R + 1>(u, lane);
    }
  }
};

// Tile sizes bwd_fr4's trip layout takes (see the kernel).
constexpr bool fr4_layout_ok(int P) { return P >= 14 && (P + 4) % 6 == 0; }

template <typename T, int LPR, int NM>
__global__ __launch_bounds__(kPipeBlock) void bwd_fr4(Params p, WalkCfg c) {
  __shared__ PipeStash stash_lds[kPipeWaves];
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int G = 64 / LPR, esz = (int)sizeof(T);
  const int h0 = wt.hg * G;
  using W = BwdFr4<T, LPR, NM>;
  W w;
  w.q = make_stream(p.q, esz, wt.b, h0, wt.hl, wt.li);
  w.k = make_stream(p.k, esz, wt.b, h0, wt.hl, wt.li);
  w.v = make_stream(p.v, esz, wt.b, h0, wt.hl, wt.li);
  w.go = make_stream(p.dout, esz, wt.b, h0, wt.hl, wt.li);
  w.dq = make_stream(p.dq, esz, wt.b, h0, wt.hl, wt.li);
  w.dk = make_stream(p.dk, esz, wt.b, h0, wt.hl, wt.li);
  w.dv = make_stream(p.dv, esz, wt.b, h0, wt.hl, wt.li);
  w.lse = lse_stream(p, wt.b, h0, wt.hl);
  w.scale = p.scale;
  w.T_ = p.T;
  w.Tm1 = p.T - 1;
  w.a = wt.a;
  w.end = min(wt.a + c.P, p.T);
  const int u0 = wt.a - W::FR;
  w.last = wt.a + c.P + W::FR - 1;
  // Trips of RD steps from u0 (slot of u is (u - u0) % RD); the trip count
  // depends only on P.
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Halo rows from LDS: the four rows after the tile (steps a + P .. a + P + 3)
  // are the first four rows of the next tile, which the next wave of the
  // workgroup loads at its start (long gone from L2 when this wave gets
  // there) and leaves in its stash.  The layout needs those steps to open the
  // last trip, after at least two looped ones (P + 4 a multiple of RD, P >=
  // 14: P = 32; the launch checks it).  At T = 2^20, layer 3: 1.40 -> 1.34 ms.
  constexpr int RD = W::RD;
  const int m = (c.P + 4) / RD;   // trip of step a + P
  bool next_adj = false, has_prev = false;
  {
    const int64_t n = xcd_remap(blockIdx.x, gridDim.x, c.xs) * c.waves + wv;
    int b2, hg2, a2;
    if (wt.a < p.T && wv + 1 < c.waves && decode_tile(p, c, n + 1, b2, hg2, a2))
      next_adj = b2 == wt.b && hg2 == wt.hg && a2 == wt.a + c.P;
    if (wt.a < p.T && wv > 0 && decode_tile(p, c, n - 1, b2, hg2, a2))
      has_prev = b2 == wt.b && hg2 == wt.hg && a2 + c.P == wt.a;
  }
  w.mine = &stash_lds[wv];
  w.next = &stash_lds[wv + 1 < kPipeWaves ? wv + 1 : wv];
  w.template prefetch<0>(u0);
  // Trips 0 .. m - 2; rows a .. a + 3 (steps 4 .. 7, in trips 0 and 1) also
  // go to the stash when the wave before walks the tile before.
  const int um = u0 + (m - 1) * RD;   // trip m - 1
  w.stash_from = has_prev ? wt.a : wt.a + c.P + 8;   // past every step of the loop: no write
  for (int u = u0; u < um; u += RD) {
    __syncthreads();
    w.template steps_stash<0>(u, lane);
  }
  // Trips m - 1 and m (steps a + P .. a + P + 3 open trip m; its last two
  // steps lie past the walk and are skipped).
  const int ul = um + RD;
  if (next_adj) {
    __syncthreads();
    w.template prefetch<1>(um + 1);
    w.template compute<0>(um);
    w.template prefetch<2>(um + 2);
    w.template compute<1>(um + 1);
    w.template prefetch<3>(um + 3);
    w.template compute<2>(um + 2);
    w.template prefetch<4>(um + 4);
    w.template compute<3>(um + 3);
    w.template prefetch<5>(um + 5);
    w.template compute<4>(um + 4);
    w.template prefetch_lds<0>(0, lane);
    w.template compute<5>(um + 5);
    __syncthreads();
    w.template prefetch_lds<1>(1, lane);
    w.template compute<0>(ul);
    w.template prefetch_lds<2>(2, lane);
    w.template compute<1>(ul + 1);
    w.template prefetch_lds<3>(3, lane);
    w.template compute<2>(ul + 2);
    w.template compute<3>(ul + 3);
  } else {
    __syncthreads();
    w.template prefetch<1>(um + 1);
    w.template compute<0>(um);
    w.template prefetch<2>(um + 2);
    w.template compute<1>(um + 1);
    w.template prefetch<3>(um + 3);
    w.template compute<2>(um + 2);
    w.template prefetch<4>(um + 4);
    w.template compute<3>(um + 3);
    w.template prefetch<5>(um + 5);
    w.template compute<4>(um + 4);
    w.template prefetch<0>(ul);
    w.template compute<5>(um + 5);
    __syncthreads();
    w.template prefetch<1>(ul + 1);
    w.template compute<0>(ul);
    w.template prefetch<2>(ul + 2);
    w.template compute<1>(ul + 1);
    w.template prefetch<3>(ul + 3);
    w.template compute<2>(ul + 2);
    w.template compute<3>(ul + 3);
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

  // As BwdPipe::prefetch: the warm-up steps (u < a) load only k and v.
  // Their q / dO rows are still published (zeros) and read by nobody who
  // stores: wave w - 1 finishes its keys j from this wave's queries j + F,
  // all of them at or after a.
  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, Tm1);
    const bool live = u >= a;
    // Own rows: k/v cached where the chain above or below reads them (first
    // and last wave), q/dO where the chain above does (first wave).  (Buffer
    // loads here, to skip the prefetch past the last step, measured 5-10%
    // slower: four more buffer resources on a kernel that already spills
    // scalar registers.)
    kr[R] = load_at<LEFT_LDS && RIGHT_LDS>(k, uc);
    vr[R] = load_at<LEFT_LDS && RIGHT_LDS>(v, uc);
    qr[R] = load_at_if<LEFT_LDS>(q, uc, live);
    gr[R] = load_at_if<LEFT_LDS>(go, uc, live);
    lr[R] = load_f32_if(lse, uc, live);
    if constexpr (!LEFT_LDS) {
      const int ul = clampi(u - F, Tm1);
      kl[R & 1] = load_at_if(k, ul, live);
      vl[R & 1] = load_at_if(v, ul, live);
    }
    if constexpr (!RIGHT_LDS) {
      const int i = clampi(u - 2 + F, Tm1);
      fk[R] = load_at_if(k, i, live);
      fv[R] = load_at_if(v, i, live);
      qi[R & 1] = load_at_if(q, i, live);
      gi[R & 1] = load_at_if(go, i, live);
      li_[R & 1] = load_f32_if(lse, i, live);
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
    // u = a-2 .. a+P+1 for every wave of the workgroup (same trip count); the
    // last trip issues no prefetch past the walk.
    const int u0 = steps_from;
    prefetch<0>(u0);
    int u = u0;
    for (; u + 3 < end_u; u += 4) {
      prefetch<1>(u + 1);
      compute<0>(u);
      prefetch<2>(u + 2);
      compute<1>(u + 1);
      prefetch<3>(u + 3);
      compute<2>(u + 2);
      prefetch<0>(u + 4);
      compute<3>(u + 3);
    }
    prefetch<1>(u + 1);
    compute<0>(u);
    prefetch<2>(u + 2);
    compute<1>(u + 1);
    prefetch<3>(u + 3);
    compute<2>(u + 2);
    compute<3>(u + 3);
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
  // Workgroup -> (batch, head group, band group, row block), XCD-contiguous,
  // row blocks or band groups fastest; wave w -> row w % L of the block, band
  // w / L of the group.
  int64_t g = xcd_remap(blockIdx.x, gridDim.x, c.xs);
  int rb, bgi;
  if (c.band_fast) {
    bgi = (int)(g % c.bgroups);
    g /= c.bgroups;
    rb = (int)(g % c.blocks);
    g /= c.blocks;
  } else {
    rb = (int)(g % c.blocks);
    g /= c.blocks;
    bgi = (int)(g % c.bgroups);
    g /= c.bgroups;
  }
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

// ============================================ transposed chain (far = 8)
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

  // Rows r0 - 1 .. r0 + R are used (sources of the first row, queries of the
  // last keys); the walk's alignment steps before and after them load
  // nothing (load_at_if: zeros, no traffic).
  template <int K>
  __device__ inline void prefetch(int r) {
    const int t = clampi(r * F + c, Tm1);
    const bool used = r >= r0 - 1 && r <= r0 + R;
    kr[K] = load_at_if<true>(k, t, used);
    vr[K] = load_at_if<true>(v, t, used);
    qr[K] = load_at_if<true>(q, t, used);
    gr[K] = load_at_if<true>(go, t, used);
    lr[K] = load_f32_if(lse, t, used);
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

template <typename T, int LPR, int NM>
hipError_t launch_chain(const Params& p, const WalkCfg& wc, hipStream_t st) {
  const int64_t stride = p.q.st * (int64_t)sizeof(T);
  const bool pairs = chain_pairs_apply(wc, stride);
  ChainCfg c = make_chain_cfg(p.B, stride, wc, pairs);
  if (c.nwg <= 0) return hipErrorInvalidValue;
  const int64_t fs = (int64_t)c.F * stride;
  c.xs = xcd_stagger(c.nwg, fs, false);
  // Row pairs at 1-4 MiB row strides take the band groups of a row block
  // first: an XCD's workgroups then stream whole rows (contiguous memory)
  // instead of the same columns of many rows.  At T = 2^20, layer 11 1.386 ->
  // 1.362 ms and layer 12 1.496 -> 1.422 ms (two repetitions); at 512 KiB and
  // from 4 MiB it measured equal or slower (layer 14: 1.42 -> 1.79 ms), and
  // so did the forward's row groups (layer 12: 0.771 -> 0.785 ms).
  c.band_fast = pairs && fs >= ((int64_t)1 << 20) && fs < ((int64_t)4 << 20);
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


}  // namespace

hipError_t launch_bwd(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype, int lpr,
                      hipStream_t st) {
  return by_type_lpr(dtype, lpr, [&](auto tag, auto lprc) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int L = decltype(lprc)::value;
    if (pat.far != 0 && c.column)
      return pat.nm == 7 ? launch_chain<T, L, 7>(p, c, st) : launch_chain<T, L, 1>(p, c, st);
    const dim3 grid((unsigned)c.nwg), block(kPipeBlock);
    if (pat.far == 4 && !c.column) {
      if (!fr4_layout_ok(c.P)) return hipErrorInvalidValue;
      // Static LDS (the halo stash, 136 KiB) keeps one workgroup per CU.
      if (pat.nm == 7) hipLaunchKernelGGL((bwd_fr4<T, L, 7>), grid, block, 0, st, p, c);
      else hipLaunchKernelGGL((bwd_fr4<T, L, 1>), grid, block, 0, st, p, c);
      return hipGetLastError();
    }
    if (pat.far == 8 && !c.column)
      return pat.nm == 7 ? launch_tc<T, L, 7, 8>(p, c, st) : launch_tc<T, L, 1, 8>(p, c, st);
    // The far-free walks hold their stashes in static LDS (136 KiB: one
    // workgroup per CU without the extra allocation).
    if (pat.far == 0 && pat.nm == 3)
      hipLaunchKernelGGL((bwd_pipe<T, L, 3, false>), grid, block, 0, st, p, c);
    else if (pat.far == 0 && pat.nm == 5)
      hipLaunchKernelGGL((bwd_pipe<T, L, 5, false>), grid, block, 0, st, p, c);
    else if (pat.far != 0 && pat.nm == 7)
      hipLaunchKernelGGL((bwd_pipe<T, L, 7, true>), grid, block, kPipeLds, st, p, c);
    else if (pat.far != 0 && pat.nm == 1)
      hipLaunchKernelGGL((bwd_pipe<T, L, 1, true>), grid, block, kPipeLds, st, p, c);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  });
}

}  // namespace walk
}  // namespace sbda
