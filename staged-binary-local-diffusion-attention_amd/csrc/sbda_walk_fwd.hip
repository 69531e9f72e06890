// Forward walks (fwd_pipe): scores against the near rows and the far row,
// softmax, O and one log-normaliser per row.  Reference semantics:
// BiAttn/left_v2.py:313-405.

#include "sbda_walk.h"

namespace sbda {
namespace walk {

namespace {

// FR > 0: the far offset is the compile-time constant FR (4 or 8) and the far
// row is taken from the rotation (depth FR + 2) instead of being loaded: a
// row loaded FR steps earlier is long gone from L2 at the streaming rate.
// The rows a wave loads before its tile (the warm-up steps: H = 2, or FR for
// a rotation far source) are the last H rows of the tile before it.  A wave
// whose left neighbour in the workgroup walks that tile leaves their k and v
// here, and the neighbour takes its last H steps' k/v from LDS instead of
// loading them a second time (long gone from L2 by then).  Linear tiles
// only (far-free and rotation walks; at T = 2^20 layers 3 and 4: 0.746 ->
// 0.724 and 0.774 -> 0.731 ms): the walks with loaded far rows measured
// 3-6% slower with it.
template <int H>
struct FwdStash {
  u32x4 kv[H][2][64];   // [warm-up step][k, v][lane]
};

template <typename T, int LPR, int NM, bool FAR, int FR>
struct FwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);
  static constexpr int RD = FR > 0 ? FR + 2 : 4;   // rotation depth (even)
  static_assert(FR == 0 || FAR, "a rotation far source needs a far slot");

  static constexpr int H = FR > 2 ? FR : 2;        // warm-up steps
  static constexpr bool STASH = !FAR || FR > 0;     // linear tiles
  using Stash = FwdStash<H>;

  Stream q, k, v, o, lse;
  float scale;
  int F, Tm1, li, lane;
  int a_, ls;            // tile start; first position whose k/v come from the next stash
  bool has_prev, next_adj;
  Stash* mine;
  const Stash* next;
  Raw kr[RD];           // k at t (slot R), t-1, ...; slot R+1 is being fetched
  Raw vraw[2], qn[2];   // this step's v and q (stage R & 1)
  Raw kl[2], vl[2];     // far source t - F (FR == 0)
  float vr[RD][VEC];    // widened v rotation

  // Defined contents for slots a skipped load leaves stale.
  __device__ inline void init() {
#pragma unroll
    for (int i = 0; i < RD; ++i) kr[i] = Raw{};
#pragma unroll
    for (int i = 0; i < 2; ++i) vraw[i] = qn[i] = kl[i] = vl[i] = Raw{};
  }

  // Rows of position t.  A query row (and its far source) only for positions
  // the tile stores (q_ok); k and v also for the warm-up positions before the
  // tile, whose rows are the first queries' sources, but not past its end
  // (kv_ok).  A skipped row reads zeros and moves no bytes (load_at_if); only
  // steps that store nothing read such a slot.
  template <int R>
  __device__ inline void prefetch(int t, bool q_ok, bool kv_ok) {
    const int tc = clampi(t, Tm1);
    if constexpr (STASH) kv_ok = kv_ok && !(next_adj && t >= ls);   // from the next stash
    kr[R] = load_at_if<!FAR>(k, tc, kv_ok);
    vraw[R & 1] = load_at_if<!FAR>(v, tc, kv_ok);
    qn[R & 1] = load_at_if<true>(q, tc, q_ok);
    if constexpr (FAR && FR == 0) {
      const int tf = clampi(t - F, Tm1);
      kl[R & 1] = load_at_if(k, tf, q_ok);
      vl[R & 1] = load_at_if(v, tf, q_ok);
    }
  }

  template <int R>
  __device__ inline void compute(int t, bool store) {
    if constexpr (STASH) {
      if (next_adj && t >= ls) {
        kr[R] = unpack(next->kv[t - ls][0][lane]);
        vraw[R & 1] = unpack(next->kv[t - ls][1][lane]);
      }
      if (has_prev && t < a_) {
        mine->kv[t - (a_ - H)][0][lane] = pack(kr[R]);
        mine->kv[t - (a_ - H)][1][lane] = pack(vraw[R & 1]);
      }
    }
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
    // l >= 1 whenever a source is valid (the largest term is exp(0)).
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= inv;
    if (store) {
      store_at<T>(o, t, acc);
      if (li == 0) store_f32(lse, t, l > 0.f ? m + fast_log(l) : INFINITY);
    }
  }

  __device__ static inline u32x4 pack(const Raw& r) { return u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}; }
  __device__ static inline Raw unpack(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

  // Steps R .. RD-1 of one trip around the rotation (position of slot 0 is t).
  template <int R>
  __device__ inline void steps(int t, int a, int end) {
    if constexpr (R < RD) {
      const int n = t + R + 1;
      prefetch<(R + 1) % RD>(n, n >= a && n < end, n < end);
      compute<R>(t + R, t + R >= a && t + R < end);
      steps<R + 1>(t, a, end);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR, int FR>
__global__ __launch_bounds__(kPipeBlock) void fwd_pipe(Params p, WalkCfg c) {
  using W = FwdPipe<T, LPR, NM, FAR, FR>;
  constexpr bool STASH = W::STASH;
  __shared__ FwdStash<(FR > 2 ? FR : 2)> stash[STASH ? kPipeWaves : 1];
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  constexpr int G = 64 / LPR, esz = (int)sizeof(T);
  const int h0 = wt.hg * G;
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
  w.lane = threadIdx.x & 63;
  const int a = wt.a, end = min(a + c.P, p.T);
  // The tile before / after this one, when a wave of this workgroup walks
  // it (linear tiles: the next wave; head groups interleave the waves, so
  // only for one head group).
  if constexpr (STASH) {
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int d = (c.HG == 1 && !c.column) ? 1 : 0;
    w.has_prev = w.next_adj = false;
    if (d && a < p.T) {
      const int64_t n = xcd_remap(blockIdx.x, gridDim.x, c.xs) * c.waves + wv;
      int b2, hg2, a2;
      if (wv + d < c.waves && decode_tile(p, c, n + d, b2, hg2, a2))
        w.next_adj = b2 == wt.b && a2 == a + c.P;
      if (wv - d >= 0 && decode_tile(p, c, n - d, b2, hg2, a2))
        w.has_prev = b2 == wt.b && a2 + c.P == a;
    }
    w.a_ = a;
    w.ls = a + c.P - W::H;
    w.mine = &stash[wv];
    w.next = &stash[wv + d < kPipeWaves ? wv + d : wv];
  }
  // The walk starts early enough to fill the rotation (2 positions, or FR
  // for a rotation far source); those steps store nothing.  Slot of
  // position t is (t - t0) % RD.
  // The trip count depends only on P (same for every wave of the workgroup).
  const int t0 = a - (FR > 2 ? FR : 2);
  w.init();
  w.template prefetch<0>(t0, false, t0 < end);
  for (int t = t0; t < a + c.P; t += W::RD) {
    __syncthreads();
    w.template steps<0>(t, a, end);
  }
}


}  // namespace

// Dynamic LDS that, with the kernel's stashes, keeps one workgroup per CU.
template <bool FAR, int FR>
constexpr unsigned fwd_extra_lds() {
  constexpr unsigned s = sizeof(FwdStash<(FR > 2 ? FR : 2)>) * ((!FAR || FR > 0) ? kPipeWaves : 1);
  return s >= kPipeLds ? 0u : kPipeLds - s;
}

template <typename T, int LPR, int NM, bool FAR>
hipError_t fwd_pattern(const Params& p, const WalkCfg& c, const Pattern& pat, hipStream_t st) {
  const dim3 grid((unsigned)c.nwg), block(64 * c.waves);
  if constexpr (FAR) {
    if (pat.far == 4 && !c.column) {
      hipLaunchKernelGGL((fwd_pipe<T, LPR, NM, true, 4>), grid, block, (fwd_extra_lds<true, 4>()), st, p, c);
      return hipGetLastError();
    }
    if (pat.far == 8 && !c.column) {
      hipLaunchKernelGGL((fwd_pipe<T, LPR, NM, true, 8>), grid, block, (fwd_extra_lds<true, 8>()), st, p, c);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((fwd_pipe<T, LPR, NM, FAR, 0>), grid, block, (fwd_extra_lds<FAR, 0>()), st, p, c);
  return hipGetLastError();
}

hipError_t launch_fwd(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype, int lpr,
                      hipStream_t st) {
  return by_type_lpr(dtype, lpr, [&](auto tag, auto lprc) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int L = decltype(lprc)::value;
    if (pat.far == 0) {
      if (pat.nm == 3) return fwd_pattern<T, L, 3, false>(p, c, pat, st);
      if (pat.nm == 5) return fwd_pattern<T, L, 5, false>(p, c, pat, st);
    } else {
      if (pat.nm == 7) return fwd_pattern<T, L, 7, true>(p, c, pat, st);
      if (pat.nm == 1) return fwd_pattern<T, L, 1, true>(p, c, pat, st);
    }
    return hipErrorInvalidValue;
  });
}

}  // namespace walk
}  // namespace sbda
