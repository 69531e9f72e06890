// Walks with the fused head-RMSNorm + RoPE prologue (BiAttn/left_v2.py:237-239,
// BiAttn/attention_common.py:25-50,64-76): forward and the two-pass backward.

#include "sbda_walk.h"

namespace sbda {
namespace walk {

namespace {

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
  // A walk row is LPR lanes of 16 bytes, so the head dimension is a
  // compile-time power of two and the norm's mean is an exact scaling.
  static constexpr int D = 16 * LPR / (int)sizeof(T);
  Stream rc, rs;   // fp32 [T, D/2] RoPE tables: this lane's HV entries of a position
  float eps;
  int li, Tm1;
  float wq[VEC], wk[VEC];

  __device__ inline void init(const Params& p, int lane_in_row) {
    li = lane_in_row;
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
    // l >= 1 whenever a source is valid (the largest term is exp(0)).
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
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
  // Steps first .. last (a multiple of 4 of them); the last trip issues no
  // prefetch past the walk.
  w.template prefetch<0>(first);
  int u = first;
  for (; u + 3 < last; u += 4) {
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
  __syncthreads();
  w.template prefetch<1>(u + 1);
  w.template compute<0>(u);
  w.template prefetch<2>(u + 2);
  w.template compute<1>(u + 1);
  w.template prefetch<3>(u + 3);
  w.template compute<2>(u + 2);
  w.template compute<3>(u + 3);
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


// ---- fused single-pass backward (far-free patterns)
//
// One walk per row as in the plain backward: each query's weights and score
// gradients once, dQ through the transposed prologue at once, key j = u - 2
// finalised from queries j, j + 1, j + 2 (roped q rows kept in registers),
// then dK through the transposed prologue.  No weight table in global memory.
// (A lockstep row-chain version for far offsets measured slower than the
// two-pass backward -- 256 VGPRs with spills and five prologue applications
// per step -- so far offsets keep the two passes.)


template <typename T, int LPR, int NM>
struct BwdFusedPro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using PL = typename B_::PL;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN;

  SplitStream q, k, v, go, dq, dk, dv;
  Stream lse;
  float scale;
  int T_, a, end;
  Raw kr[4], vr[4], gr[4];    // raw k (self slot and dK), v, dO rotations
  Raw qr[2];                  // raw q of this step
  float lr[2];
  float kh[4][VEC];           // roped k rotation (near sources)
  float qh[4][VEC];           // roped q rotation (near queries of a key)
  float rk[4];                // k norm factors
  float sp[4][3], sd[4][3];   // query's near-slot p_n and scale * dS_n
  float dwq[VEC], dwk[VEC];

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, this->Tm1);
    kr[R] = load_split<true>(k, uc);
    vr[R] = load_split<true>(v, uc);
    qr[R & 1] = load_split<true>(q, uc);
    gr[R] = load_split<true>(go, uc);
    lr[R & 1] = load_f32(lse, uc);
  }

  template <int R>
  __device__ inline void compute(int u) {
    float cu[HV], su[HV];
    this->cs(clampi(u, this->Tm1), cu, su);
    rk[R] = this->rope(kr[R], this->wk, cu, su, kh[R]);
    float qx[VEC];
    widen<T>(qr[R & 1], qx);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qh[R][e] = qx[e];
    const float rq = PL::forward_w(qh[R], this->wq, cu, su, this->D, this->eps);
    {
      const float* ks[NS];
      const Raw* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          ks[idx] = kh[(R + 4 - n) & 3];
          vs[idx] = &vr[(R + 4 - n) & 3];
          ok[idx] = u - n >= 0;
          ++idx;
        }
      }
      float pp[NS], dp[NS], delta = 0.f;
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) {
        float a_ = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) a_ = __builtin_fmaf(qh[R][e], ks[s_][e], a_);
        const float sc = row_sum<LPR>(a_) * scale;
        dp[s_] = row_sum<LPR>(dot_raw<T>(gr[R], *vs[s_]));
        pp[s_] = ok[s_] ? fast_exp(sc - lr[R & 1]) : 0.f;
        delta = __builtin_fmaf(pp[s_], dp[s_], delta);
      }
      float ds[NS];
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) ds[s_] = pp[s_] * (dp[s_] - delta) * scale;
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        sp[R][n] = pp[n];
        sd[R][n] = ds[n];
      }
      if (u >= a && u < end) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
        for (int s_ = 0; s_ < NS; ++s_) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(ds[s_], ks[s_][e], g[e]);
        }
        PL::backward_w(g, qx, rq, this->wq, cu, su, this->D, dwq);
        store_split<T>(dq, u, g);
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
          const int slot = (R + 2 + n) & 3;   // query j + n
          const bool there = j + n < T_;
          const float cs_ = there ? sd[slot][idx] : 0.f;
          const float cp_ = there ? sp[slot][idx] : 0.f;
          float gx[VEC];
          widen<T>(gr[slot], gx);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs_, qh[slot][e], ak[e]);
            av[e] = __builtin_fmaf(cp_, gx[e], av[e]);
          }
          ++idx;
        }
      }
      float kx[VEC], cj[HV], sj[HV];
      widen<T>(kr[(R + 2) & 3], kx);
      this->cs(clampi(j, this->Tm1), cj, sj);
      PL::backward_w(ak, kx, rk[(R + 2) & 3], this->wk, cj, sj, this->D, dwk);
      store_split<T>(dk, j, ak);
      store_split<T>(dv, j, av);
    }
  }
};

// Far-free patterns: lockstep 8-wave workgroups over consecutive tiles (the
// same decode and trip counts as the other pipelined walks).
template <typename T, int LPR, int NM>
__global__ __launch_bounds__(kPipeBlock) void bwd_fused_pro(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value, esz = (int)sizeof(T);
  WaveTile wt;
  wave_tile<LPR>(p, c, wt);
  const int h0 = wt.hg * (64 / LPR);
  BwdFusedPro<T, LPR, NM> x;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    x.dwq[e] = 0.f;
    x.dwk[e] = 0.f;
  }
  x.init(p, wt.li);
  x.q = make_split(p.q, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.k = make_split(p.k, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.v = make_split(p.v, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.go = make_split(p.dout, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.dq = make_split(p.dq, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.dk = make_split(p.dk, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.dv = make_split(p.dv, esz, wt.b, h0, wt.hl, wt.li, p.D, x.HV);
  x.lse = lse_stream(p, wt.b, h0, wt.hl);
  x.scale = p.scale;
  x.T_ = p.T;
  x.a = wt.a;
  x.end = min(wt.a + c.P, p.T);
  // u = a-2 .. a+P+1 (slot of u is (u - a + 2) & 3); the trip count depends only on P.
  walk4(x, wt.a - 2, wt.a + c.P + 1);
  const int64_t wave = pipe_wave_id(c);
  write_wave_partial<T, LPR, true>(x.dwq, p.dwq_part, wave, p.D);
  write_wave_partial<T, LPR, true>(x.dwk, p.dwk_part, wave, p.D);
}

// ===================================== chained backward, fused prologue (F >= 16)
//
// Far offsets F >= 16 that tile the sequence into rows (t = r * F + c): a
// workgroup of W waves walks W consecutive rows of one column band in
// lockstep, one barrier per step, as the plain chained backward does, and
// every raw q/k row gets the prologue once, when it arrives.  Wave w
// publishes in LDS its roped k and raw v rows (wave w + 1's far-left sources,
// read in the same step) and its roped q, raw dO and far-slot weights
// (wave w - 1's far-key contribution, read two steps later).  The first wave
// of a chain loads and ropes its far-left rows.  The keys of the last wave
// whose far query lies in the next chain's first row are finished by
// bwd_fix_pro: the last wave stores their near-slot dK' and dV (fp32, before
// the transposed prologue), the next chain's first wave stores those far
// queries' weight pairs, and bwd_fix_pro adds the far term and applies the
// transposed prologue -- the same sums in the same order as a key finished in
// one pass.  Every wave runs the same trip count (rows past the end walk
// clamped rows and store nothing), so all barriers are reached.

constexpr int kProRing = 4;   // q/dO/weight ring: written at step u, read at u + 2

template <int VEC>
struct ChainProSlot {
  float4 kf[2][VEC / 4][64];         // [u & 1][quarter][lane]: roped k of position u
  u32x4 vf[2][64];                   // [u & 1][lane]: raw v
  float4 qf[kProRing][VEC / 4][64];  // [u & 3][quarter][lane]: roped q
  u32x4 gf[kProRing][64];            // [u & 3][lane]: raw dO
  float2 pc[kProRing][16];           // [u & 3][head]: (p_far, scale * dS_far) of query u
};

__device__ inline u32x4 pack_raw(const Raw& r) { return u32x4{r.w[0], r.w[1], r.w[2], r.w[3]}; }
__device__ inline Raw unpack_raw(const u32x4& x) { return Raw{{x.x, x.y, x.z, x.w}}; }

template <int VEC>
__device__ inline void put_rows(float4 (&dst)[VEC / 4][64], int lane, const float (&x)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC / 4; ++i)
    dst[i][lane] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
}

template <int VEC>
__device__ inline void get_rows(const float4 (&src)[VEC / 4][64], int lane, float (&x)[VEC]) {
#pragma unroll
  for (int i = 0; i < VEC / 4; ++i) {
    const float4 v = src[i][lane];
    x[4 * i] = v.x;
    x[4 * i + 1] = v.y;
    x[4 * i + 2] = v.z;
    x[4 * i + 3] = v.w;
  }
}

// RoPE cos/sin of the last 4 positions a wave walked, in LDS: [u & 3][lane
// in row][cos (HV), sin (HV)].  A position's entries are loaded with the rows
// one step ahead and stashed here once they arrive, so no table load sits
// inside a step: such a load (its result needed at once) made every step wait
// for the next step's row loads too, serialising load latency and VALU work.
template <int LPR, int HV>
using CsRing = float[4][LPR][2 * HV];

template <typename T, int LPR, int NM, bool LEFT_LDS, bool RIGHT_LDS, bool RING>
struct BwdChainPro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using PL = typename B_::PL;
  using Slot = ChainProSlot<VecOf<T>::value>;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + 1;

  SplitStream q, k, v, go, dq, dk, dv;
  Stream lse;
  float scale;
  int F, T_, a, end, lane, hl;
  Slot* mine;
  const Slot* up;      // wave w - 1 (far-left provider)
  const Slot* down;    // wave w + 1 (far-right provider)
  float4* defer;       // last wave: deferred dK'/dV slots of its band's columns
  float2* defer_pc;    // first wave: far weight pairs of the previous chain's deferred keys
  Raw kr[4], vr[4], gr[4];
  Raw qr[2];
  float lr[2];
  Raw kl[2], vl[2];            // far-left raw rows of query u (first wave)
  float clc[2][HV], cls[2][HV];
  float cpf[HV], spf[HV];      // cos/sin of the position in flight (RING)
  float (*ring)[LPR][2 * HV];  // this wave's CsRing (RING)
  float kh[4][VEC];            // roped k rotation
  float qh[VEC];               // roped q of this step (earlier steps' rows: mine->qf)
  float rk[4];
  float sp[4][3], sd[4][3];
  float dwq[VEC], dwk[VEC];

  template <int R>
  __device__ inline void prefetch(int u) {
    const int uc = clampi(u, this->Tm1);
    kr[R] = load_split(k, uc);
    vr[R] = load_split(v, uc);
    qr[R & 1] = load_split(q, uc);
    gr[R] = load_split(go, uc);
    lr[R & 1] = load_f32(lse, uc);
    if constexpr (!LEFT_LDS) {
      const int ul = clampi(u - F, this->Tm1);
      kl[R & 1] = load_split(k, ul);
      vl[R & 1] = load_split(v, ul);
      this->cs(ul, clc[R & 1], cls[R & 1]);
    }
    if constexpr (RING) this->cs(uc, cpf, spf);
  }

  // The arrived cos/sin of step R's position into the ring (before the next
  // prefetch reuses cpf/spf).  The first head's lanes write and every lane
  // reads: a wavefront-scope fence orders those cross-lane LDS accesses (no
  // wait is needed within one wave, but the compiler must not move the reads
  // above the writes).
  template <int R>
  __device__ inline void stash() {
    if constexpr (RING) {
      if (hl == 0) {
#pragma unroll
        for (int i = 0; i < HV; ++i) {
          ring[R][this->li][i] = cpf[i];
          ring[R][this->li][HV + i] = spf[i];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // cos/sin of step R's position (u clamped into the sequence).
  template <int R>
  __device__ inline void cs_of(int u, float (&c)[HV], float (&s)[HV]) const {
    if constexpr (RING) {
#pragma unroll
      for (int i = 0; i < HV; ++i) {
        c[i] = ring[R][this->li][i];
        s[i] = ring[R][this->li][HV + i];
      }
    } else {
      this->cs(clampi(u, this->Tm1), c, s);
    }
  }

  // dK' -> dK through the transposed prologue, then both rows out.
  template <int R>
  __device__ inline void finish_key(int j, float (&ak)[VEC], const float (&av)[VEC]) {
    float kx[VEC], cj[HV], sj[HV];
    widen<T>(kr[(R + 2) & 3], kx);
    cs_of<(R + 2) & 3>(j, cj, sj);
    PL::backward_w(ak, kx, rk[(R + 2) & 3], this->wk, cj, sj, this->D, dwk);
    store_split<T>(dk, j, ak);
    store_split<T>(dv, j, av);
  }

  template <int R>
  __device__ inline void compute(int u) {
    float cu[HV], su[HV];
    cs_of<R>(u, cu, su);
    rk[R] = this->rope(kr[R], this->wk, cu, su, kh[R]);
    float qx[VEC];
    widen<T>(qr[R & 1], qx);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qh[e] = qx[e];
    const float rq = PL::forward_w(qh, this->wq, cu, su, this->D, this->eps);
    // Publish this step's rows, then wait for the neighbours'.
    put_rows<VEC>(mine->kf[R & 1], lane, kh[R]);
    mine->vf[R & 1][lane] = pack_raw(vr[R]);
    put_rows<VEC>(mine->qf[R], lane, qh);
    mine->gf[R][lane] = pack_raw(gr[R]);
    __syncthreads();
    float kfar[VEC];
    Raw vfar;
    if constexpr (LEFT_LDS) {
      get_rows<VEC>(up->kf[R & 1], lane, kfar);
      vfar = unpack_raw(up->vf[R & 1][lane]);
    } else {
      this->rope(kl[R & 1], this->wk, clc[R & 1], cls[R & 1], kfar);
      vfar = vl[R & 1];
    }
    {
      const float* ks[NS];
      const Raw* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          ks[idx] = kh[(R + 4 - n) & 3];
          vs[idx] = &vr[(R + 4 - n) & 3];
          ok[idx] = u - n >= 0;
          ++idx;
        }
      }
      ks[NS - 1] = kfar;
      vs[NS - 1] = &vfar;
      ok[NS - 1] = u - F >= 0;
      float pp[NS], dp[NS], delta = 0.f;
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) {
        float a_ = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) a_ = __builtin_fmaf(qh[e], ks[s_][e], a_);
        const float sc = row_sum<LPR>(a_) * scale;
        dp[s_] = row_sum<LPR>(dot_raw<T>(gr[R], *vs[s_]));
        pp[s_] = ok[s_] ? fast_exp(sc - lr[R & 1]) : 0.f;
        delta = __builtin_fmaf(pp[s_], dp[s_], delta);
      }
      float ds[NS];
#pragma unroll
      for (int s_ = 0; s_ < NS; ++s_) ds[s_] = pp[s_] * (dp[s_] - delta) * scale;
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        sp[R][n] = pp[n];
        sd[R][n] = ds[n];
      }
      const float2 far_w = make_float2(pp[NS - 1], ds[NS - 1]);
      if (this->li == 0) mine->pc[R][hl] = far_w;
      if constexpr (!LEFT_LDS) {
        if (defer_pc != nullptr && u >= a && u < end && this->li == 0)
          defer_pc[(int64_t)(u - a) * (64 / LPR) + hl] = far_w;
      }
      if (u >= a && u < end) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) g[e] = 0.f;
#pragma unroll
        for (int s_ = 0; s_ < NS; ++s_) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) g[e] = __builtin_fmaf(ds[s_], ks[s_][e], g[e]);
        }
        PL::backward_w(g, qx, rq, this->wq, cu, su, this->D, dwq);
        store_split<T>(dq, u, g);
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
          const int slot = (R + 2 + n) & 3;   // query j + n
          const bool there = j + n < T_;
          const float cs_ = there ? sd[slot][idx] : 0.f;
          const float cp_ = there ? sp[slot][idx] : 0.f;
          float gx[VEC], qs[VEC];
          widen<T>(gr[slot], gx);
          if (slot == R) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) qs[e] = qh[e];
          } else {
            get_rows<VEC>(mine->qf[slot], lane, qs);   // this wave's own earlier row
          }
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[e] = __builtin_fmaf(cs_, qs[e], ak[e]);
            av[e] = __builtin_fmaf(cp_, gx[e], av[e]);
          }
          ++idx;
        }
      }
      const bool there = j + F < T_;
      if constexpr (RIGHT_LDS) {
        // Query j + F is wave w + 1's query of step u - 2.
        const int sl = (R + 2) & 3;
        const float2 w2 = down->pc[sl][hl];
        float qf[VEC], gx[VEC];
        get_rows<VEC>(down->qf[sl], lane, qf);
        widen<T>(unpack_raw(down->gf[sl][lane]), gx);
        const float cs_ = there ? w2.y : 0.f;
        const float cp_ = there ? w2.x : 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          ak[e] = __builtin_fmaf(cs_, qf[e], ak[e]);
          av[e] = __builtin_fmaf(cp_, gx[e], av[e]);
        }
        finish_key<R>(j, ak, av);
      } else {
        if (there && defer != nullptr) {
          // Far query in the next chain: bwd_fix_pro finishes this key.
          float4* slot = defer + (int64_t)(j - a) * (2 * (VEC / 4) * 64);
#pragma unroll
          for (int i = 0; i < VEC / 4; ++i) {
            slot[i * 64 + lane] = make_float4(ak[4 * i], ak[4 * i + 1], ak[4 * i + 2], ak[4 * i + 3]);
            slot[(VEC / 4 + i) * 64 + lane] =
                make_float4(av[4 * i], av[4 * i + 1], av[4 * i + 2], av[4 * i + 3]);
          }
        } else {
          finish_key<R>(j, ak, av);
        }
      }
    }
  }

  __device__ inline void walk(int u0, int end_u) {
    // u = a-2 .. a+P+1 for every wave of the workgroup (same trip count); the
    // last trip issues no prefetch past the walk.
    this->template prefetch<0>(u0);
    int u = u0;
    for (; u + 3 < end_u; u += 4) {
      stash<0>();
      this->template prefetch<1>(u + 1);
      this->template compute<0>(u);
      stash<1>();
      this->template prefetch<2>(u + 2);
      this->template compute<1>(u + 1);
      stash<2>();
      this->template prefetch<3>(u + 3);
      this->template compute<2>(u + 2);
      stash<3>();
      this->template prefetch<0>(u + 4);
      this->template compute<3>(u + 3);
    }
    stash<0>();
    this->template prefetch<1>(u + 1);
    this->template compute<0>(u);
    stash<1>();
    this->template prefetch<2>(u + 2);
    this->template compute<1>(u + 1);
    stash<2>();
    this->template prefetch<3>(u + 3);
    this->template compute<2>(u + 2);
    stash<3>();
    this->template compute<3>(u + 3);
  }
};

template <typename T, int LPR, int NM, bool LEFT_LDS, bool RIGHT_LDS, int W, bool RING>
__device__ inline void chain_pro_wave(const Params& p, const ChainCfg& c,
                                      ChainProSlot<VecOf<T>::value>* lds,
                                      CsRing<LPR, VecOf<T>::value / 2>* rings, int w, int b,
                                      int hg, int rb, int cb, int a,
                                      float (&dw)[2][VecOf<T>::value]) {
  constexpr int VEC = VecOf<T>::value, esz = (int)sizeof(T);
  const int lane = threadIdx.x & 63, hl = lane / LPR, li = lane % LPR;
  const int h0 = hg * (64 / LPR);
  BwdChainPro<T, LPR, NM, LEFT_LDS, RIGHT_LDS, RING> x;
  x.ring = rings[RING ? w : 0];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    x.dwq[e] = 0.f;
    x.dwk[e] = 0.f;
  }
  x.init(p, li);
  x.q = make_split(p.q, esz, b, h0, hl, li, p.D, x.HV);
  x.k = make_split(p.k, esz, b, h0, hl, li, p.D, x.HV);
  x.v = make_split(p.v, esz, b, h0, hl, li, p.D, x.HV);
  x.go = make_split(p.dout, esz, b, h0, hl, li, p.D, x.HV);
  x.dq = make_split(p.dq, esz, b, h0, hl, li, p.D, x.HV);
  x.dk = make_split(p.dk, esz, b, h0, hl, li, p.D, x.HV);
  x.dv = make_split(p.dv, esz, b, h0, hl, li, p.D, x.HV);
  x.lse = lse_stream(p, b, h0, hl);
  x.scale = p.scale;
  x.F = c.F;
  x.T_ = p.T;
  x.a = a;
  x.end = min(a + c.P, p.T);   // < a for a row past the end: nothing is stored
  x.lane = lane;
  x.hl = hl;
  x.mine = lds + w;
  x.up = lds + (LEFT_LDS ? w - 1 : w);
  x.down = lds + (RIGHT_LDS ? w + 1 : w);
  // Deferred slots (row blocks but the last): this wave's band in block rb
  // (last wave) and in block rb - 1 (first wave, far weight pairs).
  const int64_t slots = chain_pro_slots(p.B, c);
  const int last_block = c.blocks - 1;
  x.defer = rb < last_block
                ? reinterpret_cast<float4*>(p.tab) +
                      chain_pro_slot(c, b, hg, rb, cb * c.P) * (2 * (VEC / 4) * 64)
                : nullptr;   // the last block's keys have no far query
  float2* pcs = reinterpret_cast<float2*>(p.tab + slots * chain_pro_slot_floats(LPR, p.D));
  x.defer_pc = (!LEFT_LDS && rb > 0) ? pcs + chain_pro_slot(c, b, hg, rb - 1, cb * c.P) * (64 / LPR)
                                     : nullptr;
  x.walk(a - 2, a + c.P + 1);
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    dw[0][e] = x.dwq[e];
    dw[1][e] = x.dwk[e];
  }
}

template <typename T, int LPR, int NM, int W>
__global__ __launch_bounds__(64 * W) void bwd_chain_pro(Params p, ChainCfg c) {
  constexpr int VEC = VecOf<T>::value;
  // The cos/sin rings where they fit beside the rows' rings in one CU's LDS
  // (all but 16-lane rows of 16-bit types: head_dim 128).
  constexpr bool RING =
      sizeof(ChainProSlot<VEC>) * W + sizeof(CsRing<LPR, VEC / 2>) * W <= 160 * 1024;
  __shared__ ChainProSlot<VEC> lds[W];
  __shared__ CsRing<LPR, VEC / 2> rings[RING ? W : 1];
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Workgroup -> (batch, head group, band, row block), XCD-contiguous; wave w
  // -> row w of the block (one chain per workgroup).
  int64_t g = xcd_remap(blockIdx.x, gridDim.x);
  const int rb = (int)(g % c.blocks);
  g /= c.blocks;
  const int cb = (int)(g % c.bands);
  g /= c.bands;
  const int hg = (int)(g % c.HG);
  const int b = (int)(g / c.HG);
  const int r = rb * W + w;
  const int64_t a64 = (int64_t)r * c.F + (int64_t)cb * c.P;
  const int a = (r < c.rows && a64 < p.T) ? (int)a64 : p.T;
  float dw[2][VecOf<T>::value];
  if constexpr (W == 1) {
    chain_pro_wave<T, LPR, NM, false, false, W, RING>(p, c, lds, rings, w, b, hg, rb, cb, a, dw);
  } else {
    if (w == 0)
      chain_pro_wave<T, LPR, NM, false, true, W, RING>(p, c, lds, rings, w, b, hg, rb, cb, a, dw);
    else if (w == W - 1)
      chain_pro_wave<T, LPR, NM, true, false, W, RING>(p, c, lds, rings, w, b, hg, rb, cb, a, dw);
    else
      chain_pro_wave<T, LPR, NM, true, true, W, RING>(p, c, lds, rings, w, b, hg, rb, cb, a, dw);
  }
  // One norm-weight partial row per workgroup (the rings' LDS is free now).
  float* const parts[2] = {p.dwq_part, p.dwk_part};
  write_group_partials<T, LPR, 2>(dw, reinterpret_cast<float*>(lds), W, parts, blockIdx.x, p.D);
}

// Finishes the deferred keys: the last row of every chain (row rb * W + W - 1)
// whose far query j + F exists.  One wave per kFixCols columns of a row (the
// loop has no barriers; the workgroup's partial row at the end has two).
// dK' = near part + c * roped q_{j+F}, dV = near part + p * dO_{j+F}, then the
// transposed prologue as in the chained walk.
template <typename T, int LPR>
__global__ __launch_bounds__(256) void bwd_fix_pro(Params p, ChainCfg c, int64_t part0) {
  constexpr int VEC = VecOf<T>::value, HV = VEC / 2, esz = (int)sizeof(T);
  using PL = Prologue<T, LPR>;
  __shared__ float red[4 * 128];
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int chunks = (c.F + kFixCols - 1) / kFixCols;
  const int64_t nwaves = chain_pro_fix_waves(p.B, c);
  float dw[1][VEC];
  float (&dwk)[VEC] = dw[0];
#pragma unroll
  for (int e = 0; e < VEC; ++e) dwk[e] = 0.f;
  if (wave < nwaves) {
    int64_t g = wave;
    const int chunk = (int)(g % chunks);
    g /= chunks;
    const int nb = (int)chain_pro_deferring_blocks(c);
    const int rb = (int)(g % nb);
    g /= nb;
    const int hg = (int)(g % c.HG);
    const int b = (int)(g / c.HG);
    const int r = rb * c.W + c.W - 1;
    const int lane = threadIdx.x & 63, hl = lane / LPR, li = lane % LPR;
    const int h0 = hg * (64 / LPR);
    ProBase<T, LPR> pb;
    pb.init(p, li);
    const SplitStream q = make_split(p.q, esz, b, h0, hl, li, p.D, HV);
    const SplitStream k = make_split(p.k, esz, b, h0, hl, li, p.D, HV);
    const SplitStream go = make_split(p.dout, esz, b, h0, hl, li, p.D, HV);
    const SplitStream dk = make_split(p.dk, esz, b, h0, hl, li, p.D, HV);
    const SplitStream dv = make_split(p.dv, esz, b, h0, hl, li, p.D, HV);
    const int64_t slots = chain_pro_slots(p.B, c);
    const float4* rows = reinterpret_cast<const float4*>(p.tab);
    const float2* pcs = reinterpret_cast<const float2*>(p.tab + slots * chain_pro_slot_floats(LPR, p.D));
    const int c0 = chunk * kFixCols, c1 = min(c.F, c0 + kFixCols);
    for (int col = c0; col < c1; ++col) {
      const int64_t j64 = (int64_t)r * c.F + col;
      if (c.W < 2 || r >= c.rows || j64 + c.F >= p.T) continue;
      const int j = (int)j64, i = j + c.F;
      const int64_t slot = chain_pro_slot(c, b, hg, rb, col);
      const float4* sr = rows + slot * (2 * (VEC / 4) * 64);
      float ak[VEC], av[VEC];
#pragma unroll
      for (int n = 0; n < VEC / 4; ++n) {
        const float4 x = sr[n * 64 + lane];
        const float4 y = sr[(VEC / 4 + n) * 64 + lane];
        ak[4 * n] = x.x; ak[4 * n + 1] = x.y; ak[4 * n + 2] = x.z; ak[4 * n + 3] = x.w;
        av[4 * n] = y.x; av[4 * n + 1] = y.y; av[4 * n + 2] = y.z; av[4 * n + 3] = y.w;
      }
      const float2 w2 = pcs[slot * (64 / LPR) + hl];
      float ci[HV], si[HV], qi[VEC], gx[VEC];
      pb.cs(i, ci, si);
      pb.rope(load_split(q, i), pb.wq, ci, si, qi);
      widen<T>(load_split(go, i), gx);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        ak[e] = __builtin_fmaf(w2.y, qi[e], ak[e]);
        av[e] = __builtin_fmaf(w2.x, gx[e], av[e]);
      }
      float kx[VEC], cj[HV], sj[HV];
      widen<T>(load_split(k, j), kx);
      pb.cs(j, cj, sj);
      const float rkj = PL::rms_factor(kx, ProBase<T, LPR>::D, pb.eps);
      PL::backward_w(ak, kx, rkj, pb.wk, cj, sj, ProBase<T, LPR>::D, dwk);
      store_split<T>(dk, j, ak);
      store_split<T>(dv, j, av);
    }
  }
  float* const parts[1] = {p.dwk_part};
  write_group_partials<T, LPR, 1>(dw, red, 4, parts, part0 + blockIdx.x, p.D);
}

// ---- forward as row chains (far offsets F >= 16 in column order)
//
// The workgroup's waves walk W consecutive rows of one column band in
// lockstep (one barrier per step, as the chained backwards): wave w publishes
// its roped k and raw v rows in LDS and wave w + 1 takes them as its far-left
// sources in the same step, so only the first wave of a chain loads and ropes
// far rows.  Rows past the end walk clamped rows and store nothing.

template <int VEC>
struct FwdChainSlot {
  float4 kf[2][VEC / 4][64];   // [t & 1][quarter][lane]: roped k of position t
  u32x4 vf[2][64];             // [t & 1][lane]: raw v
};

template <typename T, int LPR, int NM, bool LEFT_LDS>
struct FwdChainPro : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using Slot = FwdChainSlot<VecOf<T>::value>;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + 1;

  SplitStream q, k, v, o;
  Stream lse;
  int F, lane;
  float scale;
  Slot* mine;
  const Slot* up;
  Raw kraw[2], qraw[2], vraw[2], klr[2], vlr[2];
  float cc[2][HV], ss[2][HV], clc[2][HV], cls[2][HV];
  float kq[4][VEC], vr[4][VEC];

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, this->Tm1);
    kraw[R & 1] = load_split(k, tc);
    qraw[R & 1] = load_split(q, tc);
    vraw[R & 1] = load_split(v, tc);
    this->cs(tc, cc[R & 1], ss[R & 1]);
    if constexpr (!LEFT_LDS) {
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
    put_rows<VEC>(mine->kf[R & 1], lane, kq[R]);
    mine->vf[R & 1][lane] = pack_raw(vraw[R & 1]);
    float qr[VEC];
    this->rope(qraw[R & 1], this->wq, cc[R & 1], ss[R & 1], qr);
    __syncthreads();
    float kf[VEC], vf[VEC];
    if constexpr (LEFT_LDS) {
      get_rows<VEC>(up->kf[R & 1], lane, kf);
      widen<T>(unpack_raw(up->vf[R & 1][lane]), vf);
    } else {
      this->rope(klr[R & 1], this->wk, clc[R & 1], cls[R & 1], kf);
      widen<T>(vlr[R & 1], vf);
    }
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
    ok[NS - 1] = t - F >= 0;
    sc[NS - 1] = row_sum<LPR>(dot_partial<VEC>(qr, kf)) * scale;
    float m = -INFINITY;
#pragma unroll
    for (int s_ = 0; s_ < NS; ++s_) m = ok[s_] ? fmaxf(m, sc[s_]) : m;
    float w[NS], l = 0.f;
#pragma unroll
    for (int s_ = 0; s_ < NS; ++s_) {
      w[s_] = ok[s_] ? fast_exp(sc[s_] - m) : 0.f;
      l += w[s_];
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
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w[NS - 1], vf[e], acc[e]);
    // l >= 1 whenever a source is valid (the largest term is exp(0)).
    const float inv = l > 0.f ? __builtin_amdgcn_rcpf(l) : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= inv;
    if (store) {
      store_split<T>(o, t, acc);
      if (this->li == 0) store_f32(lse, t, l > 0.f ? m + fast_log(l) : INFINITY);
    }
  }
};

// The extra wave of a forward chain: it walks the row before the block and
// only loads, ropes and publishes its k and v rows -- the far-left sources of
// the block's first row -- so that every wave that computes takes its far
// sources from LDS and the lockstep steps are not held by one wave doing a
// third prologue.
template <typename T, int LPR>
struct FwdChainLoader : ProBase<T, LPR> {
  using B_ = ProBase<T, LPR>;
  using B_::VEC;
  using B_::HV;
  using Slot = FwdChainSlot<VecOf<T>::value>;

  SplitStream k, v;
  int lane;
  Slot* mine;
  Raw kraw[2], vraw[2];
  float cc[2][HV], ss[2][HV];

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, this->Tm1);
    kraw[R & 1] = load_split(k, tc);
    vraw[R & 1] = load_split(v, tc);
    this->cs(tc, cc[R & 1], ss[R & 1]);
  }

  template <int R>
  __device__ inline void compute(int, bool) {
    float kq[VEC];
    this->rope(kraw[R & 1], this->wk, cc[R & 1], ss[R & 1], kq);
    put_rows<VEC>(mine->kf[R & 1], lane, kq);
    mine->vf[R & 1][lane] = pack_raw(vraw[R & 1]);
    __syncthreads();
  }
};

template <typename T, int LPR>
__device__ inline void fwd_chain_loader(const Params& p, const ChainCfg& c,
                                        FwdChainSlot<VecOf<T>::value>* lds, int b, int hg, int a) {
  constexpr int esz = (int)sizeof(T);
  const int lane = threadIdx.x & 63, hl = lane / LPR, li = lane % LPR;
  const int h0 = hg * (64 / LPR);
  FwdChainLoader<T, LPR> x;
  x.init(p, li);
  x.k = make_split(p.k, esz, b, h0, hl, li, p.D, x.HV);
  x.v = make_split(p.v, esz, b, h0, hl, li, p.D, x.HV);
  x.lane = lane;
  x.mine = lds;
  const int t0 = a - 2;
  x.template prefetch<0>(t0);
  int t = t0;
  for (; t + 4 < a + c.P; t += 4) {
    x.template prefetch<1>(t + 1);
    x.template compute<0>(t, false);
    x.template prefetch<2>(t + 2);
    x.template compute<1>(t + 1, false);
    x.template prefetch<3>(t + 3);
    x.template compute<2>(t + 2, false);
    x.template prefetch<0>(t + 4);
    x.template compute<3>(t + 3, false);
  }
  x.template prefetch<1>(t + 1);
  x.template compute<0>(t, false);
  x.template prefetch<2>(t + 2);
  x.template compute<1>(t + 1, false);
  x.template prefetch<3>(t + 3);
  x.template compute<2>(t + 2, false);
  x.template compute<3>(t + 3, false);
}

template <typename T, int LPR, int NM, bool LEFT_LDS, int W>
__device__ inline void fwd_chain_wave(const Params& p, const ChainCfg& c,
                                      FwdChainSlot<VecOf<T>::value>* lds, int w, int b, int hg,
                                      int a) {
  constexpr int esz = (int)sizeof(T);
  const int lane = threadIdx.x & 63, hl = lane / LPR, li = lane % LPR;
  const int h0 = hg * (64 / LPR);
  FwdChainPro<T, LPR, NM, LEFT_LDS> x;
  x.init(p, li);
  x.q = make_split(p.q, esz, b, h0, hl, li, p.D, x.HV);
  x.k = make_split(p.k, esz, b, h0, hl, li, p.D, x.HV);
  x.v = make_split(p.v, esz, b, h0, hl, li, p.D, x.HV);
  x.o = make_split(p.o, esz, b, h0, hl, li, p.D, x.HV);
  x.lse = lse_stream(p, b, h0, hl);
  x.scale = p.scale;
  x.F = c.F;
  x.lane = lane;
  x.mine = lds + w;
  x.up = lds + (LEFT_LDS ? w - 1 : w);
  const int end = min(a + c.P, p.T);
  // t = a-2 .. a+P-1 in steps of 4 (slot of t is (t - a + 2) & 3); the trip
  // count depends only on P.
  const int t0 = a - 2;
  x.template prefetch<0>(t0);
  int t = t0;
  for (; t + 4 < a + c.P; t += 4) {
    x.template prefetch<1>(t + 1);
    x.template compute<0>(t, t >= a && t < end);
    x.template prefetch<2>(t + 2);
    x.template compute<1>(t + 1, t + 1 >= a && t + 1 < end);
    x.template prefetch<3>(t + 3);
    x.template compute<2>(t + 2, t + 2 >= a && t + 2 < end);
    x.template prefetch<0>(t + 4);
    x.template compute<3>(t + 3, t + 3 >= a && t + 3 < end);
  }
  // Last trip: no prefetch past the walk.
  x.template prefetch<1>(t + 1);
  x.template compute<0>(t, t >= a && t < end);
  x.template prefetch<2>(t + 2);
  x.template compute<1>(t + 1, t + 1 >= a && t + 1 < end);
  x.template prefetch<3>(t + 3);
  x.template compute<2>(t + 2, t + 2 >= a && t + 2 < end);
  x.template compute<3>(t + 3, t + 3 >= a && t + 3 < end);
}

// 8-row chains run with the loader wave (layers 5-15 of the prologue forward
// at T = 2^20: 0.96-0.97x the time); the shorter chains at row strides of
// 32 MiB and more measured 5-13% slower with it and keep their first wave
// loading its own far rows.
template <int W>
constexpr int fwd_chain_loader_waves() { return W == 8 ? 1 : 0; }

template <typename T, int LPR, int NM, int W>
__global__ __launch_bounds__(64 * (W + fwd_chain_loader_waves<W>())) void fwd_chain_pro(Params p,
                                                                                       ChainCfg c) {
  constexpr int LW = fwd_chain_loader_waves<W>();
  __shared__ FwdChainSlot<VecOf<T>::value> lds[W + LW];
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // Workgroup -> (batch, head group, band, row block), XCD-contiguous; with
  // the loader, wave 0 -> the row before the block and wave w >= 1 -> row
  // w - 1; without, wave w -> row w.
  int64_t g = xcd_remap(blockIdx.x, gridDim.x);
  const int rb = (int)(g % c.blocks);
  g /= c.blocks;
  const int cb = (int)(g % c.bands);
  g /= c.bands;
  const int hg = (int)(g % c.HG);
  const int b = (int)(g / c.HG);
  const int r = rb * W + wv - LW;
  const int64_t a64 = (int64_t)r * c.F + (int64_t)cb * c.P;
  if (LW && wv == 0) {
    // Row rb * W - 1 (before the sequence for the first block: its clamped
    // rows are the sources of positions t - F < 0, which no query uses).
    fwd_chain_loader<T, LPR>(p, c, lds, b, hg, (int)a64);
  } else {
    const int a = (r < c.rows && a64 < p.T) ? (int)a64 : p.T;
    if (LW || wv > 0)
      fwd_chain_wave<T, LPR, NM, true, W>(p, c, lds, wv, b, hg, a);
    else
      fwd_chain_wave<T, LPR, NM, false, W>(p, c, lds, wv, b, hg, a);
  }
}

}  // namespace

template <typename T, int LPR, int NM, bool FAR>
hipError_t pro_pattern(bool fwd, const Params& p, const WalkCfg& c, int dtype, hipStream_t st) {
  const dim3 grid((unsigned)c.nwg), block(kPipeBlock);
  if (fwd) {
    if constexpr (FAR) {
      if (c.column) {
        const ChainCfg cc = make_chain_cfg(p.B, p.q.st * (int64_t)sizeof(T), c);
        if (cc.nwg <= 0) return hipErrorInvalidValue;
        const dim3 cgrid((unsigned)cc.nwg), cblock(64 * (cc.W + (cc.W == 8 ? 1 : 0)));
        switch (cc.W) {
          case 8: hipLaunchKernelGGL((fwd_chain_pro<T, LPR, NM, 8>), cgrid, cblock, 0, st, p, cc); break;
          case 4: hipLaunchKernelGGL((fwd_chain_pro<T, LPR, NM, 4>), cgrid, cblock, 0, st, p, cc); break;
          case 2: hipLaunchKernelGGL((fwd_chain_pro<T, LPR, NM, 2>), cgrid, cblock, 0, st, p, cc); break;
          default: hipLaunchKernelGGL((fwd_chain_pro<T, LPR, NM, 1>), cgrid, cblock, 0, st, p, cc); break;
        }
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((fwd_pipe_pro<T, LPR, NM, FAR>), grid, block, kPipeLds, st, p, c);
    return hipGetLastError();
  }
  if constexpr (!FAR) {
    hipLaunchKernelGGL((bwd_fused_pro<T, LPR, NM>), grid, block, kPipeLds, st, p, c);
    return hipGetLastError();
  } else {
    if (c.column) {
      const ChainCfg cc = make_chain_cfg(p.B, p.q.st * (int64_t)sizeof(T), c);
      if (cc.nwg <= 0) return hipErrorInvalidValue;
      const dim3 cgrid((unsigned)cc.nwg), cblock(64 * cc.W);
      switch (cc.W) {
        case 8: hipLaunchKernelGGL((bwd_chain_pro<T, LPR, NM, 8>), cgrid, cblock, 0, st, p, cc); break;
        case 4: hipLaunchKernelGGL((bwd_chain_pro<T, LPR, NM, 4>), cgrid, cblock, 0, st, p, cc); break;
        case 2: hipLaunchKernelGGL((bwd_chain_pro<T, LPR, NM, 2>), cgrid, cblock, 0, st, p, cc); break;
        default: hipLaunchKernelGGL((bwd_chain_pro<T, LPR, NM, 1>), cgrid, cblock, 0, st, p, cc); break;
      }
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const int64_t fw = chain_pro_fix_waves(p.B, cc);
      const int64_t fwg = (fw + 3) / 4;
      if (fwg > 0x7fffffff) return hipErrorInvalidValue;
      if (fwg == 0) return hipSuccess;   // a single row block defers nothing
      hipLaunchKernelGGL((bwd_fix_pro<T, LPR>), dim3((unsigned)fwg), dim3(256), 0, st, p, cc,
                         (int64_t)cc.nwg);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((bwd_q_pro<T, LPR, NM, FAR>), grid, block, kPipeLds, st, p, c);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_k_pro<T, LPR, NM, FAR>), grid, block, kPipeLds, st, p, c);
    return hipGetLastError();
  }
}

hipError_t launch_pro(bool fwd, const Params& p, const WalkCfg& c, const Pattern& pat, int dtype,
                      int lpr, hipStream_t st) {
  return by_type_lpr(dtype, lpr, [&](auto tag, auto lprc) -> hipError_t {
    using T = typename decltype(tag)::type;
    constexpr int L = decltype(lprc)::value;
    if (pat.far == 0) {
      if (pat.nm == 3) return pro_pattern<T, L, 3, false>(fwd, p, c, dtype, st);
      if (pat.nm == 5) return pro_pattern<T, L, 5, false>(fwd, p, c, dtype, st);
    } else {
      if (pat.nm == 7) return pro_pattern<T, L, 7, true>(fwd, p, c, dtype, st);
      if (pat.nm == 1) return pro_pattern<T, L, 1, true>(fwd, p, c, dtype, st);
    }
    return hipErrorInvalidValue;
  });
}

hipError_t launch_fwd_pro(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype,
                          int lpr, hipStream_t st) {
  return launch_pro(true, p, c, pat, dtype, lpr, st);
}

hipError_t launch_bwd_pro(const Params& p, const WalkCfg& c, const Pattern& pat, int dtype,
                          int lpr, hipStream_t st) {
  return launch_pro(false, p, c, pat, dtype, lpr, st);
}

}  // namespace walk
}  // namespace sbda
