// Wavefront-walk SBDA kernels: the fast path for the SBDA schedule.
//
// Layout.  One 64-lane wavefront holds all G = 64/LPR heads of one position
// ("head group"): lane = g * LPR + li, so one 16-byte-per-lane load moves one
// position's rows of the group (1 KiB for 8 heads x 64 dims x bf16).  Each
// wave owns a tile of P consecutive positions and walks it in order.
//
// Sources.  Offsets split into "near" ones (0, 1, 2: a compile-time mask NM)
// and at most one "far" offset F >= 3.  Near sources are the rows the walk
// just loaded, kept in a 3-deep register rotation (no reload); the far
// source is loaded directly.  Tiles are ordered so that the wave holding
// positions t - F (and t + F) runs next to this one -- linear order for
// F < P, column order (tile a, a + F, a + 2F, ...) otherwise -- and the
// workgroup id is remapped so consecutive tiles share an XCD (and its L2).
//
// Backward (gather form, every row written once, no atomics).  Walking
// queries u = a-2 .. end+1, the wave computes each query's weights p_s and
// score gradients dS_s once; dQ_u is complete at once, and near-slot
// contributions dK/dV_{u-n} += (scale dS_n q_u, p_n dO_u) go to three
// rotating key accumulators.  Key j = u-2 is then complete except for its
// far query i = j + F, whose weights are recomputed from q_i, dO_i, lse_i and
// i's own sources (a second rotation over positions i, i-1, i-2, plus k_j,
// v_j from the first).  Keys are written as soon as they complete.
//
// Reference semantics: BiAttn/left_v2.py:313-405 (forward maths) and the
// key-centric backward specified by BiAttn/sbda_triton.py:507-671.

#include <type_traits>

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {

namespace {

constexpr int kWaves = 4;               // independent waves per workgroup
constexpr int kWalkBlock = kWaves * 64;

struct WalkCfg {
  int P;         // positions per tile
  int HG;        // head groups (waves per position)
  int tiles_t;   // tiles per (batch, head group) along T
  int column;    // 1: column order (far offset F is a multiple of P)
  int rows;      // column order: ceil(T / F)
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

__device__ inline int64_t wave_id() {
  return xcd_remap(blockIdx.x, gridDim.x) * kWaves + (threadIdx.x >> 6);
}

__device__ inline bool decode_tile(const Params& p, const WalkCfg& c, int64_t n, int& b, int& hg,
                                   int& a) {
  if (n >= c.total) return false;
  hg = (int)(n % c.HG);
  const int64_t rest = n / c.HG;
  const int k = (int)(rest % c.tiles_t);
  b = (int)(rest / c.tiles_t);
  if (c.column) {
    const int r = k % c.rows, cb = k / c.rows;
    a = r * c.F + cb * c.P;
  } else {
    a = k * c.P;
  }
  return a < p.T;
}

template <typename T>
struct Rows {
  const T* __restrict__ base;
  int64_t st;
  __device__ inline const T* at(int64_t t) const { return base + t * st; }
};

template <typename T, int LPR, bool PRO>
struct Lane {
  static constexpr int VEC = VecOf<T>::value;
  using PL = Prologue<T, LPR>;
  int li;
  int D;
  const float* wq;
  const float* wk;
  const float* rc;
  const float* rs;
  float eps;

  __device__ inline void init(const Params& p, int lane_in_row) {
    li = lane_in_row;
    D = p.D;
    wq = p.wq;
    wk = p.wk;
    rc = p.rope_cos;
    rs = p.rope_sin;
    eps = p.eps;
  }

  __device__ inline void load(const Rows<T>& r, int64_t t, float (&x)[VEC]) const {
    load_row<T, PRO>(r.at(t), li, D, x);
  }
  __device__ inline void zero(float (&x)[VEC]) const {
#pragma unroll
    for (int i = 0; i < VEC; ++i) x[i] = 0.f;
  }
  // Loads a q or k row and, with the prologue, normalises and rotates it.
  __device__ inline void load_qk(const Rows<T>& r, int64_t t, const float* w, float (&x)[VEC]) const {
    load(r, t, x);
    if constexpr (PRO) {
      float c[PL::HV], s[PL::HV];
      PL::load_cs(rc, rs, t, li, D, c, s);
      PL::forward(x, w, c, s, li, D, eps);
    }
  }
  __device__ inline float dot(const float (&a)[VEC], const float (&b)[VEC]) const {
    return row_sum<LPR>(dot_partial<VEC>(a, b));
  }
};

// Weights and score gradients of one query from its sources.
template <int NS, int VEC, int LPR>
__device__ inline void query_grads(const float (&q)[VEC], const float (&go)[VEC], float lse,
                                   float scale, const float* const (&ks)[NS],
                                   const float* const (&vs)[NS], const bool (&ok)[NS],
                                   float (&pp)[NS], float (&ds)[NS]) {
  float dp[NS];
  float delta = 0.f;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    float a = 0.f, d = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      a = __builtin_fmaf(q[e], ks[s][e], a);
      d = __builtin_fmaf(go[e], vs[s][e], d);
    }
    a = row_sum<LPR>(a) * scale;
    d = row_sum<LPR>(d);
    pp[s] = ok[s] ? fast_exp(a - lse) : 0.f;
    dp[s] = d;
    delta = __builtin_fmaf(pp[s], d, delta);
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) ds[s] = pp[s] * (dp[s] - delta);
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

// =================================================================== forward

template <typename T, int LPR, int NM, bool FAR, bool PRO>
struct FwdWalker {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);
  using L = Lane<T, LPR, PRO>;

  L ln;
  Rows<T> q, k, v;
  T* __restrict__ o;
  int64_t ost;
  float* __restrict__ lse;
  int lst;
  float scale;
  int F;
  float kr[3][VEC], vr[3][VEC];

  template <int R>
  __device__ inline void step(int t) {
    ln.load_qk(k, t, ln.wk, kr[R]);
    ln.load(v, t, vr[R]);
    float qr[VEC];
    ln.load_qk(q, t, ln.wq, qr);
    const int tf = t - F;
    float kf[VEC], vf[VEC];
    if constexpr (FAR) {
      if (tf >= 0) {
        ln.load_qk(k, tf, ln.wk, kf);
        ln.load(v, tf, vf);
      } else {
        ln.zero(kf);
        ln.zero(vf);
      }
    }
    float sc[NS];
    bool ok[NS];
    const float* vs[NS];
    int idx = 0;
#pragma unroll
    for (int n = 0; n < 3; ++n) {
      if (NM & (1 << n)) {
        const int slot = (R + 3 - n) % 3;
        ok[idx] = t - n >= 0;
        sc[idx] = ln.dot(qr, kr[slot]) * scale;
        vs[idx] = vr[slot];
        ++idx;
      }
    }
    if constexpr (FAR) {
      ok[NS - 1] = tf >= 0;
      sc[NS - 1] = ln.dot(qr, kf) * scale;
      vs[NS - 1] = vf;
    }
    float m = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; ++s)
      if (ok[s]) m = fmaxf(m, sc[s]);
    float acc[VEC];
    ln.zero(acc);
    float l = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float w = ok[s] ? fast_exp(sc[s] - m) : 0.f;
      l += w;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(w, vs[s][e], acc[e]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= inv;
    store_row<T, PRO>(o + (int64_t)t * ost, ln.li, ln.D, acc);
    if (ln.li == 0) lse[(int64_t)t * lst] = l > 0.f ? m + fast_log(l) : INFINITY;
  }

  // Loads position t's k/v into rotation slot R (zeros before the start).
  template <int R>
  __device__ inline void prefill(int t) {
    if (t >= 0) {
      ln.load_qk(k, t, ln.wk, kr[R]);
      ln.load(v, t, vr[R]);
    } else {
      ln.zero(kr[R]);
      ln.zero(vr[R]);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR, bool PRO>
__global__ __launch_bounds__(kWalkBlock) void fwd_walk(Params p, WalkCfg c) {
  int b, hg, a;
  if (!decode_tile(p, c, wave_id(), b, hg, a)) return;
  const int lane = threadIdx.x & 63;
  const int h = hg * (64 / LPR) + lane / LPR;
  FwdWalker<T, LPR, NM, FAR, PRO> w;
  w.ln.init(p, lane % LPR);
  w.q = {reinterpret_cast<const T*>(p.q.p) + (int64_t)b * p.q.sb + (int64_t)h * p.q.sh, p.q.st};
  w.k = {reinterpret_cast<const T*>(p.k.p) + (int64_t)b * p.k.sb + (int64_t)h * p.k.sh, p.k.st};
  w.v = {reinterpret_cast<const T*>(p.v.p) + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh, p.v.st};
  w.o = reinterpret_cast<T*>(p.o.p) + (int64_t)b * p.o.sb + (int64_t)h * p.o.sh;
  w.ost = p.o.st;
  w.lse = p.lse + (int64_t)b * p.T * p.H + h;
  w.lst = p.H;
  w.scale = p.scale;
  w.F = c.F;
  const int end = min(a + c.P, p.T);
  // Rotation slot of position t is (t - a) mod 3: a-1 -> 2, a-2 -> 1.
  if constexpr ((NM & 6) != 0) {
    w.template prefill<2>(a - 1);
    w.template prefill<1>(a - 2);
  }
  int t = a;
  for (; t + 3 <= end; t += 3) {
    w.template step<0>(t);
    w.template step<1>(t + 1);
    w.template step<2>(t + 2);
  }
  if (t < end) w.template step<0>(t);
  if (t + 1 < end) w.template step<1>(t + 1);
}

// ================================================================== backward

template <typename T, int LPR, int NM, bool FAR, bool PRO>
struct BwdWalker {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);
  using L = Lane<T, LPR, PRO>;
  using PL = Prologue<T, LPR>;

  L ln;
  Rows<T> q, k, v, go;
  T* __restrict__ dq;
  T* __restrict__ dk;
  T* __restrict__ dv;
  int64_t dqst, dkst, dvst;
  const float* __restrict__ lse;
  int lst;
  float scale;
  int F, T_, a, end, qend;
  float kr[3][VEC], vr[3][VEC];     // own rotation: k, v at u (slot R), u-1, u-2
  float fk[3][VEC], fv[3][VEC];     // far-right rotation: i = u-2+F, i-1, i-2
  float ak[3][VEC], av[3][VEC];     // key accumulators: keys u, u-1, u-2
  float dwq[VEC], dwk[VEC];         // prologue weight-gradient partials

  template <int R>
  __device__ inline void step(int u) {
    constexpr int R1 = (R + 2) % 3;   // slot of u-1
    constexpr int R2 = (R + 1) % 3;   // slot of u-2
    // 1. Own rotation push and fresh accumulator for key u.
    if (u >= 0 && u < T_) {
      ln.load_qk(k, u, ln.wk, kr[R]);
      ln.load(v, u, vr[R]);
    } else {
      ln.zero(kr[R]);
      ln.zero(vr[R]);
    }
    ln.zero(ak[R]);
    ln.zero(av[R]);
    // 2. Far-right rotation push: position u - 2 + F.
    if constexpr (FAR) {
      const int i = u - 2 + F;
      if (i >= 0 && i < T_) {
        ln.load_qk(k, i, ln.wk, fk[R]);
        ln.load(v, i, fv[R]);
      } else {
        ln.zero(fk[R]);
        ln.zero(fv[R]);
      }
    }
    // 3. Own query u.
    if (u >= a && u < qend) {
      float qr[VEC], gr[VEC], xq[VEC];
      float rq = 0.f, cq[PL::HV], sq[PL::HV];
      ln.load(q, u, xq);
      if constexpr (PRO) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) qr[e] = xq[e];
        PL::load_cs(ln.rc, ln.rs, u, ln.li, ln.D, cq, sq);
        rq = PL::forward(qr, ln.wq, cq, sq, ln.li, ln.D, ln.eps);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) qr[e] = xq[e];
      }
      ln.load(go, u, gr);
      const float l = lse[(int64_t)u * lst];
      float kf[VEC], vf[VEC];
      const int uf = u - F;
      if constexpr (FAR) {
        if (uf >= 0) {
          ln.load_qk(k, uf, ln.wk, kf);
          ln.load(v, uf, vf);
        } else {
          ln.zero(kf);
          ln.zero(vf);
        }
      }
      const float* ks[NS];
      const float* vs[NS];
      bool ok[NS];
      int idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + 3 - n) % 3;
          ks[idx] = kr[slot];
          vs[idx] = vr[slot];
          ok[idx] = u - n >= 0;
          ++idx;
        }
      }
      if constexpr (FAR) {
        ks[NS - 1] = kf;
        vs[NS - 1] = vf;
        ok[NS - 1] = uf >= 0;
      }
      float pp[NS], ds[NS];
      query_grads<NS, VEC, LPR>(qr, gr, l, scale, ks, vs, ok, pp, ds);
      if (u < end) {
        float g[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          float acc = 0.f;
#pragma unroll
          for (int s = 0; s < NS; ++s) acc = __builtin_fmaf(ds[s], ks[s][e], acc);
          g[e] = acc * scale;
        }
        if constexpr (PRO) PL::backward(g, xq, rq, ln.wq, cq, sq, ln.li, ln.D, dwq);
        store_row<T, PRO>(dq + (int64_t)u * dqst, ln.li, ln.D, g);
      }
      // Near-slot contributions to keys u - n.
      idx = 0;
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        if (NM & (1 << n)) {
          const int slot = (R + 3 - n) % 3;
          const float cs = ds[idx] * scale, cp = pp[idx];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[slot][e] = __builtin_fmaf(cs, qr[e], ak[slot][e]);
            av[slot][e] = __builtin_fmaf(cp, gr[e], av[slot][e]);
          }
          ++idx;
        }
      }
    }
    // 4. Key j = u - 2 is complete but for its far query i = j + F.
    const int j = u - 2;
    if (j >= a && j < end) {
      if constexpr (FAR) {
        const int i = j + F;
        if (i < T_) {
          float qr[VEC], gr[VEC];
          ln.load_qk(q, i, ln.wq, qr);
          ln.load(go, i, gr);
          const float l = lse[(int64_t)i * lst];
          const float* ks[NS];
          const float* vs[NS];
          bool ok[NS];
          int idx = 0;
#pragma unroll
          for (int n = 0; n < 3; ++n) {
            if (NM & (1 << n)) {
              const int slot = (R + 3 - n) % 3;
              ks[idx] = fk[slot];
              vs[idx] = fv[slot];
              ok[idx] = true;   // i - n >= F - 2 > 0
              ++idx;
            }
          }
          ks[NS - 1] = kr[R2];
          vs[NS - 1] = vr[R2];
          ok[NS - 1] = true;
          float pp[NS], ds[NS];
          query_grads<NS, VEC, LPR>(qr, gr, l, scale, ks, vs, ok, pp, ds);
          const float cs = ds[NS - 1] * scale, cp = pp[NS - 1];
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            ak[R2][e] = __builtin_fmaf(cs, qr[e], ak[R2][e]);
            av[R2][e] = __builtin_fmaf(cp, gr[e], av[R2][e]);
          }
        }
      }
      if constexpr (PRO) {
        float xk[VEC], c[PL::HV], s[PL::HV];
        ln.load(k, j, xk);
        PL::load_cs(ln.rc, ln.rs, j, ln.li, ln.D, c, s);
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) ss = __builtin_fmaf(xk[e], xk[e], ss);
        ss = row_sum<LPR>(ss);
        const float r = __builtin_amdgcn_rsqf(__fadd_rn(__fdiv_rn(ss, (float)ln.D), ln.eps));
        PL::backward(ak[R2], xk, r, ln.wk, c, s, ln.li, ln.D, dwk);
      }
      store_row<T, PRO>(dk + (int64_t)j * dkst, ln.li, ln.D, ak[R2]);
      store_row<T, PRO>(dv + (int64_t)j * dvst, ln.li, ln.D, av[R2]);
    }
    (void)R1;
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

template <typename T, int LPR, int NM, bool FAR, bool PRO>
__global__ __launch_bounds__(kWalkBlock) void bwd_walk(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value;
  const int64_t wave = wave_id();
  int b, hg, a;
  const bool live = decode_tile(p, c, wave, b, hg, a);
  const int lane = threadIdx.x & 63;
  BwdWalker<T, LPR, NM, FAR, PRO> w;
  w.ln.zero(w.dwq);
  w.ln.zero(w.dwk);
  if (live) {
    const int h = hg * (64 / LPR) + lane / LPR;
    w.ln.init(p, lane % LPR);
    auto rows = [&](const View& vw) {
      return Rows<T>{reinterpret_cast<const T*>(vw.p) + (int64_t)b * vw.sb + (int64_t)h * vw.sh, vw.st};
    };
    w.q = rows(p.q);
    w.k = rows(p.k);
    w.v = rows(p.v);
    w.go = rows(p.dout);
    w.dq = reinterpret_cast<T*>(p.dq.p) + (int64_t)b * p.dq.sb + (int64_t)h * p.dq.sh;
    w.dk = reinterpret_cast<T*>(p.dk.p) + (int64_t)b * p.dk.sb + (int64_t)h * p.dk.sh;
    w.dv = reinterpret_cast<T*>(p.dv.p) + (int64_t)b * p.dv.sb + (int64_t)h * p.dv.sh;
    w.dqst = p.dq.st;
    w.dkst = p.dk.st;
    w.dvst = p.dv.st;
    w.lse = p.lse + (int64_t)b * p.T * p.H + h;
  w.lst = p.H;
    w.scale = p.scale;
    w.F = c.F;
    w.T_ = p.T;
    w.a = a;
    w.end = min(a + c.P, p.T);
    w.qend = min(w.end + 2, p.T);
    // Walk u = a-2 .. end+1; rotation slot of u is (u - a + 2) mod 3.
    const int last = w.end + 1;
    int u = a - 2;
    for (; u + 3 <= last + 1; u += 3) {
      w.template step<0>(u);
      w.template step<1>(u + 1);
      w.template step<2>(u + 2);
    }
    if (u <= last) w.template step<0>(u);
    if (u + 1 <= last) w.template step<1>(u + 1);
  }
  if constexpr (PRO) {
    write_wave_partial<T, LPR, true>(w.dwq, p.dwq_part, wave, p.D);
    write_wave_partial<T, LPR, true>(w.dwk, p.dwk_part, wave, p.D);
  }
  (void)VEC;
}

// ========================================================= pipelined walks
//
// The same walks without the prologue, software-pipelined: while step u is
// computed, every row step u+1 needs is already in flight.  Loads are
// unconditional (positions clamped into [0, T), validity applied as masks)
// so the compiler can keep them outstanding across steps.  Rows stay in
// their 16-byte raw form; dot products use v_dot2_f32_{bf16,f16} on the raw
// pairs and rows are widened to fp32 only where they are accumulated.
// Rotation depth 4 (positions u+1 .. u-2) with the loop unrolled by 4.

struct Raw {
  uint32_t w[4];
};

template <typename T>
__device__ inline Raw load_raw(const T* __restrict__ row, int li) {
  const uint4 x = *reinterpret_cast<const uint4*>(row + li * VecOf<T>::value);
  return Raw{{x.x, x.y, x.z, x.w}};
}

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

template <typename T, int LPR, int NM, bool FAR>
struct FwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  const T* __restrict__ q;
  const T* __restrict__ k;
  const T* __restrict__ v;
  T* __restrict__ o;
  float* __restrict__ lse;
  int lst;
  int64_t qst, kst, vst, ost;
  float scale;
  int F, Tm1, li;
  Raw kr[4];            // k at t (slot R), t-1, t-2; slot R+1 is being fetched
  Raw vraw[2], qn[2];   // this step's v and q (stage R & 1)
  Raw kl[2], vl[2];     // far source t - F
  float vr[4][VEC];     // widened v rotation

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, Tm1);
    kr[R] = load_raw<T>(k + (int64_t)tc * kst, li);
    vraw[R & 1] = load_raw<T>(v + (int64_t)tc * vst, li);
    qn[R & 1] = load_raw<T>(q + (int64_t)tc * qst, li);
    if constexpr (FAR) {
      const int tf = clampi(t - F, Tm1);
      kl[R & 1] = load_raw<T>(k + (int64_t)tf * kst, li);
      vl[R & 1] = load_raw<T>(v + (int64_t)tf * vst, li);
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
        sc[idx] = row_sum<LPR>(dot_raw<T>(qn[R & 1], kr[(R + 4 - n) & 3])) * scale;
        ++idx;
      }
    }
    float vf[VEC];
    if constexpr (FAR) {
      ok[NS - 1] = t - F >= 0;
      sc[NS - 1] = row_sum<LPR>(dot_raw<T>(qn[R & 1], kl[R & 1])) * scale;
      widen<T>(vl[R & 1], vf);
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
      store_row<T, false>(o + (int64_t)t * ost, li, VEC * LPR, acc);
      if (li == 0) lse[(int64_t)t * lst] = l > 0.f ? m + fast_log(l) : INFINITY;
    }
  }
};

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kWalkBlock) void fwd_pipe(Params p, WalkCfg c) {
  int b, hg, a;
  if (!decode_tile(p, c, wave_id(), b, hg, a)) return;
  const int lane = threadIdx.x & 63;
  const int h = hg * (64 / LPR) + lane / LPR;
  FwdPipe<T, LPR, NM, FAR> w;
  w.li = lane % LPR;
  w.q = reinterpret_cast<const T*>(p.q.p) + (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  w.k = reinterpret_cast<const T*>(p.k.p) + (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  w.v = reinterpret_cast<const T*>(p.v.p) + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  w.o = reinterpret_cast<T*>(p.o.p) + (int64_t)b * p.o.sb + (int64_t)h * p.o.sh;
  w.qst = p.q.st;
  w.kst = p.k.st;
  w.vst = p.v.st;
  w.ost = p.o.st;
  w.lse = p.lse + (int64_t)b * p.T * p.H + h;
  w.lst = p.H;
  w.scale = p.scale;
  w.F = c.F;
  w.Tm1 = p.T - 1;
  const int end = min(a + c.P, p.T);
  // Slot of position t is (t - a + 2) & 3: the walk starts two positions
  // early (a-2, a-1) to fill the near-source rotation; those steps store nothing.
  const int t0 = a - 2;
  w.template prefetch<0>(t0);
  for (int t = t0; t < end; t += 4) {
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

template <typename T, int LPR, int NM, bool FAR>
struct BwdPipe {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int NN = NearSet<NM>::count;
  static constexpr int NS = NN + (FAR ? 1 : 0);

  const T* __restrict__ q;
  const T* __restrict__ k;
  const T* __restrict__ v;
  const T* __restrict__ go;
  T* __restrict__ dq;
  T* __restrict__ dk;
  T* __restrict__ dv;
  const float* __restrict__ lse;
  int lst;
  int64_t qst, kst, vst, gst, dqst, dkst, dvst;
  float scale;
  int F, T_, Tm1, a, end, li;
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
    kr[R] = load_raw<T>(k + (int64_t)uc * kst, li);
    vr[R] = load_raw<T>(v + (int64_t)uc * vst, li);
    qr[R] = load_raw<T>(q + (int64_t)uc * qst, li);
    gr[R] = load_raw<T>(go + (int64_t)uc * gst, li);
    lr[R] = lse[(int64_t)uc * lst];
    if constexpr (FAR) {
      const int ul = clampi(u - F, Tm1);
      kl[R & 1] = load_raw<T>(k + (int64_t)ul * kst, li);
      vl[R & 1] = load_raw<T>(v + (int64_t)ul * vst, li);
      const int i = clampi(u - 2 + F, Tm1);
      fk[R] = load_raw<T>(k + (int64_t)i * kst, li);
      fv[R] = load_raw<T>(v + (int64_t)i * vst, li);
      qi[R & 1] = load_raw<T>(q + (int64_t)i * qst, li);
      gi[R & 1] = load_raw<T>(go + (int64_t)i * gst, li);
      li_[R & 1] = lse[(int64_t)i * lst];
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
        store_row<T, false>(dq + (int64_t)u * dqst, li, VEC * LPR, g);
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
      store_row<T, false>(dk + (int64_t)j * dkst, li, VEC * LPR, ak);
      store_row<T, false>(dv + (int64_t)j * dvst, li, VEC * LPR, av);
    }
  }
};

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kWalkBlock) void bwd_pipe(Params p, WalkCfg c) {
  int b, hg, a;
  if (!decode_tile(p, c, wave_id(), b, hg, a)) return;
  const int lane = threadIdx.x & 63;
  const int h = hg * (64 / LPR) + lane / LPR;
  BwdPipe<T, LPR, NM, FAR> w;
  w.li = lane % LPR;
  auto base = [&](const View& vw) {
    return reinterpret_cast<const T*>(vw.p) + (int64_t)b * vw.sb + (int64_t)h * vw.sh;
  };
  auto mbase = [&](const MutView& vw) {
    return reinterpret_cast<T*>(vw.p) + (int64_t)b * vw.sb + (int64_t)h * vw.sh;
  };
  w.q = base(p.q);
  w.k = base(p.k);
  w.v = base(p.v);
  w.go = base(p.dout);
  w.dq = mbase(p.dq);
  w.dk = mbase(p.dk);
  w.dv = mbase(p.dv);
  w.qst = p.q.st;
  w.kst = p.k.st;
  w.vst = p.v.st;
  w.gst = p.dout.st;
  w.dqst = p.dq.st;
  w.dkst = p.dk.st;
  w.dvst = p.dv.st;
  w.lse = p.lse + (int64_t)b * p.T * p.H + h;
  w.lst = p.H;
  w.scale = p.scale;
  w.F = c.F;
  w.T_ = p.T;
  w.Tm1 = p.T - 1;
  w.a = a;
  w.end = min(a + c.P, p.T);
  // Walk u = a-2 .. end+1 (slot of u is (u - a + 2) & 3).
  const int u0 = a - 2, last = w.end + 1;
  w.template prefetch<0>(u0);
  for (int u = u0; u <= last; u += 4) {
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

template <typename T>
__device__ inline Raw load_raw_split(const T* __restrict__ row, int li, int D) {
  constexpr int HV = VecOf<T>::value / 2;
  const uint2 x = *reinterpret_cast<const uint2*>(row + li * HV);
  const uint2 y = *reinterpret_cast<const uint2*>(row + (D >> 1) + li * HV);
  return Raw{{x.x, x.y, y.x, y.y}};
}

template <typename T, int LPR>
struct ProBase {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int HV = VEC / 2;
  using PL = Prologue<T, LPR>;
  const float* __restrict__ rc;
  const float* __restrict__ rs;
  float eps;
  int li, D, Tm1;
  float wq[VEC], wk[VEC];

  __device__ inline void init(const Params& p, int lane_in_row) {
    li = lane_in_row;
    D = p.D;
    Tm1 = p.T - 1;
    rc = p.rope_cos;
    rs = p.rope_sin;
    eps = p.eps;
    PL::load_w(p.wq, li, D, wq);
    PL::load_w(p.wk, li, D, wk);
  }
  __device__ inline void cs(int t, float (&c)[HV], float (&s)[HV]) const {
    PL::load_cs(rc, rs, t, li, D, c, s);
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

  const T* __restrict__ q;
  const T* __restrict__ k;
  const T* __restrict__ v;
  T* __restrict__ o;
  float* __restrict__ lse;
  int64_t qst, kst, vst, ost;
  int lst, F;
  float scale;
  Raw kraw[2], qraw[2], vraw[2], klr[2], vlr[2];
  float cc[2][HV], ss[2][HV], clc[2][HV], cls[2][HV];
  float kq[4][VEC], vr[4][VEC];

  template <int R>
  __device__ inline void prefetch(int t) {
    const int tc = clampi(t, this->Tm1);
    kraw[R & 1] = load_raw_split<T>(k + (int64_t)tc * kst, this->li, this->D);
    qraw[R & 1] = load_raw_split<T>(q + (int64_t)tc * qst, this->li, this->D);
    vraw[R & 1] = load_raw_split<T>(v + (int64_t)tc * vst, this->li, this->D);
    this->cs(tc, cc[R & 1], ss[R & 1]);
    if constexpr (FAR) {
      const int tf = clampi(t - F, this->Tm1);
      klr[R & 1] = load_raw_split<T>(k + (int64_t)tf * kst, this->li, this->D);
      vlr[R & 1] = load_raw_split<T>(v + (int64_t)tf * vst, this->li, this->D);
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
      store_row<T, true>(o + (int64_t)t * ost, this->li, this->D, acc);
      if (this->li == 0) lse[(int64_t)t * lst] = l > 0.f ? m + fast_log(l) : INFINITY;
    }
  }
};

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kWalkBlock) void fwd_pipe_pro(Params p, WalkCfg c) {
  int b, hg, a;
  if (!decode_tile(p, c, wave_id(), b, hg, a)) return;
  const int lane = threadIdx.x & 63;
  const int h = hg * (64 / LPR) + lane / LPR;
  FwdPipePro<T, LPR, NM, FAR> w;
  w.init(p, lane % LPR);
  w.q = reinterpret_cast<const T*>(p.q.p) + (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  w.k = reinterpret_cast<const T*>(p.k.p) + (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  w.v = reinterpret_cast<const T*>(p.v.p) + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  w.o = reinterpret_cast<T*>(p.o.p) + (int64_t)b * p.o.sb + (int64_t)h * p.o.sh;
  w.qst = p.q.st;
  w.kst = p.k.st;
  w.vst = p.v.st;
  w.ost = p.o.st;
  w.lse = p.lse + (int64_t)b * p.T * p.H + h;
  w.lst = p.H;
  w.scale = p.scale;
  w.F = c.F;
  const int end = min(a + c.P, p.T);
  const int t0 = a - 2;   // slot of t is (t - a + 2) & 3
  w.template prefetch<0>(t0);
  for (int t = t0; t < end; t += 4) {
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

  const T* __restrict__ q;
  const T* __restrict__ k;
  const T* __restrict__ v;
  const T* __restrict__ go;
  T* __restrict__ dq;
  const float* __restrict__ lse;
  float* __restrict__ tab;   // (p, scale * dS) per (row, slot)
  int64_t qst, kst, vst, gst, dqst, tst;
  int lst, F, a, end;
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
    kraw[R & 1] = load_raw_split<T>(k + (int64_t)uc * kst, this->li, this->D);
    vr[R] = load_raw_split<T>(v + (int64_t)uc * vst, this->li, this->D);
    qraw[R & 1] = load_raw_split<T>(q + (int64_t)uc * qst, this->li, this->D);
    graw[R & 1] = load_raw_split<T>(go + (int64_t)uc * gst, this->li, this->D);
    lv[R & 1] = lse[(int64_t)uc * lst];
    this->cs(uc, cc[R & 1], ss[R & 1]);
    if constexpr (FAR) {
      const int ul = clampi(u - F, this->Tm1);
      klr[R & 1] = load_raw_split<T>(k + (int64_t)ul * kst, this->li, this->D);
      vlr[R & 1] = load_raw_split<T>(v + (int64_t)ul * vst, this->li, this->D);
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
      store_row<T, true>(dq + (int64_t)u * dqst, this->li, this->D, g);
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

  const T* __restrict__ q;
  const T* __restrict__ k;
  const T* __restrict__ go;
  T* __restrict__ dk;
  T* __restrict__ dv;
  const float* __restrict__ tab;
  int64_t qst, kst, gst, dkst, dvst, tst;
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
    qraw[R & 1] = load_raw_split<T>(q + (int64_t)uc * qst, this->li, this->D);
    gr[R] = load_raw_split<T>(go + (int64_t)uc * gst, this->li, this->D);
    this->cs(uc, cc[R & 1], ss[R & 1]);
    const int j = u - 2;
    const int jc = clampi(j, this->Tm1);
    kraw[R & 1] = load_raw_split<T>(k + (int64_t)jc * kst, this->li, this->D);
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
      qir[R & 1] = load_raw_split<T>(q + (int64_t)ic * qst, this->li, this->D);
      gir[R & 1] = load_raw_split<T>(go + (int64_t)ic * gst, this->li, this->D);
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
      store_row<T, true>(dk + (int64_t)j * dkst, this->li, this->D, ak);
      store_row<T, true>(dv + (int64_t)j * dvst, this->li, this->D, av);
    }
  }
};

template <typename W>
__device__ inline void walk4(W& w, int first, int last) {
  w.template prefetch<0>(first);
  for (int u = first; u <= last; u += 4) {
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

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kWalkBlock) void bwd_q_pro(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value;
  const int64_t wave = wave_id();
  int b, hg, a;
  const bool live = decode_tile(p, c, wave, b, hg, a);
  const int lane = threadIdx.x & 63;
  BwdQPro<T, LPR, NM, FAR> w;
#pragma unroll
  for (int e = 0; e < VEC; ++e) w.dw[e] = 0.f;
  if (live) {
    const int h = hg * (64 / LPR) + lane / LPR;
    w.init(p, lane % LPR);
    auto base = [&](const View& vw) {
      return reinterpret_cast<const T*>(vw.p) + (int64_t)b * vw.sb + (int64_t)h * vw.sh;
    };
    w.q = base(p.q);
    w.k = base(p.k);
    w.v = base(p.v);
    w.go = base(p.dout);
    w.dq = reinterpret_cast<T*>(p.dq.p) + (int64_t)b * p.dq.sb + (int64_t)h * p.dq.sh;
    w.qst = p.q.st;
    w.kst = p.k.st;
    w.vst = p.v.st;
    w.gst = p.dout.st;
    w.dqst = p.dq.st;
    w.lse = p.lse + (int64_t)b * p.T * p.H + h;
    w.lst = p.H;
    w.tab = p.tab + ((int64_t)b * p.T * p.H + h) * (2 * w.NS);
    w.tst = (int64_t)p.H * 2 * w.NS;
    w.scale = p.scale;
    w.F = c.F;
    w.a = a;
    w.end = min(a + c.P, p.T);
    // Queries a-2, a-1 only fill the near-source rotation (slot of u is (u - a + 2) & 3).
    walk4(w, a - 2, w.end - 1);
  }
  write_wave_partial<T, LPR, true>(w.dw, p.dwq_part, wave, p.D);
}

template <typename T, int LPR, int NM, bool FAR>
__global__ __launch_bounds__(kWalkBlock) void bwd_k_pro(Params p, WalkCfg c) {
  constexpr int VEC = VecOf<T>::value;
  const int64_t wave = wave_id();
  int b, hg, a;
  const bool live = decode_tile(p, c, wave, b, hg, a);
  const int lane = threadIdx.x & 63;
  BwdKPro<T, LPR, NM, FAR> w;
#pragma unroll
  for (int e = 0; e < VEC; ++e) w.dw[e] = 0.f;
  if (live) {
    const int h = hg * (64 / LPR) + lane / LPR;
    w.init(p, lane % LPR);
    auto base = [&](const View& vw) {
      return reinterpret_cast<const T*>(vw.p) + (int64_t)b * vw.sb + (int64_t)h * vw.sh;
    };
    w.q = base(p.q);
    w.k = base(p.k);
    w.go = base(p.dout);
    w.dk = reinterpret_cast<T*>(p.dk.p) + (int64_t)b * p.dk.sb + (int64_t)h * p.dk.sh;
    w.dv = reinterpret_cast<T*>(p.dv.p) + (int64_t)b * p.dv.sb + (int64_t)h * p.dv.sh;
    w.qst = p.q.st;
    w.kst = p.k.st;
    w.gst = p.dout.st;
    w.dkst = p.dk.st;
    w.dvst = p.dv.st;
    w.tab = p.tab + ((int64_t)b * p.T * p.H + h) * (2 * w.NS);
    w.tst = (int64_t)p.H * 2 * w.NS;
    w.F = c.F;
    w.a = a;
    w.end = min(a + c.P, p.T);
    w.T_ = p.T;
    // Walk u = a .. end+1 (slot of u is (u - a) & 3); key u - 2 is finished at step u.
    walk4(w, a, w.end + 1);
  }
  write_wave_partial<T, LPR, true>(w.dw, p.dwk_part, wave, p.D);
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

WalkCfg make_cfg(const Params& p, int lpr, const Pattern& pat) {
  WalkCfg c{};
  c.HG = p.H / (64 / lpr);
  const int64_t lanes_rows = (int64_t)p.B * c.HG;
  // About 8192 tiles fill 256 CUs several times over; the tile is at least
  // 16 positions (halo overhead <= 2/16) and at most 256.
  int P = 256;
  while (P > 16 && lanes_rows * ((p.T + P - 1) / P) < 8192) P >>= 1;
  // A far offset inside the tile would make a wave re-read rows it loaded F
  // steps earlier, long evicted from L2.  With the tile shrunk to F the far
  // rows belong to the neighbouring tile, which a neighbouring wave walks at
  // the same time, so they are L2 hits.
  if (pat.far >= 16 && pat.far < P && (pat.far & (pat.far - 1)) == 0) P = pat.far;
  c.P = P;
  c.F = pat.far;
  if (pat.far >= P && pat.far % P == 0) {
    c.column = 1;
    c.rows = (p.T + pat.far - 1) / pat.far;
    c.tiles_t = c.rows * (pat.far / P);
  } else {
    c.column = 0;
    c.rows = 0;
    c.tiles_t = (p.T + P - 1) / P;
  }
  c.total = lanes_rows * c.tiles_t;
  c.nwg = (int)((c.total + kWaves - 1) / kWaves);
  return c;
}

template <typename T, int LPR, bool PRO, bool FWD>
hipError_t launch_pattern(const Params& p, const WalkCfg& c, const Pattern& pat, hipStream_t st) {
  const dim3 grid((unsigned)c.nwg), block(kWalkBlock);
#define SBDA_WALK_CASE(NMV, FARV)                                                            \
  if (pat.nm == NMV && (pat.far != 0) == FARV) {                                             \
    if (FWD && PRO) {                                                                        \
      hipLaunchKernelGGL((fwd_pipe_pro<T, LPR, NMV, FARV>), grid, block, 0, st, p, c);      \
    } else if (FWD) {                                                                        \
      hipLaunchKernelGGL((fwd_pipe<T, LPR, NMV, FARV>), grid, block, 0, st, p, c);          \
    } else if (PRO) {                                                                        \
      hipLaunchKernelGGL((bwd_q_pro<T, LPR, NMV, FARV>), grid, block, 0, st, p, c);         \
      hipError_t e_ = hipGetLastError();                                                     \
      if (e_ != hipSuccess) return e_;                                                       \
      hipLaunchKernelGGL((bwd_k_pro<T, LPR, NMV, FARV>), grid, block, 0, st, p, c);         \
    } else {                                                                                 \
      hipLaunchKernelGGL((bwd_pipe<T, LPR, NMV, FARV>), grid, block, 0, st, p, c);          \
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

template <typename T>
struct TypeTag {
  using type = T;
};

template <bool FWD>
hipError_t walk_launch(const Params& p, int dtype, bool pro, hipStream_t st) {
  Pattern pat;
  if (!classify(p, &pat)) return hipErrorInvalidValue;
  const int lpr = walk_lpr(p, dtype);
  const WalkCfg c = make_cfg(p, lpr, pat);
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

bool walk_applies(const Params& p, int dtype) {
  Pattern pat;
  if (p.group != 1 || p.seg != nullptr || !classify(p, &pat)) return false;
  const int lpr = walk_lpr(p, dtype);
  if (lpr == 0) return false;
  return p.H % (64 / lpr) == 0;
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
  const WalkCfg c = make_cfg(p, walk_lpr(p, dtype), pat);
  *pq = (int64_t)c.nwg * kWaves;
  *pk = *pq;
  *tab_floats = (int64_t)p.B * p.T * p.H * 2 * p.S;
}

}  // namespace sbda
