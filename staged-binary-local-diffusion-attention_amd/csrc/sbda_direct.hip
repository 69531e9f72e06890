// Row-parallel SBDA kernels for every supported shape.
//
// One lane group (LPR lanes) owns one row and reads each of its sources
// straight from global memory; neighbouring rows' re-reads are served by the
// caches.  These kernels accept any batch/head/GQA/head_dim/stride/offset
// combination the C ABI validates.  The wavefront-walk kernels in
// sbda_walk.hip are used instead where their layout applies.
//
// Maths (per batch b, query head h, kv head hk = h / group, query row i,
// slot s with source j = i - off[s], valid iff j >= 0; reference
// BiAttn/left_v2.py:313-405 and BiAttn/sbda_triton.py:135-201,507-671):
//   score_s = (q_i . k_j) * scale,     p = softmax over valid slots,
//   o_i = sum_s p_s v_j,               lse_i = log sum_valid exp(score_s),
//   dP_s = dO_i . v_j,  delta_i = sum_s p_s dP_s,  dS_s = p_s (dP_s - delta_i),
//   dQ_i = scale sum_s dS_s k_j,
//   dK_j = scale sum_{h in group} sum_t dS_t(i = j + off[t]) q_i   (i < T),
//   dV_j =       sum_{h in group} sum_t p_t(i = j + off[t]) dO_i.
// A row with no valid source has o = 0, gradient 0 and lse = +inf.
//
// Backward in two passes, neither with atomics: bwd_dq_direct computes each
// query row's p_s and dS_s once, writes dQ and stores (p_s, scale * dS_s) in
// a workspace table; bwd_dkv_direct sums, per kv row j, the table entries of
// the queries j + off[t] (over the group's query heads) against their q and
// dO rows.

#include "sbda_rows.h"

namespace sbda {

// ----------------------------------------------------------------- forward

template <typename T, int LPR, bool PRO>
__global__ __launch_bounds__(kBlock) void fwd_direct(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.H;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;  // keep every lane in the row reductions
  int b, t, h;
  decode_row(row, p.H, p.T, b, t, h);
  const int hk = h / p.group;

  float q[VEC];
  load_row<T, PRO>(row_ptr<T>(p.q, b, h, t), li, p.D, q);
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float c[PL::HV], s[PL::HV];
    PL::load_cs(p.rope_cos, p.rope_sin, t, li, p.D, c, s);
    PL::forward(q, p.wq, c, s, li, p.D, p.eps);
  }

  float sc[kMaxSlots];
  int src[kMaxSlots];
  float m = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxSlots; ++s) {
    if (s < p.S) {
      const int j = t - p.off[s];
      float k[VEC];
      load_key<T, LPR, PRO>(p, b, hk, j >= 0 ? j : 0, li, k);
      const float d = row_sum<LPR>(dot_partial<VEC>(q, k)) * p.scale;
      const bool ok = j >= 0 && same_segment(p, b, t, j);
      src[s] = ok ? j : -1;
      sc[s] = ok ? d : -INFINITY;
      m = fmaxf(m, sc[s]);
    }
  }
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
  float l = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSlots; ++s) {
    if (s < p.S) {
      const int j = src[s];
      const float w = j >= 0 ? fast_exp(sc[s] - m) : 0.f;
      l += w;
      float v[VEC];
      load_row<T, PRO>(row_ptr<T>(p.v, b, hk, j >= 0 ? j : 0), li, p.D, v);
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[i] = __builtin_fmaf(w, v[i], acc[i]);
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] *= inv;
  if (live) {
    store_row<T, PRO>(row_ptr<T>(p.o, b, h, t), li, p.D, acc);
    if (li == 0) p.lse[((int64_t)b * p.T + t) * p.H + h] = l > 0.f ? m + fast_log(l) : INFINITY;
  }
}

// -------------------------------------------------------------- query side
//
// Recomputes, for query row (b, i, h): its (roped) q, dO, per-slot weights
// p_s and score gradients dS_s.  Keys of the sources are returned in `kk`
// when WANT_K (for dQ).
template <typename T, int LPR, bool PRO, bool WANT_K>
__device__ inline void query_side(const Params& p, int b, int i, int h, int hk, int li,
                                  float (&q)[VecOf<T>::value], float (&go)[VecOf<T>::value],
                                  float (&pp)[kMaxSlots], float (&ds)[kMaxSlots],
                                  float (&kk)[kMaxSlots][VecOf<T>::value]) {
  constexpr int VEC = VecOf<T>::value;
  load_row<T, PRO>(row_ptr<T>(p.q, b, h, i), li, p.D, q);
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float c[PL::HV], s[PL::HV];
    PL::load_cs(p.rope_cos, p.rope_sin, i, li, p.D, c, s);
    PL::forward(q, p.wq, c, s, li, p.D, p.eps);
  }
  load_row<T, PRO>(row_ptr<T>(p.dout, b, h, i), li, p.D, go);
  const float lse = p.lse[((int64_t)b * p.T + i) * p.H + h];
  float dp[kMaxSlots];
  float delta = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSlots; ++s) {
    pp[s] = 0.f;
    dp[s] = 0.f;
    if (s < p.S) {
      const int j = i - p.off[s];
      const int jc = j >= 0 ? j : 0;
      float k[VEC], v[VEC];
      load_key<T, LPR, PRO>(p, b, hk, jc, li, k);
      load_row<T, PRO>(row_ptr<T>(p.v, b, hk, jc), li, p.D, v);
      const float sc = row_sum<LPR>(dot_partial<VEC>(q, k)) * p.scale;
      const float d = row_sum<LPR>(dot_partial<VEC>(go, v));
      const bool ok = j >= 0 && same_segment(p, b, i, j);
      pp[s] = ok ? fast_exp(sc - lse) : 0.f;  // lse = +inf -> 0
      dp[s] = d;
      delta = __builtin_fmaf(pp[s], d, delta);
      if constexpr (WANT_K) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kk[s][e] = k[e];
      }
    }
  }
#pragma unroll
  for (int s = 0; s < kMaxSlots; ++s) ds[s] = pp[s] * (dp[s] - delta);
}

// ------------------------------------------------------------ backward: dQ

template <typename T, int LPR, bool PRO>
__global__ __launch_bounds__(kBlock) void bwd_dq_direct(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.H;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;
  int b, t, h;
  decode_row(row, p.H, p.T, b, t, h);
  const int hk = h / p.group;

  float q[VEC], go[VEC], pp[kMaxSlots], ds[kMaxSlots], kk[kMaxSlots][VEC];
  query_side<T, LPR, PRO, true>(p, b, t, h, hk, li, q, go, pp, ds, kk);
  float dq[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    float a = 0.f;
#pragma unroll
    for (int s = 0; s < kMaxSlots; ++s)
      if (s < p.S) a = __builtin_fmaf(ds[s], kk[s][e], a);
    dq[e] = a * p.scale;
  }
  // (p_s, scale * dS_s) of this row for the key pass.
  if (live && li == 0) {
    float2* tab = reinterpret_cast<float2*>(p.tab) + row * p.S;
#pragma unroll
    for (int s = 0; s < kMaxSlots; ++s)
      if (s < p.S) tab[s] = make_float2(pp[s], ds[s] * p.scale);
  }
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float x[VEC], c[PL::HV], s[PL::HV], dw[VEC];
    load_row<T, true>(row_ptr<T>(p.q, b, h, t), li, p.D, x);
    PL::load_cs(p.rope_cos, p.rope_sin, t, li, p.D, c, s);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss = __builtin_fmaf(x[e], x[e], ss);
    ss = row_sum<LPR>(ss);
    const float r = norm_rsqrt<T>(__fadd_rn(__fdiv_rn(ss, (float)p.D), p.eps));
#pragma unroll
    for (int e = 0; e < VEC; ++e) dw[e] = 0.f;
    PL::backward(dq, x, r, p.wq, c, s, li, p.D, dw);
    if (!live) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dw[e] = 0.f;
    }
    block_reduce_dw<T, LPR, true>(dw, p.D, p.dwq_part + (int64_t)blockIdx.x * p.D);
  }
  if (live) store_row<T, PRO>(row_ptr<T>(p.dq, b, h, t), li, p.D, dq);
}

// ---------------------------------------------------------- backward: dK dV

template <typename T, int LPR, bool PRO>
__global__ __launch_bounds__(kBlock) void bwd_dkv_direct(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.Hkv;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;
  int b, j, hk;
  decode_row(row, p.Hkv, p.T, b, j, hk);

  // Query i = j + off[t] reads key j through slot t; its weight p_t and
  // scale * dS_t come from the table the dQ pass wrote.
  const float2* tab = reinterpret_cast<const float2*>(p.tab);
  float dk[VEC], dv[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) { dk[e] = 0.f; dv[e] = 0.f; }
  for (int g = 0; g < p.group; ++g) {
    const int h = hk * p.group + g;
#pragma unroll
    for (int tslot = 0; tslot < kMaxSlots; ++tslot) {
      if (tslot < p.S) {
        const int64_t i64 = (int64_t)j + p.off[tslot];
        const bool ok = i64 < p.T;
        const int i = ok ? (int)i64 : j;
        float2 w = tab[(((int64_t)b * p.T + i) * p.H + h) * p.S + tslot];
        if (!ok) w = make_float2(0.f, 0.f);
        float q[VEC], go[VEC];
        load_row<T, PRO>(row_ptr<T>(p.q, b, h, i), li, p.D, q);
        if constexpr (PRO) {
          using PL = Prologue<T, LPR>;
          float c[PL::HV], sn[PL::HV];
          PL::load_cs(p.rope_cos, p.rope_sin, i, li, p.D, c, sn);
          PL::forward(q, p.wq, c, sn, li, p.D, p.eps);
        }
        load_row<T, PRO>(row_ptr<T>(p.dout, b, h, i), li, p.D, go);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          dk[e] = __builtin_fmaf(w.y, q[e], dk[e]);
          dv[e] = __builtin_fmaf(w.x, go[e], dv[e]);
        }
      }
    }
  }
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float x[VEC], c[PL::HV], s[PL::HV], dw[VEC];
    load_row<T, true>(row_ptr<T>(p.k, b, hk, j), li, p.D, x);
    PL::load_cs(p.rope_cos, p.rope_sin, j, li, p.D, c, s);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss = __builtin_fmaf(x[e], x[e], ss);
    ss = row_sum<LPR>(ss);
    const float r = norm_rsqrt<T>(__fadd_rn(__fdiv_rn(ss, (float)p.D), p.eps));
#pragma unroll
    for (int e = 0; e < VEC; ++e) dw[e] = 0.f;
    PL::backward(dk, x, r, p.wk, c, s, li, p.D, dw);
    if (!live) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dw[e] = 0.f;
    }
    block_reduce_dw<T, LPR, true>(dw, p.D, p.dwk_part + (int64_t)blockIdx.x * p.D);
  }
  if (live) {
    store_row<T, PRO>(row_ptr<T>(p.dk, b, hk, j), li, p.D, dk);
    store_row<T, PRO>(row_ptr<T>(p.dv, b, hk, j), li, p.D, dv);
  }
}

// ------------------------------------------------------------ dispatchers

template <typename T, bool PRO>
struct DirectLaunch {
  template <int LPR>
  static hipError_t fwd(const Params& p, hipStream_t st) {
    const int64_t rows = (int64_t)p.B * p.T * p.H;
    const int64_t blocks = (rows * LPR + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((fwd_direct<T, LPR, PRO>), dim3((unsigned)blocks), dim3(kBlock), 0, st, p);
    return hipGetLastError();
  }
  template <int LPR>
  static hipError_t bwd(const Params& p, hipStream_t st) {
    const int64_t qrows = (int64_t)p.B * p.T * p.H;
    const int64_t krows = (int64_t)p.B * p.T * p.Hkv;
    const int64_t qb = (qrows * LPR + kBlock - 1) / kBlock;
    const int64_t kb = (krows * LPR + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((bwd_dq_direct<T, LPR, PRO>), dim3((unsigned)qb), dim3(kBlock), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_dkv_direct<T, LPR, PRO>), dim3((unsigned)kb), dim3(kBlock), 0, st, p);
    return hipGetLastError();
  }
};


template <typename T, bool PRO>
static hipError_t direct_forward_t(const Params& p, hipStream_t st) {
  const int lpr = lanes_per_row(p.D, sizeof(T));
  return by_lpr(lpr, [&](auto c) { return DirectLaunch<T, PRO>::template fwd<decltype(c)::value>(p, st); });
}

template <typename T, bool PRO>
static hipError_t direct_backward_t(const Params& p, hipStream_t st) {
  const int lpr = lanes_per_row(p.D, sizeof(T));
  return by_lpr(lpr, [&](auto c) { return DirectLaunch<T, PRO>::template bwd<decltype(c)::value>(p, st); });
}

hipError_t direct_forward(const Params& p, int dtype, bool pro, hipStream_t st) {
  switch (dtype) {
    case kBF16: return pro ? direct_forward_t<__bf16, true>(p, st) : direct_forward_t<__bf16, false>(p, st);
    case kFP16: return pro ? direct_forward_t<_Float16, true>(p, st) : direct_forward_t<_Float16, false>(p, st);
    case kFP32: return pro ? direct_forward_t<float, true>(p, st) : direct_forward_t<float, false>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t direct_backward(const Params& p, int dtype, bool pro, hipStream_t st) {
  switch (dtype) {
    case kBF16: return pro ? direct_backward_t<__bf16, true>(p, st) : direct_backward_t<__bf16, false>(p, st);
    case kFP16: return pro ? direct_backward_t<_Float16, true>(p, st) : direct_backward_t<_Float16, false>(p, st);
    case kFP32: return pro ? direct_backward_t<float, true>(p, st) : direct_backward_t<float, false>(p, st);
    default: return hipErrorInvalidValue;
  }
}

// Workspace of the generic backward: weight-gradient partial rows (with the
// prologue) and the (p, scale * dS) table, fp32 pairs per (row, slot).
void direct_partials(const Params& p, int esz, int64_t* parts_q, int64_t* parts_k,
                     int64_t* tab_floats) {
  *tab_floats = (int64_t)p.B * p.T * p.H * 2 * p.S;
  const int lpr = lanes_per_row(p.D, esz);
  const int64_t qrows = (int64_t)p.B * p.T * p.H;
  const int64_t krows = (int64_t)p.B * p.T * p.Hkv;
  *parts_q = (qrows * lpr + kBlock - 1) / kBlock;
  *parts_k = (krows * lpr + kBlock - 1) / kBlock;
}

// ------------------------------------------------------- partial reduction

constexpr int kReduceBlock = 256;

// Column sums of one or two partial-row arrays ([parts, D] fp32 each): block
// d < D sums column d of the first array, block D + d column d of the
// second, each in a fixed order (deterministic).  The prologue backward's two
// norm-weight gradients take one launch.
struct PartialSet {
  const float* part;
  int64_t parts;
  float* out;
};

__global__ __launch_bounds__(kReduceBlock) void reduce_partials_kernel(PartialSet a, PartialSet b,
                                                                       int D) {
  __shared__ float buf[kReduceBlock];
  const bool second = (int)blockIdx.x >= D;
  const float* part = second ? b.part : a.part;
  const int64_t parts = second ? b.parts : a.parts;
  float* out = second ? b.out : a.out;
  const int d = second ? (int)blockIdx.x - D : (int)blockIdx.x;
  float acc = 0.f;
  for (int64_t k = threadIdx.x; k < parts; k += kReduceBlock) acc += part[k * D + d];
  buf[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kReduceBlock / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) buf[threadIdx.x] += buf[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[d] = buf[0];
}

hipError_t launch_reduce_partials(const float* part, int64_t parts, int D, float* out, hipStream_t st) {
  const PartialSet a{part, parts, out};
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((unsigned)D), dim3(kReduceBlock), 0, st, a, a, D);
  return hipGetLastError();
}

hipError_t launch_reduce_partials2(const float* part_a, int64_t parts_a, float* out_a,
                                   const float* part_b, int64_t parts_b, float* out_b, int D,
                                   hipStream_t st) {
  const PartialSet a{part_a, parts_a, out_a}, b{part_b, parts_b, out_b};
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(2u * (unsigned)D), dim3(kReduceBlock), 0, st, a, b,
                     D);
  return hipGetLastError();
}

// --------------------------------------------------------------- RoPE table
//
// cos/sin[t, i] = cos/sin(fl32(t * inv_freq[i])) in fp32: the reference
// builds its angles as an fp32 outer product (BiAttn/attention_common.py:
// 18-21); inv_freq is computed on the host with the reference's own fp32
// expression so the angles agree bit for bit.
struct InvFreq {
  float v[256];
};

__global__ __launch_bounds__(256) void rope_table_kernel(float* __restrict__ cos_out,
                                                         float* __restrict__ sin_out, InvFreq f,
                                                         int64_t length, int half) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= length * half) return;
  const int64_t t = idx / half;
  const int i = (int)(idx % half);
  const float ang = __fmul_rn((float)t, f.v[i]);
  float s, c;
  sincosf(ang, &s, &c);
  cos_out[idx] = c;
  sin_out[idx] = s;
}

hipError_t launch_rope_table(float* cos_out, float* sin_out, const float* inv_freq_host,
                             int64_t length, int half, hipStream_t st) {
  if (half > 256) return hipErrorInvalidValue;
  InvFreq f;
  for (int i = 0; i < 256; ++i) f.v[i] = i < half ? inv_freq_host[i] : 0.f;
  const int64_t n = length * half;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     cos_out, sin_out, f, length, half);
  return hipGetLastError();
}

}  // namespace sbda
