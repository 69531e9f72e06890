// SBDA attention over caller-supplied source tables.
//
// The reference's eager route accepts per-query source tables
// `path_indices [B, T, S]` (int64) with `path_valid [B, T, S]` (bool) instead
// of the layer's offsets (BiAttn/left_v2.py:212-231,313-378; produced for the
// greedy H4 schedule by BinaryDiffusionAttention/run_mini_experiment.py:117-133).
// Source s of query i is j = path_indices[b, i, s]; it counts when
// path_valid[b, i, s] is set, j <= i (causal, left_v2.py:355-357), j >= 0 and,
// with segment keys, key[j] == key[i] >= 0.  Any S >= 1, duplicates allowed
// (a source listed twice enters the softmax twice, as in the reference).
//
// Forward: one lane group per row, online softmax over the S sources, one fp32
// log-normaliser per row.  Backward, deterministic and atomic-free:
//   1. `path_keys`: each (b, i, s) entry gets the key b*T + j (or B*T when it
//      does not count) and the value i*S + s;
//   2. a stable LSD radix sort (rocPRIM, only the bits of the largest key)
//      orders entries by key, ties keep their (i, s) order;
//   3. `path_starts`: per key, the first sorted entry (binary search);
//   4. `bwd_q_paths`: dQ per query row, and per (row, slot) the pair
//      (p, scale * dS) into a table;
//   5. `bwd_kv_paths`: dK/dV per key row from the table entries of the
//      queries that read it, in sorted (i, s) order.

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>

#include "sbda_rows.h"

namespace sbda {

// Source j of (b, i, slot s) in table mode, or -1 when it does not count.
__device__ inline int path_source(const Params& p, int b, int i, int s) {
  const int64_t e = ((int64_t)b * p.T + i) * p.PS + s;
  const int64_t j = p.pidx[e];
  bool ok = j >= 0 && j <= i;
  if (p.pvalid != nullptr) ok = ok && p.pvalid[e] != 0;
  ok = ok && same_segment(p, b, i, (int)(ok ? j : i));
  return ok ? (int)j : -1;
}

// ----------------------------------------------------------------- forward

template <typename T, int LPR, bool PRO>
__global__ __launch_bounds__(kBlock) void fwd_paths(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.H;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;
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
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  float m = -INFINITY, l = 0.f;
  for (int s = 0; s < p.PS; ++s) {
    const int j = path_source(p, b, t, s);
    const int jc = j >= 0 ? j : t;
    float k[VEC], v[VEC];
    load_key<T, LPR, PRO>(p, b, hk, jc, li, k);
    load_row<T, PRO>(row_ptr<T>(p.v, b, hk, jc), li, p.D, v);
    const float sc = row_sum<LPR>(dot_partial<VEC>(q, k)) * p.scale;
    if (j >= 0) {
      const float mn = fmaxf(m, sc);
      const float c = fast_exp(m - mn);  // 0 while m = -inf
      const float w = fast_exp(sc - mn);
      l = __builtin_fmaf(l, c, w);
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = __builtin_fmaf(acc[e], c, w * v[e]);
      m = mn;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] *= inv;
  if (live) {
    store_row<T, PRO>(row_ptr<T>(p.o, b, h, t), li, p.D, acc);
    if (li == 0) p.lse[((int64_t)b * p.T + t) * p.H + h] = l > 0.f ? m + fast_log(l) : INFINITY;
  }
}

// --------------------------------------------------------- inverse index

__global__ __launch_bounds__(kBlock) void path_keys(Params p, uint32_t* __restrict__ keys,
                                                     uint32_t* __restrict__ vals) {
  const int64_t n = (int64_t)p.B * p.T * p.PS;
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n) return;
  const int s = (int)(e % p.PS);
  const int64_t bi = e / p.PS;
  const int i = (int)(bi % p.T);
  const int b = (int)(bi / p.T);
  const int j = path_source(p, b, i, s);
  keys[e] = j >= 0 ? (uint32_t)((int64_t)b * p.T + j) : (uint32_t)((int64_t)p.B * p.T);
  vals[e] = (uint32_t)((int64_t)i * p.PS + s);
}

// start[key] = first sorted entry with that key (key = 0 .. B*T; the last
// start is the count of counted entries).
__global__ __launch_bounds__(kBlock) void path_starts(const uint32_t* __restrict__ sorted,
                                                       int64_t n, int64_t keys,
                                                       uint32_t* __restrict__ start) {
  const int64_t key = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (key > keys) return;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)sorted[mid] < key) lo = mid + 1; else hi = mid;
  }
  start[key] = (uint32_t)lo;
}

// ------------------------------------------------------------ backward: dQ

template <typename T, int LPR, bool PRO>
__global__ __launch_bounds__(kBlock) void bwd_q_paths(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.H;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;
  int b, t, h;
  decode_row(row, p.H, p.T, b, t, h);
  const int hk = h / p.group;

  float q[VEC], go[VEC];
  load_row<T, PRO>(row_ptr<T>(p.q, b, h, t), li, p.D, q);
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float c[PL::HV], s[PL::HV];
    PL::load_cs(p.rope_cos, p.rope_sin, t, li, p.D, c, s);
    PL::forward(q, p.wq, c, s, li, p.D, p.eps);
  }
  load_row<T, PRO>(row_ptr<T>(p.dout, b, h, t), li, p.D, go);
  const float lse = p.lse[((int64_t)b * p.T + t) * p.H + h];

  // Pass 1: delta = sum_s p_s dP_s.
  float delta = 0.f;
  for (int s = 0; s < p.PS; ++s) {
    const int j = path_source(p, b, t, s);
    const int jc = j >= 0 ? j : t;
    float k[VEC], v[VEC];
    load_key<T, LPR, PRO>(p, b, hk, jc, li, k);
    load_row<T, PRO>(row_ptr<T>(p.v, b, hk, jc), li, p.D, v);
    const float sc = row_sum<LPR>(dot_partial<VEC>(q, k)) * p.scale;
    const float dp = row_sum<LPR>(dot_partial<VEC>(go, v));
    const float pw = j >= 0 ? fast_exp(sc - lse) : 0.f;
    delta = __builtin_fmaf(pw, dp, delta);
  }
  // Pass 2: dS_s, dQ and the (p, scale * dS) table.
  float dq[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) dq[e] = 0.f;
  float2* tab = reinterpret_cast<float2*>(p.tab) + row * p.PS;
  for (int s = 0; s < p.PS; ++s) {
    const int j = path_source(p, b, t, s);
    const int jc = j >= 0 ? j : t;
    float k[VEC], v[VEC];
    load_key<T, LPR, PRO>(p, b, hk, jc, li, k);
    load_row<T, PRO>(row_ptr<T>(p.v, b, hk, jc), li, p.D, v);
    const float sc = row_sum<LPR>(dot_partial<VEC>(q, k)) * p.scale;
    const float dp = row_sum<LPR>(dot_partial<VEC>(go, v));
    const float pw = j >= 0 ? fast_exp(sc - lse) : 0.f;
    const float ds = pw * (dp - delta) * p.scale;
#pragma unroll
    for (int e = 0; e < VEC; ++e) dq[e] = __builtin_fmaf(ds, k[e], dq[e]);
    if (live && li == 0) tab[s] = make_float2(pw, ds);
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
__global__ __launch_bounds__(kBlock) void bwd_kv_paths(Params p) {
  constexpr int VEC = VecOf<T>::value;
  const int li = threadIdx.x % LPR;
  const int64_t nrows = (int64_t)p.B * p.T * p.Hkv;
  int64_t row = ((int64_t)blockIdx.x * kBlock + threadIdx.x) / LPR;
  const bool live = row < nrows;
  if (!live) row = 0;
  int b, j, hk;
  decode_row(row, p.Hkv, p.T, b, j, hk);
  const int64_t key = (int64_t)b * p.T + j;
  const uint32_t first = live ? p.inv_start[key] : 0u;
  const uint32_t last = live ? p.inv_start[key + 1] : 0u;
  const float2* tab = reinterpret_cast<const float2*>(p.tab);

  float dk[VEC], dv[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) { dk[e] = 0.f; dv[e] = 0.f; }
  for (int g = 0; g < p.group; ++g) {
    const int h = hk * p.group + g;
    for (uint32_t x = first; x < last; ++x) {
      const uint32_t ent = p.inv_entry[x];
      const int i = (int)(ent / (uint32_t)p.PS);
      const int s = (int)(ent % (uint32_t)p.PS);
      const float2 w = tab[(((int64_t)b * p.T + i) * p.H + h) * p.PS + s];
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

// ------------------------------------------------------------- launchers

namespace {

int end_bit(int64_t max_key) {
  int bits = 1;
  while (bits < 32 && (int64_t(1) << bits) <= max_key) ++bits;
  return bits;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

int64_t sort_temp_bytes(int64_t n, int64_t max_key) {
  size_t bytes = 0;
  if (rocprim::radix_sort_pairs(nullptr, bytes, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                (const uint32_t*)nullptr, (uint32_t*)nullptr, (size_t)n, 0,
                                (unsigned)end_bit(max_key), (hipStream_t)0) != hipSuccess)
    return -1;
  return (int64_t)bytes;
}

template <typename T, bool PRO>
hipError_t paths_forward_t(const Params& p, hipStream_t st) {
  return by_lpr(lanes_per_row(p.D, sizeof(T)), [&](auto c) {
    constexpr int LPR = decltype(c)::value;
    const int64_t rows = (int64_t)p.B * p.T * p.H;
    const int64_t blocks = (rows * LPR + kBlock - 1) / kBlock;
    hipLaunchKernelGGL((fwd_paths<T, LPR, PRO>), dim3((unsigned)blocks), dim3(kBlock), 0, st, p);
    return hipGetLastError();
  });
}

template <typename T, bool PRO>
hipError_t paths_backward_t(const Params& p, hipStream_t st) {
  return by_lpr(lanes_per_row(p.D, sizeof(T)), [&](auto c) {
    constexpr int LPR = decltype(c)::value;
    const int64_t qrows = (int64_t)p.B * p.T * p.H;
    const int64_t krows = (int64_t)p.B * p.T * p.Hkv;
    hipLaunchKernelGGL((bwd_q_paths<T, LPR, PRO>), dim3((unsigned)((qrows * LPR + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((bwd_kv_paths<T, LPR, PRO>), dim3((unsigned)((krows * LPR + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, st, p);
    return hipGetLastError();
  });
}

}  // namespace

// Workspace of the table-mode backward, in bytes: the (p, scale*dS) table,
// sort keys/values (in and out), key starts, the sort's temporary storage and
// (with the prologue) the weight-gradient partial rows.  Returns -1 when the
// sort cannot size its storage.
int64_t paths_workspace(const Params& p, int esz, bool pro, int64_t* parts_q, int64_t* parts_k) {
  const int64_t bt = (int64_t)p.B * p.T;
  const int64_t n = bt * p.PS;
  const int64_t temp = sort_temp_bytes(n, bt);
  if (temp < 0) return -1;
  int64_t bytes = align256(bt * p.H * p.PS * 8);          // table
  bytes += 4 * align256(n * 4);                            // keys, values: in and out
  bytes += align256((bt + 1) * 4);                         // starts
  bytes += align256(temp);
  *parts_q = *parts_k = 0;
  if (pro) {
    const int lpr = lanes_per_row(p.D, esz);
    *parts_q = ((bt * p.H) * lpr + kBlock - 1) / kBlock;
    *parts_k = ((bt * p.Hkv) * lpr + kBlock - 1) / kBlock;
    bytes += align256((*parts_q + *parts_k) * p.D * 4);
  }
  return bytes;
}

hipError_t paths_forward(const Params& p, int dtype, bool pro, hipStream_t st) {
  switch (dtype) {
    case kBF16: return pro ? paths_forward_t<__bf16, true>(p, st) : paths_forward_t<__bf16, false>(p, st);
    case kFP16: return pro ? paths_forward_t<_Float16, true>(p, st) : paths_forward_t<_Float16, false>(p, st);
    case kFP32: return pro ? paths_forward_t<float, true>(p, st) : paths_forward_t<float, false>(p, st);
    default: return hipErrorInvalidValue;
  }
}

// Carves the workspace (same order as paths_workspace), builds the inverse
// index and runs both backward kernels.  `pp` receives the partial-row
// pointers for the caller's final reduction.
hipError_t paths_backward(Params p, int dtype, bool pro, void* ws, int64_t parts_q, hipStream_t st,
                          float** dwq_part, float** dwk_part) {
  const int64_t bt = (int64_t)p.B * p.T;
  const int64_t n = bt * p.PS;
  char* w = static_cast<char*>(ws);
  p.tab = reinterpret_cast<float*>(w);
  w += align256(bt * p.H * p.PS * 8);
  uint32_t* keys_in = reinterpret_cast<uint32_t*>(w);
  w += align256(n * 4);
  uint32_t* keys_out = reinterpret_cast<uint32_t*>(w);
  w += align256(n * 4);
  uint32_t* vals_in = reinterpret_cast<uint32_t*>(w);
  w += align256(n * 4);
  uint32_t* vals_out = reinterpret_cast<uint32_t*>(w);
  w += align256(n * 4);
  uint32_t* starts = reinterpret_cast<uint32_t*>(w);
  w += align256((bt + 1) * 4);
  const int64_t temp = sort_temp_bytes(n, bt);
  if (temp < 0) return hipErrorInvalidValue;
  void* sort_tmp = w;
  w += align256(temp);
  if (pro) {
    p.dwq_part = reinterpret_cast<float*>(w);
    p.dwk_part = p.dwq_part + parts_q * p.D;
    *dwq_part = p.dwq_part;
    *dwk_part = p.dwk_part;
  }
  hipLaunchKernelGGL(path_keys, dim3((unsigned)((n + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, p,
                     keys_in, vals_in);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  size_t tb = (size_t)temp;
  e = rocprim::radix_sort_pairs(sort_tmp, tb, (const uint32_t*)keys_in, keys_out,
                                (const uint32_t*)vals_in, vals_out, (size_t)n, 0,
                                (unsigned)end_bit(bt), st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(path_starts, dim3((unsigned)((bt + 1 + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     st, keys_out, n, bt, starts);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  p.inv_start = starts;
  p.inv_entry = vals_out;
  switch (dtype) {
    case kBF16: return pro ? paths_backward_t<__bf16, true>(p, st) : paths_backward_t<__bf16, false>(p, st);
    case kFP16: return pro ? paths_backward_t<_Float16, true>(p, st) : paths_backward_t<_Float16, false>(p, st);
    case kFP32: return pro ? paths_backward_t<float, true>(p, st) : paths_backward_t<float, false>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sbda
