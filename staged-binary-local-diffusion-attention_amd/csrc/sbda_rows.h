// Row-parallel building blocks shared by the generic kernels
// (sbda_direct.hip) and the source-table kernels (sbda_paths.hip): one lane
// group of LPR lanes per row, blocks of kBlock threads.
#pragma once

#include <type_traits>

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {

constexpr int kBlock = 256;

template <typename T>
__device__ inline const T* row_ptr(const View& v, int b, int h, int64_t t) {
  return reinterpret_cast<const T*>(v.p) + (int64_t)b * v.sb + (int64_t)h * v.sh + t * v.st;
}
template <typename T>
__device__ inline T* row_ptr(const MutView& v, int b, int h, int64_t t) {
  return reinterpret_cast<T*>(v.p) + (int64_t)b * v.sb + (int64_t)h * v.sh + t * v.st;
}

// Loads k (through the prologue when fused) of source row `t` for kv head hk.
template <typename T, int LPR, bool PRO>
__device__ inline void load_key(const Params& p, int b, int hk, int64_t t, int li,
                                float (&k)[VecOf<T>::value]) {
  load_row<T, PRO>(row_ptr<T>(p.k, b, hk, t), li, p.D, k);
  if constexpr (PRO) {
    using PL = Prologue<T, LPR>;
    float c[PL::HV], s[PL::HV];
    PL::load_cs(p.rope_cos, p.rope_sin, t, li, p.D, c, s);
    PL::forward(k, p.wk, c, s, li, p.D, p.eps);
  }
}

// Segment-key check of source j for query i (true when no keys are given).
__device__ inline bool same_segment(const Params& p, int b, int i, int j) {
  if (p.seg == nullptr) return true;
  const int32_t* key = p.seg + (int64_t)b * p.T;
  const int32_t ki = key[i];
  return ki >= 0 && key[j] == ki;
}

// Decodes a global row id into (b, t, h) with heads fastest.
__device__ inline void decode_row(int64_t row, int heads, int T, int& b, int& t, int& h) {
  h = (int)(row % heads);
  const int64_t bt = row / heads;
  t = (int)(bt % T);
  b = (int)(bt / T);
}

// Deterministic block reduction of per-lane weight-gradient registers into
// out[d] (d < D): lane groups are summed in increasing order.
template <typename T, int LPR, bool SPLIT>
__device__ inline void block_reduce_dw(const float (&dw)[VecOf<T>::value], int D, float* out) {
  constexpr int VEC = VecOf<T>::value;
  constexpr int HV = VEC / 2;
  __shared__ float buf[kBlock * VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) buf[threadIdx.x * VEC + i] = dw[i];
  __syncthreads();
  const int groups = kBlock / LPR;
  for (int d = threadIdx.x; d < D; d += kBlock) {
    int li, slot;
    if constexpr (SPLIT) {
      const int half = D >> 1;
      const int dd = d < half ? d : d - half;
      li = dd / HV;
      slot = (dd % HV) + (d < half ? 0 : HV);
    } else {
      li = d / VEC;
      slot = d % VEC;
    }
    float acc = 0.f;
    for (int g = 0; g < groups; ++g) acc += buf[(g * LPR + li) * VEC + slot];
    out[d] = acc;
  }
}

// Calls f(std::integral_constant<int, LPR>) for the runtime lanes-per-row.
template <typename F>
inline hipError_t by_lpr(int lpr, F&& f) {
  switch (lpr) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sbda
