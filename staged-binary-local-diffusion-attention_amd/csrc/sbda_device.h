// Device-side building blocks shared by the SBDA attention kernels (gfx950).
//
// Row layout.  A "row" is one (batch, position, head) vector of D elements.
// LPR consecutive lanes of a 64-wide wavefront own one row; each lane holds
// VEC = 16 / sizeof(T) elements of it in fp32 registers:
//   * contiguous layout: lane li holds elements [li*VEC, li*VEC + VEC),
//     loaded with one 16-byte access;
//   * split layout (used when the RoPE prologue is fused): lane li holds
//     elements [li*HV, li*HV + HV) of the first half and the same range of
//     the second half (HV = VEC/2), loaded with two 8-byte accesses, so that
//     RoPE's (d, d + D/2) partners sit in the same lane.
// Lanes whose elements fall beyond D hold zeros and store nothing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbda {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// -------------------------------------------------------------- dtypes

template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  __device__ static inline uint32_t pack(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf2;
    bf2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <> struct Elem<_Float16> {
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ static inline uint32_t pack(float a, float b) {
    typedef __attribute__((ext_vector_type(2))) _Float16 h2;
    h2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

template <typename T> struct VecOf { static constexpr int value = 16 / (int)sizeof(T); };

// Unpack n 32-bit words holding 2n 16-bit values, or n fp32 values.
template <typename T, int NW>
__device__ inline void unpack_words(const uint32_t* w, float* x) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < NW; ++i) x[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      x[2 * i] = Elem<T>::lo(w[i]);
      x[2 * i + 1] = Elem<T>::hi(w[i]);
    }
  }
}

template <typename T, int NW>
__device__ inline void pack_words(const float* x, uint32_t* w) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = __float_as_uint(x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = Elem<T>::pack(x[2 * i], x[2 * i + 1]);
  }
}

// -------------------------------------------------------------- row I/O

// Load one row's share for lane li.  `row` points at element 0 of the row.
template <typename T, bool SPLIT>
__device__ inline void load_row(const T* __restrict__ row, int li, int D,
                                float (&x)[VecOf<T>::value]) {
  constexpr int VEC = VecOf<T>::value;
  if constexpr (!SPLIT) {
    if (li * VEC < D) {
      uint4 w = *reinterpret_cast<const uint4*>(row + li * VEC);
      uint32_t ws[4] = {w.x, w.y, w.z, w.w};
      unpack_words<T, 4>(ws, x);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[i] = 0.f;
    }
  } else {
    constexpr int HV = VEC / 2;
    const int half = D >> 1;
    if (li * HV < half) {
      uint2 a = *reinterpret_cast<const uint2*>(row + li * HV);
      uint2 b = *reinterpret_cast<const uint2*>(row + half + li * HV);
      uint32_t wa[2] = {a.x, a.y};
      uint32_t wb[2] = {b.x, b.y};
      unpack_words<T, 2>(wa, x);
      unpack_words<T, 2>(wb, x + HV);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) x[i] = 0.f;
    }
  }
}

template <typename T, bool SPLIT>
__device__ inline void store_row(T* __restrict__ row, int li, int D,
                                 const float (&x)[VecOf<T>::value]) {
  constexpr int VEC = VecOf<T>::value;
  if constexpr (!SPLIT) {
    if (li * VEC < D) {
      uint32_t ws[4];
      pack_words<T, 4>(x, ws);
      *reinterpret_cast<uint4*>(row + li * VEC) = make_uint4(ws[0], ws[1], ws[2], ws[3]);
    }
  } else {
    constexpr int HV = VEC / 2;
    const int half = D >> 1;
    if (li * HV < half) {
      uint32_t wa[2], wb[2];
      pack_words<T, 2>(x, wa);
      pack_words<T, 2>(x + HV, wb);
      *reinterpret_cast<uint2*>(row + li * HV) = make_uint2(wa[0], wa[1]);
      *reinterpret_cast<uint2*>(row + half + li * HV) = make_uint2(wb[0], wb[1]);
    }
  }
}

// Element index (within the row) of register slot i for lane li.
template <typename T, bool SPLIT>
__device__ inline int elem_index(int li, int i, int D) {
  constexpr int VEC = VecOf<T>::value;
  if constexpr (!SPLIT) {
    return li * VEC + i;
  } else {
    constexpr int HV = VEC / 2;
    return (i < HV) ? li * HV + i : (D >> 1) + li * HV + (i - HV);
  }
}

// Cross-lane move within a 16-lane DPP row (CTRL is the dpp_ctrl encoding).
template <int CTRL>
__device__ inline float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the LPR lanes of one row, every lane receiving the same bits.
// Steps: swap neighbours (quad_perm 1,0,3,2), swap pairs (quad_perm
// 2,3,0,1), mirror within 8 lanes, mirror within 16 lanes; each step adds
// two values that the partner lane adds in the other order, so all lanes
// agree exactly.  Groups wider than a DPP row finish with lane shuffles.
template <int LPR>
__device__ inline float row_sum(float x) {
  if constexpr (LPR >= 2) x += dpp<0xB1>(x);
  if constexpr (LPR >= 4) x += dpp<0x4E>(x);
  if constexpr (LPR >= 8) x += dpp<0x141>(x);
  if constexpr (LPR >= 16) x += dpp<0x140>(x);
#pragma unroll
  for (int m = 16; m < LPR; m <<= 1) x += __shfl_xor(x, m, 64);
  return x;
}

template <int VEC>
__device__ inline float dot_partial(const float (&a)[VEC], const float (&b)[VEC]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) s = __builtin_fmaf(a[i], b[i], s);
  return s;
}

// rsqrt(mean(x^2) + eps) of an RMS norm.  fp32 rows: 1 / sqrt(x) with both
// steps correctly rounded (what torch.rsqrt on fp32 CPU tensors gives to 1
// ulp), so the fp32 path meets a 1e-5 relative bar; 16-bit rows: the hardware
// approximation (~1 ulp, far below their own rounding).
template <typename T>
__device__ inline float norm_rsqrt(float x) {
  if constexpr (sizeof(T) == 4) return __fdiv_rn(1.f, __fsqrt_rn(x));
  else return __builtin_amdgcn_rsqf(x);
}

// exp(x) through the hardware exp2; exp(-inf) = 0.
__device__ inline float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ inline float fast_log(float x) { return __builtin_amdgcn_logf(x) * kLn2; }

// -------------------------------------------------------------- prologue
//
// Head-RMSNorm then half-split RoPE on a split-layout row (the reference's
// BiAttn/attention_common.py:25-50 and :64-76):
//   n = x * rsqrt(mean(x^2) + eps);  y = n * w;
//   z[d] = y[d] cos[d] - y[d + D/2] sin[d],  z[d + D/2] = y[d + D/2] cos[d] + y[d] sin[d]
// for d < D/2, with cos/sin read from fp32 [T, D/2] tables (the reference
// evaluates them in fp32; its bf16 runs then round them, which the fp32
// tables here do not).  Products are rounded one at a time (no
// contraction) to follow the reference's op order.
template <typename T, int LPR>
struct Prologue {
  static constexpr int VEC = VecOf<T>::value;
  static constexpr int HV = VEC / 2;

  // Loads this lane's HV cos and sin entries of position t from fp32 tables.
  __device__ static inline void load_cs(const float* __restrict__ cs_cos,
                                        const float* __restrict__ cs_sin, int64_t t, int li, int D,
                                        float (&c)[HV], float (&s)[HV]) {
    const int half = D >> 1;
    if (li * HV < half) {
      const float* pc = cs_cos + t * half + li * HV;
      const float* ps = cs_sin + t * half + li * HV;
      if constexpr (HV == 4) {
        const float4 a = *reinterpret_cast<const float4*>(pc);
        const float4 b = *reinterpret_cast<const float4*>(ps);
        c[0] = a.x; c[1] = a.y; c[2] = a.z; c[3] = a.w;
        s[0] = b.x; s[1] = b.y; s[2] = b.z; s[3] = b.w;
      } else {
        static_assert(HV == 2, "16-bit rows hold 4, fp32 rows 2 elements per half");
        const float2 a = *reinterpret_cast<const float2*>(pc);
        const float2 b = *reinterpret_cast<const float2*>(ps);
        c[0] = a.x; c[1] = a.y;
        s[0] = b.x; s[1] = b.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < HV; ++i) { c[i] = 1.f; s[i] = 0.f; }
    }
  }

  // In place: raw x -> roped z.  Returns the row's rsqrt factor r.
  __device__ static inline float forward(float (&x)[VEC], const float* __restrict__ w,
                                         const float (&c)[HV], const float (&s)[HV],
                                         int li, int D, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = row_sum<LPR>(ss);
    const float r = norm_rsqrt<T>(__fadd_rn(__fdiv_rn(ss, (float)D), eps));
    const int half = D >> 1;
    const bool on = li * HV < half;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int d = li * HV + i;
      const float w1 = on ? w[d] : 0.f;
      const float w2 = on ? w[half + d] : 0.f;
      const float y1 = __fmul_rn(__fmul_rn(x[i], r), w1);
      const float y2 = __fmul_rn(__fmul_rn(x[HV + i], r), w2);
      x[i] = __fadd_rn(__fmul_rn(y1, c[i]), -__fmul_rn(y2, s[i]));
      x[HV + i] = __fadd_rn(__fmul_rn(y2, c[i]), __fmul_rn(y1, s[i]));
    }
    return r;
  }

  // The lane's norm weights in register-slot order (split layout).
  __device__ static inline void load_w(const float* __restrict__ w, int li, int D,
                                       float (&wl)[VEC]) {
    const int half = D >> 1;
    const bool on = li * HV < half;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      wl[i] = on ? w[li * HV + i] : 0.f;
      wl[HV + i] = on ? w[half + li * HV + i] : 0.f;
    }
  }

  // rsqrt(mean(x^2) + eps) of a raw row.
  __device__ static inline float rms_factor(const float (&x)[VEC], int D, float eps) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VEC; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = row_sum<LPR>(ss);
    return norm_rsqrt<T>(__fadd_rn(__fdiv_rn(ss, (float)D), eps));
  }

  // forward() with the weights already in registers.
  __device__ static inline float forward_w(float (&x)[VEC], const float (&wl)[VEC],
                                           const float (&c)[HV], const float (&s)[HV], int D,
                                           float eps) {
    const float r = rms_factor(x, D, eps);
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const float y1 = __fmul_rn(__fmul_rn(x[i], r), wl[i]);
      const float y2 = __fmul_rn(__fmul_rn(x[HV + i], r), wl[HV + i]);
      x[i] = __fadd_rn(__fmul_rn(y1, c[i]), -__fmul_rn(y2, s[i]));
      x[HV + i] = __fadd_rn(__fmul_rn(y2, c[i]), __fmul_rn(y1, s[i]));
    }
    return r;
  }

  // backward() with the weights already in registers.
  __device__ static inline void backward_w(float (&g)[VEC], const float (&x)[VEC], float r,
                                           const float (&wl)[VEC], const float (&c)[HV],
                                           const float (&s)[HV], int D, float (&dw)[VEC]) {
    float dn[VEC], n[VEC];
    float nd = 0.f;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const float dy1 = g[i] * c[i] + g[HV + i] * s[i];
      const float dy2 = g[HV + i] * c[i] - g[i] * s[i];
      n[i] = x[i] * r;
      n[HV + i] = x[HV + i] * r;
      dw[i] += dy1 * n[i];
      dw[HV + i] += dy2 * n[HV + i];
      dn[i] = dy1 * wl[i];
      dn[HV + i] = dy2 * wl[HV + i];
      nd += n[i] * dn[i] + n[HV + i] * dn[HV + i];
    }
    nd = row_sum<LPR>(nd) / (float)D;
#pragma unroll
    for (int i = 0; i < VEC; ++i) g[i] = r * (dn[i] - n[i] * nd);
  }

  // g: gradient w.r.t. the roped row (fp32), x: raw row, r: rsqrt factor.
  // Writes the gradient w.r.t. the raw row into g and adds this row's
  // contribution to the weight gradient into dw (same register slots).
  __device__ static inline void backward(float (&g)[VEC], const float (&x)[VEC], float r,
                                         const float* __restrict__ w,
                                         const float (&c)[HV], const float (&s)[HV],
                                         int li, int D, float (&dw)[VEC]) {
    const int half = D >> 1;
    const bool on = li * HV < half;
    float dn[VEC], n[VEC];
    float nd = 0.f;
#pragma unroll
    for (int i = 0; i < HV; ++i) {
      const int d = li * HV + i;
      const float w1 = on ? w[d] : 0.f;
      const float w2 = on ? w[half + d] : 0.f;
      const float dy1 = g[i] * c[i] + g[HV + i] * s[i];
      const float dy2 = g[HV + i] * c[i] - g[i] * s[i];
      n[i] = x[i] * r;
      n[HV + i] = x[HV + i] * r;
      dw[i] += dy1 * n[i];
      dw[HV + i] += dy2 * n[HV + i];
      dn[i] = dy1 * w1;
      dn[HV + i] = dy2 * w2;
      nd += n[i] * dn[i] + n[HV + i] * dn[HV + i];
    }
    nd = row_sum<LPR>(nd) / (float)D;
#pragma unroll
    for (int i = 0; i < VEC; ++i) g[i] = r * (dn[i] - n[i] * nd);
  }
};

}  // namespace sbda
