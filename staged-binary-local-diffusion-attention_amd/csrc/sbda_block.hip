// Fused kernels for the steps next to the attention op in the SBDA backbone
// block (BiAttn/model.py:18-59 RMSNorm and SwiGLU, :321-335 the residual
// block): residual add + RMSNorm, and the SwiGLU activation silu(gate) * up.
//
// All four kernels are HBM-bound streams over row-major [rows, width]
// buffers.  Rounding follows the eager op sequence they replace: the
// residual sum is rounded to the activation dtype before it is normalised,
// RMSNorm computes in fp32 and rounds once, silu(gate) is rounded before the
// product with up (PyTorch's F.silu then `*`), and the backward rounds its
// intermediate gradients where the eager autograd graph does.
//
// RMSNorm (one 64-lane wave per row; lane l holds the 16-byte chunks
// l, l + 64, ... of the row):
//   s = x (+ r),  rstd = rsqrt(mean(s^2) + eps),  y = (s * rstd) * w
//   backward: xhat = s * rstd, g = dy * w,
//             ds = rstd * (g - xhat * mean(g * xhat)) (+ upstream ds),
//             dw = sum over rows of dy * xhat (per-wave partials, reduced in
//             a fixed order).
// SwiGLU on gate_up = [gate | up] (the two projections computed as one
// GEMM, gate in columns [0, H), up in [H, 2H)):
//   h = silu(gate) * up
//   backward: da = dh * up, dup = dh * silu(gate),
//             dgate = da * sig * (1 + gate * (1 - sig)),  sig = sigmoid(gate).

#include <type_traits>

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {
namespace {

constexpr int kNormWaves = 4;          // rows in flight per block (one per wave)
constexpr int kNormBlock = kNormWaves * 64;
constexpr int kActBlock = 256;

template <typename T>
__device__ inline float round_to(float x) {
  if constexpr (sizeof(T) == 4) {
    return x;
  } else {
    uint32_t w = Elem<T>::pack(x, 0.f);
    return Elem<T>::lo(w);
  }
}

// Loads chunk c (16 bytes) of a row for this lane, zeros beyond `width`.
template <typename T>
__device__ inline void load_chunk(const T* __restrict__ row, int idx, int width,
                                  float (&x)[VecOf<T>::value]) {
  constexpr int VEC = VecOf<T>::value;
  if (idx < width) {
    uint4 w = *reinterpret_cast<const uint4*>(row + idx);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    unpack_words<T, 4>(ws, x);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) x[i] = 0.f;
  }
}

template <typename T>
__device__ inline void store_chunk(T* __restrict__ row, int idx, int width,
                                   const float (&x)[VecOf<T>::value]) {
  if (idx < width) {
    uint32_t ws[4];
    pack_words<T, 4>(x, ws);
    *reinterpret_cast<uint4*>(row + idx) = make_uint4(ws[0], ws[1], ws[2], ws[3]);
  }
}

__device__ inline void load_w(const float* __restrict__ w, int idx, int width, float* out, int n) {
  for (int i = 0; i < n; ++i) out[i] = idx + i < width ? w[idx + i] : 0.f;
}

// ------------------------------------------------------------ RMSNorm fwd
//
// Each wave strides over rows U at a time and issues all loads of its U rows
// before reducing any, so every wave keeps U * C 16-byte loads per input in
// flight (short-lived one-row waves left the kernel latency-bound).

template <typename T, int C, int U, bool RES>
__global__ __launch_bounds__(kNormBlock) void rmsnorm_fwd(const T* __restrict__ x,
                                                          const T* __restrict__ r,
                                                          T* __restrict__ s_out,
                                                          T* __restrict__ y,
                                                          const float* __restrict__ w,
                                                          float* __restrict__ rstd, int64_t rows,
                                                          int dim, float eps) {
  constexpr int VEC = VecOf<T>::value;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * kNormWaves;
  float wv[C][VEC];
#pragma unroll
  for (int c = 0; c < C; ++c) load_w(w, (c * 64 + lane) * VEC, dim, wv[c], VEC);
  for (int64_t first = wave; first < rows; first += waves * U) {
    float v[U][C][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = first + u * waves;
      const int64_t rr = row < rows ? row : first;  // rows past the end reload `first`
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int idx = (c * 64 + lane) * VEC;
        load_chunk<T>(x + rr * dim, idx, dim, v[u][c]);
        if constexpr (RES) {
          float ad[VEC];
          load_chunk<T>(r + rr * dim, idx, dim, ad);
#pragma unroll
          for (int i = 0; i < VEC; ++i) v[u][c][i] = round_to<T>(v[u][c][i] + ad[i]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = first + u * waves;
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < VEC; ++i) ss = __builtin_fmaf(v[u][c][i], v[u][c][i], ss);
      ss = row_sum<64>(ss);
      const float rs = norm_rsqrt<T>(__fadd_rn(__fdiv_rn(ss, (float)dim), eps));
      if (row < rows) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int idx = (c * 64 + lane) * VEC;
          if constexpr (RES) store_chunk<T>(s_out + row * dim, idx, dim, v[u][c]);
          float o[VEC];
#pragma unroll
          for (int i = 0; i < VEC; ++i) o[i] = __fmul_rn(__fmul_rn(v[u][c][i], rs), wv[c][i]);
          store_chunk<T>(y + row * dim, idx, dim, o);
        }
        if (rstd != nullptr && lane == 0) rstd[row] = rs;
      }
    }
  }
}

// ------------------------------------------------------------ RMSNorm bwd

template <typename T, int C, int U, bool ADD>
__global__ __launch_bounds__(kNormBlock) void rmsnorm_bwd(const T* __restrict__ dy,
                                                          const T* __restrict__ s,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ rstd,
                                                          const T* __restrict__ ds_in,
                                                          T* __restrict__ dx,
                                                          float* __restrict__ dw_part,
                                                          int64_t rows, int dim) {
  constexpr int VEC = VecOf<T>::value;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * kNormWaves;
  float wv[C][VEC], dw[C][VEC];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    load_w(w, (c * 64 + lane) * VEC, dim, wv[c], VEC);
#pragma unroll
    for (int i = 0; i < VEC; ++i) dw[c][i] = 0.f;
  }
  for (int64_t first = wave; first < rows; first += waves * U) {
    float xh[U][C][VEC], d[U][C][VEC];
    float rs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = first + u * waves;
      const int64_t rr = row < rows ? row : first;
      rs[u] = rstd[rr];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const int idx = (c * 64 + lane) * VEC;
        load_chunk<T>(s + rr * dim, idx, dim, xh[u][c]);
        load_chunk<T>(dy + rr * dim, idx, dim, d[u][c]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t row = first + u * waves;
      const bool live = row < rows;
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < C; ++c)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          xh[u][c][i] *= rs[u];
          d[u][c][i] = live ? d[u][c][i] : 0.f;
          const float g = d[u][c][i] * wv[c][i];
          dot = __builtin_fmaf(g, xh[u][c][i], dot);
          dw[c][i] = __builtin_fmaf(d[u][c][i], xh[u][c][i], dw[c][i]);
        }
      const float mean = row_sum<64>(dot) / (float)dim;
      if (live) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int idx = (c * 64 + lane) * VEC;
          float o[VEC];
#pragma unroll
          for (int i = 0; i < VEC; ++i)
            o[i] = rs[u] * (d[u][c][i] * wv[c][i] - xh[u][c][i] * mean);
          if constexpr (ADD) {
            float up[VEC];
            load_chunk<T>(ds_in + row * dim, idx, dim, up);
#pragma unroll
            for (int i = 0; i < VEC; ++i) o[i] = round_to<T>(o[i]) + up[i];
          }
          store_chunk<T>(dx + row * dim, idx, dim, o);
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int idx = (c * 64 + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      if (idx + i < dim) dw_part[wave * dim + idx + i] = dw[c][i];
  }
}

// ------------------------------------------------------------- SwiGLU

__device__ inline float sigmoid(float g) { return 1.f / (1.f + expf(-g)); }

template <typename T>
__global__ __launch_bounds__(kActBlock) void swiglu_fwd(const T* __restrict__ gu,
                                                        T* __restrict__ h, int64_t rows,
                                                        int hidden) {
  constexpr int VEC = VecOf<T>::value;
  const int per_row = hidden / VEC;
  const int64_t n = rows * per_row;
  for (int64_t k = (int64_t)blockIdx.x * kActBlock + threadIdx.x; k < n;
       k += (int64_t)gridDim.x * kActBlock) {
    const int64_t row = k / per_row;
    const int col = (int)(k % per_row) * VEC;
    const T* src = gu + row * 2 * hidden;
    float g[VEC], u[VEC], o[VEC];
    load_chunk<T>(src, col, hidden, g);
    load_chunk<T>(src + hidden, col, hidden, u);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float a = round_to<T>(g[i] / (1.f + expf(-g[i])));
      o[i] = a * u[i];
    }
    store_chunk<T>(h + row * hidden, col, hidden, o);
  }
}

template <typename T>
__global__ __launch_bounds__(kActBlock) void swiglu_bwd(const T* __restrict__ dh,
                                                        const T* __restrict__ gu,
                                                        T* __restrict__ dgu, int64_t rows,
                                                        int hidden) {
  constexpr int VEC = VecOf<T>::value;
  const int per_row = hidden / VEC;
  const int64_t n = rows * per_row;
  for (int64_t k = (int64_t)blockIdx.x * kActBlock + threadIdx.x; k < n;
       k += (int64_t)gridDim.x * kActBlock) {
    const int64_t row = k / per_row;
    const int col = (int)(k % per_row) * VEC;
    const T* src = gu + row * 2 * hidden;
    float g[VEC], u[VEC], d[VEC], dg[VEC], du[VEC];
    load_chunk<T>(src, col, hidden, g);
    load_chunk<T>(src + hidden, col, hidden, u);
    load_chunk<T>(dh + row * hidden, col, hidden, d);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float sig = sigmoid(g[i]);
      const float a = round_to<T>(g[i] / (1.f + expf(-g[i])));
      const float da = round_to<T>(d[i] * u[i]);
      du[i] = d[i] * a;
      dg[i] = da * sig * (1.f + g[i] * (1.f - sig));
    }
    store_chunk<T>(dgu + row * 2 * hidden, col, hidden, dg);
    store_chunk<T>(dgu + row * 2 * hidden + hidden, col, hidden, du);
  }
}

// ----------------------------------------------------------- launchers

template <typename F>
hipError_t by_chunks(int chunks_per_lane, F&& f) {
  switch (chunks_per_lane) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return hipErrorInvalidValue;
  }
}

int chunks_per_lane(int64_t dim, int esz) {
  const int64_t chunks = (dim * esz + 15) / 16;
  int c = 1;
  while (c * 64 < chunks) c <<= 1;
  return c;
}

// Waves for the streaming row kernels: enough to fill every CU several times.
int64_t stream_blocks(int64_t rows, int per_wave) {
  const int64_t want = (rows + (int64_t)kNormWaves * per_wave - 1) / ((int64_t)kNormWaves * per_wave);
  return want < 2048 ? want : 2048;
}

template <typename T>
hipError_t norm_fwd_t(const void* x, const void* r, void* s_out, void* y, const float* w,
                      float* rstd, int64_t rows, int dim, float eps, hipStream_t st) {
  return by_chunks(chunks_per_lane(dim, sizeof(T)), [&](auto c) {
    constexpr int C = decltype(c)::value;
    constexpr int U = C == 1 ? 4 : (C == 2 ? 2 : 1);
    const unsigned blocks = (unsigned)stream_blocks(rows, U);
    if (r != nullptr)
      hipLaunchKernelGGL((rmsnorm_fwd<T, C, U, true>), dim3(blocks), dim3(kNormBlock), 0, st,
                         (const T*)x, (const T*)r, (T*)s_out, (T*)y, w, rstd, rows, dim, eps);
    else
      hipLaunchKernelGGL((rmsnorm_fwd<T, C, U, false>), dim3(blocks), dim3(kNormBlock), 0, st,
                         (const T*)x, (const T*)nullptr, (T*)nullptr, (T*)y, w, rstd, rows, dim,
                         eps);
    return hipGetLastError();
  });
}

template <typename T>
hipError_t norm_bwd_t(const void* dy, const void* s, const float* w, const float* rstd,
                      const void* ds_in, void* dx, float* part, int64_t blocks, int64_t rows,
                      int dim, hipStream_t st) {
  return by_chunks(chunks_per_lane(dim, sizeof(T)), [&](auto c) {
    constexpr int C = decltype(c)::value;
    constexpr int U = C == 1 ? 4 : (C == 2 ? 2 : 1);
    if (ds_in != nullptr)
      hipLaunchKernelGGL((rmsnorm_bwd<T, C, U, true>), dim3((unsigned)blocks), dim3(kNormBlock), 0,
                         st, (const T*)dy, (const T*)s, w, rstd, (const T*)ds_in, (T*)dx, part,
                         rows, dim);
    else
      hipLaunchKernelGGL((rmsnorm_bwd<T, C, U, false>), dim3((unsigned)blocks), dim3(kNormBlock),
                         0, st, (const T*)dy, (const T*)s, w, rstd, (const T*)nullptr, (T*)dx,
                         part, rows, dim);
    return hipGetLastError();
  });
}

unsigned act_blocks(int64_t n) {
  const int64_t want = (n + kActBlock - 1) / kActBlock;
  return (unsigned)(want < 65536 ? want : 65536);
}

}  // namespace

// Blocks of the RMSNorm backward (each wave strides over rows and keeps one
// weight-gradient partial row).
int64_t rmsnorm_bwd_blocks(int64_t rows) {
  const int64_t want = (rows + kNormWaves - 1) / kNormWaves;
  return want < 2048 ? want : 2048;
}

int rmsnorm_max_dim(int esz) { return 8 * 64 * 16 / esz; }

hipError_t rmsnorm_forward(const void* x, const void* r, void* s_out, void* y, const float* w,
                           float* rstd, int64_t rows, int dim, int dtype, float eps,
                           hipStream_t st) {
  switch (dtype) {
    case kBF16: return norm_fwd_t<__bf16>(x, r, s_out, y, w, rstd, rows, dim, eps, st);
    case kFP16: return norm_fwd_t<_Float16>(x, r, s_out, y, w, rstd, rows, dim, eps, st);
    case kFP32: return norm_fwd_t<float>(x, r, s_out, y, w, rstd, rows, dim, eps, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t rmsnorm_backward(const void* dy, const void* s, const float* w, const float* rstd,
                            const void* ds_in, void* dx, float* part, int64_t rows, int dim,
                            int dtype, hipStream_t st) {
  const int64_t blocks = rmsnorm_bwd_blocks(rows);
  switch (dtype) {
    case kBF16: return norm_bwd_t<__bf16>(dy, s, w, rstd, ds_in, dx, part, blocks, rows, dim, st);
    case kFP16: return norm_bwd_t<_Float16>(dy, s, w, rstd, ds_in, dx, part, blocks, rows, dim, st);
    case kFP32: return norm_bwd_t<float>(dy, s, w, rstd, ds_in, dx, part, blocks, rows, dim, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t swiglu_forward(const void* gu, void* h, int64_t rows, int hidden, int dtype,
                          hipStream_t st) {
  const int esz = dtype == kFP32 ? 4 : 2;
  const unsigned blocks = act_blocks(rows * hidden * esz / 16);
  switch (dtype) {
    case kBF16:
      hipLaunchKernelGGL(swiglu_fwd<__bf16>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const __bf16*)gu, (__bf16*)h, rows, hidden);
      break;
    case kFP16:
      hipLaunchKernelGGL(swiglu_fwd<_Float16>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const _Float16*)gu, (_Float16*)h, rows, hidden);
      break;
    case kFP32:
      hipLaunchKernelGGL(swiglu_fwd<float>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const float*)gu, (float*)h, rows, hidden);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t swiglu_backward(const void* dh, const void* gu, void* dgu, int64_t rows, int hidden,
                           int dtype, hipStream_t st) {
  const int esz = dtype == kFP32 ? 4 : 2;
  const unsigned blocks = act_blocks(rows * hidden * esz / 16);
  switch (dtype) {
    case kBF16:
      hipLaunchKernelGGL(swiglu_bwd<__bf16>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const __bf16*)dh, (const __bf16*)gu, (__bf16*)dgu, rows, hidden);
      break;
    case kFP16:
      hipLaunchKernelGGL(swiglu_bwd<_Float16>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const _Float16*)dh, (const _Float16*)gu, (_Float16*)dgu, rows, hidden);
      break;
    case kFP32:
      hipLaunchKernelGGL(swiglu_bwd<float>, dim3(blocks), dim3(kActBlock), 0, st,
                         (const float*)dh, (const float*)gu, (float*)dgu, rows, hidden);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sbda
