// Gate/up projection of the backbone's SwiGLU feed-forward with the
// activation in the GEMM epilogue (BiAttn/model.py:32-59, the
// `silu(gate(x)) * up(x)` of `SwiGLU.forward`):
//
//   g = x[m] . Wg[j] + bg[j],  u = x[m] . Wu[j] + bu[j],  h[m, j] = silu(g) * u
//
// with W = [Wg; Wu] one [2H, K] row-major weight (the two nn.Linear weights
// stacked) and the optional bias [2H] in fp32.  The eager sequence writes the
// [M, 2H] gate/up product and reads it back for the activation; here the
// product never leaves the registers: the HBM traffic is x, the weights and
// h (at T = 2^20, d = 512, H = 2048 in bf16: 1 + 8 + 4 GiB written and read
// back become 1 GiB read and 4 GiB written).
//
// Rounding follows the eager op sequence: g and u are rounded to the
// activation dtype (the GEMM's output), silu(g) is rounded (F.silu), and the
// product is rounded by the store.
//
// Tiling (gfx950, bf16/fp16 MFMA v_mfma_f32_32x32x16, fp32 accumulators):
//   * a workgroup (4 waves) owns 128 token rows x 128 hidden units, i.e. 128
//     rows of x against 256 weight rows (128 gate + the matching 128 up);
//   * K advances 32 at a time through two 24 KiB LDS stages; the global loads
//     of stage k + 2 are in flight (in one of two register sets) while stage
//     k feeds the MFMAs and stage k + 1 is written to LDS, and each stage's
//     fragments are all read before its first MFMA;
//   * 212 VGPRs and 48 KiB of LDS give two workgroups per CU (two waves per
//     SIMD), so one workgroup's epilogue and stage waits overlap the other's
//     MFMAs;
//   * a wave owns 64 tokens x 64 hidden units of both gate and up, so the
//     gate and up accumulators of one output sit in the same lane and the
//     epilogue is register-local.  The weight tile is the MFMA's A operand and
//     x its B operand, which puts 4 consecutive hidden units of one token in a
//     lane: each output store is 8 bytes;
//   * LDS holds the tiles in fragment order (slot()), so every fragment read
//     is one contiguous 1 KiB and neither reads nor staging writes conflict;
//   * XCD x (workgroup i runs on XCD i % 8) takes 1/8 of the hidden tiles of
//     every token tile, so its slice of the weights stays in its L2.

#include "sbda_device.h"
#include "sbda_params.h"

namespace sbda {
namespace {

constexpr int kFfnThreads = 256;
constexpr int kTokTile = 128;                      // token rows per workgroup
constexpr int kHidTile = 128;                      // hidden units per workgroup
constexpr int kBK = 32;                            // k per LDS stage
constexpr int kChunks = kBK * 2 / 16;              // 16-byte chunks per LDS row (4)
constexpr int kLdsRows = kTokTile + 2 * kHidTile;  // 384 rows of 64 bytes
constexpr int kLoadsPerThread = kLdsRows * kChunks / kFfnThreads;   // 6
constexpr int kRowsPerPass = kFfnThreads / kChunks;                 // 64
constexpr int kTokLoads = kTokTile / kRowsPerPass;                  // 2

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T> struct Mfma;
template <> struct Mfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x16 run(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline f32x16 run(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// LDS slot (16-byte units) of chunk c of row r, in fragment order: the 32
// rows of a 32-row block at one chunk are 512 contiguous bytes, chunks 2s and
// 2s + 1 side by side, so the fragment read of k sub-step s (lane l: row l %
// 32, chunk 2s + l / 32) is one contiguous 1 KiB, which the LDS serves
// without bank conflicts.  The row index is XORed with 0, 4, 10, 14 for
// chunks 0-3, which keeps the staging writes (4 lanes per row, chunks 0-3)
// conflict-free as well (measured: SQ_LDS_BANK_CONFLICT = 0 for both; rows
// at a 64-byte pitch instead put half the read cycles in conflicts).
__device__ inline int slot(int r, int c) {
  return ((r >> 5) * 2 + (c >> 1)) * 64 + (c & 1) * 32 + ((r & 31) ^ ((c & 1) * 4 + (c >> 1) * 10));
}

template <typename T>
__device__ inline void round_pair(float& a, float& b) {
  const uint32_t w = Elem<T>::pack(a, b);
  a = Elem<T>::lo(w);
  b = Elem<T>::hi(w);
}

// silu(g) = g / (1 + e^-g) with the hardware exp2 and reciprocal (the result
// is rounded to 16 bits right after).
__device__ inline float silu_fast(float g) {
  return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
}

// The MFMAs of one stage: every fragment of both 16-wide k sub-steps is read
// from LDS first, then the 16 MFMAs.
template <typename T>
__device__ __forceinline__ void stage_mma(const uint4* __restrict__ s, int wm, int wn, int l32,
                                          int khalf, f32x16 (&acc_g)[2][2],
                                          f32x16 (&acc_u)[2][2]) {
  typedef typename Mfma<T>::v8 v8;
  v8 fx[2][2], fg[2][2], fu[2][2];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int c = 2 * sub + khalf;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
      fx[sub][tb] = __builtin_bit_cast(v8, s[slot(wm * 64 + tb * 32 + l32, c)]);
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int rg = kTokTile + wn * 64 + hb * 32 + l32;
      fg[sub][hb] = __builtin_bit_cast(v8, s[slot(rg, c)]);
      fu[sub][hb] = __builtin_bit_cast(v8, s[slot(rg + kHidTile, c)]);
    }
  }
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        acc_g[tb][hb] = Mfma<T>::run(fg[sub][hb], fx[sub][tb], acc_g[tb][hb]);
        acc_u[tb][hb] = Mfma<T>::run(fu[sub][hb], fx[sub][tb], acc_u[tb][hb]);
      }
}

template <typename T>
__global__ __launch_bounds__(kFfnThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void ffn_gate_up_swiglu(const T* __restrict__ x, const T* __restrict__ w,
                        const float* __restrict__ bias, T* __restrict__ h, int64_t rows,
                        int dim, int hidden, int h_tiles) {
  __shared__ uint4 lds[2][kLdsRows * kChunks];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // Tile order: hardware places workgroup i on XCD i % 8.  With h_tiles a
  // multiple of 8, XCD x takes hidden tiles [x h_tiles / 8, (x + 1) h_tiles
  // / 8) of every token tile, so its slice of the weights stays in its L2.
  int mt, ht;
  if ((h_tiles & 7) == 0) {
    const int hx = h_tiles >> 3, s = blockIdx.x >> 3;
    mt = s / hx;
    ht = (blockIdx.x & 7) * hx + (s - mt * hx);
  } else {
    mt = blockIdx.x / h_tiles;
    ht = blockIdx.x - mt * h_tiles;
  }
  const int64_t m0 = (int64_t)mt * kTokTile;
  const int h0 = ht * kHidTile;

  // Staged chunk i of this thread: LDS row r = tid / 4 + 64 i, chunk tid % 4.
  // Rows [0, 128) are tokens (clamped to the last row), [128, 256) gate
  // weight rows, [256, 384) the matching up rows.  Element offsets fit 32
  // bits (the launcher checks rows * dim and 2 * hidden * dim).
  const int chunk = tid & (kChunks - 1);
  uint32_t src[kLoadsPerThread], dst[kLoadsPerThread];
#pragma unroll
  for (int i = 0; i < kLoadsPerThread; ++i) {
    const int r = tid / kChunks + kRowsPerPass * i;
    int64_t row;
    if (r < kTokTile) {
      row = m0 + r;
      if (row > rows - 1) row = rows - 1;
    } else if (r < kTokTile + kHidTile) {
      row = h0 + (r - kTokTile);
    } else {
      row = hidden + h0 + (r - kTokTile - kHidTile);
    }
    src[i] = (uint32_t)(row * dim + chunk * 8);
    dst[i] = (uint32_t)slot(r, chunk);
  }

  // Wave tile: tokens wm * 64 + [0, 64), hidden wn * 64 + [0, 64).
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int l32 = lane & 31;
  const int khalf = lane >> 5;
  f32x16 acc_g[2][2], acc_u[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc_g[a][b][e] = acc_u[a][b][e] = 0.f;

  // Two register sets (a0-a5, b0-b5; named registers, not arrays, so they
  // stay out of scratch): the loads of stage k + 2 are in flight while stage
  // k is computed and stage k + 1 (loaded one stage earlier) is stashed.  The
  // trip count is even (dim is a multiple of 64); loads past the last stage
  // re-read it (in bounds, never stashed into a stage that is computed).
  static_assert(kLoadsPerThread == 6 && kTokLoads == 2, "six chunks: 2 token, 4 weight");
  const int nk = dim / kBK;
  uint4 a0, a1, a2, a3, a4, a5, b0, b1, b2, b3, b4, b5;
#define FFN_LOAD(R, KT)                                                            \
  {                                                                                \
    const int k0_ = min((KT), nk - 1) * kBK;                                       \
    R##0 = *reinterpret_cast<const uint4*>(x + src[0] + k0_);                      \
    R##1 = *reinterpret_cast<const uint4*>(x + src[1] + k0_);                      \
    R##2 = *reinterpret_cast<const uint4*>(w + src[2] + k0_);                      \
    R##3 = *reinterpret_cast<const uint4*>(w + src[3] + k0_);                      \
    R##4 = *reinterpret_cast<const uint4*>(w + src[4] + k0_);                      \
    R##5 = *reinterpret_cast<const uint4*>(w + src[5] + k0_);                      \
  }
#define FFN_STASH(R, BUF)                                                          \
  {                                                                                \
    lds[BUF][dst[0]] = R##0;                                                       \
    lds[BUF][dst[1]] = R##1;                                                       \
    lds[BUF][dst[2]] = R##2;                                                       \
    lds[BUF][dst[3]] = R##3;                                                       \
    lds[BUF][dst[4]] = R##4;                                                       \
    lds[BUF][dst[5]] = R##5;                                                       \
  }
  FFN_LOAD(a, 0);
  FFN_STASH(a, 0);
  FFN_LOAD(b, 1);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    FFN_LOAD(a, kt + 2);
    stage_mma<T>(lds[0], wm, wn, l32, khalf, acc_g, acc_u);
    FFN_STASH(b, 1);
    __syncthreads();
    FFN_LOAD(b, kt + 3);
    stage_mma<T>(lds[1], wm, wn, l32, khalf, acc_g, acc_u);
    FFN_STASH(a, 0);
    __syncthreads();
  }
#undef FFN_LOAD
#undef FFN_STASH

  // Epilogue: acc[e] holds hidden 8 (e / 4) + 4 khalf + e % 4 of the 32-unit
  // block and token l32 of the 32-token block.
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int j0 = h0 + wn * 64 + hb * 32 + 8 * g4 + 4 * khalf;
      float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias != nullptr) {
        const float4 vg = *reinterpret_cast<const float4*>(bias + j0);
        const float4 vu = *reinterpret_cast<const float4*>(bias + hidden + j0);
        bg[0] = vg.x; bg[1] = vg.y; bg[2] = vg.z; bg[3] = vg.w;
        bu[0] = vu.x; bu[1] = vu.y; bu[2] = vu.z; bu[3] = vu.w;
      }
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const int64_t tok = m0 + wm * 64 + tb * 32 + l32;
        float a[4], u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] = acc_g[tb][hb][4 * g4 + e] + bg[e];
          u[e] = acc_u[tb][hb][4 * g4 + e] + bu[e];
          round_pair<T>(a[e], u[e]);         // the GEMM outputs in the dtype
          a[e] = silu_fast(a[e]);
        }
        round_pair<T>(a[0], a[1]);           // F.silu's output in the dtype
        round_pair<T>(a[2], a[3]);
        if (tok < rows) {
          uint2 pk;
          pk.x = Elem<T>::pack(a[0] * u[0], a[1] * u[1]);
          pk.y = Elem<T>::pack(a[2] * u[2], a[3] * u[3]);
          *reinterpret_cast<uint2*>(h + tok * hidden + j0) = pk;
        }
      }
    }
}

}  // namespace

// Shapes the fused kernel takes: bf16/fp16, K a multiple of 64 (the stage
// loop takes two 32-wide stages per trip), the hidden width a multiple of
// 128, 32-bit element offsets.
bool ffn_swiglu_supported(int64_t rows, int64_t dim, int64_t hidden, int dtype) {
  if (dtype != kBF16 && dtype != kFP16) return false;
  if (rows <= 0 || dim <= 0 || hidden <= 0) return false;
  if (dim % (2 * kBK) || hidden % kHidTile) return false;
  if (rows * dim >= (int64_t(1) << 31) || 2 * hidden * dim >= (int64_t(1) << 31)) return false;
  if (rows * hidden >= (int64_t(1) << 40)) return false;
  const int64_t tiles = ((rows + kTokTile - 1) / kTokTile) * (hidden / kHidTile);
  return tiles < (int64_t(1) << 31);
}

hipError_t ffn_swiglu_forward(const void* x, const void* w, const float* bias, void* h,
                              int64_t rows, int dim, int hidden, int dtype, hipStream_t st) {
  if (!ffn_swiglu_supported(rows, dim, hidden, dtype)) return hipErrorInvalidValue;
  const int h_tiles = hidden / kHidTile;
  const int64_t tiles = ((rows + kTokTile - 1) / kTokTile) * h_tiles;
  const dim3 grid((unsigned)tiles), block(kFfnThreads);
  if (dtype == kBF16) {
    hipLaunchKernelGGL(ffn_gate_up_swiglu<__bf16>, grid, block, 0, st,
                       static_cast<const __bf16*>(x), static_cast<const __bf16*>(w), bias,
                       static_cast<__bf16*>(h), rows, dim, hidden, h_tiles);
  } else {
    hipLaunchKernelGGL(ffn_gate_up_swiglu<_Float16>, grid, block, 0, st,
                       static_cast<const _Float16*>(x), static_cast<const _Float16*>(w), bias,
                       static_cast<_Float16*>(h), rows, dim, hidden, h_tiles);
  }
  return hipGetLastError();
}

}  // namespace sbda
