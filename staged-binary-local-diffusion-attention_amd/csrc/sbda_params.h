// Kernel parameter block and host-side launcher declarations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sbda {

// A [B, heads, T, D] view with element strides; the D stride is 1.
struct View {
  const void* p;
  int64_t sb, sh, st;
};

struct MutView {
  void* p;
  int64_t sb, sh, st;
};

constexpr int kMaxSlots = 4;

struct Params {
  View q, k, v, dout;          // q and k are the raw (pre-prologue) rows when the prologue is fused
  MutView o, dq, dk, dv;
  float* lse;                  // [B, T, H] fp32, contiguous
  int B, H, Hkv, group, T, D, S;
  int off[kMaxSlots];
  float scale;
  // Fused prologue (head-RMSNorm + RoPE); unused otherwise.
  const float* wq;             // [D] fp32
  const float* wk;             // [D] fp32
  const float* rope_cos;       // [T, D/2] fp32
  const float* rope_sin;
  float eps;
  float* dwq_part;             // [parts, D] fp32 per-block partial sums
  float* dwk_part;
  float* tab;                  // prologue backward: per (row, slot) (p, scale * dS), fp32
  // Optional segment keys [B, T] (row stride T): a source j of query i counts
  // only if key[i] >= 0 and key[j] == key[i].  nullptr = no masking.
  const int32_t* seg;
  // Source-table mode (sbda_paths.hip): PS sources per query read from
  // pidx [B, T, PS] int64 (contiguous), gated by pvalid [B, T, PS] bytes
  // (nullptr = all set).  inv_start [B*T + 1] / inv_entry (i * PS + s, sorted)
  // list, per key position b*T + j, the (query, slot) pairs that read it.
  const int64_t* pidx;
  const uint8_t* pvalid;
  int PS;
  const uint32_t* inv_start;
  const uint32_t* inv_entry;
};

enum DType : int { kBF16 = 0, kFP16 = 1, kFP32 = 2 };

// Launchers return hipSuccess or the launch error.  `parts_*` report how
// many per-block weight-gradient partial rows the backward writes.
hipError_t launch_forward(const Params& p, int dtype, bool prologue, hipStream_t st);
hipError_t launch_backward(const Params& p, int dtype, bool prologue, hipStream_t st);
int64_t backward_partials(const Params& p, int dtype, bool prologue, int64_t* parts_q, int64_t* parts_k);
hipError_t launch_reduce_partials(const float* part, int64_t parts, int D, float* out, hipStream_t st);
hipError_t launch_reduce_partials2(const float* part_a, int64_t parts_a, float* out_a,
                                   const float* part_b, int64_t parts_b, float* out_b, int D,
                                   hipStream_t st);
hipError_t launch_rope_table(float* cos_out, float* sin_out, const float* inv_freq_host,
                             int64_t length, int half, hipStream_t st);

// Lanes per row for head_dim D of element size esz (16 bytes per lane).
inline int lanes_per_row(int D, int esz) {
  int chunks = (D * esz + 15) / 16;
  int l = 1;
  while (l < chunks) l <<= 1;
  return l;
}

}  // namespace sbda
