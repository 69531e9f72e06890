/*
 * C ABI of the MI355X SBDA attention library (libsbda_amd.so, gfx950).
 *
 * Plain pointers and sizes only.  Every tensor is a [B, heads, T, D] view
 * given by a device pointer and four element strides {b, h, t, d}; the d
 * stride must be 1, the pointer 16-byte aligned and the b/h/t strides
 * multiples of 16 bytes.  Offsets are host int32 arrays (S in 1..4, each
 * >= 0).  `stream` is a hipStream_t (NULL = default stream).  Kernels are
 * enqueued asynchronously on `stream`; nothing allocates device memory.
 *
 * Reference interfaces replaced (paths relative to the reference checkout,
 * HaoyangMaLabs/Staged-Binary-Local-Diffusion-Attention v0.1.3):
 *   sbda_forward            -> BiAttn/sbda_triton.py:1294-1327, the forward of
 *                              _FusedSBDAKeyBackward (its two Triton launches
 *                              _sbda_block_forward_kernel + _sbda_weights_kernel
 *                              at :1312-1325).  Saves one fp32 log-normaliser
 *                              per row instead of the [B,H,T,S] weight table.
 *   sbda_backward           -> BiAttn/sbda_triton.py:1329-1360, the backward
 *                              (launches _sbda_dq_from_weights_kernel and
 *                              _sbda_dkv_key_kernel at :1342-1359); also the
 *                              GQA pair at :1363-1434 when kv_heads < heads.
 *   sbda_forward_prologue   -> BiAttn/left_v2.py:237-239 (q_norm, k_norm,
 *                              _apply_rope from BiAttn/attention_common.py:
 *                              25-50,64-76) fused into sbda_forward.
 *   sbda_backward_prologue  -> the autograd backward of the same three ops
 *                              fused into sbda_backward, plus the norm-weight
 *                              gradients.
 *   sbda_rope_table         -> BiAttn/attention_common.py:13-22
 *                              (_rope_cos_sin), as a [T, D/2] device table.
 *
 * Masks (seg_key): every entry point that runs attention takes an optional
 * device int32 array seg_key[B, T] (contiguous).  NULL = no mask.  Otherwise
 * a source j of query i counts only if seg_key[b,i] >= 0 and
 * seg_key[b,j] == seg_key[b,i]: -1 marks a padded position (valid_mask
 * false) and a new value starts a segment (seam_reset), the key being
 * valid ? cumsum(seam_reset) : -1 (BiAttn/left_v2.py:329-405, the source
 * masking of the eager route).  A row with no counted source writes zeros and
 * lse = +inf.  Masked calls run the generic kernels.
 *
 * Source tables (sbda_forward_paths / sbda_backward_paths): instead of the
 * layer's offsets, query i of batch b reads the sources path_indices[b,i,s]
 * (device int64 [B, T, S], contiguous, any S >= 1); source s counts when
 * path_valid[b,i,s] != 0 (device bytes, e.g. a torch.bool tensor; NULL = all),
 * 0 <= j <= i, and the segment keys agree.  This is the eager route of
 * BiAttn/left_v2.py:212-231,313-378 (tables produced for the greedy H4 schedule,
 * BinaryDiffusionAttention/run_mini_experiment.py:117-133).  The fused norm +
 * RoPE prologue is on when q_weight/k_weight/rope_cos/rope_sin are given (all
 * four) and off when all four are NULL.
 *
 * Return codes: SBDA_OK, or an error whose text sbda_last_error() returns
 * (thread-local).  SBDA_ERR_VALUE maps to Python ValueError, SBDA_ERR_DTYPE to
 * TypeError, SBDA_ERR_RUNTIME (a HIP error) to RuntimeError -- the error
 * classes the reference's fused path raises (sbda_triton.py:1295-1302).
 */
#ifndef SBDA_AMD_H
#define SBDA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SBDA_OK 0
#define SBDA_ERR_VALUE 1
#define SBDA_ERR_DTYPE 2
#define SBDA_ERR_RUNTIME 3

#define SBDA_DTYPE_BF16 0
#define SBDA_DTYPE_FP16 1
#define SBDA_DTYPE_FP32 2

/* ABI version of this header (bumped on any signature change). */
int sbda_abi_version(void);

/* Text of the last error on the calling thread ("" if none). */
const char* sbda_last_error(void);

/*
 * Forward.  q: [B,H,T,D]; k, v: [B,Hkv,T,D] (H % Hkv == 0, query head h reads
 * kv head h / (H/Hkv)).  Writes out ([B,H,T,D], any strides as above) and
 * lse: one fp32 log-normaliser per row, stored [B,T,H] contiguous (position
 * major, like q/k/v memory); +inf marks a row with no valid source.
 * Scale is head_dim**-0.5 in fp32.
 */
int sbda_forward(const void* q, const int64_t* q_strides,
                 const void* k, const int64_t* k_strides,
                 const void* v, const int64_t* v_strides,
                 void* out, const int64_t* out_strides,
                 float* lse,
                 int64_t batch, int64_t heads, int64_t kv_heads,
                 int64_t length, int64_t head_dim, int32_t dtype,
                 const int32_t* offsets, int32_t num_offsets,
                 const int32_t* seg_key, void* stream);

/* Workspace bytes sbda_backward needs for these shapes and masks (< 0:
 * error), enough for any strides: when the strides could send the call to the
 * generic kernels (row spans past 4 GiB) it is their weight table, although
 * the wavefront-walk kernels need none.  sbda_backward_workspace_for gives the
 * exact figure for given strides (0 on the walk path). */
int64_t sbda_backward_workspace(int64_t batch, int64_t heads, int64_t kv_heads,
                                int64_t length, int64_t head_dim, int32_t dtype,
                                const int32_t* offsets, int32_t num_offsets,
                                const int32_t* seg_key);

/*
 * Backward from the forward's saved q, k, v and lse.  Writes dq, dk, dv (each
 * row exactly once: deterministic, no atomics).  `workspace` (16-byte
 * aligned, sbda_backward_workspace bytes; may be NULL when that is 0) holds
 * the per-(row, slot) weights that the generic kernels pass from their query
 * pass to their key pass.
 */
int sbda_backward(const void* q, const int64_t* q_strides,
                  const void* k, const int64_t* k_strides,
                  const void* v, const int64_t* v_strides,
                  const void* dout, const int64_t* dout_strides,
                  const float* lse,
                  void* dq, const int64_t* dq_strides,
                  void* dk, const int64_t* dk_strides,
                  void* dv, const int64_t* dv_strides,
                  void* workspace, int64_t workspace_bytes,
                  int64_t batch, int64_t heads, int64_t kv_heads,
                  int64_t length, int64_t head_dim, int32_t dtype,
                  const int32_t* offsets, int32_t num_offsets,
                  const int32_t* seg_key, void* stream);

/*
 * Forward with the head-RMSNorm + RoPE prologue fused: q_raw and k_raw are
 * the projections before normalisation; q_weight/k_weight are fp32 [D]
 * norm weights; rope_cos/rope_sin are fp32 [T, D/2] tables
 * (sbda_rope_table).  eps is the norm epsilon (reference: 1e-6).
 */
int sbda_forward_prologue(const void* q_raw, const int64_t* q_strides,
                          const void* k_raw, const int64_t* k_strides,
                          const void* v, const int64_t* v_strides,
                          void* out, const int64_t* out_strides,
                          float* lse,
                          const float* q_weight, const float* k_weight,
                          const float* rope_cos, const float* rope_sin, float eps,
                          int64_t batch, int64_t heads, int64_t kv_heads,
                          int64_t length, int64_t head_dim, int32_t dtype,
                          const int32_t* offsets, int32_t num_offsets,
                          const int32_t* seg_key, void* stream);

/* Workspace bytes sbda_backward_prologue needs for these shapes (< 0: error);
 * enough for any strides of the tensors (sbda_backward_workspace_for: the
 * exact figure for given strides). */
int64_t sbda_backward_prologue_workspace(int64_t batch, int64_t heads, int64_t kv_heads,
                                         int64_t length, int64_t head_dim, int32_t dtype,
                                         const int32_t* offsets, int32_t num_offsets,
                                         const int32_t* seg_key);

/*
 * Workspace bytes sbda_backward (prologue = 0) or sbda_backward_prologue
 * (prologue != 0) needs for these shapes and these strides of q, k, v,
 * grad_out, dq, dk, dv (< 0: error).  Exact: the strides decide between the
 * kernel families (row spans past 4 GiB go to the generic kernels), which the
 * stride-less queries above can only bound.  No counterpart in the reference
 * (its Triton launches allocate their own tables).
 */
int64_t sbda_backward_workspace_for(int32_t prologue, const int64_t* q_strides,
                                    const int64_t* k_strides, const int64_t* v_strides,
                                    const int64_t* dout_strides, const int64_t* dq_strides,
                                    const int64_t* dk_strides, const int64_t* dv_strides,
                                    int64_t batch, int64_t heads, int64_t kv_heads,
                                    int64_t length, int64_t head_dim, int32_t dtype,
                                    const int32_t* offsets, int32_t num_offsets,
                                    const int32_t* seg_key);

/*
 * Backward of sbda_forward_prologue: gradients of the raw q/k, of v and of
 * the two norm weights (dq_weight, dk_weight: fp32 [D], overwritten; summed
 * over all rows in a fixed order through `workspace`).
 */
int sbda_backward_prologue(const void* q_raw, const int64_t* q_strides,
                           const void* k_raw, const int64_t* k_strides,
                           const void* v, const int64_t* v_strides,
                           const void* dout, const int64_t* dout_strides,
                           const float* lse,
                           const float* q_weight, const float* k_weight,
                           const float* rope_cos, const float* rope_sin, float eps,
                           void* dq_raw, const int64_t* dq_strides,
                           void* dk_raw, const int64_t* dk_strides,
                           void* dv, const int64_t* dv_strides,
                           float* dq_weight, float* dk_weight,
                           void* workspace, int64_t workspace_bytes,
                           int64_t batch, int64_t heads, int64_t kv_heads,
                           int64_t length, int64_t head_dim, int32_t dtype,
                           const int32_t* offsets, int32_t num_offsets,
                           const int32_t* seg_key, void* stream);

/*
 * sbda_backward_prologue without a workspace argument: for callers that
 * cannot allocate device memory (code under HIP-graph capture, tight serving
 * or training loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The workspace comes from a static device array of the library
 * (sbda_noalloc_scratch_bytes() = 128 MiB, one copy per GPU, held until the
 * process ends); calls needing more (sbda_backward_workspace_for) fail with
 * SBDA_ERR_VALUE before launching anything.  Nothing is allocated.  Call it
 * with the tensors' device current.  Calls that overlap on one GPU share the
 * scratch and race; the scratch keeps the last call's contents.
 */
int64_t sbda_noalloc_scratch_bytes(void);
int sbda_backward_prologue_noalloc(const void* q_raw, const int64_t* q_strides,
                                   const void* k_raw, const int64_t* k_strides,
                                   const void* v, const int64_t* v_strides,
                                   const void* dout, const int64_t* dout_strides,
                                   const float* lse,
                                   const float* q_weight, const float* k_weight,
                                   const float* rope_cos, const float* rope_sin, float eps,
                                   void* dq_raw, const int64_t* dq_strides,
                                   void* dk_raw, const int64_t* dk_strides,
                                   void* dv, const int64_t* dv_strides,
                                   float* dq_weight, float* dk_weight,
                                   int64_t batch, int64_t heads, int64_t kv_heads,
                                   int64_t length, int64_t head_dim, int32_t dtype,
                                   const int32_t* offsets, int32_t num_offsets,
                                   const int32_t* seg_key, void* stream);

/*
 * Forward over source tables (see "Source tables" above).  Writes out and
 * lse like sbda_forward / sbda_forward_prologue.
 */
int sbda_forward_paths(const void* q, const int64_t* q_strides,
                       const void* k, const int64_t* k_strides,
                       const void* v, const int64_t* v_strides,
                       void* out, const int64_t* out_strides,
                       float* lse,
                       const float* q_weight, const float* k_weight,
                       const float* rope_cos, const float* rope_sin, float eps,
                       int64_t batch, int64_t heads, int64_t kv_heads,
                       int64_t length, int64_t head_dim, int32_t dtype,
                       const int64_t* path_indices, const uint8_t* path_valid,
                       int32_t num_sources, const int32_t* seg_key, void* stream);

/* Workspace bytes sbda_backward_paths needs (prologue: 1 if the prologue
 * pointers will be given, else 0; < 0: error). */
int64_t sbda_backward_paths_workspace(int64_t batch, int64_t heads, int64_t kv_heads,
                                      int64_t length, int64_t head_dim, int32_t dtype,
                                      int32_t num_sources, int32_t prologue);

/*
 * Backward of sbda_forward_paths: gradients of q, k, v (raw q/k with the
 * prologue) and, with the prologue, of the two norm weights.  The workspace
 * (256-byte aligned) holds a per-(row, slot) weight table and an inverse
 * index built by a stable sort, so every gradient row is written once, in a
 * fixed order: deterministic, no atomics.  dq_weight/dk_weight may be NULL
 * without the prologue.
 */
int sbda_backward_paths(const void* q, const int64_t* q_strides,
                        const void* k, const int64_t* k_strides,
                        const void* v, const int64_t* v_strides,
                        const void* dout, const int64_t* dout_strides,
                        const float* lse,
                        const float* q_weight, const float* k_weight,
                        const float* rope_cos, const float* rope_sin, float eps,
                        void* dq, const int64_t* dq_strides,
                        void* dk, const int64_t* dk_strides,
                        void* dv, const int64_t* dv_strides,
                        float* dq_weight, float* dk_weight,
                        void* workspace, int64_t workspace_bytes,
                        int64_t batch, int64_t heads, int64_t kv_heads,
                        int64_t length, int64_t head_dim, int32_t dtype,
                        const int64_t* path_indices, const uint8_t* path_valid,
                        int32_t num_sources, const int32_t* seg_key, void* stream);

/*
 * Block kernels next to the attention op (BiAttn/model.py:18-59,321-335).
 * They have no C counterpart in the reference (there they are eager PyTorch
 * ops: F.rms_norm, the residual `x + ...`, F.silu(gate(x)) * up(x)); they
 * fuse those ops so each activation crosses HBM once.  Buffers are
 * contiguous row-major [rows, width], 16-byte aligned, width * element size a
 * multiple of 16 bytes.
 *
 * sbda_rmsnorm_forward: y = (s * rsqrt(mean(s^2) + eps)) * weight with
 * s = x, or s = x + residual (rounded to dtype, written to sum_out) when
 * residual is given.  weight is fp32 [dim]; rstd (optional, fp32 [rows])
 * receives the per-row rsqrt for the backward.  dim * element size <= 8 KiB.
 */
int sbda_rmsnorm_forward(const void* x, const void* residual, void* sum_out, void* y,
                         const float* weight, float* rstd, int64_t rows, int64_t dim,
                         int32_t dtype, float eps, void* stream);

/* Workspace bytes of sbda_rmsnorm_backward (< 0: error). */
int64_t sbda_rmsnorm_backward_workspace(int64_t rows, int64_t dim, int32_t dtype);

/*
 * Backward of sbda_rmsnorm_forward: dx = d(y)/d(s) applied to dy, plus dsum
 * (the gradient reaching s from its other uses, optional); dx is then the
 * gradient of x and of residual.  dweight (fp32 [dim]) is overwritten with
 * the weight gradient, summed in a fixed order through `workspace`.
 */
int sbda_rmsnorm_backward(const void* dy, const void* x, const float* weight, const float* rstd,
                          const void* dsum, void* dx, float* dweight, void* workspace,
                          int64_t workspace_bytes, int64_t rows, int64_t dim, int32_t dtype,
                          void* stream);

/* SwiGLU activation: out[r, c] = silu(gate_up[r, c]) * gate_up[r, hidden + c]. */
int sbda_swiglu_forward(const void* gate_up, void* out, int64_t rows, int64_t hidden,
                        int32_t dtype, void* stream);

/* Backward of sbda_swiglu_forward into dgate_up ([rows, 2 * hidden]). */
int sbda_swiglu_backward(const void* dout, const void* gate_up, void* dgate_up, int64_t rows,
                         int64_t hidden, int32_t dtype, void* stream);

/*
 * Gate/up projection with the SwiGLU activation in its epilogue (replaces
 * `F.silu(self.gate(x)) * self.up(x)`, BiAttn/model.py:32-59, as one MFMA
 * GEMM kernel; no autograd state is kept):
 *   out[r, j] = silu(g) * u,  g = x[r] . weight[j] + bias[j],
 *                             u = x[r] . weight[hidden + j] + bias[hidden + j]
 * x [rows, dim], weight [2 * hidden, dim] (gate rows, then up rows), out
 * [rows, hidden], all row-major in `dtype` (bf16 or fp16 only); bias is fp32
 * [2 * hidden] or NULL.  g and u are rounded to the dtype before the
 * activation, silu(g) after it.  Shapes: dim a multiple of 64, hidden a
 * multiple of 128, rows * dim and 2 * hidden * dim below 2^31
 * (sbda_swiglu_gemm_supported).  Buffers 16-byte aligned.
 */
int sbda_swiglu_gemm_supported(int64_t rows, int64_t dim, int64_t hidden, int32_t dtype);
int sbda_swiglu_gemm_forward(const void* x, const void* weight, const float* bias, void* out,
                             int64_t rows, int64_t dim, int64_t hidden, int32_t dtype,
                             void* stream);

/*
 * RoPE tables: cos/sin[t, i] = cos/sin(fl32(t * inv_freq[i])) for t < length,
 * i < head_dim/2, as fp32 [length, head_dim/2].  inv_freq is a host fp32
 * array of head_dim/2 values (head_dim <= 512).
 */
int sbda_rope_table(float* rope_cos, float* rope_sin, const float* inv_freq,
                    int64_t length, int64_t head_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SBDA_AMD_H */
