// C ABI (include/sbda_amd.h): argument validation, parameter packing and
// dispatch to the kernels.  No device allocation happens here.

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "sbda_amd.h"
#include "sbda_params.h"

namespace sbda {

hipError_t direct_forward(const Params& p, int dtype, bool pro, hipStream_t st);
hipError_t direct_backward(const Params& p, int dtype, bool pro, hipStream_t st);
void direct_partials(const Params& p, int esz, int64_t* parts_q, int64_t* parts_k,
                     int64_t* tab_floats);
bool walk_applies(const Params& p, int dtype);
hipError_t walk_forward(const Params& p, int dtype, bool pro, hipStream_t st);
hipError_t walk_backward(const Params& p, int dtype, bool pro, hipStream_t st);
void walk_partials(const Params& p, int dtype, int64_t* parts_q, int64_t* parts_k,
                   int64_t* tab_floats);
int64_t paths_workspace(const Params& p, int esz, bool pro, int64_t* parts_q, int64_t* parts_k);
hipError_t paths_forward(const Params& p, int dtype, bool pro, hipStream_t st);
hipError_t paths_backward(Params p, int dtype, bool pro, void* ws, int64_t parts_q, hipStream_t st,
                          float** dwq_part, float** dwk_part);
int64_t rmsnorm_bwd_blocks(int64_t rows);
int rmsnorm_max_dim(int esz);
hipError_t rmsnorm_forward(const void* x, const void* r, void* s_out, void* y, const float* w,
                           float* rstd, int64_t rows, int dim, int dtype, float eps,
                           hipStream_t st);
hipError_t rmsnorm_backward(const void* dy, const void* s, const float* w, const float* rstd,
                            const void* ds_in, void* dx, float* part, int64_t rows, int dim,
                            int dtype, hipStream_t st);
hipError_t swiglu_forward(const void* gu, void* h, int64_t rows, int hidden, int dtype,
                          hipStream_t st);
hipError_t swiglu_backward(const void* dh, const void* gu, void* dgu, int64_t rows, int hidden,
                           int dtype, hipStream_t st);
bool ffn_swiglu_supported(int64_t rows, int64_t dim, int64_t hidden, int dtype);
hipError_t ffn_swiglu_forward(const void* x, const void* w, const float* bias, void* h,
                              int64_t rows, int dim, int hidden, int dtype, hipStream_t st);

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int esize(int dtype) { return dtype == kFP32 ? 4 : 2; }

// Shapes and dtype shared by every entry point.
int check_shape(int64_t batch, int64_t heads, int64_t kv_heads, int64_t length, int64_t head_dim,
                int32_t dtype, Params& p) {
  if (dtype != kBF16 && dtype != kFP16 && dtype != kFP32)
    return fail(SBDA_ERR_DTYPE, "unsupported SBDA dtype code %d (bf16, fp16 or fp32)", (int)dtype);
  if (batch <= 0 || heads <= 0 || kv_heads <= 0 || length <= 0 || head_dim <= 0)
    return fail(SBDA_ERR_VALUE, "SBDA sizes must be positive (B=%lld H=%lld Hkv=%lld T=%lld D=%lld)",
                (long long)batch, (long long)heads, (long long)kv_heads, (long long)length,
                (long long)head_dim);
  if (heads % kv_heads)
    return fail(SBDA_ERR_VALUE, "query heads (%lld) must be divisible by kv heads (%lld)",
                (long long)heads, (long long)kv_heads);
  if (length >= (int64_t(1) << 31) - 1 || batch >= (int64_t(1) << 31) || heads >= (1 << 20))
    return fail(SBDA_ERR_VALUE, "SBDA sizes exceed the supported range");
  const int esz = esize(dtype);
  if ((head_dim * esz) % 16 != 0 || head_dim * esz > 512)
    return fail(SBDA_ERR_VALUE,
                "head_dim %lld unsupported: head_dim * element size must be a multiple of 16 bytes "
                "and at most 512 bytes",
                (long long)head_dim);
  std::memset(&p, 0, sizeof(p));
  p.B = (int)batch;
  p.H = (int)heads;
  p.Hkv = (int)kv_heads;
  p.group = (int)(heads / kv_heads);
  p.T = (int)length;
  p.D = (int)head_dim;
  p.scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  return SBDA_OK;
}

// Shapes, dtype and offsets of the offset-mode entry points.
int check_problem(int64_t batch, int64_t heads, int64_t kv_heads, int64_t length,
                  int64_t head_dim, int32_t dtype, const int32_t* offsets,
                  int32_t num_offsets, Params& p) {
  int rc = check_shape(batch, heads, kv_heads, length, head_dim, dtype, p);
  if (rc) return rc;
  if (offsets == nullptr || num_offsets < 1 || num_offsets > kMaxSlots)
    return fail(SBDA_ERR_VALUE, "SBDA supports 1 to %d sources, got %d", kMaxSlots, (int)num_offsets);
  for (int s = 0; s < num_offsets; ++s) {
    if (offsets[s] < 0) return fail(SBDA_ERR_VALUE, "SBDA offsets must be >= 0 (slot %d is %d)", s, offsets[s]);
    p.off[s] = offsets[s];
  }
  p.S = num_offsets;
  return SBDA_OK;
}

// Shapes, dtype and source tables of the table-mode entry points.
int check_paths(int64_t batch, int64_t heads, int64_t kv_heads, int64_t length, int64_t head_dim,
                int32_t dtype, const int64_t* pidx, const uint8_t* pvalid, int32_t num_sources,
                const int32_t* seg, Params& p) {
  int rc = check_shape(batch, heads, kv_heads, length, head_dim, dtype, p);
  if (rc) return rc;
  if (num_sources < 1) return fail(SBDA_ERR_VALUE, "source tables need at least one source");
  if (batch * length * num_sources >= (int64_t(1) << 31) - 1)
    return fail(SBDA_ERR_VALUE, "source tables exceed 2^31 entries");
  if (pidx == nullptr) return fail(SBDA_ERR_VALUE, "path_indices: null pointer");
  if (reinterpret_cast<uintptr_t>(pidx) % 8)
    return fail(SBDA_ERR_VALUE, "path_indices must be 8-byte aligned");
  p.pidx = pidx;
  p.pvalid = pvalid;
  p.PS = num_sources;
  p.seg = seg;
  return SBDA_OK;
}

int check_view(const char* name, const void* ptr, const int64_t* strides, int esz, bool writable,
               View* out) {
  if (ptr == nullptr || strides == nullptr) return fail(SBDA_ERR_VALUE, "%s: null pointer", name);
  if (reinterpret_cast<uintptr_t>(ptr) % 16)
    return fail(SBDA_ERR_VALUE, "%s: data pointer must be 16-byte aligned", name);
  if (strides[3] != 1) return fail(SBDA_ERR_VALUE, "%s: head_dim stride must be 1", name);
  for (int i = 0; i < 3; ++i)
    if ((strides[i] * esz) % 16)
      return fail(SBDA_ERR_VALUE, "%s: stride %d must be a multiple of 16 bytes", name, i);
  (void)writable;
  out->p = ptr;
  out->sb = strides[0];
  out->sh = strides[1];
  out->st = strides[2];
  return SBDA_OK;
}

int check_mut(const char* name, void* ptr, const int64_t* strides, int esz, MutView* out) {
  View v;
  int rc = check_view(name, ptr, strides, esz, true, &v);
  if (rc) return rc;
  out->p = ptr;
  out->sb = v.sb;
  out->sh = v.sh;
  out->st = v.st;
  return SBDA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return SBDA_OK;
  return fail(SBDA_ERR_RUNTIME, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

int forward_impl(bool pro, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                 const void* v, const int64_t* vs, void* out, const int64_t* os, float* lse,
                 const float* wq, const float* wk, const float* rc, const float* rs, float eps,
                 int64_t batch, int64_t heads, int64_t kv_heads, int64_t length, int64_t head_dim,
                 int32_t dtype, const int32_t* offsets, int32_t n, const int32_t* seg,
                 void* stream) {
  g_error.clear();
  Params p;
  int rc_ = check_problem(batch, heads, kv_heads, length, head_dim, dtype, offsets, n, p);
  if (rc_) return rc_;
  p.seg = seg;
  const int esz = esize(dtype);
  if ((rc_ = check_view("q", q, qs, esz, false, &p.q))) return rc_;
  if ((rc_ = check_view("k", k, ks, esz, false, &p.k))) return rc_;
  if ((rc_ = check_view("v", v, vs, esz, false, &p.v))) return rc_;
  if ((rc_ = check_mut("out", out, os, esz, &p.o))) return rc_;
  if (lse == nullptr) return fail(SBDA_ERR_VALUE, "lse: null pointer");
  p.lse = lse;
  if (pro) {
    if (!wq || !wk || !rc || !rs) return fail(SBDA_ERR_VALUE, "prologue: null weight or RoPE table");
    p.wq = wq;
    p.wk = wk;
    p.rope_cos = rc;
    p.rope_sin = rs;
    p.eps = eps;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = walk_applies(p, dtype) ? walk_forward(p, dtype, pro, st)
                                        : direct_forward(p, dtype, pro, st);
  return hip_status(e, "sbda forward launch");
}

// Workspace of the backward, in floats: weight-gradient partial rows for the
// query and key sides (prologue only), then the per-(row, slot) weight table
// (generic kernels, and the walk kernels' two-pass prologue backward).
int64_t workspace_floats(const Params& p, int dtype, bool pro, int64_t* pq, int64_t* pk) {
  int64_t tab = 0;
  *pq = *pk = 0;
  const bool walk = walk_applies(p, dtype);
  if (walk) {
    if (pro) walk_partials(p, dtype, pq, pk, &tab);
  } else {
    direct_partials(p, esize(dtype), pq, pk, &tab);
    if (!pro) *pq = *pk = 0;
  }
  const int64_t need = (*pq + *pk) * p.D + tab;
  if (walk && p.q.p == nullptr) {
    // A size query (no tensors, so no strides): strides can still send the
    // launch to the generic kernels (a row span past 4 GiB), so report the
    // larger of the two needs.  A launch lays out exactly its own need.
    int64_t dq = 0, dk = 0, dtab = 0;
    direct_partials(p, esize(dtype), &dq, &dk, &dtab);
    if (!pro) dq = dk = 0;
    return std::max(need, (dq + dk) * p.D + dtab);
  }
  return need;
}

int backward_impl(bool pro, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                  const void* v, const int64_t* vs, const void* dout, const int64_t* dos,
                  const float* lse, const float* wq, const float* wk, const float* rc,
                  const float* rs, float eps, void* dq, const int64_t* dqs, void* dk,
                  const int64_t* dks, void* dv, const int64_t* dvs, float* dwq, float* dwk,
                  void* ws, int64_t ws_bytes, int64_t batch, int64_t heads, int64_t kv_heads,
                  int64_t length, int64_t head_dim, int32_t dtype, const int32_t* offsets,
                  int32_t n, const int32_t* seg, void* stream) {
  g_error.clear();
  Params p;
  int rc_ = check_problem(batch, heads, kv_heads, length, head_dim, dtype, offsets, n, p);
  if (rc_) return rc_;
  p.seg = seg;
  const int esz = esize(dtype);
  if ((rc_ = check_view("q", q, qs, esz, false, &p.q))) return rc_;
  if ((rc_ = check_view("k", k, ks, esz, false, &p.k))) return rc_;
  if ((rc_ = check_view("v", v, vs, esz, false, &p.v))) return rc_;
  if ((rc_ = check_view("grad_out", dout, dos, esz, false, &p.dout))) return rc_;
  if ((rc_ = check_mut("dq", dq, dqs, esz, &p.dq))) return rc_;
  if ((rc_ = check_mut("dk", dk, dks, esz, &p.dk))) return rc_;
  if ((rc_ = check_mut("dv", dv, dvs, esz, &p.dv))) return rc_;
  if (lse == nullptr) return fail(SBDA_ERR_VALUE, "lse: null pointer");
  p.lse = const_cast<float*>(lse);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int64_t pq = 0, pk = 0;
  if (pro && (!wq || !wk || !rc || !rs || !dwq || !dwk))
    return fail(SBDA_ERR_VALUE, "prologue: null weight, weight-gradient or RoPE table");
  const int64_t need = workspace_floats(p, dtype, pro, &pq, &pk) * (int64_t)sizeof(float);
  if (need > 0) {
    if (ws == nullptr || ws_bytes < need)
      return fail(SBDA_ERR_VALUE, "backward: workspace of %lld bytes needed, %lld given",
                  (long long)need, (long long)ws_bytes);
    if (reinterpret_cast<uintptr_t>(ws) % 16)
      return fail(SBDA_ERR_VALUE, "workspace must be 16-byte aligned");
    p.dwq_part = reinterpret_cast<float*>(ws);
    p.dwk_part = p.dwq_part + pq * p.D;
    p.tab = p.dwk_part + pk * p.D;
  }
  if (pro) {
    p.wq = wq;
    p.wk = wk;
    p.rope_cos = rc;
    p.rope_sin = rs;
    p.eps = eps;
  }
  hipError_t e = walk_applies(p, dtype) ? walk_backward(p, dtype, pro, st)
                                        : direct_backward(p, dtype, pro, st);
  if (e == hipSuccess && pro) {
    e = launch_reduce_partials2(p.dwq_part, pq, dwq, p.dwk_part, pk, dwk, p.D, st);
  }
  return hip_status(e, "sbda backward launch");
}

int set_prologue(Params& p, const float* wq, const float* wk, const float* rc, const float* rs,
                 float eps, bool* pro) {
  *pro = wq != nullptr || wk != nullptr || rc != nullptr || rs != nullptr;
  if (!*pro) return SBDA_OK;
  if (!wq || !wk || !rc || !rs)
    return fail(SBDA_ERR_VALUE, "prologue: give all of q_weight, k_weight, rope_cos, rope_sin or none");
  p.wq = wq;
  p.wk = wk;
  p.rope_cos = rc;
  p.rope_sin = rs;
  p.eps = eps;
  return SBDA_OK;
}

int paths_forward_impl(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                       const void* v, const int64_t* vs, void* out, const int64_t* os, float* lse,
                       const float* wq, const float* wk, const float* rc, const float* rs, float eps,
                       int64_t batch, int64_t heads, int64_t kv_heads, int64_t length,
                       int64_t head_dim, int32_t dtype, const int64_t* pidx, const uint8_t* pvalid,
                       int32_t ns, const int32_t* seg, void* stream) {
  g_error.clear();
  Params p;
  int rc_ = check_paths(batch, heads, kv_heads, length, head_dim, dtype, pidx, pvalid, ns, seg, p);
  if (rc_) return rc_;
  const int esz = esize(dtype);
  if ((rc_ = check_view("q", q, qs, esz, false, &p.q))) return rc_;
  if ((rc_ = check_view("k", k, ks, esz, false, &p.k))) return rc_;
  if ((rc_ = check_view("v", v, vs, esz, false, &p.v))) return rc_;
  if ((rc_ = check_mut("out", out, os, esz, &p.o))) return rc_;
  if (lse == nullptr) return fail(SBDA_ERR_VALUE, "lse: null pointer");
  p.lse = lse;
  bool pro = false;
  if ((rc_ = set_prologue(p, wq, wk, rc, rs, eps, &pro))) return rc_;
  return hip_status(paths_forward(p, dtype, pro, reinterpret_cast<hipStream_t>(stream)),
                    "sbda table-mode forward launch");
}

int paths_backward_impl(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                        const void* v, const int64_t* vs, const void* dout, const int64_t* dos,
                        const float* lse, const float* wq, const float* wk, const float* rc,
                        const float* rs, float eps, void* dq, const int64_t* dqs, void* dk,
                        const int64_t* dks, void* dv, const int64_t* dvs, float* dwq, float* dwk,
                        void* ws, int64_t ws_bytes, int64_t batch, int64_t heads, int64_t kv_heads,
                        int64_t length, int64_t head_dim, int32_t dtype, const int64_t* pidx,
                        const uint8_t* pvalid, int32_t ns, const int32_t* seg, void* stream) {
  g_error.clear();
  Params p;
  int rc_ = check_paths(batch, heads, kv_heads, length, head_dim, dtype, pidx, pvalid, ns, seg, p);
  if (rc_) return rc_;
  const int esz = esize(dtype);
  if ((rc_ = check_view("q", q, qs, esz, false, &p.q))) return rc_;
  if ((rc_ = check_view("k", k, ks, esz, false, &p.k))) return rc_;
  if ((rc_ = check_view("v", v, vs, esz, false, &p.v))) return rc_;
  if ((rc_ = check_view("grad_out", dout, dos, esz, false, &p.dout))) return rc_;
  if ((rc_ = check_mut("dq", dq, dqs, esz, &p.dq))) return rc_;
  if ((rc_ = check_mut("dk", dk, dks, esz, &p.dk))) return rc_;
  if ((rc_ = check_mut("dv", dv, dvs, esz, &p.dv))) return rc_;
  if (lse == nullptr) return fail(SBDA_ERR_VALUE, "lse: null pointer");
  p.lse = const_cast<float*>(lse);
  bool pro = false;
  if ((rc_ = set_prologue(p, wq, wk, rc, rs, eps, &pro))) return rc_;
  if (pro && (!dwq || !dwk)) return fail(SBDA_ERR_VALUE, "prologue: null weight-gradient output");
  int64_t pq = 0, pk = 0;
  const int64_t need = paths_workspace(p, esz, pro, &pq, &pk);
  if (need < 0) return fail(SBDA_ERR_RUNTIME, "table-mode backward: cannot size the sort storage");
  if (ws == nullptr || ws_bytes < need)
    return fail(SBDA_ERR_VALUE, "table-mode backward: workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)ws_bytes);
  if (reinterpret_cast<uintptr_t>(ws) % 256)
    return fail(SBDA_ERR_VALUE, "workspace must be 256-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* dwq_part = nullptr;
  float* dwk_part = nullptr;
  hipError_t e = paths_backward(p, dtype, pro, ws, pq, st, &dwq_part, &dwk_part);
  if (e == hipSuccess && pro) {
    e = launch_reduce_partials2(dwq_part, pq, dwq, dwk_part, pk, dwk, p.D, st);
  }
  return hip_status(e, "sbda table-mode backward launch");
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Rows x width problems of the block kernels: contiguous rows, 16-byte
// aligned buffers, width a whole number of 16-byte chunks.
int check_rows(int64_t rows, int64_t width, int32_t dtype, int64_t max_width) {
  if (dtype != kBF16 && dtype != kFP16 && dtype != kFP32)
    return fail(SBDA_ERR_DTYPE, "unsupported dtype code %d (bf16, fp16 or fp32)", (int)dtype);
  if (rows <= 0 || width <= 0) return fail(SBDA_ERR_VALUE, "rows and width must be positive");
  if ((width * esize(dtype)) % 16)
    return fail(SBDA_ERR_VALUE, "width %lld: rows must be a multiple of 16 bytes", (long long)width);
  if (width > max_width)
    return fail(SBDA_ERR_VALUE, "width %lld exceeds the supported %lld", (long long)width,
                (long long)max_width);
  if (rows >= (int64_t(1) << 40)) return fail(SBDA_ERR_VALUE, "too many rows");
  return SBDA_OK;
}

// ------------------------------------------------ allocation-free backward
//
// sbda_backward_prologue_noalloc takes its workspace (norm-weight partial
// rows, deferred chain slots, weight tables) from `scratch`, a fixed device
// array of the library, instead of a caller allocation.  Every GPU the
// library runs on holds its own copy until the process ends.  The host never
// uses the array's name as an address: each device's address comes from
// hipGetSymbolAddress, once per device, on the first call there.  No part of
// the scratch has to start at zero: every partial row, slot and table entry
// the kernels read is written earlier in the same call.  Calls that overlap
// on one GPU (two streams, two threads) share the array and race.
constexpr int64_t kScratchBytes = int64_t(128) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch` (the caller's current device).
int device_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SBDA_ERR_RUNTIME, "device ordinal %d outside the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(SBDA_ERR_RUNTIME, "scratch has no address on device %d", dev);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SBDA_OK;
}

}  // namespace
}  // namespace sbda

using namespace sbda;

extern "C" {

int sbda_abi_version(void) { return 10; }

const char* sbda_last_error(void) { return g_error.c_str(); }

int sbda_forward(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                 const int64_t* vs, void* out, const int64_t* os, float* lse, int64_t batch,
                 int64_t heads, int64_t kv_heads, int64_t length, int64_t head_dim, int32_t dtype,
                 const int32_t* offsets, int32_t n, const int32_t* seg_key, void* stream) {
  return forward_impl(false, q, qs, k, ks, v, vs, out, os, lse, nullptr, nullptr, nullptr, nullptr,
                      0.f, batch, heads, kv_heads, length, head_dim, dtype, offsets, n, seg_key,
                      stream);
}

int64_t sbda_backward_workspace(int64_t batch, int64_t heads, int64_t kv_heads, int64_t length,
                                int64_t head_dim, int32_t dtype, const int32_t* offsets,
                                int32_t n, const int32_t* seg_key) {
  g_error.clear();
  Params p;
  int rc = check_problem(batch, heads, kv_heads, length, head_dim, dtype, offsets, n, p);
  if (rc) return -rc;
  p.seg = seg_key;
  int64_t pq = 0, pk = 0;
  return workspace_floats(p, dtype, false, &pq, &pk) * (int64_t)sizeof(float);
}

int64_t sbda_backward_workspace_for(int32_t prologue, const int64_t* q_strides,
                                    const int64_t* k_strides, const int64_t* v_strides,
                                    const int64_t* dout_strides, const int64_t* dq_strides,
                                    const int64_t* dk_strides, const int64_t* dv_strides,
                                    int64_t batch, int64_t heads, int64_t kv_heads,
                                    int64_t length, int64_t head_dim, int32_t dtype,
                                    const int32_t* offsets, int32_t n, const int32_t* seg_key) {
  g_error.clear();
  Params p;
  int rc = check_problem(batch, heads, kv_heads, length, head_dim, dtype, offsets, n, p);
  if (rc) return -rc;
  p.seg = seg_key;
  // The strides decide between the kernel families; the tensors themselves
  // are not needed (a 16-byte-aligned stand-in address passes the checks and
  // is never dereferenced).
  const void* stand_in = reinterpret_cast<const void*>(uintptr_t(16));
  const int esz = esize(dtype);
  if ((rc = check_view("q", stand_in, q_strides, esz, false, &p.q))) return -rc;
  if ((rc = check_view("k", stand_in, k_strides, esz, false, &p.k))) return -rc;
  if ((rc = check_view("v", stand_in, v_strides, esz, false, &p.v))) return -rc;
  if ((rc = check_view("grad_out", stand_in, dout_strides, esz, false, &p.dout))) return -rc;
  if ((rc = check_mut("dq", const_cast<void*>(stand_in), dq_strides, esz, &p.dq))) return -rc;
  if ((rc = check_mut("dk", const_cast<void*>(stand_in), dk_strides, esz, &p.dk))) return -rc;
  if ((rc = check_mut("dv", const_cast<void*>(stand_in), dv_strides, esz, &p.dv))) return -rc;
  int64_t pq = 0, pk = 0;
  return workspace_floats(p, dtype, prologue != 0, &pq, &pk) * (int64_t)sizeof(float);
}

int sbda_backward(const void* q, const int64_t* qs, const void* k, const int64_t* ks, const void* v,
                  const int64_t* vs, const void* dout, const int64_t* dos, const float* lse, void* dq,
                  const int64_t* dqs, void* dk, const int64_t* dks, void* dv, const int64_t* dvs,
                  void* workspace, int64_t workspace_bytes, int64_t batch, int64_t heads,
                  int64_t kv_heads, int64_t length, int64_t head_dim, int32_t dtype,
                  const int32_t* offsets, int32_t n, const int32_t* seg_key, void* stream) {
  return backward_impl(false, q, qs, k, ks, v, vs, dout, dos, lse, nullptr, nullptr, nullptr, nullptr,
                       0.f, dq, dqs, dk, dks, dv, dvs, nullptr, nullptr, workspace,
                       workspace_bytes, batch, heads, kv_heads, length, head_dim, dtype, offsets, n,
                       seg_key, stream);
}

int sbda_forward_prologue(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                          const void* v, const int64_t* vs, void* out, const int64_t* os,
                          float* lse, const float* wq, const float* wk, const float* rc,
                          const float* rs, float eps, int64_t batch, int64_t heads,
                          int64_t kv_heads, int64_t length, int64_t head_dim, int32_t dtype,
                          const int32_t* offsets, int32_t n, const int32_t* seg_key,
                          void* stream) {
  return forward_impl(true, q, qs, k, ks, v, vs, out, os, lse, wq, wk, rc, rs, eps, batch, heads,
                      kv_heads, length, head_dim, dtype, offsets, n, seg_key, stream);
}

int64_t sbda_backward_prologue_workspace(int64_t batch, int64_t heads, int64_t kv_heads,
                                         int64_t length, int64_t head_dim, int32_t dtype,
                                         const int32_t* offsets, int32_t n,
                                         const int32_t* seg_key) {
  g_error.clear();
  Params p;
  int rc = check_problem(batch, heads, kv_heads, length, head_dim, dtype, offsets, n, p);
  if (rc) return -rc;
  p.seg = seg_key;
  int64_t pq = 0, pk = 0;
  return workspace_floats(p, dtype, true, &pq, &pk) * (int64_t)sizeof(float);
}

int sbda_backward_prologue(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                           const void* v, const int64_t* vs, const void* dout, const int64_t* dos,
                           const float* lse, const float* wq, const float* wk, const float* rc,
                           const float* rs, float eps, void* dq, const int64_t* dqs, void* dk,
                           const int64_t* dks, void* dv, const int64_t* dvs, float* dwq,
                           float* dwk, void* ws, int64_t ws_bytes, int64_t batch, int64_t heads,
                           int64_t kv_heads, int64_t length, int64_t head_dim, int32_t dtype,
                           const int32_t* offsets, int32_t n, const int32_t* seg_key,
                           void* stream) {
  return backward_impl(true, q, qs, k, ks, v, vs, dout, dos, lse, wq, wk, rc, rs, eps, dq, dqs, dk,
                       dks, dv, dvs, dwq, dwk, ws, ws_bytes, batch, heads, kv_heads, length, head_dim,
                       dtype, offsets, n, seg_key, stream);
}

int64_t sbda_noalloc_scratch_bytes(void) { return kScratchBytes; }

int sbda_backward_prologue_noalloc(const void* q, const int64_t* qs, const void* k,
                                   const int64_t* ks, const void* v, const int64_t* vs,
                                   const void* dout, const int64_t* dos, const float* lse,
                                   const float* wq, const float* wk, const float* rc,
                                   const float* rs, float eps, void* dq, const int64_t* dqs,
                                   void* dk, const int64_t* dks, void* dv, const int64_t* dvs,
                                   float* dwq, float* dwk, int64_t batch, int64_t heads,
                                   int64_t kv_heads, int64_t length, int64_t head_dim,
                                   int32_t dtype, const int32_t* offsets, int32_t n,
                                   const int32_t* seg_key, void* stream) {
  // The exact need for these strides (the strides pick the kernel family);
  // refused before anything is launched when the scratch cannot hold it.
  const int64_t need = sbda_backward_workspace_for(1, qs, ks, vs, dos, dqs, dks, dvs, batch, heads,
                                                   kv_heads, length, head_dim, dtype, offsets, n,
                                                   seg_key);
  if (need < 0) return (int)-need;
  if (need > kScratchBytes)
    return fail(SBDA_ERR_VALUE,
                "allocation-free backward: this call needs %lld bytes of workspace, the library's "
                "static scratch holds %lld; call sbda_backward_prologue with a workspace instead",
                (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  int rc_ = device_scratch(&ws);
  if (rc_) return rc_;
  return backward_impl(true, q, qs, k, ks, v, vs, dout, dos, lse, wq, wk, rc, rs, eps, dq, dqs, dk,
                       dks, dv, dvs, dwq, dwk, ws, kScratchBytes, batch, heads, kv_heads, length,
                       head_dim, dtype, offsets, n, seg_key, stream);
}

int sbda_forward_paths(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                       const void* v, const int64_t* vs, void* out, const int64_t* os, float* lse,
                       const float* wq, const float* wk, const float* rc, const float* rs, float eps,
                       int64_t batch, int64_t heads, int64_t kv_heads, int64_t length,
                       int64_t head_dim, int32_t dtype, const int64_t* path_indices,
                       const uint8_t* path_valid, int32_t num_sources, const int32_t* seg_key,
                       void* stream) {
  return paths_forward_impl(q, qs, k, ks, v, vs, out, os, lse, wq, wk, rc, rs, eps, batch, heads,
                            kv_heads, length, head_dim, dtype, path_indices, path_valid,
                            num_sources, seg_key, stream);
}

int64_t sbda_backward_paths_workspace(int64_t batch, int64_t heads, int64_t kv_heads,
                                      int64_t length, int64_t head_dim, int32_t dtype,
                                      int32_t num_sources, int32_t prologue) {
  g_error.clear();
  Params p;
  int rc = check_shape(batch, heads, kv_heads, length, head_dim, dtype, p);
  if (rc) return -rc;
  if (num_sources < 1 || batch * length * num_sources >= (int64_t(1) << 31) - 1)
    return -fail(SBDA_ERR_VALUE, "source tables need 1 to 2^31 entries");
  p.PS = num_sources;
  int64_t pq = 0, pk = 0;
  const int64_t need = paths_workspace(p, esize(dtype), prologue != 0, &pq, &pk);
  if (need < 0) return -fail(SBDA_ERR_RUNTIME, "table-mode backward: cannot size the sort storage");
  return need;
}

int sbda_backward_paths(const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                        const void* v, const int64_t* vs, const void* dout, const int64_t* dos,
                        const float* lse, const float* wq, const float* wk, const float* rc,
                        const float* rs, float eps, void* dq, const int64_t* dqs, void* dk,
                        const int64_t* dks, void* dv, const int64_t* dvs, float* dwq, float* dwk,
                        void* ws, int64_t ws_bytes, int64_t batch, int64_t heads,
                        int64_t kv_heads, int64_t length, int64_t head_dim, int32_t dtype,
                        const int64_t* path_indices, const uint8_t* path_valid,
                        int32_t num_sources, const int32_t* seg_key, void* stream) {
  return paths_backward_impl(q, qs, k, ks, v, vs, dout, dos, lse, wq, wk, rc, rs, eps, dq, dqs, dk,
                             dks, dv, dvs, dwq, dwk, ws, ws_bytes, batch, heads, kv_heads, length,
                             head_dim, dtype, path_indices, path_valid, num_sources, seg_key,
                             stream);
}

int sbda_rmsnorm_forward(const void* x, const void* residual, void* sum_out, void* y,
                         const float* weight, float* rstd, int64_t rows, int64_t dim,
                         int32_t dtype, float eps, void* stream) {
  g_error.clear();
  int rc = check_rows(rows, dim, dtype, rmsnorm_max_dim(esize(dtype)));
  if (rc) return rc;
  if (!x || !y || !weight) return fail(SBDA_ERR_VALUE, "rmsnorm: null x, y or weight");
  if (residual && !sum_out) return fail(SBDA_ERR_VALUE, "rmsnorm: residual given without sum_out");
  if (!aligned16(x) || !aligned16(y) || (residual && (!aligned16(residual) || !aligned16(sum_out))))
    return fail(SBDA_ERR_VALUE, "rmsnorm: buffers must be 16-byte aligned");
  return hip_status(rmsnorm_forward(x, residual, sum_out, y, weight, rstd, rows, (int)dim, dtype,
                                    eps, reinterpret_cast<hipStream_t>(stream)),
                    "sbda rmsnorm forward launch");
}

int64_t sbda_rmsnorm_backward_workspace(int64_t rows, int64_t dim, int32_t dtype) {
  g_error.clear();
  int rc = check_rows(rows, dim, dtype, rmsnorm_max_dim(esize(dtype)));
  if (rc) return -rc;
  return rmsnorm_bwd_blocks(rows) * 4 * dim * (int64_t)sizeof(float);
}

int sbda_rmsnorm_backward(const void* dy, const void* x, const float* weight, const float* rstd,
                          const void* dsum, void* dx, float* dweight, void* workspace,
                          int64_t workspace_bytes, int64_t rows, int64_t dim, int32_t dtype,
                          void* stream) {
  g_error.clear();
  int rc = check_rows(rows, dim, dtype, rmsnorm_max_dim(esize(dtype)));
  if (rc) return rc;
  if (!dy || !x || !weight || !rstd || !dx || !dweight)
    return fail(SBDA_ERR_VALUE, "rmsnorm backward: null pointer");
  if (!aligned16(dy) || !aligned16(x) || !aligned16(dx) || (dsum && !aligned16(dsum)))
    return fail(SBDA_ERR_VALUE, "rmsnorm backward: buffers must be 16-byte aligned");
  const int64_t parts = rmsnorm_bwd_blocks(rows) * 4;
  const int64_t need = parts * dim * (int64_t)sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(SBDA_ERR_VALUE, "rmsnorm backward: workspace of %lld bytes needed, %lld given",
                (long long)need, (long long)workspace_bytes);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  hipError_t e = rmsnorm_backward(dy, x, weight, rstd, dsum, dx, part, rows, (int)dim, dtype, st);
  if (e == hipSuccess) e = launch_reduce_partials(part, parts, (int)dim, dweight, st);
  return hip_status(e, "sbda rmsnorm backward launch");
}

int sbda_swiglu_forward(const void* gate_up, void* out, int64_t rows, int64_t hidden,
                        int32_t dtype, void* stream) {
  g_error.clear();
  int rc = check_rows(rows, hidden, dtype, int64_t(1) << 24);
  if (rc) return rc;
  if (!gate_up || !out) return fail(SBDA_ERR_VALUE, "swiglu: null pointer");
  if (!aligned16(gate_up) || !aligned16(out))
    return fail(SBDA_ERR_VALUE, "swiglu: buffers must be 16-byte aligned");
  return hip_status(swiglu_forward(gate_up, out, rows, (int)hidden, dtype,
                                   reinterpret_cast<hipStream_t>(stream)),
                    "sbda swiglu forward launch");
}

int sbda_swiglu_backward(const void* dout, const void* gate_up, void* dgate_up, int64_t rows,
                         int64_t hidden, int32_t dtype, void* stream) {
  g_error.clear();
  int rc = check_rows(rows, hidden, dtype, int64_t(1) << 24);
  if (rc) return rc;
  if (!dout || !gate_up || !dgate_up) return fail(SBDA_ERR_VALUE, "swiglu backward: null pointer");
  if (!aligned16(dout) || !aligned16(gate_up) || !aligned16(dgate_up))
    return fail(SBDA_ERR_VALUE, "swiglu backward: buffers must be 16-byte aligned");
  return hip_status(swiglu_backward(dout, gate_up, dgate_up, rows, (int)hidden, dtype,
                                    reinterpret_cast<hipStream_t>(stream)),
                    "sbda swiglu backward launch");
}

int sbda_swiglu_gemm_supported(int64_t rows, int64_t dim, int64_t hidden, int32_t dtype) {
  return ffn_swiglu_supported(rows, dim, hidden, dtype) ? 1 : 0;
}

int sbda_swiglu_gemm_forward(const void* x, const void* weight, const float* bias, void* out,
                             int64_t rows, int64_t dim, int64_t hidden, int32_t dtype,
                             void* stream) {
  g_error.clear();
  if (dtype != kBF16 && dtype != kFP16)
    return fail(SBDA_ERR_DTYPE, "swiglu gemm: dtype code %d (bf16 or fp16 only)", (int)dtype);
  if (!x || !weight || !out) return fail(SBDA_ERR_VALUE, "swiglu gemm: null pointer");
  if (!ffn_swiglu_supported(rows, dim, hidden, dtype))
    return fail(SBDA_ERR_VALUE,
                "swiglu gemm: unsupported shape rows=%lld dim=%lld hidden=%lld (dim a multiple "
                "of 64, hidden a multiple of 128, rows*dim and 2*hidden*dim below 2^31)",
                (long long)rows, (long long)dim, (long long)hidden);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (bias && !aligned16(bias)))
    return fail(SBDA_ERR_VALUE, "swiglu gemm: buffers must be 16-byte aligned");
  return hip_status(ffn_swiglu_forward(x, weight, bias, out, rows, (int)dim, (int)hidden, dtype,
                                       reinterpret_cast<hipStream_t>(stream)),
                    "sbda swiglu gemm launch");
}

int sbda_rope_table(float* rope_cos, float* rope_sin, const float* inv_freq, int64_t length,
                    int64_t head_dim, void* stream) {
  g_error.clear();
  if (!rope_cos || !rope_sin || !inv_freq) return fail(SBDA_ERR_VALUE, "RoPE table: null pointer");
  if (length <= 0 || length >= (int64_t(1) << 31) || head_dim <= 0 || head_dim % 2 || head_dim > 512)
    return fail(SBDA_ERR_VALUE, "RoPE table: bad length %lld or head_dim %lld", (long long)length,
                (long long)head_dim);
  hipError_t e = launch_rope_table(rope_cos, rope_sin, inv_freq, length, (int)(head_dim / 2),
                                   reinterpret_cast<hipStream_t>(stream));
  return hip_status(e, "sbda rope table launch");
}

}  // extern "C"
