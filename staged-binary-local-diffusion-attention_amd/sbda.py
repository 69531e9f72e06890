"""Fused SBDA attention ops: the drop-in boundary of the reference's fused path.

``fused_sbda_key_backward(q, k, v, offsets) -> out`` keeps the signature of
the reference (``BiAttn/sbda_triton.py:1468-1475``), called from
``BiAttn/left_v2.py:268-294``: q, k, v are ``[B, H, T, D]`` tensors (usually
permuted views of ``[B, T, H, D]`` memory), ``offsets`` the layer's int32
offset buffer, and the result a new ``[B, H, T, D]`` tensor with q's dtype
and strides.  The forward saves one fp32 log-normaliser per row; the
backward writes each gradient row once (deterministic, no atomics).

``fused_sbda``, ``fused_sbda_block`` and ``fused_sbda_block_full`` -- the
reference's other backward variants of the same maths
(``sbda_triton.py:1437-1466``) -- are the same op here, and
``fused_sbda_gqa_key_backward`` accepts ``k``/``v`` with fewer heads
(``sbda_triton.py:1477-1493``).

``fused_sbda_prologue`` additionally fuses the per-head RMSNorm and RoPE of
``BiAttn/left_v2.py:237-239`` into the kernels.

Every op takes an optional ``seg_key`` (int32 ``[B, T]``, see
:func:`segment_keys`): the source masking of the reference's eager route
(``valid_mask`` holes and ``seam_reset`` segments, ``left_v2.py:329-378``)
as one key per position.  ``fused_sbda_paths`` (and ``fused_sbda_prologue``
with ``path_indices=``) take caller-supplied source tables instead of
offsets (``left_v2.py:212-231,313-378``).

Errors follow the reference's classes (``sbda_triton.py:1295-1302``):
``RuntimeError`` for a non-GPU tensor, ``ValueError`` for shapes / source
counts, ``TypeError`` for dtypes.  A missing library raises
``SBDALibraryError`` (a ``RuntimeError``); nothing falls back to another
implementation.
"""

from __future__ import annotations

import contextlib
import ctypes
import weakref
from collections import OrderedDict
from typing import Sequence

import torch

from . import _lib

_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


# ------------------------------------------------------------------ helpers

_OFFSET_CACHE: dict[int, tuple[weakref.ref, int, tuple[int, ...]]] = {}


def host_offsets(offsets) -> tuple[int, ...]:
    """Offsets as host ints.  A device tensor is read once (one sync) and
    cached until it is modified or freed."""
    if isinstance(offsets, torch.Tensor):
        if offsets.ndim != 1:
            raise ValueError("offsets must be a 1-D tensor")
        if offsets.is_inference():
            # Inference tensors keep no version counter (and may change in
            # place inside inference mode): read them every time.
            return tuple(int(x) for x in offsets.detach().to("cpu", torch.int64).tolist())
        key = id(offsets)
        hit = _OFFSET_CACHE.get(key)
        if hit is not None and hit[0]() is offsets and hit[1] == offsets._version:
            return hit[2]
        vals = tuple(int(x) for x in offsets.detach().to("cpu", torch.int64).tolist())
        _OFFSET_CACHE[key] = (weakref.ref(offsets, lambda _r, k=key: _OFFSET_CACHE.pop(k, None)),
                              offsets._version, vals)
        return vals
    return tuple(int(x) for x in offsets)


def _kernel_view(t: torch.Tensor) -> torch.Tensor:
    """``t`` if the kernels can read it in place, else a contiguous copy."""
    esz = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all((s * esz) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def _dense_like(t: torch.Tensor) -> torch.Tensor:
    """An uninitialised tensor of ``t``'s shape whose memory is dense in
    ``t``'s stride order -- ``empty_like`` for dense tensors, and for a
    strided view (q sliced out of a fused QKV projection) the same
    position-major order instead of PyTorch's contiguous fallback."""
    if t.ndim == 4 and t.transpose(1, 2).is_contiguous():
        return torch.empty_like(t)   # [B,T,H,D] memory seen as [B,H,T,D]: strides kept
    order = sorted(range(t.ndim), key=lambda i: -t.stride(i))
    base = torch.empty([t.shape[i] for i in order], dtype=t.dtype, device=t.device)
    return base.permute([order.index(i) for i in range(t.ndim)])


if hasattr(torch._C, "_cuda_getCurrentRawStream"):
    _raw_stream = torch._C._cuda_getCurrentRawStream
else:                                         # pragma: no cover - other torch builds
    def _raw_stream(index: int) -> int:
        return torch.cuda.current_stream(index).cuda_stream


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    """The current stream of ``t``'s device (the one torch's own kernels use)."""
    index = t.device.index
    return ctypes.c_void_p(_raw_stream(torch.cuda.current_device() if index is None else index))


_NO_GUARD = contextlib.nullcontext()


def _on_device(device: torch.device):
    """A device guard that switches only when ``device`` is not current."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(device)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _validate(q, k, v, offs: Sequence[int], *, gqa: bool) -> None:
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("fused SBDA requires ROCm device tensors")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must have [B,H,L,D] shapes")
    if gqa:
        if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
            raise ValueError("q/k/v sequence and head dimensions must match")
        if k.shape[1] <= 0 or q.shape[1] % k.shape[1]:
            raise ValueError("query heads must be divisible by kv heads")
    elif q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have matching [B,H,L,D] shapes")
    if len(offs) not in (2, 4):
        raise ValueError("fused SBDA supports two or four sources")
    if any(o < 0 for o in offs):
        raise ValueError("SBDA offsets must be non-negative")
    if q.dtype not in _DTYPES:
        raise TypeError("unsupported SBDA dtype")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k and v must share one dtype")
    if k.device != q.device or v.device != q.device:
        raise ValueError("q, k and v must be on one device")


def _shape_args(q, k, offs):
    b, h, t, d = q.shape
    return (b, h, k.shape[1], t, d, _DTYPES[q.dtype], _lib.offsets_array(offs), len(offs))


def segment_keys(valid_mask: torch.Tensor | None,
                 seam_reset: torch.Tensor | None) -> torch.Tensor | None:
    """One int32 key per position (``[B, T]``, contiguous) encoding the
    reference's source masks (``BiAttn/left_v2.py:329-378``).

    The segment of a position is ``cumsum(seam_reset)`` along the sequence; a
    position whose ``valid_mask`` is false gets ``-1``.  The kernels count a
    source only when its key equals the query's and the query's key is not
    ``-1``.  ``None`` when neither mask is given.

    The reference forces slot 0 of a padded query row valid so its softmax is
    finite (``left_v2.py:371``); here such a row has no source and returns
    zeros.  Its output row is multiplied by ``valid_mask`` afterwards in both,
    so module outputs and gradients agree.
    """
    if valid_mask is None and seam_reset is None:
        return None
    ref = valid_mask if valid_mask is not None else seam_reset
    if ref.ndim != 2:
        raise ValueError("masks must have shape [batch, sequence]")
    if seam_reset is not None:
        if seam_reset.shape != ref.shape:
            raise ValueError("valid_mask and seam_reset must have one shape")
        key = seam_reset.to(torch.int32).cumsum(dim=1, dtype=torch.int32)
    else:
        key = torch.zeros(ref.shape, dtype=torch.int32, device=ref.device)
    if valid_mask is not None:
        key = key.masked_fill(~valid_mask.to(torch.bool), -1)
    return key.contiguous()


def _seg_arg(seg_key: torch.Tensor | None, q: torch.Tensor) -> ctypes.c_void_p:
    if seg_key is None:
        return ctypes.c_void_p(0)
    if (seg_key.dtype != torch.int32 or seg_key.device != q.device
            or seg_key.shape != (q.shape[0], q.shape[2]) or not seg_key.is_contiguous()):
        raise ValueError("seg_key must be a contiguous int32 [B, T] tensor on q's device")
    return ctypes.c_void_p(seg_key.data_ptr())


def _workspace_bytes(lib, prologue: bool, views, shape, seg) -> int:
    """Exact backward workspace for these tensors' strides (q, k, v, grad_out,
    dq, dk, dv): the strides decide between the walk and generic kernels."""
    need = lib.sbda_backward_workspace_for(int(prologue), *(_lib.strides(x) for x in views),
                                           *shape, seg)
    if need < 0:
        _lib.check(-need)
    return int(need)


# -------------------------------------------------------- raw entry points

def _lse_storage(b: int, h: int, t: int, device) -> torch.Tensor:
    """Per-row log-normalisers, stored position-major ``[B, T, H]`` (each
    position's heads are adjacent, as in q/k/v memory) and handed out as a
    ``[B, H, T]`` view."""
    return torch.empty_strided((b, h, t), (t * h, 1, h), dtype=torch.float32, device=device)


def _lse_buffer(lse: torch.Tensor) -> torch.Tensor:
    """The ``[B, T, H]`` contiguous buffer behind a ``[B, H, T]`` lse view."""
    buf = lse.permute(0, 2, 1)
    return buf if buf.is_contiguous() else buf.contiguous()


def sbda_forward(q, k, v, offsets, seg_key=None) -> tuple[torch.Tensor, torch.Tensor]:
    """Forward without autograd: ``(out [B,H,T,D], lse [B,H,T] fp32)``."""
    offs = host_offsets(offsets)
    _validate(q, k, v, offs, gqa=True)
    lib = _lib.load()
    q, k, v = (_kernel_view(x) for x in (q, k, v))
    out = _dense_like(q)
    b, h, t, _ = q.shape
    lse = _lse_storage(b, h, t, q.device)
    with _on_device(q.device):
        _lib.check(lib.sbda_forward(
            _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
            _ptr(out), _lib.strides(out), _ptr(lse), *_shape_args(q, k, offs),
            _seg_arg(seg_key, q), _stream(q)))
    return out, lse


def sbda_backward(q, k, v, grad_out, lse, offsets, seg_key=None):
    """Backward without autograd: ``(dq, dk, dv)`` from saved ``lse``."""
    offs = host_offsets(offsets)
    _validate(q, k, v, offs, gqa=True)
    lib = _lib.load()
    q, k, v, grad_out = (_kernel_view(x) for x in (q, k, v, grad_out))
    if grad_out.shape != q.shape or grad_out.dtype != q.dtype:
        raise ValueError("grad_out must match q's shape and dtype")
    if lse.shape != q.shape[:3] or lse.dtype != torch.float32:
        raise ValueError("lse must be the fp32 [B,H,T] log-normalisers of the forward")
    lse = _lse_buffer(lse)
    dq, dk, dv = _dense_like(q), _dense_like(k), _dense_like(v)
    shape = _shape_args(q, k, offs)
    seg = _seg_arg(seg_key, q)
    need = _workspace_bytes(lib, False, (q, k, v, grad_out, dq, dk, dv), shape, seg)
    ws = torch.empty(int(need), dtype=torch.uint8, device=q.device) if need else None
    with _on_device(q.device):
        _lib.check(lib.sbda_backward(
            _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
            _ptr(grad_out), _lib.strides(grad_out), _ptr(lse),
            _ptr(dq), _lib.strides(dq), _ptr(dk), _lib.strides(dk), _ptr(dv), _lib.strides(dv),
            _ptr(ws), 0 if ws is None else ws.numel(), *shape, seg, _stream(q)))
    return dq, dk, dv


# ----------------------------------------------------------------- autograd

class _FusedSBDAKeyBackward(torch.autograd.Function):
    """O + per-row LSE forward; gather-form, atomic-free backward."""

    @staticmethod
    def forward(ctx, q, k, v, offsets, seg_key):
        out, lse = sbda_forward(q, k, v, offsets, seg_key)
        ctx.save_for_backward(_kernel_view(q), _kernel_view(k), _kernel_view(v), lse)
        ctx.offs, ctx.seg_key = host_offsets(offsets), seg_key
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, lse = ctx.saved_tensors
        dq, dk, dv = sbda_backward(q, k, v, grad_out, lse, ctx.offs, ctx.seg_key)
        return dq, dk, dv, None, None


def fused_sbda_key_backward(q, k, v, offsets, *, seg_key=None):
    """Fused SBDA attention, ``[B,H,T,D]`` in and out (``sbda_triton.py:1468-1475``)."""
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, and v must have matching [B,H,L,D] shapes")
    return _FusedSBDAKeyBackward.apply(q, k, v, offsets, seg_key)


def fused_sbda_gqa_key_backward(q, k, v, offsets, *, seg_key=None):
    """Fused SBDA with ``k``/``v`` at ``kv_heads`` (``sbda_triton.py:1477-1493``)."""
    return _FusedSBDAKeyBackward.apply(q, k, v, offsets, seg_key)


# The reference's token/block backward variants compute the same maths with
# other (atomic) backward kernels; here they are the one deterministic op.
fused_sbda = fused_sbda_key_backward
fused_sbda_block = fused_sbda_key_backward
fused_sbda_block_full = fused_sbda_key_backward


# ------------------------------------------------------ source-table ops

def _paths_check(q, path_indices, path_valid):
    b, _, t, _ = q.shape
    if (path_indices.ndim != 3 or tuple(path_indices.shape[:2]) != (b, t)
            or path_indices.shape[2] < 1):
        raise ValueError("path_indices must have shape [batch, sequence, source_count]")
    if path_indices.dtype != torch.long:
        raise ValueError("path_indices must use torch.long")
    if path_indices.device != q.device:
        raise ValueError("path_indices must be on the same device as x")
    pidx = path_indices.contiguous()
    pval = None
    if path_valid is not None:
        if (path_valid.shape != path_indices.shape or path_valid.dtype != torch.bool
                or path_valid.device != q.device):
            raise ValueError("path_valid must match path_indices as a bool tensor")
        pval = path_valid.contiguous()
    return pidx, pval


def _prologue_ptrs(pro):
    if pro is None:
        return (ctypes.c_void_p(0),) * 4 + (0.0,)
    wq, wk, cos, sin, eps = pro
    return _ptr(wq), _ptr(wk), _ptr(cos), _ptr(sin), float(eps)


def _paths_shape(q, k, pidx):
    b, h, t, d = q.shape
    return (b, h, k.shape[1], t, d, _DTYPES[q.dtype])


def sbda_forward_paths(q, k, v, path_indices, path_valid=None, seg_key=None, *, prologue=None):
    """Table-mode forward without autograd: ``(out [B,H,T,D], lse [B,H,T])``.

    ``prologue``: ``(q_weight32, k_weight32, cos, sin, eps)`` to fuse the
    head-RMSNorm + RoPE of raw q/k, or ``None``."""
    _validate(q, k, v, (0, 0), gqa=True)
    pidx, pval = _paths_check(q, path_indices, path_valid)
    lib = _lib.load()
    q, k, v = (_kernel_view(x) for x in (q, k, v))
    out = _dense_like(q)
    b, h, t, _ = q.shape
    lse = _lse_storage(b, h, t, q.device)
    with _on_device(q.device):
        _lib.check(lib.sbda_forward_paths(
            _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
            _ptr(out), _lib.strides(out), _ptr(lse), *_prologue_ptrs(prologue),
            *_paths_shape(q, k, pidx), _ptr(pidx), _ptr(pval), pidx.shape[2],
            _seg_arg(seg_key, q), _stream(q)))
    return out, lse


def sbda_backward_paths(q, k, v, grad_out, lse, path_indices, path_valid=None, seg_key=None,
                        *, prologue=None):
    """Table-mode backward: ``(dq, dk, dv, dq_weight, dk_weight)``, the last
    two fp32 ``[D]`` with the prologue and ``None`` without."""
    _validate(q, k, v, (0, 0), gqa=True)
    pidx, pval = _paths_check(q, path_indices, path_valid)
    lib = _lib.load()
    q, k, v, grad_out = (_kernel_view(x) for x in (q, k, v, grad_out))
    if grad_out.shape != q.shape or grad_out.dtype != q.dtype:
        raise ValueError("grad_out must match q's shape and dtype")
    if lse.shape != q.shape[:3] or lse.dtype != torch.float32:
        raise ValueError("lse must be the fp32 [B,H,T] log-normalisers of the forward")
    lse = _lse_buffer(lse)
    dq, dk, dv = _dense_like(q), _dense_like(k), _dense_like(v)
    d = q.shape[-1]
    dwq = dwk = None
    if prologue is not None:
        dwq = torch.empty(d, dtype=torch.float32, device=q.device)
        dwk = torch.empty_like(dwq)
    shape = _paths_shape(q, k, pidx)
    need = lib.sbda_backward_paths_workspace(*shape, pidx.shape[2], int(prologue is not None))
    if need < 0:
        _lib.check(-need)
    ws = torch.empty(int(need) + 256, dtype=torch.uint8, device=q.device)
    ws_view = ws[(-ws.data_ptr()) % 256:]
    with _on_device(q.device):
        _lib.check(lib.sbda_backward_paths(
            _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
            _ptr(grad_out), _lib.strides(grad_out), _ptr(lse), *_prologue_ptrs(prologue),
            _ptr(dq), _lib.strides(dq), _ptr(dk), _lib.strides(dk), _ptr(dv), _lib.strides(dv),
            _ptr(dwq), _ptr(dwk), _ptr(ws_view), ws_view.numel(),
            *shape, _ptr(pidx), _ptr(pval), pidx.shape[2], _seg_arg(seg_key, q), _stream(q)))
    return dq, dk, dv, dwq, dwk


class _FusedSBDAPaths(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_weight, k_weight, path_indices, path_valid, seg_key, theta, eps):
        pro = None
        if q_weight is not None:
            d = q.shape[-1]
            wq, wk = _weight32(q_weight, d, q.device), _weight32(k_weight, d, q.device)
            cos, sin = rope_tables(q.shape[2], d, theta, q.device)
            pro = (wq, wk, cos, sin, float(eps))
            ctx.wdtypes = (q_weight.dtype, k_weight.dtype)
        out, lse = sbda_forward_paths(q, k, v, path_indices, path_valid, seg_key, prologue=pro)
        ctx.save_for_backward(_kernel_view(q), _kernel_view(k), _kernel_view(v), lse)
        ctx.tables = (path_indices, path_valid, seg_key)
        ctx.pro = pro
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, lse = ctx.saved_tensors
        g = grad_out if grad_out.dtype == q.dtype else grad_out.to(q.dtype)
        dq, dk, dv, dwq, dwk = sbda_backward_paths(q, k, v, g, lse, *ctx.tables, prologue=ctx.pro)
        if ctx.pro is not None:
            dwq, dwk = dwq.to(ctx.wdtypes[0]), dwk.to(ctx.wdtypes[1])
        return dq, dk, dv, dwq, dwk, None, None, None, None, None


def fused_sbda_paths(q, k, v, path_indices, path_valid=None, *, seg_key=None):
    """SBDA attention over caller-supplied source tables, ``[B,H,T,D]`` in and out.

    ``path_indices``: int64 ``[B, T, S]`` source positions, ``path_valid``:
    bool ``[B, T, S]`` or ``None``; a source counts when valid, ``j <= i`` and
    (with ``seg_key``) in the query's segment -- the eager route of
    ``BiAttn/left_v2.py:313-378``.  ``k``/``v`` may have fewer heads (GQA)."""
    return _FusedSBDAPaths.apply(q, k, v, None, None, path_indices, path_valid, seg_key,
                                 0.0, 0.0)


# ------------------------------------------------------- fused prologue op

_ROPE_CACHE: "OrderedDict[tuple, tuple[torch.Tensor, torch.Tensor]]" = OrderedDict()
_ROPE_CACHE_LIMIT = 4


def rope_inverse_frequencies(head_dim: int, theta: float) -> torch.Tensor:
    """``theta ** (-arange(0, D, 2) / D)`` in fp32 on the CPU, the expression of
    ``BiAttn/attention_common.py:16-17``, so angles match the reference bit for bit."""
    idx = torch.arange(0, head_dim, 2, dtype=torch.float32)
    return theta ** (-idx / head_dim)


def rope_tables(length: int, head_dim: int, theta: float,
                device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    """Device fp32 ``[length, head_dim/2]`` cos/sin tables (cached).

    The angles and their cos/sin are evaluated in fp32 as the reference does
    (``attention_common.py:16-19``); the reference then rounds the tables to
    the activation dtype (``:20-21``), these stay fp32 for every dtype (a
    deliberate difference: the parity bar is an fp32 reference).

    A table is built outside HIP-graph capture only: built during capture, its
    memory would come from the graph's pool and its fill kernel would run only
    on replay, so eager calls before the first replay would read garbage.
    Call once (a warm-up step) before capturing."""
    device = torch.device(device)
    key = (device, int(length), int(head_dim), float(theta))
    hit = _ROPE_CACHE.get(key)
    if hit is not None:
        _ROPE_CACHE.move_to_end(key)
        return hit
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"RoPE tables for length {length}, head_dim {head_dim}, theta {theta} are not "
            "built yet; run one eager call (a warm-up step) before HIP-graph capture")
    inv = rope_inverse_frequencies(head_dim, theta).contiguous()
    cos = torch.empty((length, head_dim // 2), dtype=torch.float32, device=device)
    sin = torch.empty_like(cos)
    lib = _lib.load()
    with torch.cuda.device(device):
        _lib.check(lib.sbda_rope_table(
            _ptr(cos), _ptr(sin), ctypes.cast(inv.data_ptr(), ctypes.POINTER(ctypes.c_float)),
            length, head_dim, ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)))
    _ROPE_CACHE[key] = (cos, sin)
    while len(_ROPE_CACHE) > _ROPE_CACHE_LIMIT:
        _ROPE_CACHE.popitem(last=False)
    return cos, sin


def _weight32(w: torch.Tensor, d: int, device) -> torch.Tensor:
    if w.shape != (d,):
        raise ValueError(f"norm weight must have shape ({d},)")
    return w.detach().to(device=device, dtype=torch.float32).contiguous()


class _FusedSBDAPrologue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_raw, k_raw, v, q_weight, k_weight, offsets, theta, eps, seg_key):
        offs = host_offsets(offsets)
        _validate(q_raw, k_raw, v, offs, gqa=True)
        lib = _lib.load()
        q, k, v = (_kernel_view(x) for x in (q_raw, k_raw, v))
        b, h, t, d = q.shape
        wq, wk = _weight32(q_weight, d, q.device), _weight32(k_weight, d, q.device)
        cos, sin = rope_tables(t, d, theta, q.device)
        out = _dense_like(q)
        lse = _lse_storage(b, h, t, q.device)
        with _on_device(q.device):
            _lib.check(lib.sbda_forward_prologue(
                _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
                _ptr(out), _lib.strides(out), _ptr(lse), _ptr(wq), _ptr(wk), _ptr(cos), _ptr(sin),
                float(eps), *_shape_args(q, k, offs), _seg_arg(seg_key, q), _stream(q)))
        ctx.save_for_backward(q, k, v, wq, wk, lse, cos, sin)
        ctx.offs, ctx.eps, ctx.seg_key = offs, float(eps), seg_key
        ctx.wdtypes = (q_weight.dtype, k_weight.dtype)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v, wq, wk, lse, cos, sin = ctx.saved_tensors
        offs = ctx.offs
        lib = _lib.load()
        g = _kernel_view(grad_out)
        if g.dtype != q.dtype:
            g = g.to(q.dtype)
        dq, dk, dv = _dense_like(q), _dense_like(k), _dense_like(v)
        d = q.shape[-1]
        dwq = torch.empty(d, dtype=torch.float32, device=q.device)
        dwk = torch.empty_like(dwq)
        shape = _shape_args(q, k, offs)
        seg = _seg_arg(ctx.seg_key, q)
        need = _workspace_bytes(lib, True, (q, k, v, g, dq, dk, dv), shape, seg)
        ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=q.device)
        with _on_device(q.device):
            _lib.check(lib.sbda_backward_prologue(
                _ptr(q), _lib.strides(q), _ptr(k), _lib.strides(k), _ptr(v), _lib.strides(v),
                _ptr(g), _lib.strides(g), _ptr(lse), _ptr(wq), _ptr(wk), _ptr(cos), _ptr(sin),
                ctx.eps, _ptr(dq), _lib.strides(dq), _ptr(dk), _lib.strides(dk),
                _ptr(dv), _lib.strides(dv), _ptr(dwq), _ptr(dwk), _ptr(ws), ws.numel(),
                *shape, seg, _stream(q)))
        return (dq, dk, dv, dwq.to(ctx.wdtypes[0]), dwk.to(ctx.wdtypes[1]),
                None, None, None, None)


def fused_sbda_prologue(q_raw, k_raw, v, offsets, q_weight, k_weight, *,
                        theta: float, eps: float = 1e-6, seg_key=None,
                        path_indices=None, path_valid=None):
    """Head-RMSNorm(q, k) -> RoPE -> SBDA attention in one fused op.

    ``q_raw``: ``[B, H, T, D]`` projections before normalisation; ``k_raw``,
    ``v``: ``[B, Hkv, T, D]``; ``q_weight``/``k_weight``: ``[D]`` norm
    weights.  Equals ``fused_sbda_key_backward(rope(norm(q)), rope(norm(k)),
    v, offsets)`` with the reference's prologue (``BiAttn/left_v2.py:237-239``).
    With ``path_indices`` (and optionally ``path_valid``) the sources come from
    those tables and ``offsets`` is ignored (see :func:`fused_sbda_paths`).
    """
    if path_indices is not None:
        return _FusedSBDAPaths.apply(q_raw, k_raw, v, q_weight, k_weight, path_indices,
                                     path_valid, seg_key, float(theta), float(eps))
    return _FusedSBDAPrologue.apply(q_raw, k_raw, v, q_weight, k_weight, offsets,
                                    float(theta), float(eps), seg_key)


__all__ = [
    "fused_sbda", "fused_sbda_block", "fused_sbda_block_full",
    "fused_sbda_key_backward", "fused_sbda_gqa_key_backward",
    "fused_sbda_paths", "fused_sbda_prologue", "host_offsets", "rope_inverse_frequencies", "rope_tables",
    "sbda_backward", "sbda_backward_paths", "sbda_forward", "sbda_forward_paths",
    "segment_keys",
]
