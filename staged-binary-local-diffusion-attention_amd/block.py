"""Fused ops for the steps next to the attention in the SBDA backbone block.

``BiAttn/model.py`` runs, per block, ``F.rms_norm`` twice, two residual adds
and ``F.silu(gate(x)) * up(x)`` as separate eager ops (``model.py:18-59,
321-335``); each is a full pass over a ``[T, dim]`` or ``[T, hidden]``
activation.  Here they are HIP kernels (``csrc/sbda_block.hip``):

* :func:`fused_add_rms_norm` -- ``s = x + residual`` and ``rms_norm(s)`` in one
  pass (both returned), with a backward that adds the gradient reaching ``s``
  from its other uses;
* :func:`fused_rms_norm` -- ``rms_norm(x)`` alone;
* :func:`fused_swiglu` -- ``silu(gate) * up`` on the output of one
  ``[gate | up]`` GEMM;
* :func:`fused_swiglu_gemm` -- the ``[gate | up]`` GEMM itself with the
  activation in its epilogue (an MFMA kernel, ``csrc/sbda_ffn.hip``), for
  calls that need no gradient: the ``[T, 2 * hidden]`` product is never
  written.

Device tensors only; errors follow the attention ops' classes.
"""

from __future__ import annotations

import torch

from . import _lib
from .sbda import _DTYPES, _on_device, _ptr, _stream


def _rows(x: torch.Tensor, width: int) -> torch.Tensor:
    if not x.is_cuda:
        raise RuntimeError("fused block ops require ROCm device tensors")
    if x.dtype not in _DTYPES:
        raise TypeError("unsupported dtype for the fused block ops")
    if x.shape[-1] != width:
        raise ValueError(f"last dimension must be {width}")
    x = x.contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    return x


class _AddRMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, residual, weight, eps):
        dim = x.shape[-1]
        xs = _rows(x, dim)
        rs = None if residual is None else _rows(residual, dim)
        if rs is not None and (rs.shape != xs.shape or rs.dtype != xs.dtype):
            raise ValueError("residual must match x")
        w32 = weight.detach().to(device=x.device, dtype=torch.float32).contiguous()
        rows = xs.numel() // dim
        y = torch.empty_like(xs)
        s = torch.empty_like(xs) if rs is not None else xs
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        lib = _lib.load()
        with _on_device(x.device):
            _lib.check(lib.sbda_rmsnorm_forward(
                _ptr(xs), _ptr(rs), _ptr(s if rs is not None else None), _ptr(y), _ptr(w32),
                _ptr(rstd), rows, dim, _DTYPES[x.dtype], float(eps), _stream(x)))
        ctx.save_for_backward(s, w32, rstd)
        ctx.has_residual = rs is not None
        ctx.wdtype = weight.dtype
        if rs is None:
            return y
        return s, y

    @staticmethod
    def backward(ctx, *grads):
        s, w32, rstd = ctx.saved_tensors
        if ctx.has_residual:
            ds, dy = grads
        else:
            ds, dy = None, grads[0]
        dim = s.shape[-1]
        rows = s.numel() // dim
        dy = _rows(dy.to(s.dtype), dim) if dy is not None else torch.zeros_like(s)
        ds = None if ds is None else _rows(ds.to(s.dtype), dim)
        dx = torch.empty_like(s)
        dw = torch.empty(dim, dtype=torch.float32, device=s.device)
        lib = _lib.load()
        need = lib.sbda_rmsnorm_backward_workspace(rows, dim, _DTYPES[s.dtype])
        if need < 0:
            _lib.check(-need)
        ws = torch.empty(max(int(need), 16), dtype=torch.uint8, device=s.device)
        with _on_device(s.device):
            _lib.check(lib.sbda_rmsnorm_backward(
                _ptr(dy), _ptr(s), _ptr(w32), _ptr(rstd), _ptr(ds), _ptr(dx), _ptr(dw), _ptr(ws),
                ws.numel(), rows, dim, _DTYPES[s.dtype], _stream(s)))
        dw = dw.to(ctx.wdtype)
        if ctx.has_residual:
            return dx, dx, dw, None
        return dx, None, dw, None


def fused_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``F.rms_norm(x, (dim,), weight, eps)`` as one HIP pass."""
    return _AddRMSNorm.apply(x, None, weight, eps)


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                       eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """``s = x + residual`` (rounded to the dtype) and ``rms_norm(s)``, one pass."""
    return _AddRMSNorm.apply(x, residual, weight, eps)


class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate_up):
        two_h = gate_up.shape[-1]
        if two_h % 2:
            raise ValueError("gate_up must hold [gate | up] halves")
        hidden = two_h // 2
        gu = _rows(gate_up, two_h)
        rows = gu.numel() // two_h
        out = torch.empty(*gu.shape[:-1], hidden, dtype=gu.dtype, device=gu.device)
        lib = _lib.load()
        with _on_device(gu.device):
            _lib.check(lib.sbda_swiglu_forward(_ptr(gu), _ptr(out), rows, hidden,
                                               _DTYPES[gu.dtype], _stream(gu)))
        ctx.save_for_backward(gu)
        return out

    @staticmethod
    def backward(ctx, dout):
        (gu,) = ctx.saved_tensors
        two_h = gu.shape[-1]
        hidden = two_h // 2
        rows = gu.numel() // two_h
        d = _rows(dout.to(gu.dtype), hidden)
        dgu = torch.empty_like(gu)
        lib = _lib.load()
        with _on_device(gu.device):
            _lib.check(lib.sbda_swiglu_backward(_ptr(d), _ptr(gu), _ptr(dgu), rows, hidden,
                                                _DTYPES[gu.dtype], _stream(gu)))
        return dgu


def fused_swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` for ``gate_up = [gate | up]`` along the last dim."""
    return _SwiGLU.apply(gate_up)


def swiglu_gemm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether :func:`fused_swiglu_gemm` takes these operands (device bf16 or
    fp16, ``dim`` a multiple of 64, ``hidden`` a multiple of 128)."""
    if not (x.is_cuda and weight.is_cuda) or x.dtype != weight.dtype:
        return False
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.ndim != 2:
        return False
    dim = x.shape[-1]
    if weight.shape[1] != dim or weight.shape[0] % 2:
        return False
    rows = x.numel() // dim if dim else 0
    return bool(_lib.load().sbda_swiglu_gemm_supported(rows, dim, weight.shape[0] // 2,
                                                        _DTYPES[x.dtype]))


def fused_swiglu_gemm(x: torch.Tensor, weight: torch.Tensor,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(x @ Wg.T + bg) * (x @ Wu.T + bu)`` for ``weight = [Wg; Wu]``
    (``[2 * hidden, dim]``) as one HIP kernel.  No autograd graph is
    recorded: call it where no gradient is needed (inference, ``no_grad``)."""
    if not swiglu_gemm_supported(x, weight):
        raise ValueError("fused_swiglu_gemm: unsupported operands (device bf16/fp16, dim a "
                         "multiple of 64, hidden a multiple of 128)")
    dim = x.shape[-1]
    hidden = weight.shape[0] // 2
    xs = _rows(x.detach(), dim)
    ws = _rows(weight.detach(), dim)
    b32 = None
    if bias is not None:
        if bias.shape != (2 * hidden,):
            raise ValueError("bias must have shape [2 * hidden]")
        b32 = bias.detach().to(device=x.device, dtype=torch.float32).contiguous()
    rows = xs.numel() // dim
    out = torch.empty(*xs.shape[:-1], hidden, dtype=xs.dtype, device=xs.device)
    lib = _lib.load()
    with _on_device(x.device):
        _lib.check(lib.sbda_swiglu_gemm_forward(_ptr(xs), _ptr(ws), _ptr(b32), _ptr(out), rows,
                                                dim, hidden, _DTYPES[xs.dtype], _stream(xs)))
    return out


__all__ = ["fused_add_rms_norm", "fused_rms_norm", "fused_swiglu", "fused_swiglu_gemm",
           "swiglu_gemm_supported"]
