"""Row-concatenated weights kept between calls.

The modules run one GEMM over several projections whose parameters keep the
reference's names (``q``/``k``/``v`` of ``BiAttn/left_v2.py:128-133``,
``gate``/``up`` of ``BiAttn/model.py:41-44``), so the GEMM needs their rows
stacked in one matrix.  :class:`StackedRows` builds that matrix once and
rebuilds it only when a parameter changes (an in-place update bumps its
version counter; ``.to()`` or ``.data =`` gives it new storage).  Under
autograd the stacked matrix is the output of a function whose backward
splits the incoming gradient into the parameters' rows, exactly the
gradient of ``torch.cat(params, dim=0)``.
"""

from __future__ import annotations

import torch
from torch import Tensor


class StackedRows:
    """``torch.cat(tensors, dim=0)`` served from a cache."""

    def __init__(self) -> None:
        self._key: tuple | None = None
        self._buf: Tensor | None = None

    def _stacked(self, tensors: tuple[Tensor, ...]) -> Tensor:
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device, tuple(t.shape))
                    for t in tensors)
        if key != self._key or self._buf is None:
            with torch.no_grad():
                self._buf = torch.cat([t.detach() for t in tensors], dim=0)
            self._key = key
        return self._buf

    def __call__(self, *tensors: Tensor) -> Tensor:
        if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
            return _StackRows.apply(self, *tensors)
        # A fresh alias per call, so no caller can hold the cache itself.
        return self._stacked(tensors).detach()


class _StackRows(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cache: StackedRows, *tensors: Tensor) -> Tensor:
        ctx.rows = [t.shape[0] for t in tensors]
        return cache._stacked(tensors).detach()

    @staticmethod
    def backward(ctx, grad: Tensor):
        return (None, *torch.split(grad, ctx.rows, dim=0))


__all__ = ["StackedRows"]
