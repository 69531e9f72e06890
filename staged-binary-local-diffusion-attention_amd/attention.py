"""Module counterpart of the reference's sparse attention layer.

``BinaryPathAttention`` / ``SBDAttention`` keep the constructor keywords and
the ``forward(x, valid_mask, seam_reset, path_indices, path_valid)``
signature of ``BiAttn/left_v2.py:100-116,191-198,413-438`` and the same
parameter names (``q``, ``k``, ``v``, ``q_norm.weight``, ``k_norm.weight``,
``out.weight``), so a reference state dict loads unchanged.

The fused route is the only route: projections run in PyTorch, then
head-RMSNorm + RoPE + SBDA attention run as one HIP op
(:func:`sbda.fused_sbda_prologue`), then the output projection and the
``valid_mask`` multiply (``left_v2.py:295-305``).  What the reference sends
to its eager gather path also runs in HIP here: a ``valid_mask`` with
interior holes and ``seam_reset`` (``left_v2.py:329-378``) through a
per-position segment key (:func:`sbda.segment_keys`), caller-supplied
``path_indices``/``path_valid`` through the source-table kernels
(:func:`sbda.fused_sbda_paths`).  What is left -- offset routes with other
than two or four offsets, ``use_fused``/``use_sdpa`` off, a CPU tensor --
raises ``NotImplementedError`` rather than silently taking a slower path.
"""

from __future__ import annotations

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from ._weights import StackedRows
from .sbda import fused_sbda_prologue, segment_keys
from .topology import PATH_TOPOLOGIES, topology_offsets


class _HeadRMSNorm(nn.Module):
    """Holds the per-head norm weight (``attention_common.py:64-73``); the
    normalisation itself runs inside the fused kernel."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class BinaryPathAttention(nn.Module):
    """Causal exact-token attention over a sparse per-layer source set."""

    def __init__(self, dim: int, heads: int, layer: int, *, kv_heads: int | None = None,
                 rope_theta: float = 1_000_000.0, topology: str = "binary",
                 total_layers: int = 12, use_sdpa: bool = True, use_fused: bool = True,
                 backward_mode: str = "token") -> None:
        super().__init__()
        if dim <= 0 or heads <= 0 or dim % heads:
            raise ValueError("dim must be positive, heads must be positive, and divide dim")
        if layer < 1:
            raise ValueError("layer must be positive")
        if backward_mode not in ("token", "block", "key"):
            raise ValueError("backward_mode must be token, block, or key")
        if topology not in PATH_TOPOLOGIES:
            raise ValueError(f"unknown path topology: {topology}")
        self.dim, self.heads, self.layer = int(dim), int(heads), int(layer)
        self.total_layers = int(total_layers)
        self.use_sdpa, self.use_fused = bool(use_sdpa), bool(use_fused)
        self.backward_mode = backward_mode
        self.topology = topology
        self.offsets = topology_offsets(self.layer, topology=topology,
                                        total_layers=self.total_layers)
        self.register_buffer("_fused_offsets", torch.tensor(self.offsets, dtype=torch.int32),
                             persistent=False)
        self.kv_heads = self.heads if kv_heads is None else int(kv_heads)
        if self.kv_heads <= 0 or self.heads % self.kv_heads:
            raise ValueError("heads must be divisible by kv_heads")
        self.head_dim = self.dim // self.heads
        self.rope_theta = float(rope_theta)
        if self.rope_theta <= 0:
            raise ValueError("rope_theta must be positive")
        self.q = nn.Linear(dim, dim, bias=False)
        self.k = nn.Linear(dim, self.kv_heads * self.head_dim, bias=False)
        self.v = nn.Linear(dim, self.kv_heads * self.head_dim, bias=False)
        self.q_norm = _HeadRMSNorm(self.head_dim)
        self.k_norm = _HeadRMSNorm(self.head_dim)
        self.out = nn.Linear(dim, dim, bias=False)
        # [q; k; v] rows for the one projection GEMM, rebuilt only when a weight changes.
        self._qkv_weight = StackedRows()

    def _check_inputs(self, x, valid_mask, seam_reset, path_indices, path_valid):
        # Same validation and messages as left_v2.py:199-232.
        if x.ndim != 3:
            raise ValueError("x must have shape [batch, sequence, dim]")
        batch, length, dim = x.shape
        if dim != self.dim:
            raise ValueError(f"expected dim={self.dim}, got {dim}")
        if valid_mask is not None and (valid_mask.shape != (batch, length)
                                       or valid_mask.dtype != torch.bool):
            raise ValueError("valid_mask must be bool with input shape")
        if seam_reset is not None and (seam_reset.shape != (batch, length)
                                       or seam_reset.dtype != torch.bool):
            raise ValueError("seam_reset must be bool with input shape")
        if path_indices is not None:
            if path_indices.ndim != 3 or path_indices.shape[:2] != (batch, length):
                raise ValueError("path_indices must have shape [batch, sequence, source_count]")
            if path_indices.dtype != torch.long:
                raise ValueError("path_indices must use torch.long")
            if path_indices.device != x.device:
                raise ValueError("path_indices must be on the same device as x")
            if path_valid is not None and (path_valid.shape != path_indices.shape
                                           or path_valid.dtype != torch.bool
                                           or path_valid.device != x.device):
                raise ValueError("path_valid must match path_indices as a bool tensor")
            if path_indices.numel() and (int(path_indices.min()) < 0
                                         or int(path_indices.max()) >= length):
                raise ValueError("path_indices contains an out-of-range source")

    def forward(self, x: Tensor, valid_mask: Tensor | None = None,
                seam_reset: Tensor | None = None, path_indices: Tensor | None = None,
                path_valid: Tensor | None = None) -> Tensor:
        self._check_inputs(x, valid_mask, seam_reset, path_indices, path_valid)
        batch, length, dim = x.shape
        # A right-padded prefix mask needs no per-source check (left_v2.py:252-262):
        # causal sources of a valid row are valid.
        prefix_mask = (valid_mask is None or valid_mask.shape[1] < 2
                       or bool(torch.all(~valid_mask[:, 1:] | valid_mask[:, :-1])))
        reasons = []
        if not x.is_cuda:
            reasons.append("a CPU tensor")
        if not (self.use_fused and self.use_sdpa):
            reasons.append("use_fused/use_sdpa disabled")
        if path_indices is None and path_valid is not None:
            reasons.append("path_valid without path_indices")
        if path_indices is None and len(self.offsets) not in (2, 4):
            reasons.append(f"{len(self.offsets)} offsets")
        if reasons:
            raise NotImplementedError(
                "SBDA-AMD runs only the reference's fused route; this call needs the eager "
                "gather path because of " + ", ".join(reasons))
        seg_key = None if prefix_mask and seam_reset is None else segment_keys(
            valid_mask, seam_reset)
        # One GEMM for q, k and v; the kernels read the three column blocks of
        # its output in place (strided views, no copies).
        kvd = self.kv_heads * self.head_dim
        qkv = F.linear(x, self._qkv_weight(self.q.weight, self.k.weight, self.v.weight))
        q = qkv[..., :dim].view(batch, length, self.heads, self.head_dim)
        k = qkv[..., dim:dim + kvd].view(batch, length, self.kv_heads, self.head_dim)
        v = qkv[..., dim + kvd:].view(batch, length, self.kv_heads, self.head_dim)
        attended = fused_sbda_prologue(
            q.permute(0, 2, 1, 3), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3),
            self._fused_offsets, self.q_norm.weight, self.k_norm.weight,
            theta=self.rope_theta, eps=self.q_norm.eps, seg_key=seg_key,
            path_indices=path_indices, path_valid=path_valid)
        out = self.out(attended.transpose(1, 2).reshape(batch, length, dim))
        if valid_mask is not None:
            out = out * valid_mask[:, :, None].to(dtype=out.dtype)
        return out


class SBDAttention(BinaryPathAttention):
    """Staged Binary-Local Diffusion Attention (``left_v2.py:413-438``)."""

    def __init__(self, dim: int, heads: int, layer: int, *, kv_heads: int | None = None,
                 rope_theta: float = 1_000_000.0, total_layers: int = 12,
                 use_sdpa: bool = True, use_fused: bool = True,
                 backward_mode: str = "key") -> None:
        super().__init__(dim, heads, layer, kv_heads=kv_heads, rope_theta=rope_theta,
                         topology="sbda", total_layers=total_layers, use_sdpa=use_sdpa,
                         use_fused=use_fused, backward_mode=backward_mode)


SBDAAttention = SBDAttention

__all__ = ["BinaryPathAttention", "SBDAttention", "SBDAAttention"]
