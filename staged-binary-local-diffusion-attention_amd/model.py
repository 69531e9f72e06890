"""Backbone counterpart of ``BiAttn/model.py`` for the SBDA backend.

The caller of the fused attention: ``BiAttnConfig``, ``BiAttnBlock`` and
``BiAttnLM`` keep the reference's names, config fields, defaults (except the
backend, see below), parameter names and weight initialisation
(``BiAttn/model.py:18-59,151-247,248-502``), with every attention layer an
:class:`SBDAttention` that runs norm + RoPE + attention as one HIP op.

Only what the SBDA route uses is here: ``attention_backend`` must be
``"sbda"`` (the default in this mirror), the feed-forward is the dense SwiGLU,
token IO is a plain (tied) embedding.  The reference's other backends, the
DeepSeekMoE feed-forward and factorized token IO raise ``ValueError``.
Per-layer source tables (``path_indices [B, layers, T, S]``) and the
per-row layer switch ``path_active [B, layers]`` follow
``BiAttn/model.py:397-466``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor, nn
from torch.nn import functional as F

from ._weights import StackedRows
from .attention import SBDAttention
from .block import (fused_add_rms_norm, fused_rms_norm, fused_swiglu, fused_swiglu_gemm,
                    swiglu_gemm_supported)


class RMSNorm(nn.Module):
    """``BiAttn/model.py:18-29``.  Device tensors run the HIP kernel
    (:func:`block.fused_rms_norm`); CPU tensors run ``F.rms_norm`` as the
    reference module does."""

    def __init__(self, dim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: Tensor) -> Tensor:
        if x.is_cuda:
            return fused_rms_norm(x, self.weight, self.eps)
        return F.rms_norm(x, (self.dim,), self.weight, self.eps)

    def add_forward(self, x: Tensor, residual: Tensor) -> tuple[Tensor, Tensor]:
        """``(x + residual, norm(x + residual))`` in one pass (device tensors)."""
        return fused_add_rms_norm(x, residual, self.weight, self.eps)


class SwiGLU(nn.Module):
    """``BiAttn/model.py:32-59``: width ``ceil(dim * pi / 64) * 64`` unless given."""

    def __init__(self, dim: int, ff_mult: float, dropout: float = 0.0, *,
                 hidden_size: int | None = None, bias: bool = True) -> None:
        super().__init__()
        hidden = (max(64, math.ceil(dim * math.pi / 64) * 64)
                  if hidden_size is None else hidden_size)
        if hidden < 1:
            raise ValueError("SwiGLU hidden_size must be positive")
        self.hidden_size = hidden
        self.gate = nn.Linear(dim, hidden, bias=bias)
        self.up = nn.Linear(dim, hidden, bias=bias)
        self.down = nn.Linear(hidden, dim, bias=bias)
        self.dropout = nn.Dropout(dropout)
        # [gate; up] rows (and biases) for the one GEMM, rebuilt only when they change.
        self._gate_up_weight = StackedRows()
        self._gate_up_bias = StackedRows()

    def forward(self, x: Tensor) -> Tensor:
        if not x.is_cuda:
            return self.dropout(self.down(F.silu(self.gate(x)) * self.up(x)))
        weight = self._gate_up_weight(self.gate.weight, self.up.weight)
        bias = (None if self.gate.bias is None
                else self._gate_up_bias(self.gate.bias, self.up.bias))
        if not torch.is_grad_enabled() and swiglu_gemm_supported(x, weight):
            # No gradient needed: the [gate | up] GEMM with the activation in
            # its epilogue, one MFMA kernel.
            return self.dropout(self.down(fused_swiglu_gemm(x, weight, bias)))
        # One [gate | up] GEMM, then silu(gate) * up in one HIP pass.
        return self.dropout(self.down(fused_swiglu(F.linear(x, weight, bias))))


@dataclass
class BiAttnConfig:
    """The reference's config fields that the SBDA route reads (``model.py:151-247``)."""

    vocab_size: int
    dim: int = 128
    layers: int = 12
    heads: int = 4
    kv_heads: int | None = None
    rope_theta: float = 1_000_000.0
    ff_mult: float = 2.0
    ff_hidden: int | None = None
    ff_bias: bool = False
    ff_mode: str = "dense"
    dropout: float = 0.0
    tie_embeddings: bool = True
    attention_backend: str = "sbda"
    path_sdpa: bool = True
    sbda_fused: bool = True
    sbda_backward: str = "key"
    token_emb_dim: int | None = None

    def window_schedule(self) -> tuple[int, ...]:
        return tuple(2 ** (index + 1) for index in range(self.layers))

    def validate(self) -> None:
        if self.vocab_size <= 0 or self.dim <= 0 or self.layers <= 0:
            raise ValueError("vocab_size, dim, and layers must be positive")
        if self.attention_backend != "sbda":
            raise ValueError("this backbone mirrors the sbda attention backend only")
        if self.heads <= 0 or self.dim % self.heads:
            raise ValueError("dim must be divisible by heads")
        kv_heads = self.heads if self.kv_heads is None else self.kv_heads
        if kv_heads <= 0 or self.heads % kv_heads:
            raise ValueError("heads must be divisible by kv_heads")
        if self.rope_theta <= 0:
            raise ValueError("rope_theta must be positive")
        if self.ff_mult <= 0 or not 0 <= self.dropout < 1:
            raise ValueError("ff_mult must be positive and dropout in [0, 1)")
        if self.ff_mode != "dense":
            raise ValueError("only the dense SwiGLU feed-forward is mirrored")
        if self.sbda_backward not in ("token", "block", "key"):
            raise ValueError("sbda_backward must be token, block, or key")
        if self.ff_hidden is not None and self.ff_hidden <= 0:
            raise ValueError("ff_hidden must be positive when provided")
        if self.token_emb_dim is not None:
            raise ValueError("factorized token IO is not mirrored")


class BiAttnBlock(nn.Module):
    """Pre-norm block: ``x + attn(norm1(x))``, then ``+ ff(norm2(x))`` masked
    by ``valid_mask`` (``BiAttn/model.py:248-335``)."""

    def __init__(self, config: BiAttnConfig, layer_index: int) -> None:
        super().__init__()
        self.layer_index = int(layer_index)
        self.norm1 = RMSNorm(config.dim)
        self.attn = SBDAttention(
            config.dim, config.heads, layer=layer_index + 1, kv_heads=config.kv_heads,
            rope_theta=config.rope_theta, total_layers=config.layers,
            use_sdpa=config.path_sdpa, use_fused=config.sbda_fused,
            backward_mode=config.sbda_backward)
        self.norm2 = RMSNorm(config.dim)
        self.ff = SwiGLU(config.dim, config.ff_mult, config.dropout,
                         hidden_size=config.ff_hidden, bias=config.ff_bias)

    def forward(self, x: Tensor, valid_mask: Optional[Tensor],
                seam_reset: Optional[Tensor] = None, path_indices: Optional[Tensor] = None,
                path_valid: Optional[Tensor] = None) -> Tensor:
        x, ff = self.forward_pending(x, None, valid_mask, seam_reset, path_indices, path_valid)
        return x + ff

    def forward_pending(self, x: Tensor, pending: Optional[Tensor], valid_mask: Optional[Tensor],
                        seam_reset: Optional[Tensor] = None,
                        path_indices: Optional[Tensor] = None,
                        path_valid: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
        """The block on ``x + pending`` (``pending`` = the previous block's
        feed-forward output, not yet added), returning ``(x', ff)`` with the
        block output ``x' + ff`` left unsummed so the next norm can fuse the
        add.  Each residual add runs inside an RMSNorm pass."""
        layer_paths = None if path_indices is None else path_indices[:, self.layer_index]
        layer_valid = None if path_valid is None else path_valid[:, self.layer_index]
        if pending is None:
            normed = self.norm1(x)
        else:
            x, normed = self.norm1.add_forward(x, pending)
        attended = self.attn(normed, valid_mask, seam_reset, layer_paths, layer_valid)
        x, normed = self.norm2.add_forward(x, attended)
        ff = self.ff(normed)
        if valid_mask is not None:
            ff = ff * valid_mask[:, :, None].to(x.dtype)
        return x, ff


class BiAttnLM(nn.Module):
    """Character LM backbone (``BiAttn/model.py:338-502``), SBDA layers only."""

    def __init__(self, config: BiAttnConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self.embedding = nn.Embedding(config.vocab_size, config.dim)
        self.drop = nn.Dropout(config.dropout)
        self.layers = nn.ModuleList(BiAttnBlock(config, i) for i in range(config.layers))
        self.norm = RMSNorm(config.dim)
        self.lm_head = nn.Linear(config.dim, config.vocab_size, bias=False)
        if config.tie_embeddings:
            self.lm_head.weight = self.embedding.weight
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        elif isinstance(module, RMSNorm):
            nn.init.ones_(module.weight)

    def forward_hidden(self, input_ids: Tensor, valid_mask: Optional[Tensor] = None,
                       seam_reset: Optional[Tensor] = None,
                       path_indices: Optional[Tensor] = None,
                       path_valid: Optional[Tensor] = None,
                       path_active: Optional[Tensor] = None) -> Tensor:
        """Final hidden states before the vocabulary projection."""
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        if valid_mask is not None and (valid_mask.shape != input_ids.shape
                                       or valid_mask.dtype != torch.bool):
            raise ValueError("valid_mask must be bool with input_ids shape")
        if seam_reset is not None and (seam_reset.shape != input_ids.shape
                                       or seam_reset.dtype != torch.bool):
            raise ValueError("seam_reset must be bool with input_ids shape")
        if path_indices is not None and (
                path_indices.ndim != 4 or path_indices.shape[0] != input_ids.shape[0]
                or path_indices.shape[2] != input_ids.shape[1]
                or path_indices.dtype != torch.long):
            raise ValueError("path_indices must have shape [batch, layers, sequence, source_count]")
        if path_valid is not None and (path_indices is None
                                       or path_valid.shape != path_indices.shape
                                       or path_valid.dtype != torch.bool):
            raise ValueError("path_valid must match path_indices as a bool tensor")
        if path_active is not None and (path_indices is None or path_active.ndim != 2
                                        or path_active.shape != path_indices.shape[:2]
                                        or path_active.dtype != torch.bool
                                        or path_active.device != input_ids.device):
            raise ValueError("path_active must have shape [batch, layers] and match path_indices")
        if path_indices is not None and path_indices.shape[1] != len(self.layers):
            raise ValueError("path_indices layer count must match the model")
        # An all-true mask is dropped once here (model.py:439-440).
        if valid_mask is not None and bool(valid_mask.all()):
            valid_mask = None
        x = self.drop(self.embedding(input_ids))
        if path_active is None:
            pending = None
            for layer in self.layers:
                x, pending = layer.forward_pending(x, pending, valid_mask, seam_reset,
                                                   path_indices, path_valid)
            return self.norm.add_forward(x, pending)[1]
        for index, layer in enumerate(self.layers):
            # Rows whose layer is inactive pass through unchanged (model.py:446-466).
            active = path_active[:, index]
            if not bool(active.any()):
                continue
            if bool(active.all()):
                x = layer(x, valid_mask, seam_reset, path_indices, path_valid)
                continue
            rows = active.nonzero(as_tuple=False).flatten()

            def pick(t):
                return None if t is None else t.index_select(0, rows)

            updated = layer(x.index_select(0, rows), pick(valid_mask), pick(seam_reset),
                            pick(path_indices), pick(path_valid))
            x = x.clone()
            x.index_copy_(0, rows, updated)
        return self.norm(x)

    def forward(self, input_ids: Tensor, valid_mask: Optional[Tensor] = None,
                seam_reset: Optional[Tensor] = None, path_indices: Optional[Tensor] = None,
                path_valid: Optional[Tensor] = None,
                path_active: Optional[Tensor] = None) -> Tensor:
        return self.lm_head(self.forward_hidden(input_ids, valid_mask, seam_reset,
                                                path_indices, path_valid, path_active))

    def next_logits(self, input_ids: Tensor, valid_mask: Tensor) -> Tensor:
        """One logit vector per row, at its last valid token."""
        hidden = self.forward_hidden(input_ids, valid_mask)
        lengths = valid_mask.sum(dim=1) - 1
        rows = torch.arange(input_ids.shape[0], device=input_ids.device)
        return self.lm_head(hidden[rows, lengths])

    def triangle_loss(self, input_ids: Tensor, valid_mask: Tensor, targets: Tensor) -> Tensor:
        if targets.ndim != 1 or targets.shape[0] != input_ids.shape[0]:
            raise ValueError("targets must contain one next token per triangle row")
        return F.cross_entropy(self.next_logits(input_ids, valid_mask), targets)


__all__ = ["BiAttnBlock", "BiAttnConfig", "BiAttnLM", "RMSNorm", "SwiGLU"]
