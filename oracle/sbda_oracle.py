"""CPU restatement of the reference's exact SBDA attention path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the product package
never imports this module.

What is restated, and from where (paths relative to the reference checkout):

* ``sbda_layer_offsets``      -- ``BiAttn/topology.py:13-21,37-38,65-66``
* ``path_tables``             -- ``BiAttn/left_v2.py:165-189``
* ``head_rmsnorm``            -- ``BiAttn/attention_common.py:64-76``
* ``rope_tables`` / ``rotate_half`` / ``apply_rope`` -- ``BiAttn/attention_common.py:8-50``
* ``gather_attention``        -- ``BiAttn/left_v2.py:313-405`` (both the
  matmul route ``use_sdpa=True`` and the elementwise route)
* ``attention_lse``           -- the log-normaliser of the softmax in
  ``left_v2.py:385-392`` (the fused path saves it per row)
* ``brute_force_attention`` / ``brute_force_sources`` -- the paper's formula
  (``paper_en.md:44-81``) as scalar loops, for tiny fp64 cases
* ``key_gather_backward``     -- the key-centric closed form of the backward
  that ``BiAttn/sbda_triton.py:507-671`` specifies (dQ from weights, dK/dV
  gathered per key, no scatter)
* ``prologue``                -- ``left_v2.py:237-239`` (head-RMSNorm of q
  and k, then half-split RoPE)
* ``masked_source_valid`` / ``gather_attention_masked`` -- the eager route's
  ``valid_mask`` / ``seam_reset`` masking (``left_v2.py:329-378``)
* ``table_source_valid`` / ``gather_attention_tables`` -- the same route over
  caller-supplied ``path_indices`` / ``path_valid`` (``left_v2.py:313-378``)
* ``valid_cell_count`` / ``unique_cell_count`` -- the cell statistics of
  ``BinaryDiffusionAttention/run_graph_coverage.py:47-89``

Tensors follow the reference's attention layout: q is ``[B, H, T, D]``, k and
v are ``[B, Hkv, T, D]`` with ``H % Hkv == 0`` (query head h reads kv head
``h // (H // Hkv)``, which is ``_repeat_kv`` at
``attention_common.py:53-61``).  ``offsets`` is a sequence of ints.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch
from torch import Tensor

NO_SOURCE_LSE = math.inf
"""Log-normaliser stored for a row with no valid source (its output is 0)."""


# --------------------------------------------------------------------------
# Source schedule and source tables (integer work; must match bit-exactly)
# --------------------------------------------------------------------------

def sbda_layer_offsets(layer: int) -> tuple[int, ...]:
    """Offsets of SBDA layer ``layer`` (1-based), in slot order.

    ``topology.py:65-66``: ``(0, 2**(layer-1))`` for layers 1-2 and the
    de-duplicated ``(0, 1, 2, 2**(layer-1))`` from layer 3 on
    (``_unique_offsets`` at ``:20-21`` keeps first occurrences, drops
    negatives).  ``layer < 1`` raises ``ValueError`` (``:37-38``).
    """
    if layer < 1:
        raise ValueError("layer must be positive")
    jump = 1 << (layer - 1)
    if layer <= 2:
        return (0, jump)
    seen: list[int] = []
    for off in (0, 1, 2, jump):
        if off >= 0 and off not in seen:
            seen.append(off)
    return tuple(seen)


def sbda_stage(layer: int) -> str:
    """``topology.py:13-17``."""
    if layer < 1:
        raise ValueError("layer must be positive")
    return "binary" if layer <= 2 else "local_diffusion"


def path_tables(length: int, offsets: Sequence[int]) -> tuple[Tensor, Tensor]:
    """``(indices, valid)`` of ``left_v2.py:172-182``.

    ``indices[i, t] = max(i - offsets[t], 0)`` as int64 and
    ``valid[i, t] = i >= offsets[t]`` as bool, both ``[length, S]``.
    """
    pos = torch.arange(length, dtype=torch.int64)
    off = torch.tensor(list(offsets), dtype=torch.int64)
    diff = pos[:, None] - off[None, :]
    return diff.clamp_min(0), diff >= 0


def valid_cell_count(length: int, offsets_by_layer: Sequence[Sequence[int]]) -> int:
    """Total (query, source) cells over layers (``run_graph_coverage.py:77-85``)."""
    total = 0
    for offsets in offsets_by_layer:
        cells = {(i, i - o) for i in range(length) for o in offsets if o <= i}
        total += len(cells)
    return total


def unique_cell_count(length: int, offsets_by_layer: Sequence[Sequence[int]]) -> int:
    """Distinct (query, source) cells over layers (``run_graph_coverage.py:86``)."""
    cells: set[tuple[int, int]] = set()
    for offsets in offsets_by_layer:
        cells.update((i, i - o) for i in range(length) for o in offsets if o <= i)
    return len(cells)


def sbda_edge_count_closed_form(length: int, layers: int) -> int:
    """``E = (4L - 5) N - 3L + 7`` valid edges per head for ``N = 2**L``
    (``paper_en.md:125``).  Only defined for ``length == 2**layers``."""
    if length != 1 << layers:
        raise ValueError("closed form holds for N = 2**L")
    return (4 * layers - 5) * length - 3 * layers + 7


# --------------------------------------------------------------------------
# Prologue: per-head RMSNorm and half-split RoPE
# --------------------------------------------------------------------------

def head_rmsnorm(x: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """``attention_common.py:67-76``: fp32 normalisation over the last dim,
    times the weight, cast back to ``x.dtype``.  fp64 inputs stay fp64 (an
    extension used only for gradchecks; every other dtype computes in fp32
    exactly as the reference's ``x.float()``)."""
    xf = x.double() if x.dtype == torch.float64 else x.float()
    inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv * weight).to(dtype=x.dtype)


def rope_inverse_frequencies(head_dim: int, theta: float) -> Tensor:
    """``theta ** (-arange(0, D, 2) / D)`` in fp32 (``attention_common.py:16-17``)."""
    idx = torch.arange(0, head_dim, 2, dtype=torch.float32)
    return theta ** (-idx / head_dim)


def rope_tables(length: int, head_dim: int, theta: float,
                dtype: torch.dtype, positions: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``cos, sin`` of shape ``[length, head_dim]`` (``attention_common.py:13-22``).

    Angles are the fp32 product ``position * inverse_frequency``; each half
    of the last dim repeats the same ``D/2`` angles; the tables are cast to
    the activation dtype.  Positions are ``0 .. length-1`` unless given
    (the reference's ``q_positions`` / ``k_positions``, ``:31-46``).
    """
    inv = rope_inverse_frequencies(head_dim, theta)
    pos = torch.arange(length) if positions is None else positions
    ang = torch.outer(pos.to(torch.float32), inv)
    cos = torch.cat((ang.cos(), ang.cos()), dim=-1).to(dtype)
    sin = torch.cat((ang.sin(), ang.sin()), dim=-1).to(dtype)
    return cos, sin


def rotate_half(x: Tensor) -> Tensor:
    """``cat(-x2, x1)`` over the last dim (``attention_common.py:8-10``)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: Tensor, theta: float, positions: Tensor | None = None) -> Tensor:
    """Half-split RoPE of ``x`` laid out ``[B, T, H, D]`` (``attention_common.py:25-50``).

    ``x * cos + rotate_half(x) * sin`` (``:48-49``): each pair
    ``(x[d], x[d + D/2])`` at position m is rotated by ``+m * inv_freq[d]``;
    odd ``D`` is the identity (``:36-40``).  ``positions`` (``[T]``) are the
    positions of the T rows, ``0 .. T-1`` by default (``:41-44``).
    """
    d = x.shape[-1]
    if d % 2:
        return x
    cos, sin = rope_tables(x.shape[1], d, theta, x.dtype, positions)
    cos = cos[None, :, None, :]
    sin = sin[None, :, None, :]
    return x * cos + rotate_half(x) * sin


def prologue(q_raw: Tensor, k_raw: Tensor, q_weight: Tensor, k_weight: Tensor,
             theta: float, eps: float = 1e-6,
             positions: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``left_v2.py:237-239`` on ``[B, T, H, D]`` inputs: norm, then RoPE
    (rows at ``positions``, ``0 .. T-1`` by default)."""
    qn = head_rmsnorm(q_raw, q_weight, eps)
    kn = head_rmsnorm(k_raw, k_weight, eps)
    return apply_rope(qn, theta, positions), apply_rope(kn, theta, positions)


# --------------------------------------------------------------------------
# Attention (the eager gather path) and its log-normaliser
# --------------------------------------------------------------------------

def _expand_kv(x: Tensor, heads: int) -> Tensor:
    """``[B, Hkv, T, D]`` -> ``[B, H, T, D]``, head h reading ``h // group``."""
    group = heads // x.shape[1]
    if group == 1:
        return x
    return x.repeat_interleave(group, dim=1)


def _gathered(q: Tensor, k: Tensor, v: Tensor, offsets: Sequence[int]):
    b, h, t, d = q.shape
    k = _expand_kv(k, h)
    v = _expand_kv(v, h)
    idx, valid = path_tables(t, offsets)
    s = idx.shape[1]
    src = idx[None, None, :, :, None].expand(b, h, t, s, d)
    kg = k.unsqueeze(3).expand(b, h, t, s, d).gather(2, src)
    vg = v.unsqueeze(3).expand(b, h, t, s, d).gather(2, src)
    return kg, vg, valid


def gather_attention(q: Tensor, k: Tensor, v: Tensor, offsets: Sequence[int], *,
                     matmul_route: bool = True) -> Tensor:
    """Eager SBDA attention, ``[B, H, T, D]`` in and out (``left_v2.py:313-405``).

    Scores ``(q . k_src) * D**-0.5``; invalid sources get ``finfo.min`` before
    the softmax and weight 0 after it; output ``sum_t w_t v_src``.  Autograd
    through this function is the reference backward.
    """
    d = q.shape[-1]
    kg, vg, valid = _gathered(q, k, v, offsets)
    invalid = ~valid[None, None]
    if matmul_route:
        scores = torch.matmul(q.unsqueeze(-2), kg.transpose(-1, -2)).squeeze(-2)
    else:
        scores = (q.unsqueeze(3) * kg).sum(dim=-1)
    scores = scores * (d ** -0.5)
    scores = scores.masked_fill(invalid, torch.finfo(scores.dtype).min)
    weights = scores.softmax(dim=-1).masked_fill(invalid, 0.0)
    if matmul_route:
        return torch.matmul(weights.unsqueeze(-2), vg).squeeze(-2)
    return (weights.unsqueeze(-1) * vg).sum(dim=3)


def attention_lse(q: Tensor, k: Tensor, offsets: Sequence[int]) -> Tensor:
    """Per-row ``log(sum_valid exp(score))``, ``[B, H, T]``; ``+inf`` where a
    row has no valid source."""
    d = q.shape[-1]
    kg, _, valid = _gathered(q, k, k, offsets)
    scores = (q.unsqueeze(3) * kg).sum(dim=-1) * (d ** -0.5)
    scores = scores.masked_fill(~valid[None, None], -math.inf)
    lse = torch.logsumexp(scores, dim=-1)
    return torch.where(valid.any(dim=-1)[None, None], lse,
                       torch.full_like(lse, NO_SOURCE_LSE))


def brute_force_attention(q: Tensor, k: Tensor, v: Tensor,
                          offsets: Sequence[int]) -> tuple[Tensor, Tensor]:
    """Scalar-loop fp64 evaluation of ``paper_en.md:73-81``; tiny inputs only."""
    b_, h_, t_, d_ = q.shape
    group = h_ // k.shape[1]
    qd, kd, vd = (x.double().tolist() for x in (q, k, v))
    out = torch.zeros(b_, h_, t_, d_, dtype=torch.float64)
    lse = torch.full((b_, h_, t_), NO_SOURCE_LSE, dtype=torch.float64)
    scale = 1.0 / math.sqrt(d_)
    for b in range(b_):
        for h in range(h_):
            hk = h // group
            for i in range(t_):
                srcs = [i - o for o in offsets if o <= i]
                if not srcs:
                    continue
                sc = [scale * sum(qd[b][h][i][e] * kd[b][hk][j][e] for e in range(d_))
                      for j in srcs]
                m = max(sc)
                ex = [math.exp(s - m) for s in sc]
                z = sum(ex)
                lse[b, h, i] = m + math.log(z)
                for e in range(d_):
                    out[b, h, i, e] = sum(w * vd[b][hk][j][e] for w, j in zip(ex, srcs)) / z
    return out, lse


def brute_force_sources(q: Tensor, k: Tensor, v: Tensor,
                        sources: Sequence[Sequence[Sequence[int]]]) -> Tensor:
    """Scalar-loop fp64 softmax attention where query ``i`` of batch ``b`` reads
    the positions ``sources[b][i]`` (repeats count repeatedly; an empty list
    gives a zero row).  Tiny inputs only."""
    b_, h_, t_, d_ = q.shape
    group = h_ // k.shape[1]
    qd, kd, vd = (x.double().tolist() for x in (q, k, v))
    out = torch.zeros(b_, h_, t_, d_, dtype=torch.float64)
    scale = 1.0 / math.sqrt(d_)
    for b in range(b_):
        for h in range(h_):
            hk = h // group
            for i in range(t_):
                srcs = list(sources[b][i])
                if not srcs:
                    continue
                sc = [scale * sum(qd[b][h][i][e] * kd[b][hk][j][e] for e in range(d_))
                      for j in srcs]
                m = max(sc)
                ex = [math.exp(x - m) for x in sc]
                z = sum(ex)
                for e in range(d_):
                    out[b, h, i, e] = sum(w * vd[b][hk][j][e] for w, j in zip(ex, srcs)) / z
    return out


def key_gather_backward(q: Tensor, k: Tensor, v: Tensor, dout: Tensor,
                        offsets: Sequence[int]) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients in the key-centric (gather) form, each row written once.

    Per query i and slot s with source ``j = i - o_s`` (valid iff ``j >= 0``):
    ``p`` = softmax weights, ``dP = dO_i . v_j``, ``delta_i = sum_s p dP``,
    ``dS = p (dP - delta_i)``, ``dQ_i = scale sum_s dS k_j``.
    Per key j and slot t with query ``i = j + o_t`` (valid iff ``i < T``):
    ``dK_j = scale sum_t dS_t(i) q_i`` and ``dV_j = sum_t p_t(i) dO_i``
    (summed over the query heads that share kv head j's head).
    """
    b_, h_, t_, d_ = q.shape
    hkv = k.shape[1]
    group = h_ // hkv
    scale = d_ ** -0.5
    kg, vg, valid = _gathered(q, k, v, offsets)
    vmask = valid[None, None].to(q.dtype)
    scores = (q.unsqueeze(3) * kg).sum(-1) * scale
    lse = attention_lse(q, k, offsets)
    finite = torch.isfinite(lse)
    p = torch.where(finite[..., None], torch.exp(scores - lse.nan_to_num(0.0, posinf=0.0)[..., None]),
                    torch.zeros_like(scores)) * vmask
    dp = (dout.unsqueeze(3) * vg).sum(-1) * vmask
    delta = (p * dp).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    dq = scale * (ds.unsqueeze(-1) * kg).sum(3)
    dk_full = torch.zeros(b_, h_, t_, d_, dtype=q.dtype)
    dv_full = torch.zeros(b_, h_, t_, d_, dtype=q.dtype)
    for slot, off in enumerate(offsets):
        if off >= t_:
            continue
        # key j gathers from query j + off (all such queries are in range
        # for j < T - off; slot validity j >= 0 always holds).
        n = t_ - off
        dk_full[:, :, :n] += scale * ds[:, :, off:, slot, None] * q[:, :, off:]
        dv_full[:, :, :n] += p[:, :, off:, slot, None] * dout[:, :, off:]
    dk = dk_full.view(b_, hkv, group, t_, d_).sum(2)
    dv = dv_full.view(b_, hkv, group, t_, d_).sum(2)
    return dq, dk, dv


# --------------------------------------------------------------------------
# Masked variants: valid_mask with holes and seam_reset segments
# --------------------------------------------------------------------------

def masked_source_valid(length: int, offsets: Sequence[int], valid_mask: Tensor | None,
                        seam_reset: Tensor | None) -> tuple[Tensor, Tensor]:
    """``(indices [T,S], source_valid [B,T,S])`` of ``left_v2.py:329-378``.

    A source is valid when it is in range, (with ``valid_mask``) is itself a
    valid position, and (with ``seam_reset``) lies in the query's segment,
    segments being ``cumsum(seam_reset)``.  With ``valid_mask``, slot 0 of a
    padded query row is forced valid (``:371``) so its softmax is finite.
    """
    idx, base = path_tables(length, offsets)
    batch = (valid_mask if valid_mask is not None else seam_reset).shape[0]
    s = idx.shape[1]
    ib = idx.unsqueeze(0).expand(batch, -1, -1)
    valid = base.unsqueeze(0).expand(batch, -1, -1).clone()
    if valid_mask is not None:
        valid &= valid_mask.unsqueeze(-1).expand(-1, -1, s).gather(1, ib)
        if seam_reset is not None:
            seg = seam_reset.to(torch.int64).cumsum(dim=1)
            valid &= seg.unsqueeze(-1).expand(-1, -1, s).gather(1, ib) == seg[:, :, None]
        valid[:, :, 0] |= ~valid_mask
    elif seam_reset is not None:
        seg = seam_reset.to(torch.int64).cumsum(dim=1)
        valid &= seg.unsqueeze(-1).expand(-1, -1, s).gather(1, ib) == seg[:, :, None]
    return idx, valid


def table_source_valid(path_indices: Tensor, path_valid: Tensor | None,
                       valid_mask: Tensor | None, seam_reset: Tensor | None) -> Tensor:
    """``source_valid [B, T, S]`` for caller-supplied tables (``left_v2.py:349-378``):
    ``path_valid`` (all set when absent), causality ``idx <= i`` (``:355-357``),
    then the same ``valid_mask`` / ``seam_reset`` rules as the offset route,
    including slot 0 forced valid for padded query rows (``:371``)."""
    b, t, s = path_indices.shape
    valid = torch.ones(b, t, s, dtype=torch.bool)
    if path_valid is not None:
        valid &= path_valid
    positions = torch.arange(t)
    valid &= path_indices <= positions[None, :, None]
    if valid_mask is not None:
        valid &= valid_mask.unsqueeze(-1).expand(-1, -1, s).gather(1, path_indices)
        if seam_reset is not None:
            seg = seam_reset.to(torch.int64).cumsum(dim=1)
            valid &= seg.unsqueeze(-1).expand(-1, -1, s).gather(1, path_indices) == seg[:, :, None]
        valid[:, :, 0] |= ~valid_mask
    elif seam_reset is not None:
        seg = seam_reset.to(torch.int64).cumsum(dim=1)
        valid &= seg.unsqueeze(-1).expand(-1, -1, s).gather(1, path_indices) == seg[:, :, None]
    return valid


def _table_attention(q: Tensor, k: Tensor, v: Tensor, idx: Tensor, valid: Tensor) -> Tensor:
    """``left_v2.py:333-396`` with per-batch tables ``idx``/``valid [B, T, S]``:
    gather, scaled scores, ``finfo.min`` fill, softmax, zero fill, weighted sum."""
    b, h, t, d = q.shape
    k = _expand_kv(k, h)
    v = _expand_kv(v, h)
    s = idx.shape[-1]
    src = idx[:, None, :, :, None].expand(b, h, t, s, d)
    kg = k.unsqueeze(3).expand(b, h, t, s, d).gather(2, src)
    vg = v.unsqueeze(3).expand(b, h, t, s, d).gather(2, src)
    invalid = ~valid[:, None]
    scores = torch.matmul(q.unsqueeze(-2), kg.transpose(-1, -2)).squeeze(-2) * (d ** -0.5)
    scores = scores.masked_fill(invalid, torch.finfo(scores.dtype).min)
    weights = scores.softmax(dim=-1).masked_fill(invalid, 0.0)
    return torch.matmul(weights.unsqueeze(-2), vg).squeeze(-2)


def gather_attention_masked(q: Tensor, k: Tensor, v: Tensor, offsets: Sequence[int],
                            valid_mask: Tensor | None = None,
                            seam_reset: Tensor | None = None) -> Tensor:
    """Eager attention with the reference's mask semantics (``left_v2.py:313-405``),
    ``[B, H, T, D]`` in and out (before the output projection and the final
    ``valid_mask`` multiply)."""
    if valid_mask is None and seam_reset is None:
        return gather_attention(q, k, v, offsets)
    b, _, t, _ = q.shape
    idx, valid = masked_source_valid(t, offsets, valid_mask, seam_reset)
    return _table_attention(q, k, v, idx.unsqueeze(0).expand(b, -1, -1), valid)


def gather_attention_tables(q: Tensor, k: Tensor, v: Tensor, path_indices: Tensor,
                            path_valid: Tensor | None = None,
                            valid_mask: Tensor | None = None,
                            seam_reset: Tensor | None = None) -> Tensor:
    """Eager attention over caller-supplied source tables (``left_v2.py:313-405``
    with ``path_indices [B, T, S]`` int64 in ``[0, T)`` and ``path_valid``)."""
    valid = table_source_valid(path_indices, path_valid, valid_mask, seam_reset)
    return _table_attention(q, k, v, path_indices, valid)
