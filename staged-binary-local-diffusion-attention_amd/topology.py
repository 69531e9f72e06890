"""Per-layer source offsets (pure Python), as the reference schedules them.

``topology_offsets(layer, topology=..., total_layers=...)`` returns the
ordered leftward offsets a layer reads; ``0`` is the self source.  The
rules are fixed by ``BiAttn/topology.py:3-155`` of the reference and must
agree with it exactly, because the offsets decide which positions the
kernels gather.  The fused kernels accept any route with two or four
offsets; ``sbda`` (``:65-66``) is the one this library is tuned for.
"""

from __future__ import annotations

PATH_TOPOLOGIES = (
    "binary", "local_jump", "mesh", "torus", "butterfly", "high4",
    "radix4", "radix8", "mixed_local_radix4", "longformer_local",
    "sparse_local_stride", "dinat_like", "longnet_like", "power_attention",
    "h0", "h1", "h2", "h3", "h4_greedy", "h5", "h6", "h7", "h8",
    "h8a", "h8b", "h8c", "h8d", "h8e", "h8f", "h8g", "sbda",
)


def sbda_stage(layer: int) -> str:
    """``"binary"`` for layers 1-2, ``"local_diffusion"`` after (``topology.py:13-17``)."""
    if layer < 1:
        raise ValueError("layer must be positive")
    return "binary" if layer <= 2 else "local_diffusion"


def _dedup(*offsets: int) -> tuple[int, ...]:
    """Drop negatives and repeats, keeping first occurrences (``topology.py:20-21``)."""
    out: list[int] = []
    for off in offsets:
        off = int(off)
        if off >= 0 and off not in out:
            out.append(off)
    return tuple(out)


def _radix(radix: int, stride: int) -> tuple[int, ...]:
    return tuple(q * stride for q in range(radix))


def topology_offsets(layer: int, *, topology: str = "binary",
                     total_layers: int = 12) -> tuple[int, ...]:
    """Ordered offsets of ``layer`` (1-based) for ``topology``.

    Mirrors ``BiAttn/topology.py:24-155``: the same validation
    (``ValueError`` for ``layer < 1``, ``total_layers < 1`` or an unknown
    name) and the same offsets, in the same slot order.
    """
    if layer < 1:
        raise ValueError("layer must be positive")
    if total_layers < 1:
        raise ValueError("total_layers must be positive")
    if topology not in PATH_TOPOLOGIES:
        raise ValueError(f"unknown path topology: {topology}")
    level = layer - 1
    s = 1 << level
    early = layer <= 2
    table = {
        "h0": lambda: (0, s),
        "h1": lambda: _dedup(0, 1, 2, s),
        "h2": lambda: _dedup(0, s, 3 * s),
        "h3": lambda: _dedup(0, *range(s, 2 * s)),
        "h4_greedy": lambda: _dedup(0, 3 ** level, 2 * 3 ** level),
        "h5": lambda: (0, 1, 2) if layer == 1 else (0, 2 ** layer),
        "h6": lambda: _dedup(0, s, 2 * s + 1),
        "h7": lambda: (0, 1, 2) if early else (0, s),
        "h8": lambda: (0, s) if early else _dedup(0, 1, 2, s),
        "sbda": lambda: (0, s) if early else _dedup(0, 1, 2, s),
        "h8a": lambda: (0, s) if early else _dedup(0, 1, s),
        "h8b": lambda: (0, s) if early else _dedup(0, 2, s),
        "h8c": lambda: (0, s) if early else _dedup(0, 1, 2, s),
        "h8d": lambda: (0, 1, 2, s) if layer >= 3 and layer % 2 == 1 else (0, s),
        "h8e": lambda: _dedup(0, 1, 2, s) if layer > max(2, total_layers - 2) else (0, s),
        "h8f": lambda: (0, s) if early else _dedup(0, 1, 2, 3, s),
        "h8g": lambda: (0, s) if early else _dedup(0, 1, 2, 3, 4, s),
        "binary": lambda: (0, s),
        "local_jump": lambda: _dedup(0, 1, 2, s),
        "mesh": lambda: _dedup(0, 1, s, s + 1),
        "torus": lambda: _dedup(0, 1, max(1, s - 1), s, s + 1),
        "butterfly": lambda: _dedup(0, s, 2 * s, 3 * s),
        "high4": lambda: _dedup(0, 1, 2, s, 2 * s, 3 * s),
        "longformer_local": lambda: (0, 1, 2, 3),
        "sparse_local_stride": lambda: _dedup(
            0, 1, 2, 3, max(4, 2 ** max(1, total_layers // 2))),
        "dinat_like": lambda: _dedup(0, 1, 2, 3, 2 * s, 4 * s, 6 * s),
        "longnet_like": lambda: _dedup(0, 1, 2, 3, s, 2 * s, 3 * s),
        "power_attention": lambda: _dedup(
            0, 1, 2, 3, *(1 << e for e in range(total_layers))),
        "radix4": lambda: _radix(4, 4 ** level),
        "radix8": lambda: _radix(8, 8 ** level),
    }
    rule = table.get(topology)
    if rule is not None:
        return rule()
    # mixed_local_radix4: binary steps for the first half of the stack, then
    # radix-4 steps whose stride continues from 2**split.
    split = max(1, total_layers // 2)
    if level < split:
        return (0, s)
    return _radix(4, (2 ** split) * (4 ** (level - split)))


__all__ = ["PATH_TOPOLOGIES", "sbda_stage", "topology_offsets"]
