"""MI355X-native SBDA attention (fused sparse gather-softmax, HIP for gfx950).

Drop-in for the fused path of Staged Binary-Local Diffusion Attention:
``fused_sbda_key_backward(q, k, v, offsets)`` and its sibling names, the
fused norm+RoPE variant ``fused_sbda_prologue``, the per-layer schedule
``topology_offsets`` and the ``SBDAttention`` module.  All compute runs in
``libsbda_amd.so`` (built by ``build.py``); importing this package does not
load it, the first op call does.
"""

from .sbda import (
    fused_sbda,
    fused_sbda_block,
    fused_sbda_block_full,
    fused_sbda_gqa_key_backward,
    fused_sbda_key_backward,
    fused_sbda_paths,
    fused_sbda_prologue,
    host_offsets,
    rope_inverse_frequencies,
    rope_tables,
    sbda_backward,
    sbda_backward_paths,
    sbda_forward,
    sbda_forward_paths,
    segment_keys,
)
from .block import (fused_add_rms_norm, fused_rms_norm, fused_swiglu, fused_swiglu_gemm,
                    swiglu_gemm_supported)
from .topology import PATH_TOPOLOGIES, sbda_stage, topology_offsets
from .attention import BinaryPathAttention, SBDAAttention, SBDAttention
from .model import BiAttnBlock, BiAttnConfig, BiAttnLM
from ._lib import LIBRARY_PATH, SBDALibraryError

__all__ = [
    "BiAttnBlock", "BiAttnConfig", "BiAttnLM", "BinaryPathAttention", "LIBRARY_PATH",
    "PATH_TOPOLOGIES", "SBDAAttention", "SBDALibraryError", "SBDAttention",
    "fused_add_rms_norm", "fused_rms_norm", "fused_swiglu", "fused_swiglu_gemm", "fused_sbda",
    "fused_sbda_block", "fused_sbda_block_full", "fused_sbda_gqa_key_backward",
    "fused_sbda_key_backward", "fused_sbda_paths", "fused_sbda_prologue", "host_offsets",
    "rope_inverse_frequencies", "rope_tables", "sbda_backward", "sbda_backward_paths",
    "sbda_forward", "sbda_forward_paths",
    "sbda_stage", "segment_keys", "swiglu_gemm_supported", "topology_offsets",
]
