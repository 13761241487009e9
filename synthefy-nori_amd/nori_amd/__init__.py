"""nori_amd: MI355X-native kernels for Nori's in-context-learning (ICL) hot path.

Drop-in operators for the reference's context-cache path (Synthefy/synthefy-nori):
the int8 K/V cache codec and cache containers (``kv_cache_scaling``), query-row ->
context attention over the cached K/V (``attention``) and RMSNorm (``norm``), all
computed by hand-written gfx950 kernels in libnori_hip.so, and the per-layer cache build
and cached apply built on them (``layer``).
"""

from . import _native, layer
from .attention import attend_dense, compute_attention_blockwise, icl_attention
from .kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV, dequantize_int8, quantize_int8, scale_caches
from .norm import RMSNorm, rms_norm

__all__ = [
    "BlockwiseSeqKV",
    "layer",
    "RMSNorm",
    "ScalableSeqKV",
    "attend_dense",
    "compute_attention_blockwise",
    "dequantize_int8",
    "icl_attention",
    "quantize_int8",
    "rms_norm",
    "scale_caches",
]
