"""nori_amd: MI355X-native kernels for Nori's in-context-learning (ICL) hot path.

Drop-in operators for the reference's context-cache path (Synthefy/synthefy-nori):
the int8 K/V cache codec and cache containers (``kv_cache_scaling``), query-row ->
context attention over the cached K/V (``attention``), RMSNorm (``norm``) and the
fused (RMSNorm ->) K/V projection -> int8 cache write (``kv_project``), all
computed by hand-written gfx950 kernels in libnori_hip.so, the per-layer cache build
and cached apply built on them (``layer``), and the context-cache API around the layer
stack -- ``FeaturesTransformer.build_context_cache`` / ``apply_context_cache`` with the
input encoders (``transformer``, ``encoders``).
"""

from . import _native, encoders, layer, transformer
from .attention import attend_dense, compute_attention_blockwise, icl_attention
from .kv_cache_scaling import BlockwiseSeqKV, ScalableSeqKV, dequantize_int8, quantize_int8, scale_caches
from .kv_project import project_quantize_kv
from .api import NoriRegressor
from .degradation import CacheQuantizedWarning, DegradedPipelineWarning, SvdFallbackWarning, strict_pipeline
from .norm import RMSNorm, rms_norm
from .transformer import ContextCache, FeaturesTransformer

__all__ = [
    "BlockwiseSeqKV",
    "CacheQuantizedWarning",
    "DegradedPipelineWarning",
    "SvdFallbackWarning",
    "strict_pipeline",
    "ContextCache",
    "FeaturesTransformer",
    "NoriRegressor",
    "encoders",
    "layer",
    "RMSNorm",
    "ScalableSeqKV",
    "attend_dense",
    "compute_attention_blockwise",
    "dequantize_int8",
    "icl_attention",
    "project_quantize_kv",
    "quantize_int8",
    "rms_norm",
    "scale_caches",
    "transformer",
]
