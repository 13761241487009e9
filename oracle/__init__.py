"""CPU oracle for the Nori ICL hot path -- TEST INFRASTRUCTURE ONLY.

A restatement of the reference's algorithms (Synthefy/synthefy-nori,
src/synthefy_nori/model/kv_cache_scaling.py and model/layer.py) that the HIP kernels
are checked against. Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it; the product package (synthefy-nori_amd/nori_amd)
never does, and has no CPU fallback that could route through it.

* ``oracle.codec``      int8 quantize/dequantize with per-op dtype rounding, RMSNorm (C)
* ``oracle.attention``  float64 attention, fp32 online-softmax block scan, LSE merge
"""
