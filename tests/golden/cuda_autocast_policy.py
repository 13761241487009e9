"""CUDA's fp16 autocast op policy for CPU runs of the reference (test infrastructure: the golden
recipes run the reference's modules under ``torch.autocast("cpu", dtype=torch.float16)``).

The reference's predictor runs on a GPU under CUDA autocast (predictor.py:3208-3217). torch's
CPU autocast casts the same matrix products to fp16 (linear, matmul, bmm, SDPA, ...) but keeps
a different list of ops that run in fp32: CUDA autocast runs ``layer_norm``, ``exp``, ``log``,
``rsqrt``, ``pow``, ``softplus``, ``logsumexp``, ... in fp32 (fp16 inputs are cast up, the output
is fp32) and ``sum``, ``cumsum``, ``prod``, ``softmax``, ``log_softmax`` with an fp32 result,
where CPU autocast leaves them in their inputs' dtype. For the reference's models that
difference is not small: its encoders end in a ``LayerNorm``, which on the GPU hands the layer
stack an fp32 residual stream and on the CPU an fp16 one, whose rounding then compounds over
the layers.

``cuda_policy()`` is a torch function mode that applies CUDA's fp32 list on top of CPU autocast
(only while CPU autocast is on), so a CPU run computes in the dtypes a GPU run of the same code
computes in; what is left between the two is the order of the sums.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.overrides import TorchFunctionMode
from torch.utils._pytree import tree_map

T = torch.Tensor

# CUDA autocast's "fp32" ops that the reference's model code calls (function and method forms)
FP32 = {
    F.layer_norm, torch.layer_norm, F.group_norm, torch.group_norm,
    torch.exp, T.exp, torch.expm1, T.expm1, torch.log, T.log, torch.log2, T.log2, torch.log10, T.log10,
    torch.log1p, T.log1p, torch.reciprocal, T.reciprocal, torch.rsqrt, T.rsqrt, torch.pow, T.pow, T.__pow__,
    T.__rpow__, F.softplus, torch.logsumexp, T.logsumexp, torch.acos, T.acos, torch.asin, T.asin, torch.cosh, T.cosh,
    torch.sinh, T.sinh, torch.tan, T.tan, torch.erfinv, T.erfinv, F.cosine_similarity, torch.cdist, torch.dist,
    T.dist, torch.renorm, T.renorm,
}
# CUDA autocast's "fp32_set_opt_dtype" ops: run with dtype=float32 unless a dtype is given
FP32_RESULT = {
    torch.sum, T.sum, torch.cumsum, T.cumsum, torch.prod, T.prod, torch.cumprod, T.cumprod,
    torch.softmax, T.softmax, F.softmax, torch.log_softmax, T.log_softmax, F.log_softmax,
}


def _up(x):
    return x.float() if isinstance(x, torch.Tensor) and x.dtype in (torch.float16, torch.bfloat16) else x


def _has_low(args, kwargs) -> bool:
    found = []
    tree_map(lambda x: found.append(1) if isinstance(x, torch.Tensor) and x.dtype in (torch.float16, torch.bfloat16)
             else None, (args, kwargs))
    return bool(found)


class cuda_policy(TorchFunctionMode):
    def __torch_function__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if torch.is_autocast_enabled("cpu") and _has_low(args, kwargs):
            if func in FP32:
                with torch.autocast("cpu", enabled=False):
                    return func(*tree_map(_up, args), **tree_map(_up, kwargs))
            if func in FP32_RESULT and kwargs.get("dtype") is None:
                with torch.autocast("cpu", enabled=False):
                    return func(*tree_map(_up, args), **tree_map(_up, kwargs))
        return func(*args, **kwargs)
