"""Warnings for a prediction that got less than the configured pipeline promised.

The reference raises one warning category per kind of silent degradation, all under one base
class (src/synthefy_nori/inference/degradation.py:45-80), so a caller can escalate every kind,
or one, to an error with ``strict_pipeline`` (degradation.py:85-101) instead of threading a flag
through the predictor. The same tree here: ``DegradedPipelineWarning`` (a ``UserWarning``), with
``SvdFallbackWarning`` (the wide-table SVD failed and was worked around) and
``CacheQuantizedWarning`` (the context K/V cache was stored int8) below it.
"""

from __future__ import annotations

import contextlib
import warnings

__all__ = ["CacheQuantizedWarning", "DegradedPipelineWarning", "SvdFallbackWarning", "strict_pipeline"]


class DegradedPipelineWarning(UserWarning):
    """The model was handed less than the configured pipeline promised (degradation.py:45-53)."""


class SvdFallbackWarning(DegradedPipelineWarning):
    """The wide-table SVD failed: a fit failure passes the raw columns through, a transform
    failure leaves ``svd_all`` one all-zero column and ``svd_binary`` its non-binary columns
    (degradation.py:55-62, raised at preprocess.py:1481-1504)."""


class CacheQuantizedWarning(DegradedPipelineWarning):
    """The context K/V cache was stored int8 (degradation.py:73-80, raised at predictor.py:3286-3305)."""


@contextlib.contextmanager
def strict_pipeline(*categories: type[Warning]):
    """Inside the block, the given degradation categories (default: all of them) raise instead of
    warning; the caller's warning filters are restored on exit."""
    with warnings.catch_warnings():
        for category in categories or (DegradedPipelineWarning,):
            warnings.simplefilter("error", category)
        yield
