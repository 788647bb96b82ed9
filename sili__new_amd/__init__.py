"""sili__new_amd -- MI355X (gfx950) FP4 delta-CSR sparse linear layer.

Drop-in for sili's `sili._cpu.SparseLinearLayer` hot path
(SimLeek/sili__new sili/cpu_backend.cpp:349-984): same constructor, method
names, argument meaning and exception types, with every compute call running
in hand-written HIP kernels behind the C ABI in include/sili_hip.h.

There is no CPU fallback: importing this package fails loudly when the HIP
extension has not been built (python -m sili__new_amd.build).
"""
from __future__ import annotations

import os

_HERE = os.path.dirname(os.path.abspath(__file__))

try:
    from . import _sili_hip as _ext  # noqa: F401
except ImportError as e:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "sili__new_amd: the HIP extension is not built; run `python -m sili__new_amd.build` "
        f"(looked in {_HERE}): {e}") from e

SparseLinearLayer = _ext.SparseLinearLayer
SparseLinearLayerDeterministic = _ext.SparseLinearLayerDeterministic
SparseLinearLayerResync = _ext.SparseLinearLayerResync
SparseLinearLayerResyncDeterministic = _ext.SparseLinearLayerResyncDeterministic
SparseLinearLayerNoScale = _ext.SparseLinearLayerNoScale
SparseLinearLayerNoScaleDeterministic = _ext.SparseLinearLayerNoScaleDeterministic
fp4_quantize_array = _ext.fp4_quantize_array
dense_to_csr = _ext.dense_to_csr
dense_to_top_k_csr = _ext.dense_to_top_k_csr
seed_fp4_stochastic_rng = _ext.seed_fp4_stochastic_rng

LIB_PATH = os.path.join(_HERE, "libsili_hip.so")

__all__ = ["SparseLinearLayer", "SparseLinearLayerDeterministic", "SparseLinearLayerResync",
           "SparseLinearLayerResyncDeterministic", "SparseLinearLayerNoScale", "SparseLinearLayerNoScaleDeterministic",
           "fp4_quantize_array", "dense_to_csr", "dense_to_top_k_csr", "seed_fp4_stochastic_rng", "LIB_PATH"]
