"""HIP kernels of SISA (AMD Instinct MI355X, gfx950), bound through ``libsisa_hip.so``.

Loaded lazily (as the reference's ``sisa.kernels``, src/sisa/kernels/__init__.py:29-50): ``import sisa_amd.kernels``
works without a GPU or a built library; the attributes below are resolved on first access. Check availability with
:func:`sisa_amd.backends.hip_status`.

``sisa_attention_hip(q, k, v, c, b, g, lam, fgate=None) -> o``  (:mod:`sisa_amd.kernels.attention`)
``sisa_fused(proj, z, lam, n_head) -> y``, ``fused_layout``, ``concat_fused_weights``  (:mod:`.fused_prep`)
``linear_cross_entropy(hidden, weight, labels, ignore_index=-100) -> loss``  (:mod:`.linear_ce`)
"""
from __future__ import annotations

import importlib

__all__ = ["sisa_attention_hip", "sisa_fused", "fused_layout", "concat_fused_weights", "linear_cross_entropy",
           "reference_linear_cross_entropy"]

_LAZY = {
    "sisa_attention_hip": "attention",
    "sisa_fused": "fused_prep",
    "fused_layout": "fused_prep",
    "concat_fused_weights": "fused_prep",
    "linear_cross_entropy": "linear_ce",
    "reference_linear_cross_entropy": "linear_ce",
}


def __getattr__(name):
    mod = _LAZY.get(name)
    if mod is None:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    value = getattr(importlib.import_module(f"{__name__}.{mod}"), name)
    globals()[name] = value
    return value


def __dir__():
    return sorted(list(globals()) + list(_LAZY))
