"""MI355X-native SISA hot path: HIP (gfx950) kernels for the fused prep, the exact attention forward/backward and
the chunked linear cross-entropy, behind the Python API of the reference package ``sisa`` (tlstngud/sisa 0.1.0).

Main entry points (same names as the reference):

* :func:`sisa_attention` - the attention function on prepared tensors (``impl="auto" | "torch" | "hip"``).
* :class:`SISAAttention` - the attention sublayer (``attn_impl="auto" | "torch" | "hip" | "hip_fused"``).
* :class:`SISAForCausalLM` - the language model (blocks of SISA attention and SwiGLU, tied LM head, fused CE,
  ``generate``, ``save_pretrained`` / ``from_pretrained``); :func:`load_paper_checkpoint`.
* :mod:`sisa_amd.kernels` - ``sisa_attention_hip``, ``sisa_fused``, ``fused_layout``, ``concat_fused_weights``,
  ``linear_cross_entropy``.
* :mod:`sisa_amd.backends` - HIP availability, backend selection and the runtime check mode.
"""
from __future__ import annotations

import importlib
from typing import Any

from .config import ATTN_IMPLS, PRESETS, SISAConfig
from .functional import rotate_pairs, sisa_attention, sisa_attention_torch
from .generation import SISACache, generate
from .modeling import RMSNorm, SISAAttention, SISABlock, SISAForCausalLM, SISAModel, SISAOutput, SwiGLU

__version__ = "0.1.0"

__all__ = ["SISAConfig", "PRESETS", "ATTN_IMPLS", "SISAAttention", "SISABlock", "SISAModel", "SISAForCausalLM",
           "SISAOutput", "RMSNorm", "SwiGLU", "SISACache", "generate", "sisa_attention", "sisa_attention_torch",
           "rotate_pairs", "set_check_mode", "load_paper_checkpoint", "__version__"]


def load_paper_checkpoint(path, **kwargs):
    """Load a paper training checkpoint; see :func:`sisa_amd.checkpoint.load_paper_checkpoint`."""
    from .checkpoint import load_paper_checkpoint as _load

    return _load(path, **kwargs)


def set_check_mode(mode: str) -> None:
    """Set how the HIP kernels check their inputs: ``"async"`` (default), ``"sync"`` or ``"off"``."""
    from .backends import set_check_mode as _set

    _set(mode)


_LAZY_SUBMODULES = ("backends", "kernels", "checkpoint")


def __getattr__(name: str) -> Any:
    if name in _LAZY_SUBMODULES:
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
