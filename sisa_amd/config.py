"""The SISA model configuration: field set, defaults and presets of the reference (src/sisa/config.py), with the
attention implementation names of this build ("hip", "hip_fused" in place of the Triton ones).

Design: the parameter set of a model is spelled out once, by :meth:`SISAConfig.parameter_shapes` (state-dict name ->
shape). Parameter counts, checkpoint checks and the model's own construction tests all read that one table, so a
config and a state dict can be compared without building a model. Field checks are a table of (predicate, message).
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass
from typing import Any, Callable, Mapping

__all__ = ["SISAConfig", "PRESETS", "ATTN_IMPLS", "HIP_D_HEAD", "HIP_D_STATE"]

#: Values of :attr:`SISAConfig.attn_impl`.
ATTN_IMPLS = ("auto", "torch", "hip", "hip_fused")

#: The head and state sizes the HIP kernels are built for.
HIP_D_HEAD = 64
HIP_D_STATE = 32

_POSITIVE_INTS = ("vocab_size", "d_model", "n_layer", "n_head", "d_ff", "d_state", "max_seq_len", "torch_block_q")


@dataclass
class SISAConfig:
    """Hyper-parameters of a SISA language model; the defaults are the 50M paper model (``PRESETS["sisa-50m"]``).

    ``d_head = d_model // n_head``. The HIP implementations need d_head 64 and d_state 32; ``attn_impl="auto"``
    falls back to the torch path at run time for other shapes. ``d_ff`` is the SwiGLU width as given (no
    parameter-matching rule). ``max_seq_len`` is informational (there is no positional table).
    """

    vocab_size: int = 50277
    d_model: int = 512
    n_layer: int = 6
    n_head: int = 8
    d_ff: int = 1829
    d_state: int = 32
    norm_eps: float = 1e-6
    init_std: float = 0.02
    theta_init_std: float = 0.01
    decay_bias_init: float = -5.0
    forget_bias_init: float = 4.0
    lambda_raw_init: float = -1.0
    zero_init_c: bool = True
    max_seq_len: int = 2048
    attn_impl: str = "auto"
    torch_block_q: int = 256
    gradient_checkpointing: bool = False

    def __post_init__(self) -> None:
        for name in _POSITIVE_INTS:
            v = getattr(self, name)
            if type(v) is not int or v <= 0:
                raise ValueError(f"SISAConfig.{name} = {v!r}: expected a positive integer")
        checks: tuple[tuple[Callable[[], bool], str], ...] = (
            (lambda: self.d_model % self.n_head == 0,
             f"d_model {self.d_model} is not divisible by n_head {self.n_head}"),
            (lambda: self.d_state % 2 == 0,
             f"d_state {self.d_state} must be even: the state channels rotate in pairs"),
            (lambda: self.norm_eps > 0, f"norm_eps {self.norm_eps} must be positive"),
            (lambda: self.attn_impl in ATTN_IMPLS, f"attn_impl {self.attn_impl!r} is not one of {ATTN_IMPLS}"),
        )
        for ok, message in checks:
            if not ok():
                raise ValueError(message)
        if self.attn_impl in ("hip", "hip_fused") and (self.d_head, self.d_state) != (HIP_D_HEAD, HIP_D_STATE):
            raise ValueError(f"attn_impl {self.attn_impl!r} runs d_head {HIP_D_HEAD} and d_state {HIP_D_STATE} only "
                             f"(this config: d_head {self.d_head}, d_state {self.d_state}); choose 'torch' or 'auto'")

    @property
    def d_head(self) -> int:
        return self.d_model // self.n_head

    def parameter_shapes(self) -> dict[str, tuple[int, ...]]:
        """State-dict names and shapes of :class:`sisa_amd.SISAForCausalLM` (the tied LM head has no entry of its
        own). The names are the reference's (src/sisa/modeling.py:122-141, 258-330), so checkpoints interchange."""
        d, h, s, f = self.d_model, self.n_head, self.d_state, self.d_ff
        block = {"attn_norm.weight": (d,),
                 "attn.W_Q.weight": (d, d), "attn.W_K.weight": (d, d), "attn.W_V.weight": (d, d),
                 "attn.W_B.weight": (h * s, d), "attn.W_C.weight": (h * s, d),
                 "attn.theta_proj.weight": (h * s // 2, d),
                 "attn.alpha_proj.weight": (h, d), "attn.alpha_proj.bias": (h,),
                 "attn.forget_proj.weight": (h, d), "attn.forget_proj.bias": (h,),
                 "attn.lambda_raw": (h,), "attn.W_O.weight": (d, d),
                 "ffn_norm.weight": (d,),
                 "ffn.w_gate.weight": (f, d), "ffn.w_up.weight": (f, d), "ffn.w_down.weight": (d, f)}
        shapes = {"embed.weight": (self.vocab_size, d)}
        for i in range(self.n_layer):
            shapes.update({f"layers.{i}.{k}": v for k, v in block.items()})
        shapes["final_norm.weight"] = (d,)
        return shapes

    def num_parameters(self) -> int:
        """Number of parameters (the tied embedding / LM head counted once)."""
        total = 0
        for shape in self.parameter_shapes().values():
            n = 1
            for x in shape:
                n *= x
            total += n
        return total

    def to_dict(self) -> dict[str, Any]:
        return dataclasses.asdict(self)

    @classmethod
    def from_dict(cls, data: Mapping[str, Any], **overrides: Any) -> "SISAConfig":
        """A config from a mapping (e.g. a ``config.json``) plus overrides; keys that are not fields raise
        ``ValueError``."""
        fields = {f.name for f in dataclasses.fields(cls)}
        values = dict(data)
        values.update(overrides)
        extra = sorted(k for k in values if k not in fields)
        if extra:
            raise ValueError(f"unknown SISAConfig fields: {extra}")
        return cls(**values)

    @classmethod
    def preset(cls, name: str, **overrides: Any) -> "SISAConfig":
        """The config of a paper model size (``"sisa-50m"``, ``"sisa-152m"``, ``"sisa-369m"``) plus overrides."""
        if name not in PRESETS:
            raise ValueError(f"unknown preset {name!r} (known: {', '.join(sorted(PRESETS))})")
        return cls.from_dict(PRESETS[name], **overrides)

    def replace(self, **changes: Any) -> "SISAConfig":
        """A checked copy with ``changes`` applied."""
        return dataclasses.replace(self, **changes)


#: The paper model sizes (d_head 64, d_state 32, vocabulary 50,277); the values of src/sisa/config.py:145-149.
PRESETS: dict[str, dict[str, Any]] = {
    "sisa-50m": dict(d_model=512, n_layer=6, n_head=8, d_ff=1829),
    "sisa-152m": dict(d_model=768, n_layer=12, n_head=12, d_ff=2744),
    "sisa-369m": dict(d_model=1024, n_layer=24, n_head=16, d_ff=2507),
}
