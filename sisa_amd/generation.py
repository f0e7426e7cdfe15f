"""Incremental decoding with a per-layer cache (src/sisa/generation.py:1-191).

Besides ``k`` and ``v`` a SISA layer caches, per head and token, the rotated state write vector ``b~_j`` (``d_state``
values), the cumulative decay ``g_j`` and the cumulative forget value ``F_j``; the running phase ``Phi`` is kept for
the last position only. A new token extends ``g``, ``F`` and ``Phi`` in float32 and attends to the cache with the
exact score. The prompt (prefill) goes through the regular unfused attention backend; decode steps use the HIP decode
kernel on the GPU (:mod:`sisa_amd.kernels.decode`) and the exact float32 torch rows elsewhere. Batched decoding
assumes equal-length prompts (there is no padding mask).
"""
from __future__ import annotations

import numbers
from dataclasses import dataclass
from typing import TYPE_CHECKING, Iterable

import torch
from torch import Tensor

if TYPE_CHECKING:  # pragma: no cover
    from .modeling import SISAForCausalLM

__all__ = ["LayerState", "SISACache", "generate"]


@dataclass
class LayerState:
    """Cached tensors of one layer: ``k, v`` ``(B, H, T, d_head)`` and ``b`` ``(B, H, T, d_state)`` in the attention
    compute dtype; ``g, fgate`` ``(B, H, T)`` float32; ``phi`` ``(B, H, d_state // 2)`` float32 at the last
    position."""

    k: Tensor
    v: Tensor
    b: Tensor
    g: Tensor
    fgate: Tensor
    phi: Tensor

    @property
    def length(self) -> int:
        return self.k.shape[2]


class SISACache:
    """Decode cache holding one :class:`LayerState` per layer."""

    def __init__(self) -> None:
        self._layers: dict[int, LayerState] = {}

    def get(self, layer_idx: int) -> LayerState | None:
        return self._layers.get(layer_idx)

    def update(self, layer_idx: int, *, k: Tensor, v: Tensor, b: Tensor, g: Tensor, fgate: Tensor,
               phi: Tensor) -> LayerState:
        """Append new positions to a layer's cache and return the updated state."""
        old = self._layers.get(layer_idx)
        if old is None:
            state = LayerState(k=k, v=v, b=b, g=g, fgate=fgate, phi=phi)
        else:
            state = LayerState(k=torch.cat([old.k, k], dim=2), v=torch.cat([old.v, v], dim=2),
                               b=torch.cat([old.b, b], dim=2), g=torch.cat([old.g, g], dim=2),
                               fgate=torch.cat([old.fgate, fgate], dim=2), phi=phi)
        self._layers[layer_idx] = state
        return state

    @property
    def seq_len(self) -> int:
        """Number of cached positions (0 when empty)."""
        state = self._layers.get(0)
        return 0 if state is None else state.length

    def reset(self) -> None:
        self._layers.clear()

    def __len__(self) -> int:
        return len(self._layers)


def _eos_ids(eos_token_id: int | Iterable[int] | Tensor | None) -> list[int]:
    """``eos_token_id`` as a list of ints. Accepted: ``None``, an integer, a 0-d or 1-d integer tensor or array, an
    iterable of integers; anything else (bools, strings, floats, nested arrays) raises ``TypeError``."""
    def reject() -> TypeError:
        return TypeError(f"eos_token_id must be an integer or an iterable of integers, "
                         f"got {eos_token_id!r} ({type(eos_token_id).__name__})")

    if eos_token_id is None:
        return []
    if isinstance(eos_token_id, (bool, str, bytes)):
        raise reject()
    if isinstance(eos_token_id, numbers.Integral):
        return [int(eos_token_id)]
    if torch.is_tensor(eos_token_id):
        integral = not (eos_token_id.dtype.is_floating_point or eos_token_id.dtype.is_complex
                        or eos_token_id.dtype == torch.bool)
        if not integral or eos_token_id.dim() > 1:
            raise reject()
        return [int(t) for t in eos_token_id.reshape(-1).tolist()]
    if hasattr(eos_token_id, "dtype") and hasattr(eos_token_id, "ndim"):   # numpy array or scalar
        if eos_token_id.dtype.kind not in "iu" or eos_token_id.ndim > 1:
            raise reject()
        return [int(t) for t in eos_token_id.reshape(-1).tolist()]
    try:
        ids = list(eos_token_id)
    except TypeError:
        raise reject() from None
    if any(isinstance(t, bool) or not isinstance(t, numbers.Integral) for t in ids):
        raise reject()
    return [int(t) for t in ids]


def _next_token(logits: Tensor, *, do_sample: bool, temperature: float, top_k: int | None,
                generator: torch.Generator | None) -> Tensor:
    """Greedy argmax, or a sample from softmax(logits / temperature) restricted to the ``top_k`` largest logits."""
    scores = logits.float()
    if not do_sample:
        return scores.argmax(dim=-1)
    scores = scores / temperature
    if top_k is not None and top_k < scores.shape[-1]:
        cutoff = torch.topk(scores, top_k, dim=-1).values[..., -1:]
        scores = torch.where(scores < cutoff, torch.full_like(scores, float("-inf")), scores)
    return torch.multinomial(scores.softmax(dim=-1), num_samples=1, generator=generator).squeeze(-1)


@torch.no_grad()
def generate(model: "SISAForCausalLM", input_ids: Tensor, max_new_tokens: int, temperature: float = 1.0,
             top_k: int | None = None, eos_token_id: int | Iterable[int] | Tensor | None = None,
             do_sample: bool = False, *, generator: torch.Generator | None = None) -> Tensor:
    """Generate continuations of ``input_ids`` ``(B, L)`` or ``(L,)`` (equal-length prompts). Finished rows (after
    an ``eos_token_id``) are padded with the first id; generation stops when all rows finished. Returns
    ``(B, L + n)`` ids with ``n <= max_new_tokens`` (same rank as ``input_ids``)."""
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be >= 0")
    if do_sample and temperature <= 0:
        raise ValueError("temperature must be positive when do_sample=True")
    if top_k is not None and top_k <= 0:
        raise ValueError("top_k must be a positive integer")
    squeeze = input_ids.dim() == 1
    if squeeze:
        input_ids = input_ids.unsqueeze(0)
    if input_ids.dim() != 2 or input_ids.shape[1] == 0:
        raise ValueError("input_ids must be a non-empty (B, L) tensor")
    if max_new_tokens == 0:
        return input_ids.squeeze(0) if squeeze else input_ids
    eos = _eos_ids(eos_token_id)
    eos_t = torch.tensor(eos, device=input_ids.device, dtype=input_ids.dtype) if eos else None
    cache = SISACache()
    logits = model(input_ids, cache=cache, logits_to_keep=1).logits[:, -1]
    pieces = [input_ids]
    done = torch.zeros(input_ids.shape[0], dtype=torch.bool, device=input_ids.device)
    for step in range(max_new_tokens):
        nxt = _next_token(logits, do_sample=do_sample, temperature=temperature, top_k=top_k,
                          generator=generator).to(input_ids.dtype)
        if eos_t is not None:
            nxt = torch.where(done, eos_t[0], nxt)
            done = done | torch.isin(nxt, eos_t)
        pieces.append(nxt.unsqueeze(1))
        if step + 1 == max_new_tokens or (eos_t is not None and bool(done.all())):
            break
        logits = model(nxt.unsqueeze(1), cache=cache, logits_to_keep=1).logits[:, -1]
    out = torch.cat(pieces, dim=1)
    return out.squeeze(0) if squeeze else out
