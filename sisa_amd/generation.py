"""Incremental decoding: the per-layer cache and ``generate`` (the API of the reference's src/sisa/generation.py).

Per head and cached position a SISA layer keeps, besides ``k`` and ``v``, the rotated state write vector ``b~``
(``d_state`` values) and the cumulative decay ``g`` and forget ``F`` values; the running phase ``Phi`` is kept for the
last position only. A new token extends ``g``, ``F`` and ``Phi`` in float32 and attends to the whole cache with the
exact score (on the GPU through the HIP decode kernel, :mod:`sisa_amd.kernels.decode`).

The cache is a set of preallocated slabs per layer, ``(B, H, capacity, .)``, filled front to back: a decode step
writes its rows in place and the layer state handed to the attention is a view of the filled prefix, so a step costs
the new rows' bytes, not a copy of the whole cache. ``generate`` sizes the slabs for the prompt plus every new token
up front; a cache made without a capacity grows by doubling. When the appended rows carry autograd history the slab
is rebuilt out of place instead, so gradients still flow. Batched decoding assumes equal-length prompts (there is no
padding mask).
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
    """One layer's cached positions: ``k, v`` ``(B, H, T, d_head)`` and ``b`` ``(B, H, T, d_state)`` in the
    attention's compute dtype, ``g, fgate`` ``(B, H, T)`` float32, and ``phi`` ``(B, H, d_state // 2)`` float32 at the
    last position. The position tensors may be views of a larger slab."""

    k: Tensor
    v: Tensor
    b: Tensor
    g: Tensor
    fgate: Tensor
    phi: Tensor

    @property
    def length(self) -> int:
        return self.k.shape[2]


class _Slab:
    """Position-axis buffers of one layer with room for ``capacity`` positions, ``filled`` of them in use."""

    def __init__(self, buffers: dict[str, Tensor], filled: int, phi: Tensor):
        self.buffers, self.filled, self.phi = buffers, filled, phi

    @property
    def capacity(self) -> int:
        return self.buffers["k"].shape[2]

    def state(self) -> LayerState:
        return LayerState(**{n: t[:, :, :self.filled] for n, t in self.buffers.items()}, phi=self.phi)


class SISACache:
    """Decode cache: one slab of :class:`LayerState` tensors per layer. ``capacity``: positions to reserve per layer
    when a layer is first filled (default: what the first fill needs, then doubling)."""

    def __init__(self, capacity: int | None = None) -> None:
        if capacity is not None and capacity < 1:
            raise ValueError(f"SISACache capacity must be positive, got {capacity}")
        self.capacity = capacity
        self._slabs: dict[int, _Slab] = {}

    def get(self, layer_idx: int) -> LayerState | None:
        slab = self._slabs.get(layer_idx)
        return None if slab is None else slab.state()

    def update(self, layer_idx: int, *, k: Tensor, v: Tensor, b: Tensor, g: Tensor, fgate: Tensor,
               phi: Tensor) -> LayerState:
        """Append positions (dim 2 of ``k, v, b, g, fgate``) to a layer's cache, take ``phi`` as its new last phase,
        and return the layer's whole cached state."""
        new = dict(k=k, v=v, b=b, g=g, fgate=fgate)
        slab = self._slabs.get(layer_idx)
        n_new = k.shape[2]
        if any(t.shape[2] != n_new for t in new.values()):
            raise ValueError(f"SISACache.update: position counts differ: "
                             f"{ {n: t.shape[2] for n, t in new.items()} }")
        if torch.is_grad_enabled() and any(t.requires_grad for t in new.values()):
            old = None if slab is None else slab.state()
            bufs = new if old is None else {n: torch.cat([getattr(old, n), t], 2) for n, t in new.items()}
            slab = _Slab(bufs, bufs["k"].shape[2], phi)
        else:
            filled = 0 if slab is None else slab.filled
            need = filled + n_new
            if slab is None or need > slab.capacity:
                room = max(need, self.capacity or 0, 2 * slab.capacity if slab is not None else 0)
                grown = {n: t.new_empty(t.shape[:2] + (room,) + t.shape[3:]) for n, t in new.items()}
                if slab is not None:
                    for n, t in grown.items():
                        t[:, :, :filled].copy_(slab.buffers[n][:, :, :filled])
                slab = _Slab(grown, filled, phi)
            for n, t in new.items():
                slab.buffers[n][:, :, filled:need].copy_(t)
            slab.filled, slab.phi = need, phi
        self._slabs[layer_idx] = slab
        return slab.state()

    @property
    def seq_len(self) -> int:
        """How many positions the cache holds (0 before the prefill)."""
        slab = self._slabs.get(0)
        return 0 if slab is None else slab.filled

    def reset(self) -> None:
        self._slabs.clear()

    def __len__(self) -> int:
        return len(self._slabs)


def _eos_ids(eos_token_id: int | Iterable[int] | Tensor | None) -> list[int]:
    """The end-of-sequence ids as a list: from ``None``, an integer, a 0-d or 1-d integer tensor or numpy array, or
    an iterable of integers. Booleans, strings, floats and arrays of more than one dimension raise ``TypeError``."""
    if eos_token_id is None:
        return []
    err = TypeError(f"eos_token_id takes one token id or a flat collection of ids; {eos_token_id!r} "
                    f"({type(eos_token_id).__name__}) is neither")
    if isinstance(eos_token_id, (bool, str, bytes)):
        raise err
    if isinstance(eos_token_id, numbers.Integral):
        return [int(eos_token_id)]
    if torch.is_tensor(eos_token_id):
        integer = eos_token_id.dtype not in (torch.bool,) and not (eos_token_id.dtype.is_floating_point
                                                                   or eos_token_id.dtype.is_complex)
        if not integer or eos_token_id.dim() > 1:
            raise err
        return eos_token_id.reshape(-1).tolist()
    kind = getattr(getattr(eos_token_id, "dtype", None), "kind", None)       # numpy arrays and scalars
    if kind is not None:
        if kind not in "iu" or eos_token_id.ndim > 1:
            raise err
        return [int(t) for t in eos_token_id.reshape(-1).tolist()]
    try:
        ids = list(eos_token_id)
    except TypeError:
        raise err from None
    if not all(isinstance(t, numbers.Integral) and not isinstance(t, bool) for t in ids):
        raise err
    return [int(t) for t in ids]


def _pick(logits: Tensor, do_sample: bool, temperature: float, top_k: int | None,
          generator: torch.Generator | None) -> Tensor:
    """The next token per row: argmax, or a draw from ``softmax(logits / temperature)`` over the whole vocabulary
    with every logit below the row's ``top_k``-th largest set to -inf (the reference's sampling rule,
    src/sisa/generation.py:126-135: ties at the k-th value stay candidates, and a seeded generator yields the same
    draws as the reference's)."""
    scores = logits.float()
    if not do_sample:
        return scores.argmax(dim=-1)
    scores = scores / temperature
    if top_k is not None and top_k < scores.shape[-1]:
        floor = scores.topk(top_k, dim=-1).values[..., -1:]
        scores = torch.where(scores < floor, torch.full_like(scores, float("-inf")), scores)
    return torch.multinomial(scores.softmax(-1), 1, generator=generator).squeeze(-1)


@torch.no_grad()
def generate(model: "SISAForCausalLM", input_ids: Tensor, max_new_tokens: int, temperature: float = 1.0,
             top_k: int | None = None, eos_token_id: int | Iterable[int] | Tensor | None = None,
             do_sample: bool = False, *, generator: torch.Generator | None = None) -> Tensor:
    """Continue the prompts ``input_ids`` (``(B, L)`` of equal-length rows, or ``(L,)``) by up to ``max_new_tokens``
    tokens: greedy, or sampled at ``temperature`` from the ``top_k`` most likely tokens with ``do_sample``.

    A row that emits an ``eos_token_id`` is finished and padded with the first such id from then on; generation
    ends when every row is finished. Returns ``(B, L + n)`` ids, ``n <= max_new_tokens``, with the rank of
    ``input_ids``.
    """
    if max_new_tokens < 0:
        raise ValueError(f"max_new_tokens = {max_new_tokens} is negative")
    if do_sample and temperature <= 0:
        raise ValueError(f"sampling needs a positive temperature, got {temperature}")
    if top_k is not None and top_k <= 0:
        raise ValueError(f"top_k = {top_k}: expected a positive integer or None")
    rows = input_ids if input_ids.dim() == 2 else input_ids.unsqueeze(0)
    if rows.dim() != 2 or rows.shape[1] == 0:
        raise ValueError(f"generate needs at least one prompt token per row in a (B, L) or (L,) tensor, got shape "
                         f"{tuple(input_ids.shape)}")
    stops = _eos_ids(eos_token_id)
    stop_ids = torch.tensor(stops, device=rows.device, dtype=rows.dtype) if stops else None
    prompt = rows.shape[1]
    out = rows.new_empty((rows.shape[0], prompt + max_new_tokens))
    out[:, :prompt] = rows
    length = prompt
    if max_new_tokens:
        cache = SISACache(capacity=prompt + max_new_tokens)
        finished = torch.zeros(rows.shape[0], dtype=torch.bool, device=rows.device)
        logits = model(rows, cache=cache, logits_to_keep=1).logits[:, -1]
        while True:
            token = _pick(logits, do_sample, temperature, top_k, generator).to(rows.dtype)
            if stop_ids is not None:
                token = torch.where(finished, stop_ids[0], token)
                finished |= torch.isin(token, stop_ids)
            out[:, length] = token
            length += 1
            if length == out.shape[1] or (stop_ids is not None and bool(finished.all())):
                break
            logits = model(token[:, None], cache=cache, logits_to_keep=1).logits[:, -1]
    result = out[:, :length].contiguous()
    return result if input_ids.dim() == 2 else result.squeeze(0)
