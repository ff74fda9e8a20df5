"""Incremental causal decoding over a per-layer KV cache.

The reference has no cache: ``SetupNetwork`` is re-run over the whole prefix
for each of the 40 placed pieces (``stratego/training/selfplay.py:139-146,181``)
and only the last position is used (``selfplay.py:182``).  With a cache each
step costs one query row per layer; :func:`ops.attention_decode` returns the
last row of the causal attention the reference recomputes
(``stratego/networks/attention.py:281-316`` with ``is_causal=True``).
"""

from __future__ import annotations

import torch

from . import ops

__all__ = ["KVCache"]


class KVCache:
    """Preallocated ``[B, H_kv, T, D]`` key/value caches for ``num_layers`` layers.

    All layers live in one allocation ``[L, 2, B, H_kv, T, D]`` so a whole
    decode (e.g. 40 setup pieces x 4 layers at B=8192: 2.7 GB in bf16) sits
    resident in HBM.
    """

    def __init__(
        self,
        num_layers: int,
        batch: int,
        num_kv_heads: int,
        capacity: int,
        head_dim: int,
        dtype: torch.dtype = torch.bfloat16,
        device: torch.device | str = "cuda",
    ) -> None:
        self.num_layers, self.batch, self.capacity = num_layers, batch, capacity
        self.storage = torch.empty(
            (num_layers, 2, batch, num_kv_heads, capacity, head_dim), dtype=dtype, device=device
        )
        self.length = 0

    def keys(self, layer: int) -> torch.Tensor:
        return self.storage[layer, 0]

    def values(self, layer: int) -> torch.Tensor:
        return self.storage[layer, 1]

    def reset(self) -> None:
        self.length = 0

    def step(
        self,
        layer: int,
        q: torch.Tensor,
        k_new: torch.Tensor,
        v_new: torch.Tensor,
        scale: float | None = None,
    ) -> torch.Tensor:
        """Append ``k_new``/``v_new`` (``[B, H_kv, D]``) at the current position
        of ``layer`` and attend ``q`` (``[B, H, D]``) over the prefix including
        it.  Call :meth:`advance` once all layers of a step are done."""
        n = self.length + 1
        if n > self.capacity:
            raise RuntimeError(f"KVCache full: capacity {self.capacity}")
        return ops.attention_decode(q, self.keys(layer), self.values(layer), n, k_new, v_new, scale=scale)

    def advance(self) -> None:
        self.length += 1
