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

__all__ = ["KVCache", "SetupDecoder"]


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


class SetupDecoder:
    """Token-by-token evaluation of a Setup network over per-layer KV caches.

    ``net`` is the reference ``SetupNetwork`` (``stratego/networks/setup_net.py:80-123``)
    or any module with its structure: ``token_emb``, ``pos_emb.embed``,
    ``blocks.blocks[i]`` pre-LN blocks with ``ln1`` / ``attn`` (q/k/v/out
    projections) / ``ln2`` / ``ff`` (``stratego/networks/transformer.py:117-145``),
    and ``value_head`` / ``entropy_head`` / ``policy_head``.  The network is
    causal, so the output at position t depends only on tokens 0..t: one
    :meth:`step` per placed piece gives what the reference gets by re-running
    the network over the whole prefix (``selfplay.py:139-146,181``), with one
    query row per layer instead of t.

    :meth:`step` returns ``(value_logits [B, 3], entropy [B],
    policy_logits [B, num_types])``: the value and entropy heads read position
    0 (``transformer.py:193-250``), the policy the newest position
    (``selfplay.py:182``).
    """

    def __init__(self, net: torch.nn.Module, batch: int, capacity: int = 40) -> None:
        self.net = net
        blocks = list(net.blocks.blocks)
        attn = blocks[0].attn
        p = next(net.parameters())
        self.heads, self.kv_heads, self.head_dim = attn.num_heads, attn.num_kv_heads, attn.head_dim
        self.cache = KVCache(len(blocks), batch, self.kv_heads, capacity, self.head_dim, dtype=p.dtype, device=p.device)
        self.first: torch.Tensor | None = None  # position 0's output (value / entropy heads)

    def reset(self) -> None:
        self.cache.reset()
        self.first = None

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Feed the newest token ``[B]`` (int) of every sequence."""
        net, t = self.net, self.cache.length
        x = net.token_emb(tokens) + net.pos_emb.embed[t]
        b = x.shape[0]
        for layer, blk in enumerate(net.blocks.blocks):
            a = blk.attn
            hn = blk.ln1(x)
            q = a.q_proj(hn).view(b, self.heads, self.head_dim)
            k = a.k_proj(hn).view(b, self.kv_heads, self.head_dim)
            v = a.v_proj(hn).view(b, self.kv_heads, self.head_dim)
            o = self.cache.step(layer, q, k, v)
            x = x + a.out_proj(o.reshape(b, -1))
            x = x + blk.ff(blk.ln2(x))
        self.cache.advance()
        if self.first is None:
            self.first = x
        return net.value_head(self.first), net.entropy_head(self.first), net.policy_head(x)
