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
import torch.nn.functional as F  # noqa: N812

from . import ops

__all__ = ["KVCache", "SetupDecoder", "BeliefDecoder"]


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
        not_causal = [i for i, blk in enumerate(blocks) if not getattr(blk.attn, "causal", False)]
        if not_causal:
            # SetupNetwork(causal=False) is a valid reference configuration
            # (setup_net.py:78,95), but then position t sees later tokens and
            # a KV-cache decode is not the full-prefix recompute.
            raise ValueError(f"SetupDecoder: blocks {not_causal} are not causal; token-by-token decoding "
                             "equals the full recompute only for a causal network")
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


class BeliefDecoder:
    """Token-by-token decoding of a Belief network with the encoder run once.

    ``net`` is the reference ``BeliefNetwork`` (``stratego/networks/belief_net.py:67-180``)
    or any module with its structure: ``net(infostate, hidden_mask)`` returning
    the encoder output ``[B, 100, dim]`` (:148-152), ``token_emb``,
    ``dec_pos_emb.embed`` and ``decoder``, an ``nn.TransformerDecoder`` of
    ``norm_first`` layers (:105-114), and ``output_proj``.

    The reference's ``BeliefSampler.sample_configs``
    (``stratego/search/belief_sampler.py:36-101``) re-runs the whole network
    -- encoder included -- for every hidden square of every sample, one sample
    at a time.  Here the encoder runs once for the batch, each decoder layer's
    cross-attention keys and values are projected once from its output, the
    self-attention keeps per-layer KV caches, and a step costs one or two
    query rows per layer: the cross-attention through the attention kernel with the
    key padding ``~hidden_mask`` (:159), the self-attention through
    :func:`ops.attention_decode`.  Step t returns what the reference's full
    decoder gives at its last position (``logits[:, -1]`` with ``t + 1``
    tokens, belief_sampler.py:92-94); :meth:`sample` draws a whole
    configuration for every row of the batch (the samples in parallel) with
    the reference's placeholder convention.
    """

    def __init__(self, net: torch.nn.Module, infostate: torch.Tensor, hidden_mask: torch.Tensor,
                 capacity: int = 40) -> None:
        self.net = net
        self.layers = list(net.decoder.layers)
        not_pre_ln = [i for i, layer in enumerate(self.layers) if not getattr(layer, "norm_first", False)]
        if not_pre_ln:
            # _row applies norm1/norm2/norm3 before each sublayer, the order of
            # norm_first=True (belief_net.py:105-114).
            raise ValueError(f"BeliefDecoder: decoder layers {not_pre_ln} are not norm_first (pre-LN)")
        with torch.no_grad():
            enc = net(infostate, hidden_mask)  # [B, 100, dim]: target_tokens None -> encoder output
        first = self.layers[0].self_attn
        self.dim, self.heads = first.embed_dim, first.num_heads
        self.head_dim = self.dim // self.heads
        b, n, _ = enc.shape
        self.pad = (~hidden_mask.bool()).contiguous()  # True = key ignored (memory_key_padding_mask)
        self.memory: list[tuple[torch.Tensor, torch.Tensor]] = []
        with torch.no_grad():
            for layer in self.layers:
                mha = layer.multihead_attn
                _, w_k, w_v = mha.in_proj_weight.chunk(3)
                b_k = b_v = None
                if mha.in_proj_bias is not None:
                    _, b_k, b_v = mha.in_proj_bias.chunk(3)
                k = F.linear(enc, w_k, b_k).view(b, n, self.heads, self.head_dim)
                v = F.linear(enc, w_v, b_v).view(b, n, self.heads, self.head_dim)
                self.memory.append((k, v))
        self.cache = KVCache(len(self.layers), b, self.heads, capacity, self.head_dim, dtype=enc.dtype,
                             device=enc.device)
        self.batch = b

    def reset(self) -> None:
        self.cache.reset()

    def _row(self, pos: int, tokens: torch.Tensor) -> torch.Tensor:
        """Run position ``pos`` with input tokens ``[B]`` through every decoder
        layer, writing its self-attention K/V at cache row ``pos`` (attending
        over rows 0..pos); returns the decoder output ``[B, dim]``."""
        net, b, e = self.net, self.batch, self.dim
        x = net.token_emb(tokens) + net.dec_pos_emb.embed[pos]
        for li, layer in enumerate(self.layers):
            sa = layer.self_attn
            qkv = F.linear(layer.norm1(x), sa.in_proj_weight, sa.in_proj_bias)
            q, k, v = (t_.reshape(b, self.heads, self.head_dim).contiguous() for t_ in qkv.chunk(3, dim=-1))
            o = ops.attention_decode(q, self.cache.keys(li), self.cache.values(li), pos + 1, k, v)
            x = x + sa.out_proj(o.reshape(b, e))
            ca = layer.multihead_attn
            w_q = ca.in_proj_weight[:e]
            b_q = ca.in_proj_bias[:e] if ca.in_proj_bias is not None else None
            qc = F.linear(layer.norm2(x), w_q, b_q).view(b, 1, self.heads, self.head_dim)
            kc, vc = self.memory[li]
            oc = ops.attention(qc, kc, vc, key_padding_mask=self.pad)
            x = x + ca.out_proj(oc.reshape(b, e))
            x = x + layer.linear2(layer.activation(layer.linear1(layer.norm3(x))))
        if net.decoder.norm is not None:
            x = net.decoder.norm(x)
        return x

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Feed the token ``[B]`` (int) of the next position; returns that
        position's logits ``[B, num_types]`` -- the last row of the full decoder
        run over every token fed so far."""
        if self.cache.length >= self.cache.capacity:
            raise RuntimeError(f"BeliefDecoder: capacity {self.cache.capacity} reached")
        x = self._row(self.cache.length, tokens)
        self.cache.advance()
        return self.net.output_proj(x)

    @torch.no_grad()
    def sample(self, num_tokens: int, generator: torch.Generator | None = None,
               return_probs: bool = False) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
        """Draw ``num_tokens`` piece types per row as the reference's sampler
        does (belief_sampler.py:84-99): at step j the decoder input is the
        tokens drawn so far followed by the placeholder 0, and p_j is a
        ``multinomial`` draw from the softmax of the last position's logits.
        Each step rewrites cache row j-1 with the drawn token and runs row j
        with the placeholder: two query rows per layer.  Returns ``[B,
        num_tokens]`` token indices (the reference's ``PieceType`` is index + 1)
        and, with ``return_probs``, the step probabilities ``[B, num_tokens, types]``."""
        if num_tokens > self.cache.capacity:
            raise ValueError(f"BeliefDecoder.sample: {num_tokens} tokens > capacity {self.cache.capacity}")
        self.reset()
        zero = torch.zeros(self.batch, dtype=torch.long, device=self.pad.device)
        toks, probs_all = [], []
        for j in range(num_tokens):
            if j > 0:
                self._row(j - 1, toks[-1])  # row j-1 now holds the drawn token
            probs = torch.softmax(self.net.output_proj(self._row(j, zero)).float(), dim=-1)
            tok = torch.multinomial(probs, 1, generator=generator).squeeze(1)
            toks.append(tok)
            probs_all.append(probs)
        self.cache.length = num_tokens
        out = torch.stack(toks, dim=1)
        return (out, torch.stack(probs_all, dim=1)) if return_probs else out
