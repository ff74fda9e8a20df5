"""The Belief network's decoder attention through the fused kernel.

The reference's Belief decoder is ``nn.TransformerDecoder`` over
``nn.TransformerDecoderLayer(batch_first=True, norm_first=True)``
(``stratego/networks/belief_net.py:105-114``), called with a float causal
``tgt_mask`` (``triu(full(-inf), 1)``, ``belief_net.py:167-170``) and a bool
``memory_key_padding_mask = ~hidden_mask`` (``belief_net.py:159,172-177``).
Inside, each layer calls ``self_attn`` and ``multihead_attn``, both
``nn.MultiheadAttention`` with a packed ``in_proj_weight [3E, E]``,
``in_proj_bias`` and a biased ``out_proj``.

:class:`KernelMultiheadAttention` is ``nn.MultiheadAttention`` with the same
parameters, ``state_dict`` keys and call signature, whose GPU forward runs
the projections as ``F.linear`` and the attention as one HIP kernel launch
(causal self-attention; cross-attention with key padding).
:func:`use_hip_attention` converts every ``nn.MultiheadAttention`` inside a
module in place, so an existing decoder (and its checkpoint) is used as is.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .attention import FUSED_MIN_SEQ

__all__ = ["KernelMultiheadAttention", "use_hip_attention"]


class KernelMultiheadAttention(nn.MultiheadAttention):
    """``nn.MultiheadAttention`` whose GPU forward is the fused HIP kernel.

    Covered on the GPU: ``need_weights=False`` (what ``TransformerDecoderLayer``
    passes), no mask or the causal mask (``is_causal=True``, the hint
    ``nn.TransformerDecoder`` derives from a ``triu(-inf, 1)`` mask), and a
    bool ``key_padding_mask`` ``[B, S_kv]`` (True = ignore).  Anything else
    raises on the GPU instead of silently taking another path.  In training
    with ``dropout > 0`` at head_dim 48 or 64 (the Belief decoder's 512 / 8)
    the kernel drops the attention weights itself, as
    ``nn.MultiheadAttention`` does (``ops.attention`` with ``dropout_p``: the
    keep decisions a hash of each weight's index under a seed drawn from
    torch's default generator per call).  On the CPU, and in training with
    dropout at other head sizes, the forward is ``nn.MultiheadAttention``'s
    own, as in the reference.

    Self-attention (``query``, ``key`` and ``value`` the same tensor, as
    ``TransformerDecoderLayer`` calls it) without a key padding mask and
    without autograd runs as one launch of the fused layer
    (``ops.mha_forward``, weights rearranged into its tile order on every
    call) where that is
    faster (``FUSED_MIN_SEQ``, head_dim 64); ``fuse_layer = False`` keeps the
    projections + attention kernel path.
    """

    fuse_layer: bool = True  # class default: converted modules skip __init__

    def forward(  # type: ignore[override]
        self,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        key_padding_mask: torch.Tensor | None = None,
        need_weights: bool = True,
        attn_mask: torch.Tensor | None = None,
        average_attn_weights: bool = True,
        is_causal: bool = False,
    ) -> tuple[torch.Tensor, torch.Tensor | None]:
        drop = self.dropout if (self.training and self.dropout > 0.0) else 0.0
        if not query.is_cuda or (drop > 0.0 and self.embed_dim // self.num_heads not in ops.DROPOUT_HEAD_DIMS):
            return super().forward(
                query, key, value, key_padding_mask=key_padding_mask, need_weights=need_weights,
                attn_mask=attn_mask, average_attn_weights=average_attn_weights, is_causal=is_causal,
            )
        if need_weights:
            raise NotImplementedError("KernelMultiheadAttention on the GPU returns no weights: pass need_weights=False")
        if attn_mask is not None and not is_causal:
            raise NotImplementedError(
                "KernelMultiheadAttention on the GPU supports no attn_mask other than the causal one (is_causal=True)"
            )
        if key_padding_mask is not None and key_padding_mask.dtype != torch.bool:
            raise NotImplementedError("KernelMultiheadAttention on the GPU takes a bool key_padding_mask")
        self_attention = query is key and key is value
        if not self.batch_first:
            query, key, value = (t.transpose(0, 1) for t in (query, key, value))
        b, sq, e = query.shape
        skv = key.shape[1]
        h = self.num_heads
        d = e // h
        if self._qkv_same_embed_dim:
            w_q, w_k, w_v = self.in_proj_weight.chunk(3)
        else:
            w_q, w_k, w_v = self.q_proj_weight, self.k_proj_weight, self.v_proj_weight
        b_q = b_k = b_v = None
        if self.in_proj_bias is not None:
            b_q, b_k, b_v = self.in_proj_bias.chunk(3)
        if self_attention and key_padding_mask is None and drop == 0.0 and self._fused_ok(query):
            assert self.in_proj_weight is not None
            ws = (w_q, w_k, w_v, self.out_proj.weight)
            out = ops.mha_forward(
                query, *(t.detach() for t in ws),
                num_heads=h, b_q=b_q, b_k=b_k, b_v=b_v, b_o=self.out_proj.bias, causal=is_causal,
                scale=d**-0.5, repack=True,
            )
            return (out if self.batch_first else out.transpose(0, 1)), None
        q = F.linear(query, w_q, b_q).view(b, sq, h, d)
        k = F.linear(key, w_k, b_k).view(b, skv, h, d)
        v = F.linear(value, w_v, b_v).view(b, skv, h, d)
        o = ops.attention(q, k, v, causal=is_causal, key_padding_mask=key_padding_mask, dropout_p=drop)
        out = self.out_proj(o.reshape(b, sq, e))
        if not self.batch_first:
            out = out.transpose(0, 1)
        return out, None


    def _fused_ok(self, x: torch.Tensor) -> bool:
        """The one-launch layer applies to self-attention over ``x``
        ``[B, S, E]``: no autograd, packed q/k/v weights, head_dim 64, a
        16-bit dtype matching the weights, and a sequence at least
        ``FUSED_MIN_SEQ`` long for the head count."""
        if not self.fuse_layer or not self._qkv_same_embed_dim or self.in_proj_weight is None:
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        e, h, s = self.embed_dim, self.num_heads, x.shape[1]
        if e != 64 * h or x.dtype != self.in_proj_weight.dtype or s < FUSED_MIN_SEQ.get(h, 1 << 30):
            return False
        return ops.mha_forward_supported(e, h, s, x.dtype)


def use_hip_attention(module: nn.Module) -> nn.Module:
    """Convert every ``nn.MultiheadAttention`` inside ``module`` (itself
    included) to :class:`KernelMultiheadAttention`, in place: parameters,
    buffers and ``state_dict`` keys are unchanged.  Returns ``module``."""
    for m in module.modules():
        if type(m) is nn.MultiheadAttention:
            if m.bias_k is not None or m.add_zero_attn:
                raise NotImplementedError("use_hip_attention: add_bias_kv / add_zero_attn are not supported")
            if (m.embed_dim // m.num_heads) % 16 != 0:
                raise NotImplementedError(f"use_hip_attention: head_dim {m.embed_dim // m.num_heads} not supported")
            m.__class__ = KernelMultiheadAttention
    return module
