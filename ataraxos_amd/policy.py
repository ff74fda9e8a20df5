"""Key-query policy head of the Move network on the gfx950 fused kernel.

Interface parity with ``KeyQueryPolicyHead`` (``stratego/networks/move_net.py:37-95``):
same constructor ``(embedding_dim, policy_d_model=None)``, submodules
``policy_embedding, wq, wk`` (created and xavier-initialised in that order),
``scale = d ** 0.5`` and ``forward(encoder_output, legal_move_mask=None)``
returning the flattened ``(B, S*S)`` logits with illegal entries at -1e10.

:meth:`KeyQueryPolicyHead.policy` additionally fuses the softmax that every
caller applies to those logits (``stratego/training/selfplay.py:284``,
``stratego/training/move_trainer.py:118``) into the same kernel.

Gradients (the Move trainer's ``loss.backward()``, move_trainer.py:140) of
either output go through one HIP launch (:func:`ops.kq_policy_backward`) for
bf16, fp16 and fp32 q, k, at the reference's d = 384 too; only a 16-bit d
above 128 that is not a multiple of 64 is differentiated with torch ops.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F  # noqa: N812

from . import ops

__all__ = ["KeyQueryPolicyHead", "masked_policy_softmax", "masked_policy_logits"]

ILLEGAL_LOGIT = -1e10


def _math_logits(q, k, mask, scale):
    logits = torch.matmul(q, k.transpose(-2, -1)) * scale
    if mask is not None:
        logits = logits.masked_fill(~mask, ILLEGAL_LOGIT)
    return logits.reshape(logits.shape[0], -1)


def _logit_grads(g: torch.Tensor, q: torch.Tensor, k: torch.Tensor, mask, scale: float):
    """Gradients of ``scale * q k^T`` (masked entries receive none)."""
    b, s, _ = q.shape
    g = g.reshape(b, s, s)
    if mask is not None:
        g = g.masked_fill(~mask, 0.0)
    gq = torch.matmul(g, k.float()) * scale
    gk = torch.matmul(g.transpose(1, 2).contiguous(), q.float()) * scale
    return gq.to(q.dtype), gk.to(k.dtype)


class _KqLogits(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, mask, scale):  # type: ignore[override]
        out = ops.kq_policy(q, k, mask, scale=scale, output="logits")
        ctx.save_for_backward(q, k)
        ctx.mask, ctx.scale = mask, scale
        return out

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        q, k = ctx.saved_tensors
        if ops.kq_policy_backward_supported(q.shape[1], q.shape[2], q.dtype):
            gq, gk = ops.kq_policy_backward(q, k, g, ctx.mask, ctx.scale, output="logits")
        else:
            gq, gk = _logit_grads(g.float(), q, k, ctx.mask, ctx.scale)
        return gq, gk, None, None


class _KqProbs(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, mask, scale):  # type: ignore[override]
        probs = ops.kq_policy(q, k, mask, scale=scale, output="probs")
        ctx.save_for_backward(q, k, probs)
        ctx.mask, ctx.scale = mask, scale
        return probs

    @staticmethod
    def backward(ctx, g):  # type: ignore[override]
        q, k, probs = ctx.saved_tensors
        if ops.kq_policy_backward_supported(q.shape[1], q.shape[2], q.dtype):
            gq, gk = ops.kq_policy_backward(q, k, g, ctx.mask, ctx.scale, output="probs", probs=probs)
            return gq, gk, None, None
        g = g.float()
        glogit = probs * (g - (g * probs).sum(dim=-1, keepdim=True))
        gq, gk = _logit_grads(glogit, q, k, ctx.mask, ctx.scale)
        return gq, gk, None, None


def masked_policy_logits(q, k, legal_move_mask=None, scale=None):
    """``scale * q k^T`` with illegal entries at -1e10, fp32 ``[B, S*S]`` (GPU)."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return _KqLogits.apply(q, k, legal_move_mask, scale)


def masked_policy_softmax(q, k, legal_move_mask=None, scale=None):
    """Softmax of :func:`masked_policy_logits` over all ``S*S`` entries (GPU).

    Illegal entries are exactly 0; a sample with no legal entry gets the
    uniform ``1/(S*S)``, as the softmax of an all -1e10 row does.
    """
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return _KqProbs.apply(q, k, legal_move_mask, scale)


class KeyQueryPolicyHead(nn.Module):
    """Asymmetric single-head ``Q K^T / sqrt(d)`` policy over square pairs."""

    def __init__(self, embedding_dim: int, policy_d_model: int | None = None) -> None:
        super().__init__()
        d = policy_d_model or embedding_dim
        self.policy_embedding = nn.Linear(embedding_dim, embedding_dim)
        self.wq = nn.Linear(embedding_dim, d, bias=False)
        self.wk = nn.Linear(embedding_dim, d, bias=False)
        self.scale: float = d**0.5
        nn.init.xavier_normal_(self.policy_embedding.weight)
        nn.init.xavier_normal_(self.wq.weight)
        nn.init.xavier_normal_(self.wk.weight)

    def _queries_keys(self, encoder_output: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        tokens = F.mish(self.policy_embedding(encoder_output))
        return self.wq(tokens), self.wk(tokens)

    def forward(self, encoder_output: torch.Tensor, legal_move_mask: torch.Tensor | None = None) -> torch.Tensor:
        """Flattened ``(B, S*S)`` logits in the input dtype, illegal = -1e10."""
        q, k = self._queries_keys(encoder_output)
        if q.device.type == "cuda":
            return masked_policy_logits(q, k, legal_move_mask, 1.0 / self.scale).to(q.dtype)
        return _math_logits(q, k, legal_move_mask, 1.0 / self.scale)

    def policy(self, encoder_output: torch.Tensor, legal_move_mask: torch.Tensor | None = None) -> torch.Tensor:
        """Move probabilities ``(B, S*S)`` fp32: logits, mask and softmax fused on the GPU."""
        q, k = self._queries_keys(encoder_output)
        if q.device.type == "cuda":
            return masked_policy_softmax(q, k, legal_move_mask, 1.0 / self.scale)
        return torch.softmax(_math_logits(q.float(), k.float(), legal_move_mask, 1.0 / self.scale), dim=-1)
