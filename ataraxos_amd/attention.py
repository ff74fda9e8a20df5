"""Drop-in ``MultiHeadAttention`` whose GPU path is the gfx950 fused kernel.

Interface parity with ``stratego/networks/attention.py:64-204``:

* constructor ``(embed_dim, num_heads, num_kv_heads=None, dropout=0.0,
  causal=False, qkv_bias=False)`` with the same ``ValueError`` checks
  (attention.py:97-103);
* attributes ``embed_dim, num_heads, num_kv_heads, head_dim, dropout,
  causal`` and submodules ``q_proj, k_proj, v_proj, out_proj`` created in that
  order, so ``state_dict`` keys and the RNG draws of their initialisation are
  the reference's (attention.py:105-116);
* ``forward(x, key_value=None)``: projections, BSHD views, causal masking only
  for self-attention, output projection (attention.py:152-204).

Backends (``backend`` property, the slot of attention.py:122-146):

* ``"hip"``  — tensors on a GPU: the fused HIP kernel (``ops.attention``).
  Its range is head_dim a multiple of 16 up to 128 and at most 256 keys;
  outside that the forward raises instead of switching to another path.
  Self-attention without autograd (inference, self-play) with head_dim 64
  and 2/4/6/8 heads, or head_dim 48 with 8 heads (the reference Move
  network's 384 = 8 x 48), no GQA, 16-bit and up to 128 positions runs the
  whole layer -- projections, attention, output projection -- as one launch
  (``ops.mha_forward``, weights rearranged into its tile order by one more
  launch on every call) where that is faster, i.e. from the sequence length
  :data:`FUSED_MIN_SEQ` (:data:`FUSED_MIN_SEQ_D48`) gives for the head count;
  with autograd the projections stay ``nn.Linear`` and the attention
  kernel's backward applies.  Training with ``dropout > 0`` at head_dim 64
  or 48 runs the kernels' own attention dropout (``ops.attention`` with
  ``dropout_p``: each weight dropped by a hash of its index under a seed
  drawn from torch's default generator per call; the backward recomputes the
  same decisions).
* ``"math"`` — tensors on the CPU, or training with ``dropout > 0`` at
  other head sizes (attention.py:134-138 likewise routes dropout away from
  its FA3 backend).  It keeps the semantics of attention.py:281-316.
"""

from __future__ import annotations

import math
from typing import cast

import torch
import torch.nn as nn
import torch.nn.functional as F  # noqa: N812

from . import ops

__all__ = ["MultiHeadAttention", "math_attention", "FUSED_MIN_SEQ", "FUSED_MIN_SEQ_D48"]

# Shortest sequence at which the one-launch layer (ops.mha_forward with packed
# weights) beats the unfused path (hipBLASLt projections + the attention
# kernel), by head count at head_dim 64, measured on MI355X through this
# module in inference at B=4096 (8 heads: B=2048), bf16, causal and not.  The
# fused layer streams every weight from L2 once per sample whatever the
# length, so the shortest sequences stay cheaper unfused: at 8 heads 158 us
# fused against 116 us unfused at L=16, 191 against 198 at L=24.
FUSED_MIN_SEQ = {2: 1, 4: 1, 6: 16, 8: 24}
# The same at head_dim 48 (8 heads, embed_dim 384: the reference Move
# network), measured at B=4096: 202 us fused against 153 us unfused at L=8,
# 211 against 241 at L=16, 856 against 1631 at the network's L=101.
FUSED_MIN_SEQ_D48 = {8: 16}


def math_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool,
    dropout_p: float = 0.0,
    scale: float | None = None,
    key_padding_mask: torch.Tensor | None = None,
) -> torch.Tensor:
    """Unfused attention with the semantics of attention.py:281-316.

    q ``[B, S_q, H, D]``, k/v ``[B, S_kv, H_kv, D]`` -> ``[B, S_q, H, D]``.
    The scale multiplies the product after the matmul; the causal mask is
    top-left aligned (``triu(ones(S_q, S_kv), 1)`` set to -inf); KV heads are
    repeated per query group as ``repeat_interleave`` does.
    """
    n_heads, n_kv = q.shape[2], k.shape[2]
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if n_kv != n_heads:
        kh = kh.repeat_interleave(n_heads // n_kv, dim=1)
        vh = vh.repeat_interleave(n_heads // n_kv, dim=1)
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(qh, kh.transpose(-2, -1).contiguous()) * scale
    if is_causal:
        above = torch.ones(q.shape[1], k.shape[1], dtype=torch.bool, device=q.device).triu(1)
        scores = scores.masked_fill(above, float("-inf"))
    if key_padding_mask is not None:
        scores = scores.masked_fill(key_padding_mask[:, None, None, :], float("-inf"))
    probs = F.softmax(scores, dim=-1)
    if dropout_p > 0.0:
        probs = F.dropout(probs, p=dropout_p)
    return torch.matmul(probs, vh).transpose(1, 2)


class MultiHeadAttention(nn.Module):
    """Multi-head / grouped-query attention; see the module docstring."""

    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        num_kv_heads: int | None = None,
        dropout: float = 0.0,
        causal: bool = False,
        qkv_bias: bool = False,
    ) -> None:
        super().__init__()
        if embed_dim % num_heads != 0:
            raise ValueError(f"embed_dim ({embed_dim}) must be divisible by num_heads ({num_heads})")
        kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        if num_heads % kv_heads != 0:
            raise ValueError(f"num_heads ({num_heads}) must be divisible by num_kv_heads ({kv_heads})")

        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads: int = kv_heads
        self.head_dim: int = embed_dim // num_heads
        self.dropout: float = dropout
        self.causal: bool = causal
        # Not in the reference: False keeps the unfused GPU path (nn.Linear
        # projections + the attention kernel) also where the one-launch
        # layer would apply.  Not part of the state_dict.
        self.fuse_layer: bool = True

        kv_dim = kv_heads * self.head_dim
        self.q_proj = nn.Linear(embed_dim, num_heads * self.head_dim, bias=qkv_bias)
        self.k_proj = nn.Linear(embed_dim, kv_dim, bias=qkv_bias)
        self.v_proj = nn.Linear(embed_dim, kv_dim, bias=qkv_bias)
        self.out_proj = nn.Linear(num_heads * self.head_dim, embed_dim, bias=qkv_bias)

    @property
    def backend(self) -> str:
        """``"hip"`` on a GPU, ``"math"`` on the CPU or when dropout must run
        at a head size the kernels have no dropout for."""
        device = next(self.parameters()).device
        if device.type != "cuda":
            return "math"
        if self.training and self.dropout > 0.0 and self.head_dim not in ops.DROPOUT_HEAD_DIMS:
            return "math"
        return "hip"

    def forward(self, x: torch.Tensor, key_value: torch.Tensor | None = None) -> torch.Tensor:
        """``x`` ``[B, S_q, E]``; ``key_value`` ``[B, S_kv, E]`` or None -> ``[B, S_q, E]``."""
        batch, seq_q, _ = x.shape
        if key_value is None and self._fused_ok(x):
            return self._forward_fused(x)
        src = x if key_value is None else key_value
        q = self.q_proj(x).view(batch, seq_q, self.num_heads, self.head_dim)
        k = self.k_proj(src)
        seq_kv = k.shape[1]
        k = k.view(batch, seq_kv, self.num_kv_heads, self.head_dim)
        v = self.v_proj(src).view(batch, seq_kv, self.num_kv_heads, self.head_dim)
        is_causal = self.causal and key_value is None

        if self.backend == "hip":
            attn = self._forward_hip(q, k, v, is_causal)
        else:
            attn = self._forward_math(q, k, v, is_causal)
        return cast(torch.Tensor, self.out_proj(attn.reshape(batch, seq_q, self.embed_dim)))

    def _fused_ok(self, x: torch.Tensor) -> bool:
        """The one-launch layer applies: GPU, no autograd, no dropout to run,
        a shape the fused kernel covers, and a sequence long enough for it to
        beat the unfused path (:data:`FUSED_MIN_SEQ`)."""
        if not self.fuse_layer or self.backend != "hip" or self.num_kv_heads != self.num_heads:
            return False
        if self.training and self.dropout > 0.0:
            return False
        if self.head_dim not in (48, 64):
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        table = FUSED_MIN_SEQ if self.head_dim == 64 else FUSED_MIN_SEQ_D48
        if x.shape[1] < table.get(self.num_heads, 1 << 30):
            return False
        w = self.q_proj.weight
        return x.dtype == w.dtype and ops.mha_forward_supported(self.embed_dim, self.num_heads, x.shape[1], x.dtype)

    def _forward_fused(self, x: torch.Tensor) -> torch.Tensor:
        """Projections + attention + output projection in one kernel launch,
        after one launch that rearranges the four weights into the kernel's
        tile order.  The rearrangement is redone on every call (a few
        microseconds against the layer's hundreds), so weights changed in
        place by any route -- an optimizer step, ``load_state_dict``, the
        EMA swap's ``param.data.copy_`` -- are always the ones used."""
        w = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.out_proj.weight)
        return ops.mha_forward(
            x, *(t.detach() for t in w),
            num_heads=self.num_heads, b_q=self.q_proj.bias, b_k=self.k_proj.bias, b_v=self.v_proj.bias,
            b_o=self.out_proj.bias, causal=self.causal, scale=1.0 / math.sqrt(self.head_dim), repack=True,
        )

    def _expand_kv_heads(self, k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Repeat ``(B, H_kv, S, D)`` KV heads up to ``H`` (attention.py:210-220)."""
        if self.num_kv_heads == self.num_heads:
            return k, v
        rep = self.num_heads // self.num_kv_heads
        return k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)

    def _forward_hip(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool) -> torch.Tensor:
        """Fused gfx950 kernel on the BSHD views; GQA is indexed, not expanded."""
        if not ops.attention_supported(self.head_dim, k.shape[1], q.dtype):
            raise RuntimeError(
                f"MultiHeadAttention: the HIP kernel does not cover head_dim={self.head_dim}, "
                f"seq_kv={k.shape[1]}, dtype={q.dtype} (head_dim in {ops.HEAD_DIMS}, seq_kv <= {ops.MAX_SEQ_KV})"
            )
        p = self.dropout if (self.training and self.dropout > 0.0) else 0.0
        return ops.attention(q, k, v, causal=is_causal, dropout_p=p)

    def _forward_math(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool) -> torch.Tensor:
        p = self.dropout if (self.training and self.dropout > 0.0) else 0.0
        return math_attention(q, k, v, is_causal, dropout_p=p)
