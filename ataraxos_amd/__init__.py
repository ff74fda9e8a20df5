"""MI355X (gfx950) attention hot path of the ataraxos transformer networks.

* :class:`MultiHeadAttention` — drop-in for ``stratego.networks.attention.MultiHeadAttention``;
  its GPU path is one fused HIP kernel (``libataraxos_attn.so``).
* :class:`KeyQueryPolicyHead` — drop-in for the Move network's policy head,
  with the logits, legal-move mask and softmax fused on the GPU.
* :class:`KVCache` / :func:`ops.attention_decode` — incremental causal decode;
  :class:`SetupDecoder` runs a Setup network token by token over it and
  :class:`BeliefDecoder` a Belief network with its encoder run once.
* :func:`use_hip_attention` / :class:`KernelMultiheadAttention` — the Belief
  network's ``nn.TransformerDecoder`` attention through the same kernel.
* :class:`PreLNTransformerBlock` / :class:`TransformerStack` — drop-ins for
  the reference's pre-LN blocks; the attention half (LayerNorm, projections,
  attention, residual) is one launch where the persistent kernel applies.
* :class:`StrategoRolloutBuffer` — drop-in for the reference's CUDA self-play
  simulator: N games on the GPU producing the legal-move masks and
  infostates the networks consume.

Importing the package does not load the library or touch the GPU.
"""

from . import ops
from .attention import MultiHeadAttention, math_attention
from .decode import BeliefDecoder, KVCache, SetupDecoder
from .decoder import KernelMultiheadAttention, use_hip_attention
from .policy import KeyQueryPolicyHead, masked_policy_logits, masked_policy_softmax
from .rollout import StrategoRolloutBuffer
from .transformer import PreLNTransformerBlock, TransformerStack

__all__ = [
    "ops",
    "MultiHeadAttention",
    "math_attention",
    "KeyQueryPolicyHead",
    "masked_policy_logits",
    "masked_policy_softmax",
    "KVCache",
    "SetupDecoder",
    "BeliefDecoder",
    "KernelMultiheadAttention",
    "use_hip_attention",
    "StrategoRolloutBuffer",
    "PreLNTransformerBlock",
    "TransformerStack",
]
