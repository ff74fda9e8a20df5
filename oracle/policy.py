"""float64 numpy restatement of the key-query policy head (oracle).

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np

from .attention import softmax_lastdim

ILLEGAL_LOGIT = -1e10


def kq_logits(q: np.ndarray, k: np.ndarray, mask: np.ndarray | None, scale: float) -> np.ndarray:
    """``[B, S*S]`` logits, illegal entries ``-1e10``, from-major flatten.

    Restates ``KeyQueryPolicyHead.forward`` after the projections
    (stratego/networks/move_net.py:92-95): ``q k^T`` divided by
    ``sqrt(policy_d_model)`` (here multiplied by ``scale = 1/sqrt(d)``),
    ``masked_fill(~mask, -1e10)``, ``reshape(B, -1)`` so entry ``i*S + j`` is
    from-square ``i`` to to-square ``j`` (the order of selfplay.py:245 and of
    the simulator's legal mask, stratego_buffer.cuh:45).
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    logits = np.matmul(q64, k64.swapaxes(-1, -2)) * scale
    if mask is not None:
        logits = np.where(np.asarray(mask, dtype=bool), logits, ILLEGAL_LOGIT)
    return logits.reshape(logits.shape[0], -1)


def kq_probs(q: np.ndarray, k: np.ndarray, mask: np.ndarray | None, scale: float) -> np.ndarray:
    """Softmax of :func:`kq_logits` over the ``S*S`` entries of each sample.

    Restates the callers' ``torch.softmax(policy, dim=-1)``
    (stratego/training/selfplay.py:284, stratego/training/move_trainer.py:118).
    Illegal entries come out exactly 0.0 in float64 whenever a legal entry
    exists; with none, every entry is ``1/(S*S)``.
    """
    return softmax_lastdim(kq_logits(q, k, mask, scale))


def kq_backward(
    q: np.ndarray,
    k: np.ndarray,
    mask: np.ndarray | None,
    scale: float,
    grad: np.ndarray,
    wrt: str = "logits",
) -> tuple[np.ndarray, np.ndarray]:
    """Gradients ``(dq, dk)`` of the policy head for an upstream ``grad``
    ``[B, S*S]`` with respect to :func:`kq_logits` (``wrt="logits"``, what the
    Move trainer's loss back-propagates into, stratego/training/move_trainer.py:115-140)
    or to :func:`kq_probs` (``wrt="probs"``), in float64.

    By the chain rule through move_net.py:92-95: the softmax over all ``S*S``
    entries gives ``dL = P * (G - sum(G * P))``; ``masked_fill`` passes no
    gradient to illegal entries (``dL = 0`` there, also in a sample with no
    legal entry, whose P is uniform); ``L = scale * q k^T`` gives
    ``dq = scale * dL k`` and ``dk = scale * dL^T q`` with ``dL`` as
    ``[B, S, S]`` from-major.
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    b, s, _ = q64.shape
    g = np.asarray(grad, dtype=np.float64).reshape(b, s * s)
    if wrt == "probs":
        p = kq_probs(q64, k64, mask, scale)
        g = p * (g - np.sum(g * p, axis=-1, keepdims=True))
    elif wrt != "logits":
        raise ValueError(f"wrt must be 'logits' or 'probs', got {wrt!r}")
    g = g.reshape(b, s, s)
    if mask is not None:
        g = np.where(np.asarray(mask, dtype=bool), g, 0.0)
    return np.matmul(g, k64) * scale, np.matmul(g.swapaxes(-1, -2), q64) * scale
