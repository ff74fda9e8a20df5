"""float64 numpy restatement of the reference attention math path (oracle).

Test infrastructure only (see ``oracle/__init__.py``).
"""

from __future__ import annotations

import numpy as np

NEG_INF = -np.inf


def expand_kv_heads(x: np.ndarray, num_heads: int) -> np.ndarray:
    """``[B, H_kv, S, D] -> [B, H, S, D]``: each KV head repeated ``H/H_kv``
    times consecutively, so query head ``h`` reads KV head ``h // (H/H_kv)``.

    Restates ``MultiHeadAttention._expand_kv_heads``
    (stratego/networks/attention.py:210-220, ``repeat_interleave`` on dim 1).
    """
    group = num_heads // x.shape[1]
    return x if group == 1 else np.repeat(x, group, axis=1)


def softmax_lastdim(s: np.ndarray) -> np.ndarray:
    """Max-shifted softmax over the last axis; an all ``-inf`` row gives NaN,
    as ``torch.softmax`` does."""
    m = s.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(s - m)
        return e / e.sum(axis=-1, keepdims=True)


def attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    causal: bool = False,
    scale: float | None = None,
    key_pad: np.ndarray | None = None,
    drop: np.ndarray | None = None,
) -> np.ndarray:
    """BSHD attention in float64.

    q ``[B, S_q, H, D]``, k/v ``[B, S_kv, H_kv, D]`` -> ``[B, S_q, H, D]``.

    Restates ``_forward_math`` (stratego/networks/attention.py:281-316):
    transpose to BHSD (:293-296), expand KV heads (:299), scores
    ``(Q K^T) * (1/sqrt(D))`` with the scale applied after the product
    (:300-301), top-left causal mask ``triu(ones(S_q, S_kv), 1) -> -inf``
    (:303-308), softmax over keys (:310), ``P V`` and back to BSHD (:315-316).
    ``drop`` (``[B, H, S_q, S_kv]``: ``keep / (1 - p)``, e.g. from
    :func:`oracle.dropout.keep_mask`) multiplies the softmax weights before
    ``P V``, as ``F.dropout`` on them does in training (:312-313); None is
    inference.  ``key_pad`` (``[B, S_kv]``, True = ignore) adds the
    key-padding mask the Belief decoder passes as ``memory_key_padding_mask``
    (belief_net.py:159,172-177).
    """
    q64 = np.asarray(q, dtype=np.float64).transpose(0, 2, 1, 3)
    k64 = np.asarray(k, dtype=np.float64).transpose(0, 2, 1, 3)
    v64 = np.asarray(v, dtype=np.float64).transpose(0, 2, 1, 3)
    num_heads, seq_q, head_dim = q64.shape[1], q64.shape[2], q64.shape[3]
    seq_kv = k64.shape[2]
    k64 = expand_kv_heads(k64, num_heads)
    v64 = expand_kv_heads(v64, num_heads)
    if scale is None:
        scale = 1.0 / np.sqrt(head_dim)
    scores = np.matmul(q64, k64.swapaxes(-1, -2)) * scale
    if causal:
        above = np.triu(np.ones((seq_q, seq_kv), dtype=bool), 1)
        scores = np.where(above, NEG_INF, scores)
    if key_pad is not None:
        scores = np.where(np.asarray(key_pad, dtype=bool)[:, None, None, :], NEG_INF, scores)
    probs = softmax_lastdim(scores)
    if drop is not None:
        probs = probs * np.asarray(drop, dtype=np.float64)
    return np.matmul(probs, v64).transpose(0, 2, 1, 3)


def attention_backward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    d_o: np.ndarray,
    causal: bool = False,
    scale: float | None = None,
    key_pad: np.ndarray | None = None,
    drop: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Gradients ``(dq, dk, dv)`` of :func:`attention` for the upstream
    gradient ``d_o`` (``[B, S_q, H, D]``), in float64.

    This is what autograd takes through ``_forward_math``
    (stratego/networks/attention.py:281-316) when the training step calls
    ``backward`` (stratego/training/move_trainer.py:140), written out by the
    chain rule: ``O = P V`` gives ``dV = P^T dO`` and ``dP = dO V^T``; the
    softmax over keys (:310) gives ``dS = P * (dP - rowsum(dP * P))``; the
    post-product scale (:300-301) gives ``dQ = scale dS K`` and
    ``dK = scale dS^T Q``.  The mask is applied with ``masked_fill``
    (:303-308), whose gradient is 0 at masked scores, so ``dS = 0`` there.
    The GQA expansion (:210-220) sums the gradients of the ``H / H_kv`` query
    heads that share a KV head.  An all-masked row has ``P = NaN`` (as in the
    forward): its ``dS`` is still 0 (every entry is masked), so it adds 0 to
    ``dq`` and ``dk``, but ``dV = P^T dO`` makes the whole ``(batch, head)``
    slice of ``dv`` NaN -- what autograd through that math gives.  With
    ``drop`` (the forward's dropout multipliers M) the weights that reach V
    are ``P o M``: ``dV = (P o M)^T dO`` and the softmax sees ``dP o M``.
    """
    q64 = np.asarray(q, dtype=np.float64).transpose(0, 2, 1, 3)
    k64 = np.asarray(k, dtype=np.float64).transpose(0, 2, 1, 3)
    v64 = np.asarray(v, dtype=np.float64).transpose(0, 2, 1, 3)
    g64 = np.asarray(d_o, dtype=np.float64).transpose(0, 2, 1, 3)
    b, num_heads, seq_q, head_dim = q64.shape
    kv_heads, seq_kv = k64.shape[1], k64.shape[2]
    ke = expand_kv_heads(k64, num_heads)
    ve = expand_kv_heads(v64, num_heads)
    if scale is None:
        scale = 1.0 / np.sqrt(head_dim)
    scores = np.matmul(q64, ke.swapaxes(-1, -2)) * scale
    masked = np.zeros((1, 1, seq_q, seq_kv), dtype=bool)
    if causal:
        masked = masked | np.triu(np.ones((seq_q, seq_kv), dtype=bool), 1)
    if key_pad is not None:
        masked = masked | np.asarray(key_pad, dtype=bool)[:, None, None, :]
    p = softmax_lastdim(np.where(masked, NEG_INF, scores))
    mult = None if drop is None else np.asarray(drop, dtype=np.float64)
    with np.errstate(invalid="ignore"):
        dv = np.matmul(p.swapaxes(-1, -2) if mult is None else (p * mult).swapaxes(-1, -2), g64)
        dp = np.matmul(g64, ve.swapaxes(-1, -2))
        if mult is not None:
            dp = dp * mult
        ds = np.where(masked, 0.0, p * (dp - np.sum(dp * p, axis=-1, keepdims=True)))
        dq = np.matmul(ds, ke) * scale
        dk = np.matmul(ds.swapaxes(-1, -2), q64) * scale
    group = num_heads // kv_heads
    if group > 1:
        dk = dk.reshape(b, kv_heads, group, seq_kv, head_dim).sum(axis=2)
        dv = dv.reshape(b, kv_heads, group, seq_kv, head_dim).sum(axis=2)
    return dq.transpose(0, 2, 1, 3), dk.transpose(0, 2, 1, 3), dv.transpose(0, 2, 1, 3)


def linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """``x W^T + b`` as ``torch.nn.Linear`` (weight ``[out, in]``)."""
    y = np.asarray(x, np.float64) @ np.asarray(weight, np.float64).T
    return y if bias is None else y + np.asarray(bias, np.float64)


def mha_forward(
    x: np.ndarray,
    key_value: np.ndarray | None,
    weights: dict[str, np.ndarray],
    num_heads: int,
    num_kv_heads: int | None = None,
    causal: bool = False,
) -> np.ndarray:
    """Module-level forward of ``MultiHeadAttention`` in float64.

    Restates stratego/networks/attention.py:152-204: q/k/v projections from
    ``x`` / ``key_value`` (:175-179), BSHD views (:184-186), causal masking only
    for self-attention (:189), attention (:193-200), reshape and ``out_proj``
    (:203-204).  ``weights`` holds the module's state_dict entries
    (``q_proj.weight`` ... and optional ``*.bias``).
    """
    kv_heads = num_heads if num_kv_heads is None else num_kv_heads
    src = x if key_value is None else key_value
    b, s_q, e = x.shape
    s_kv = src.shape[1]
    d = e // num_heads
    q = linear(x, weights["q_proj.weight"], weights.get("q_proj.bias")).reshape(b, s_q, num_heads, d)
    k = linear(src, weights["k_proj.weight"], weights.get("k_proj.bias")).reshape(b, s_kv, kv_heads, d)
    v = linear(src, weights["v_proj.weight"], weights.get("v_proj.bias")).reshape(b, s_kv, kv_heads, d)
    o = attention(q, k, v, causal=causal and key_value is None)
    return linear(o.reshape(b, s_q, num_heads * d), weights["out_proj.weight"], weights.get("out_proj.bias"))


def layer_norm(x: np.ndarray, weight: np.ndarray | None, bias: np.ndarray | None, eps: float = 1e-5) -> np.ndarray:
    """``nn.LayerNorm`` over the last axis in float64: ``(x - mean) /
    sqrt(var + eps) * weight + bias`` with the biased variance, as torch's
    layer_norm defines it (the ``ln1`` / ``ln2`` of
    stratego/networks/transformer.py:116-118)."""
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def preln_attention_half(
    x: np.ndarray,
    weights: dict[str, np.ndarray],
    num_heads: int,
    causal: bool = False,
    eps: float = 1e-5,
) -> np.ndarray:
    """The attention half of ``PreLNTransformerBlock.forward``
    (stratego/networks/transformer.py:143 with dropout inactive):
    ``x + attn(ln1(x))``.  ``weights`` holds the block's state_dict entries
    ``ln1.weight``, ``ln1.bias`` and ``attn.{q,k,v,out}_proj.weight`` (and
    optional ``.bias``)."""
    h = layer_norm(x, weights.get("ln1.weight"), weights.get("ln1.bias"), eps)
    attn_w = {k[len("attn."):]: v for k, v in weights.items() if k.startswith("attn.")}
    return x + mha_forward(h, None, attn_w, num_heads, causal=causal)
