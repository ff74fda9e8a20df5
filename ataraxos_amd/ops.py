"""Torch-facing entry points of the gfx950 kernels.

Every function here takes device tensors, checks them, and launches a kernel
from ``libataraxos_attn.so`` on the current HIP stream.  There is no CPU or
PyTorch substitute behind them: a CPU tensor, a missing library or a shape
outside the kernels' range raises.

* :func:`attention` — fused ``softmax(Q K^T * scale + mask) V`` on BSHD views
  (the seam ``_forward_<backend>(q, k, v, is_causal)`` of
  ``stratego/networks/attention.py:222-316``), differentiable.
* :func:`attention_backward` — its dQ, dK, dV in one launch (the gradient
  ``stratego/training/move_trainer.py:140`` takes through that attention).
* :func:`kq_policy` — the key-query policy head's logits, legal-move mask and
  softmax (``stratego/networks/move_net.py:92-95`` plus the callers' softmax,
  ``stratego/training/selfplay.py:284``).
* :func:`kq_policy_backward` — its dq, dk for the gradient of the logits or
  of the probabilities, in one launch.
* :func:`mha_forward` — a whole self-attention layer (projections, attention,
  output projection) in one launch, ``stratego/networks/attention.py:152-204``.
* :func:`attention_decode` — one query per (batch, head) against a KV cache.
* :func:`dropout_mask` — the keep decisions of attention dropout (the
  ``dropout_p`` / ``dropout_seed`` / ``dropout_offset`` arguments of the
  attention functions) as a ``[B, H, S_q, S_kv]`` uint8 tensor.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

_DTYPES = {
    torch.float32: _lib.DTYPE_FP32,
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_FP16,
}

MAX_SEQ_KV = 256
HEAD_DIMS = (16, 32, 48, 64, 80, 96, 112, 128)
# head_dims whose attention kernels are built with dropout (the reference
# networks' 64 and 48)
DROPOUT_HEAD_DIMS = (48, 64)
_U64 = (1 << 64) - 1


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_device(name: str, *tensors: torch.Tensor) -> None:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(f"{name}: expected GPU tensors, got a tensor on {t.device}")
        if t.device != dev:
            raise RuntimeError(f"{name}: tensors on different devices ({dev} vs {t.device})")


def _rows_ok(t: torch.Tensor) -> bool:
    """Every row of the last dim is contiguous and starts on a 16-byte boundary."""
    es = t.element_size()
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all((s * es) % 16 == 0 for s in t.stride()[:-1]))


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` or a copy of it whose rows of the last dim are contiguous
    and start on 16-byte boundaries, as the kernels require.  A contiguous
    view at a misaligned address (``contiguous()`` returns it unchanged) is
    copied into a fresh allocation."""
    if _rows_ok(t):
        return t
    c = t.contiguous()
    if not _rows_ok(c):
        c = t.clone(memory_format=torch.contiguous_format)
    return c


def _check_out(name: str, out: torch.Tensor, shape: tuple, dtype: torch.dtype, device: torch.device) -> None:
    """A caller-supplied output must have exactly ``shape``, ``dtype`` and
    ``device``, a contiguous last dim and 16-byte aligned rows: the ABI
    passes no stride for the last dim and sizes its bounds from the strides."""
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device:
        raise ValueError(f"{name}: out must be {tuple(shape)} {dtype} on {device}, "
                         f"got {tuple(out.shape)} {out.dtype} on {out.device}")
    if not _rows_ok(out):
        raise ValueError(f"{name}: out needs a contiguous last dim and 16-byte aligned rows")


def _padding_bytes(key_padding_mask: torch.Tensor | None, b: int, skv: int, ref: torch.Tensor):
    if key_padding_mask is None:
        return None
    if tuple(key_padding_mask.shape) != (b, skv):
        raise ValueError(f"attention: key_padding_mask must be [{b}, {skv}]")
    _require_device("attention", ref, key_padding_mask)
    # bool and uint8 share one byte per element: reinterpret, no copy
    return (key_padding_mask.view(torch.uint8) if key_padding_mask.dtype == torch.bool
            else (key_padding_mask != 0).view(torch.uint8)).contiguous()


def attention_supported(head_dim: int, seq_kv: int, dtype: torch.dtype, dropout: bool = False) -> bool:
    """True when :func:`attention` covers this shape and dtype (with
    ``dropout``: with a nonzero ``dropout_p``)."""
    if dropout and head_dim not in DROPOUT_HEAD_DIMS:
        return False
    return dtype in _DTYPES and head_dim in HEAD_DIMS and 1 <= seq_kv <= MAX_SEQ_KV


def _set_dropout(p, dropout_p: float, seed: int, offset: int) -> None:
    if not 0.0 <= dropout_p < 1.0:
        raise ValueError(f"dropout_p must be in [0, 1), got {dropout_p}")
    p.dropout_p = float(dropout_p)
    p.dropout_seed = int(seed) & _U64
    p.dropout_offset = int(offset) & _U64


def new_dropout_seed() -> int:
    """A fresh 63-bit dropout seed from torch's default (CPU) generator, so
    ``torch.manual_seed`` makes a dropout run repeatable."""
    return int(torch.randint(0, 1 << 62, (1,), dtype=torch.int64).item())


def dropout_mask(
    batch: int, num_heads: int, seq_q: int, seq_kv: int, p: float, seed: int, offset: int = 0,
    device: torch.device | str = "cuda",
) -> torch.Tensor:
    """``keep[b, h, i, j]`` (uint8, 1 = kept) of attention dropout with
    ``(p, seed, offset)``: the decisions :func:`attention_forward` and
    :func:`attention_backward` make for the same arguments.  One launch of
    ``atx_dropout_mask``."""
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout_mask: p must be in [0, 1), got {p}")
    keep = torch.empty((batch, num_heads, seq_q, seq_kv), dtype=torch.uint8, device=device)
    _require_device("dropout_mask", keep)
    rc = _lib.load().atx_dropout_mask(batch, num_heads, seq_q, seq_kv, float(p), int(seed) & _U64,
                                      int(offset) & _U64, keep.data_ptr(), _stream(keep))
    _lib.check(rc, "atx_dropout_mask")
    return keep


def attention_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: float | None = None,
    key_padding_mask: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    dropout_seed: int = 0,
    dropout_offset: int = 0,
) -> torch.Tensor:
    """Forward only (no autograd).  q ``[B, S_q, H, D]``, k/v ``[B, S_kv, H_kv, D]``.

    ``key_padding_mask`` is ``[B, S_kv]`` bool, True = ignore the key (the
    ``key_padding_mask`` convention of ``torch.nn.MultiheadAttention``).
    ``dropout_p > 0`` (head_dim 48 or 64) drops each softmax weight with
    that probability and scales the rest by ``1 / (1 - dropout_p)``, as
    ``nn.Dropout`` on the weights does (attention.py:312-313); the decisions
    are a function of ``(dropout_seed, dropout_offset)`` and the weight's
    index (:func:`dropout_mask`).
    Returns ``[B, S_q, H, D]`` contiguous in q's dtype.
    """
    _require_device("attention", q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("attention: q, k, v must be [batch, seq, heads, head_dim]")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in _DTYPES:
        raise ValueError(f"attention: q/k/v dtypes {q.dtype}/{k.dtype}/{v.dtype} unsupported or mixed")
    b, sq, h, d = q.shape
    bk, skv, hkv, dk = k.shape
    if bk != b or dk != d or tuple(v.shape) != (b, skv, hkv, d):
        raise ValueError(f"attention: shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if h % hkv != 0:
        raise ValueError(f"attention: {h} query heads not divisible by {hkv} kv heads")
    q, k, v = _aligned_rows(q), _aligned_rows(k), _aligned_rows(v)
    if out is None:
        out = torch.empty((b, sq, h, d), dtype=q.dtype, device=q.device)
    else:
        _check_out("attention", out, (b, sq, h, d), q.dtype, q.device)
    pad = _padding_bytes(key_padding_mask, b, skv, q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)

    p = _lib.AttnParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.seq_q, p.seq_kv, p.num_heads, p.num_kv_heads, p.head_dim = b, sq, skv, h, hkv, d
    p.q, (p.q_stride_b, p.q_stride_s, p.q_stride_h) = q.data_ptr(), q.stride()[:3]
    p.k, (p.k_stride_b, p.k_stride_s, p.k_stride_h) = k.data_ptr(), k.stride()[:3]
    p.v, (p.v_stride_b, p.v_stride_s, p.v_stride_h) = v.data_ptr(), v.stride()[:3]
    p.o, (p.o_stride_b, p.o_stride_s, p.o_stride_h) = out.data_ptr(), out.stride()[:3]
    p.scale = float(scale)
    p.causal = 1 if causal else 0
    p.key_pad = pad.data_ptr() if pad is not None else None
    p.key_pad_stride_b = pad.stride(0) if pad is not None else 0
    _set_dropout(p, dropout_p, dropout_seed, dropout_offset)
    _lib.check(_lib.call("atx_attn_fwd", p, _stream(q)), "atx_attn_fwd")
    return out


def _attention_reference_fp32(q, k, v, causal, scale, key_padding_mask):
    """Differentiable fp32 restatement used only to form gradients."""
    b, sq, h, d = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    qh = q.float().transpose(1, 2)
    kh = k.float().transpose(1, 2)
    vh = v.float().transpose(1, 2)
    if hkv != h:
        kh = kh.repeat_interleave(h // hkv, dim=1)
        vh = vh.repeat_interleave(h // hkv, dim=1)
    s = torch.matmul(qh, kh.transpose(-2, -1).contiguous()) * scale
    if causal:
        s = s.masked_fill(torch.ones(sq, skv, dtype=torch.bool, device=q.device).triu(1), float("-inf"))
    if key_padding_mask is not None:
        s = s.masked_fill(key_padding_mask[:, None, None, :], float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vh).transpose(1, 2)


_BWD_DTYPES = (torch.bfloat16, torch.float16)
_ATTN_BWD_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
_LDS_BYTES = 160 * 1024


def _bwd_lds_bytes(head_dim: int, rows_q: int, seq_kv: int, fp32: bool = False, key_chunks: int | None = None) -> int:
    """LDS of one backward workgroup: K, V (S_kv rounded up to 32-key chunks),
    ``rows_q`` query rows of Q and dO, and per query the log-sum-exp and
    delta (fp32).  16-bit rows are padded to an odd number of 16-byte units
    except at head_dim 64 / 128; fp32 rows are not padded."""
    nkc = key_chunks if key_chunks is not None else -(-seq_kv // 32)
    rk = nkc * 32
    if fp32:
        return (2 * rk + 2 * rows_q) * head_dim * 4 + rows_q * 8
    rs = head_dim * 2 if head_dim in (64, 128) else head_dim * 2 + 16
    return (2 * rk + 2 * rows_q) * rs + rows_q * 8


def _pow2_chunks(nkc: int) -> int:
    return 1 if nkc <= 1 else 2 if nkc <= 2 else 4 if nkc <= 4 else 8


def attention_backward_plan(
    head_dim: int, seq_q: int, seq_kv: int, num_heads: int, num_kv_heads: int, dtype: torch.dtype,
    dropout: bool = False,
) -> dict | None:
    """How ``atx_attn_bwd`` runs this shape (the library's own rule, restated):
    ``{"loop": bool, "key_chunks": int, "query_block": int, "lds": int}``, or
    None when the kernels do not cover it.  ``loop`` is the variant that runs
    the query heads of a KV group and blocks of ``query_block`` query rows one
    after another (grouped-query attention, more than 256 queries, or more
    query rows than LDS holds at once).  ``dropout`` (a nonzero
    ``dropout_p``) runs the same plan, at head_dim 48 or 64 only."""
    if (dtype not in _ATTN_BWD_DTYPES or num_kv_heads < 1 or num_heads % num_kv_heads
            or head_dim % 16 or not 16 <= head_dim <= 128 or not 1 <= seq_kv <= MAX_SEQ_KV
            or not 1 <= seq_q <= (1 << 20) or (dropout and head_dim not in DROPOUT_HEAD_DIMS)):
        return None
    fp32 = dtype == torch.float32
    qalign = 16 if fp32 else 32
    rq_all = -(-seq_q // qalign) * qalign
    exact = -(-seq_kv // 32)
    nkc = _pow2_chunks(exact) if fp32 else exact
    loop = num_heads != num_kv_heads or seq_q > 256 or _bwd_lds_bytes(head_dim, rq_all, seq_kv, fp32, nkc) > _LDS_BYTES
    qb = 0
    if loop:
        nkc = _pow2_chunks(exact)
        qb = min(rq_all, 256)
        while qb > qalign and _bwd_lds_bytes(head_dim, qb, seq_kv, fp32, nkc) > _LDS_BYTES:
            qb -= qalign
    lds = _bwd_lds_bytes(head_dim, qb if loop else rq_all, seq_kv, fp32, nkc)
    if lds > _LDS_BYTES:
        return None
    return {"loop": loop, "key_chunks": nkc, "query_block": qb, "lds": lds}


def attention_backward_supported(
    head_dim: int, seq_q: int, seq_kv: int, num_heads: int, num_kv_heads: int, dtype: torch.dtype,
    dropout: bool = False,
) -> bool:
    """True when :func:`attention_backward` covers this shape and dtype:
    bf16 / fp16 / fp32, GQA included, head_dim a multiple of 16 up to 128, up
    to 256 keys and any number of queries; fp32 with head_dim >= 80 only up
    to 128 keys (its K and V rows must fit in LDS); with dropout head_dim 48
    or 64."""
    return attention_backward_plan(head_dim, seq_q, seq_kv, num_heads, num_kv_heads, dtype, dropout) is not None


def attention_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    grad_out: torch.Tensor,
    causal: bool = False,
    scale: float | None = None,
    key_padding_mask: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    dropout_seed: int = 0,
    dropout_offset: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients ``(dq, dk, dv)`` of :func:`attention_forward` for the
    upstream gradient ``grad_out``, given its inputs and its output ``out``
    (q, out, grad_out ``[B, S_q, H, D]``; k, v ``[B, S_kv, H_kv, D]``; bf16,
    fp16 or fp32).  One kernel launch; the softmax is recomputed from Q and K,
    so nothing but the output is kept from the forward.  With grouped-query
    attention, dk and dv sum the gradients of the query heads that share a KV
    head (``repeat_interleave``, attention.py:210-220).  A forward run with
    dropout passes the same ``dropout_p``, ``dropout_seed`` and
    ``dropout_offset``: the kernel recomputes the same keep decisions.
    Returns contiguous tensors in the inputs' dtype, dk / dv with H_kv
    heads."""
    _require_device("attention_backward", q, k, v, out, grad_out)
    if not (q.dtype == k.dtype == v.dtype == out.dtype == grad_out.dtype):
        raise ValueError("attention_backward: mixed dtypes")
    b, sq, h, d = q.shape
    skv, hkv = k.shape[1], k.shape[2]
    if (tuple(k.shape) != (b, skv, hkv, d) or tuple(v.shape) != (b, skv, hkv, d)
            or tuple(out.shape) != (b, sq, h, d) or tuple(grad_out.shape) != (b, sq, h, d)):
        raise ValueError("attention_backward: shape mismatch")
    if not attention_backward_supported(d, sq, skv, h, hkv, q.dtype, dropout_p > 0.0):
        raise NotImplementedError(
            f"attention_backward: {q.dtype}, heads {h}/{hkv}, head_dim {d}, seq {sq}x{skv}"
            f"{', dropout' if dropout_p > 0.0 else ''} not covered by the kernel"
        )
    q, k, v, out, grad_out = (_aligned_rows(t) for t in (q, k, v, out, grad_out))
    pad = _padding_bytes(key_padding_mask, b, skv, q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    dq = torch.empty((b, sq, h, d), dtype=q.dtype, device=q.device)
    dk = torch.empty((b, skv, hkv, d), dtype=q.dtype, device=q.device)
    dv = torch.empty((b, skv, hkv, d), dtype=q.dtype, device=q.device)

    p = _lib.AttnBwdParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.seq_q, p.seq_kv, p.num_heads, p.num_kv_heads, p.head_dim = b, sq, skv, h, hkv, d
    for name, t in (("q", q), ("k", k), ("v", v), ("o", out), ("do", grad_out), ("dq", dq), ("dk", dk), ("dv", dv)):
        setattr(p, "d_o" if name == "do" else name, t.data_ptr())
        for axis, stride in zip("bsh", t.stride()[:3]):
            setattr(p, f"{name}_stride_{axis}", stride)
    p.scale = float(scale)
    p.causal = 1 if causal else 0
    p.key_pad = pad.data_ptr() if pad is not None else None
    p.key_pad_stride_b = pad.stride(0) if pad is not None else 0
    _set_dropout(p, dropout_p, dropout_seed, dropout_offset)
    _lib.check(_lib.call("atx_attn_bwd", p, _stream(q)), "atx_attn_bwd")
    return dq, dk, dv


class _HipAttention(torch.autograd.Function):
    """HIP forward and HIP backward (:func:`attention_backward`: bf16, fp16
    and fp32, GQA included).  The one shape family the backward kernels do
    not hold in LDS -- fp32 with head_dim >= 80 and more than 128 keys, which
    no network of the reference uses -- takes its gradients from an fp32
    recomputation with torch ops on the same device.  With dropout only the
    seed and offset are kept: the backward recomputes the keep decisions."""

    @staticmethod
    def forward(ctx, q, k, v, causal, scale, key_padding_mask, dropout_p, seed, offset):  # type: ignore[override]
        out = attention_forward(q, k, v, causal=causal, scale=scale, key_padding_mask=key_padding_mask,
                                dropout_p=dropout_p, dropout_seed=seed, dropout_offset=offset)
        ctx.save_for_backward(q, k, v, out)
        ctx.causal, ctx.scale, ctx.kpm = causal, scale, key_padding_mask
        ctx.drop = (dropout_p, seed, offset)
        return out

    @staticmethod
    def backward(ctx, grad_out):  # type: ignore[override]
        q, k, v, out = ctx.saved_tensors
        b, sq, h, d = q.shape
        dropout_p, seed, offset = ctx.drop
        none = (None,) * 6
        if attention_backward_supported(d, sq, k.shape[1], h, k.shape[2], q.dtype, dropout_p > 0.0):
            dq, dk, dv = attention_backward(q, k, v, out, grad_out.to(q.dtype), ctx.causal, ctx.scale, ctx.kpm,
                                            dropout_p, seed, offset)
            return (dq, dk, dv, *none)
        if dropout_p > 0.0:  # the forward accepted it, so the backward covers it: not reached
            raise NotImplementedError("attention backward with dropout: shape not covered by the kernel")
        with torch.enable_grad():
            qf = q.detach().float().requires_grad_(True)
            kf = k.detach().float().requires_grad_(True)
            vf = v.detach().float().requires_grad_(True)
            o = _attention_reference_fp32(qf, kf, vf, ctx.causal, ctx.scale, ctx.kpm)
            gq, gk, gv = torch.autograd.grad(o, (qf, kf, vf), grad_out.float())
        return (gq.to(q.dtype), gk.to(k.dtype), gv.to(v.dtype), *none)


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    scale: float | None = None,
    key_padding_mask: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    dropout_seed: int | None = None,
    dropout_offset: int = 0,
) -> torch.Tensor:
    """Fused attention on BSHD tensors, with autograd (see :func:`attention_forward`).

    With ``dropout_p > 0`` and no ``dropout_seed`` a seed is drawn from
    torch's default generator (:func:`new_dropout_seed`)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if dropout_p > 0.0 and dropout_seed is None:
        dropout_seed = new_dropout_seed()
    seed = 0 if dropout_seed is None else dropout_seed
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return _HipAttention.apply(q, k, v, causal, scale, key_padding_mask, dropout_p, seed, dropout_offset)
    return attention_forward(q, k, v, causal=causal, scale=scale, key_padding_mask=key_padding_mask,
                             dropout_p=dropout_p, dropout_seed=seed, dropout_offset=dropout_offset)


def kq_policy(
    q: torch.Tensor,
    k: torch.Tensor,
    legal_move_mask: torch.Tensor | None = None,
    scale: float | None = None,
    output: str = "probs",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Policy over from x to squares for every sample.

    q, k: ``[B, S, d]`` (from-queries, to-keys).  ``legal_move_mask``: bool
    ``[B, S, S]``, True = legal.  ``scale`` defaults to ``1/sqrt(d)`` (the
    reference divides by ``policy_d_model ** 0.5``).  ``output="probs"``
    returns the softmax over all ``S*S`` entries with illegal entries exactly
    0; ``output="logits"`` returns the scaled logits with illegal entries
    -1e10.  Both are fp32 ``[B, S*S]`` in from-major order.
    """
    _require_device("kq_policy", q, k)
    if q.dim() != 3 or q.shape != k.shape:
        raise ValueError(f"kq_policy: q{tuple(q.shape)} and k{tuple(k.shape)} must both be [B, S, d]")
    if q.dtype != k.dtype or q.dtype not in _DTYPES:
        raise ValueError(f"kq_policy: unsupported or mixed dtypes {q.dtype}/{k.dtype}")
    if output not in ("probs", "logits"):
        raise ValueError(f"kq_policy: output must be 'probs' or 'logits', got {output!r}")
    b, s, d = q.shape
    q, k = _aligned_rows(q), _aligned_rows(k)
    if out is None:
        out = torch.empty((b, s * s), dtype=torch.float32, device=q.device)
    elif tuple(out.shape) != (b, s * s) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("kq_policy: out must be a contiguous fp32 [B, S*S] tensor")
    mask = None
    if legal_move_mask is not None:
        if tuple(legal_move_mask.shape) != (b, s, s):
            raise ValueError(f"kq_policy: legal_move_mask must be [{b}, {s}, {s}]")
        _require_device("kq_policy", q, legal_move_mask)
        mask = legal_move_mask if legal_move_mask.dtype == torch.bool else legal_move_mask != 0
        mask = mask.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(d)

    p = _lib.KqParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.seq, p.dim = b, s, d
    p.out_mode = _lib.KQ_OUT_PROBS if output == "probs" else _lib.KQ_OUT_LOGITS
    p.q, p.q_stride_b, p.q_stride_s = q.data_ptr(), q.stride(0), q.stride(1)
    p.k, p.k_stride_b, p.k_stride_s = k.data_ptr(), k.stride(0), k.stride(1)
    p.mask = mask.data_ptr() if mask is not None else None
    p.mask_stride_b = mask.stride(0) if mask is not None else 0
    p.mask_stride_s = mask.stride(1) if mask is not None else 0
    p.out, p.out_stride_b = out.data_ptr(), out.stride(0)
    p.scale = float(scale)
    _lib.check(_lib.call("atx_kq_masked_softmax_fwd", p, _stream(q)), "atx_kq_masked_softmax_fwd")
    return out


def kq_policy_backward_supported(seq: int, dim: int, dtype: torch.dtype) -> bool:
    """True when :func:`kq_policy_backward` covers this shape and dtype:
    bf16 / fp16 / fp32, ``seq`` up to 128, ``dim`` a multiple of 16 up to 128
    or of 64 up to 4096 (the reference's policy head has dim 384); fp32: any
    multiple of 16 up to 4096."""
    return (dtype in _ATTN_BWD_DTYPES and 1 <= seq <= 128 and dim % 16 == 0 and 16 <= dim <= 4096
            and (dim <= 128 or dim % 64 == 0 or dtype == torch.float32))


def kq_policy_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    grad: torch.Tensor,
    legal_move_mask: torch.Tensor | None = None,
    scale: float | None = None,
    output: str = "logits",
    probs: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Gradients ``(dq, dk)`` of :func:`kq_policy` for the upstream gradient
    ``grad`` (fp32 ``[B, S*S]``) of its ``output`` ("logits", or "probs" with
    the forward's ``probs``).  Illegal entries pass no gradient.  One kernel
    launch; returns contiguous tensors in q's dtype."""
    _require_device("kq_policy_backward", q, k, grad)
    if q.dim() != 3 or q.shape != k.shape:
        raise ValueError(f"kq_policy_backward: q{tuple(q.shape)} and k{tuple(k.shape)} must both be [B, S, d]")
    if q.dtype != k.dtype:
        raise ValueError("kq_policy_backward: mixed dtypes")
    if output not in ("probs", "logits"):
        raise ValueError(f"kq_policy_backward: output must be 'probs' or 'logits', got {output!r}")
    b, s, d = q.shape
    if not kq_policy_backward_supported(s, d, q.dtype):
        raise NotImplementedError(f"kq_policy_backward: {q.dtype}, seq {s}, dim {d} not covered by the kernel")
    if tuple(grad.shape) != (b, s * s):
        raise ValueError(f"kq_policy_backward: grad must be [{b}, {s * s}]")
    grad = grad.float()
    if grad.stride(1) != 1:
        grad = grad.contiguous()
    if output == "probs":
        if probs is None or tuple(probs.shape) != (b, s * s):
            raise ValueError("kq_policy_backward: output='probs' needs the forward's probs [B, S*S]")
        _require_device("kq_policy_backward", q, probs)
        probs = probs.float()
        if probs.stride(1) != 1:
            probs = probs.contiguous()
    q, k = _aligned_rows(q), _aligned_rows(k)
    mask = None
    if legal_move_mask is not None:
        if tuple(legal_move_mask.shape) != (b, s, s):
            raise ValueError(f"kq_policy_backward: legal_move_mask must be [{b}, {s}, {s}]")
        _require_device("kq_policy_backward", q, legal_move_mask)
        mask = legal_move_mask if legal_move_mask.dtype == torch.bool else legal_move_mask != 0
        if mask.stride(2) != 1:
            mask = mask.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    dq = torch.empty((b, s, d), dtype=q.dtype, device=q.device)
    dk = torch.empty((b, s, d), dtype=q.dtype, device=q.device)

    p = _lib.KqBwdParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.seq, p.dim = b, s, d
    p.out_mode = _lib.KQ_OUT_PROBS if output == "probs" else _lib.KQ_OUT_LOGITS
    p.q, p.q_stride_b, p.q_stride_s = q.data_ptr(), q.stride(0), q.stride(1)
    p.k, p.k_stride_b, p.k_stride_s = k.data_ptr(), k.stride(0), k.stride(1)
    p.mask = mask.data_ptr() if mask is not None else None
    p.mask_stride_b = mask.stride(0) if mask is not None else 0
    p.mask_stride_s = mask.stride(1) if mask is not None else 0
    p.grad, p.grad_stride_b = grad.data_ptr(), grad.stride(0)
    p.probs = probs.data_ptr() if output == "probs" else None
    p.probs_stride_b = probs.stride(0) if output == "probs" else 0
    p.dq, p.dq_stride_b, p.dq_stride_s = dq.data_ptr(), dq.stride(0), dq.stride(1)
    p.dk, p.dk_stride_b, p.dk_stride_s = dk.data_ptr(), dk.stride(0), dk.stride(1)
    p.scale = float(scale)
    _lib.check(_lib.call("atx_kq_bwd", p, _stream(q)), "atx_kq_bwd")
    return dq, dk


MHA_HEADS = (2, 4, 6, 8)


def _mha_lds_bytes(embed_dim: int, seq: int) -> int:
    np_ = -(-seq // 16)
    return np_ * 16 * embed_dim * 2 + (2 * np_ * 16 + 32 * ((np_ + 1) // 2)) * 64 * 2


def mha_forward_supported(embed_dim: int, num_heads: int, seq: int, dtype: torch.dtype) -> bool:
    """True when :func:`mha_forward` covers this layer: bf16/fp16, head_dim
    64 with 2/4/6/8 heads, or head_dim 48 with 8 heads (embed_dim 384, the
    reference Move network), up to 128 positions within 160 KiB of LDS."""
    return (
        dtype in _BWD_DTYPES
        and num_heads in MHA_HEADS
        and (embed_dim == 64 * num_heads or (num_heads == 8 and embed_dim == 384))
        and 1 <= seq <= 128
        and _mha_lds_bytes(embed_dim, seq) <= _LDS_BYTES
    )


def mha_block_supported(embed_dim: int, num_heads: int, seq: int, dtype: torch.dtype) -> bool:
    """True when :func:`mha_forward` also takes the pre-LN and the residual of
    a pre-LN block (the persistent kernel's shape): bf16/fp16, 6 heads of 64,
    65 to 101 positions -- the Move network layer of BASELINE config 3."""
    return dtype in _BWD_DTYPES and num_heads == 6 and embed_dim == 384 and 65 <= seq <= 101


def mha_forward(
    x: torch.Tensor,
    w_q: torch.Tensor,
    w_k: torch.Tensor,
    w_v: torch.Tensor,
    w_o: torch.Tensor,
    num_heads: int,
    b_q: torch.Tensor | None = None,
    b_k: torch.Tensor | None = None,
    b_v: torch.Tensor | None = None,
    b_o: torch.Tensor | None = None,
    causal: bool = False,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    packed: bool = False,
    repack: bool = False,
    workspace: torch.Tensor | None = None,
    noalloc: bool = False,
    ln_weight: torch.Tensor | None = None,
    ln_bias: torch.Tensor | None = None,
    ln_eps: float = 1e-5,
    residual: bool = False,
) -> torch.Tensor:
    """Whole self-attention layer in one launch (no autograd):
    ``out_proj(attention(q_proj(x), k_proj(x), v_proj(x)))`` with the
    ``nn.Linear`` weights ``[E, E]`` and optional biases ``[E]``.  x ``[B, L, E]``
    -> ``[B, L, E]`` in x's dtype.  Q, K, V and the attention output are
    rounded to x's dtype, as the reference's bf16 modules round them.

    Weight orders (identical results):

    * default: the ``nn.Linear`` matrices, read as they are (``atx_mha_fwd``);
    * ``packed=True``: the outputs of :func:`mha_pack_weight`
      (``atx_mha_fwd_packed``, the faster kernel);
    * ``repack=True``: the ``nn.Linear`` matrices, rearranged into
      ``workspace`` (a uint8 device tensor of at least
      :func:`mha_workspace_bytes` bytes, allocated here when None) by one
      extra launch on every call, then the packed kernel (``atx_mha_fwd_ws``).
      What the modules use: no cached copy can go stale;
    * ``noalloc=True``: as ``repack``, with the library's own per-GPU array in
      place of the workspace (``atx_mha_fwd_noalloc``: the C call allocates
      nothing; embed_dim <= 512; calls that overlap on one GPU race).

    The attention half of a pre-LN block, ``x + layer(LayerNorm(x))``
    (stratego/networks/transformer.py:143, dropout inactive), in the same
    launch: ``ln_weight`` / ``ln_bias`` / ``ln_eps`` (an ``nn.LayerNorm``'s
    parameters) normalise each row first, ``residual=True`` adds x to the
    layer output (rounded, then rounded again after the add).  Shapes of
    :func:`mha_block_supported` only; ``out`` may be x."""
    _require_device("mha_forward", x, w_q, w_k, w_v, w_o)
    if x.dim() != 3:
        raise ValueError("mha_forward: x must be [batch, seq, embed_dim]")
    b, l, e = x.shape
    for name, w in (("w_q", w_q), ("w_k", w_k), ("w_v", w_v), ("w_o", w_o)):
        if tuple(w.shape) != (e, e) or w.dtype != x.dtype:
            raise ValueError(f"mha_forward: {name} must be [{e}, {e}] in {x.dtype}")
    if not mha_forward_supported(e, num_heads, l, x.dtype):
        raise NotImplementedError(
            f"mha_forward: {x.dtype}, embed_dim {e}, {num_heads} heads, seq {l} not covered by the fused kernel"
        )
    biases = []
    for name, t in (("b_q", b_q), ("b_k", b_k), ("b_v", b_v), ("b_o", b_o)):
        if t is not None:
            if tuple(t.shape) != (e,) or t.dtype != x.dtype:
                raise ValueError(f"mha_forward: {name} must be [{e}] in {x.dtype}")
            _require_device("mha_forward", x, t)
            t = t.contiguous()
        biases.append(t)
    if packed + repack + noalloc > 1:
        raise ValueError("mha_forward: packed, repack and noalloc are exclusive")
    ln = []
    if ln_bias is not None and ln_weight is None:
        raise ValueError("mha_forward: ln_bias without ln_weight")
    if ln_weight is not None or residual:
        if not mha_block_supported(e, num_heads, l, x.dtype):
            raise NotImplementedError(
                f"mha_forward: pre-LN / residual need 6 heads of 64 at 65..101 positions (got {num_heads} heads, "
                f"embed_dim {e}, seq {l})"
            )
        for name, t in (("ln_weight", ln_weight), ("ln_bias", ln_bias)):
            if t is not None:
                if tuple(t.shape) != (e,) or t.dtype != x.dtype:
                    raise ValueError(f"mha_forward: {name} must be [{e}] in {x.dtype}")
                _require_device("mha_forward", x, t)
                t = _aligned_rows(t.contiguous())
            ln.append(t)
        if not (ln_eps >= 0.0 and math.isfinite(ln_eps)):
            raise ValueError(f"mha_forward: ln_eps must be finite and >= 0 (got {ln_eps})")
    else:
        ln = [None, None]
    x = _aligned_rows(x)
    ws = [_aligned_rows(w) if w.is_contiguous() else _aligned_rows(w.contiguous()) for w in (w_q, w_k, w_v, w_o)]
    if out is None:
        out = torch.empty((b, l, e), dtype=x.dtype, device=x.device)
    else:
        _check_out("mha_forward", out, (b, l, e), x.dtype, x.device)
    if scale is None:
        scale = 1.0 / math.sqrt(e // num_heads)  # 1 / sqrt(head_dim)

    p = _lib.MhaParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[x.dtype]
    p.batch, p.seq, p.embed_dim, p.num_heads = b, l, e, num_heads
    p.causal = 1 if causal else 0
    p.x, p.x_stride_b, p.x_stride_s = x.data_ptr(), x.stride(0), x.stride(1)
    p.w_q, p.w_k, p.w_v, p.w_o = (w.data_ptr() for w in ws)
    p.b_q, p.b_k, p.b_v, p.b_o = (t.data_ptr() if t is not None else None for t in biases)
    p.y, p.y_stride_b, p.y_stride_s = out.data_ptr(), out.stride(0), out.stride(1)
    p.scale = float(scale)
    p.ln_weight, p.ln_bias = (t.data_ptr() if t is not None else None for t in ln)
    p.ln_eps = float(ln_eps)
    p.residual = 1 if residual else 0
    if repack:
        need = mha_workspace_bytes(e)
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        elif (workspace.dtype != torch.uint8 or workspace.device != x.device or not workspace.is_contiguous()
              or workspace.numel() < need):
            raise ValueError(f"mha_forward: workspace must be a contiguous uint8 tensor of >= {need} bytes on {x.device}")
        rc = _lib.load().atx_mha_fwd_ws(ctypes.byref(p), workspace.data_ptr(), workspace.numel(), _stream(x))
        _lib.check(rc, "atx_mha_fwd_ws")
        return out
    if noalloc:
        with torch.cuda.device(x.device):  # the entry point uses the current device's array
            _lib.check(_lib.call("atx_mha_fwd_noalloc", p, _stream(x)), "atx_mha_fwd_noalloc")
        return out
    name = "atx_mha_fwd_packed" if packed else "atx_mha_fwd"
    _lib.check(_lib.call(name, p, _stream(x)), name)
    return out


def mha_workspace_bytes(embed_dim: int) -> int:
    """Bytes of the workspace of ``mha_forward(..., repack=True)``: the four
    weights in the packed order (``atx_mha_workspace_bytes``)."""
    return 4 * embed_dim * embed_dim * 2


def mha_pack_weight(w: torch.Tensor) -> torch.Tensor:
    """An ``nn.Linear`` weight ``[E, E]`` (bf16 / fp16, on the GPU) rearranged
    into the tile order :func:`mha_forward` reads with ``packed=True``
    (``atx_mha_pack_weight``); a new tensor of the same shape and dtype."""
    _require_device("mha_pack_weight", w)
    if w.dim() != 2 or w.shape[0] != w.shape[1] or w.dtype not in _BWD_DTYPES:
        raise ValueError("mha_pack_weight: w must be a square bf16/fp16 matrix")
    if not w.is_contiguous() or w.data_ptr() % 16:
        w = w.contiguous().clone()
    out = torch.empty_like(w, memory_format=torch.contiguous_format)
    rc = _lib.load().atx_mha_pack_weight(_DTYPES[w.dtype], w.shape[0], w.data_ptr(), out.data_ptr(), _stream(w))
    _lib.check(rc, "atx_mha_pack_weight")
    return out


def attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    kv_len: int | torch.Tensor,
    k_new: torch.Tensor | None = None,
    v_new: torch.Tensor | None = None,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One decode step: q ``[B, H, D]`` against caches ``[B, H_kv, T, D]``.

    ``kv_len`` is the number of valid cache rows after this step (an int, or a
    device int32 tensor ``[B]`` of per-sample lengths).  With ``k_new`` /
    ``v_new`` (``[B, H_kv, D]``) the row ``kv_len - 1`` is taken from them and
    written into the caches in the same launch.  Returns ``[B, H, D]``.
    """
    tensors = [q, k_cache, v_cache] + [t for t in (k_new, v_new) if t is not None]
    _require_device("attention_decode", *tensors)
    if q.dim() != 3 or k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("attention_decode: q must be [B, H, D] and caches [B, H_kv, T, D]")
    b, h, d = q.shape
    bc, hkv, cap, dc = k_cache.shape
    if bc != b or dc != d or h % hkv != 0:
        raise ValueError(f"attention_decode: q{tuple(q.shape)} does not match cache{tuple(k_cache.shape)}")
    if any(t.dtype != q.dtype for t in tensors) or q.dtype not in _DTYPES:
        raise ValueError("attention_decode: all tensors must share one supported dtype")
    if (k_new is None) != (v_new is None):
        raise ValueError("attention_decode: give k_new and v_new together")
    for t in (k_cache, v_cache):
        es = t.element_size()
        if t.stride(-1) != 1 or t.data_ptr() % 16 or any((s * es) % 16 for s in t.stride()[:-1]):
            raise ValueError("attention_decode: cache rows must be contiguous and 16-byte aligned")
    q = _aligned_rows(q)
    if k_new is not None:
        if tuple(k_new.shape) != (b, hkv, d) or tuple(v_new.shape) != (b, hkv, d):
            raise ValueError(f"attention_decode: k_new/v_new must be [{b}, {hkv}, {d}]")
        k_new, v_new = _aligned_rows(k_new), _aligned_rows(v_new)
    if out is None:
        out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
    else:
        _check_out("attention_decode", out, (b, h, d), q.dtype, q.device)
    if scale is None:
        scale = 1.0 / math.sqrt(d)

    p = _lib.DecodeParams()
    p.abi_version = _lib.ABI_VERSION
    p.dtype = _DTYPES[q.dtype]
    p.batch, p.num_heads, p.num_kv_heads, p.head_dim = b, h, hkv, d
    p.kv_capacity = cap
    lens = None
    if isinstance(kv_len, torch.Tensor):
        _require_device("attention_decode", q, kv_len)
        lens = kv_len.to(torch.int32).contiguous()
        if tuple(lens.shape) != (b,):
            raise ValueError(f"attention_decode: kv_len tensor must be [{b}]")
        p.kv_len, p.kv_lens = 0, lens.data_ptr()
    else:
        p.kv_len, p.kv_lens = int(kv_len), None
    p.q, p.q_stride_b, p.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
    p.k_cache, (p.k_stride_b, p.k_stride_h, p.k_stride_s) = k_cache.data_ptr(), k_cache.stride()[:3]
    p.v_cache, (p.v_stride_b, p.v_stride_h, p.v_stride_s) = v_cache.data_ptr(), v_cache.stride()[:3]
    if k_new is not None:
        p.k_new, p.k_new_stride_b, p.k_new_stride_h = k_new.data_ptr(), k_new.stride(0), k_new.stride(1)
        p.v_new, p.v_new_stride_b, p.v_new_stride_h = v_new.data_ptr(), v_new.stride(0), v_new.stride(1)
    p.o, p.o_stride_b, p.o_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    p.scale = float(scale)
    _lib.check(_lib.call("atx_attn_decode_fwd", p, _stream(q)), "atx_attn_decode_fwd")
    return out
